"""Python face of the tokenizer (include/wsp_decoder.h wsp_tokenizer_*): the
reference's WSP::Tokenizer (Tokenizer/Tokenizer.h:27-80), byte-level BPE from
a HuggingFace tokenizer.json, host code."""

from __future__ import annotations

import ctypes
from typing import List, Sequence

from . import _native as N


class TokenizerError(RuntimeError):
    """Tokenizer/Tokenizer.h:20-24 (and a malformed JSON document)."""


class Tokenizer:
    def __init__(self, handle, lib):
        self.handle, self.lib = handle, lib

    @classmethod
    def from_file(cls, path: str) -> "Tokenizer":
        return cls._open(lambda lib, out, err: lib.wsp_tokenizer_open(path.encode(), out, err, len(err)))

    @classmethod
    def from_json_text(cls, text) -> "Tokenizer":
        data = text.encode() if isinstance(text, str) else bytes(text)
        return cls._open(lambda lib, out, err: lib.wsp_tokenizer_open_bytes(data, len(data), out, err, len(err)))

    @classmethod
    def _open(cls, call) -> "Tokenizer":
        lib = N.load()
        handle = ctypes.c_void_p()
        err = ctypes.create_string_buffer(512)
        status = call(lib, ctypes.byref(handle), err)
        if status != N.WSP_OK:
            raise TokenizerError(err.value.decode(errors="replace"))
        return cls(handle, lib)

    def close(self):
        if getattr(self, "handle", None):
            self.lib.wsp_tokenizer_close(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def size(self) -> int:
        return self.lib.wsp_tokenizer_size(self.handle)

    def is_special(self, token: int) -> bool:
        return bool(self.lib.wsp_tokenizer_is_special(self.handle, token))

    def token_for_text(self, text) -> int:
        data = text.encode() if isinstance(text, str) else bytes(text)
        return self.lib.wsp_tokenizer_token_for_text(self.handle, data, len(data))

    def encode(self, text) -> List[int]:
        data = text.encode() if isinstance(text, str) else bytes(text)
        count = ctypes.c_int()
        capacity = 4 * len(data) + 16
        ids = (ctypes.c_int * capacity)()
        status = self.lib.wsp_tokenizer_encode(self.handle, data, len(data), ids, capacity, ctypes.byref(count))
        if status != N.WSP_OK:
            raise TokenizerError(f"wsp_tokenizer_encode failed with {status}")
        return list(ids[:count.value])

    def _decode(self, tokens: Sequence[int], keep: int) -> bytes:
        ids = (ctypes.c_int * max(1, len(tokens)))(*tokens)
        length = ctypes.c_int()
        capacity = 64
        while True:
            buf = ctypes.create_string_buffer(capacity)
            status = self.lib.wsp_tokenizer_decode(self.handle, ids, len(tokens), keep, buf, capacity,
                                                   ctypes.byref(length))
            if status == N.WSP_ERR_CAPACITY:
                capacity = length.value + 1
                continue
            if status != N.WSP_OK:
                raise TokenizerError(f"wsp_tokenizer_decode failed with {status}")
            return buf.raw[:length.value]

    def decode_bytes(self, tokens: Sequence[int]) -> bytes:
        return self._decode(tokens, 0)

    def decode(self, tokens: Sequence[int]) -> str:
        return self._decode(tokens, 0).decode("utf-8", errors="replace")

    def decode_keeping_special_tokens(self, tokens: Sequence[int]) -> str:
        return self._decode(tokens, 1).decode("utf-8", errors="replace")
