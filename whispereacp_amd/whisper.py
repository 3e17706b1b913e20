"""Python face of Whisper end to end (include/wsp_decoder.h wsp_whisper_*): the
reference's WSP::Whisper (Whisper/Whisper.h:144-560) on the gfx950 kernels —
load() reads a HuggingFace Whisper directory (config.json,
preprocessor_config.json, tokenizer.json, model.safetensors) without touching
the GPU, prepare() builds the mel front end, the encoder and the greedy
decoder on the device, and transcribe() runs one 30 s window of samples to the
transcript's tokens."""

from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence, Tuple

import numpy as np

from . import _native as N
from .decoder import _raise, current_stream


class Whisper:
    audio_context_tile = 64
    audio_context_floor = 448
    default_audio_context_margin = 2.5

    def __init__(self):
        self.lib = N.load()
        handle = ctypes.c_void_p()
        status = self.lib.wsp_whisper_create(ctypes.byref(handle))
        if status != N.WSP_OK:
            raise MemoryError("wsp_whisper_create failed")
        self.handle = handle

    def close(self):
        if getattr(self, "handle", None):
            self.lib.wsp_whisper_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def _check(self, status: int):
        if status != N.WSP_OK:
            _raise(self.lib.wsp_whisper_last_error_kind(self.handle),
                   self.lib.wsp_whisper_last_error(self.handle).decode(errors="replace"), status)

    # -- load and prepare --------------------------------------------------
    def load(self, model_directory: str) -> "Whisper":
        self._check(self.lib.wsp_whisper_load(self.handle, model_directory.encode()))
        return self

    def load_files(self, config_json: str, preprocessor_json: str, tokenizer_json: str,
                   weights_path: str) -> "Whisper":
        self._check(self.lib.wsp_whisper_load_files(self.handle, config_json.encode(), preprocessor_json.encode(),
                                                    tokenizer_json.encode(), weights_path.encode()))
        return self

    def set_packs_weights(self, pack: bool):
        self._check(self.lib.wsp_whisper_set_packs_weights(self.handle, 1 if pack else 0))

    def prepare(self, device: int = 0) -> "Whisper":
        self._check(self.lib.wsp_whisper_prepare(self.handle, device, current_stream()))
        return self

    # -- generation config -------------------------------------------------
    def prompt(self) -> List[int]:
        count = ctypes.c_int(0)
        out = (ctypes.c_int * 16)()
        self._check(self.lib.wsp_whisper_prompt(self.handle, out, 16, ctypes.byref(count)))
        return list(out[:count.value])

    def masks(self, vocabulary_size: int) -> Tuple[np.ndarray, np.ndarray]:
        first = np.zeros(vocabulary_size, dtype=np.float32)
        later = np.zeros(vocabulary_size, dtype=np.float32)
        self._check(self.lib.wsp_whisper_masks(self.handle, first.ctypes.data, later.ctypes.data, vocabulary_size))
        return first, later

    def end_of_text(self) -> int:
        out = ctypes.c_int(0)
        self._check(self.lib.wsp_whisper_end_of_text(self.handle, ctypes.byref(out)))
        return out.value

    @property
    def maximum_tokens(self) -> int:
        out = ctypes.c_int(0)
        self._check(self.lib.wsp_whisper_maximum_tokens(self.handle, ctypes.byref(out)))
        return out.value

    def set_maximum_tokens(self, count: int):
        self._check(self.lib.wsp_whisper_set_maximum_tokens(self.handle, count))

    def set_audio_context(self, positions: int):
        self._check(self.lib.wsp_whisper_set_audio_context(self.handle, positions))

    def audio_context_for_samples(self, sample_count: int,
                                  margin_seconds: float = default_audio_context_margin) -> int:
        out = ctypes.c_int(0)
        self._check(self.lib.wsp_whisper_audio_context_for_samples(self.handle, sample_count, margin_seconds,
                                                                   ctypes.byref(out)))
        return out.value

    # -- runs --------------------------------------------------------------
    def transcribe(self, samples: Sequence[float], capacity: int = 448) -> List[int]:
        data = np.ascontiguousarray(samples, dtype=np.float32)
        out = (ctypes.c_int * max(1, capacity))()
        count = ctypes.c_int(0)
        self._check(self.lib.wsp_whisper_transcribe(self.handle, data.ctypes.data if data.size else None,
                                                    int(data.size), out, capacity, ctypes.byref(count)))
        return list(out[:count.value])

    def text_for_tokens(self, tokens: Sequence[int]) -> str:
        ids = (ctypes.c_int * max(1, len(tokens)))(*tokens)
        capacity = 64 + 64 * len(tokens)
        text = ctypes.create_string_buffer(capacity)
        length = ctypes.c_int(0)
        self._check(self.lib.wsp_whisper_text_for_tokens(self.handle, ids, len(tokens), text, capacity,
                                                         ctypes.byref(length)))
        return text.raw[:length.value].decode("utf-8", errors="replace")

    def transcribe_text(self, samples: Sequence[float]) -> str:
        return self.text_for_tokens(self.transcribe(samples))

    def timing(self) -> Tuple[float, float, int]:
        """(mel + encoder seconds, decode seconds, steps) of the last run."""
        e, d, s = ctypes.c_double(0), ctypes.c_double(0), ctypes.c_int(0)
        self._check(self.lib.wsp_whisper_timing(self.handle, ctypes.byref(e), ctypes.byref(d), ctypes.byref(s)))
        return e.value, d.value, s.value

    def encoded_rows(self) -> Tuple[int, int, int]:
        """(device pointer, positions, width) of the last run's encoded rows."""
        p, n, w = ctypes.c_void_p(), ctypes.c_int(0), ctypes.c_int(0)
        self._check(self.lib.wsp_whisper_encoded_rows(self.handle, ctypes.byref(p), ctypes.byref(n),
                                                      ctypes.byref(w)))
        return p.value, n.value, w.value


def load(model_directory: str, device: Optional[int] = 0, pack_weights: bool = True) -> Whisper:
    """Whisper().load(dir), then prepare(device) unless device is None."""
    w = Whisper()
    w.load(model_directory)
    if device is not None:
        w.set_packs_weights(pack_weights)
        w.prepare(device)
    return w
