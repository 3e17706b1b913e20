"""Python face of the gfx950 decoder: the reference's WSP::Decoder / Argmax /
greedy-loop surface (Decoder/Decoder.h:49-148, Kernels/Argmax.h:221-248,
Whisper/Whisper.cpp:1361-1443) over the C binding in include/wsp_decoder.h,
plus a kernel context over include/wsp_hip.h for the per-op calls.

Device buffers are torch tensors on the current HIP device, passed by pointer;
every call records on torch's current stream, so torch work and the
library's kernels are ordered by that one stream. Errors come back as the
reference's exceptions: ModelError, logic_error -> RuntimeError subclass
LogicError, invalid_argument -> ValueError.
"""

from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _native as N
from .synthetic import DecoderFile, DecoderShape


class ModelError(RuntimeError):
    """Model/ModelError.h:16-20."""


class LogicError(RuntimeError):
    """std::logic_error from the decoder surface."""


def _raise(kind: int, message: str, code: int):
    if kind == N.WSP_KIND_MODEL_ERROR:
        raise ModelError(message)
    if kind == N.WSP_KIND_LOGIC_ERROR or code == N.WSP_ERR_LOGIC:
        raise LogicError(message)
    if kind == N.WSP_KIND_INVALID_ARGUMENT or code in (N.WSP_ERR_ARGUMENT, N.WSP_ERR_SHAPE,
                                                       N.WSP_ERR_CAPACITY):
        raise ValueError(message)
    raise RuntimeError(message)


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def current_stream() -> Optional[int]:
    """torch's current stream (a hipStream_t), or the default stream where
    there is no device to ask."""
    if not torch.cuda.is_available():
        return None
    return torch.cuda.current_stream().cuda_stream


def c_shape(shape: DecoderShape) -> N.wsp_decoder_shape:
    return N.wsp_decoder_shape(*shape.as_tuple())


class KernelContext:
    """A wsp_hip_ctx: the per-op kernels of include/wsp_hip.h."""

    def __init__(self, shape: DecoderShape, device: int = 0):
        self.lib = N.load()
        self.shape = shape
        handle = ctypes.c_void_p()
        self._cshape = c_shape(shape)
        status = self.lib.wsp_hip_ctx_create(ctypes.byref(self._cshape), device, current_stream(),
                                             ctypes.byref(handle))
        if status != N.WSP_OK:
            raise RuntimeError(f"wsp_hip_ctx_create failed with {status}")
        self.handle = handle

    def close(self):
        if getattr(self, "handle", None):
            self.lib.wsp_hip_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def _check(self, status: int):
        if status != N.WSP_OK:
            _raise(N.WSP_KIND_NONE, self.lib.wsp_hip_last_error(self.handle).decode(), status)

    def linear(self, x, rows, inner, weight, wdtype, bias, y, out, flags=0):
        self._check(self.lib.wsp_hip_linear(self.handle, ptr(x), rows, inner, ptr(weight), wdtype, ptr(bias),
                                            ptr(y), out, flags))

    def layernorm(self, x, gamma, beta, y, rows, width, eps=1e-5):
        self._check(self.lib.wsp_hip_layernorm(self.handle, ptr(x), ptr(gamma), ptr(beta), ptr(y), rows, width,
                                               eps))

    def embed(self, tokens, count, token_table, position_table, first, y, width):
        self._check(self.lib.wsp_hip_embed(self.handle, ptr(tokens), count, ptr(token_table),
                                           ptr(position_table), first, ptr(y), width))

    def attention(self, q, q_count, keys, values, k_count, width, heads, causal, scale, out):
        self._check(self.lib.wsp_hip_attention(self.handle, ptr(q), q_count, ptr(keys), ptr(values), k_count,
                                               width, heads, int(causal), scale, ptr(out)))

    def argmax(self, logits, rows, row_length, mask, out):
        self._check(self.lib.wsp_hip_argmax(self.handle, ptr(logits), rows, row_length, ptr(mask), ptr(out)))

    def project_cross_kv(self, x, rows, width, wk, wv, bv, wdtype, k_out, v_out):
        self._check(self.lib.wsp_hip_project_cross_kv(self.handle, ptr(x), rows, width, ptr(wk), ptr(wv),
                                                      ptr(bv), wdtype, ptr(k_out), ptr(v_out)))


def tensor_entries(decoder_file: DecoderFile):
    """wsp_tensor_entry array (plus keep-alive objects) for a decoder file."""
    keep: List[object] = []
    entries = (N.wsp_tensor_entry * len(decoder_file))()
    for i, (name, t) in enumerate(decoder_file.items()):
        data = np.ascontiguousarray(t.data)
        extents = (ctypes.c_longlong * len(t.extents))(*t.extents)
        name_b, dtype_b = name.encode(), t.dtype.encode()
        keep += [data, extents, name_b, dtype_b]
        entries[i] = N.wsp_tensor_entry(name_b, dtype_b, len(t.extents), extents, data.ctypes.data)
    return entries, keep


class Decoder:
    """DecoderWeights + Decoder + Argmax over the gfx950 library
    (include/wsp_decoder.h)."""

    def __init__(self, shape: DecoderShape, decoder_file: Optional[DecoderFile] = None, packing: str = "Float",
                 device: int = 0, path: Optional[str] = None):
        """From the tensors of decoder_file, or of the safetensors file at path."""
        self.lib = N.load()
        self.shape = shape
        self._cshape = c_shape(shape)
        handle = ctypes.c_void_p()
        pack = 1 if packing == "ExactHalf" else 0
        if path is not None:
            status = self.lib.wsp_decoder_create_from_file(path.encode(), ctypes.byref(self._cshape), pack, device,
                                                           current_stream(), ctypes.byref(handle))
        else:
            entries, keep = tensor_entries(decoder_file)
            status = self.lib.wsp_decoder_create(ctypes.byref(self._cshape), entries, len(decoder_file), pack,
                                                 device, current_stream(), ctypes.byref(handle))
            del keep
        self.handle = handle
        if status != N.WSP_OK:
            message = self.lib.wsp_decoder_last_error(handle).decode() if handle else "create failed"
            kind = self.lib.wsp_decoder_last_error_kind(handle) if handle else N.WSP_KIND_NONE
            self.close()
            _raise(kind, message, status)

    def close(self):
        if getattr(self, "handle", None):
            self.lib.wsp_decoder_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def _check(self, status: int):
        if status != N.WSP_OK:
            _raise(self.lib.wsp_decoder_last_error_kind(self.handle),
                   self.lib.wsp_decoder_last_error(self.handle).decode(), status)

    def begin_sequence(self, encoder_rows: torch.Tensor, cross_position_count: int = 0):
        self._check(self.lib.wsp_decoder_begin_sequence(self.handle, ptr(encoder_rows), cross_position_count))

    def step(self, tokens: torch.Tensor, count: int, logits: torch.Tensor):
        self._check(self.lib.wsp_decoder_step(self.handle, ptr(tokens), count, ptr(logits)))

    def step_and_sample(self, token: torch.Tensor, logits: torch.Tensor, mask: Optional[torch.Tensor],
                        slot: torch.Tensor):
        self._check(self.lib.wsp_decoder_step_and_sample(self.handle, ptr(token), ptr(logits), ptr(mask),
                                                         ptr(slot)))

    @property
    def position(self) -> int:
        return self.lib.wsp_decoder_position(self.handle)

    @property
    def cross_positions(self) -> int:
        return self.lib.wsp_decoder_cross_positions(self.handle)

    def hidden_states_pointer(self) -> int:
        return self.lib.wsp_decoder_hidden_states(self.handle)

    def read_hidden(self, rows: int) -> np.ndarray:
        """The last step's hidden rows, copied to the host."""
        out = torch.empty((rows, self.shape.width), dtype=torch.float32, device="cuda")
        copy_device(out, self.hidden_states_pointer(), rows * self.shape.width * 4)
        torch.cuda.synchronize()
        return out.cpu().numpy()

    def set_fused(self, enabled: bool):
        self._check(self.lib.wsp_decoder_set_fused(self.handle, int(enabled)))

    @property
    def uses_fused(self) -> bool:
        return bool(self.lib.wsp_decoder_uses_fused(self.handle))

    @property
    def uses_persistent_step(self) -> bool:
        """Whether fused single-token steps run as the one persistent launch."""
        return bool(self.lib.wsp_decoder_step_persistent(self.handle))

    def device_status(self, clear: bool = False) -> int:
        """Waits for the stream; 0 when every persistent step completed its
        hand-overs, 1 when its watchdog cut a step short."""
        status = ctypes.c_int(0)
        self._check(self.lib.wsp_decoder_device_status(self.handle, ctypes.byref(status), int(clear)))
        return status.value

    def raise_device_status(self):
        """Sets the watchdog word as a timed-out wait would (later steps leave
        early and greedy() raises until it is cleared)."""
        self._check(self.lib.wsp_decoder_raise_device_status(self.handle))

    def argmax(self, logits: torch.Tensor, rows: int, row_length: int, mask: Optional[torch.Tensor],
               out: torch.Tensor):
        self._check(self.lib.wsp_decoder_argmax(self.handle, ptr(logits), rows, row_length, ptr(mask), ptr(out)))

    def greedy(self, encoder_rows: torch.Tensor, prompt: Sequence[int], maximum_tokens: int,
               end_of_text: int = -1, first_mask: Optional[torch.Tensor] = None,
               later_mask: Optional[torch.Tensor] = None, cross_position_count: int = 0
               ) -> Tuple[List[int], float]:
        p = (ctypes.c_int * len(prompt))(*prompt)
        out = (ctypes.c_int * max(1, maximum_tokens))()
        count = ctypes.c_int(0)
        seconds = ctypes.c_double(0.0)
        self._check(self.lib.wsp_decoder_greedy(self.handle, ptr(encoder_rows), cross_position_count, p,
                                                len(prompt), maximum_tokens, end_of_text, ptr(first_mask),
                                                ptr(later_mask), out, maximum_tokens, ctypes.byref(count),
                                                ctypes.byref(seconds)))
        return list(out[:min(count.value, maximum_tokens)]), seconds.value


class BatchedDecoder:
    """DecoderWeights + BatchedDecoder over the gfx950 library
    (wsp_batch_decoder_* in include/wsp_decoder.h): `streams` independent
    sequences that advance together and share one weight read per step."""

    def __init__(self, shape: DecoderShape, decoder_file: Optional[DecoderFile], streams: int,
                 max_step_tokens: int = 4, packing: str = "ExactHalf", device: int = 0, path: Optional[str] = None):
        """From the tensors of decoder_file, or of the safetensors file at path."""
        self.lib = N.load()
        self.shape = shape
        self.streams = streams
        self._cshape = c_shape(shape)
        handle = ctypes.c_void_p()
        pack = 1 if packing == "ExactHalf" else 0
        if path is not None:
            status = self.lib.wsp_batch_decoder_create_from_file(path.encode(), ctypes.byref(self._cshape), pack,
                                                                 streams, max_step_tokens, device, current_stream(),
                                                                 ctypes.byref(handle))
        else:
            entries, keep = tensor_entries(decoder_file)
            status = self.lib.wsp_batch_decoder_create(ctypes.byref(self._cshape), entries, len(decoder_file), pack,
                                                       streams, max_step_tokens, device, current_stream(),
                                                       ctypes.byref(handle))
            del keep
        self.handle = handle
        if status != N.WSP_OK:
            message = self.lib.wsp_batch_decoder_last_error(handle).decode() if handle else "create failed"
            kind = self.lib.wsp_batch_decoder_last_error_kind(handle) if handle else N.WSP_KIND_NONE
            self.close()
            _raise(kind, message, status)

    def close(self):
        if getattr(self, "handle", None):
            self.lib.wsp_batch_decoder_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def _check(self, status: int):
        if status != N.WSP_OK:
            _raise(self.lib.wsp_batch_decoder_last_error_kind(self.handle),
                   self.lib.wsp_batch_decoder_last_error(self.handle).decode(), status)

    def begin(self, encoder_rows: torch.Tensor, cross_position_count: int = 0):
        """encoder_rows: device f32 [streams, rows, width]."""
        self._check(self.lib.wsp_batch_decoder_begin(self.handle, ptr(encoder_rows), cross_position_count))

    def step(self, tokens: torch.Tensor, count: int, logits: torch.Tensor, mask: Optional[torch.Tensor] = None,
             argmax_slots: Optional[torch.Tensor] = None):
        """tokens: device int32 [streams, count]; logits [streams·count, vocabulary]."""
        self._check(self.lib.wsp_batch_decoder_step(self.handle, ptr(tokens), count, ptr(logits), ptr(mask),
                                                    ptr(argmax_slots)))

    def ring_step(self, ring: torch.Tensor, logits: torch.Tensor, mask: Optional[torch.Tensor] = None):
        """ring: device int32 [max_positions + 1, streams]; reads row p (the
        position), writes row p + 1; logits [streams, vocabulary]."""
        self._check(self.lib.wsp_batch_decoder_ring_step(self.handle, ptr(ring), ptr(logits), ptr(mask)))

    @property
    def position(self) -> int:
        return self.lib.wsp_batch_decoder_position(self.handle)

    @property
    def product_storage(self) -> str:
        """"F16" or "BF16": the weight storage the step's products read (bf16
        weights are held as exact scaled fp16 when they narrow), "" before
        the first step."""
        return {N.WSP_F16: "F16", N.WSP_BF16: "BF16"}.get(self.lib.wsp_batch_decoder_product_storage(self.handle), "")

    def read_hidden(self, rows: int) -> np.ndarray:
        out = torch.empty((rows, self.shape.width), dtype=torch.float32, device="cuda")
        copy_device(out, self.lib.wsp_batch_decoder_hidden_states(self.handle), rows * self.shape.width * 4)
        torch.cuda.synchronize()
        return out.cpu().numpy()


class SafeTensorsFile:
    """A safetensors file opened by the library's reader (wsp_safetensors_*):
    mapped, validated when opened (ModelError with the reason otherwise)."""

    def __init__(self, path: Optional[str] = None, data: Optional[bytes] = None):
        self.lib = N.load()
        handle = ctypes.c_void_p()
        if path is not None:
            status = self.lib.wsp_safetensors_open(path.encode(), ctypes.byref(handle))
        else:
            self._data = bytes(data or b"")
            status = self.lib.wsp_safetensors_open_bytes(self._data, len(self._data), ctypes.byref(handle))
        self.handle = handle
        if status != N.WSP_OK:
            message = self.lib.wsp_safetensors_last_error(handle).decode() if handle else "open failed"
            self.close()
            raise ModelError(message)

    def close(self):
        if getattr(self, "handle", None):
            self.lib.wsp_safetensors_close(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def tensors(self) -> List[Tuple[str, str, Tuple[int, ...], int]]:
        """(name, dtype, shape, byte count) in name order."""
        out = []
        for i in range(self.lib.wsp_safetensors_count(self.handle)):
            name, dtype = ctypes.c_char_p(), ctypes.c_char_p()
            rank, nbytes = ctypes.c_int(), ctypes.c_longlong()
            extents = (ctypes.c_longlong * 16)()
            self.lib.wsp_safetensors_tensor(self.handle, i, ctypes.byref(name), ctypes.byref(dtype),
                                            ctypes.byref(rank), extents, 16, ctypes.byref(nbytes))
            out.append((name.value.decode(), dtype.value.decode(), tuple(extents[:rank.value]), nbytes.value))
        return out

    def read_floats(self, name: str, count: int) -> np.ndarray:
        out = np.empty(count, dtype=np.float32)
        status = self.lib.wsp_safetensors_read_floats(self.handle, name.encode(), out.ctypes.data, count)
        if status != N.WSP_OK:
            _raise(N.WSP_KIND_MODEL_ERROR if status == N.WSP_ERR_SHAPE else N.WSP_KIND_NONE,
                   self.lib.wsp_safetensors_last_error(self.handle).decode(), status)
        return out

    def metadata(self, key: str) -> Optional[str]:
        v = self.lib.wsp_safetensors_metadata(self.handle, key.encode())
        return None if v is None else v.decode()


def shape_from_config(path: str, cross_positions: int = 0) -> DecoderShape:
    """DecoderShape::fromConfig over a HuggingFace config.json."""
    lib = N.load()
    out = N.wsp_decoder_shape()
    error = ctypes.create_string_buffer(512)
    if lib.wsp_shape_from_config(path.encode(), cross_positions, ctypes.byref(out), error, 512) != N.WSP_OK:
        raise ModelError(error.value.decode())
    return DecoderShape(out.width, out.heads, out.layers, out.feed_forward_width, out.vocabulary_size,
                        out.max_positions, out.cross_positions)


def decoding_from_config(path: str, vocabulary_size: int):
    """Whisper::buildSuppressionMasks from a config.json: (first-step mask,
    later-step mask, decoder_start_token_id, eos_token_id), masks as float32
    numpy arrays (1 = suppressed), ids -1 when absent."""
    lib = N.load()
    first = np.zeros(vocabulary_size, dtype=np.float32)
    later = np.zeros(vocabulary_size, dtype=np.float32)
    start, end = ctypes.c_int(-1), ctypes.c_int(-1)
    error = ctypes.create_string_buffer(512)
    if lib.wsp_decoding_from_config(path.encode(), first.ctypes.data, later.ctypes.data, vocabulary_size,
                                    ctypes.byref(start), ctypes.byref(end), error, 512) != N.WSP_OK:
        raise ModelError(error.value.decode())
    return first, later, start.value, end.value


def special_tokens_from_file(path: str) -> Dict[str, float]:
    """WSP::SpecialTokens of a tokenizer.json (its added_tokens), by field
    name; -1 where the vocabulary names none."""
    lib = N.load()
    out = N.wsp_special_tokens()
    error = ctypes.create_string_buffer(512)
    if lib.wsp_special_tokens_from_file(path.encode(), ctypes.byref(out), error, 512) != N.WSP_OK:
        raise ModelError(error.value.decode())
    return {name: getattr(out, name) for name, _ in N.wsp_special_tokens._fields_}


def prompt_from_files(config_path: str, tokenizer_path: str) -> List[int]:
    """Whisper::buildPrompt: [decoder_start_token_id or <|startoftranscript|>,
    <|notimestamps|>] from a config.json and a tokenizer.json."""
    lib = N.load()
    out = (ctypes.c_int * 8)()
    count = ctypes.c_int(0)
    error = ctypes.create_string_buffer(512)
    if lib.wsp_prompt_from_files(config_path.encode(), tokenizer_path.encode(), out, 8, ctypes.byref(count), error,
                                 512) != N.WSP_OK:
        raise ModelError(error.value.decode())
    return list(out[:count.value])


_hip = None


def copy_device(dst: torch.Tensor, src_pointer: int, nbytes: int):
    """Stream-ordered device-to-device copy from a raw pointer into dst."""
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so.7")
        _hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                        ctypes.c_void_p]
        _hip.hipMemcpyAsync.restype = ctypes.c_int
    status = _hip.hipMemcpyAsync(dst.data_ptr(), src_pointer, nbytes, 3, current_stream())
    if status != 0:
        raise RuntimeError(f"hipMemcpyAsync failed with {status}")


def to_device(array: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(array)).cuda()


def stored_to_device(t) -> Tuple[torch.Tensor, int]:
    """A StoredTensor's bytes on the device and its wsp dtype."""
    data = np.ascontiguousarray(t.data)
    if t.dtype == "F32":
        return to_device(data.astype(np.float32)), N.WSP_F32
    if t.dtype == "F16":
        return to_device(data.view(np.int16)), N.WSP_F16
    return to_device(data.view(np.int16)), N.WSP_BF16
