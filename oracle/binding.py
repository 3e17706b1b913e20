"""ctypes binding of oracle/oracle.c — TEST INFRASTRUCTURE.

The oracle restates the reference's double-precision decoder
(Tests/Decoder/Common.h:202-509). This module only marshals numpy arrays in and
out; see oracle.h for what each call restates and what pins it.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Dict, List, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")

_dp = ctypes.POINTER(ctypes.c_double)
_fp = ctypes.POINTER(ctypes.c_float)
_ip = ctypes.POINTER(ctypes.c_int)
_up = ctypes.POINTER(ctypes.c_uint32)


class _Shape(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "width", "heads", "layers", "feed_forward_width", "vocabulary_size", "max_positions",
        "cross_positions")]


class _EncoderShape(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "mel_bins", "width", "heads", "layers", "feed_forward_width", "input_frames")]


def build_oracle(force: bool = False) -> str:
    """Compile oracle.c with its Makefile (gcc) into oracle/_build/."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "all"], cwd=_HERE, check=True)
    return _LIB_PATH


def _ptr(array: np.ndarray, kind):
    return array.ctypes.data_as(kind)


class Oracle:
    def __init__(self, path: str):
        lib = ctypes.CDLL(path)
        self.lib = lib
        lib.oracle_set_threads.argtypes = [ctypes.c_int]
        lib.oracle_set_threads.restype = ctypes.c_int
        lib.oracle_layernorm.argtypes = [_dp, ctypes.c_int, ctypes.c_int, _fp, _fp, _dp]
        lib.oracle_linear.argtypes = [_dp, ctypes.c_int, ctypes.c_int, _fp, _fp, ctypes.c_int, _dp]
        lib.oracle_attention.argtypes = [_dp, ctypes.c_int, ctypes.c_int, _dp, _dp, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_int, _dp]
        lib.oracle_gelu.argtypes = [ctypes.c_double]
        lib.oracle_gelu.restype = ctypes.c_double
        lib.oracle_argmax_masked.argtypes = [_dp, _fp, ctypes.c_int]
        lib.oracle_argmax_masked.restype = ctypes.c_uint32
        lib.oracle_argmax_masked_f32.argtypes = [_fp, _fp, ctypes.c_int]
        lib.oracle_argmax_masked_f32.restype = ctypes.c_uint32
        lib.oracle_embed.argtypes = [_up, ctypes.c_int, _fp, _fp, ctypes.c_int, ctypes.c_int, _dp]
        lib.oracle_f32_to_f16_bits.argtypes = [ctypes.c_float]
        lib.oracle_f32_to_f16_bits.restype = ctypes.c_uint16
        lib.oracle_f16_bits_to_f32.argtypes = [ctypes.c_uint16]
        lib.oracle_f16_bits_to_f32.restype = ctypes.c_float
        lib.oracle_f32_to_bf16_bits.argtypes = [ctypes.c_float]
        lib.oracle_f32_to_bf16_bits.restype = ctypes.c_uint16
        lib.oracle_bf16_bits_to_f32.argtypes = [ctypes.c_uint16]
        lib.oracle_bf16_bits_to_f32.restype = ctypes.c_float
        lib.oracle_mt19937_fill.argtypes = [ctypes.c_uint32, ctypes.c_int64, _up]
        lib.oracle_decode_full.argtypes = [ctypes.POINTER(_Shape), ctypes.POINTER(_fp), _fp,
                                           ctypes.c_int, _ip, ctypes.c_int, _dp, _dp]
        lib.oracle_session_create.argtypes = [ctypes.POINTER(_Shape), ctypes.POINTER(_fp)]
        lib.oracle_session_create.restype = ctypes.c_void_p
        lib.oracle_session_destroy.argtypes = [ctypes.c_void_p]
        lib.oracle_session_begin.argtypes = [ctypes.c_void_p, _fp, ctypes.c_int]
        lib.oracle_session_step.argtypes = [ctypes.c_void_p, _ip, ctypes.c_int, _dp, _dp]
        lib.oracle_session_position.argtypes = [ctypes.c_void_p]
        lib.oracle_greedy.argtypes = [ctypes.c_void_p, _ip, ctypes.c_int, ctypes.c_int, _fp, _ip,
                                      _dp, _dp]
        lib.oracle_conv1d_output_length.argtypes = [ctypes.c_int, ctypes.c_int]
        lib.oracle_conv1d_output_length.restype = ctypes.c_int
        lib.oracle_conv1d.argtypes = [_dp, ctypes.c_int, ctypes.c_int, _fp, _fp, ctypes.c_int, ctypes.c_int,
                                      _dp]
        lib.oracle_encode.argtypes = [ctypes.POINTER(_EncoderShape), ctypes.POINTER(_fp), _fp, _dp]
        lib.oracle_mel_spectrogram.argtypes = [_fp, ctypes.c_int, _fp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int, _dp]

    # -- primitives -------------------------------------------------------
    def set_threads(self, threads: int) -> int:
        return self.lib.oracle_set_threads(int(threads))

    def layernorm(self, rows: np.ndarray, weight: np.ndarray, bias: np.ndarray) -> np.ndarray:
        rows = np.ascontiguousarray(rows, dtype=np.float64)
        r, w = rows.shape
        out = np.empty_like(rows)
        wt = np.ascontiguousarray(weight, dtype=np.float32)
        bs = np.ascontiguousarray(bias, dtype=np.float32)
        self.lib.oracle_layernorm(_ptr(rows, _dp), r, w, _ptr(wt, _fp), _ptr(bs, _fp),
                                  _ptr(out, _dp))
        return out

    def linear(self, x: np.ndarray, weight: np.ndarray, bias: Optional[np.ndarray]) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float64)
        rows, inner = x.shape
        wt = np.ascontiguousarray(weight, dtype=np.float32)
        out_w = wt.shape[0]
        out = np.empty((rows, out_w), dtype=np.float64)
        bp = None
        if bias is not None:
            bs = np.ascontiguousarray(bias, dtype=np.float32)
            bp = _ptr(bs, _fp)
        self.lib.oracle_linear(_ptr(x, _dp), rows, inner, _ptr(wt, _fp), bp, out_w,
                               _ptr(out, _dp))
        return out

    def attention(self, q: np.ndarray, k: np.ndarray, v: np.ndarray, heads: int, causal: bool,
                  first_query: int = 0) -> np.ndarray:
        q = np.ascontiguousarray(q, dtype=np.float64)
        k = np.ascontiguousarray(k, dtype=np.float64)
        v = np.ascontiguousarray(v, dtype=np.float64)
        out = np.empty_like(q)
        self.lib.oracle_attention(_ptr(q, _dp), q.shape[0], first_query, _ptr(k, _dp),
                                  _ptr(v, _dp), k.shape[0], q.shape[1], heads, int(causal),
                                  _ptr(out, _dp))
        return out

    def gelu(self, x: float) -> float:
        return self.lib.oracle_gelu(float(x))

    def argmax(self, row: np.ndarray, mask: Optional[np.ndarray] = None) -> int:
        mp = None
        if mask is not None:
            m = np.ascontiguousarray(mask, dtype=np.float32)
            mp = _ptr(m, _fp)
        if row.dtype == np.float32:
            r = np.ascontiguousarray(row)
            return int(self.lib.oracle_argmax_masked_f32(_ptr(r, _fp), mp, r.shape[0]))
        r = np.ascontiguousarray(row, dtype=np.float64)
        return int(self.lib.oracle_argmax_masked(_ptr(r, _dp), mp, r.shape[0]))

    def embed(self, tokens, token_table, position_table, first_position: int) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        tt = np.ascontiguousarray(token_table, dtype=np.float32)
        pt = np.ascontiguousarray(position_table, dtype=np.float32)
        width = tt.shape[1]
        if pt.shape[1] != width or first_position < 0 or first_position + t.shape[0] > pt.shape[0]:
            raise ValueError("embed: the position table has no row for every position")
        if t.size and int(t.max()) >= tt.shape[0]:
            raise ValueError("embed: a token id past the token table")
        out = np.empty((t.shape[0], width), dtype=np.float64)
        self.lib.oracle_embed(_ptr(t, _up), t.shape[0], _ptr(tt, _fp), _ptr(pt, _fp),
                              first_position, width, _ptr(out, _dp))
        return out

    def f32_to_f16_bits(self, x: float) -> int:
        return int(self.lib.oracle_f32_to_f16_bits(x))

    def f16_bits_to_f32(self, bits: int) -> float:
        return float(self.lib.oracle_f16_bits_to_f32(bits))

    def f32_to_bf16_bits(self, x: float) -> int:
        return int(self.lib.oracle_f32_to_bf16_bits(x))

    def bf16_bits_to_f32(self, bits: int) -> float:
        return float(self.lib.oracle_bf16_bits_to_f32(bits))

    def mt19937(self, seed: int, count: int) -> np.ndarray:
        out = np.empty(count, dtype=np.uint32)
        self.lib.oracle_mt19937_fill(seed, count, _ptr(out, _up))
        return out

    # -- the decoder ------------------------------------------------------
    @staticmethod
    def tensor_table(shape, tensors: Sequence[np.ndarray]):
        """Keep-alive list and the float* array for ``tensors`` in the
        canonical order (whispereacp_amd.synthetic.canonical_names)."""
        keep = [np.ascontiguousarray(t, dtype=np.float32) for t in tensors]
        table = (_fp * len(keep))(*[_ptr(t, _fp) for t in keep])
        return keep, table

    @staticmethod
    def c_shape(shape) -> _Shape:
        return _Shape(shape.width, shape.heads, shape.layers, shape.feed_forward_width,
                      shape.vocabulary_size, shape.max_positions, shape.cross_positions)

    def decode_full(self, shape, tensors: Sequence[np.ndarray], encoder: np.ndarray,
                    tokens: Sequence[int], encoder_rows: int = 0):
        keep, table = self.tensor_table(shape, tensors)
        enc = np.ascontiguousarray(encoder, dtype=np.float32)
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        n = toks.shape[0]
        hidden = np.empty((n, shape.width), dtype=np.float64)
        logits = np.empty((n, shape.vocabulary_size), dtype=np.float64)
        cs = self.c_shape(shape)
        status = self.lib.oracle_decode_full(ctypes.byref(cs), table, _ptr(enc, _fp),
                                             encoder_rows, _ptr(toks, _ip), n,
                                             _ptr(hidden, _dp), _ptr(logits, _dp))
        del keep
        if status != 0:
            raise ValueError("oracle_decode_full refused the inputs")
        return hidden, logits

    def session(self, shape, tensors: Sequence[np.ndarray]) -> "OracleSession":
        return OracleSession(self, shape, tensors)

    # -- the encoder ------------------------------------------------------
    def conv1d_output_length(self, length: int, stride: int) -> int:
        return int(self.lib.oracle_conv1d_output_length(length, stride))

    def conv1d(self, x: np.ndarray, weight: np.ndarray, bias: np.ndarray, stride: int) -> np.ndarray:
        """[in_channels, length] channel-major -> [out_channels, out_length]."""
        xs = np.ascontiguousarray(x, dtype=np.float64)
        w = np.ascontiguousarray(weight, dtype=np.float32)
        b = np.ascontiguousarray(bias, dtype=np.float32)
        out_channels = w.shape[0]
        out = np.empty((out_channels, self.conv1d_output_length(xs.shape[1], stride)), dtype=np.float64)
        self.lib.oracle_conv1d(_ptr(xs, _dp), xs.shape[0], xs.shape[1], _ptr(w, _fp), _ptr(b, _fp),
                               out_channels, stride, _ptr(out, _dp))
        return out

    def mel_spectrogram(self, samples: np.ndarray, filters: np.ndarray, fft_length: int, hop_length: int,
                        frame_count: int) -> np.ndarray:
        """[mel_count, frame_count] normalised log-mel (oracle_mel_spectrogram)."""
        x = np.ascontiguousarray(samples, dtype=np.float32)
        f = np.ascontiguousarray(filters, dtype=np.float32)
        out = np.empty((f.shape[0], frame_count), dtype=np.float64)
        status = self.lib.oracle_mel_spectrogram(_ptr(x, _fp), x.shape[0], _ptr(f, _fp), fft_length, hop_length,
                                                 frame_count, f.shape[0], _ptr(out, _dp))
        if status != 0:
            raise ValueError("oracle_mel_spectrogram refused the inputs")
        return out

    def encode(self, shape, tensors: Sequence[np.ndarray], mel: np.ndarray) -> np.ndarray:
        """The whole encoder (oracle_encode): ``shape`` has mel_bins, width,
        heads, layers, feed_forward_width and input_frames; ``tensors`` are in
        the canonical encoder order; ``mel`` is [mel_bins, input_frames]."""
        keep = [np.ascontiguousarray(t, dtype=np.float32) for t in tensors]
        table = (_fp * len(keep))(*[_ptr(t, _fp) for t in keep])
        m = np.ascontiguousarray(mel, dtype=np.float32)
        cs = _EncoderShape(shape.mel_bins, shape.width, shape.heads, shape.layers, shape.feed_forward_width,
                           shape.input_frames)
        positions = self.conv1d_output_length(self.conv1d_output_length(shape.input_frames, 1), 2)
        out = np.empty((positions, shape.width), dtype=np.float64)
        status = self.lib.oracle_encode(ctypes.byref(cs), table, _ptr(m, _fp), _ptr(out, _dp))
        del keep
        if status != 0:
            raise ValueError("oracle_encode refused the inputs")
        return out


class OracleSession:
    """The KV-cached oracle decoder (bitwise equal to Oracle.decode_full)."""

    def __init__(self, oracle: Oracle, shape, tensors: Sequence[np.ndarray]):
        self.oracle = oracle
        self.shape = shape
        self._keep, self._table = Oracle.tensor_table(shape, tensors)
        self._cshape = Oracle.c_shape(shape)
        self.handle = oracle.lib.oracle_session_create(ctypes.byref(self._cshape), self._table)

    def __del__(self):
        handle = getattr(self, "handle", None)
        if handle:
            self.oracle.lib.oracle_session_destroy(handle)
            self.handle = None

    def begin(self, encoder: np.ndarray, rows: int = 0) -> None:
        self._enc = np.ascontiguousarray(encoder, dtype=np.float32)
        if self.oracle.lib.oracle_session_begin(self.handle, _ptr(self._enc, _fp), rows) != 0:
            raise ValueError(f"oracle session refused {rows} cross rows")

    @property
    def position(self) -> int:
        return int(self.oracle.lib.oracle_session_position(self.handle))

    def step(self, tokens: Sequence[int]):
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        n = toks.shape[0]
        hidden = np.empty((n, self.shape.width), dtype=np.float64)
        logits = np.empty((n, self.shape.vocabulary_size), dtype=np.float64)
        status = self.oracle.lib.oracle_session_step(self.handle, _ptr(toks, _ip), n,
                                                     _ptr(hidden, _dp), _ptr(logits, _dp))
        if status != 0:
            raise ValueError("oracle session refused the step")
        return hidden, logits

    def greedy(self, prompt: Sequence[int], steps: int, mask: Optional[np.ndarray] = None):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        toks = np.empty(steps, dtype=np.int32)
        margins = np.empty(steps, dtype=np.float64)
        last = np.empty(self.shape.vocabulary_size, dtype=np.float64)
        mp = None
        if mask is not None:
            m = np.ascontiguousarray(mask, dtype=np.float32)
            mp = _ptr(m, _fp)
        status = self.oracle.lib.oracle_greedy(self.handle, _ptr(p, _ip), p.shape[0], steps, mp,
                                               _ptr(toks, _ip), _ptr(margins, _dp),
                                               _ptr(last, _dp))
        if status != 0:
            raise ValueError("oracle greedy decode refused the inputs")
        return toks, margins, last


_cached: Optional[Oracle] = None


def load_oracle() -> Oracle:
    """Load oracle/_build/liboracle.so, building it first only if it is absent."""
    global _cached
    if _cached is None:
        _cached = Oracle(build_oracle(force=False))
    return _cached


def tensors_in_order(decoder_file: Dict, names: List[str]) -> List[np.ndarray]:
    """Widened float32 arrays of ``decoder_file`` in ``names`` order."""
    return [decoder_file[n].floats() for n in names]
