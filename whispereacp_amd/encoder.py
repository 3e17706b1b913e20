"""Python face of the gfx950 encoder (include/wsp_hip.h wsp_encoder_*): the
reference's WSP::Encoder (Encoder/Encoder.h:8-71) — built for one
EncoderShape, encode() runs a mel through the convolutions, the transformer
layers and the final LayerNorm into [positions, width] rows.

Weights stay on the device as the file stores them for the projections
(F32, F16 or BF16) and widened to fp32 for everything else, as the
reference's EncoderWeights does (Encoder/EncoderWeights.h:44-52). BF16
projections are held as exact fp16 multiples w·2^k with their scale
(wsp_encoder_scaled_halves) when every value narrows exactly and the
shape's products run over pre-split inputs: the products then read two
fp16 parts of their input instead of three bf16 ones.
"""

from __future__ import annotations

import ctypes
from typing import Dict, Optional

import numpy as np
import torch

from . import _native as N
from .decoder import ModelError, _raise, current_stream, ptr
from .synthetic import DecoderFile, ENCODER_LAYER_SUFFIXES, ENCODER_MODEL_NAMES, EncoderShape, encoder_layer_name

_DTYPES = {"F32": N.WSP_F32, "F16": N.WSP_F16, "BF16": N.WSP_BF16}


def _device_tensor(stored, widen: bool) -> torch.Tensor:
    data = stored.floats() if widen else np.ascontiguousarray(stored.data)
    return torch.from_numpy(np.ascontiguousarray(data)).cuda()


_SCALES = {"self_attn.q_proj.weight": "q_scale", "self_attn.k_proj.weight": "k_scale",
           "self_attn.v_proj.weight": "v_scale", "self_attn.out_proj.weight": "out_scale",
           "fc1.weight": "fc1_scale", "fc2.weight": "fc2_scale"}


def _scaled_halves(lib, cshape, stored) -> Optional[tuple]:
    """(fp16 array, scale) for a BF16 projection, or None when it does not
    narrow exactly (or the shape takes no scaled projections)."""
    bits = np.ascontiguousarray(stored.data, dtype=np.uint16)
    halves = np.empty(bits.shape, dtype=np.float16)
    scale = ctypes.c_float()
    status = lib.wsp_encoder_scaled_halves(ctypes.byref(cshape), bits.ctypes.data, bits.size, halves.ctypes.data,
                                           ctypes.byref(scale))
    if status in (N.WSP_ERR_LOGIC, N.WSP_ERR_SHAPE):
        return None
    if status != N.WSP_OK:
        _raise(N.WSP_KIND_NONE, f"wsp_encoder_scaled_halves failed with {status}", status)
    return halves, scale.value


class EncoderWeights:
    """Encoder/EncoderWeights.h:70-93 over a (synthetic or loaded) tensor
    dictionary keyed by the HuggingFace names. scaled_halves=False keeps BF16
    projections as stored."""

    def __init__(self, shape: EncoderShape, file: DecoderFile, scaled_halves: bool = True):
        self.shape = shape
        projections = [file[encoder_layer_name(layer, s)] for layer in range(shape.layers)
                       for s in ENCODER_LAYER_SUFFIXES if s.endswith("proj.weight") or s.startswith("fc")
                       and s.endswith("weight")]
        dtypes = {t.dtype for t in projections}
        if len(dtypes) > 1:
            raise ValueError(f"the encoder's projections mix storages {sorted(dtypes)}")
        self.dtype = dtypes.pop() if dtypes else "F32"
        self.stored_dtype = self.dtype
        # BF16 projections as exact fp16 multiples, all or none.
        scaled: Dict[str, tuple] = {}
        if self.dtype == "BF16" and scaled_halves and shape.layers > 0:
            lib = N.load()
            cshape = N.wsp_encoder_shape(shape.mel_bins, shape.width, shape.heads, shape.layers,
                                         shape.feed_forward_width, shape.input_frames)
            for name in [encoder_layer_name(layer, suffix) for layer in range(shape.layers) for suffix in _SCALES]:
                converted = _scaled_halves(lib, cshape, file[name])
                if converted is None:
                    scaled = {}
                    break
                scaled[name] = converted
            if scaled:
                self.dtype = "F16"
        self._keep: Dict[str, torch.Tensor] = {}
        for name in ENCODER_MODEL_NAMES:
            self._keep[name] = _device_tensor(file[name], True)
        for layer in range(shape.layers):
            for suffix in ENCODER_LAYER_SUFFIXES:
                name = encoder_layer_name(layer, suffix)
                projection = suffix.endswith("proj.weight") or suffix in ("fc1.weight", "fc2.weight")
                if name in scaled:
                    self._keep[name] = torch.from_numpy(scaled[name][0]).cuda()
                else:
                    self._keep[name] = _device_tensor(file[name], not projection)
        self._layers = (N.wsp_encoder_layer_tensors * max(1, shape.layers))()
        fields = ["attention_norm_w", "attention_norm_b", "q_w", "q_b", "k_w", "v_w", "v_b", "out_w", "out_b",
                  "final_norm_w", "final_norm_b", "fc1_w", "fc1_b", "fc2_w", "fc2_b"]
        for layer in range(shape.layers):
            values = [self._keep[encoder_layer_name(layer, s)].data_ptr() for s in ENCODER_LAYER_SUFFIXES]
            entry = dict(zip(fields, values))
            for suffix, field in _SCALES.items():
                name = encoder_layer_name(layer, suffix)
                entry[field] = scaled[name][1] if name in scaled else 1.0
            self._layers[layer] = N.wsp_encoder_layer_tensors(**entry)
        k = self._keep
        self.table = N.wsp_encoder_tensors(
            _DTYPES[self.dtype], ptr(k[ENCODER_MODEL_NAMES[0]]), ptr(k[ENCODER_MODEL_NAMES[1]]),
            ptr(k[ENCODER_MODEL_NAMES[2]]), ptr(k[ENCODER_MODEL_NAMES[3]]), ptr(k[ENCODER_MODEL_NAMES[4]]),
            ptr(k[ENCODER_MODEL_NAMES[5]]), ptr(k[ENCODER_MODEL_NAMES[6]]), self._layers)
        table_rows = k[ENCODER_MODEL_NAMES[4]].shape[0]
        if table_rows < shape.positions():
            raise ModelError(f"tensor 'model.encoder.embed_positions.weight' carries {table_rows} positions, "
                             f"and this run needs {shape.positions()}")


class Encoder:
    """Encoder/Encoder.h:28-62: prepare() sizes everything for the shape's
    window (here, at construction); encode() only launches."""

    def __init__(self, shape: EncoderShape, device: int = 0):
        self.lib = N.load()
        self.shape = shape
        self._cshape = N.wsp_encoder_shape(shape.mel_bins, shape.width, shape.heads, shape.layers,
                                           shape.feed_forward_width, shape.input_frames)
        handle = ctypes.c_void_p()
        status = self.lib.wsp_encoder_create(ctypes.byref(self._cshape), device, current_stream(),
                                             ctypes.byref(handle))
        if status != N.WSP_OK:
            _raise(N.WSP_KIND_NONE, f"wsp_encoder_create failed with {status}", status)
        self.handle = handle

    def close(self):
        if getattr(self, "handle", None):
            self.lib.wsp_encoder_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def encode(self, mel: torch.Tensor, weights: EncoderWeights, output: torch.Tensor,
               position_count: int = 0) -> None:
        """mel: device [mel_bins, input_frames] float32; output: device, at least
        position_count (or positions()) rows of width floats."""
        if weights.shape != self.shape:
            raise ModelError("the weights were loaded against a different encoder shape than this encoder was "
                             "built for")
        status = self.lib.wsp_encoder_encode(self.handle, ctypes.byref(weights.table), ptr(mel), ptr(output),
                                             position_count)
        if status != N.WSP_OK:
            message = self.lib.wsp_encoder_last_error(self.handle).decode()
            # Encoder/Encoder.cpp:159-163: a context past the window is a ModelError.
            _raise(N.WSP_KIND_MODEL_ERROR if status == N.WSP_ERR_SHAPE else N.WSP_KIND_NONE, message, status)
