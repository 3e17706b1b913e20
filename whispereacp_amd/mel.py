"""Python face of the gfx950 mel front end (include/wsp_hip.h wsp_mel_*): the
reference's WSP::MelSpectrogram (Mel/MelSpectrogram.h:12-65) — built for one
MelShape, encode() turns samples and a filterbank into the normalised
[mel_count, frame_count] log-mel."""

from __future__ import annotations

import ctypes

import torch

from . import _native as N
from .decoder import _raise, current_stream, ptr
from .synthetic import MelShape


class MelSpectrogram:
    def __init__(self, shape: MelShape = MelShape(), device: int = 0):
        self.lib = N.load()
        self.shape = shape
        self._cshape = N.wsp_mel_shape(shape.sample_count, shape.fft_length, shape.hop_length, shape.frame_count,
                                       shape.mel_count)
        handle = ctypes.c_void_p()
        status = self.lib.wsp_mel_create(ctypes.byref(self._cshape), device, current_stream(), ctypes.byref(handle))
        if status != N.WSP_OK:
            _raise(N.WSP_KIND_NONE, f"wsp_mel_create failed with {status}", status)
        self.handle = handle

    def close(self):
        if getattr(self, "handle", None):
            self.lib.wsp_mel_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def encode(self, samples: torch.Tensor, filters: torch.Tensor, output: torch.Tensor) -> None:
        status = self.lib.wsp_mel_encode(self.handle, ptr(samples), ptr(filters), ptr(output))
        if status != N.WSP_OK:
            _raise(N.WSP_KIND_NONE, self.lib.wsp_mel_last_error(self.handle).decode(), status)
