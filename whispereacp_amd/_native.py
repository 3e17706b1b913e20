"""Loads the gfx950 library and declares its C ABI (include/wsp_hip.h,
include/wsp_decoder.h) for ctypes.

torch is imported first on purpose: it carries its own HIP runtime, and the
library must bind to that same runtime rather than load a second one. The
library has no CPU fallback: if it is not built, loading fails loudly.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch  # noqa: F401  (the process's one HIP runtime)

HERE = os.path.dirname(os.path.abspath(__file__))
# The in-tree build, unless WSP_LIBRARY names another build of the same sources.
LIBRARY = os.environ.get("WSP_LIBRARY") or os.path.join(HERE, "_build", "libwhispereacp_hip.so")

c_int, c_float, c_void_p, c_char_p, c_double = ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_double

WSP_OK = 0
WSP_ERR_ARGUMENT = -1
WSP_ERR_SHAPE = -2
WSP_ERR_CAPACITY = -3
WSP_ERR_HIP = -4
WSP_ERR_LOGIC = -5
WSP_ERR_DEVICE = -6

WSP_F32, WSP_F16, WSP_BF16 = 0, 1, 2
WSP_LINEAR_GELU, WSP_LINEAR_RESIDUAL = 1, 2

WSP_KIND_NONE, WSP_KIND_MODEL_ERROR, WSP_KIND_LOGIC_ERROR, WSP_KIND_INVALID_ARGUMENT, WSP_KIND_RUNTIME_ERROR = range(5)


class wsp_decoder_shape(ctypes.Structure):
    _fields_ = [(n, c_int) for n in ("width", "heads", "layers", "feed_forward_width", "vocabulary_size",
                                     "max_positions", "cross_positions")]


class wsp_tensor_entry(ctypes.Structure):
    _fields_ = [("name", c_char_p), ("dtype", c_char_p), ("rank", c_int),
                ("extents", ctypes.POINTER(ctypes.c_longlong)), ("data", c_void_p)]


class wsp_layer_tensors(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in (
        "self_norm_w", "self_norm_b", "self_qkv_w", "self_qkv_b", "self_out_w", "self_out_b", "cross_norm_w",
        "cross_norm_b", "cross_q_w", "cross_q_b", "cross_out_w", "cross_out_b", "final_norm_w", "final_norm_b",
        "fc1_w", "fc1_b", "fc2_w", "fc2_b", "self_keys", "self_values", "cross_keys", "cross_values")]


class wsp_decoder_tensors(ctypes.Structure):
    _fields_ = [("wdtype", c_int), ("token_embedding", c_void_p), ("logits_weight", c_void_p),
                ("logits_wdtype", c_int), ("position_embedding", c_void_p), ("final_norm_w", c_void_p),
                ("final_norm_b", c_void_p), ("layers", ctypes.POINTER(wsp_layer_tensors))]


class wsp_cross_tensors(ctypes.Structure):
    _fields_ = [("key_w", c_void_p), ("value_w", c_void_p), ("value_b", c_void_p)]


class wsp_encoder_shape(ctypes.Structure):
    _fields_ = [(n, c_int) for n in ("mel_bins", "width", "heads", "layers", "feed_forward_width", "input_frames")]


class wsp_encoder_layer_tensors(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in (
        "attention_norm_w", "attention_norm_b", "q_w", "q_b", "k_w", "v_w", "v_b", "out_w", "out_b",
        "final_norm_w", "final_norm_b", "fc1_w", "fc1_b", "fc2_w", "fc2_b")] + [
        (n, c_float) for n in ("q_scale", "k_scale", "v_scale", "out_scale", "fc1_scale", "fc2_scale")]


class wsp_encoder_tensors(ctypes.Structure):
    _fields_ = [("wdtype", c_int)] + [(n, c_void_p) for n in (
        "conv1_w", "conv1_b", "conv2_w", "conv2_b", "positions", "final_norm_w", "final_norm_b")] + [
        ("layers", ctypes.POINTER(wsp_encoder_layer_tensors))]


class wsp_mel_shape(ctypes.Structure):
    _fields_ = [(n, c_int) for n in ("sample_count", "fft_length", "hop_length", "frame_count", "mel_count")]


class wsp_special_tokens(ctypes.Structure):
    _fields_ = [(name, c_int) for name in ("end_of_text", "start_of_transcript", "start_of_previous",
                                           "start_of_language_model", "translate", "transcribe", "no_timestamps",
                                           "no_speech", "first_timestamp", "timestamp_count")] + [
        ("timestamp_interval", c_float), ("language_count", c_int), ("english", c_int)]


# name -> (restype, argtypes)
SIGNATURES = {
    "wsp_hip_ctx_create": (c_int, [ctypes.POINTER(wsp_decoder_shape), c_int, c_void_p, ctypes.POINTER(c_void_p)]),
    "wsp_hip_ctx_destroy": (None, [c_void_p]),
    "wsp_hip_last_error": (c_char_p, [c_void_p]),
    "wsp_hip_stream": (c_void_p, [c_void_p]),
    "wsp_hip_linear": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_int, c_void_p, c_void_p, c_int, c_int]),
    "wsp_hip_layernorm": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_float]),
    "wsp_hip_embed": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p, c_int]),
    "wsp_hip_attention": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                  c_float, c_void_p]),
    "wsp_hip_attention_static": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_float,
                                         c_void_p, c_void_p, ctypes.c_char_p, c_int]),
    "wsp_hip_argmax": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "wsp_hip_project_cross_kv": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int,
                                         c_void_p, c_void_p]),
    "wsp_hip_decoder_step": (c_int, [c_void_p, ctypes.POINTER(wsp_decoder_tensors), c_void_p, c_int, c_int,
                                     c_void_p, c_void_p, c_void_p, c_void_p]),
    "wsp_hip_decoder_step_tokens": (c_int, [c_void_p, ctypes.POINTER(wsp_decoder_tensors), c_void_p, c_int, c_int,
                                            c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
    "wsp_hip_step_persistent": (c_int, [c_void_p]),
    "wsp_hip_device_status": (c_int, [c_void_p, ctypes.POINTER(c_int), c_int]),
    "wsp_hip_device_status_copy": (c_int, [c_void_p, ctypes.POINTER(c_int)]),
    "wsp_hip_step_report": (c_int, [c_void_p, c_void_p, c_void_p]),
    "wsp_hip_step_report_next": (c_int, [c_void_p, c_void_p]),
    "wsp_hip_raise_device_status": (c_int, [c_void_p]),
    "wsp_decoder_create": (c_int, [ctypes.POINTER(wsp_decoder_shape), ctypes.POINTER(wsp_tensor_entry), c_int,
                                   c_int, c_int, c_void_p, ctypes.POINTER(c_void_p)]),
    "wsp_decoder_destroy": (None, [c_void_p]),
    "wsp_decoder_last_error": (c_char_p, [c_void_p]),
    "wsp_decoder_last_error_kind": (c_int, [c_void_p]),
    "wsp_decoder_begin_sequence": (c_int, [c_void_p, c_void_p, c_int]),
    "wsp_decoder_step": (c_int, [c_void_p, c_void_p, c_int, c_void_p]),
    "wsp_decoder_step_and_sample": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "wsp_decoder_position": (c_int, [c_void_p]),
    "wsp_decoder_cross_positions": (c_int, [c_void_p]),
    "wsp_decoder_hidden_states": (c_void_p, [c_void_p]),
    "wsp_decoder_set_fused": (c_int, [c_void_p, c_int]),
    "wsp_decoder_uses_fused": (c_int, [c_void_p]),
    "wsp_decoder_step_persistent": (c_int, [c_void_p]),
    "wsp_decoder_device_status": (c_int, [c_void_p, ctypes.POINTER(c_int), c_int]),
    "wsp_decoder_raise_device_status": (c_int, [c_void_p]),
    "wsp_decoder_argmax": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "wsp_decoder_greedy": (c_int, [c_void_p, c_void_p, c_int, ctypes.POINTER(c_int), c_int, c_int, c_int, c_void_p,
                                   c_void_p, ctypes.POINTER(c_int), c_int, ctypes.POINTER(c_int),
                                   ctypes.POINTER(c_double)]),
    "wsp_batch_create": (c_int, [ctypes.POINTER(wsp_decoder_shape), c_int, c_int, c_int, c_int, c_void_p,
                                 ctypes.POINTER(c_void_p)]),
    "wsp_batch_destroy": (None, [c_void_p]),
    "wsp_batch_last_error": (c_char_p, [c_void_p]),
    "wsp_batch_product_storage": (c_int, [c_void_p]),
    "wsp_batch_position": (c_int, [c_void_p]),
    "wsp_batch_cross_rows": (c_int, [c_void_p]),
    "wsp_batch_begin": (c_int, [c_void_p, ctypes.POINTER(wsp_cross_tensors), c_int, c_void_p, c_int]),
    "wsp_batch_step": (c_int, [c_void_p, ctypes.POINTER(wsp_decoder_tensors), c_void_p, c_int, c_void_p, c_void_p,
                               c_void_p, c_void_p]),
    "wsp_batch_ring_step": (c_int, [c_void_p, ctypes.POINTER(wsp_decoder_tensors), c_void_p, c_void_p, c_void_p]),
    "wsp_batch_self_cache": (c_int, [c_void_p, c_int, ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p)]),
    "wsp_batch_cross_cache": (c_int, [c_void_p, c_int, ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p)]),
    "wsp_batch_decoder_create": (c_int, [ctypes.POINTER(wsp_decoder_shape), ctypes.POINTER(wsp_tensor_entry), c_int,
                                         c_int, c_int, c_int, c_int, c_void_p, ctypes.POINTER(c_void_p)]),
    "wsp_batch_decoder_destroy": (None, [c_void_p]),
    "wsp_batch_decoder_last_error": (c_char_p, [c_void_p]),
    "wsp_batch_decoder_last_error_kind": (c_int, [c_void_p]),
    "wsp_batch_decoder_begin": (c_int, [c_void_p, c_void_p, c_int]),
    "wsp_batch_decoder_step": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
    "wsp_batch_decoder_ring_step": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p]),
    "wsp_batch_decoder_position": (c_int, [c_void_p]),
    "wsp_batch_decoder_product_storage": (c_int, [c_void_p]),
    "wsp_batch_decoder_create_from_file": (c_int, [c_char_p, ctypes.POINTER(wsp_decoder_shape), c_int, c_int, c_int,
                                                   c_int, c_void_p, ctypes.POINTER(c_void_p)]),
    "wsp_decoder_create_from_file": (c_int, [c_char_p, ctypes.POINTER(wsp_decoder_shape), c_int, c_int, c_void_p,
                                             ctypes.POINTER(c_void_p)]),
    "wsp_safetensors_open": (c_int, [c_char_p, ctypes.POINTER(c_void_p)]),
    "wsp_safetensors_open_bytes": (c_int, [c_void_p, ctypes.c_size_t, ctypes.POINTER(c_void_p)]),
    "wsp_safetensors_close": (None, [c_void_p]),
    "wsp_safetensors_last_error": (c_char_p, [c_void_p]),
    "wsp_safetensors_count": (c_int, [c_void_p]),
    "wsp_safetensors_tensor": (c_int, [c_void_p, c_int, ctypes.POINTER(c_char_p), ctypes.POINTER(c_char_p),
                                       ctypes.POINTER(c_int), ctypes.POINTER(ctypes.c_longlong), c_int,
                                       ctypes.POINTER(ctypes.c_longlong)]),
    "wsp_safetensors_read_floats": (c_int, [c_void_p, c_char_p, c_void_p, ctypes.c_longlong]),
    "wsp_safetensors_metadata": (c_char_p, [c_void_p, c_char_p]),
    "wsp_decoding_from_config": (c_int, [c_char_p, c_void_p, c_void_p, c_int, ctypes.POINTER(c_int),
                                         ctypes.POINTER(c_int), ctypes.c_char_p, c_int]),
    "wsp_shape_from_config": (c_int, [c_char_p, c_int, ctypes.POINTER(wsp_decoder_shape), ctypes.c_char_p, c_int]),
    "wsp_special_tokens_from_file": (c_int, [c_char_p, ctypes.POINTER(wsp_special_tokens), ctypes.c_char_p, c_int]),
    "wsp_prompt_from_files": (c_int, [c_char_p, c_char_p, ctypes.POINTER(c_int), c_int, ctypes.POINTER(c_int),
                                      ctypes.c_char_p, c_int]),
    "wsp_batch_decoder_hidden_states": (c_void_p, [c_void_p]),
    "wsp_encoder_create": (c_int, [ctypes.POINTER(wsp_encoder_shape), c_int, c_void_p, ctypes.POINTER(c_void_p)]),
    "wsp_encoder_destroy": (None, [c_void_p]),
    "wsp_encoder_last_error": (c_char_p, [c_void_p]),
    "wsp_encoder_encode": (c_int, [c_void_p, ctypes.POINTER(wsp_encoder_tensors), c_void_p, c_void_p, c_int]),
    "wsp_encoder_scaled_halves": (c_int, [ctypes.POINTER(wsp_encoder_shape), c_void_p, ctypes.c_size_t, c_void_p,
                                          ctypes.POINTER(c_float)]),
    "wsp_mel_create": (c_int, [ctypes.POINTER(wsp_mel_shape), c_int, c_void_p, ctypes.POINTER(c_void_p)]),
    "wsp_mel_destroy": (None, [c_void_p]),
    "wsp_mel_last_error": (c_char_p, [c_void_p]),
    "wsp_mel_encode": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p]),
    "wsp_tokenizer_open": (c_int, [c_char_p, ctypes.POINTER(c_void_p), ctypes.c_char_p, c_int]),
    "wsp_tokenizer_open_bytes": (c_int, [c_char_p, ctypes.c_size_t, ctypes.POINTER(c_void_p), ctypes.c_char_p,
                                         c_int]),
    "wsp_tokenizer_close": (None, [c_void_p]),
    "wsp_tokenizer_size": (c_int, [c_void_p]),
    "wsp_tokenizer_is_special": (c_int, [c_void_p, c_int]),
    "wsp_tokenizer_token_for_text": (c_int, [c_void_p, c_char_p, ctypes.c_size_t]),
    "wsp_tokenizer_encode": (c_int, [c_void_p, c_char_p, ctypes.c_size_t, ctypes.POINTER(c_int), c_int,
                                     ctypes.POINTER(c_int)]),
    "wsp_tokenizer_decode": (c_int, [c_void_p, ctypes.POINTER(c_int), c_int, c_int, ctypes.c_char_p, c_int,
                                     ctypes.POINTER(c_int)]),
    "wsp_whisper_create": (c_int, [ctypes.POINTER(c_void_p)]),
    "wsp_whisper_destroy": (None, [c_void_p]),
    "wsp_whisper_last_error": (c_char_p, [c_void_p]),
    "wsp_whisper_last_error_kind": (c_int, [c_void_p]),
    "wsp_whisper_load": (c_int, [c_void_p, c_char_p]),
    "wsp_whisper_load_files": (c_int, [c_void_p, c_char_p, c_char_p, c_char_p, c_char_p]),
    "wsp_whisper_set_packs_weights": (c_int, [c_void_p, c_int]),
    "wsp_whisper_prepare": (c_int, [c_void_p, c_int, c_void_p]),
    "wsp_whisper_prompt": (c_int, [c_void_p, ctypes.POINTER(c_int), c_int, ctypes.POINTER(c_int)]),
    "wsp_whisper_masks": (c_int, [c_void_p, c_void_p, c_void_p, c_int]),
    "wsp_whisper_end_of_text": (c_int, [c_void_p, ctypes.POINTER(c_int)]),
    "wsp_whisper_set_maximum_tokens": (c_int, [c_void_p, c_int]),
    "wsp_whisper_maximum_tokens": (c_int, [c_void_p, ctypes.POINTER(c_int)]),
    "wsp_whisper_set_audio_context": (c_int, [c_void_p, c_int]),
    "wsp_whisper_audio_context_for_samples": (c_int, [c_void_p, c_int, ctypes.c_double, ctypes.POINTER(c_int)]),
    "wsp_whisper_transcribe": (c_int, [c_void_p, c_void_p, c_int, ctypes.POINTER(c_int), c_int,
                                       ctypes.POINTER(c_int)]),
    "wsp_whisper_text_for_tokens": (c_int, [c_void_p, ctypes.POINTER(c_int), c_int, ctypes.c_char_p, c_int,
                                            ctypes.POINTER(c_int)]),
    "wsp_whisper_timing": (c_int, [c_void_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                   ctypes.POINTER(c_int)]),
    "wsp_whisper_encoded_rows": (c_int, [c_void_p, ctypes.POINTER(c_void_p), ctypes.POINTER(c_int),
                                         ctypes.POINTER(c_int)]),
}

_lib: Optional[ctypes.CDLL] = None


def library_path() -> str:
    return LIBRARY


def load() -> ctypes.CDLL:
    """The library, with every entry point declared. Raises if not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            raise RuntimeError(f"the gfx950 library is not built ({LIBRARY}); run __graft_entry__.build()")
        lib = ctypes.CDLL(LIBRARY)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib
