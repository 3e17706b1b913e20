"""Synthetic decoder weights and encoder states: the inputs the parity tests
and the benchmark run on.

Two families, both from generators whose sequences are fixed by a standard
rather than by an implementation (std::mt19937 draws, which numpy's legacy
``RandomState(seed)`` reproduces exactly):

* the reference test-suite's own fixture weights — ``spread_values`` /
  ``shifted_values`` / ``synthetic_decoder_file`` / ``synthetic_encoder_output``
  restate Tests/Kernels/Common.h:75-88, Tests/Encoder/Common.h:148-157 and
  Tests/Decoder/Common.h:66-169, 473-488 (same seeds, same float arithmetic);
* the benchmark workloads — every projection, bias and both embeddings drawn
  N(0, 0.02) by Box-Muller over ``u = (raw + 0.5) / 2**32``, LayerNorm gamma = 1
  and beta = 0, encoder states N(0, 1), one seed per tensor counting up in the
  file's tensor order.

Stored dtypes are "F32", "F16" or "BF16"; an F16 array is numpy float16 and a
BF16 array is the uint16 bit pattern (round to nearest even from float32).
"""

from __future__ import annotations

import concurrent.futures
import dataclasses
import math
import os
from typing import Dict, List, Optional, Tuple

import numpy as np


@dataclasses.dataclass(frozen=True)
class DecoderShape:
    """Decoder/DecoderShape.h:20-83. Every extent one decoder is built against."""

    width: int
    heads: int
    layers: int
    feed_forward_width: int
    vocabulary_size: int
    max_positions: int
    cross_positions: int

    @property
    def head_width(self) -> int:
        return self.width // self.heads

    def attention_scale(self) -> float:
        """Decoder/DecoderShape.cpp:23-26: 1/sqrt(head width), in float."""
        return float(np.float32(1.0) / np.sqrt(np.float32(self.head_width)))

    def as_tuple(self) -> Tuple[int, ...]:
        return dataclasses.astuple(self)


def small_decoder_shape() -> DecoderShape:
    """Tests/Decoder/Common.h:41-54: deliberately lopsided extents."""
    return DecoderShape(8, 2, 2, 16, 24, 16, 6)


# The five workloads: the reference's CPU-runnable tiny.en shape and the four
# MI355X decode configurations (d, heads, layers, vocab, weight dtype, streams,
# single-token steps, the weights' first seed). The encoder states of stream s
# are seeded 7 + s. tiny.en takes seed 1003: with 1000 its greedy sequence
# settles on one token after five steps, with 1003 it holds seven distinct
# tokens over its 26.
WORKLOADS = {
    "tiny.en": dict(width=384, heads=6, layers=4, vocab=51864, dtype="F32", streams=1, steps=25, seed=1003),
    "base.en": dict(width=512, heads=8, layers=6, vocab=51864, dtype="F32", streams=1, steps=64, seed=1000),
    "small": dict(width=768, heads=12, layers=12, vocab=51865, dtype="F16", streams=1, steps=224, seed=1000),
    "medium": dict(width=1024, heads=16, layers=24, vocab=51865, dtype="F16", streams=16, steps=128, seed=1000),
    "large-v3": dict(width=1280, heads=20, layers=32, vocab=51866, dtype="BF16", streams=32, steps=444,
                     seed=1000),
}

# Fixed four-token start-of-transcript prefixes from the public Whisper
# vocabularies (any in-vocabulary ids serve with random weights).
SOT_PREFIX = {
    51864: [50257, 50258, 50358, 50362],
    51865: [50258, 50259, 50359, 50363],
    51866: [50258, 50259, 50360, 50364],
}


def workload_shape(name: str, cross_positions: int = 1500) -> DecoderShape:
    w = WORKLOADS[name]
    return DecoderShape(w["width"], w["heads"], w["layers"], 4 * w["width"], w["vocab"], 448,
                        cross_positions)


# ---------------------------------------------------------------------------
# tensor names (the HuggingFace names a Whisper safetensors file carries)
# ---------------------------------------------------------------------------

_ATTENTION_SUFFIXES = [
    "{norm}.weight", "{norm}.bias",
    "{attn}.q_proj.weight", "{attn}.q_proj.bias",
    "{attn}.k_proj.weight",
    "{attn}.v_proj.weight", "{attn}.v_proj.bias",
    "{attn}.out_proj.weight", "{attn}.out_proj.bias",
]

LAYER_SUFFIXES: List[str] = (
    [s.format(norm="self_attn_layer_norm", attn="self_attn") for s in _ATTENTION_SUFFIXES]
    + [s.format(norm="encoder_attn_layer_norm", attn="encoder_attn") for s in _ATTENTION_SUFFIXES]
    + ["final_layer_norm.weight", "final_layer_norm.bias", "fc1.weight", "fc1.bias", "fc2.weight",
       "fc2.bias"]
)

MODEL_NAMES = [
    "model.decoder.embed_tokens.weight",
    "model.decoder.embed_positions.weight",
    "model.decoder.layer_norm.weight",
    "model.decoder.layer_norm.bias",
]


def layer_name(index: int, suffix: str) -> str:
    return f"model.decoder.layers.{index}.{suffix}"


def canonical_names(layers: int) -> List[str]:
    """Model tensors, then the 24 per-layer tensors in order — the order the
    oracle and the C-ABI weight tables index by."""
    names = list(MODEL_NAMES)
    for layer in range(layers):
        names += [layer_name(layer, s) for s in LAYER_SUFFIXES]
    return names


def tensor_extents(shape: DecoderShape, name: str) -> Tuple[int, ...]:
    d, f = shape.width, shape.feed_forward_width
    if name.endswith("embed_tokens.weight"):
        return (shape.vocabulary_size, d)
    if name.endswith("embed_positions.weight"):
        return (shape.max_positions, d)
    if name.endswith("fc1.weight"):
        return (f, d)
    if name.endswith("fc1.bias"):
        return (f,)
    if name.endswith("fc2.weight"):
        return (d, f)
    if name.endswith("proj.weight"):
        return (d, d)
    return (d,)


def is_projection(name: str) -> bool:
    return name.endswith("proj.weight") or name.endswith("fc1.weight") or name.endswith(
        "fc2.weight")


def is_norm_weight(name: str) -> bool:
    return "layer_norm.weight" in name


def is_norm_bias(name: str) -> bool:
    return "layer_norm.bias" in name


# ---------------------------------------------------------------------------
# generators
# ---------------------------------------------------------------------------

def mt19937_raw(seed: int, count: int) -> np.ndarray:
    """``count`` raw std::mt19937 draws for ``seed`` (uint32)."""
    rs = np.random.RandomState(seed & 0xFFFFFFFF)
    return rs.randint(0, 2 ** 32, size=count, dtype=np.uint32)


def spread_values(count: int, seed: int, value_range: float) -> np.ndarray:
    """Tests/Kernels/Common.h:75-88, in float32 arithmetic:
    range * ((float)(engine() % 2001) / 1000.f - 1.f)."""
    raw = mt19937_raw(seed, count) % np.uint32(2001)
    v = raw.astype(np.float32) / np.float32(1000.0) - np.float32(1.0)
    return (np.float32(value_range) * v).astype(np.float32)


def shifted_values(count: int, seed: int, value_range: float) -> np.ndarray:
    """Tests/Encoder/Common.h:148-157: spread values plus one."""
    return (spread_values(count, seed, value_range) + np.float32(1.0)).astype(np.float32)


def _box_muller(raw: np.ndarray, out: np.ndarray, std: float) -> None:
    u1 = (raw[0::2].astype(np.float64) + 0.5) / 4294967296.0
    u2 = (raw[1::2].astype(np.float64) + 0.5) / 4294967296.0
    np.log(u1, out=u1)
    u1 *= -2.0
    np.sqrt(u1, out=u1)
    u2 *= 2.0 * math.pi
    first = np.cos(u2)
    first *= u1
    first *= std
    out[0::2] = first
    np.sin(u2, out=u2)
    u2 *= u1
    u2 *= std
    out[1::2] = u2


_pool: Optional[concurrent.futures.ThreadPoolExecutor] = None


def normal_values(count: int, seed: int, std: float) -> np.ndarray:
    """N(0, std) as float32 by Box-Muller over mt19937 pairs: each pair of raw
    draws gives r*cos(2*pi*u2) then r*sin(2*pi*u2), r = sqrt(-2 ln u1), all in
    double. The transform runs in chunks on a thread pool (numpy releases the
    GIL), which changes nothing in the values."""
    global _pool
    if _pool is None:
        _pool = concurrent.futures.ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1))
    pairs = (count + 1) // 2
    raw = mt19937_raw(seed, 2 * pairs)
    out = np.empty(2 * pairs, dtype=np.float64)
    step = 1 << 20
    jobs = [_pool.submit(_box_muller, raw[i:i + step], out[i:i + step], std) for i in range(0, 2 * pairs, step)]
    for job in jobs:
        job.result()
    return out[:count].astype(np.float32)


def f32_to_bf16_bits(values: np.ndarray) -> np.ndarray:
    """Round to nearest even; NaN stays a quiet NaN."""
    x = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32)
    rounded = ((x + np.uint32(0x7FFF) + ((x >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16))
    nan = (x & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    rounded = np.where(nan, (x >> np.uint32(16)) | np.uint32(0x40), rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def store(values: np.ndarray, dtype: str) -> np.ndarray:
    """The stored form of float32 ``values`` under ``dtype``."""
    if dtype == "F32":
        return np.ascontiguousarray(values, dtype=np.float32)
    if dtype == "F16":
        return np.ascontiguousarray(values, dtype=np.float32).astype(np.float16)
    if dtype == "BF16":
        return f32_to_bf16_bits(values)
    raise ValueError(f"unknown dtype {dtype}")


def widen(stored: np.ndarray, dtype: str) -> np.ndarray:
    """Exact float32 widening of a stored tensor."""
    if dtype == "F32":
        return np.ascontiguousarray(stored, dtype=np.float32)
    if dtype == "F16":
        return stored.astype(np.float32)
    if dtype == "BF16":
        return bf16_bits_to_f32(stored)
    raise ValueError(f"unknown dtype {dtype}")


@dataclasses.dataclass
class StoredTensor:
    name: str
    dtype: str  # "F32" | "F16" | "BF16"
    extents: Tuple[int, ...]
    data: np.ndarray  # float32, float16, or uint16 (bf16 bits)

    def floats(self) -> np.ndarray:
        return widen(self.data, self.dtype).reshape(self.extents)


DecoderFile = Dict[str, StoredTensor]


def synthetic_decoder_file(shape: DecoderShape, storage: str = "Float") -> DecoderFile:
    """Tests/Decoder/Common.h:66-169: seeds count up from 2000 in file order;
    projections in [-0.5, 0.5], embeddings +-0.3, biases +-0.2, LayerNorm gamma
    1 +- 0.2. ``storage`` is "Float", "PackedHalf" (projection weights F16) or
    "EveryTensorHalf" (every tensor F16)."""
    seed = [2000]
    out: DecoderFile = {}

    def nxt(count, value_range):
        v = spread_values(count, seed[0], value_range)
        seed[0] += 1
        return v

    def shifted(count, value_range):
        v = shifted_values(count, seed[0], value_range)
        seed[0] += 1
        return v

    def add(name, values, projection=False):
        extents = tensor_extents(shape, name)
        half = storage == "EveryTensorHalf" or (projection and storage != "Float")
        dtype = "F16" if half else "F32"
        out[name] = StoredTensor(name, dtype, extents, store(values, dtype))

    d, f = shape.width, shape.feed_forward_width
    add(MODEL_NAMES[0], nxt(shape.vocabulary_size * d, 0.3))
    add(MODEL_NAMES[1], nxt(shape.max_positions * d, 0.3))

    for layer in range(shape.layers):
        for norm, attn in (("self_attn_layer_norm", "self_attn"),
                           ("encoder_attn_layer_norm", "encoder_attn")):
            add(layer_name(layer, f"{norm}.weight"), shifted(d, 0.2))
            add(layer_name(layer, f"{norm}.bias"), nxt(d, 0.2))
            add(layer_name(layer, f"{attn}.q_proj.weight"), nxt(d * d, 0.5), True)
            add(layer_name(layer, f"{attn}.q_proj.bias"), nxt(d, 0.2))
            add(layer_name(layer, f"{attn}.k_proj.weight"), nxt(d * d, 0.5), True)
            add(layer_name(layer, f"{attn}.v_proj.weight"), nxt(d * d, 0.5), True)
            add(layer_name(layer, f"{attn}.v_proj.bias"), nxt(d, 0.2))
            add(layer_name(layer, f"{attn}.out_proj.weight"), nxt(d * d, 0.5), True)
            add(layer_name(layer, f"{attn}.out_proj.bias"), nxt(d, 0.2))
        add(layer_name(layer, "final_layer_norm.weight"), shifted(d, 0.2))
        add(layer_name(layer, "final_layer_norm.bias"), nxt(d, 0.2))
        add(layer_name(layer, "fc1.weight"), nxt(f * d, 0.5), True)
        add(layer_name(layer, "fc1.bias"), nxt(f, 0.2))
        add(layer_name(layer, "fc2.weight"), nxt(d * f, 0.5), True)
        add(layer_name(layer, "fc2.bias"), nxt(d, 0.2))

    add(MODEL_NAMES[2], shifted(d, 0.2))
    add(MODEL_NAMES[3], nxt(d, 0.2))
    return out


def file_order(layers: int) -> List[str]:
    """The order a Whisper decoder file lists its tensors in (the seed order)."""
    names = MODEL_NAMES[:2]
    for layer in range(layers):
        names = names + [layer_name(layer, s) for s in LAYER_SUFFIXES]
    return names + MODEL_NAMES[2:]


def workload_decoder_file(shape: DecoderShape, dtype: str, base_seed: int = 1000) -> DecoderFile:
    """The benchmark weights: N(0, 0.02) for projections, biases and both
    embeddings; LayerNorm gamma 1 and beta 0. Tensor i in file order gets seed
    base_seed + i. Every tensor is stored in ``dtype``. Tensors are generated
    on a few threads; each depends on its own seed only."""

    def make(index: int, name: str) -> StoredTensor:
        extents = tensor_extents(shape, name)
        count = int(np.prod(extents))
        if is_norm_weight(name):
            values = np.ones(count, dtype=np.float32)
        elif is_norm_bias(name):
            values = np.zeros(count, dtype=np.float32)
        else:
            values = normal_values(count, base_seed + index, 0.02)
        return StoredTensor(name, dtype, extents, store(values, dtype))

    names = file_order(shape.layers)
    with concurrent.futures.ThreadPoolExecutor(max_workers=4) as pool:
        tensors = list(pool.map(make, range(len(names)), names))
    return {t.name: t for t in tensors}


def synthetic_encoder_output(shape: DecoderShape) -> np.ndarray:
    """Tests/Decoder/Common.h:473-488: a sin/cos sweep of unit-ish spread."""
    position = np.arange(shape.cross_positions, dtype=np.float64)[:, None]
    column = np.arange(shape.width, dtype=np.float64)[None, :]
    phase = 0.13 * position + 0.041 * column
    return (np.sin(phase) + 0.5 * np.cos(2.7 * phase)).astype(np.float32)


def normal_encoder_output(rows: int, width: int, seed: int) -> np.ndarray:
    """[rows, width] float32 N(0, 1) encoder states."""
    return normal_values(rows * width, seed, 1.0).reshape(rows, width)


# ---------------------------------------------------------------------------
# The encoder (the step before the decode path)
# ---------------------------------------------------------------------------

def conv_length(length: int, stride: int) -> int:
    """Kernels/Conv1d.h:121-124 with kernel 3 and padding 1."""
    return (length + 2 - 3) // stride + 1


@dataclasses.dataclass(frozen=True)
class EncoderShape:
    """Encoder/EncoderShape.h:25-67."""

    mel_bins: int
    width: int
    heads: int
    layers: int
    feed_forward_width: int
    input_frames: int

    @property
    def head_width(self) -> int:
        return self.width // self.heads

    def convolution_frames(self, frames: Optional[int] = None) -> int:
        return conv_length(self.input_frames if frames is None else frames, 1)

    def positions(self, frames: Optional[int] = None) -> int:
        return conv_length(self.convolution_frames(frames), 2)

    def frames_for_positions(self, count: int) -> int:
        """Encoder/EncoderShape.cpp:35-38."""
        return min(2 * count, self.input_frames)

    def attention_scale(self) -> float:
        return float(np.float32(1.0) / np.sqrt(np.float32(self.head_width)))

    def with_frames(self, frames: int) -> "EncoderShape":
        return dataclasses.replace(self, input_frames=frames)


def small_encoder_shape() -> EncoderShape:
    """Tests/Encoder/EncoderTests.cpp:15-24: no two extents equal."""
    return EncoderShape(6, 8, 2, 2, 16, 12)


ENCODER_WORKLOADS = {
    # name: (mel bins, width, heads, layers) of the public checkpoints' encoders; ffn = 4 width, 3000 frames
    "tiny.en": (80, 384, 6, 4),
    "base.en": (80, 512, 8, 6),
    "small": (80, 768, 12, 12),
    "medium": (80, 1024, 16, 24),
    "large-v3": (128, 1280, 20, 32),
}


def encoder_workload_shape(name: str, frames: int = 3000) -> EncoderShape:
    bins, width, heads, layers = ENCODER_WORKLOADS[name]
    return EncoderShape(bins, width, heads, layers, 4 * width, frames)


ENCODER_MODEL_NAMES = [
    "model.encoder.conv1.weight", "model.encoder.conv1.bias",
    "model.encoder.conv2.weight", "model.encoder.conv2.bias",
    "model.encoder.embed_positions.weight",
    "model.encoder.layer_norm.weight", "model.encoder.layer_norm.bias",
]

ENCODER_LAYER_SUFFIXES = [
    "self_attn_layer_norm.weight", "self_attn_layer_norm.bias",
    "self_attn.q_proj.weight", "self_attn.q_proj.bias",
    "self_attn.k_proj.weight",
    "self_attn.v_proj.weight", "self_attn.v_proj.bias",
    "self_attn.out_proj.weight", "self_attn.out_proj.bias",
    "final_layer_norm.weight", "final_layer_norm.bias",
    "fc1.weight", "fc1.bias", "fc2.weight", "fc2.bias",
]


def encoder_layer_name(index: int, suffix: str) -> str:
    return f"model.encoder.layers.{index}.{suffix}"


def encoder_canonical_names(layers: int) -> List[str]:
    """Model tensors, then the 15 per-layer tensors: the oracle's order."""
    names = list(ENCODER_MODEL_NAMES)
    for layer in range(layers):
        names += [encoder_layer_name(layer, s) for s in ENCODER_LAYER_SUFFIXES]
    return names


def encoder_tensor_extents(shape: EncoderShape, name: str, table_rows: Optional[int] = None) -> Tuple[int, ...]:
    d, f = shape.width, shape.feed_forward_width
    if name.endswith("conv1.weight"):
        return (d, shape.mel_bins, 3)
    if name.endswith("conv2.weight"):
        return (d, d, 3)
    if name.endswith("embed_positions.weight"):
        return (table_rows if table_rows is not None else shape.positions(), d)
    if name.endswith("fc1.weight"):
        return (f, d)
    if name.endswith("fc1.bias"):
        return (f,)
    if name.endswith("fc2.weight"):
        return (d, f)
    if name.endswith("proj.weight"):
        return (d, d)
    return (d,)


def synthetic_encoder_file(shape: EncoderShape, storage: str = "Float") -> DecoderFile:
    """Tests/Encoder/Common.h:205-302: seeds count up from 1000 in file order;
    convolutions +-0.4, positions +-0.3, projections +-0.5, biases +-0.2,
    LayerNorm gamma 1 +- 0.2. ``storage`` is "Float", "PackedHalf" or
    "EveryTensorHalf" as in the decoder file."""
    seed = [1000]
    out: DecoderFile = {}

    def nxt(count, value_range):
        v = spread_values(count, seed[0], value_range)
        seed[0] += 1
        return v

    def shifted(count, value_range):
        v = shifted_values(count, seed[0], value_range)
        seed[0] += 1
        return v

    def add(name, values, projection=False):
        extents = encoder_tensor_extents(shape, name)
        half = storage == "EveryTensorHalf" or (projection and storage != "Float")
        dtype = "F16" if half else "F32"
        out[name] = StoredTensor(name, dtype, extents, store(values, dtype))

    d, f, bins = shape.width, shape.feed_forward_width, shape.mel_bins
    add(ENCODER_MODEL_NAMES[0], nxt(d * bins * 3, 0.4))
    add(ENCODER_MODEL_NAMES[1], nxt(d, 0.2))
    add(ENCODER_MODEL_NAMES[2], nxt(d * d * 3, 0.4))
    add(ENCODER_MODEL_NAMES[3], nxt(d, 0.2))
    add(ENCODER_MODEL_NAMES[4], nxt(shape.positions() * d, 0.3))
    for layer in range(shape.layers):
        n = lambda suffix: encoder_layer_name(layer, suffix)  # noqa: E731
        add(n("self_attn_layer_norm.weight"), shifted(d, 0.2))
        add(n("self_attn_layer_norm.bias"), nxt(d, 0.2))
        add(n("self_attn.q_proj.weight"), nxt(d * d, 0.5), True)
        add(n("self_attn.q_proj.bias"), nxt(d, 0.2))
        add(n("self_attn.k_proj.weight"), nxt(d * d, 0.5), True)
        add(n("self_attn.v_proj.weight"), nxt(d * d, 0.5), True)
        add(n("self_attn.v_proj.bias"), nxt(d, 0.2))
        add(n("self_attn.out_proj.weight"), nxt(d * d, 0.5), True)
        add(n("self_attn.out_proj.bias"), nxt(d, 0.2))
        add(n("final_layer_norm.weight"), shifted(d, 0.2))
        add(n("final_layer_norm.bias"), nxt(d, 0.2))
        add(n("fc1.weight"), nxt(f * d, 0.5), True)
        add(n("fc1.bias"), nxt(f, 0.2))
        add(n("fc2.weight"), nxt(d * f, 0.5), True)
        add(n("fc2.bias"), nxt(d, 0.2))
    add(ENCODER_MODEL_NAMES[5], shifted(d, 0.2))
    add(ENCODER_MODEL_NAMES[6], nxt(d, 0.2))
    return out


def synthetic_mel(shape: EncoderShape) -> np.ndarray:
    """Tests/Encoder/Common.h:749-765: [mel_bins, input_frames] in about [-1.5, 1.5]."""
    band = np.arange(shape.mel_bins, dtype=np.float64)[:, None]
    frame = np.arange(shape.input_frames, dtype=np.float64)[None, :]
    phase = 0.11 * band + 0.037 * frame
    return (np.sin(phase) + 0.5 * np.cos(2.3 * phase)).astype(np.float32)


def workload_encoder_file(shape: EncoderShape, dtype: str, base_seed: int = 3000) -> DecoderFile:
    """Benchmark encoder weights: N(0, 0.02) convolutions, projections, biases
    and positions (1500 rows), LayerNorm gamma 1 and beta 0; projections in
    ``dtype``, everything else F32 (as the reference widens them). Tensor i in
    canonical order gets seed base_seed + i."""
    names = encoder_canonical_names(shape.layers)

    def make(index: int, name: str) -> StoredTensor:
        extents = encoder_tensor_extents(shape, name)
        count = int(np.prod(extents))
        if is_norm_weight(name):
            values = np.ones(count, dtype=np.float32)
        elif is_norm_bias(name):
            values = np.zeros(count, dtype=np.float32)
        else:
            values = normal_values(count, base_seed + index, 0.02)
        stored = dtype if is_projection(name) else "F32"
        return StoredTensor(name, stored, extents, store(values, stored))

    with concurrent.futures.ThreadPoolExecutor(max_workers=4) as pool:
        tensors = list(pool.map(make, range(len(names)), names))
    return {t.name: t for t in tensors}


def normal_mel(shape: EncoderShape, seed: int) -> np.ndarray:
    """A [mel_bins, input_frames] log-mel-sized input: N(0, 0.5) clipped to [-1.5, 1.5]."""
    values = normal_values(shape.mel_bins * shape.input_frames, seed, 0.5)
    return np.clip(values, -1.5, 1.5).reshape(shape.mel_bins, shape.input_frames)


# ---------------------------------------------------------------------------
# The mel front end's inputs
# ---------------------------------------------------------------------------

@dataclasses.dataclass(frozen=True)
class MelShape:
    """Mel/MelShape.h:16-30: Whisper's 30 s of 16 kHz audio, 400-point
    windows every 160 samples, 3000 frames, 80 bands by default."""

    sample_count: int = 480000
    fft_length: int = 400
    hop_length: int = 160
    frame_count: int = 3000
    mel_count: int = 80

    @property
    def bin_count(self) -> int:
        return self.fft_length // 2 + 1


def reduced_mel_shape() -> MelShape:
    """Tests/Mel/MelSpectrogramTests.cpp:27-36."""
    return MelShape(3200, 64, 16, 200, 12)


def tone_and_noise(sample_count: int) -> np.ndarray:
    """Tests/Mel/MelTestSupport.h:47-66: two tones and a 32-bit LCG's noise,
    with no exact spectral null."""
    state = np.empty(sample_count, dtype=np.uint64)
    s = 12345
    for i in range(sample_count):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        state[i] = s
    noise = (state >> np.uint64(8)).astype(np.float64) / float(1 << 24) - 0.5
    phase = 2.0 * math.pi * np.arange(sample_count, dtype=np.float64)
    return (0.6 * np.sin(phase * 440.0 / 16000) + 0.3 * np.sin(phase * 1237.0 / 16000) + 0.1 * noise).astype(
        np.float32)


def triangular_filters(mel_count: int, bin_count: int) -> np.ndarray:
    """Tests/Mel/MelTestSupport.h:70-88: overlapping triangles shaped like the
    published filterbank."""
    span = (bin_count - 1) / (mel_count + 1)
    bins = np.arange(bin_count, dtype=np.float64)[None, :]
    centre = span * (np.arange(mel_count, dtype=np.float64)[:, None] + 1)
    distance = np.abs(bins - centre) / span
    return np.where(distance < 1.0, 1.0 - distance, 0.0).astype(np.float32)


# ---------------------------------------------------------------------------
# A whole Whisper model directory (config.json, preprocessor_config.json,
# tokenizer.json, model.safetensors) from synthetic tensors
# ---------------------------------------------------------------------------

def safetensors_bytes(tensors: Dict[str, StoredTensor], metadata: Optional[Dict[str, str]] = None) -> bytes:
    """The safetensors layout: an 8-byte little-endian header length, the JSON
    header (name -> dtype, shape, data_offsets), then the tensors' bytes in
    header order."""
    import json
    header: Dict[str, object] = {}
    if metadata:
        header["__metadata__"] = dict(metadata)
    blobs = []
    offset = 0
    for name in sorted(tensors):
        t = tensors[name]
        raw = np.ascontiguousarray(t.data).tobytes()
        header[name] = {"dtype": t.dtype, "shape": list(t.extents), "data_offsets": [offset, offset + len(raw)]}
        blobs.append(raw)
        offset += len(raw)
    text = json.dumps(header, separators=(",", ":")).encode()
    text += b" " * ((8 - len(text) % 8) % 8)
    return len(text).to_bytes(8, "little") + text + b"".join(blobs)


def whisper_config(encoder: EncoderShape, decoder: DecoderShape, **decoding) -> Dict[str, object]:
    """A HuggingFace config.json for these two shapes; ``decoding`` adds
    suppress_tokens, begin_suppress_tokens, decoder_start_token_id, eos_token_id."""
    config: Dict[str, object] = {
        "model_type": "whisper", "num_mel_bins": encoder.mel_bins, "d_model": decoder.width,
        "encoder_attention_heads": encoder.heads, "encoder_layers": encoder.layers,
        "encoder_ffn_dim": encoder.feed_forward_width, "decoder_attention_heads": decoder.heads,
        "decoder_layers": decoder.layers, "decoder_ffn_dim": decoder.feed_forward_width,
        "vocab_size": decoder.vocabulary_size, "max_target_positions": decoder.max_positions,
        "max_source_positions": encoder.input_frames // 2,
    }
    config.update(decoding)
    return config


def preprocessor_config(mel: MelShape, filters: np.ndarray, sample_rate: int = 16000) -> Dict[str, object]:
    return {
        "feature_extractor_type": "WhisperFeatureExtractor", "sampling_rate": sample_rate,
        "n_fft": mel.fft_length, "hop_length": mel.hop_length, "feature_size": mel.mel_count,
        "chunk_length": max(1, mel.sample_count // sample_rate), "n_samples": mel.sample_count,
        "nb_max_frames": mel.frame_count,
        "mel_filters": np.asarray(filters, dtype=np.float64).tolist(),
    }


def write_whisper_directory(path: str, config: Dict[str, object], preprocessor: Dict[str, object],
                            tokenizer_json: str, tensors: Dict[str, StoredTensor]) -> str:
    import json
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(config, f)
    with open(os.path.join(path, "preprocessor_config.json"), "w") as f:
        json.dump(preprocessor, f)
    with open(os.path.join(path, "tokenizer.json"), "w") as f:
        f.write(tokenizer_json)
    with open(os.path.join(path, "model.safetensors"), "wb") as f:
        f.write(safetensors_bytes(tensors, {"format": "pt"}))
    return path


def byte_alphabet() -> List[str]:
    """The byte-level BPE's printable stand-in for each byte (GPT-2's
    bytes_to_unicode): printable Latin-1 bytes stand for themselves, the rest
    take code points from 256 upwards in byte order."""
    keep = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAC + 1)) + list(range(0xAE, 0xFF + 1))
    out, extra = [], 0
    for b in range(256):
        if b in keep:
            out.append(chr(b))
        else:
            out.append(chr(256 + extra))
            extra += 1
    return out


def synthetic_tokenizer_json(vocabulary_size: int = 51864) -> str:
    """A tokenizer.json laid out like tiny.en's: the 256 byte tokens, two-byte
    tokens up to id 50255 (no merges), then the added tokens — <|endoftext|>
    50256, <|startoftranscript|> 50257, <|en|> 50258, the task and prompt
    tokens, <|notimestamps|> 50362 and the timestamps from 50363 — for a
    vocabulary of ``vocabulary_size`` ids."""
    import json
    alphabet = byte_alphabet()
    vocab = {alphabet[b]: b for b in range(256)}
    for i in range(256, 50256):
        j = i - 256
        vocab[alphabet[j // 256] + alphabet[j % 256]] = i
    named = {50256: "<|endoftext|>", 50257: "<|startoftranscript|>", 50258: "<|en|>", 50358: "<|translate|>",
             50359: "<|transcribe|>", 50360: "<|startoflm|>", 50361: "<|startofprev|>", 50362: "<|notimestamps|>"}
    added = []
    for i in range(50256, vocabulary_size):
        if i in named:
            content = named[i]
        elif i >= 50363:
            content = f"<|{(i - 50363) * 0.02:.2f}|>"
        else:
            content = f"<|x{i}|>"
        added.append({"id": i, "content": content, "single_word": False, "lstrip": False, "rstrip": False,
                      "normalized": False, "special": True})
    return json.dumps({"version": "1.0", "added_tokens": added,
                       "model": {"type": "BPE", "vocab": vocab, "merges": []}})


def tiny_en_whisper_directory(path: str, seed: int = 1003) -> str:
    """A tiny.en-shaped Whisper directory with synthetic weights: N(0, 0.02)
    projections rounded to fp16-exact floats in F32 storage (as OpenAI's fp16
    checkpoints are after HuggingFace's conversion, so ExactHalf packs them),
    the published mel shape (30 s, 400-point frames every 160, 80 bands) with
    a triangular filterbank, and the synthetic vocabulary above."""
    encoder = encoder_workload_shape("tiny.en")
    decoder = workload_shape("tiny.en")
    tensors: Dict[str, StoredTensor] = {}
    for source in (workload_encoder_file(encoder, "F32", seed + 2000), workload_decoder_file(decoder, "F32", seed)):
        for name, t in source.items():
            exact = t.data.astype(np.float16).astype(np.float32)
            tensors[name] = StoredTensor(name, "F32", t.extents, exact)
    mel = MelShape()
    config = whisper_config(encoder, decoder, suppress_tokens=[1, 2, 7, 8, 9, 10, 50257, 50360, 50361],
                            begin_suppress_tokens=[220, 50256], decoder_start_token_id=50257,
                            eos_token_id=50256)
    return write_whisper_directory(path, config, preprocessor_config(mel, triangular_filters(80, mel.bin_count)),
                                   synthetic_tokenizer_json(decoder.vocabulary_size), tensors)
