"""The encoder on the MI355X against the oracle (oracle_encode, pinned in
tests/test_encoder_oracle.py), in the manner of Tests/Encoder/EncoderTests.cpp:
the reference test suite's small encoder over float, packed-half and all-half
files, a reduced context against the shorter shape, a Whisper-width encoder
with 16-bit projections on the matrix cores, the tiny.en encoder over the
full 30 s window, and one large-v3 layer over it (the product tile shapes
the full model runs). Bar: the reference's own 5e-6 worst error
(Tests/Encoder/EncoderTests.cpp:97-108) for the small encoder; 1e-4 for the
larger ones (float32 sums over 1500-key softmaxes and 1536-wide products)."""

import ctypes
import json
import os

import numpy as np
import pytest
import torch

from whispereacp_amd import synthetic as S

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def worst_error(actual, expected):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return float(np.max(np.abs(a - e) / (1.0 + np.abs(e))))


def oracle_rows(oracle, shape, encoder_file, mel, positions=0):
    run = shape.with_frames(shape.frames_for_positions(positions)) if positions else shape
    tensors = [encoder_file[n].floats() for n in S.encoder_canonical_names(shape.layers)]
    return oracle.encode(run, tensors, np.ascontiguousarray(mel[:, :run.input_frames]))


def gpu_rows(shape, encoder_file, mel, positions=0, fill=None, scaled_halves=True):
    from whispereacp_amd.encoder import Encoder, EncoderWeights
    encoder = Encoder(shape)
    weights = EncoderWeights(shape, encoder_file, scaled_halves)
    mel_d = torch.from_numpy(np.ascontiguousarray(mel, dtype=np.float32)).cuda()
    out = torch.full((shape.positions(), shape.width), float("nan") if fill is None else fill,
                     dtype=torch.float32, device="cuda")
    encoder.encode(mel_d, weights, out, positions)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("storage", ["Float", "PackedHalf", "EveryTensorHalf"])
def test_small_encoder_matches_oracle(oracle, storage):
    shape = S.small_encoder_shape()
    encoder_file = S.synthetic_encoder_file(shape, storage)
    mel = S.synthetic_mel(shape)
    got = gpu_rows(shape, encoder_file, mel)
    err = worst_error(got, oracle_rows(oracle, shape, encoder_file, mel))
    print(f"small encoder, {storage}: worst error {err:.2e}")
    assert err <= 5e-6


def test_reduced_context_matches_the_shorter_shape(oracle):
    shape = S.small_encoder_shape()
    encoder_file = S.synthetic_encoder_file(shape, "Float")
    mel = S.synthetic_mel(shape)
    got = gpu_rows(shape, encoder_file, mel, positions=3, fill=-7.0)
    err = worst_error(got[:3], oracle_rows(oracle, shape, encoder_file, mel, positions=3))
    assert err <= 5e-6
    # the rows past the run's are neither read nor written (Encoder/Encoder.h:46-56)
    assert np.all(got[3:] == -7.0)
    # and the full run is still the full run
    assert worst_error(gpu_rows(shape, encoder_file, mel), oracle_rows(oracle, shape, encoder_file, mel)) <= 5e-6


def test_too_long_a_context_is_a_model_error():
    from whispereacp_amd.decoder import ModelError
    shape = S.small_encoder_shape()
    with pytest.raises(ModelError, match="more positions"):
        gpu_rows(shape, S.synthetic_encoder_file(shape, "Float"), S.synthetic_mel(shape), positions=7)


def test_short_positional_table_is_a_model_error():
    from whispereacp_amd.decoder import ModelError
    from whispereacp_amd.encoder import EncoderWeights
    shape = S.small_encoder_shape()
    encoder_file = S.synthetic_encoder_file(shape, "Float")
    with pytest.raises(ModelError, match="carries 6 positions"):
        EncoderWeights(shape.with_frames(40), encoder_file)


@pytest.mark.parametrize("dtype,frames,scaled", [("F16", 64, True), ("BF16", 64, True), ("BF16", 64, False),
                                                 ("F32", 64, True), ("F16", 74, True), ("BF16", 27, True),
                                                 ("BF16", 27, False)])
def test_whisper_width_encoder_matches_oracle(oracle, dtype, frames, scaled):
    # 80 mel bins and head width 64: the projections (more than 16 rows) take
    # the matrix-core product for 16-bit weights, and the attention the
    # matrix-core flash kernel — over 32 positions, and over 37 and 14, which
    # leave part-filled query blocks and key tiles. BF16 runs both as exact
    # scaled fp16 (the pre-split products at every position count, 14 too)
    # and as stored (three bf16 parts).
    shape = S.EncoderShape(80, 128, 2, 2, 512, frames)
    encoder_file = S.workload_encoder_file(shape, dtype, 3000)
    mel = S.normal_mel(shape, 3500)
    got = gpu_rows(shape, encoder_file, mel, scaled_halves=scaled)
    err = worst_error(got, oracle_rows(oracle, shape, encoder_file, mel))
    print(f"width 128 encoder, {dtype}, scaled halves {scaled}: worst error {err:.2e}")
    assert err <= 1e-4


def test_bf16_projections_are_held_as_scaled_halves():
    from whispereacp_amd.encoder import EncoderWeights
    shape = S.EncoderShape(80, 128, 2, 2, 512, 64)
    encoder_file = S.workload_encoder_file(shape, "BF16", 3000)
    weights = EncoderWeights(shape, encoder_file)
    assert (weights.stored_dtype, weights.dtype) == ("BF16", "F16")
    layer = weights._layers[1]
    for field in ("q_scale", "k_scale", "v_scale", "out_scale", "fc1_scale", "fc2_scale"):
        mantissa, exponent = np.frexp(getattr(layer, field))
        assert mantissa == 0.5 and exponent > 1, field
    stored = encoder_file[S.encoder_layer_name(1, "fc1.weight")]
    held = weights._keep[S.encoder_layer_name(1, "fc1.weight")].cpu().numpy().astype(np.float64)
    assert np.array_equal(held / layer.fc1_scale, stored.floats().astype(np.float64).reshape(held.shape))
    assert EncoderWeights(shape, encoder_file, scaled_halves=False).dtype == "BF16"
    # A narrow shape keeps its BF16 storage: its products take no scales.
    narrow = S.EncoderShape(80, 64, 2, 1, 256, 64)
    assert EncoderWeights(narrow, S.workload_encoder_file(narrow, "BF16", 3000)).dtype == "BF16"


def test_a_scale_that_is_not_a_power_of_two_is_refused():
    from whispereacp_amd import _native as N
    from whispereacp_amd.encoder import Encoder, EncoderWeights
    shape = S.EncoderShape(80, 128, 2, 1, 512, 64)
    weights = EncoderWeights(shape, S.workload_encoder_file(shape, "BF16", 3000))
    encoder = Encoder(shape)
    mel = torch.zeros((shape.mel_bins, shape.input_frames), dtype=torch.float32, device="cuda")
    out = torch.empty((shape.positions(), shape.width), dtype=torch.float32, device="cuda")
    # Not a power of two; a power of two whose reciprocal is not a normal float; not finite.
    for bad in (3.0, 2.0 ** -140, float("inf"), -4.0):
        weights._layers[0].fc2_scale = bad
        status = encoder.lib.wsp_encoder_encode(encoder.handle, ctypes.byref(weights.table), mel.data_ptr(),
                                                out.data_ptr(), 0)
        assert status == N.WSP_ERR_ARGUMENT, bad
        assert b"power of two" in encoder.lib.wsp_encoder_last_error(encoder.handle)


def test_golden_fixture_through_the_gpu():
    with open(os.path.join(HERE, "golden", "encoder_mid_f16.json")) as f:
        fx = json.load(f)
    shape = S.EncoderShape(**fx["shape"])
    encoder_file = S.workload_encoder_file(shape, "F16", fx["weights"]["seed"])
    mel = S.normal_mel(shape, fx["weights"]["seed"] + 500)
    expected = np.array([float.fromhex(v) for v in fx["rows"]]).reshape(-1, shape.width)
    assert worst_error(gpu_rows(shape, encoder_file, mel), expected) <= 1e-4


def test_tiny_en_encoder_full_window_matches_oracle(oracle):
    # The tiny.en encoder over Whisper's whole 30 s window: 3000 frames, 1500 rows.
    shape = S.encoder_workload_shape("tiny.en")
    encoder_file = S.workload_encoder_file(shape, "F16", 3000)
    mel = S.normal_mel(shape, 3500)
    got = gpu_rows(shape, encoder_file, mel)
    err = worst_error(got, oracle_rows(oracle, shape, encoder_file, mel))
    print(f"tiny.en encoder, 1500 positions: worst error {err:.2e}")
    assert err <= 1e-4


@pytest.mark.parametrize("dtype,scaled", [("BF16", True), ("BF16", False), ("F16", True)])
@pytest.mark.timeout(300)
def test_large_v3_layer_over_the_full_window_matches_oracle(oracle, dtype, scaled):
    # One layer of the large-v3 encoder (d 1280, 20 heads, ffn 5120) over the
    # whole window: the products take 128-column tiles (q/k/v: 360 blocks,
    # fc1: 480) and 64-column ones (out, fc2), and the attention its 128-query
    # blocks writing the out product's parts — the shapes the full model runs.
    shape = S.EncoderShape(128, 1280, 20, 1, 5120, 3000)
    encoder_file = S.workload_encoder_file(shape, dtype, 3000)
    mel = S.normal_mel(shape, 3500)
    got = gpu_rows(shape, encoder_file, mel, scaled_halves=scaled)
    err = worst_error(got, oracle_rows(oracle, shape, encoder_file, mel))
    print(f"large-v3 layer, {dtype}, scaled halves {scaled}, 1500 positions: worst error {err:.2e}")
    assert err <= 1e-4
