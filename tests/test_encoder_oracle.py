"""The encoder's oracle (oracle_conv1d, oracle_encode), checked before the
GPU encoder is checked against it (CPU only).

Pins: the reference's own shape counts (Tests/Encoder/EncoderTests.cpp:72-90,
310-329); hand-worked convolution taps (identity kernel, the padded ends,
stride two); torch conv1d in float64; the golden encoder fixtures written by
an independent torch float64 WhisperEncoder.forward (tests/golden/
make_golden.py); the reduced-context rule (a run over the first 2p frames is
the shorter shape's own encode, Tests/Encoder/EncoderTests.cpp:259-304); and
planted mistakes in the inputs (a transposed convolution weight, a dropped
positional table, a mis-scaled norm) that the golden comparison must reject.
"""

import json
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from whispereacp_amd import synthetic as S

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
FIXTURES = ["encoder_small_float.json", "encoder_small_packed_half.json", "encoder_small_all_half.json",
            "encoder_small_reduced.json", "encoder_mid_f16.json"]


def worst_error(actual, expected):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return float(np.max(np.abs(a - e) / (1.0 + np.abs(e))))


def load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def fixture_inputs(fx):
    """The fixture's shape, weights, mel and expected rows, regenerated from
    the recorded seeds (and checked against the recorded input digest)."""
    import hashlib
    shape = S.EncoderShape(**fx["shape"])
    w = fx["weights"]
    if w["kind"] == "reference-fixture":
        encoder_file = S.synthetic_encoder_file(shape, w["storage"])
        mel = S.synthetic_mel(shape)
    else:
        encoder_file = S.workload_encoder_file(shape, w["storage"], w["seed"])
        mel = S.normal_mel(shape, w["seed"] + 500)
    h = hashlib.sha256()
    for name in S.encoder_canonical_names(shape.layers):
        t = encoder_file[name]
        h.update(name.encode())
        h.update(t.dtype.encode())
        h.update(np.ascontiguousarray(t.data).tobytes())
    h.update(np.ascontiguousarray(mel, dtype=np.float32).tobytes())
    assert h.hexdigest() == fx["input_sha256"], "the generator drifted from the fixture's inputs"
    expected = np.array([float.fromhex(v) for v in fx["rows"]], dtype=np.float64).reshape(-1, shape.width)
    return shape, encoder_file, mel, expected


def oracle_tensors(shape, encoder_file):
    return [encoder_file[n].floats() for n in S.encoder_canonical_names(shape.layers)]


def oracle_run(oracle, shape, encoder_file, mel, positions=0):
    run = shape.with_frames(shape.frames_for_positions(positions)) if positions else shape
    return oracle.encode(run, oracle_tensors(shape, encoder_file),
                         np.ascontiguousarray(mel[:, :run.input_frames]))


def test_shape_counts_match_the_reference():
    shape = S.small_encoder_shape()
    assert shape.convolution_frames() == 12
    assert shape.positions() == 6
    assert shape.head_width == 4
    assert shape.positions() * shape.width == 48
    assert shape.attention_scale() == 0.5
    whisper = shape.with_frames(3000)
    assert whisper.convolution_frames() == 3000 and whisper.positions() == 1500
    assert shape.frames_for_positions(3) == 6 and shape.positions(6) == 3
    assert shape.frames_for_positions(shape.positions()) == shape.input_frames
    assert shape.frames_for_positions(shape.positions() + 4) == shape.input_frames
    assert whisper.frames_for_positions(768) == 1536 and whisper.positions(1536) == 768
    assert whisper.positions(2 * 64) == 64


def test_conv_lengths(oracle):
    assert oracle.conv1d_output_length(3000, 1) == 3000
    assert oracle.conv1d_output_length(3000, 2) == 1500
    assert oracle.conv1d_output_length(12, 2) == 6
    assert oracle.conv1d_output_length(7, 2) == 4


def test_conv1d_hand_worked_taps(oracle):
    x = np.arange(1, 11, dtype=np.float64).reshape(2, 5)   # two channels, five frames
    # Identity: output channel c takes channel c's centre tap.
    w = np.zeros((2, 2, 3), np.float32)
    w[0, 0, 1] = w[1, 1, 1] = 1.0
    b = np.array([0.5, -1.0], np.float32)
    assert np.array_equal(oracle.conv1d(x, w, b, 1), x + b[:, None])
    # The left tap reads frame t - 1: zero (skipped) at t = 0.
    w = np.zeros((1, 2, 3), np.float32)
    w[0, 1, 0] = 1.0
    out = oracle.conv1d(x, w, np.zeros(1, np.float32), 1)
    assert out.tolist() == [[0.0, 6.0, 7.0, 8.0, 9.0]]
    # The right tap at the last frame reads past the end: skipped.
    w = np.zeros((1, 2, 3), np.float32)
    w[0, 0, 2] = 2.0
    out = oracle.conv1d(x, w, np.zeros(1, np.float32), 1)
    assert out.tolist() == [[4.0, 6.0, 8.0, 10.0, 0.0]]
    # Stride two centres frames 0, 2, 4.
    w = np.zeros((1, 2, 3), np.float32)
    w[0, 1, 1] = 1.0
    assert oracle.conv1d(x, w, np.zeros(1, np.float32), 2).tolist() == [[6.0, 8.0, 10.0]]


@pytest.mark.parametrize("stride", [1, 2])
def test_conv1d_matches_torch(oracle, stride):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((7, 19))
    w = rng.standard_normal((5, 7, 3)).astype(np.float32)
    b = rng.standard_normal(5).astype(np.float32)
    expected = F.conv1d(torch.from_numpy(x)[None], torch.from_numpy(w.astype(np.float64)),
                        torch.from_numpy(b.astype(np.float64)), stride=stride, padding=1)[0].numpy()
    assert worst_error(oracle.conv1d(x, w, b, stride), expected) < 1e-13


@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_matches_golden_encoder(oracle, name):
    fx = load(name)
    shape, encoder_file, mel, expected = fixture_inputs(fx)
    got = oracle_run(oracle, shape, encoder_file, mel, fx["positions"])
    assert got.shape == expected.shape
    assert worst_error(got, expected) < 1e-12


def test_reduced_context_is_the_shorter_shapes_encode(oracle):
    # Tests/Encoder/EncoderTests.cpp:259-304: a run over positions p reads the
    # first 2p frames, and its rows are not the full run's first rows.
    fx = load("encoder_small_float.json")
    shape, encoder_file, mel, full = fixture_inputs(fx)
    reduced = oracle_run(oracle, shape, encoder_file, mel, 3)
    assert reduced.shape == (3, shape.width)
    assert worst_error(reduced, full[:3]) > 1e-3
    shorter = load("encoder_small_reduced.json")
    expected = np.array([float.fromhex(v) for v in shorter["rows"]]).reshape(3, shape.width)
    assert worst_error(reduced, expected) < 1e-12


def test_encoder_thread_count_does_not_change_results(oracle):
    fx = load("encoder_mid_f16.json")
    shape, encoder_file, mel, _ = fixture_inputs(fx)
    threads = oracle.set_threads(1)
    one = oracle_run(oracle, shape, encoder_file, mel)
    oracle.set_threads(8)
    many = oracle_run(oracle, shape, encoder_file, mel)
    oracle.set_threads(threads if threads > 1 else 8)
    assert np.array_equal(one, many)


@pytest.mark.parametrize("mistake", ["transposed_conv_taps", "no_positions", "norm_scaled", "k_bias"])
def test_planted_mistakes_fail_the_golden(oracle, mistake):
    fx = load("encoder_small_float.json")
    shape, encoder_file, mel, expected = fixture_inputs(fx)
    tensors = oracle_tensors(shape, encoder_file)
    names = S.encoder_canonical_names(shape.layers)
    i = {n: k for k, n in enumerate(names)}
    if mistake == "transposed_conv_taps":       # taps read in the wrong order
        tensors[i["model.encoder.conv2.weight"]] = np.ascontiguousarray(tensors[i["model.encoder.conv2.weight"]][:, :, ::-1])
    elif mistake == "no_positions":             # the positional table left out
        tensors[i["model.encoder.embed_positions.weight"]] = np.zeros_like(tensors[i["model.encoder.embed_positions.weight"]])
    elif mistake == "norm_scaled":              # gamma applied twice
        n = "model.encoder.layer_norm.weight"
        tensors[i[n]] = tensors[i[n]] * tensors[i[n]]
    else:                                       # a bias added to k_proj, which has none
        n = S.encoder_layer_name(0, "self_attn.k_proj.weight")
        tensors[i[n]] = tensors[i[n]] + np.float32(0.01)
    got = oracle.encode(shape, tensors, mel)
    assert worst_error(got, expected) > 1e-4
