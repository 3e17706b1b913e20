"""The decoder body checked on the CPU, and checked by mutation
(Tests/Decoder/DecoderTests.cpp:7-21).

host/DecoderRecording.cpp — recordSequenceStart / recordDecoderStep, the
composition of the decoder that HipNet runs on gfx950 — is recorded against a
host Net in double precision (tests/native/host_net.h) with the weights of a
safetensors file placed in host memory, and its logits are compared with the
oracle's KV-cached decoder (oracle/oracle.c, which restates referenceDecode
directly, not through Net ops). The reference's small decoder shape and its
prompt are used: a 4-token prompt step (so the causal flag is load bearing)
and six single-token steps fed their own argmax.

Each mutation of the list in DecoderRecording.cpp is built into its own driver
(tests/native/Makefile, WSP_MUTATION=N) and must fail the same comparison that
the unmutated build passes (its logits within 4.4e-8 of the oracle's,
max |a - e| / max |e|); measured as written:

    1  cross-attention before self-attention                  1.73
    2  self keys and values projected from the unnormalised   0.69
    3  every step embedded at position zero                   0.30
    4  the causal flag dropped                                0.63
    5  fc2 without its residual                               1.53
    6  the final LayerNorm skipped before the logits          0.70
    7  the cross values' bias dropped                         0.059

These are host-side mistakes in the composition; the kernels themselves are
held to the oracle by the GPU parity tests, never by deliberately broken
kernels on the GPU.
"""

import os
import subprocess

import numpy as np
import pytest

from helpers import HERE, oracle_tensors
from whispereacp_amd import synthetic as S

NATIVE = os.path.join(HERE, "native")
MUTATIONS = {1: "cross-attention before self-attention",
             2: "self keys and values from the unnormalised rows",
             3: "every step embedded at position zero",
             4: "the causal flag dropped",
             5: "fc2 without its residual",
             6: "the final LayerNorm skipped",
             7: "the cross values' bias dropped"}
PROMPT = [5, 17, 3, 11]  # Tests/Decoder/DecoderTests.cpp:31-37
STEPS = 6


@pytest.fixture(scope="module")
def drivers():
    targets = ["_build/decoder_on_host"] + [f"_build/decoder_on_host_m{n}" for n in MUTATIONS]
    subprocess.run(["make", "-s", "-j8"] + targets, cwd=NATIVE, check=True)
    return {0: os.path.join(NATIVE, targets[0]),
            **{n: os.path.join(NATIVE, f"_build/decoder_on_host_m{n}") for n in MUTATIONS}}


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    shape = S.small_decoder_shape()
    decoder_file = S.synthetic_decoder_file(shape)
    encoder = S.synthetic_encoder_output(shape).astype(np.float32)
    directory = tmp_path_factory.mktemp("host_decoder")
    weights = directory / "model.safetensors"
    weights.write_bytes(S.safetensors_bytes(decoder_file))
    rows = directory / "encoder.f32"
    rows.write_bytes(np.ascontiguousarray(encoder).tobytes())
    return shape, decoder_file, encoder, str(weights), str(rows), directory


def host_run(binary, model, out_name):
    shape, _, _, weights, rows, directory = model
    out = directory / out_name
    args = [binary, weights] + [str(v) for v in shape.as_tuple()] + [rows, str(STEPS), str(out)]
    subprocess.run(args + [str(t) for t in PROMPT], check=True, capture_output=True, text=True)
    logits = np.fromfile(out, dtype=np.float32)
    return logits.reshape(len(PROMPT) + STEPS, shape.vocabulary_size)


def oracle_run(model):
    from oracle import load_oracle
    shape, decoder_file, encoder, *_ = model
    session = load_oracle().session(shape, oracle_tensors(decoder_file, shape))
    session.begin(encoder)
    _, logits = session.step(PROMPT)
    rows = [row for row in logits]
    token = int(np.argmax(logits[-1]))
    for _ in range(STEPS):
        _, logits = session.step([token])
        rows.append(logits[0])
        token = int(np.argmax(logits[0]))
    return np.array(rows)


def relative_error(actual, expected):
    return float(np.max(np.abs(actual - expected)) / np.max(np.abs(expected)))


def test_host_recording_matches_the_oracle(drivers, model):
    expected = oracle_run(model)
    actual = host_run(drivers[0], model, "plain.f32")
    # Double-precision ops written out to float32 rows: only the final
    # rounding separates the two.
    assert relative_error(actual, expected) < 1e-6
    assert [int(np.argmax(r)) for r in actual] == [int(np.argmax(r)) for r in expected]


@pytest.mark.parametrize("mutation", sorted(MUTATIONS), ids=lambda n: MUTATIONS[n].replace(" ", "-"))
def test_each_mutation_is_caught(drivers, model, mutation):
    expected = oracle_run(model)
    actual = host_run(drivers[mutation], model, f"m{mutation}.f32")
    # The parity bar the GPU path is held to: logits within 1e-3 of the
    # oracle's. Every mutation must land far outside it.
    assert relative_error(actual, expected) > 1e-2, MUTATIONS[mutation]
