"""Multi-token persistent steps (a t-token Decoder::step whose rows share each
weight read, Decoder/Decoder.cpp:270-308 with tokenCount = t and the causal
self attention of Kernels/Attention.h:34-47) through the C binding.

Each token of a launch runs the same arithmetic in the same order as a
single-token launch at its position (the dot products, the folded LayerNorm
sums, the attention over the same key slots), so a t-token step must match t
single-token steps bit for bit; the oracle checks both against the reference
arithmetic, at t = 2..16, at a later position and with reduced cross rows."""

import numpy as np
import pytest

from helpers import ensure_library, oracle_tensors, worst_error
from whispereacp_amd import synthetic as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def library():
    ensure_library()


def run_steps(decoder, shape, enc, steps, rows_used=0):
    """begin_sequence, then each list in `steps` as one decoder step; returns
    every row's (hidden, logits) in order."""
    import torch
    from whispereacp_amd.decoder import to_device
    V = shape.vocabulary_size
    decoder.begin_sequence(to_device(enc), rows_used)
    hidden, logits = [], []
    for tokens in steps:
        n = len(tokens)
        ids = to_device(np.array(tokens, dtype=np.int32))
        out = torch.empty((n, V), dtype=torch.float32, device="cuda")
        decoder.step(ids, n, out)
        torch.cuda.synchronize()
        hidden.append(decoder.read_hidden(n))
        logits.append(out.cpu().numpy())
    assert decoder.device_status() == 0
    return np.concatenate(hidden), np.concatenate(logits)


def tiny_setup(storage="Float"):
    shape = S.small_decoder_shape()
    return shape, S.synthetic_decoder_file(shape, storage), S.synthetic_encoder_output(shape)


@pytest.mark.parametrize("count", [2, 3, 4, 5, 7, 8, 16])
def test_tokens_in_one_step_match_single_steps_and_the_oracle(oracle, count):
    from whispereacp_amd.decoder import Decoder
    shape, f, enc = tiny_setup()
    tokens = [(7 * i + 3) % shape.vocabulary_size for i in range(count)]
    together = Decoder(shape, f)
    assert together.uses_persistent_step
    h1, l1 = run_steps(together, shape, enc, [tokens])
    single = Decoder(shape, f)
    h2, l2 = run_steps(single, shape, enc, [[t] for t in tokens])
    assert np.array_equal(h1, h2) and np.array_equal(l1, l2)
    h, l = oracle.decode_full(shape, oracle_tensors(f, shape), enc, tokens)
    worst = max(worst_error(h1, h), worst_error(l1, l))
    assert worst <= 5e-6, worst  # the reference's bar at this shape (Tests/Decoder/DecoderTests.cpp:98-110)


def test_a_later_multi_token_step_sees_the_earlier_keys(oracle):
    from whispereacp_amd.decoder import Decoder
    shape, f, enc = tiny_setup()
    tokens = [5, 17, 3, 11, 2, 9, 14, 1, 6]
    steps = [tokens[:3], tokens[3:7], tokens[7:]]
    together = Decoder(shape, f)
    h1, l1 = run_steps(together, shape, enc, steps)
    single = Decoder(shape, f)
    h2, l2 = run_steps(single, shape, enc, [[t] for t in tokens])
    assert np.array_equal(h1, h2) and np.array_equal(l1, l2)
    h, l = oracle.decode_full(shape, oracle_tensors(f, shape), enc, tokens)
    assert max(worst_error(h1, h), worst_error(l1, l)) <= 5e-6


def test_reduced_cross_rows_in_a_multi_token_step(oracle):
    from whispereacp_amd.decoder import Decoder
    shape = S.DecoderShape(128, 2, 2, 512, 1000, 64, 200)
    f = S.workload_decoder_file(shape, "F32", 4000)
    enc = S.normal_encoder_output(shape.cross_positions, shape.width, 9)
    rows_used = 77
    tokens = [5, 6, 7, 8]
    together = Decoder(shape, f, packing="Float")
    h1, l1 = run_steps(together, shape, enc, [tokens], rows_used)
    single = Decoder(shape, f, packing="Float")
    h2, l2 = run_steps(single, shape, enc, [[t] for t in tokens], rows_used)
    assert np.array_equal(h1, h2) and np.array_equal(l1, l2)
    session = oracle.session(shape, oracle_tensors(f, shape))
    session.begin(enc, rows_used)
    h, l = session.step(tokens)
    assert max(worst_error(h1, h), worst_error(l1, l)) <= 1e-4


@pytest.mark.timeout(300)
def test_small_shape_prompt_matches_single_steps_and_the_oracle(oracle):
    # The small configuration (d 768, 12 heads, 12 layers, vocab 51865, fp16
    # weights, 1500 cross rows): a 4-token prompt in one launch, then 6 more
    # tokens in one step (two launches), against single-token steps and the
    # oracle.
    from whispereacp_amd.decoder import Decoder
    shape = S.workload_shape("small")
    f = S.workload_decoder_file(shape, "F16", 1000)
    enc = S.normal_encoder_output(1500, 768, 7)
    tokens = list(S.SOT_PREFIX[shape.vocabulary_size]) + [440, 2034, 11, 1029, 264, 3123]
    steps = [tokens[:4], tokens[4:]]
    together = Decoder(shape, f, packing="ExactHalf")
    h1, l1 = run_steps(together, shape, enc, steps)
    single = Decoder(shape, f, packing="ExactHalf")
    h2, l2 = run_steps(single, shape, enc, [[t] for t in tokens])
    assert np.array_equal(h1, h2) and np.array_equal(l1, l2)
    session = oracle.session(shape, oracle_tensors(f, shape))
    session.begin(enc, 0)
    h, l = session.step(tokens)
    assert worst_error(l1, l) <= 1e-4
    assert [int(np.argmax(r)) for r in l1] == [int(np.argmax(r)) for r in l]


def test_widest_shape_bf16_two_tokens_a_launch(oracle):
    # The large-v3 layer shape (d 1280, 20 heads, ffn 5120, bf16) with two
    # layers: its 20 heads leave head groups for two tokens a launch, so a
    # 5-token step is three launches (2 + 2 + 1).
    from whispereacp_amd.decoder import Decoder
    shape = S.DecoderShape(1280, 20, 2, 5120, 5003, 448, 1500)
    f = S.workload_decoder_file(shape, "BF16", 5000)
    enc = S.normal_encoder_output(shape.cross_positions, shape.width, 11)
    tokens = [1, 2, 3, 4, 77]
    together = Decoder(shape, f, packing="ExactHalf")
    h1, l1 = run_steps(together, shape, enc, [tokens])
    single = Decoder(shape, f, packing="ExactHalf")
    h2, l2 = run_steps(single, shape, enc, [[t] for t in tokens])
    assert np.array_equal(h1, h2) and np.array_equal(l1, l2)
    session = oracle.session(shape, oracle_tensors(f, shape))
    session.begin(enc, 0)
    h, l = session.step(tokens)
    assert worst_error(l1, l) <= 1e-4


def test_a_step_across_the_self_key_block(oracle):
    # Launches carry several tokens only while the self keys stay inside one
    # 256-key block: a step over positions 250..259 runs 250..253 in one
    # launch and 254 on one token a launch (past 256 the keys split over two
    # head groups), and still equals the single-token steps.
    from whispereacp_amd.decoder import Decoder
    shape = S.DecoderShape(256, 4, 2, 1024, 4099, 448, 300)
    f = S.workload_decoder_file(shape, "F16", 3000)
    enc = S.normal_encoder_output(shape.cross_positions, shape.width, 5)
    tokens = [(37 * i + 11) % shape.vocabulary_size for i in range(260)]
    prefix = [tokens[i:i + 16] for i in range(0, 240, 16)] + [tokens[240:250]]
    together = Decoder(shape, f, packing="ExactHalf")
    h1, l1 = run_steps(together, shape, enc, prefix + [tokens[250:]])
    single = Decoder(shape, f, packing="ExactHalf")
    h2, l2 = run_steps(single, shape, enc, [[t] for t in tokens])
    assert np.array_equal(h1, h2) and np.array_equal(l1, l2)
    session = oracle.session(shape, oracle_tensors(f, shape))
    session.begin(enc, 0)
    h, l = session.step(tokens)
    assert worst_error(l1[-10:], l[-10:]) <= 1e-4
