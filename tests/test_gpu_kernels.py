"""Each gfx950 kernel against the oracle's primitive on the same inputs,
through the C ABI (include/wsp_hip.h). Tolerances follow the reference's own
kernel tests: 1e-5 + 2.4e-7·inner for the split GEMV
(Tests/Kernels/TiledProduct.h:145-156), 1e-5 for attention
(Tests/Kernels/AttentionTests.cpp:824-828), 1e-4 for LayerNorm
(Tests/Kernels/LayerNormTests.cpp:66-99); embed and argmax exact."""

import numpy as np
import pytest

from helpers import ensure_library, worst_error
from whispereacp_amd import synthetic as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    ensure_library()
    import torch
    from whispereacp_amd.decoder import KernelContext
    assert torch.cuda.is_available()
    # Large enough for every case below: 12 heads of 64 over 1500 keys, 448 rows of 51866.
    shape = S.DecoderShape(768, 12, 1, 3072, 51866, 448, 1500)
    return KernelContext(shape)


def dev(a):
    from whispereacp_amd.decoder import to_device
    return to_device(a)


def sync():
    import torch
    torch.cuda.synchronize()


def weights(out, inner, dtype, seed):
    w = S.normal_values(out * inner, seed, 0.05).reshape(out, inner)
    stored = S.store(w, dtype)
    return stored, S.widen(stored, dtype).reshape(out, inner)


@pytest.mark.parametrize("dtype", ["F32", "F16", "BF16"])
@pytest.mark.parametrize("rows,inner,out", [(1, 768, 768), (1, 768, 3072), (1, 3072, 768), (3, 384, 1536),
                                            (16, 64, 100), (1, 100, 37), (5, 36, 52), (40, 64, 96),
                                            (1500, 256, 64), (40, 256, 128), (130, 96, 384), (300, 512, 256)])
@pytest.mark.parametrize("flags", [0, 1, 2])
def test_linear_matches_oracle(ctx, oracle, dtype, rows, inner, out, flags):
    # More than 16 rows of 16-bit weights with out % 128 == 0 and inner % 32 == 0
    # take the matrix-core product with split activations.
    import torch
    from whispereacp_amd import _native as N
    from whispereacp_amd.decoder import stored_to_device
    x = S.normal_values(rows * inner, 7, 1.0).reshape(rows, inner)
    stored, w = weights(out, inner, dtype, 11)
    bias = S.normal_values(out, 13, 0.1)
    start = S.normal_values(rows * out, 17, 1.0).reshape(rows, out)
    wt = S.StoredTensor("w", dtype, (out, inner), stored)
    wdev, wdtype = stored_to_device(wt)
    y = dev(start.copy())
    ctx.linear(dev(x), rows, inner, wdev, wdtype, dev(bias), y, out, flags)
    sync()
    got = y.cpu().numpy()
    expected = oracle.linear(x.astype(np.float64), w, bias)
    if flags & 1:
        expected = np.vectorize(oracle.gelu)(expected)
    if flags & 2:
        expected = expected + start
    assert worst_error(got, expected) <= 1e-5 + 2.4e-7 * inner


def test_linear_without_bias(ctx, oracle):
    x = S.normal_values(2 * 64, 3, 1.0).reshape(2, 64)
    stored, w = weights(32, 64, "F32", 5)
    y = dev(np.zeros((2, 32), np.float32))
    ctx.linear(dev(x), 2, 64, dev(stored), 0, None, y, 32, 0)
    sync()
    assert worst_error(y.cpu().numpy(), oracle.linear(x.astype(np.float64), w, None)) < 1e-5


def test_layernorm_matches_oracle(ctx, oracle):
    rows, width = 6, 37
    x = (S.normal_values(rows * width, 1, 1.0).reshape(rows, width) * np.arange(1, rows + 1)[:, None]
         + np.arange(rows)[:, None]).astype(np.float32)
    w = S.spread_values(width, 11, 1.5)
    b = S.spread_values(width, 22, 0.75)
    y = dev(np.zeros_like(x))
    ctx.layernorm(dev(x), dev(w), dev(b), y, rows, width)
    sync()
    assert worst_error(y.cpu().numpy(), oracle.layernorm(x.astype(np.float64), w, b)) < 1e-4


@pytest.mark.parametrize("width", [384, 768, 1280, 8])
def test_layernorm_widths(ctx, oracle, width):
    x = S.normal_values(3 * width, width, 1.0).reshape(3, width)
    w, b = np.ones(width, np.float32), np.zeros(width, np.float32)
    y = dev(np.zeros_like(x))
    ctx.layernorm(dev(x), dev(w), dev(b), y, 3, width)
    sync()
    assert worst_error(y.cpu().numpy(), oracle.layernorm(x.astype(np.float64), w, b)) < 1e-4


def test_layernorm_constant_row_yields_bias(ctx):
    w = S.spread_values(32, 33, 2.0)
    b = S.spread_values(32, 44, 2.0)
    y = dev(np.zeros((1, 32), np.float32))
    ctx.layernorm(dev(np.full((1, 32), 2.5, np.float32)), dev(w), dev(b), y, 1, 32)
    sync()
    assert worst_error(y.cpu().numpy()[0], b) < 1e-5


def test_embed_counted_tables(ctx):
    width, vocab, first = 5, 13, 9
    tokens = np.array([12, 0, 5, 7], np.int32)
    table = (8.0 * np.arange(vocab)[:, None] + 0.25 * np.arange(width)[None, :]).astype(np.float32)
    pos = (64.0 * np.arange(448)[:, None] + 0.25 * np.arange(width)[None, :]).astype(np.float32)
    y = dev(np.zeros((4, width), np.float32))
    ctx.embed(dev(tokens), 4, dev(table), dev(np.zeros_like(pos)), first, y, width)
    sync()
    assert np.array_equal(y.cpu().numpy(), table[tokens])
    ctx.embed(dev(tokens), 4, dev(np.zeros_like(table)), dev(pos), first, y, width)
    sync()
    assert np.array_equal(y.cpu().numpy(), pos[first:first + 4])


def test_embed_whole_vocabulary_exactly(ctx):
    vocab, width = 51866, 3
    ids = np.array([0, 1, 220, 50256, 50257, vocab - 1], np.int32)
    table = np.repeat(np.arange(vocab, dtype=np.float32)[:, None], width, axis=1)
    y = dev(np.zeros((len(ids), width), np.float32))
    ctx.embed(dev(ids), len(ids), dev(table), dev(np.zeros((448, width), np.float32)), 0, y, width)
    sync()
    assert np.array_equal(y.cpu().numpy()[:, 0], ids.astype(np.float32))


def test_embed_out_of_vocabulary_poisons_the_row(ctx):
    ids = np.array([3, 60000], np.int32)
    table = np.ones((51866, 4), np.float32)
    y = dev(np.zeros((2, 4), np.float32))
    ctx.embed(dev(ids), 2, dev(table), dev(np.zeros((448, 4), np.float32)), 0, y, 4)
    sync()
    out = y.cpu().numpy()
    assert np.all(out[0] == 1.0) and np.all(np.isnan(out[1]))


def test_embed_refuses_positions_past_the_table(ctx):
    ids = dev(np.array([1], np.int32))
    with pytest.raises(ValueError):
        ctx.embed(ids, 1, dev(np.ones((10, 4), np.float32)), dev(np.ones((448, 4), np.float32)), 448,
                  dev(np.zeros((1, 4), np.float32)), 4)


@pytest.mark.parametrize("q_count,k_count,width,heads,causal", [
    (1, 1, 64, 4, True), (1, 11, 768, 12, True), (1, 203, 64, 1, True), (1, 257, 384, 6, True),
    (1, 700, 64, 4, False), (1, 1500, 768, 12, False), (1, 448, 512, 8, True), (4, 4, 8, 2, True),
    (4, 9, 8, 2, True), (16, 16, 64, 4, True), (3, 1500, 64, 4, False), (2, 6, 8, 2, False),
    # prompt steps (2..16 queries in one launch): causal self attention at the
    # sequence start and further in, cross attention over full and reduced
    # encoder rows, at the decode configurations' head counts and narrower heads
    (2, 2, 768, 12, True), (4, 4, 768, 12, True), (7, 40, 512, 8, True), (16, 300, 1280, 20, True),
    (5, 448, 384, 6, True), (4, 1500, 768, 12, False), (16, 1500, 1280, 20, False), (9, 77, 768, 12, False),
    (3, 65, 256, 4, False), (12, 129, 128, 4, True), (16, 1500, 128, 32, False), (8, 3, 64, 16, False)])
def test_attention_matches_oracle(ctx, oracle, q_count, k_count, width, heads, causal):
    q = S.normal_values(q_count * width, 1, 1.0).reshape(q_count, width)
    k = S.normal_values(k_count * width, 2, 1.0).reshape(k_count, width)
    v = S.normal_values(k_count * width, 3, 1.0).reshape(k_count, width)
    out = dev(np.zeros((q_count, width), np.float32))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(width // heads)))
    ctx.attention(dev(q), q_count, dev(k), dev(v), k_count, width, heads, causal, scale, out)
    sync()
    expected = oracle.attention(q, k, v, heads, causal, first_query=k_count - q_count)
    assert worst_error(out.cpu().numpy(), expected) < 1e-5


def test_attention_single_key_returns_the_value_row(ctx):
    q = S.normal_values(64, 1, 1.0).reshape(1, 64)
    k = S.normal_values(64, 2, 1.0).reshape(1, 64)
    v = S.normal_values(64, 3, 1.0).reshape(1, 64)
    out = dev(np.zeros((1, 64), np.float32))
    ctx.attention(dev(q), 1, dev(k), dev(v), 1, 64, 4, True, 0.25, out)
    sync()
    assert np.array_equal(out.cpu().numpy(), v)


def test_attention_causal_future_keys_are_never_read(ctx):
    # The last two keys are future keys for the first two of three queries;
    # a huge value there would leak into the output if weighted at all.
    q = S.normal_values(3 * 8, 1, 1.0).reshape(3, 8)
    k = S.normal_values(3 * 8, 2, 1.0).reshape(3, 8)
    v = S.normal_values(3 * 8, 3, 1.0).reshape(3, 8)
    out_a = dev(np.zeros((3, 8), np.float32))
    ctx.attention(dev(q), 3, dev(k), dev(v), 3, 8, 2, True, 0.5, out_a)
    v2 = v.copy()
    v2[2] = 1e30
    out_b = dev(np.zeros((3, 8), np.float32))
    ctx.attention(dev(q), 3, dev(k), dev(v2), 3, 8, 2, True, 0.5, out_b)
    sync()
    assert np.array_equal(out_a.cpu().numpy()[:2], out_b.cpu().numpy()[:2])


def test_attention_refuses_wide_heads(ctx):
    from whispereacp_amd.decoder import LogicError
    q = dev(np.zeros((1, 128), np.float32))
    with pytest.raises(LogicError):
        ctx.attention(q, 1, q, q, 1, 128, 1, True, 1.0, q)


def run_argmax(ctx, logits, mask, rows, n):
    import torch
    out = torch.empty(rows, dtype=torch.int32, device="cuda")
    ctx.argmax(dev(logits), rows, n, dev(mask) if mask is not None else None, out)
    sync()
    return out.cpu().numpy().tolist()


def test_argmax_hand_built_rows(ctx):
    n = 37
    i = np.arange(n, dtype=np.float32)
    rows = np.stack([-i, -np.abs(i - 18), i, np.where((i == 5) | (i == 29), 4.0, i * 0.01)]).astype(np.float32)
    assert run_argmax(ctx, rows, None, 4, n) == [0, 18, n - 1, 5]


def test_argmax_matches_oracle_with_a_mask(ctx, oracle):
    rows, n = 11, 37
    logits = S.spread_values(rows * n, 606, 8.0).reshape(rows, n)
    mask = np.zeros(n, np.float32)
    mask[[0, 1, 2, 17, 36]] = 1
    got = run_argmax(ctx, logits, mask, rows, n)
    assert got == [oracle.argmax(logits[r], mask) for r in range(rows)]


def test_argmax_suppression_and_the_only_token_left(ctx):
    n = 37
    logits = (np.arange(n) * 0.5).astype(np.float32)
    logits[7], logits[23] = 100.0, 50.0
    mask = np.zeros(n, np.float32)
    assert run_argmax(ctx, logits, mask, 1, n) == [7]
    mask[7] = 1
    assert run_argmax(ctx, logits, mask, 1, n) == [23]
    mask[23] = 1
    assert run_argmax(ctx, logits, mask, 1, n) == [n - 1]
    desc = (1000.0 - np.arange(n)).astype(np.float32)
    desc[11] = -1000.0
    only = np.where(np.arange(n) == 11, 0.0, 1.0).astype(np.float32)
    assert run_argmax(ctx, desc, only, 1, n) == [11]
    assert run_argmax(ctx, desc, np.ones(n, np.float32), 1, n) == [0]


def test_argmax_over_the_vocabulary(ctx, oracle):
    vocab = 51864
    logits = S.spread_values(vocab, 51864, 4.0)
    logits[50361], logits[318] = 900.0, 800.0
    assert run_argmax(ctx, logits, None, 1, vocab) == [50361]
    mask = np.zeros(vocab, np.float32)
    mask[50361] = 1
    assert run_argmax(ctx, logits, mask, 1, vocab) == [318] == [oracle.argmax(logits, mask)]


def test_argmax_ties_keep_the_lowest_index_across_groups(ctx):
    vocab = 51865
    logits = np.zeros(vocab, np.float32)
    logits[[40000, 9000, 51000]] = 3.0
    assert run_argmax(ctx, logits, None, 1, vocab) == [9000]


def test_argmax_refuses_beyond_its_capacity(ctx):
    with pytest.raises(ValueError):
        run_argmax(ctx, np.zeros((449, 4), np.float32), None, 449, 51866)


@pytest.mark.parametrize("dtype", ["F32", "F16", "BF16"])
@pytest.mark.parametrize("width", [64, 768])
def test_cross_kv_projection_matches_oracle(ctx, oracle, dtype, width):
    # width 768 with 16-bit weights takes the matrix-core product (keys and
    # values in one launch); the other cases the fp32 tiled product.
    from whispereacp_amd.decoder import stored_to_device
    rows = 1500
    x = S.normal_values(rows * width, 21, 1.0).reshape(rows, width)
    sk, wk = weights(width, width, dtype, 22)
    sv, wv = weights(width, width, dtype, 23)
    bv = S.normal_values(width, 24, 0.1)
    kd, code = stored_to_device(S.StoredTensor("k", dtype, (width, width), sk))
    vd, _ = stored_to_device(S.StoredTensor("v", dtype, (width, width), sv))
    k_out = dev(np.zeros((rows, width), np.float32))
    v_out = dev(np.zeros((rows, width), np.float32))
    ctx.project_cross_kv(dev(x), rows, width, kd, vd, dev(bv), code, k_out, v_out)
    sync()
    xd = x.astype(np.float64)
    assert worst_error(k_out.cpu().numpy(), oracle.linear(xd, wk, None)) < 1e-5
    assert worst_error(v_out.cpu().numpy(), oracle.linear(xd, wv, bv)) < 1e-5


def test_prompt_attention_is_deterministic_and_independent_of_the_last_block(ctx):
    # 16 queries over 1500 keys split across blocks whose partials the last one
    # to finish combines in split order: repeated launches give the same bits,
    # and the per-head counters stay usable (zero between launches).
    q = S.normal_values(16 * 768, 4, 1.0).reshape(16, 768)
    k = S.normal_values(1500 * 768, 5, 1.0).reshape(1500, 768)
    v = S.normal_values(1500 * 768, 6, 1.0).reshape(1500, 768)
    qd, kd, vd = dev(q), dev(k), dev(v)
    outs = []
    for _ in range(5):
        out = dev(np.zeros((16, 768), np.float32))
        ctx.attention(qd, 16, kd, vd, 1500, 768, 12, False, 0.125, out)
        sync()
        outs.append(out.cpu().numpy())
    assert all(np.array_equal(outs[0], o) for o in outs[1:])
