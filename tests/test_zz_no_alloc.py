"""wsp_hip_attention_static, the entry point that allocates nothing, against
wsp_hip_attention on a context: the same kernels, so the outputs must be
bit-equal. Two calls in a row on one stream, the second smaller, show that
the shared device array carries nothing from one call into the next."""

import ctypes

import numpy as np
import pytest

from helpers import ensure_library
from whispereacp_amd import synthetic as S

pytestmark = pytest.mark.gpu


def attention_pair(ctx, lib, q_count, k_count, width, heads, causal, seed):
    import torch
    from whispereacp_amd.decoder import current_stream
    q = torch.from_numpy(S.normal_values(q_count * width, seed, 1.0).reshape(q_count, width)).cuda()
    k = torch.from_numpy(S.normal_values(k_count * width, seed + 1, 1.0).reshape(k_count, width)).cuda()
    v = torch.from_numpy(S.normal_values(k_count * width, seed + 2, 1.0).reshape(k_count, width)).cuda()
    scale = float(np.float32(1.0) / np.sqrt(np.float32(width // heads)))
    with_context = torch.zeros((q_count, width), dtype=torch.float32, device="cuda")
    ctx.attention(q, q_count, k, v, k_count, width, heads, causal, scale, with_context)
    without = torch.full((q_count, width), float("nan"), dtype=torch.float32, device="cuda")
    error = ctypes.create_string_buffer(256)
    status = lib.wsp_hip_attention_static(q.data_ptr(), q_count, k.data_ptr(), v.data_ptr(), k_count, width, heads,
                                          int(causal), scale, without.data_ptr(), current_stream(), error, 256)
    assert status == 0, error.value.decode()
    torch.cuda.synchronize()
    return with_context.cpu().numpy(), without.cpu().numpy()


def test_static_attention_matches_the_context_entry_point_twice():
    lib = ensure_library()
    import torch
    from whispereacp_amd.decoder import KernelContext
    assert torch.cuda.is_available()
    ctx = KernelContext(S.DecoderShape(1280, 20, 1, 5120, 51866, 448, 1500))
    # First a prompt step's cross attention at the widest shape (16 queries,
    # 20 heads over 1500 keys: two key chunks per query and head), then a
    # smaller single-query self attention (4 heads over 300 keys, 10 chunks).
    cases = [(16, 1500, 1280, 20, False, 11), (1, 300, 256, 4, True, 21)]
    for q_count, k_count, width, heads, causal, seed in cases:
        expected, got = attention_pair(ctx, lib, q_count, k_count, width, heads, causal, seed)
        assert np.isfinite(got).all()
        assert np.array_equal(expected, got), (q_count, k_count, width, heads)
    # A causal multi-query case, after the smaller one.
    expected, got = attention_pair(ctx, lib, 4, 40, 512, 8, True, 31)
    assert np.array_equal(expected, got)
