"""The allocation-free W4A8 entry on fp32 activations against the entry it mirrors.

rocket_matmul_int4_prepacked_gw_f32in_noalloc writes its pre-pass codes and row scales into a
fixed per-GPU device array instead of the handle's arena. Its results must be the bits of
rocket_matmul_int4_prepacked_gw_f32in on the same device operands, on two calls in a row
(the second with fewer rows, so stale codes of the first would show), and sampled rows must
match the oracle (per-row quantisation, then the per-row-scale group-wise formula).
"""
import numpy as np
import pytest

import rocketnpu as R

pytestmark = pytest.mark.gpu


def test_noalloc_matches_the_allocating_entry(lib, orc):
    import torch
    dev = torch.device("cuda:0")
    K, N, group = 3840, 15360, 128
    nG = K // group
    B = orc.gen_i8((N, K), 0x52434D01, -8, 7)
    bsc = orc.gen_uniform((N, nG), 0x52434D02, 0.005, 0.02)
    ctx = lib.rocket_i4_ctx_create(1)
    assert ctx
    w = lib.rocket_i4_weights_pack_gw(ctx, 512, K, N, R.ptr(B), group)
    assert w
    dbs = torch.from_numpy(bsc).to(dev)
    for M, seed in ((512, 0x52434D03), (64, 0x52434D04)):
        x = orc.gen_normal((M, K), seed)
        dx = torch.from_numpy(x).to(dev)
        c_ref = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        c_na = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        assert lib.rocket_matmul_int4_prepacked_gw_f32in(ctx, M, K, N, R.ptr(dx), R.ptr(dbs), R.ptr(c_ref), w) == 0
        assert lib.rocket_matmul_int4_prepacked_gw_f32in_noalloc(ctx, M, K, N, R.ptr(dx), R.ptr(dbs), R.ptr(c_na),
                                                                  w) == 0
        torch.cuda.synchronize()
        got, want = c_na.cpu().numpy(), c_ref.cpu().numpy()
        assert np.array_equal(got, want), M
        rows = np.unique(np.r_[0:2, M // 2, M - 2:M])
        q, rs = orc.quant_rows(np.ascontiguousarray(x[rows]))
        assert np.array_equal(got[rows], orc.matmul_gw_rowscale_f32(q, B, rs, bsc, group)), M
    # the fixed scratch bounds M * K; host operands cannot be staged without allocating
    big = 8192
    dxb = torch.zeros((big, K), dtype=torch.float32, device=dev)
    cb = torch.empty((big, N), dtype=torch.float32, device=dev)
    assert lib.rocket_matmul_int4_prepacked_gw_f32in_noalloc(ctx, big, K, N, R.ptr(dxb), R.ptr(dbs), R.ptr(cb),
                                                              w) == R.ROCKET_E_SHAPE
    xh = np.zeros((4, K), np.float32)
    ch = np.zeros((4, N), np.float32)
    assert lib.rocket_matmul_int4_prepacked_gw_f32in_noalloc(ctx, 4, K, N, R.ptr(xh), R.ptr(dbs), R.ptr(ch),
                                                              w) == R.ROCKET_E_SHAPE
    assert lib.rocket_matmul_int4_prepacked_gw_f32in_noalloc(ctx, 6, K, N, R.ptr(dxb), R.ptr(dbs), R.ptr(cb),
                                                              w) == R.ROCKET_E_SHAPE
    lib.rocket_i4_weights_free(ctx, w)
    lib.rocket_i4_ctx_free(ctx)
