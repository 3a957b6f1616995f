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


def test_noalloc_under_graph_capture(lib, orc):
    """One call recorded into a HIP graph on the handle's stream (the default synchronous mode:
    under capture the entry records its launches and does not wait), replayed three times with
    eager work and new inputs between the replays: every replay equals the eager call on the
    same inputs. Misaligned device operands are refused up front."""
    import torch
    dev = torch.device("cuda:0")
    M, K, N, group = 64, 3840, 1536, 128
    nG = K // group
    B = orc.gen_i8((N, K), 0x52434D11, -8, 7)
    bsc = orc.gen_uniform((N, nG), 0x52434D12, 0.005, 0.02)
    ctx = lib.rocket_i4_ctx_create(1)
    assert ctx
    w = lib.rocket_i4_weights_pack_gw(ctx, M, K, N, R.ptr(B), group)
    assert w
    fd = lib.rocket_i4_ctx_fd(ctx)
    s = torch.cuda.Stream()
    assert lib.rocket_hip_set_stream(fd, R.ptr(s.cuda_stream)) == 0
    dbs = torch.from_numpy(bsc).to(dev)
    dx = torch.empty((M, K), dtype=torch.float32, device=dev)
    c_g = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    c_e = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    call = lib.rocket_matmul_int4_prepacked_gw_f32in_noalloc
    with torch.cuda.stream(s):
        dx.copy_(torch.from_numpy(orc.gen_normal((M, K), 0x52434D13)))
    s.synchronize()
    # eager first: the kernels' one-time set-up happens outside the capture
    assert call(ctx, M, K, N, R.ptr(dx), R.ptr(dbs), R.ptr(c_e), w) == 0
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        rc = call(ctx, M, K, N, R.ptr(dx), R.ptr(dbs), R.ptr(c_g), w)
    assert rc == 0
    for rep in range(3):
        x = orc.gen_normal((M, K), 0x52434D20 + rep)
        with torch.cuda.stream(s):
            dx.copy_(torch.from_numpy(x))
            c_g.fill_(float("nan"))
        s.synchronize()
        g.replay()
        s.synchronize()
        assert call(ctx, M, K, N, R.ptr(dx), R.ptr(dbs), R.ptr(c_e), w) == 0
        got, want = c_g.cpu().numpy(), c_e.cpu().numpy()
        assert np.array_equal(got, want), rep
        rows = np.array([0, M // 2, M - 1])
        q, rs = orc.quant_rows(np.ascontiguousarray(x[rows]))
        assert np.array_equal(got[rows], orc.matmul_gw_rowscale_f32(q, B, rs, bsc, group)), rep
    # device operands off a 16-byte boundary are refused (nothing is staged without allocating)
    flat = torch.zeros(M * K + 4, dtype=torch.float32, device=dev)
    cflat = torch.zeros(M * N + 4, dtype=torch.float32, device=dev)
    assert call(ctx, M, K, N, R.ptr(flat.data_ptr() + 4), R.ptr(dbs), R.ptr(c_e), w) == R.ROCKET_E_SHAPE
    assert call(ctx, M, K, N, R.ptr(dx), R.ptr(dbs), R.ptr(cflat.data_ptr() + 4), w) == R.ROCKET_E_SHAPE
    assert lib.rocket_hip_set_stream(fd, None) == 0
    del g
    lib.rocket_i4_weights_free(ctx, w)
    lib.rocket_i4_ctx_free(ctx)
