"""GPU parity over seeded shape sweeps: each one-shot matmul entry at shapes drawn from a fixed
seed within the entry's alignment rules (M a multiple of 4 or 1; N and K multiples of the
entry's alignment), so that the tile choice, partial row and column tiles, partial last
stages and K slices vary with the draw rather than with a hand-picked list.

Two pools per entry: medium shapes (M <= 640, N <= 2048, K <= 4096: the 64- and 128-row tiles
and the K-sliced plans) and wide ones (M up to 1024, N up to 16384, short K: the 256-row tiles
and, for fp16, the 256 x 256 tile). Bars as in tests/test_gpu_parity.py: integer results
bit-exact; group-wise int32 partials bit-exact, fp32 results bit-identical to the oracle's fold
order and within 1e-5 rms of fp64; fp16 / bf16 / tf32 against the oracle's own rounding of
the same operands. Wide outputs are compared on rows sampled across every row tile.
"""
import sys

import numpy as np
import pytest

import gworder
import rocketnpu as R

pytestmark = pytest.mark.gpu

SWEEP_SEED = 0x5EED5EED


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def draw(tag, n_med, n_wide, nmul, kmul=32, mmul=4, m_one=True, kmax=4096):
    """n_med medium and n_wide wide (M, K, N) shapes for one entry, from a seed of its own."""
    rng = np.random.default_rng([SWEEP_SEED, sum(map(ord, tag))])
    out = []
    for i in range(n_med):
        M = 1 if (m_one and i == 0) else int(rng.integers(1, 640 // mmul + 1)) * mmul
        K = int(rng.integers(1, kmax // kmul + 1)) * kmul
        N = int(rng.integers(1, 2048 // nmul + 1)) * nmul
        out.append((M, K, N))
    for _ in range(n_wide):
        M = int(rng.integers(257 // mmul, 1024 // mmul + 1)) * mmul
        K = int(rng.integers(1, 1024 // kmul + 1)) * kmul
        N = int(rng.integers(4096 // nmul, 16384 // nmul + 1)) * nmul
        out.append((M, K, N))
    return out


def seed_of(M, K, N, salt):
    return (M * 1000003 + K * 10007 + N * 101 + salt) & 0x7FFFFFFF


def rows_of(M, full=256):
    """All rows of a short output; else the first, last and middle rows of every 256-row
    tile, and the matrix's last rows."""
    if M <= full:
        return np.arange(M)
    r = set()
    for t in range(0, M, 256):
        r.update(range(t, min(t + 3, M)))
        r.update(range(max(t, min(t + 256, M) - 3), min(t + 256, M)))
        r.add(min(t + 128, M - 1))
    r.update(range(M - 2, M))
    return np.array(sorted(r))


def sub(X, rows):
    return np.ascontiguousarray(X[rows])


@pytest.mark.parametrize("M,K,N", draw("int8", 8, 3, 32))
def test_sweep_int8(lib, orc, fd, M, K, N):
    say(f"sweep int8 M={M} K={K} N={N}")
    A = orc.gen_i8((M, K), seed_of(M, K, N, 1))
    B = orc.gen_i8((N, K), seed_of(M, K, N, 2))
    C = np.full((M, N), 0x5A5A5A5A, np.int32)
    assert lib.rocket_matmul_int8(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(C)) == 0
    rows = rows_of(M)
    assert np.array_equal(C[rows], orc.matmul_int8(sub(A, rows), B))


@pytest.mark.parametrize("M,K,N", draw("int16", 6, 2, 32))
def test_sweep_int16_exact(lib, orc, fd, M, K, N):
    say(f"sweep int16 M={M} K={K} N={N}")
    A = orc.gen_i16((M, K), seed_of(M, K, N, 3))
    B = orc.gen_i16((N, K), seed_of(M, K, N, 4))
    C = np.full((M, N), -1, np.int64)
    assert lib.rocket_matmul_int16_exact(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(C)) == 0
    rows = rows_of(M)
    assert np.array_equal(C[rows], orc.matmul_int16_exact(sub(A, rows), B))


@pytest.mark.parametrize("M,K,N", draw("int4", 6, 2, 64))
def test_sweep_int4(lib, orc, fd, M, K, N):
    """int4 x int4 (values in int8 storage) and the W4A8 form with full int8 activations."""
    say(f"sweep int4 M={M} K={K} N={N}")
    A4 = orc.gen_i8((M, K), seed_of(M, K, N, 5), -8, 7)
    A8 = orc.gen_i8((M, K), seed_of(M, K, N, 6))
    B = orc.gen_i8((N, K), seed_of(M, K, N, 7), -8, 7)
    rows = rows_of(M)
    C = np.full((M, N), 0x5A5A5A5A, np.int32)
    assert lib.rocket_matmul_int4(fd, M, K, N, R.ptr(A4), R.ptr(B), R.ptr(C)) == 0
    assert np.array_equal(C[rows], orc.matmul_int8(sub(A4, rows), B))
    assert lib.rocket_matmul_int4_ex(fd, M, K, N, R.ptr(A8), R.ptr(B), R.ptr(C), 0) == 0
    assert np.array_equal(C[rows], orc.matmul_int8(sub(A8, rows), B))


def _f16(orc, shape, seed):
    return orc.f32_to_f16_bits(orc.gen_uniform(shape, seed, -1.0, 1.0))


@pytest.mark.parametrize("M,K,N", draw("fp16", 8, 3, 16) + [(512, 544, 30720), (388, 320, 30704)])
def test_sweep_fp16(lib, orc, fd, M, K, N):
    """fp16 results within 1e-2 normalised error of the fp32 product and the fp32-output form
    within 1e-5 of the oracle's fp16-operand product (the last two shapes take the 256 x 256
    tile, the second with partial row, column and stage tiles)."""
    say(f"sweep fp16 M={M} K={K} N={N}")
    A = _f16(orc, (M, K), seed_of(M, K, N, 8))
    B = _f16(orc, (N, K), seed_of(M, K, N, 9))
    rows = rows_of(M)
    C = np.empty((M, N), np.uint16)
    assert lib.rocket_matmul_fp16(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(C)) == 0
    Ar = sub(A, rows)
    ref = orc.matmul_f32(orc.f16_bits_to_f32(Ar), orc.f16_bits_to_f32(B))
    assert orc.norm_err(orc.f16_bits_to_f32(sub(C, rows)), ref) <= 1e-2
    Cf = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_fp16_f32out(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cf)) == 0
    assert orc.norm_err(Cf[rows], orc.matmul_fp16_f32out(Ar, B)) < 1e-5


@pytest.mark.parametrize("M,K,N", draw("bf16", 6, 2, 16))
def test_sweep_bf16_tf32(lib, orc, fd, M, K, N):
    """bf16 and tf32 against the oracle's truncation of the same fp32 operands. bf16 products
    are exact in fp32, so only the fp32 sum differs (1e-5). tf32 runs as three bf16 products of
    an exact hi / lo split and drops lo x lo, at most 2^-14 of each product and of the
    product's sign (the truncated lo parts share their operands' signs): a bias that grows with
    K (1.07e-5 normalised at K = 3936). Each element is held to 2^-13 sum_k |a_k b_k| (the
    dropped terms plus the fp32 sum), and the whole to the 1e-4 of the config-4 test."""
    say(f"sweep bf16/tf32 M={M} K={K} N={N}")
    A = orc.gen_normal((M, K), seed_of(M, K, N, 10))
    B = orc.gen_normal((N, K), seed_of(M, K, N, 11), 0, 0.02)
    rows = rows_of(M)
    Ar = sub(A, rows)
    C = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_bf16(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(C)) == 0
    assert orc.norm_err(C[rows], orc.matmul_bf16(Ar, B)) < 1e-5
    assert lib.rocket_matmul_tf32(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(C)) == 0
    ref = orc.matmul_tf32(Ar, B)
    assert orc.norm_err(C[rows], ref) < 1e-4
    bound = 2.0 ** -13 * (np.abs(Ar.astype(np.float64)) @ np.abs(B.astype(np.float64)).T)
    assert np.all(np.abs(C[rows].astype(np.float64) - ref) <= bound)


def gw_draw(tag, n, int4, nmul):
    """(M, K, N, group) with group a multiple of 32 dividing K (int4: 49 * group < 32767)."""
    rng = np.random.default_rng([SWEEP_SEED, sum(map(ord, tag))])
    groups = [32, 64, 96, 128, 192, 256] + ([] if int4 else [512])
    out = []
    for i in range(n):
        g = int(rng.choice(groups))
        nG = int(rng.integers(1, 65))
        wide = i >= n - 2
        M = int(rng.integers(257 // 4, 1024 // 4 + 1)) * 4 if wide else int(rng.integers(1, 161)) * 4
        N = int(rng.integers((4096 if wide else nmul) // nmul, (12288 if wide else 2048) // nmul + 1)) * nmul
        if wide:
            nG = min(nG, max(1, 1024 // g))
        out.append((M, g * nG, N, g))
    return out


def _gw_check(lib, orc, fd, M, K, N, group, int4):
    nG = K // group
    A = orc.gen_i8((M, K), seed_of(M, K, N, 12))
    B = orc.gen_i8((N, K), seed_of(M, K, N, 13), *((-8, 7) if int4 else (-128, 127)))
    asc = orc.gen_uniform((M, nG), seed_of(M, K, N, 14), 0.5, 1.5)
    bsc = orc.gen_uniform((N, nG), seed_of(M, K, N, 15), 0.005, 0.02)
    rows = rows_of(M)
    # a window of rows for the int32 partials, inside the last row tile
    r0 = max(0, M - 12)
    nr = M - r0
    P = np.full((nr, nG, N), 0x5A5A5A5A, np.int32)
    Cf = np.empty((M, N), np.float32)
    f = lib.rocket_matmul_int4_groupwise_dump if int4 else lib.rocket_matmul_int8_groupwise_dump
    assert f(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(asc), R.ptr(bsc), R.ptr(Cf), group, r0, nr, R.ptr(P)) == 0
    assert np.array_equal(P, orc.gw_partials(sub(A, np.arange(r0, M)), B, group))
    want = gworder.gw_f32(orc, sub(A, rows), B, sub(asc, rows), bsc, group)
    assert np.array_equal(Cf[rows], want)
    assert orc.rms_err(Cf[rows], orc.matmul_gw_f64(sub(A, rows), B, sub(asc, rows), bsc, group)) <= 1e-5
    # the plain entry runs the same kernel without the dump
    C2 = np.empty((M, N), np.float32)
    g = lib.rocket_matmul_int4_groupwise if int4 else lib.rocket_matmul_int8_groupwise
    assert g(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(asc), R.ptr(bsc), R.ptr(C2), group) == 0
    assert np.array_equal(C2[rows], Cf[rows])


@pytest.mark.parametrize("M,K,N,group", gw_draw("int8gw", 8, False, 32))
def test_sweep_int8_groupwise(lib, orc, fd, M, K, N, group):
    say(f"sweep int8 gw M={M} K={K} N={N} g={group}")
    _gw_check(lib, orc, fd, M, K, N, group, False)


@pytest.mark.parametrize("M,K,N,group", gw_draw("int4gw", 8, True, 64))
def test_sweep_int4_groupwise(lib, orc, fd, M, K, N, group):
    say(f"sweep int4 gw M={M} K={K} N={N} g={group}")
    _gw_check(lib, orc, fd, M, K, N, group, True)


def grouped_draw(n):
    """(E, K, N, group, M_e...) for the grouped resident launches: 1..20 products (more than
    16 take a second launch) with empty and ragged M_e; the last two draws are config-5-like
    (8 experts of ~1000 rows, N = 1408, K = 2048, group 32: 256-row tiles with light last-row
    tiles)."""
    rng = np.random.default_rng([SWEEP_SEED, 0x6E])
    out = []
    for i in range(n):
        if i >= n - 2:
            E, g, K, N = 8, 32, 2048, 1408
            Ms = [int(rng.integers(230, 300)) * 4 for _ in range(E)]
        else:
            E = int(rng.integers(1, 21))
            g = int(rng.choice([32, 64, 128]))
            K = g * int(rng.integers(1, 2048 // g + 1))
            N = int(rng.integers(2, 49)) * 32
            Ms = [0 if rng.random() < 0.2 else int(rng.integers(1, 161)) * 4 for _ in range(E)]
        out.append((E, K, N, g, tuple(Ms)))
    return out


@pytest.mark.parametrize("E,K,N,group,Ms", grouped_draw(8))
def test_sweep_grouped(lib, orc, fd, E, K, N, group, Ms):
    """Both grouped launches against the oracle, product by product: per-row activation scales
    (the row-scale fold order) and per-group ones (random, so the reference's order); empty
    products leave their output untouched. The per-row launch again with fp16 results, each
    the fp32 result rounded once."""
    import ctypes as C
    say(f"sweep grouped E={E} K={K} N={N} g={group} M={list(Ms)}")
    nG = K // group
    ctx = lib.rocket_i8_ctx_create(1)
    try:
        Bs, Ws, bss = [], [], []
        for e in range(E):
            Bs.append(orc.gen_i8((N, K), seed_of(e, K, N, 20)))
            Ws.append(lib.rocket_i8_weights_pack_gw(ctx, 4, K, N, R.ptr(Bs[-1]), group))
            assert Ws[-1]
            bss.append(orc.gen_uniform((N, nG), seed_of(e, K, N, 21), 0.005, 0.02))
        As = [orc.gen_i8((max(m, 4), K), seed_of(e, m, K, 22)) for e, m in enumerate(Ms)]
        ars = [orc.gen_uniform((max(m, 4),), seed_of(e, m, K, 23), 0.5, 1.5) for e, m in enumerate(Ms)]
        ags = [orc.gen_uniform((max(m, 4), nG), seed_of(e, m, K, 24), 0.5, 1.5) for e, m in enumerate(Ms)]
        pW = (C.c_void_p * E)(*Ws)
        pM, k0 = R.int_array(list(Ms))
        pA, k1 = R.ptr_array(As)
        pbs, k2 = R.ptr_array(bss)
        for per_group in (False, True):
            Cs = [np.full((max(m, 4), N), -7.0, np.float32) for m in Ms]
            pC, k3 = R.ptr_array(Cs)
            if per_group:
                pa, k4 = R.ptr_array(ags)
                f = lib.rocket_matmul_int8_prepacked_gw_grouped
            else:
                pa, k4 = R.ptr_array(ars)
                f = lib.rocket_matmul_int8_prepacked_gw_grouped_rowscale
            assert f(ctx, E, pM, K, N, pA, pa, pbs, pC, C.cast(pW, R.pp)) == 0
            for e, m in enumerate(Ms):
                if m == 0:
                    assert np.all(Cs[e] == -7.0)
                    continue
                rows = rows_of(m)
                Ae = sub(As[e], rows)
                if per_group:
                    ag = ags[e][:m]
                    want = gworder.gw_f32(orc, Ae, Bs[e], sub(ag, rows), bss[e], group)
                else:
                    want = orc.matmul_gw_rowscale_f32(Ae, Bs[e], sub(ars[e], rows), bss[e], group)
                assert np.array_equal(Cs[e][rows], want), (per_group, e)
            if not per_group:   # fp16 results: the fp32 ones rounded once
                Hs = [np.full((max(m, 4), N), 0x7E00, np.uint16) for m in Ms]
                pH, k5 = R.ptr_array(Hs)
                assert lib.rocket_matmul_int8_prepacked_gw_grouped_rowscale_f16out(
                    ctx, E, pM, K, N, pA, pa, pbs, pH, C.cast(pW, R.pp)) == 0
                for e, m in enumerate(Ms):
                    if m == 0:
                        assert np.all(Hs[e] == 0x7E00)
                    else:
                        assert np.array_equal(Hs[e][:m], Cs[e][:m].astype(np.float16).view(np.uint16)), e
    finally:
        for w in Ws:
            lib.rocket_i8_weights_free(ctx, w)
        lib.rocket_i8_ctx_free(ctx)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M,K,N,group", gw_draw("resident", 6, True, 64))
def test_sweep_resident_groupwise(lib, orc, fd, bits, M, K, N, group):
    """The resident group-wise entries on one packed weight: per-row activation scales (the
    bench's entry), the reference layout with random per-group scales (the reference's fold
    order) and with a per-row scale repeated over the groups (the row-scale order when
    4 <= nG <= 64, then bit-identical to the per-row entry)."""
    say(f"sweep resident int{bits} gw M={M} K={K} N={N} g={group}")
    nG = K // group
    A = orc.gen_i8((M, K), seed_of(M, K, N, 30))
    B = orc.gen_i8((N, K), seed_of(M, K, N, 31), *((-8, 7) if bits == 4 else (-128, 127)))
    arow = orc.gen_uniform((M,), seed_of(M, K, N, 32), 0.5, 1.5)
    agrp = orc.gen_uniform((M, nG), seed_of(M, K, N, 33), 0.5, 1.5)
    arep = np.ascontiguousarray(np.repeat(arow[:, None], nG, axis=1))
    bsc = orc.gen_uniform((N, nG), seed_of(M, K, N, 34), 0.005, 0.02)
    if bits == 4:
        ctx = lib.rocket_i4_ctx_create(1)
        w = lib.rocket_i4_weights_pack_gw(ctx, M, K, N, R.ptr(B), group)
        f_row, f_ref = lib.rocket_matmul_int4_prepacked_gw_rowscale, lib.rocket_matmul_int4_prepacked_gw
        free_w, free_ctx = lib.rocket_i4_weights_free, lib.rocket_i4_ctx_free
    else:
        ctx = lib.rocket_i8_ctx_create(1)
        w = lib.rocket_i8_weights_pack_gw(ctx, M, K, N, R.ptr(B), group)
        f_row, f_ref = lib.rocket_matmul_int8_prepacked_gw_rowscale, lib.rocket_matmul_int8_prepacked_gw
        free_w, free_ctx = lib.rocket_i8_weights_free, lib.rocket_i8_ctx_free
    assert w
    try:
        rows = rows_of(M)
        Ar = sub(A, rows)
        Crow = np.empty((M, N), np.float32)
        assert f_row(ctx, M, K, N, R.ptr(A), R.ptr(arow), R.ptr(bsc), R.ptr(Crow), w) == 0
        assert np.array_equal(Crow[rows], orc.matmul_gw_rowscale_f32(Ar, B, sub(arow, rows), bsc, group))
        Cg = np.empty((M, N), np.float32)
        assert f_ref(ctx, M, K, N, R.ptr(A), R.ptr(agrp), R.ptr(bsc), R.ptr(Cg), w) == 0
        assert np.array_equal(Cg[rows], orc.matmul_gw_f32(Ar, B, sub(agrp, rows), bsc, group))
        assert orc.rms_err(Cg[rows], orc.matmul_gw_f64(Ar, B, sub(agrp, rows), bsc, group)) <= 1e-5
        Cp = np.empty((M, N), np.float32)
        assert f_ref(ctx, M, K, N, R.ptr(A), R.ptr(arep), R.ptr(bsc), R.ptr(Cp), w) == 0
        row = gworder.row_order(arep)
        assert np.array_equal(Cp[rows], gworder.gw_f32(orc, Ar, B, sub(arep, rows), bsc, group))
        if row:
            assert np.array_equal(Cp, Crow)
    finally:
        free_w(ctx, w)
        free_ctx(ctx)


def attn_draw(n):
    """(T, n_kv, dh, dv, nh, nkvh, window, softcap, masked) within the entry's rules: head_dim
    a multiple of 32 and dv of 16, both <= 256; n_head a multiple of n_kv_heads; n_kv >= T so
    every causal row keeps its own key."""
    rng = np.random.default_rng([SWEEP_SEED, 0xA7])
    out = []
    for _ in range(n):
        dh = int(rng.integers(1, 9)) * 32
        dv = int(rng.integers(1, 17)) * 16
        nkvh = int(rng.integers(1, 5))
        nh = nkvh * int(rng.choice([1, 2, 4]))
        T = int(rng.integers(1, 257))
        n_kv = T + int(rng.integers(0, 769))
        masked = bool(rng.random() < 0.75)
        window = int(rng.integers(1, n_kv + 1)) if (masked and rng.random() < 0.4) else 0
        softcap = float(rng.choice([0.0, 0.0, 30.0, 50.0]))
        out.append((T, n_kv, dh, dv, nh, nkvh, window, softcap, masked))
    return out


def _lcg(shape, amp, seed):
    """Uniform fp16 operands in (-amp, amp) (the parity tests' LCG generator, closed form)."""
    n = int(np.prod(shape))
    a, c = np.uint64(1664525), np.uint64(1013904223)
    s0 = np.uint64((0x9E3779B9 ^ seed) & 0xFFFFFFFF)
    with np.errstate(over="ignore"):
        pw = np.cumprod(np.full(n, a, np.uint64))
        geo = np.cumsum(np.concatenate([[np.uint64(1)], pw[:-1]]))
        st = (pw * s0 + c * geo) & np.uint64(0xFFFFFFFF)
    u = ((st >> np.uint64(8)) & np.uint64(0xFFFF)).astype(np.float32) / np.float32(65535.0)
    return ((u * np.float32(2.0) - np.float32(1.0)) * np.float32(amp)).astype(np.float16).view(np.uint16).reshape(shape)


@pytest.mark.parametrize("T,n_kv,dh,dv,nh,nkvh,window,softcap,masked", attn_draw(12))
def test_sweep_flash_attn(lib, orc, fd, T, n_kv, dh, dv, nh, nkvh, window, softcap, masked):
    """Flash attention against the oracle at the reference's bar (cosine >= 0.9995 and
    max |got - ref| <= 0.02 max |ref| + 1e-3, tests/flash_attn_rocket.c:89-96)."""
    say(f"sweep attn T={T} n_kv={n_kv} dh={dh} dv={dv} nh={nh} nkvh={nkvh} win={window} cap={softcap} mask={masked}")
    scale = np.float32(1.0) / np.sqrt(np.float32(dh))
    Q = _lcg((nh, T, dh), 1.0, T * 7 + dh)
    K = _lcg((nkvh, n_kv, dh), 1.0, n_kv * 3 + 1)
    V = _lcg((nkvh, dv, n_kv), 1.0, n_kv * 5 + 2)
    Mk = None
    if masked:
        pos = n_kv - T + np.arange(T)[:, None]
        j = np.arange(n_kv)[None, :]
        keep = (j <= pos) & ((window <= 0) | (j > pos - window))
        Mk = np.where(keep, 0.0, -np.inf).astype(np.float16).view(np.uint16)
    want = orc.flash_attn_f16(Q, K, V, Mk, scale, softcap)
    out = np.full((nh, T, dv), 0x7FFF, np.uint16)
    assert lib.rocket_flash_attn_fp16(fd, T, n_kv, dh, dv, nh, nkvh, scale, softcap, R.ptr(Q), R.ptr(K), R.ptr(V),
                                      R.ptr(Mk) if masked else None, R.ptr(out)) == 0
    assert not np.any(out == 0x7FFF)
    g = out.view(np.float16).astype(np.float64).ravel()
    r = want.view(np.float16).astype(np.float64).ravel()
    cos = g @ r / (np.sqrt(g @ g) * np.sqrt(r @ r) + 1e-30)
    err = np.abs(g - r).max()
    say(f"  cos={cos:.7f} max_abs={err:.3g}")
    assert cos >= 0.9995 and err <= 0.02 * np.abs(r).max() + 1e-3


def ffn_draw(n):
    rng = np.random.default_rng([SWEEP_SEED, 0xFF])
    out = []
    for i in range(n):
        M = 1 if i == 0 else int(rng.integers(1, 129)) * 4
        H = int(rng.integers(1, 33)) * 32
        I = int(rng.integers(1, 65)) * 32
        out.append((M, H, I, [R.ROCKET_ACTIVATION_SILU, R.ROCKET_ACTIVATION_GELU][int(rng.integers(0, 2))]))
    return out


@pytest.mark.parametrize("M,H,I,kind", ffn_draw(6))
def test_sweep_ffn(lib, orc, fd, M, H, I, kind):
    """The gated FFN block, fused and unfused, against the oracle (cosine >= 0.999,
    tests/ffn_fused_rocket.c:151; normalised error <= 1e-2), the two entries bit-identical."""
    say(f"sweep ffn M={M} H={H} I={I} kind={kind}")
    a = np.float32(3.0) / np.sqrt(np.float32(H))
    x = _lcg((M, H), 1.0, 1 + kind)
    Wg, Wu = _lcg((I, H), a, 2 + kind), _lcg((I, H), a, 3 + kind)
    Wd = _lcg((H, I), np.float32(1.5) / np.sqrt(np.float32(I)), 4 + kind)
    want = orc.ffn_f16(x, Wg, Wu, Wd, kind)
    outs = []
    for f in (lib.rocket_ffn_fp16_fused, lib.rocket_ffn_fp16):
        out = np.full((M, H), 0x7FFF, np.uint16)
        assert f(fd, M, H, I, R.ptr(x), R.ptr(Wg), R.ptr(Wu), R.ptr(Wd), kind, R.ptr(out)) == 0
        assert not np.any(out == 0x7FFF)
        outs.append(out)
    g = outs[0].view(np.float16).astype(np.float64).ravel()
    r = want.view(np.float16).astype(np.float64).ravel()
    assert g @ r / (np.sqrt(g @ g) * np.sqrt(r @ r) + 1e-30) >= 0.999
    assert orc.norm_err(orc.f16_bits_to_f32(outs[0]), orc.f16_bits_to_f32(want)) <= 1e-2
    assert np.array_equal(outs[0], outs[1])


def fp16_family_draw(n):
    rng = np.random.default_rng([SWEEP_SEED, 0xF16])
    out = []
    for i in range(n):
        M = int(rng.integers(1, 161)) * 4
        K = int(rng.integers(1, 65)) * 32
        Ns = tuple(int(rng.integers(1, 97)) * 16 for _ in range(int(rng.integers(1, 4))))
        nb = int(rng.integers(1, 7))
        out.append((M, K, Ns, nb, int(rng.integers(1, 9))))
    return out


@pytest.mark.parametrize("M,K,Ns,nb,threads", fp16_family_draw(6))
def test_sweep_fp16_resident_stream_batch(lib, orc, fd, M, K, Ns, nb, threads):
    """The fp16 entries beside the one-shot call, on drawn shapes: the resident weight (at M
    and at a smaller M), the stream and its fused N, the multi-worker entry, the batch and the
    batch context: each bit-identical to the one-shot call and within the fp16 gate of the
    fp32 product."""
    say(f"sweep fp16 family M={M} K={K} Ns={list(Ns)} nb={nb} threads={threads}")
    N = Ns[0]
    A = _f16(orc, (M, K), seed_of(M, K, N, 40))
    Bs = [_f16(orc, (n, K), seed_of(M, K, n, 41 + i)) for i, n in enumerate(Ns)]
    B = Bs[0]
    ref = orc.matmul_f32(orc.f16_bits_to_f32(A), orc.f16_bits_to_f32(B))

    def check(C, Co):
        assert np.array_equal(C, Co)
        assert orc.norm_err(orc.f16_bits_to_f32(C), ref[: C.shape[0]]) <= 1e-2

    Co = np.empty((M, N), np.uint16)
    assert lib.rocket_matmul_fp16(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Co)) == 0
    assert orc.norm_err(orc.f16_bits_to_f32(Co), ref) <= 1e-2
    ctx = lib.rocket_ctx_create(threads)
    w = lib.rocket_weights_pack(ctx, M, K, N, R.ptr(B))
    assert w
    try:
        for Mc in (M, max(4, (M // 8) * 4)):
            Cr = np.empty((Mc, N), np.uint16)
            assert lib.rocket_matmul_fp16_prepacked(ctx, Mc, K, N, R.ptr(A), R.ptr(Cr), w) == 0
            check(Cr, Co[:Mc])
    finally:
        lib.rocket_weights_free(ctx, w)
        lib.rocket_ctx_free(ctx)
    s = lib.rocket_stream_create(threads)
    try:
        Cs = np.empty((M, N), np.uint16)
        assert lib.rocket_matmul_fp16_stream(s, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cs)) == 0
        check(Cs, Co)
        pB, k1 = R.ptr_array(Bs)
        pN, k2 = R.int_array(list(Ns))
        Cf = np.empty((M, sum(Ns)), np.uint16)
        assert lib.rocket_matmul_fp16_stream_fused(s, M, K, pB, pN, len(Ns), R.ptr(A), R.ptr(Cf)) == 0
        c0 = 0
        for Bi, n in zip(Bs, Ns):
            Ci = np.empty((M, n), np.uint16)
            assert lib.rocket_matmul_fp16(fd, M, K, n, R.ptr(A), R.ptr(Bi), R.ptr(Ci)) == 0
            assert np.array_equal(Cf[:, c0:c0 + n], Ci)
            c0 += n
    finally:
        lib.rocket_stream_free(s)
    Cm = np.empty((M, N), np.uint16)
    assert lib.rocket_matmul_fp16_mt(M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cm), threads) == 0
    check(Cm, Co)
    As = [_f16(orc, (M, K), seed_of(M, K, N, 50 + i)) for i in range(nb)]
    Bb = [_f16(orc, (N, K), seed_of(M, K, N, 60 + i)) for i in range(nb)]
    Cb = [np.empty((M, N), np.uint16) for _ in range(nb)]
    Cx = [np.empty((M, N), np.uint16) for _ in range(nb)]
    pa, k3 = R.ptr_array(As)
    pb, k4 = R.ptr_array(Bb)
    pc, k5 = R.ptr_array(Cb)
    px, k6 = R.ptr_array(Cx)
    assert lib.rocket_matmul_fp16_batch(fd, M, K, N, nb, pa, pb, pc) == 0
    bctx = lib.rocket_mm_batch_create(fd)
    assert bctx
    try:
        assert lib.rocket_mm_batch_run(bctx, M, K, N, nb, pa, pb, px) == 0
    finally:
        lib.rocket_mm_batch_free(bctx)
    for i in range(nb):
        Ci = np.empty((M, N), np.uint16)
        assert lib.rocket_matmul_fp16(fd, M, K, N, R.ptr(As[i]), R.ptr(Bb[i]), R.ptr(Ci)) == 0
        assert np.array_equal(Cb[i], Ci) and np.array_equal(Cx[i], Ci)
        ri = orc.matmul_f32(orc.f16_bits_to_f32(As[i]), orc.f16_bits_to_f32(Bb[i]))
        assert orc.norm_err(orc.f16_bits_to_f32(Cb[i]), ri) <= 1e-2


def quant_draw(n):
    rng = np.random.default_rng([SWEEP_SEED, 0x9A])
    out = []
    for _ in range(n):
        g = int(rng.choice([32, 64, 128, 256]))
        K = g * int(rng.integers(1, 4096 // g + 1))
        out.append((int(rng.integers(1, 161)) * 4, K, int(rng.integers(1, 49)) * 64, g))
    return out


@pytest.mark.parametrize("M,K,N,group", quant_draw(6))
def test_sweep_quant_f32in_and_int32_resident(lib, orc, fd, M, K, N, group):
    """The per-row quantisation pre-pass (bit-exact against the oracle), the fp32-input resident
    products (the same bits as quantising and then calling the per-row entry) and the int32
    resident products, int8 and int4, on drawn shapes."""
    say(f"sweep quant / f32in / int32 resident M={M} K={K} N={N} g={group}")
    nG = K // group
    A = (orc.gen_normal((M, K), seed_of(M, K, N, 70)) * np.float32(3.0)).astype(np.float32)
    q, rs = np.empty((M, K), np.int8), np.empty(M, np.float32)
    assert lib.rocket_quantize_rows_int8(fd, M, K, R.ptr(A), R.ptr(q), R.ptr(rs)) == 0
    wq, wrs = orc.quant_rows(A)
    assert np.array_equal(q, wq) and np.array_equal(rs.view(np.uint32), wrs.view(np.uint32))
    bsc = orc.gen_uniform((N, nG), seed_of(M, K, N, 71), 0.005, 0.02)
    rows = rows_of(M)
    for int4 in (False, True):
        B = orc.gen_i8((N, K), seed_of(M, K, N, 72), -8 if int4 else -128, 7 if int4 else 127)
        pre, nm = ("rocket_i4", "int4") if int4 else ("rocket_i8", "int8")
        ctx = getattr(lib, pre + "_ctx_create")(1)
        w = getattr(lib, pre + "_weights_pack_gw")(ctx, M, K, N, R.ptr(B), group)
        wp = getattr(lib, pre + "_weights_pack")(ctx, M, K, N, R.ptr(B))
        assert w and wp
        try:
            C1, C2 = np.full((M, N), np.nan, np.float32), np.full((M, N), np.nan, np.float32)
            assert getattr(lib, f"rocket_matmul_{nm}_prepacked_gw_f32in")(ctx, M, K, N, R.ptr(A), R.ptr(bsc), R.ptr(C1), w) == 0
            assert getattr(lib, f"rocket_matmul_{nm}_prepacked_gw_rowscale")(ctx, M, K, N, R.ptr(q), R.ptr(rs), R.ptr(bsc),
                                                                              R.ptr(C2), w) == 0
            assert np.array_equal(C1.view(np.uint32), C2.view(np.uint32))
            assert np.array_equal(C1[rows], orc.matmul_gw_rowscale_f32(sub(q, rows), B, sub(rs, rows), bsc, group))
            C32 = np.full((M, N), 0x5A5A5A5A, np.int32)
            assert getattr(lib, f"rocket_matmul_{nm}_prepacked")(ctx, M, K, N, R.ptr(q), R.ptr(C32), wp) == 0
            assert np.array_equal(C32[rows], orc.matmul_int8(sub(q, rows), B))
        finally:
            getattr(lib, pre + "_weights_free")(ctx, wp)
            getattr(lib, pre + "_weights_free")(ctx, w)
            getattr(lib, pre + "_ctx_free")(ctx)


def _weights_fx():
    """The test-side writer of the serialised weight format (tests/golden/make_weights_fixture.py)."""
    import importlib.util
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "make_weights_fixture.py")
    spec = importlib.util.spec_from_file_location("make_weights_fixture", path)
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def weights_draw(n):
    rng = np.random.default_rng([SWEEP_SEED, 0x3E])
    out = []
    for i in range(n):
        int4 = bool(i % 2)
        g = int(rng.choice([0, 32, 64, 128, 256]))
        K = (g if g else 32) * int(rng.integers(1, 2048 // (g if g else 32) + 1))
        N = int(rng.integers(1, 33)) * 64
        out.append((int4, g, K, N, int(rng.integers(1, 65)) * 4))
    return out


@pytest.mark.parametrize("int4,group,K,N,M", weights_draw(6))
def test_sweep_weights_round_trip(lib, orc, fd, tmp_path, int4, group, K, N, M):
    """Serialised resident weights at drawn shapes: the bytes equal the test-side writer's,
    and the deserialised and reloaded weights give products bit-identical to the packed one
    and to the oracle."""
    say(f"sweep weights int4={int4} group={group} K={K} N={N} M={M}")
    fx = _weights_fx()
    pre, kind = ("rocket_i4", "int4") if int4 else ("rocket_i8", "int8")
    B = orc.gen_i8((N, K), seed_of(N, K, group, 80), -8 if int4 else -128, 7 if int4 else 127)
    ctx = getattr(lib, pre + "_ctx_create")(1)
    w = (getattr(lib, pre + "_weights_pack_gw")(ctx, M, K, N, R.ptr(B), group) if group
         else getattr(lib, pre + "_weights_pack")(ctx, M, K, N, R.ptr(B)))
    assert w
    ws = [w]
    try:
        bsc = orc.gen_uniform((N, K // group), seed_of(N, K, group, 81), 0.005, 0.02) if group else None
        nbytes = getattr(lib, pre + "_weights_serialized_bytes")(w, 1)
        buf = np.zeros(nbytes, np.uint8)
        assert getattr(lib, pre + "_weights_serialize")(ctx, w, R.ptr(bsc) if group else None, R.ptr(buf), nbytes) == nbytes
        codes = fx.pack_int4(B) if int4 else B.tobytes()
        assert buf.tobytes() == fx.serialise(2 if int4 else 1, N, K, group, M, codes, bsc)
        w2 = getattr(lib, pre + "_weights_deserialize")(ctx, R.ptr(buf), nbytes, None)
        assert w2
        ws.append(w2)
        path = str(tmp_path / "w.rktw").encode()
        assert getattr(lib, pre + "_weights_save")(ctx, w, R.ptr(bsc) if group else None, path) == 0
        w3 = getattr(lib, pre + "_weights_load")(ctx, path, None)
        assert w3
        ws.append(w3)
        A = orc.gen_i8((M, K), seed_of(M, K, N, 82))
        asc = orc.gen_uniform((M, K // group), seed_of(M, K, N, 83), 0.5, 1.5) if group else None
        outs = []
        for ww in ws:
            if group:
                C = np.empty((M, N), np.float32)
                assert getattr(lib, f"rocket_matmul_{kind}_prepacked_gw")(ctx, M, K, N, R.ptr(A), R.ptr(asc), R.ptr(bsc),
                                                                         R.ptr(C), ww) == 0
            else:
                C = np.empty((M, N), np.int32)
                assert getattr(lib, f"rocket_matmul_{kind}_prepacked")(ctx, M, K, N, R.ptr(A), R.ptr(C), ww) == 0
            outs.append(C)
        assert all(np.array_equal(outs[0], o) for o in outs[1:])
        want = gworder.gw_f32(orc, A, B, asc, bsc, group) if group else orc.matmul_int8(A, B)
        assert np.array_equal(outs[0], want)
    finally:
        for ww in ws:
            getattr(lib, pre + "_weights_free")(ctx, ww)
        getattr(lib, pre + "_ctx_free")(ctx)
