"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Each check comes from outside the oracle's own formulas: published test vectors, numpy's
independent conversions and integer/float64 matmuls, exhaustive sweeps, closed-form
identities and brute force on tiny shapes. A plausible mistake (a dropped term, a wrong
sign or index, a transposed operand, a wrong rounding) fails at least one of them.
"""
import ctypes as C

import numpy as np
import pytest


# ---- generators --------------------------------------------------------------------

def test_splitmix64_published_vector(orc):
    # Reference output of splitmix64 seeded with 1234567 (Vigna, splitmix64.c test vector).
    s = C.c_uint64(1234567)
    got = [orc.lib().rko_splitmix64_next(C.byref(s)) for _ in range(5)]
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                   4593380528125082431, 16408922859458223821]
    assert [orc.lib().rko_splitmix64_at(1234567, i) for i in range(5)] == got


def test_generators_ranges_and_determinism(orc):
    a = orc.gen_i8(200000, 7)
    assert a.min() == -128 and a.max() == 127
    assert np.array_equal(a, orc.gen_i8(200000, 7))
    assert not np.array_equal(a, orc.gen_i8(200000, 8))
    # element i depends only on (seed, i): a slice regenerates as the head of a longer run
    assert np.array_equal(orc.gen_i8(1000, 7), a[:1000])
    b = orc.gen_i8(100000, 3, -8, 7)
    assert b.min() == -8 and b.max() == 7 and abs(b.mean() + 0.5) < 0.05
    u = orc.gen_uniform(100000, 5, 0.005, 0.02)
    assert u.min() >= 0.005 and u.max() < 0.02
    n = orc.gen_normal(400000, 9, 0.0, 0.02)
    assert abs(n.mean()) < 2e-4 and abs(n.std() - 0.02) < 2e-4
    h = orc.gen_i16(1000000, 11)
    assert h.min() == -32768 and h.max() == 32767


# ---- conversions -------------------------------------------------------------------

def test_f16_to_f32_all_patterns(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne(orc):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=4_000_000, dtype=np.uint64).astype(np.uint32)
    # bias towards the binary16 range, subnormals and the overflow edge as well
    near = (rng.integers(0x33000000, 0x47800000, size=2_000_000, dtype=np.uint64).astype(np.uint32)
            | (rng.integers(0, 2, size=2_000_000, dtype=np.uint64).astype(np.uint32) << 31))
    edges = np.array([0x477FE000, 0x477FEFFF, 0x477FF000, 0x477FF001, 0x33000000, 0x33000001,
                      0x32FFFFFF, 0x38800000, 0x387FFFFF, 0x387FE000, 0x387FF000, 0x00000000,
                      0x80000000, 0x7F800000, 0xFF800000, 0x3F800000, 0x3F801000, 0x3F803000],
                     dtype=np.uint32)
    x = np.concatenate([bits, near, edges]).view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = x.astype(np.float16)
    got = orc.f32_to_f16_bits(x).view(np.float16)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint16), ref[~nan].view(np.uint16))


def test_bf16_and_tf32_truncation_kats(orc):
    L = orc.lib()
    f = np.array([0x3F80FFFF], np.uint32).view(np.float32)[0]
    assert L.rko_f32_to_bf16_trunc(float(f)) == 0x3F80                     # truncates, never rounds
    g = np.array([0xBF7FFFFF], np.uint32).view(np.float32)[0]
    assert L.rko_f32_to_bf16_trunc(float(g)) == 0xBF7F
    t = L.rko_tf32_trunc(float(np.array([0x3F9FFFFF], np.uint32).view(np.float32)[0]))
    assert np.array([t], np.float32).view(np.uint32)[0] == 0x3F9FE000       # low 13 bits cleared
    rng = np.random.default_rng(2)
    xs = rng.standard_normal(10000).astype(np.float32)
    for x in xs[:2000]:
        assert L.rko_f32_to_bf16_trunc(float(x)) == (int(np.float32(x).view(np.uint32)) >> 16)
        tt = np.float32(L.rko_tf32_trunc(float(x))).view(np.uint32)
        assert tt == (int(np.float32(x).view(np.uint32)) & 0xFFFFE000)


def test_int16_split_exhaustive(orc):
    """x = 256*hi + lo with hi, lo in [-128,127] for every clamped int16
    (rocket_matmul.c:3399-3406); the clamp is [-32768, 32639]."""
    for x in range(-32768, 32768):
        hi, lo = orc.int16_split(x)
        v = min(x, 32639)
        assert -128 <= hi <= 127 and -128 <= lo <= 127
        assert 256 * hi + lo == v, x
    assert orc.int16_split(32640) == orc.int16_split(32639) == orc.int16_split(32767)
    assert orc.int16_split(-32768) == (-128, 0)


# ---- integer references ------------------------------------------------------------

@pytest.mark.parametrize("M,K,N", [(1, 32, 32), (4, 64, 32), (8, 96, 64), (12, 4096, 32)])
def test_int8_matches_numpy_int64(orc, M, K, N):
    rng = np.random.default_rng(M * 1000 + K + N)
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (N, K), dtype=np.int8)
    ref = (A.astype(np.int64) @ B.astype(np.int64).T).astype(np.int32)
    assert np.array_equal(orc.matmul_int8(A, B), ref)


def test_int8_extremes_and_brute_force(orc):
    A = np.full((4, 4096), -128, np.int8)
    B = np.full((32, 4096), -128, np.int8)
    assert np.all(orc.matmul_int8(A, B) == 4096 * 16384)                   # 2^26, exact
    rng = np.random.default_rng(3)
    A = rng.integers(-128, 128, (3, 32), dtype=np.int8)
    B = rng.integers(-128, 128, (5, 32), dtype=np.int8)
    got = orc.matmul_int8(np.ascontiguousarray(A), np.ascontiguousarray(B))
    for m in range(3):
        for n in range(5):
            assert got[m, n] == sum(int(A[m, k]) * int(B[n, k]) for k in range(32))
    # a transposed operand is caught: C[m,n] pairs row m of A with row n of B
    A2 = rng.integers(-128, 128, (4, 32), dtype=np.int8)
    B2 = rng.integers(-128, 128, (8, 32), dtype=np.int8)
    assert orc.matmul_int8(A2, B2).shape == (4, 8)
    assert orc.matmul_int8(A2, B2)[1, 6] == int(A2[1].astype(np.int64) @ B2[6].astype(np.int64))


def test_int16_exact_matches_clamped_int64(orc):
    rng = np.random.default_rng(4)
    A = rng.integers(-32768, 32768, (8, 256), dtype=np.int16)
    B = rng.integers(-32768, 32768, (32, 256), dtype=np.int16)
    A[0, :8] = [32767, 32640, 32639, -32768, 32641, -1, 0, 1]
    ref = np.minimum(A.astype(np.int64), 32639) @ np.minimum(B.astype(np.int64), 32639).T
    assert np.array_equal(orc.matmul_int16_exact(A, B), ref)


def test_int16_exact_equals_four_byte_plane_products(orc):
    """The reference's route: 65536*HH + 256*(HL+LH) + LL over int8 planes."""
    rng = np.random.default_rng(5)
    A = rng.integers(-32768, 32768, (4, 64), dtype=np.int16)
    B = rng.integers(-32768, 32768, (32, 64), dtype=np.int16)
    def planes(X):
        hi = np.empty(X.shape, np.int8)
        lo = np.empty(X.shape, np.int8)
        for idx, v in np.ndenumerate(X):
            hi[idx], lo[idx] = orc.int16_split(int(v))
        return hi, lo
    Ah, Al = planes(A)
    Bh, Bl = planes(B)
    mm = lambda x, y: orc.matmul_int8(x, y).astype(np.int64)
    comb = 65536 * mm(Ah, Bh) + 256 * (mm(Ah, Bl) + mm(Al, Bh)) + mm(Al, Bl)
    assert np.array_equal(orc.matmul_int16_exact(A, B), comb)


# ---- group-wise --------------------------------------------------------------------

@pytest.mark.parametrize("group", [32, 64, 96, 128])
def test_gw_partials_match_numpy_blocks(orc, group):
    rng = np.random.default_rng(group)
    M, K, N = 8, 384, 64
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (N, K), dtype=np.int8)
    P = orc.gw_partials(A, B, group)
    for g in range(K // group):
        sl = slice(g * group, (g + 1) * group)
        ref = A[:, sl].astype(np.int64) @ B[:, sl].astype(np.int64).T
        assert np.array_equal(P[:, g, :], ref)


def test_gw_f64_matches_numpy_and_f32_tracks_it(orc):
    rng = np.random.default_rng(6)
    M, K, N, group = 8, 512, 64, 128
    nG = K // group
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-8, 8, (N, K), dtype=np.int8)
    asc = rng.uniform(0.5, 1.5, (M, nG)).astype(np.float32)
    bsc = rng.uniform(0.005, 0.02, (N, nG)).astype(np.float32)
    P = np.stack([A[:, g * group:(g + 1) * group].astype(np.int64) @ B[:, g * group:(g + 1) * group].astype(np.int64).T
                  for g in range(nG)], axis=1)                               # [M, nG, N]
    ref = np.einsum("mg,ng,mgn->mn", asc.astype(np.float64), bsc.astype(np.float64), P.astype(np.float64))
    f64 = orc.matmul_gw_f64(A, B, asc, bsc, group)
    assert np.allclose(f64, ref, rtol=1e-12, atol=1e-9)
    f32 = orc.matmul_gw_f32(A, B, asc, bsc, group)
    assert orc.rms_err(f32, ref) < 1e-5


def test_gw_special_cases(orc):
    rng = np.random.default_rng(7)
    M, K, N = 4, 256, 32
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (N, K), dtype=np.int8)
    # unit scales: the group-wise result is the int8 product itself (exact below 2^24)
    ones_a = np.ones((M, 4), np.float32)
    ones_b = np.ones((N, 4), np.float32)
    assert np.array_equal(orc.matmul_gw_f32(A, B, ones_a, ones_b, 64),
                          orc.matmul_int8(A, B).astype(np.float32))
    # one group: per-channel dequant, a single rounding of (as*bs)*P
    asc = rng.uniform(0.1, 1.0, (M, 1)).astype(np.float32)
    bsc = rng.uniform(0.1, 1.0, (N, 1)).astype(np.float32)
    P = orc.matmul_int8(A, B).astype(np.float32)
    ref = (asc * bsc.T).astype(np.float32) * P
    assert np.array_equal(orc.matmul_gw_f32(A, B, asc, bsc, K), ref.astype(np.float32))


def test_gw_rowscale_order(orc):
    rng = np.random.default_rng(9)
    M, K, N, group = 8, 384, 64, 128
    nG = K // group
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-8, 8, (N, K), dtype=np.int8)
    bsc = rng.uniform(0.005, 0.02, (N, nG)).astype(np.float32)
    arow = rng.uniform(0.5, 2.0, M).astype(np.float32)
    # unit row scales: exactly the reference-order combine with unit activation scales
    assert np.array_equal(orc.matmul_gw_rowscale_f32(A, B, np.ones(M, np.float32), bsc, group),
                          orc.matmul_gw_f32(A, B, np.ones((M, nG), np.float32), bsc, group))
    # the row scale is one multiply after the group sum: fp64 agreement at fp32 rounding level
    P = np.stack([A[:, g * group:(g + 1) * group].astype(np.int64) @ B[:, g * group:(g + 1) * group].astype(np.int64).T
                  for g in range(nG)], axis=1)
    ref = arow[:, None].astype(np.float64) * np.einsum("ng,mgn->mn", bsc.astype(np.float64), P.astype(np.float64))
    assert orc.rms_err(orc.matmul_gw_rowscale_f32(A, B, arow, bsc, group), ref) < 1e-6
    # one group: round(bs * P) then one rounding of the row multiply, in that order
    b1 = rng.uniform(0.1, 1.0, (N, 1)).astype(np.float32)
    P1 = orc.matmul_int8(A, B).astype(np.float32)
    want = arow[:, None] * (b1.T * P1)                                    # numpy float32 ops
    assert np.array_equal(orc.matmul_gw_rowscale_f32(A, B, arow, b1, K), want)


# ---- floating-point references -----------------------------------------------------

def test_fp16_identity_onehot_and_exact_integers(orc):
    rng = np.random.default_rng(8)
    M, K = 8, 64
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    A16 = orc.f32_to_f16_bits(A)
    I16 = orc.f32_to_f16_bits(np.eye(K, dtype=np.float32))                  # B = I (N = K)
    assert np.array_equal(orc.matmul_fp16(A16, I16), A16)
    sel = np.zeros((16, K), np.float32)
    cols = rng.integers(0, K, 16)
    sel[np.arange(16), cols] = 1.0
    assert np.array_equal(orc.matmul_fp16(A16, orc.f32_to_f16_bits(sel)), A16[:, cols])
    # small integers: every partial sum is exact, so the fp16 result is exact
    Ai = rng.integers(-3, 4, (M, K)).astype(np.float32)
    Bi = rng.integers(-3, 4, (32, K)).astype(np.float32)
    got = orc.f16_bits_to_f32(orc.matmul_fp16(orc.f32_to_f16_bits(Ai), orc.f32_to_f16_bits(Bi)))
    assert np.array_equal(got, Ai @ Bi.T)


def test_fp16_and_float_refs_track_numpy(orc):
    rng = np.random.default_rng(9)
    M, K, N = 16, 256, 48
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (N, K)).astype(np.float32)
    A16, B16 = orc.f32_to_f16_bits(A), orc.f32_to_f16_bits(B)
    Af = A16.view(np.float16).astype(np.float64)
    Bf = B16.view(np.float16).astype(np.float64)
    ref = Af @ Bf.T
    c16 = orc.f16_bits_to_f32(orc.matmul_fp16(A16, B16))
    assert np.max(np.abs(c16 - ref)) <= np.max(np.abs(ref)) * 2e-3
    c32 = orc.matmul_fp16_f32out(A16, B16)
    assert np.allclose(c32, ref, rtol=1e-6, atol=1e-5)
    # bf16 / tf32 / f32: double accumulation of the (truncated) operands, as numpy computes it
    trunc = lambda X, mask: (X.view(np.uint32) & np.uint32(mask)).view(np.float32).astype(np.float64)
    assert np.allclose(orc.matmul_bf16(A, B), trunc(A, 0xFFFF0000) @ trunc(B, 0xFFFF0000).T, rtol=1e-6, atol=1e-6)
    assert np.allclose(orc.matmul_tf32(A, B), trunc(A, 0xFFFFE000) @ trunc(B, 0xFFFFE000).T, rtol=1e-6, atol=1e-6)
    assert np.allclose(orc.matmul_f32(A, B), A.astype(np.float64) @ B.astype(np.float64).T, rtol=1e-6, atol=1e-6)
    # truncation is visible: the bf16 result differs from the exact fp32 one
    assert orc.norm_err(orc.matmul_bf16(A, B), orc.matmul_f32(A, B)) > 1e-4


def test_fp16_naive_loop_is_the_sequential_fp32_sum(orc):
    """The single-thread comparability loop (the reference tests' form) gives the threaded
    oracle's bits, and both are the k-ascending fp32 sum of exact fp16 products rounded once to
    fp16, as numpy computes it element by element."""
    rng = np.random.default_rng(12)
    M, K, N = 3, 64, 5
    A16 = orc.f32_to_f16_bits(rng.uniform(-1, 1, (M, K)).astype(np.float32))
    B16 = orc.f32_to_f16_bits(rng.uniform(-1, 1, (N, K)).astype(np.float32))
    naive = orc.matmul_fp16_naive(A16, B16)
    assert np.array_equal(naive, orc.matmul_fp16(A16, B16))
    Af, Bf = A16.view(np.float16).astype(np.float32), B16.view(np.float16).astype(np.float32)
    want = np.empty((M, N), np.float16)
    for i in range(M):
        for j in range(N):
            acc = np.float32(0)
            for l in range(K):
                acc = np.float32(acc + np.float32(Af[i, l] * Bf[j, l]))
            want[i, j] = np.float16(acc)
    assert np.array_equal(naive, want.view(np.uint16))


# ---- feed-forward blocks (reference src/rocket_ffn.c) -------------------------------

def test_f64_to_f16_matches_numpy_rne(orc):
    # numpy converts binary64 -> binary16 directly (one rounding, ties to even)
    rng = np.random.default_rng(21)
    v = rng.standard_normal(300000) * 10.0 ** rng.integers(-9, 6, 300000)
    h = rng.integers(0, 0x7BFF, 30000).astype(np.uint16)            # exact ties between halves
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    edges = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 2.0 ** -24, 2.0 ** -25,
                      np.nextafter(2.0 ** -25, 1), 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 1e-300, np.inf, -np.inf])
    v = np.concatenate([v, (lo + hi) / 2, -(lo + hi) / 2, edges])
    f = np.vectorize(orc.lib().rko_f64_to_f16, otypes=[np.uint16])
    with np.errstate(over="ignore"):
        want = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(f(v), want)
    # a double just above a tie must round up although its float32 rounding is the tie itself
    x = 1.0 + 2.0 ** -11 + 2.0 ** -40
    assert orc.lib().rko_f64_to_f16(x) == np.float16(1.0 + 2.0 ** -10).view(np.uint16)
    assert orc.lib().rko_f64_to_f16(float("nan")) & 0x7FFF > 0x7C00


def test_activation_known_values_and_identities(orc):
    act = orc.lib().rko_act_exact
    # Phi(1) = 0.841344746068543 (standard normal CDF tables), sigmoid(1) = e / (1 + e)
    assert act(5, 1.0) == pytest.approx(0.8413447460685429, abs=1e-15)
    assert act(3, 1.0) == pytest.approx(np.e / (1 + np.e), abs=1e-15)
    assert act(5, 0.0) == 0.0 and act(3, 0.0) == 0.0
    # act(x) - act(-x) = x for both (sigmoid(x) + sigmoid(-x) = 1, Phi(x) + Phi(-x) = 1)
    for x in (0.1, 0.7, 2.5, 6.0, 11.0):
        for k in (3, 5):
            assert act(k, x) - act(k, -x) == pytest.approx(x, rel=1e-14)
    assert act(5, -10.0) == pytest.approx(0.0, abs=1e-20) and act(3, 40.0) == pytest.approx(40.0)
    # every kind other than GELU is SiLU (reference rocket_ffn.c:23-27)
    assert act(0, 1.3) == act(3, 1.3) == act(7, 1.3)
    # GELU matches the normal CDF that scipy computes independently (the 1 + erf form loses
    # relative accuracy in the negative tail, to about 1e-16 absolute)
    from scipy.special import ndtr
    xs = np.linspace(-7, 7, 57)
    assert np.allclose([act(5, x) for x in xs], xs * ndtr(xs), rtol=1e-13, atol=1e-14)


def _ulp16(a, b):
    """Distance in fp16 units in the last place between two arrays of fp16 bits."""
    def ordered(h):
        h = h.astype(np.int32)
        return np.where(h & 0x8000, -(h & 0x7FFF), h)
    return np.abs(ordered(a) - ordered(b))


def test_geglu_matches_numpy(orc):
    from scipy.special import ndtr
    n = 20000
    gate = orc.f32_to_f16_bits(orc.gen_uniform(n, 31, -6, 6))
    up = orc.f32_to_f16_bits(orc.gen_uniform(n, 32, -2.5, 2.5))
    g = gate.view(np.float16).astype(np.float64)
    u = up.view(np.float16).astype(np.float64)
    for kind, a in ((3, g / (1 + np.exp(-g))), (5, g * ndtr(g))):
        got = orc.geglu_f16(gate, up, kind)
        want = (a * u).astype(np.float16).view(np.uint16)
        assert _ulp16(got, want).max() <= 1
        assert np.mean(got == want) > 0.999
    z = np.zeros(16, np.uint16)
    assert np.all(orc.geglu_f16(z, up[:16], 3) & 0x7FFF == 0)          # act(0) = 0


def _ffn_np(x, Wg, Wu, Wd, kind):
    from scipy.special import ndtr
    X, G, U, D = (t.view(np.float16).astype(np.float64) for t in (x, Wg, Wu, Wd))
    g, u = X @ G.T, X @ U.T
    a = g * ndtr(g) if kind == 5 else g / (1 + np.exp(-g))
    return (a * u) @ D.T


@pytest.mark.parametrize("M,H,I,kind", [(3, 64, 96, 3), (5, 32, 160, 5), (16, 128, 256, 3)])
def test_ffn_matches_numpy_float64(orc, M, H, I, kind):
    a = 3.0 / np.sqrt(H)
    x = orc.f32_to_f16_bits(orc.gen_uniform((M, H), 41, -1, 1))
    Wg = orc.f32_to_f16_bits(orc.gen_uniform((I, H), 42, -a, a))
    Wu = orc.f32_to_f16_bits(orc.gen_uniform((I, H), 43, -a, a))
    Wd = orc.f32_to_f16_bits(orc.gen_uniform((H, I), 44, -1.5 / np.sqrt(I), 1.5 / np.sqrt(I)))
    got = orc.ffn_f16(x, Wg, Wu, Wd, kind)
    want = _ffn_np(x, Wg, Wu, Wd, kind).astype(np.float16).view(np.uint16)
    assert _ulp16(got, want).max() <= 1                 # summation order differs from numpy's
    other = orc.ffn_f16(x, Wg, Wu, Wd, 8 - kind)        # the activation kind matters
    assert not np.array_equal(got, other)


def test_ffn_special_cases(orc):
    M, H, I = 4, 32, 64
    x = orc.f32_to_f16_bits(orc.gen_uniform((M, H), 51, -1, 1))
    W = orc.f32_to_f16_bits(orc.gen_uniform((I, H), 52, -1, 1))
    Wd = orc.f32_to_f16_bits(orc.gen_uniform((H, I), 53, -1, 1))
    zero = np.zeros((I, H), np.uint16)
    # a zero gate gives act(0) = 0 everywhere, so the block's output is exactly zero
    assert np.all(orc.ffn_f16(x, zero, W, Wd, 3) & 0x7FFF == 0)
    # gate = up = x (I = H, identity weights): prod = act(x) * x, and Wd = I returns it
    eye = orc.f32_to_f16_bits(np.eye(H, dtype=np.float32))
    xs = orc.f32_to_f16_bits(orc.gen_uniform((M, H), 54, -4, 4))
    got = orc.ffn_f16(xs, eye, eye, eye, 3)
    assert np.array_equal(got, orc.geglu_f16(xs, xs, 3))


def test_mlp_matches_numpy_and_bias_closed_form(orc):
    from scipy.special import ndtr
    M, Din, Dff, Dout = 6, 64, 96, 48
    x = orc.f32_to_f16_bits(orc.gen_uniform((M, Din), 61, -1, 1))
    W1 = orc.f32_to_f16_bits(orc.gen_uniform((Dff, Din), 62, -0.3, 0.3))
    b1 = orc.f32_to_f16_bits(orc.gen_uniform(Dff, 63, -1, 1))
    W2 = orc.f32_to_f16_bits(orc.gen_uniform((Dout, Dff), 64, -0.2, 0.2))
    X, A, B, C2 = (t.view(np.float16).astype(np.float64) for t in (x, W1, b1, W2))
    for kind in (3, 5):
        for bias in (None, b1):
            h = X @ A.T + (0 if bias is None else B)
            act = (h * ndtr(h) if kind == 5 else h / (1 + np.exp(-h))).astype(np.float16)   # rounded
            want = (act.astype(np.float64) @ C2.T).astype(np.float16).view(np.uint16)
            got = orc.mlp_f16(x, W1, bias, W2, kind)
            assert _ulp16(got, want).max() <= 1
    # W1 = 0: every row's hidden layer is f16(act(b1)), so out = f16(act(b1)) W2^T for every row
    zeros = np.zeros_like(W1)
    got = orc.mlp_f16(x, zeros, b1, W2, 3)
    hb = np.float16(B / (1 + np.exp(-B))).astype(np.float64)
    assert _ulp16(got, np.tile((C2 @ hb).astype(np.float16).view(np.uint16), (M, 1))).max() <= 1
    assert np.all(got == got[0])


# ---- per-row activation quantisation (reference tools/rk3576-w8a8-hostterm.c:51-68) ---

def test_quant_rows_known_answers(orc):
    # amax = 127 makes the scale exactly 1: the codes are rint of the inputs, ties to even
    A = np.array([[127.0, 2.5, -3.5, 0.5, -0.5, 1.5, -126.6, 3.49999],
                  [0.0] * 8,
                  [1.0, -2.0, 0.5, 2.0, 0.0, -0.25, 1.0e-3, -1.0]], np.float32)
    q, rs = orc.quant_rows(A)
    assert q[0].tolist() == [127, 2, -4, 0, 0, 2, -127, 3]
    assert q[1].tolist() == [0] * 8 and rs[1] == 0.0
    # amax = 2: scale 63.5, so 1.0 -> 63.5 -> 64 (even), 0.5 -> 31.75 -> 32, 0.25 -> 15.875 -> 16
    assert q[2].tolist() == [64, -127, 32, 127, 0, -16, 0, -64]
    assert rs[0] == np.float32(1.0) and rs[2] == np.float32(2.0) / np.float32(127.0)


def test_quant_rows_properties(orc):
    rng = np.random.default_rng(81)
    M, K = 64, 1024
    A = (rng.standard_normal((M, K)) * 10.0 ** rng.integers(-3, 3, (M, 1))).astype(np.float32)
    q, rs = orc.quant_rows(A)
    amax = np.abs(A).max(axis=1)
    assert np.array_equal(np.abs(q.astype(np.int32)).max(axis=1), np.full(M, 127))
    assert np.all(np.abs(q[np.arange(M), np.abs(A).argmax(axis=1)]) == 127)
    assert np.array_equal(rs, (amax / np.float32(127)).astype(np.float32))
    # dequantisation error within half a step (plus fp32 rounding of the scale)
    err = np.abs(A - rs[:, None] * q.astype(np.float32))
    assert np.all(err <= rs[:, None] * (0.5 + 1e-5))
    # odd symmetry, and exact scaling by powers of two
    qn, rsn = orc.quant_rows(-A)
    assert np.array_equal(qn, -q) and np.array_equal(rsn, rs)
    q4, rs4 = orc.quant_rows(A * np.float32(4))
    assert np.array_equal(q4, q) and np.array_equal(rs4, rs * 4)
    # idempotent on its own dequantised values when the scale is a power of two
    Ap = np.array([[-64.0, 127.0, 3.0, -128.0 / 2]], np.float32)
    qp, rp = orc.quant_rows(Ap)
    assert qp.tolist() == [[-64, 127, 3, -64]] and rp[0] == 1.0


# ---- attention (reference src/rocket_attn.c) -------------------------------------------

def _h(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def _fa_np(Q, K, V, mask, scale, softcap):
    """float64 numpy attention with the reference's fp32 score step (cast, scale, tanh, mask,
    clamp at -30000)."""
    nh, T, dk = Q.shape
    nkvh = K.shape[0]
    out = np.empty((nh, T, V.shape[1]))
    for h in range(nh):
        hk = h // (nh // nkvh)
        q = Q[h].view(np.float16).astype(np.float64)
        k = K[hk].view(np.float16).astype(np.float64)
        v = V[hk].view(np.float16).astype(np.float64)
        s = (q @ k.T).astype(np.float32) * np.float32(scale)
        if softcap:
            s = np.float32(softcap) * np.tanh(s / np.float32(softcap))
        if mask is not None:
            s = s + mask.view(np.float16).astype(np.float32)
        s = np.maximum(s, np.float32(-30000)).astype(np.float64)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[h] = (p / p.sum(axis=1, keepdims=True)) @ v.T
    return out


def test_flash_attn_closed_forms(orc):
    rng = np.random.default_rng(91)
    nh, T, n_kv, dk, dv = 2, 5, 7, 32, 16
    Q = _h(rng.uniform(-1, 1, (nh, T, dk)))
    V = _h(rng.uniform(-1, 1, (1, dv, n_kv)))
    Vf = V.view(np.float16).astype(np.float64)
    # K = 0: every score is 0, the weights uniform, the output the mean of V's columns
    K0 = np.zeros((1, n_kv, dk), np.uint16)
    got = orc.flash_attn_f16(Q, K0, V, None, 0.5, 0.0)
    want = _h(np.broadcast_to(Vf[0].mean(axis=1), (nh, T, dv)))
    assert np.array_equal(got, want)
    # a mask that leaves one key per query selects that key's V column exactly
    K = _h(rng.uniform(-1, 1, (1, n_kv, dk)))
    pick = rng.integers(0, n_kv, T)
    mask = np.full((T, n_kv), -np.inf, np.float32)
    mask[np.arange(T), pick] = 0.0
    got = orc.flash_attn_f16(Q, K, V, _h(mask), 0.5, 0.0)
    assert np.array_equal(got, np.broadcast_to(V[0][:, pick].T, (nh, T, dv)))
    # a fully masked row clamps every score to -30000: uniform weights again
    mask[:] = -np.inf
    got = orc.flash_attn_f16(Q, K, V, _h(mask), 0.5, 0.0)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("nh,nkvh,T,n_kv,dk,dv,softcap", [(4, 2, 6, 9, 32, 32, 0.0), (3, 1, 5, 40, 64, 16, 0.0),
                                                          (2, 2, 4, 12, 32, 48, 5.0)])
def test_flash_attn_matches_numpy(orc, nh, nkvh, T, n_kv, dk, dv, softcap):
    rng = np.random.default_rng(92)
    Q = _h(rng.uniform(-2, 2, (nh, T, dk)))
    K = _h(rng.uniform(-2, 2, (nkvh, n_kv, dk)))
    V = _h(rng.uniform(-1, 1, (nkvh, dv, n_kv)))
    pos = n_kv - T + np.arange(T)[:, None]
    mask = _h(np.where(np.arange(n_kv)[None, :] <= pos, 0.0, -np.inf))
    scale = 1 / np.sqrt(dk)
    got = orc.flash_attn_f16(Q, K, V, mask, scale, softcap)
    want = _fa_np(Q, K, V, mask, scale, softcap).astype(np.float16).view(np.uint16)
    d = np.abs(got.view(np.float16).astype(np.float64) - want.view(np.float16).astype(np.float64))
    assert np.all(d <= np.abs(want.view(np.float16).astype(np.float64)) * 2 ** -10 + 1e-7)
    # GQA: head h reads kv head h // (nh / nkvh), as a single-head call on that kv head shows
    for h in range(nh):
        hk = h // (nh // nkvh)
        one = orc.flash_attn_f16(Q[h:h + 1], K[hk:hk + 1], V[hk:hk + 1], mask, scale, softcap)
        assert np.array_equal(one[0], got[h])
    if softcap:   # the soft-cap changes the result
        assert not np.array_equal(got, orc.flash_attn_f16(Q, K, V, mask, scale, 0.0))


def test_mha_self_matches_numpy_and_uniform_case(orc):
    rng = np.random.default_rng(93)
    T, d, nh = 6, 64, 2
    x = _h(rng.uniform(-1, 1, (T, d)))
    W = [_h(rng.uniform(-0.1, 0.1, (d, d))) for _ in range(4)]
    b = [_h(rng.uniform(-0.1, 0.1, d)) for _ in range(4)]
    got = orc.mha_self_f16(x, W[0], b[0], W[1], None, W[2], b[2], W[3], b[3], nh)
    X = x.view(np.float16).astype(np.float64)
    f = lambda a: a.view(np.float16).astype(np.float64)
    q, k, v = X @ f(W[0]).T + f(b[0]), X @ f(W[1]).T, X @ f(W[2]).T + f(b[2])
    dh = d // nh
    ctx = np.empty((T, d))
    for h in range(nh):
        sl = slice(h * dh, (h + 1) * dh)
        s = q[:, sl] @ k[:, sl].T / np.sqrt(dh)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        ctx[:, sl] = (p / p.sum(axis=1, keepdims=True)) @ v[:, sl]
    want = (ctx @ f(W[3]).T + f(b[3])).astype(np.float16).view(np.uint16)
    d16 = np.abs(got.view(np.float16).astype(np.float64) - want.view(np.float16).astype(np.float64))
    assert np.all(d16 <= np.abs(want.view(np.float16).astype(np.float64)) * 2 ** -10 + 1e-7)
    # Wq = 0 and no bq: uniform attention, so every token's context is the mean of v
    Z = np.zeros_like(W[0])
    got0 = orc.mha_self_f16(x, Z, None, W[1], None, W[2], b[2], W[3], b[3], nh)
    want0 = (np.broadcast_to(v.mean(axis=0), (T, d)) @ f(W[3]).T + f(b[3])).astype(np.float16).view(np.uint16)
    assert np.array_equal(got0, want0)
