"""GPU parity: every matmul entry of librocketnpu, called through its C-ABI, against the
pinned CPU oracle on the same seeded inputs.

Bars: integer results bit-exact; group-wise per-group int32 partials bit-exact and the fp32
combine bit-identical to the oracle's fmaf chain (and within 1e-5 rms of fp64, the
reference's own gate); fp16 <= 1e-2, bf16 <= 2e-2, tf32 <= 5e-3 normalised error
(max|act-ref| / max|ref|, tests/matmul_bf16_tiled_rocket.c:84-111) against an fp32
reference with double accumulation.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import gworder
import rocketnpu as R

pytestmark = pytest.mark.gpu

SEED = 0x52434B00


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def f16(orc, shape, seed, lo=-1.0, hi=1.0):
    return orc.f32_to_f16_bits(orc.gen_uniform(shape, seed, lo, hi))


# ---------------------------------------------------------------------------------------
# int8
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("M,K,N", [(4, 32, 32), (1, 64, 32), (12, 96, 64), (64, 256, 128),
                                   (132, 160, 96), (256, 1024, 512)])
def test_int8_small(lib, orc, fd, M, K, N):
    say(f"int8 M={M} K={K} N={N}")
    A = orc.gen_i8((M, K), SEED + 1)
    B = orc.gen_i8((N, K), SEED + 2)
    Cg = np.full((M, N), 7, np.int32)
    assert lib.rocket_matmul_int8(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
    assert np.array_equal(Cg, orc.matmul_int8(A, B))


def test_int8_config2_full(lib, orc, fd):
    M, K, N = 512, 4096, 4096
    say("int8 config2 512x4096x4096")
    A = orc.gen_i8((M, K), 0x52434B02)
    B = orc.gen_i8((N, K), 0x52434B02 + 1)
    Cg = np.empty((M, N), np.int32)
    assert lib.rocket_matmul_int8(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
    assert np.array_equal(Cg, orc.matmul_int8(A, B))


@pytest.fixture
def split_k():
    """Raises the split-K cap to 8 for one test (int32 K slices add their sums into C with
    atomic adds; the default cap is 4)."""
    import os
    old = os.environ.get("ROCKET_HIP_SPLITK")
    os.environ["ROCKET_HIP_SPLITK"] = "8"
    yield
    if old is None:
        del os.environ["ROCKET_HIP_SPLITK"]
    else:
        os.environ["ROCKET_HIP_SPLITK"] = old


@pytest.mark.parametrize("M,K,N", [(256, 4160, 512), (100, 8192, 256), (512, 4096, 4096)])
def test_int8_split_k(lib, orc, fd, split_k, M, K, N):
    """Shapes that run as K slices: a partial last stage (4160 = 32.5 stages), a partial
    row tile (M=100) and the config-2 shape."""
    say(f"int8 split-K M={M} K={K} N={N}")
    A = orc.gen_i8((M, K), SEED + 5)
    B = orc.gen_i8((N, K), SEED + 6)
    Cg = np.full((M, N), 99, np.int32)
    assert lib.rocket_matmul_int8(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
    assert np.array_equal(Cg, orc.matmul_int8(A, B))


def test_int4_raw_split_k_and_chunked_accumulate(lib, orc, fd, split_k):
    # K > 65536 runs as two accumulating K chunks, each split into K slices
    M, K, N = 4, 65536 + 1024, 64
    say(f"int4 raw chunked M={M} K={K} N={N}")
    A = orc.gen_i8((M, K), SEED + 7)
    B = orc.gen_i8((N, K), SEED + 8, -8, 7)
    ctx = lib.rocket_i4_ctx_create(1)
    w = lib.rocket_i4_weights_pack(ctx, M, K, N, R.ptr(B))
    assert w
    Cg = np.full((M, N), 5, np.int32)
    assert lib.rocket_matmul_int4_prepacked(ctx, M, K, N, R.ptr(A), R.ptr(Cg), w) == 0
    assert np.array_equal(Cg, orc.matmul_int8(A, B))
    lib.rocket_i4_weights_free(ctx, w)
    lib.rocket_i4_ctx_free(ctx)
    M, K, N = 256, 4096, 256
    A = orc.gen_i8((M, K), SEED + 9)
    B = orc.gen_i8((N, K), SEED + 10, -8, 7)
    Cg = np.empty((M, N), np.int32)
    assert lib.rocket_matmul_int4(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
    assert np.array_equal(Cg, orc.matmul_int8(A, B))


def test_eight_wave_tiles_partial(lib, orc, fd):
    """Shapes that fill the GPU with 256x128 tiles run the 8-wave kernels (A by LDS DMA):
    int8 and int4 to int32, bf16 and fp16 to fp32, each with a partial last row tile, a
    partial last column tile and a partial last K stage."""
    M, K, N = 2000, 1056, 4032
    say(f"8-wave int8/int4 M={M} K={K} N={N}")
    A = orc.gen_i8((M, K), SEED + 50)
    B = orc.gen_i8((N, K), SEED + 51)
    Cg = np.full((M, N), 3, np.int32)
    assert lib.rocket_matmul_int8(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
    assert np.array_equal(Cg, orc.matmul_int8(A, B))
    B4 = orc.gen_i8((N, K), SEED + 52, -8, 7)
    assert lib.rocket_matmul_int4(fd, M, K, N, R.ptr(A), R.ptr(B4), R.ptr(Cg)) == 0
    assert np.array_equal(Cg, orc.matmul_int8(A, B4))
    M, K, N = 2000, 544, 4000
    say(f"8-wave bf16/fp16 M={M} K={K} N={N}")
    Af = orc.gen_normal((M, K), SEED + 53)
    Bf = orc.gen_normal((N, K), SEED + 54, 0, 0.02)
    Cf = np.full((M, N), np.nan, np.float32)
    assert lib.rocket_matmul_bf16(fd, M, K, N, R.ptr(Af), R.ptr(Bf), R.ptr(Cf)) == 0
    assert orc.norm_err(Cf, orc.matmul_bf16(Af, Bf)) < 1e-5
    A16 = f16(orc, (M, K), SEED + 55)
    B16 = f16(orc, (N, K), SEED + 56)
    assert lib.rocket_matmul_fp16_f32out(fd, M, K, N, R.ptr(A16), R.ptr(B16), R.ptr(Cf)) == 0
    assert orc.norm_err(Cf, orc.matmul_fp16_f32out(A16, B16)) < 1e-5


def test_eight_wave_dma_stages_complete(lib, orc, fd):
    """Long K loops over many 8-wave tiles, checked exactly: every stage's DMA loads must be
    in LDS before its MFMAs read them. (A wait that counted loads never issued once let a
    stage's last B rows arrive late in about one tile in five hundred.) Small integers make
    every fp32 sum exact, so float64 BLAS is an exact reference."""
    M, K, N = 2048, 4096, 8192
    A = orc.gen_i8((M, K), SEED + 57)
    B = orc.gen_i8((N, K), SEED + 58)
    want = A.astype(np.float64) @ B.astype(np.float64).T                # |sum| < 2^53: exact
    Cg = np.empty((M, N), np.int32)
    A16 = orc.f32_to_f16_bits(orc.gen_i8((M, K), SEED + 59, -3, 3).astype(np.float32))
    B16 = orc.f32_to_f16_bits(orc.gen_i8((N, K), SEED + 60, -3, 3).astype(np.float32))
    want16 = orc.f16_bits_to_f32(A16).astype(np.float64) @ orc.f16_bits_to_f32(B16).astype(np.float64).T
    Cf = np.empty((M, N), np.float32)
    for rep in range(3):
        say(f"8-wave DMA stages M={M} K={K} N={N} rep {rep}")
        assert lib.rocket_matmul_int8(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
        assert np.array_equal(Cg, want)
        assert lib.rocket_matmul_fp16_f32out(fd, M, K, N, R.ptr(A16), R.ptr(B16), R.ptr(Cf)) == 0
        assert np.array_equal(Cf, want16)                              # |sum| <= 9 K < 2^24


def test_fp16_bf16_split_k(lib, orc, fd):
    """fp16 / bf16 products with too few 256x128 tiles for the CUs and long K run as K slices
    whose fp32 partial planes a second kernel sums in slice order. Small integers keep every sum
    exact, so the result equals float64 BLAS bit for bit whatever the slicing; with random
    values repeated calls agree bit for bit and stay within the fp16 bar."""
    M, K, N = 512, 15360, 3840
    say(f"fp16/bf16 split-K M={M} K={K} N={N}")
    Ai = orc.gen_i8((M, K), SEED + 61, -1, 1).astype(np.float32)
    Bi = orc.gen_i8((N, K), SEED + 62, -1, 1).astype(np.float32)
    want = Ai.astype(np.float64) @ Bi.astype(np.float64).T
    A16, B16 = orc.f32_to_f16_bits(Ai), orc.f32_to_f16_bits(Bi)
    C16 = np.empty((M, N), np.uint16)
    assert lib.rocket_matmul_fp16(fd, M, K, N, R.ptr(A16), R.ptr(B16), R.ptr(C16)) == 0
    assert np.array_equal(C16, want.astype(np.float16).view(np.uint16))
    Cf = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_fp16_f32out(fd, M, K, N, R.ptr(A16), R.ptr(B16), R.ptr(Cf)) == 0
    assert np.array_equal(Cf, want)
    Cf[:] = np.nan
    assert lib.rocket_matmul_bf16(fd, M, K, N, R.ptr(Ai), R.ptr(Bi), R.ptr(Cf)) == 0
    assert np.array_equal(Cf, want)
    A = f16(orc, (M, K), SEED + 63)
    B = f16(orc, (N, K), SEED + 64)
    C1, C2 = np.empty((M, N), np.uint16), np.empty((M, N), np.uint16)
    assert lib.rocket_matmul_fp16(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(C1)) == 0
    assert lib.rocket_matmul_fp16(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(C2)) == 0
    assert np.array_equal(C1, C2)
    ref = orc.f16_bits_to_f32(A).astype(np.float64) @ orc.f16_bits_to_f32(B).astype(np.float64).T
    assert orc.norm_err(orc.f16_bits_to_f32(C1), ref) <= 1e-2


def test_int8_extreme_values(lib, orc, fd):
    M, K, N = 8, 4096, 64
    A = np.full((M, K), -128, np.int8)
    B = np.full((N, K), -128, np.int8)
    B[1::2] = 127
    Cg = np.empty((M, N), np.int32)
    assert lib.rocket_matmul_int8(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
    assert np.array_equal(Cg, orc.matmul_int8(A, B))


# ---------------------------------------------------------------------------------------
# int16 exact
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("M,K,N", [(4, 64, 32), (1, 32, 32), (36, 288, 96)])
def test_int16_exact_small(lib, orc, fd, M, K, N):
    say(f"int16 M={M} K={K} N={N}")
    A = orc.gen_i16((M, K), SEED + 3)
    B = orc.gen_i16((N, K), SEED + 4)
    A.flat[:6] = [32767, 32640, 32639, -32768, -32767, 32641]
    Cg = np.empty((M, N), np.int64)
    assert lib.rocket_matmul_int16_exact(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
    assert np.array_equal(Cg, orc.matmul_int16_exact(A, B))


def test_int16_exact_config2_shape(lib, orc, fd):
    M, K, N = 512, 4096, 4096
    say("int16 exact 512x4096x4096")
    A = orc.gen_i16((M, K), 0x52434B12, -32768, 32639)
    B = orc.gen_i16((N, K), 0x52434B13, -32768, 32639)
    Cg = np.empty((M, N), np.int64)
    assert lib.rocket_matmul_int16_exact(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
    rows = np.r_[0:8, 250:258, 504:512]
    ref = orc.matmul_int16_exact(np.ascontiguousarray(A[rows]), B)
    assert np.array_equal(Cg[rows], ref)


@pytest.mark.parametrize("M,K,N", [(36, 288, 96), (256, 256, 4096)])
def test_int16_exact_split_boundaries(lib, orc, fd, M, K, N):
    """Both operands drawn from the values where the byte-plane split changes behaviour: the
    clamp at 32639, the hi byte's rounding at lo = +-128, the int16 extremes. (256, 256, 4096)
    runs the 128 x 64 tiles of config 2b, (36, 288, 96) the small ones."""
    say(f"int16 split boundaries M={M} K={K} N={N}")
    edge = np.array([-32768, -32767, -32640, -32639, -129, -128, -127, -1, 0, 1, 127, 128, 129, 255, 256,
                     383, 384, 32511, 32512, 32638, 32639, 32640, 32641, 32767], np.int16)
    rng = np.random.default_rng(SEED + 16)
    A = edge[rng.integers(0, edge.size, (M, K))]
    B = edge[rng.integers(0, edge.size, (N, K))]
    Cg = np.empty((M, N), np.int64)
    assert lib.rocket_matmul_int16_exact(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
    assert np.array_equal(Cg, orc.matmul_int16_exact(A, B))


# ---------------------------------------------------------------------------------------
# fp16
# ---------------------------------------------------------------------------------------
def fp16_check(got16, A16, B16, orc, tol=1e-2):
    ref = orc.matmul_f32(orc.f16_bits_to_f32(A16), orc.f16_bits_to_f32(B16))
    got = orc.f16_bits_to_f32(got16)
    e = orc.norm_err(got, ref)
    assert e <= tol, e
    return e


def test_fp16_config1(lib, orc, fd):
    M, K, N = 64, 256, 128
    say("fp16 config1")
    A = f16(orc, (M, K), 0x52434B01)
    B = f16(orc, (N, K), 0x52434B01 + 1)
    Cg = np.empty((M, N), np.uint16)
    assert lib.rocket_matmul_fp16(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
    e = fp16_check(Cg, A, B, orc)
    # the fp32-accumulated result rounds once: within an fp16 ulp of the oracle's
    o = orc.f16_bits_to_f32(orc.matmul_fp16(A, B))
    g = orc.f16_bits_to_f32(Cg)
    assert np.max(np.abs(g - o)) <= np.max(np.abs(o)) * 2 ** -10
    say(f"  norm_err={e:.3g}")


@pytest.mark.parametrize("M,K,N", [(1, 32, 16), (4, 64, 48), (100, 320, 80)])
def test_fp16_shapes_and_f32out(lib, orc, fd, M, K, N):
    A = f16(orc, (M, K), SEED + 5)
    B = f16(orc, (N, K), SEED + 6)
    Cg = np.empty((M, N), np.uint16)
    assert lib.rocket_matmul_fp16(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
    fp16_check(Cg, A, B, orc)
    Cf = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_fp16_f32out(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cf)) == 0
    ref = orc.matmul_fp16_f32out(A, B)
    assert orc.norm_err(Cf, ref) < 1e-5


@pytest.mark.parametrize("wide", [1, 0])
@pytest.mark.parametrize("M,K,N", [(512, 1024, 30720), (500, 1056, 30720), (512, 1024, 30656)])
def test_fp16_wide_tiles(lib, orc, fd, M, K, N, wide, monkeypatch):
    """N = 30720 gives 2 x 120 tiles of 256 x 256 (the wide fp16 / bf16 tile: 8 waves of 64 x
    128, one stage in flight); M = 500 leaves a partial last row tile, K = 1056 a partial last
    stage and N = 30656 a partial last column tile. Rows across both row tiles against the
    oracle, fp16 and fp32 results; again with ROCKET_HIP_WIDE=0 (the same products on 256 x
    128 tiles)."""
    say(f"fp16 wide tiles M={M} K={K} N={N} wide={wide}")
    monkeypatch.setenv("ROCKET_HIP_WIDE", str(wide))
    A = f16(orc, (M, K), SEED + 40)
    B = f16(orc, (N, K), SEED + 41)
    rows = np.r_[0:3, 254:258, M - 3:M]
    Ar = np.ascontiguousarray(A[rows])
    Cg = np.empty((M, N), np.uint16)
    assert lib.rocket_matmul_fp16(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
    fp16_check(np.ascontiguousarray(Cg[rows]), Ar, B, orc)
    Cf = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_fp16_f32out(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cf)) == 0
    assert orc.norm_err(Cf[rows], orc.matmul_fp16_f32out(Ar, B)) < 1e-5


def test_fp16_identity_and_integers(lib, orc, fd):
    M, K = 16, 64
    A = f16(orc, (M, K), SEED + 7)
    I = orc.f32_to_f16_bits(np.eye(K, dtype=np.float32))
    Cg = np.empty((M, K), np.uint16)
    assert lib.rocket_matmul_fp16(fd, M, K, K, R.ptr(A), R.ptr(I), R.ptr(Cg)) == 0
    assert np.array_equal(Cg, A)
    Ai = orc.f32_to_f16_bits(np.round(orc.gen_uniform((M, 128), SEED + 8, -3, 3)))
    Bi = orc.f32_to_f16_bits(np.round(orc.gen_uniform((32, 128), SEED + 9, -3, 3)))
    C2 = np.empty((M, 32), np.uint16)
    assert lib.rocket_matmul_fp16(fd, M, 128, 32, R.ptr(Ai), R.ptr(Bi), R.ptr(C2)) == 0
    assert np.array_equal(C2, orc.matmul_fp16(Ai, Bi))      # every partial sum exact


# ---------------------------------------------------------------------------------------
# bf16 / tf32
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("M,K,N", [(4, 64, 16), (1, 96, 32), (132, 544, 272)])
def test_bf16_tf32_small(lib, orc, fd, M, K, N):
    A = orc.gen_normal((M, K), SEED + 10)
    B = orc.gen_normal((N, K), SEED + 11, 0, 0.02)
    ref32 = orc.matmul_f32(A, B)
    Cb = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_bf16(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cb)) == 0
    assert orc.norm_err(Cb, orc.matmul_bf16(A, B)) < 1e-5     # same truncated operands
    assert orc.norm_err(Cb, ref32) <= 2e-2
    Ct = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_tf32(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Ct)) == 0
    assert orc.norm_err(Ct, orc.matmul_tf32(A, B)) < 1e-5
    assert orc.norm_err(Ct, ref32) <= 5e-3


@pytest.mark.parametrize("M,K,N", [(132, 544, 272), (260, 1040, 400), (4, 64, 16), (512, 2048, 1024)])
def test_f32_prepass_matches_fused(lib, orc, fd, M, K, N):
    """fp32 operands converted in a separate pass (bf16, or tf32 hi/lo pairs; both operands,
    or A alone) give the same bits as conversion inside the GEMM's loads; all equal the
    oracle's truncated product.
    K = 1040 leaves a partial 64-element stage for tf32 (bf16 needs K % 32)."""
    import os
    say(f"f32 prepass M={M} K={K} N={N}")
    A = orc.gen_normal((M, K), SEED + 14)
    B = orc.gen_normal((N, K), SEED + 15, 0, 0.02)
    old = os.environ.get("ROCKET_HIP_F32_PREPASS")
    out = {}
    try:
        for path in ("0", "1", "2"):
            os.environ["ROCKET_HIP_F32_PREPASS"] = path
            for name, fn in (("bf16", lib.rocket_matmul_bf16), ("tf32", lib.rocket_matmul_tf32)):
                if name == "bf16" and K % 32:
                    continue
                C = np.full((M, N), np.nan, np.float32)
                assert fn(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(C)) == 0
                out[name, path] = C
    finally:
        if old is None:
            del os.environ["ROCKET_HIP_F32_PREPASS"]
        else:
            os.environ["ROCKET_HIP_F32_PREPASS"] = old
    # tf32: the GPU's three bf16 products drop lo*lo (<= 2^-16 of each product), which the
    # oracle keeps; the golden fixture bound
    for name, orf, tol in (("bf16", orc.matmul_bf16, 1e-5), ("tf32", orc.matmul_tf32, 5e-5)):
        if (name, "0") not in out:
            continue
        assert np.array_equal(out[name, "0"], out[name, "1"]), name
        assert np.array_equal(out[name, "0"], out[name, "2"]), name
        assert orc.norm_err(out[name, "1"], orf(A, B)) < tol, name


def test_tf32_k_multiple_of_16(lib, orc, fd):
    M, K, N = 8, 48, 16
    A = orc.gen_normal((M, K), SEED + 12)
    B = orc.gen_normal((N, K), SEED + 13)
    Ct = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_tf32(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Ct)) == 0
    assert orc.norm_err(Ct, orc.matmul_tf32(A, B)) < 1e-5


def test_bf16_tf32_config4(lib, orc, fd):
    M, K, N = 2048, 15360, 3840
    say("bf16/tf32 config4")
    A = orc.gen_normal((M, K), 0x52434B04)
    B = orc.gen_normal((N, K), 0x52434B04 + 1, 0.0, 0.02)
    # rows from every 256-row tile: both ends of tiles 0 and 7, a tile boundary, and one row
    # inside each other tile
    rows = np.r_[0:4, 255:257, 300, 600, 1022:1026, 1300, 1600, 1900, 2044:2048]
    assert set(rows // 256) == set(range(8))
    Ar = np.ascontiguousarray(A[rows])
    ref32 = orc.matmul_f32(Ar, B)
    for name, fn, orf, tol in (("bf16", lib.rocket_matmul_bf16, orc.matmul_bf16, 2e-2),
                               ("tf32", lib.rocket_matmul_tf32, orc.matmul_tf32, 5e-3)):
        Cg = np.empty((M, N), np.float32)
        assert fn(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
        e_trunc = orc.norm_err(Cg[rows], orf(Ar, B))
        e32 = orc.norm_err(Cg[rows], ref32)
        say(f"  {name}: vs truncated ref {e_trunc:.3g}, vs fp32 ref {e32:.3g}")
        assert e_trunc < 1e-4 and e32 <= tol


@pytest.fixture
def band_env():
    """Sets ROCKET_HIP_BANDM for a test (row-band height of one-problem launches; unset = the
    library's choice) and restores it afterwards."""
    import os
    old = os.environ.get("ROCKET_HIP_BANDM")

    def set_(v):
        if v is None:
            os.environ.pop("ROCKET_HIP_BANDM", None)
        else:
            os.environ["ROCKET_HIP_BANDM"] = str(v)
    yield set_
    set_(old)


# band heights: off, one row tile, three (the last band shorter), the library's choice
BANDS = (0, 1, 3, None)


def test_row_bands_int_and_groupwise(lib, orc, fd, band_env):
    """One-problem launches whose heavy tiles run in row bands: every band height gives the
    oracle's exact results. int8 1792 x 256 x 1024 (7 row tiles of 256: bands of 3 leave one
    of 1), and the reference MoE entry's per-expert shape at short K (1024 x 256 x 1408, group
    32, 8 row tiles of 128, 22 column blocks)."""
    M, K, N = 1792, 256, 1024
    A = orc.gen_i8((M, K), SEED + 60)
    B = orc.gen_i8((N, K), SEED + 61)
    ref = orc.matmul_int8(A, B)
    for h in BANDS:
        say(f"row bands int8 M={M} K={K} N={N} bandm={h}")
        band_env(h)
        Cg = np.full((M, N), 0x5A5A5A5A, np.int32)
        assert lib.rocket_matmul_int8(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
        assert np.array_equal(Cg, ref)
    M, K, N, group = 1024, 256, 1408, 32
    A, B, asc, bsc = gw_inputs(orc, M, K, N, group, SEED + 62)
    ref = orc.matmul_gw_f32(A, B, asc, bsc, group)
    ctx = lib.rocket_i8_ctx_create(1)
    w = lib.rocket_i8_weights_pack_gw(ctx, 4, K, N, R.ptr(B), group)
    assert w
    for h in BANDS:
        say(f"row bands int8 gw M={M} K={K} N={N} g={group} bandm={h}")
        band_env(h)
        Cf = np.full((M, N), np.nan, np.float32)
        assert lib.rocket_matmul_int8_prepacked_gw(ctx, M, K, N, R.ptr(A), R.ptr(asc), R.ptr(bsc), R.ptr(Cf), w) == 0
        assert np.array_equal(Cf, ref)
    lib.rocket_i8_weights_free(ctx, w)
    lib.rocket_i8_ctx_free(ctx)


def test_row_bands_fp16_bf16(lib, orc, fd, band_env):
    """fp16 1280 x 128 x 2048 and bf16 1280 x 256 x 1024 (5 row tiles of 256: bands of 3 leave
    one of 2), and fp16 1024 x 16384 x 1024 in 8 K slices: each band height gives the bits of
    the plain order, which matches the oracle on rows from every row tile."""
    rows = np.r_[0:3, 254:258, 511, 767, 1023:1026, 1277:1280]
    M, K, N = 1280, 128, 2048
    A = f16(orc, (M, K), SEED + 63)
    B = f16(orc, (N, K), SEED + 64)
    outs = []
    for h in BANDS:
        say(f"row bands fp16 M={M} K={K} N={N} bandm={h}")
        band_env(h)
        Cg = np.full((M, N), 0x7E00, np.uint16)
        assert lib.rocket_matmul_fp16(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
        outs.append(Cg)
    fp16_check(np.ascontiguousarray(outs[0][rows]), np.ascontiguousarray(A[rows]), B, orc)
    for Cg in outs[1:]:
        assert np.array_equal(Cg, outs[0])
    M, K, N = 1280, 256, 1024
    A = orc.gen_normal((M, K), SEED + 65)
    B = orc.gen_normal((N, K), SEED + 66, 0.0, 0.02)
    outs = []
    for h in BANDS:
        say(f"row bands bf16 M={M} K={K} N={N} bandm={h}")
        band_env(h)
        Cg = np.full((M, N), np.nan, np.float32)
        assert lib.rocket_matmul_bf16(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
        outs.append(Cg)
    Ar = np.ascontiguousarray(A[rows])
    assert orc.norm_err(outs[0][rows], orc.matmul_bf16(Ar, B)) < 1e-4
    for Cg in outs[1:]:
        assert np.array_equal(Cg, outs[0])
    # fp16 in 8 K slices (fp32 planes summed in slice order): 32 tiles of 256 x 128 x 8 slices,
    # the slices of a tile adjacent in the workgroup order, 4 row tiles in bands
    import os
    old_split = os.environ.get("ROCKET_HIP_SPLITK")
    os.environ["ROCKET_HIP_SPLITK"] = "8"
    try:
        M, K, N = 1024, 16384, 1024
        A = f16(orc, (M, K), SEED + 67)
        B = f16(orc, (N, K), SEED + 68)
        rows = np.r_[0:3, 255:258, 511, 767:770, 1021:1024]
        outs = []
        for h in BANDS:
            say(f"row bands fp16 K slices M={M} K={K} N={N} bandm={h}")
            band_env(h)
            Cg = np.full((M, N), 0x7E00, np.uint16)
            assert lib.rocket_matmul_fp16(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
            outs.append(Cg)
        fp16_check(np.ascontiguousarray(outs[0][rows]), np.ascontiguousarray(A[rows]), B, orc)
        for Cg in outs[1:]:
            assert np.array_equal(Cg, outs[0])
    finally:
        if old_split is None:
            os.environ.pop("ROCKET_HIP_SPLITK", None)
        else:
            os.environ["ROCKET_HIP_SPLITK"] = old_split


# ---------------------------------------------------------------------------------------
# group-wise int8 / int4
# ---------------------------------------------------------------------------------------
def gw_inputs(orc, M, K, N, group, seed, b_lo=-128, b_hi=127):
    nG = K // group
    A = orc.gen_i8((M, K), seed)
    B = orc.gen_i8((N, K), seed + 1, b_lo, b_hi)
    asc = orc.gen_uniform((M, nG), seed + 2, 0.5, 1.5)
    bsc = orc.gen_uniform((N, nG), seed + 3, 0.005, 0.02)
    return A, B, asc, bsc


# (8, 160, 64, 32) and (4, 416, 64, 32): a partial last stage whose four-group scale window
# is moved back to end inside each row (nG = 5 and 13); (4, 64, 32, 32): nG < 4, the arrays'
# last rows load their window early
@pytest.mark.parametrize("M,K,N,group", [(4, 64, 32, 32), (8, 256, 64, 64), (12, 288, 96, 96),
                                         (16, 512, 64, 128), (64, 1152, 128, 576), (4, 2048, 32, 2048),
                                         (8, 160, 64, 32), (4, 416, 64, 32)])
def test_int8_groupwise(lib, orc, fd, M, K, N, group):
    say(f"int8 gw M={M} K={K} N={N} g={group}")
    A, B, asc, bsc = gw_inputs(orc, M, K, N, group, SEED + 20)
    Cf = np.empty((M, N), np.float32)
    nG = K // group
    P = np.empty((M, nG, N), np.int32)
    assert lib.rocket_matmul_int8_groupwise_dump(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(asc), R.ptr(bsc),
                                                 R.ptr(Cf), group, 0, M, R.ptr(P)) == 0
    assert np.array_equal(P, orc.gw_partials(A, B, group))
    assert np.array_equal(Cf, orc.matmul_gw_f32(A, B, asc, bsc, group))
    assert orc.rms_err(Cf, orc.matmul_gw_f64(A, B, asc, bsc, group)) <= 1e-5
    C2 = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_int8_groupwise(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(asc), R.ptr(bsc),
                                            R.ptr(C2), group) == 0
    assert np.array_equal(C2, Cf)


@pytest.mark.parametrize("M,K,N,group", [(4, 128, 64, 32), (8, 256, 128, 128), (12, 384, 64, 96), (4, 416, 64, 32)])
def test_int4_groupwise(lib, orc, fd, M, K, N, group):
    A, B, asc, bsc = gw_inputs(orc, M, K, N, group, SEED + 30, -8, 7)
    Cf = np.empty((M, N), np.float32)
    nG = K // group
    P = np.empty((M, nG, N), np.int32)
    assert lib.rocket_matmul_int4_groupwise_dump(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(asc), R.ptr(bsc),
                                                 R.ptr(Cf), group, 0, M, R.ptr(P)) == 0
    assert np.array_equal(P, orc.gw_partials(A, B, group))
    assert np.array_equal(Cf, orc.matmul_gw_f32(A, B, asc, bsc, group))


def test_int4_groupwise_config3(lib, orc, fd):
    """W4A8 at the Gemma-12B FFN-up shape: int8 activations round(N(0,1)*32) clipped, per-row
    fp32 scale, int4 weights in [-8,7] with fp16 group scales (group 128)."""
    M, K, N, group = 512, 3840, 15360, 128
    nG = K // group
    say("int4 gw config3")
    x = orc.gen_normal((M, K), 0x52434B03)
    A = np.clip(np.round(x * 32), -128, 127).astype(np.int8)
    row_scale = (np.abs(x).max(axis=1) / 127).astype(np.float32)
    asc = np.ascontiguousarray(np.repeat(row_scale[:, None], nG, axis=1))
    B = orc.gen_i8((N, K), 0x52434B03 + 1, -8, 7)
    bsc = orc.f16_bits_to_f32(orc.f32_to_f16_bits(orc.gen_uniform((N, nG), 0x52434B03 + 2, 0.005, 0.02)))
    rows = np.r_[0:4, 255:259, 508:512]
    Cf = np.empty((M, N), np.float32)
    P = np.empty((4, nG, N), np.int32)
    assert lib.rocket_matmul_int4_groupwise_dump(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(asc), R.ptr(bsc),
                                                 R.ptr(Cf), group, 255, 4, R.ptr(P)) == 0
    assert np.array_equal(P, orc.gw_partials(np.ascontiguousarray(A[255:259]), B, group))
    Ar, ar = np.ascontiguousarray(A[rows]), np.ascontiguousarray(asc[rows])
    # one scale per row in the reference layout: the row-scale fold order
    assert gworder.row_order(asc)
    assert np.array_equal(Cf[rows], orc.matmul_gw_rowscale_f32(Ar, B, np.ascontiguousarray(row_scale[rows]), bsc, group))
    ref = orc.matmul_gw_f64(Ar, B, ar, bsc, group)
    rel = orc.norm_err(Cf[rows], ref)
    say(f"  config3 norm rel err vs fp64 {rel:.3g}")
    assert rel <= 1e-3


@pytest.mark.parametrize("M,K,N,group", [(4, 64, 32, 32), (8, 256, 64, 64), (12, 288, 96, 96),
                                         (132, 512, 192, 128), (64, 1152, 128, 576), (260, 2048, 256, 256),
                                         (2000, 1024, 4032, 128), (1000, 640, 8064, 32)])
def test_groupwise_rowscale(lib, orc, fd, M, K, N, group):
    say(f"gw rowscale M={M} K={K} N={N} g={group}")
    nG = K // group
    A = orc.gen_i8((M, K), SEED + 80)
    B8 = orc.gen_i8((N, K), SEED + 81)
    B4 = orc.gen_i8((N, K), SEED + 82, -8, 7)
    arow = orc.gen_uniform((M,), SEED + 83, 0.5, 1.5)
    bsc = orc.gen_uniform((N, nG), SEED + 84, 0.005, 0.02)
    for entry, B in (("rocket_matmul_int8_groupwise_rowscale", B8), ("rocket_matmul_int4_groupwise_rowscale", B4)):
        if entry.startswith("rocket_matmul_int4") and (49 * group >= 32767 or N % 64):
            continue   # the int4 entries keep the reference's N % 64 and group bounds
        Cf = np.full((M, N), np.nan, np.float32)
        assert getattr(lib, entry)(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(arow), R.ptr(bsc), R.ptr(Cf), group) == 0
        assert np.array_equal(Cf, orc.matmul_gw_rowscale_f32(A, B, arow, bsc, group)), entry
    # unit row scales reproduce the reference-layout entry with unit activation scales bit for bit
    ones = np.ones(M, np.float32)
    Cr = np.empty((M, N), np.float32)
    Co = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_int8_groupwise_rowscale(fd, M, K, N, R.ptr(A), R.ptr(B8), R.ptr(ones), R.ptr(bsc),
                                                     R.ptr(Cr), group) == 0
    onesg = np.ones((M, nG), np.float32)
    assert lib.rocket_matmul_int8_groupwise(fd, M, K, N, R.ptr(A), R.ptr(B8), R.ptr(onesg), R.ptr(bsc),
                                            R.ptr(Co), group) == 0
    assert np.array_equal(Cr, Co)


def test_int4_prepacked_rowscale_config3(lib, orc, fd):
    """Config 3 through the resident int4 weight with per-row activation scales (the bench
    path): sampled rows bit-identical to the oracle's order, fp64 agreement <= 1e-3."""
    M, K, N, group = 512, 3840, 15360, 128
    nG = K // group
    say("int4 prepacked rowscale config3")
    x = orc.gen_normal((M, K), 0x52434B03)
    A = np.clip(np.round(x * 32), -128, 127).astype(np.int8)
    arow = (np.abs(x).max(axis=1) / 127).astype(np.float32)
    B = orc.gen_i8((N, K), 0x52434B03 + 1, -8, 7)
    bsc = orc.f16_bits_to_f32(orc.f32_to_f16_bits(orc.gen_uniform((N, nG), 0x52434B03 + 2, 0.005, 0.02)))
    ctx = lib.rocket_i4_ctx_create(1)
    w = lib.rocket_i4_weights_pack_gw(ctx, M, K, N, R.ptr(B), group)
    assert w
    Cf = np.empty((M, N), np.float32)
    for _ in range(2):   # resident weight reused
        assert lib.rocket_matmul_int4_prepacked_gw_rowscale(ctx, M, K, N, R.ptr(A), R.ptr(arow), R.ptr(bsc),
                                                            R.ptr(Cf), w) == 0
    rows = np.r_[0:4, 127:133, 255:259, 508:512]
    Ar = np.ascontiguousarray(A[rows])
    assert np.array_equal(Cf[rows], orc.matmul_gw_rowscale_f32(Ar, B, np.ascontiguousarray(arow[rows]), bsc, group))
    asc = np.ascontiguousarray(np.repeat(arow[rows][:, None], nG, axis=1))
    rel = orc.norm_err(Cf[rows], orc.matmul_gw_f64(Ar, B, asc, bsc, group))
    say(f"  config3 rowscale norm rel err vs fp64 {rel:.3g}")
    assert rel <= 1e-3
    assert np.all(np.isfinite(Cf))
    lib.rocket_i4_weights_free(ctx, w)
    lib.rocket_i4_ctx_free(ctx)


def test_integer_k_tail_dma_tiles(lib, orc, fd):
    """Integer DMA tiles (8-wave 256 x 128: M > 128 and enough tiles for the CUs; 4-wave
    128 x 64 int8 otherwise) with a partial last K stage (K % 128 = 64): only B's tail chunks
    are zeroed; A's tail bytes (the next row's values, or zero past the last row) meet those
    zeros. Large A values everywhere make any leak visible."""
    M, K, N = 260, 4160, 8192
    say(f"integer K tail M={M} K={K} N={N}")
    A = orc.gen_i8((M, K), SEED + 90, 100, 127)
    B8 = orc.gen_i8((N, K), SEED + 91)
    B4 = orc.gen_i8((N, K), SEED + 92, -8, 7)
    Cg = np.empty((M, N), np.int32)
    assert lib.rocket_matmul_int8(fd, M, K, N, R.ptr(A), R.ptr(B8), R.ptr(Cg)) == 0
    assert np.array_equal(Cg, orc.matmul_int8(A, B8))
    # 128 x 64 DMA tiles (too few 256 x 128 tiles at N = 4096), same K tail
    N2 = 4096
    C2 = np.empty((M, N2), np.int32)
    assert lib.rocket_matmul_int8(fd, M, K, N2, R.ptr(A), R.ptr(B8[:N2].copy()), R.ptr(C2)) == 0
    assert np.array_equal(C2, orc.matmul_int8(A, B8[:N2].copy()))
    assert lib.rocket_matmul_int4_ex(fd, M, K, N, R.ptr(A), R.ptr(B4), R.ptr(Cg), 480) == 0
    assert np.array_equal(Cg, orc.matmul_int8(A, B4))
    group, N = 32, 12288          # the group-wise 256 x 128 tile wants 3/4 of the CUs busy
    B4 = orc.gen_i8((N, K), SEED + 95, -8, 7)
    arow = orc.gen_uniform((M,), SEED + 93, 0.5, 1.5)
    bsc = orc.gen_uniform((N, K // group), SEED + 94, 0.005, 0.02)
    Cf = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_int4_groupwise_rowscale(fd, M, K, N, R.ptr(A), R.ptr(B4), R.ptr(arow), R.ptr(bsc),
                                                    R.ptr(Cf), group) == 0
    assert np.array_equal(Cf, orc.matmul_gw_rowscale_f32(A, B4, arow, bsc, group))


def test_int4_raw(lib, orc, fd):
    M, K, N = 12, 512, 128
    A = orc.gen_i8((M, K), SEED + 40, -8, 7)
    B = orc.gen_i8((N, K), SEED + 41, -8, 7)
    Cg = np.empty((M, N), np.int32)
    assert lib.rocket_matmul_int4(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
    assert np.array_equal(Cg, orc.matmul_int8(A, B))
    A8 = orc.gen_i8((M, K), SEED + 42)     # W4A8: full int8 activations
    assert lib.rocket_matmul_int4_ex(fd, M, K, N, R.ptr(A8), R.ptr(B), R.ptr(Cg), 480) == 0
    assert np.array_equal(Cg, orc.matmul_int8(A8, B))
    C1 = np.empty((1, N), np.int32)
    assert lib.rocket_matmul_int4(fd, 1, K, N, R.ptr(A8), R.ptr(B), R.ptr(C1)) == 0
    assert np.array_equal(C1[0], Cg[0])


# ---------------------------------------------------------------------------------------
# resident weights
# ---------------------------------------------------------------------------------------
def test_i8_resident_matches_oneshot_and_guards(lib, orc, fd):
    K, N, group = 2880, 512, 576
    nG = K // group
    ctx = lib.rocket_i8_ctx_create(3)
    assert ctx
    B = orc.gen_i8((N, K), SEED + 50)
    bsc = orc.gen_uniform((N, nG), SEED + 51, 0.5, 1.5)
    wg = lib.rocket_i8_weights_pack_gw(ctx, 256, K, N, R.ptr(B), group)
    wc = lib.rocket_i8_weights_pack(ctx, 256, K, N, R.ptr(B))
    assert wg and wc
    assert lib.rocket_i8_weights_bytes(wg) <= 1.2 * N * K
    for M in (512, 256, 768, 64, 8):
        A = orc.gen_i8((M, K), SEED + 52 + M)
        asc = orc.gen_uniform((M, nG), SEED + 53 + M, 0.5, 1.5)
        Cr = np.empty((M, N), np.float32)
        Co = np.empty((M, N), np.float32)
        assert lib.rocket_matmul_int8_prepacked_gw(ctx, M, K, N, R.ptr(A), R.ptr(asc), R.ptr(bsc), R.ptr(Cr), wg) == 0
        assert lib.rocket_matmul_int8_groupwise(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(asc), R.ptr(bsc), R.ptr(Co), group) == 0
        assert np.array_equal(Cr, Co)
        rows = np.unique(np.r_[0:4, M // 2, M - 4:M])
        Ar, ar = np.ascontiguousarray(A[rows]), np.ascontiguousarray(asc[rows])
        assert np.array_equal(Cr[rows], orc.matmul_gw_f32(Ar, B, ar, bsc, group))
        assert orc.rms_err(Cr[rows], orc.matmul_gw_f64(Ar, B, ar, bsc, group)) <= 1e-5
        C32 = np.empty((M, N), np.int32)
        assert lib.rocket_matmul_int8_prepacked(ctx, M, K, N, R.ptr(A), R.ptr(C32), wc) == 0
        assert np.array_equal(C32, orc.matmul_int8(A, B))
    A = orc.gen_i8((8, K), 1)
    C32 = np.empty((8, N), np.int32)
    assert lib.rocket_matmul_int8_prepacked(ctx, 8, K, N, R.ptr(A), R.ptr(C32), wg) < 0   # wrong mode
    Cf = np.empty((8, N), np.float32)
    asc = np.ones((8, nG), np.float32)
    assert lib.rocket_matmul_int8_prepacked_gw(ctx, 8, K, N, R.ptr(A), R.ptr(asc), R.ptr(bsc), R.ptr(Cf), wc) < 0
    for bad in (1, 2, 3, 5, 6):
        assert lib.rocket_matmul_int8_prepacked_gw(ctx, bad, K, N, R.ptr(A), R.ptr(asc), R.ptr(bsc), R.ptr(Cf), wg) < 0
    assert lib.rocket_matmul_int8_prepacked_gw(ctx, 8, K + 32, N, R.ptr(A), R.ptr(asc), R.ptr(bsc), R.ptr(Cf), wg) < 0
    lib.rocket_i8_weights_free(ctx, wg)
    lib.rocket_i8_weights_free(ctx, wc)
    lib.rocket_i8_ctx_free(ctx)


def test_i4_resident_matches_oneshot(lib, orc, fd):
    M, K, N, group = 64, 1024, 256, 128
    nG = K // group
    ctx = lib.rocket_i4_ctx_create(1)
    A, B, asc, bsc = gw_inputs(orc, M, K, N, group, SEED + 60, -8, 7)
    w = lib.rocket_i4_weights_pack_gw(ctx, M, K, N, R.ptr(B), group)
    assert w and lib.rocket_i4_weights_bytes(w) == N * K // 2
    Cr = np.empty((M, N), np.float32)
    Co = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_int4_prepacked_gw(ctx, M, K, N, R.ptr(A), R.ptr(asc), R.ptr(bsc), R.ptr(Cr), w) == 0
    assert lib.rocket_matmul_int4_groupwise(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(asc), R.ptr(bsc), R.ptr(Co), group) == 0
    assert np.array_equal(Cr, Co)
    assert np.array_equal(Cr, orc.matmul_gw_f32(A, B, asc, bsc, group))
    C32 = np.empty((M, N), np.int32)
    assert lib.rocket_matmul_int4_prepacked(ctx, M, K, N, R.ptr(A), R.ptr(C32), w) == 0
    assert np.array_equal(C32, orc.matmul_int8(A, B))
    assert lib.rocket_matmul_int4_prepacked_gw(ctx, 6, K, N, R.ptr(A), R.ptr(asc), R.ptr(bsc), R.ptr(Cr), w) < 0
    lib.rocket_i4_weights_free(ctx, w)
    lib.rocket_i4_ctx_free(ctx)


def test_fp16_resident_stream_fused_batch_mt(lib, orc, fd):
    M, K, N = 64, 256, 96
    A = f16(orc, (M, K), SEED + 70)
    B = f16(orc, (N, K), SEED + 71)
    Co = np.empty((M, N), np.uint16)
    assert lib.rocket_matmul_fp16(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Co)) == 0
    fp16_check(Co, A, B, orc)
    ctx = lib.rocket_ctx_create(3)
    w = lib.rocket_weights_pack(ctx, 256, K, N, R.ptr(B))
    assert w
    for Mc in (M, 8):
        Cr = np.empty((Mc, N), np.uint16)
        assert lib.rocket_matmul_fp16_prepacked(ctx, Mc, K, N, R.ptr(A), R.ptr(Cr), w) == 0
        assert np.array_equal(Cr, Co[:Mc])
        fp16_check(Cr, np.ascontiguousarray(A[:Mc]), B, orc)
    assert lib.rocket_matmul_fp16_prepacked(ctx, M, K + 32, N, R.ptr(A), R.ptr(Co), w) < 0
    lib.rocket_weights_free(ctx, w)
    lib.rocket_ctx_free(ctx)
    s = lib.rocket_stream_create(3)
    Cs = np.empty((M, N), np.uint16)
    assert lib.rocket_matmul_fp16_stream(s, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cs)) == 0
    assert np.array_equal(Cs, Co)
    fp16_check(Cs, A, B, orc)
    B2 = f16(orc, (32, K), SEED + 72)
    Bs, keep = R.ptr_array([B, B2])
    Ns, keep2 = R.int_array([N, 32])
    Cfz = np.empty((M, N + 32), np.uint16)
    assert lib.rocket_matmul_fp16_stream_fused(s, M, K, Bs, Ns, 2, R.ptr(A), R.ptr(Cfz)) == 0
    C2 = np.empty((M, 32), np.uint16)
    assert lib.rocket_matmul_fp16(fd, M, K, 32, R.ptr(A), R.ptr(B2), R.ptr(C2)) == 0
    assert np.array_equal(Cfz[:, :N], Co) and np.array_equal(Cfz[:, N:], C2)
    fp16_check(np.ascontiguousarray(Cfz), A, np.concatenate([B, B2]), orc)   # the fused N against the stacked weights
    lib.rocket_stream_free(s)
    Cm = np.empty((M, N), np.uint16)
    assert lib.rocket_matmul_fp16_mt(M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cm), 3) == 0
    assert np.array_equal(Cm, Co)
    fp16_check(Cm, A, B, orc)
    # batch: three items, bit-identical to per-item calls
    As = [f16(orc, (M, K), SEED + 80 + i) for i in range(3)]
    Bb = [f16(orc, (N, K), SEED + 90 + i) for i in range(3)]
    Cb = [np.empty((M, N), np.uint16) for _ in range(3)]
    pa, k1 = R.ptr_array(As)
    pb, k2 = R.ptr_array(Bb)
    pc, k3 = R.ptr_array(Cb)
    assert lib.rocket_matmul_fp16_batch(fd, M, K, N, 3, pa, pb, pc) == 0
    for i in range(3):
        Ci = np.empty((M, N), np.uint16)
        assert lib.rocket_matmul_fp16(fd, M, K, N, R.ptr(As[i]), R.ptr(Bb[i]), R.ptr(Ci)) == 0
        assert np.array_equal(Cb[i], Ci)
        fp16_check(Cb[i], As[i], Bb[i], orc)


def test_mm_batch_context(lib, orc, fd):
    """rocket_mm_batch_create/run/free (reference rocket_matmul.h:80-115): a context runs
    the same shape twice, then a new shape, each bit-identical to rocket_matmul_fp16_batch
    and within the fp16 gate of the fp32 reference."""
    b = lib.rocket_mm_batch_create(fd)
    assert b
    for M, K, N, nb, seed in ((64, 256, 96, 3, 0), (64, 256, 96, 3, 10), (132, 512, 272, 5, 20)):
        say(f"mm_batch M={M} K={K} N={N} nbatch={nb}")
        As = [f16(orc, (M, K), SEED + 1300 + seed + i) for i in range(nb)]
        Bs = [f16(orc, (N, K), SEED + 1400 + seed + i) for i in range(nb)]
        Cr = [np.empty((M, N), np.uint16) for _ in range(nb)]
        Co = [np.empty((M, N), np.uint16) for _ in range(nb)]
        pa, k1 = R.ptr_array(As)
        pb, k2 = R.ptr_array(Bs)
        pr, k3 = R.ptr_array(Cr)
        po, k4 = R.ptr_array(Co)
        assert lib.rocket_mm_batch_run(b, M, K, N, nb, pa, pb, pr) == 0
        assert lib.rocket_matmul_fp16_batch(fd, M, K, N, nb, pa, pb, po) == 0
        for i in range(nb):
            assert np.array_equal(Cr[i], Co[i])
            fp16_check(Cr[i], As[i], Bs[i], orc)
    assert lib.rocket_mm_batch_run(b, 6, 256, 96, 2, pa, pb, pr) == R.ROCKET_E_SHAPE   # M % 4
    assert lib.rocket_mm_batch_run(None, 64, 256, 96, 2, pa, pb, pr) == R.ROCKET_E_SHAPE
    lib.rocket_mm_batch_free(b)


def test_bf16_stream_and_mt(lib, orc, fd):
    M, K, N = 32, 128, 64
    A = orc.gen_normal((M, K), SEED + 100)
    B = orc.gen_normal((N, K), SEED + 101)
    Co = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_bf16(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Co)) == 0
    ref = orc.matmul_bf16(A, B)
    assert orc.norm_err(Co, ref) < 1e-5
    Cm = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_bf16_mt(M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cm), 3) == 0
    assert np.array_equal(Cm, Co)
    s = lib.rocket_bf16_stream_create(3)
    Cs = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_bf16_stream(s, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cs)) == 0
    assert np.array_equal(Cs, Co)
    assert orc.norm_err(Cs, ref) < 1e-5 and orc.norm_err(Cm, ref) < 1e-5
    lib.rocket_bf16_stream_free(s)


def test_moe_grouped_matches_per_expert(lib, orc, fd):
    """Config-5 structure at reduced size: 8 experts, group 32, ragged per-expert M."""
    E, K, N, group = 8, 512, 192, 32
    nG = K // group
    ctx = lib.rocket_i8_ctx_create(1)
    Ws, bss = [], []
    for e in range(E):
        B = orc.gen_i8((N, K), SEED + 200 + e)
        Ws.append(lib.rocket_i8_weights_pack_gw(ctx, 4, K, N, R.ptr(B), group))
        bss.append(orc.gen_uniform((N, nG), SEED + 300 + e, 0.005, 0.02))
        assert Ws[-1]
    Ms = [0, 4, 8, 12, 64, 100, 4, 132]
    As = [orc.gen_i8((max(m, 4), K), SEED + 400 + e) for e, m in enumerate(Ms)]
    ass = [orc.gen_uniform((max(m, 4), nG), SEED + 500 + e, 0.5, 1.5) for e, m in enumerate(Ms)]
    Cs = [np.full((max(m, 4), N), -1.0, np.float32) for m in Ms]
    pM, k0 = R.int_array(Ms)
    pA, k1 = R.ptr_array(As)
    pas, k2 = R.ptr_array(ass)
    pbs, k3 = R.ptr_array(bss)
    pC, k4 = R.ptr_array(Cs)
    pW = (C.c_void_p * E)(*Ws)
    assert lib.rocket_matmul_int8_prepacked_gw_grouped(ctx, E, pM, K, N, pA, pas, pbs, pC,
                                                       C.cast(pW, R.pp)) == 0
    for e, m in enumerate(Ms):
        if m == 0:
            assert np.all(Cs[e] == -1.0)
            continue
        Ce = np.empty((m, N), np.float32)
        assert lib.rocket_matmul_int8_prepacked_gw(ctx, m, K, N, R.ptr(As[e]), R.ptr(ass[e]), R.ptr(bss[e]),
                                                   R.ptr(Ce), Ws[e]) == 0
        assert np.array_equal(Cs[e][:m], Ce)
        Ae, ae = np.ascontiguousarray(As[e][:m]), np.ascontiguousarray(ass[e][:m])
        Be = orc.gen_i8((N, K), SEED + 200 + e)
        assert np.array_equal(Ce, orc.matmul_gw_f32(Ae, Be, ae, bss[e], group))
    for w in Ws:
        lib.rocket_i8_weights_free(ctx, w)
    lib.rocket_i8_ctx_free(ctx)


def test_moe_grouped_rowscale(lib, orc, fd):
    E, K, N, group = 8, 512, 192, 32
    nG = K // group
    ctx = lib.rocket_i8_ctx_create(1)
    Ws, bss = [], []
    for e in range(E):
        B = orc.gen_i8((N, K), SEED + 700 + e)
        Ws.append(lib.rocket_i8_weights_pack_gw(ctx, 4, K, N, R.ptr(B), group))
        bss.append(orc.gen_uniform((N, nG), SEED + 710 + e, 0.005, 0.02))
        assert Ws[-1]
    Ms = [16, 0, 4, 260, 8, 64, 132, 12]
    As = [orc.gen_i8((max(m, 4), K), SEED + 720 + e) for e, m in enumerate(Ms)]
    ars = [orc.gen_uniform((max(m, 4),), SEED + 730 + e, 0.5, 1.5) for e, m in enumerate(Ms)]
    Cs = [np.full((max(m, 4), N), -1.0, np.float32) for m in Ms]
    pM, k0 = R.int_array(Ms)
    pA, k1 = R.ptr_array(As)
    par, k2 = R.ptr_array(ars)
    pbs, k3 = R.ptr_array(bss)
    pC, k4 = R.ptr_array(Cs)
    pW = (C.c_void_p * E)(*Ws)
    assert lib.rocket_matmul_int8_prepacked_gw_grouped_rowscale(ctx, E, pM, K, N, pA, par, pbs, pC,
                                                                C.cast(pW, R.pp)) == 0
    # fp16 results: the fp32 results rounded once
    Hs = [np.full((max(m, 4), N), 0x7E00, np.uint16) for m in Ms]
    pH, k5 = R.ptr_array(Hs)
    assert lib.rocket_matmul_int8_prepacked_gw_grouped_rowscale_f16out(ctx, E, pM, K, N, pA, par, pbs, pH,
                                                                       C.cast(pW, R.pp)) == 0
    for e, m in enumerate(Ms):
        if m == 0:
            assert np.all(Cs[e] == -1.0) and np.all(Hs[e] == 0x7E00)
            continue
        assert np.array_equal(Hs[e][:m], Cs[e][:m].astype(np.float16).view(np.uint16))
        Ce = np.empty((m, N), np.float32)
        assert lib.rocket_matmul_int8_prepacked_gw_rowscale(ctx, m, K, N, R.ptr(As[e]), R.ptr(ars[e]), R.ptr(bss[e]),
                                                            R.ptr(Ce), Ws[e]) == 0
        assert np.array_equal(Cs[e][:m], Ce)
        assert np.array_equal(Ce, orc.matmul_gw_rowscale_f32(np.ascontiguousarray(As[e][:m]),
                                                             orc.gen_i8((N, K), SEED + 700 + e),
                                                             np.ascontiguousarray(ars[e][:m]), bss[e], group))
    for w in Ws:
        lib.rocket_i8_weights_free(ctx, w)
    lib.rocket_i8_ctx_free(ctx)


# ---------------------------------------------------------------------------------------
# per-row activation quantisation (rocket_quant.h) and the fp32-input resident products
# ---------------------------------------------------------------------------------------
def quant_inputs(orc, M, K, seed):
    A = orc.gen_normal((M, K), seed) * np.float32(3.0)
    A[1] = 0.0                                             # an all-zero row
    A[2, :8] = [127.0, 2.5, -3.5, 0.5, -0.5, 1.5, -126.6, 3.49999]   # ties at scale 1
    A[2, 8:] = np.clip(A[2, 8:], -100, 100)
    A[3] *= np.float32(1e-30)                              # tiny magnitudes
    return np.ascontiguousarray(A, np.float32)


@pytest.mark.parametrize("M,K", [(4, 8), (512, 3840), (37, 2056), (4096, 2048), (8, 16392)])
def test_quantize_rows_bit_exact(lib, orc, fd, M, K):
    say(f"quantize rows M={M} K={K}")
    A = quant_inputs(orc, max(M, 4), K, SEED + 800)[:M].copy()
    q, rs = np.empty((M, K), np.int8), np.empty(M, np.float32)
    assert lib.rocket_quantize_rows_int8(fd, M, K, R.ptr(A), R.ptr(q), R.ptr(rs)) == 0
    wq, wrs = orc.quant_rows(A)
    assert np.array_equal(q, wq) and np.array_equal(rs.view(np.uint32), wrs.view(np.uint32))
    # fp16 activations: the same as fp32 activations holding the fp16 values
    A16 = orc.f32_to_f16_bits(np.clip(A, -60000, 60000))
    assert lib.rocket_quantize_rows_int8_fp16(fd, M, K, R.ptr(A16), R.ptr(q), R.ptr(rs)) == 0
    wq, wrs = orc.quant_rows(orc.f16_bits_to_f32(A16))
    assert np.array_equal(q, wq) and np.array_equal(rs.view(np.uint32), wrs.view(np.uint32))


def test_quantize_rows_rejections(lib, fd):
    buf = np.zeros(64, np.float32)
    assert lib.rocket_quantize_rows_int8(fd, 4, 12, R.ptr(buf), R.ptr(buf), R.ptr(buf)) == R.ROCKET_E_SHAPE
    assert lib.rocket_quantize_rows_int8(fd, 0, 8, R.ptr(buf), R.ptr(buf), R.ptr(buf)) == R.ROCKET_E_SHAPE
    assert lib.rocket_quantize_rows_int8(fd, 4, 8, None, R.ptr(buf), R.ptr(buf)) == R.ROCKET_E_SHAPE
    assert lib.rocket_quantize_rows_int8(77, 4, 8, R.ptr(buf), R.ptr(buf), R.ptr(buf)) == R.ROCKET_E_DEVICE


@pytest.mark.parametrize("M,K,N,group", [(8, 256, 64, 64), (512, 3840, 15360, 128)])
def test_f32in_resident_matches_quantize_then_rowscale(lib, orc, fd, M, K, N, group):
    """The fp32-input entries quantise on the device and run the *_rowscale kernel: the same
    bits as the two calls in sequence, and (on sampled rows) as the oracle chain."""
    say(f"f32in resident M={M} K={K} N={N} g={group}")
    nG = K // group
    A = quant_inputs(orc, M, K, SEED + 810)
    bsc = orc.gen_uniform((N, nG), SEED + 811, 0.005, 0.02)
    q, rs = orc.quant_rows(A)
    rows = np.r_[0:4, M - 4:M]
    for int4 in (False, True):
        B = orc.gen_i8((N, K), SEED + 812, -8 if int4 else -128, 7 if int4 else 127)
        pre = "rocket_i4" if int4 else "rocket_i8"
        ctx = getattr(lib, pre + "_ctx_create")(1)
        w = getattr(lib, pre + "_weights_pack_gw")(ctx, M, K, N, R.ptr(B), group)
        assert w
        f32in = getattr(lib, f"rocket_matmul_{'int4' if int4 else 'int8'}_prepacked_gw_f32in")
        rowsc = getattr(lib, f"rocket_matmul_{'int4' if int4 else 'int8'}_prepacked_gw_rowscale")
        C1, C2 = np.full((M, N), np.nan, np.float32), np.full((M, N), np.nan, np.float32)
        assert f32in(ctx, M, K, N, R.ptr(A), R.ptr(bsc), R.ptr(C1), w) == 0
        assert rowsc(ctx, M, K, N, R.ptr(q), R.ptr(rs), R.ptr(bsc), R.ptr(C2), w) == 0
        assert np.array_equal(C1.view(np.uint32), C2.view(np.uint32))
        assert np.array_equal(C1[rows], orc.matmul_gw_rowscale_f32(np.ascontiguousarray(q[rows]), B,
                                                                   np.ascontiguousarray(rs[rows]), bsc, group))
        assert f32in(ctx, M, K, N, R.ptr(A), None, R.ptr(C1), w) == R.ROCKET_E_SHAPE
        getattr(lib, pre + "_weights_free")(ctx, w)
        getattr(lib, pre + "_ctx_free")(ctx)


def test_moe_grouped_f32in(lib, orc, fd):
    E, K, N, group = 8, 512, 192, 32
    nG = K // group
    ctx = lib.rocket_i8_ctx_create(1)
    Ws, bss, Bs = [], [], []
    for e in range(E):
        Bs.append(orc.gen_i8((N, K), SEED + 820 + e))
        Ws.append(lib.rocket_i8_weights_pack_gw(ctx, 4, K, N, R.ptr(Bs[-1]), group))
        bss.append(orc.gen_uniform((N, nG), SEED + 830 + e, 0.005, 0.02))
        assert Ws[-1]
    Ms = [16, 0, 4, 260, 8, 64, 132, 12]
    As = [quant_inputs(orc, max(m, 4), K, SEED + 840 + e) for e, m in enumerate(Ms)]
    Cs = [np.full((max(m, 4), N), -1.0, np.float32) for m in Ms]
    pM, k0 = R.int_array(Ms)
    pA, k1 = R.ptr_array(As)
    pbs, k3 = R.ptr_array(bss)
    pC, k4 = R.ptr_array(Cs)
    pW = (C.c_void_p * E)(*Ws)
    assert lib.rocket_matmul_int8_prepacked_gw_grouped_f32in(ctx, E, pM, K, N, pA, pbs, pC, C.cast(pW, R.pp)) == 0
    for e, m in enumerate(Ms):
        if m == 0:
            assert np.all(Cs[e] == -1.0)
            continue
        q, rs = orc.quant_rows(np.ascontiguousarray(As[e][:m]))
        assert np.array_equal(Cs[e][:m], orc.matmul_gw_rowscale_f32(q, Bs[e], rs, bss[e], group))
    for w in Ws:
        lib.rocket_i8_weights_free(ctx, w)
    lib.rocket_i8_ctx_free(ctx)


def act64(kind, g):
    """SiLU x / (1 + e^-x) and GELU 0.5 x (1 + erf(x / sqrt 2)) in float64 (the definitions the
    reference's FFN host code uses, rocket_ffn.c:33-38)."""
    from scipy.special import erf
    g = g.astype(np.float64)
    if kind == R.ROCKET_ACTIVATION_GELU:
        return 0.5 * g * (1.0 + erf(g / np.sqrt(2.0)))
    return g / (1.0 + np.exp(-g))


@pytest.mark.parametrize("kind", ["SILU", "GELU"])
def test_moe_grouped_glu_f32in(lib, orc, fd, kind):
    """The down products on act(gate) * up rows, formed and quantised in the pre-pass.
    (1) Gate values in [18, 30]: there 1 + e^-x and erfc(-x / sqrt 2) round to 1 and 2 in
    fp32, so both activations return x exactly and each row is the fp32 product gate * up:
    the result is bit-identical to the oracle's quantisation of that product followed by its
    row-scale fold. K = 1408 keeps each row in registers between its amax and its codes;
    K = 8224 (> 8192) takes the kernel's two-pass rows, which recompute the gated values.
    (2) N(0, 1) gates (the nonlinear range): within 2e-3 normalised error (max|d| / max|ref|)
    of the oracle on rows formed in float64 and rounded to fp32 — the device's expf / erfcf
    may differ from float64 by an ulp, which can move a code by one step. Both again through
    the fp16-input entry on the same values rounded to fp16 (widened exactly on the device)."""
    act = getattr(R, f"ROCKET_ACTIVATION_{kind}")
    E, N, group = 4, 192, 32
    ctx = lib.rocket_i8_ctx_create(1)
    for K, Ms in ((1408, [16, 0, 260, 8]), (8224, [4, 36, 0, 12])):
        nG = K // group
        Ws, bss, Bs = [], [], []
        for e in range(E):
            Bs.append(orc.gen_i8((N, K), SEED + 860 + e))
            Ws.append(lib.rocket_i8_weights_pack_gw(ctx, 4, K, N, R.ptr(Bs[-1]), group))
            bss.append(orc.gen_uniform((N, nG), SEED + 870 + e, 0.005, 0.02))
            assert Ws[-1]
        pM, k0 = R.int_array(Ms)
        pbs, k3 = R.ptr_array(bss)
        pW = (C.c_void_p * E)(*Ws)
        for exact, half in ((True, False), (False, False), (True, True), (False, True)):
            say(f"moe glu {'f16' if half else 'f32'}in {kind} K={K} exact={exact}")
            if exact:
                Gs = [orc.gen_uniform((max(m, 4), K), SEED + 880 + e, 18.0, 30.0) for e, m in enumerate(Ms)]
            else:
                Gs = [orc.gen_normal((max(m, 4), K), SEED + 880 + e) for e, m in enumerate(Ms)]
            Us = [orc.gen_normal((max(m, 4), K), SEED + 890 + e) for e, m in enumerate(Ms)]
            if half:   # fp16 rows; the references below take their exact fp32 values
                G16 = [orc.f32_to_f16_bits(g) for g in Gs]
                U16 = [orc.f32_to_f16_bits(u) for u in Us]
                Gs = [orc.f16_bits_to_f32(g) for g in G16]
                Us = [orc.f16_bits_to_f32(u) for u in U16]
            Cs = [np.full((max(m, 4), N), -1.0, np.float32) for m in Ms]
            pG, k1 = R.ptr_array(G16 if half else Gs)
            pU, k2 = R.ptr_array(U16 if half else Us)
            pC, k4 = R.ptr_array(Cs)
            entry = (lib.rocket_matmul_int8_prepacked_gw_grouped_glu_f16in if half
                     else lib.rocket_matmul_int8_prepacked_gw_grouped_glu_f32in)
            assert entry(ctx, E, pM, K, N, pG, pU, act, pbs, pC, C.cast(pW, R.pp)) == 0
            for e, m in enumerate(Ms):
                if m == 0:
                    assert np.all(Cs[e] == -1.0)
                    continue
                g, u = Gs[e][:m], Us[e][:m]
                if exact:
                    H = np.ascontiguousarray(g * u, np.float32)
                else:
                    H = np.ascontiguousarray((act64(act, g) * u.astype(np.float64)).astype(np.float32))
                q, rs = orc.quant_rows(H)
                ref = orc.matmul_gw_rowscale_f32(q, Bs[e], rs, bss[e], group)
                if exact:
                    assert np.array_equal(Cs[e][:m], ref)
                else:
                    assert orc.norm_err(Cs[e][:m], ref) <= 2e-3
        # rejected: another activation kind, a null up array
        assert lib.rocket_matmul_int8_prepacked_gw_grouped_glu_f32in(ctx, E, pM, K, N, pG, pU,
                                                                     R.ROCKET_ACTIVATION_TANH, pbs, pC,
                                                                     C.cast(pW, R.pp)) == R.ROCKET_E_SHAPE
        assert lib.rocket_matmul_int8_prepacked_gw_grouped_glu_f32in(ctx, E, pM, K, N, pG, None, act, pbs, pC,
                                                                     C.cast(pW, R.pp)) == R.ROCKET_E_SHAPE
        for w in Ws:
            lib.rocket_i8_weights_free(ctx, w)
    lib.rocket_i8_ctx_free(ctx)


# ---------------------------------------------------------------------------------------
# attention (rocket_attn.h)
# ---------------------------------------------------------------------------------------
def causal_mask(T, n_kv, window):
    """tests/flash_attn_rocket.c:43-53: key j visible to token t (at position n_kv - T + t)
    when j <= pos and, with a window, j > pos - window; -inf elsewhere."""
    pos = n_kv - T + np.arange(T)[:, None]
    j = np.arange(n_kv)[None, :]
    keep = (j <= pos) & ((window <= 0) | (j > pos - window))
    return np.where(keep, 0.0, -np.inf).astype(np.float16).view(np.uint16)


def attn_check(got, want):
    """The reference's bar (tests/flash_attn_rocket.c:89-96): cosine >= 0.9995 and
    max |got - ref| <= 0.02 max |ref| + 1e-3."""
    g = got.view(np.float16).astype(np.float64).ravel()
    r = want.view(np.float16).astype(np.float64).ravel()
    cos = g @ r / (np.sqrt(g @ g) * np.sqrt(r @ r) + 1e-30)
    err = np.abs(g - r).max()
    assert cos >= 0.9995 and err <= 0.02 * np.abs(r).max() + 1e-3, (cos, err)
    return cos, err


# the reference's shapes (tests/flash_attn_rocket.c:172-246): Gemma-12B local / global layers,
# MLA (dk 192, dv 128), unaligned T / n_kv, cached prefixes, long context, soft-cap
FA_CASES = [(128, 128, 256, 256, 16, 8, 0, 0.0), (128, 128, 256, 256, 16, 8, 64, 0.0),
            (128, 128, 256, 256, 16, 1, 0, 0.0), (100, 100, 256, 256, 16, 8, 0, 0.0),
            (64, 512, 256, 256, 16, 8, 0, 0.0), (128, 128, 256, 256, 16, 8, 0, 50.0),
            (128, 128, 192, 128, 16, 1, 0, 0.0), (100, 100, 192, 128, 16, 1, 0, 0.0),
            (128, 128, 192, 128, 16, 1, 64, 0.0), (64, 512, 192, 128, 16, 1, 0, 0.0),
            (64, 8192, 256, 256, 16, 8, 0, 0.0), (512, 2048, 256, 256, 16, 8, 640, 0.0),
            (96, 600, 256, 256, 16, 8, 0, 0.0), (300, 257, 64, 64, 4, 2, 0, 0.0), (33, 70, 128, 48, 6, 3, 0, 0.0)]


@pytest.mark.parametrize("T,n_kv,dh,dv,nh,nkvh,window,softcap", FA_CASES)
def test_flash_attn(lib, orc, fd, T, n_kv, dh, dv, nh, nkvh, window, softcap):
    say(f"flash attn T={T} n_kv={n_kv} dh={dh} dv={dv} nh={nh} nkvh={nkvh} win={window} cap={softcap}")
    scale = np.float32(1.0) / np.sqrt(np.float32(dh))
    Q = lcg_fill((nh, T, dh), 1.0, T * 7 + dh)
    K = lcg_fill((nkvh, n_kv, dh), 1.0, n_kv * 3 + 1)
    V = lcg_fill((nkvh, dv, n_kv), 1.0, n_kv * 5 + 2)
    M = causal_mask(T, n_kv, window)
    want = orc.flash_attn_f16(Q, K, V, M, scale, softcap)
    out = np.full((nh, T, dv), 0x7FFF, np.uint16)
    assert lib.rocket_flash_attn_fp16(fd, T, n_kv, dh, dv, nh, nkvh, scale, softcap, R.ptr(Q), R.ptr(K), R.ptr(V),
                                      R.ptr(M), R.ptr(out)) == 0
    assert not np.any(out == 0x7FFF)
    cos, err = attn_check(out, want)
    say(f"  cos={cos:.7f} max_abs={err:.3g}")
    # the multi-worker and persistent-context entries are the same computation
    out2 = np.empty_like(out)
    assert lib.rocket_flash_attn_fp16_mt(fd, T, n_kv, dh, dv, nh, nkvh, scale, softcap, R.ptr(Q), R.ptr(K), R.ptr(V),
                                         R.ptr(M), R.ptr(out2), 5) == 0
    assert np.array_equal(out2, out)
    ctx = lib.rocket_fa_ctx_create(5)
    assert ctx
    assert lib.rocket_flash_attn_fp16_ctx(ctx, T, n_kv, dh, dv, nh, nkvh, scale, softcap, R.ptr(Q), R.ptr(K),
                                          R.ptr(V), R.ptr(M), R.ptr(out2)) == 0
    lib.rocket_fa_ctx_free(ctx)
    assert np.array_equal(out2, out)


def test_flash_attn_mask_load_paths_agree(lib, orc, fd):
    """The three ways a mask reaches the kernel give the same bits: rows of a multiple of 8
    halves go to LDS by DMA (n_kv = 128), rows of a multiple of 4 by 8-byte loads (n_kv = 132)
    and others by 2-byte loads (n_kv = 130). The extra keys are masked (-inf), so with one key
    split they add exact zeros and every call equals the 128-key one; that one also meets the
    reference's bar against the oracle."""
    T, dh, dv, nh, nkvh = 128, 256, 256, 4, 2
    scale = np.float32(1.0) / np.sqrt(np.float32(dh))
    Q = lcg_fill((nh, T, dh), 1.0, 901)
    K = lcg_fill((nkvh, 132, dh), 1.0, 902)
    V = lcg_fill((nkvh, dv, 132), 1.0, 903)
    M = causal_mask(T, 132, 0)
    outs = {}
    for n_kv in (128, 132, 130):
        say(f"flash attn mask path n_kv={n_kv}")
        Kn = np.ascontiguousarray(K[:, :n_kv])
        Vn = np.ascontiguousarray(V[:, :, :n_kv])
        Mn = np.ascontiguousarray(M[:, :n_kv])
        Mn[:, 128:] = np.float16(-np.inf).view(np.uint16)
        Mn[:, :128] = causal_mask(T, 128, 0)
        out = np.full((nh, T, dv), 0x7FFF, np.uint16)
        assert lib.rocket_flash_attn_fp16(fd, T, n_kv, dh, dv, nh, nkvh, scale, 0.0, R.ptr(Q), R.ptr(Kn), R.ptr(Vn),
                                          R.ptr(Mn), R.ptr(out)) == 0
        outs[n_kv] = out
    assert not np.any(outs[128] == 0x7FFF)
    attn_check(outs[128], orc.flash_attn_f16(Q, np.ascontiguousarray(K[:, :128]), np.ascontiguousarray(V[:, :, :128]),
                                             causal_mask(T, 128, 0), scale, 0.0))
    assert np.array_equal(outs[132], outs[128])
    assert np.array_equal(outs[130], outs[128])


def test_flash_attn_unmasked_and_device_operands(lib, orc, fd):
    import torch
    T, n_kv, dh, dv, nh, nkvh = 200, 320, 128, 128, 8, 2
    Q = lcg_fill((nh, T, dh), 1.0, 11)
    K = lcg_fill((nkvh, n_kv, dh), 1.0, 12)
    V = lcg_fill((nkvh, dv, n_kv), 1.0, 13)
    want = orc.flash_attn_f16(Q, K, V, None, 0.09, 0.0)
    out = np.empty((nh, T, dv), np.uint16)
    assert lib.rocket_flash_attn_fp16(fd, T, n_kv, dh, dv, nh, nkvh, 0.09, 0.0, R.ptr(Q), R.ptr(K), R.ptr(V), None,
                                      R.ptr(out)) == 0
    attn_check(out, want)
    dQ, dK, dV = (torch.from_numpy(a.view(np.int16)).cuda() for a in (Q, K, V))
    dO = torch.empty((nh, T, dv), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()
    assert lib.rocket_flash_attn_fp16(fd, T, n_kv, dh, dv, nh, nkvh, 0.09, 0.0, R.ptr(dQ), R.ptr(dK), R.ptr(dV), None,
                                      R.ptr(dO)) == 0
    assert np.array_equal(dO.cpu().numpy().view(np.uint16), out)


@pytest.mark.parametrize("dh,dv,masked", [(256, 256, True), (256, 256, False), (128, 128, True)])
def test_flash_attn_running_max_growth(lib, orc, fd, dh, dv, masked):
    """Scores that grow along the key axis for some queries and shrink for others: each key
    row carries a component along the all-ones direction that rises with its position, and
    each query a mean of random sign and size. A rising query's running max passes its old
    value by more than the rescale threshold (8 natural units) in later key tiles of the
    same key split (this shape runs 8 splits of 4 tiles), in some waves of a workgroup and
    not in others; the scores reach ~270."""
    say(f"flash attn running-max growth dh={dh} dv={dv} masked={masked}")
    T, n_kv, nh, nkvh = 256, 2048, 4, 2
    rng = np.random.default_rng(SEED + 40)
    Q = rng.uniform(-1, 1, (nh, T, dh)) + rng.uniform(-1, 1, (nh, T, 1))
    K = 0.25 * rng.uniform(-1, 1, (nkvh, n_kv, dh)) + (16.0 * np.arange(n_kv) / n_kv)[None, :, None]
    V = rng.uniform(-1, 1, (nkvh, dv, n_kv))
    Q, K, V = (x.astype(np.float16).view(np.uint16) for x in (Q, K, V))
    M = causal_mask(T, n_kv, 0) if masked else None
    scale = float(np.float32(1.0) / np.sqrt(np.float32(dh)))
    # the growth is what the case is for: in some 256-key window, a later 64-key tile's max
    # passes the window's first tile's max by more than 8 natural units
    qf = Q.view(np.float16).astype(np.float32)[0]
    kf = K.view(np.float16).astype(np.float32)[0]
    tmax = (qf @ kf.T * scale).reshape(T, n_kv // 256, 4, 64).max(-1)
    assert (tmax[:, :, 1:].max(-1) - tmax[:, :, 0]).max() > 8
    want = orc.flash_attn_f16(Q, K, V, M, scale, 0.0)
    out = np.full((nh, T, dv), 0x7FFF, np.uint16)
    assert lib.rocket_flash_attn_fp16(fd, T, n_kv, dh, dv, nh, nkvh, scale, 0.0, R.ptr(Q), R.ptr(K), R.ptr(V),
                                      R.ptr(M) if masked else None, R.ptr(out)) == 0
    assert not np.any(out == 0x7FFF)
    cos, err = attn_check(out, want)
    say(f"  cos={cos:.7f} max_abs={err:.3g}")


@pytest.mark.parametrize("T,d,nh", [(64, 512, 8), (128, 512, 8), (100, 512, 8), (64, 384, 6), (300, 1024, 16)])
def test_mha_self(lib, orc, fd, T, d, nh):
    """tests/mha_rocket.c:37-88: Whisper-style encoder attention (bq, bv, bo; no bk); the
    reference's bar: cosine >= 0.9999 and max |got - ref| <= 0.02 max |ref| + 1e-3."""
    say(f"mha T={T} d={d} nh={nh}")
    x = lcg_fill((T, d), 1.0, T * 7 + d)
    Wq, Wk, Wv, Wo = (lcg_fill((d, d), 0.05, s) for s in (1, 2, 3, 4))
    bq, bv, bo = (lcg_fill(d, 0.1, s) for s in (5, 6, 7))
    want = orc.mha_self_f16(x, Wq, bq, Wk, None, Wv, bv, Wo, bo, nh)
    out = np.full((T, d), 0x7FFF, np.uint16)
    assert lib.rocket_mha_self_fp16(fd, T, d, nh, R.ptr(x), R.ptr(Wq), R.ptr(bq), R.ptr(Wk), None, R.ptr(Wv),
                                    R.ptr(bv), R.ptr(Wo), R.ptr(bo), R.ptr(out)) == 0
    g = out.view(np.float16).astype(np.float64).ravel()
    r = want.view(np.float16).astype(np.float64).ravel()
    cos = g @ r / (np.sqrt(g @ g) * np.sqrt(r @ r) + 1e-30)
    err = np.abs(g - r).max()
    say(f"  cos={cos:.7f} max_abs={err:.3g}")
    assert cos >= 0.9999 and err <= 0.02 * np.abs(r).max() + 1e-3


# ---------------------------------------------------------------------------------------
# serialised resident weights (rocket_weights_io.h)
# ---------------------------------------------------------------------------------------
def weights_fixtures():
    import importlib.util
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "make_weights_fixture.py")
    spec = importlib.util.spec_from_file_location("make_weights_fixture", path)
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m, os.path.dirname(path)


def test_weights_load_committed_fixtures(lib, orc, fd):
    """The committed files (written from the format's definition, not by the library) load
    into working resident weights: products equal the oracle's on the fixture's values."""
    import os
    fx, here = weights_fixtures()
    B4, sc4, _ = fx.int4_fixture()
    ctx4 = lib.rocket_i4_ctx_create(1)
    scales = np.zeros_like(sc4)
    w4 = lib.rocket_i4_weights_load(ctx4, os.path.join(here, "weights_int4_g32.rktw").encode(), R.ptr(scales))
    assert w4 and np.array_equal(scales, sc4)
    M, N, K, group = 8, 64, 128, 32
    A = orc.gen_i8((M, K), SEED + 900)
    asc = orc.gen_uniform((M, K // group), SEED + 901, 0.5, 1.5)
    Cf = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_int4_prepacked_gw(ctx4, M, K, N, R.ptr(A), R.ptr(asc), R.ptr(sc4), R.ptr(Cf), w4) == 0
    assert np.array_equal(Cf, orc.matmul_gw_f32(A, B4, asc, sc4, group))
    lib.rocket_i4_weights_free(ctx4, w4)
    B8, _ = fx.int8_fixture()
    ctx8 = lib.rocket_i8_ctx_create(1)
    w8 = lib.rocket_i8_weights_load(ctx8, os.path.join(here, "weights_int8_pc.rktw").encode(), None)
    assert w8
    Ci = np.empty((8, 32), np.int32)
    A8 = orc.gen_i8((8, 64), SEED + 902)
    assert lib.rocket_matmul_int8_prepacked(ctx8, 8, 64, 32, R.ptr(A8), R.ptr(Ci), w8) == 0
    assert np.array_equal(Ci, orc.matmul_int8(A8, B8))
    # a file of the other kind is refused
    assert not lib.rocket_i8_weights_load(ctx8, os.path.join(here, "weights_int4_g32.rktw").encode(), None)
    lib.rocket_i8_weights_free(ctx8, w8)
    lib.rocket_i8_ctx_free(ctx8)
    lib.rocket_i4_ctx_free(ctx4)


@pytest.mark.parametrize("int4,group", [(False, 0), (False, 64), (True, 0), (True, 128)])
def test_weights_round_trip(lib, orc, fd, tmp_path, int4, group):
    """pack -> serialise -> deserialise (buffer and file) gives a weight whose products are
    bit-identical to the original's; the int4 codes on disk are the documented layout."""
    fx, _ = weights_fixtures()
    M, K, N = 16, 512, 192
    say(f"weights round trip int4={int4} group={group}")
    pre = "rocket_i4" if int4 else "rocket_i8"
    B = orc.gen_i8((N, K), SEED + 910, -8 if int4 else -128, 7 if int4 else 127)
    ctx = getattr(lib, pre + "_ctx_create")(1)
    w = (getattr(lib, pre + "_weights_pack_gw")(ctx, M, K, N, R.ptr(B), group) if group
         else getattr(lib, pre + "_weights_pack")(ctx, M, K, N, R.ptr(B)))
    assert w
    bsc = orc.gen_uniform((N, K // group), SEED + 911, 0.005, 0.02) if group else None
    nbytes = getattr(lib, pre + "_weights_serialized_bytes")(w, 1)
    buf = np.zeros(nbytes, np.uint8)
    assert getattr(lib, pre + "_weights_serialize")(ctx, w, R.ptr(bsc) if group else None, R.ptr(buf),
                                                    nbytes - 1) == R.ROCKET_E_SHAPE
    n = getattr(lib, pre + "_weights_serialize")(ctx, w, R.ptr(bsc) if group else None, R.ptr(buf), nbytes)
    assert n == nbytes
    codes = buf[64:64 + (N * K // 2 if int4 else N * K)].tobytes()
    assert codes == (fx.pack_int4(B) if int4 else B.tobytes())
    assert buf.tobytes() == fx.serialise(2 if int4 else 1, N, K, group, M, codes, bsc)
    sc_out = np.zeros_like(bsc) if group else None
    w2 = getattr(lib, pre + "_weights_deserialize")(ctx, R.ptr(buf), nbytes, R.ptr(sc_out) if group else None)
    assert w2
    if group:
        assert np.array_equal(sc_out, bsc)
    path = str(tmp_path / "w.rktw").encode()
    assert getattr(lib, pre + "_weights_save")(ctx, w, R.ptr(bsc) if group else None, path) == 0
    w3 = getattr(lib, pre + "_weights_load")(ctx, path, None)
    assert w3
    A = orc.gen_i8((M, K), SEED + 912)
    kind = "int4" if int4 else "int8"
    outs = []
    for ww in (w, w2, w3):
        if group:
            asc = orc.gen_uniform((M, K // group), SEED + 913, 0.5, 1.5)
            Cf = np.empty((M, N), np.float32)
            assert getattr(lib, f"rocket_matmul_{kind}_prepacked_gw")(ctx, M, K, N, R.ptr(A), R.ptr(asc), R.ptr(bsc),
                                                                     R.ptr(Cf), ww) == 0
            outs.append(Cf)
        else:
            Ci = np.empty((M, N), np.int32)
            assert getattr(lib, f"rocket_matmul_{kind}_prepacked")(ctx, M, K, N, R.ptr(A), R.ptr(Ci), ww) == 0
            outs.append(Ci)
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    if not group:
        assert np.array_equal(outs[0], orc.matmul_int8(A, B))
    else:
        assert np.array_equal(outs[0], orc.matmul_gw_f32(A, B, asc, bsc, group))
    # a corrupted file is refused
    raw = bytearray(open(path, "rb").read())
    raw[100] ^= 0x10
    open(path, "wb").write(bytes(raw))
    assert not getattr(lib, pre + "_weights_load")(ctx, path, None)
    for ww in (w, w2, w3):
        getattr(lib, pre + "_weights_free")(ctx, ww)
    getattr(lib, pre + "_ctx_free")(ctx)


# ---------------------------------------------------------------------------------------
# device operands (torch tensors in HBM) take the same kernels, in place
# ---------------------------------------------------------------------------------------
def test_device_pointers_in_place(lib, orc, fd):
    import torch
    M, K, N = 256, 1024, 512
    A = orc.gen_i8((M, K), SEED + 600)
    B = orc.gen_i8((N, K), SEED + 601)
    dA = torch.from_numpy(A).cuda()
    dB = torch.from_numpy(B).cuda()
    dC = torch.empty((M, N), dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    assert lib.rocket_matmul_int8(fd, M, K, N, R.ptr(dA), R.ptr(dB), R.ptr(dC)) == 0
    assert np.array_equal(dC.cpu().numpy(), orc.matmul_int8(A, B))
    # async on a caller stream: returns once queued; the stream orders the rest
    s = torch.cuda.Stream()
    assert lib.rocket_hip_set_stream(fd, C.c_void_p(s.cuda_stream)) == 0
    assert lib.rocket_hip_set_mode(fd, R.ROCKET_HIP_ASYNC) == 0
    dC.zero_()
    torch.cuda.synchronize()
    assert lib.rocket_matmul_int8(fd, M, K, N, R.ptr(dA), R.ptr(dB), R.ptr(dC)) == 0
    s.synchronize()
    assert lib.rocket_hip_set_mode(fd, 0) == 0
    assert lib.rocket_hip_set_stream(fd, None) == 0
    assert np.array_equal(dC.cpu().numpy(), orc.matmul_int8(A, B))


def test_counters_count_launches(lib, orc, fd):
    lib.rocket_submit_counters_reset()
    A = orc.gen_i8((4, 64), 1)
    B = orc.gen_i8((32, 64), 2)
    Cg = np.empty((4, 32), np.int32)
    assert lib.rocket_matmul_int8(fd, 4, 64, 32, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
    assert lib.rocket_submit_ioctl_count() == 1 and lib.rocket_submit_task_count() >= 1


# ---------------------------------------------------------------------------------------
# feed-forward blocks (rocket_ffn.h): the gated core, the gated FFN and the MLP
# ---------------------------------------------------------------------------------------
def lcg_fill(shape, amp, seed):
    """The reference tests' input generator (tests/ffn_rocket.c:24-32): a 32-bit LCG whose
    bits 8..23 scale to (u * 2 - 1) * amp in fp32, rounded to fp16. Evaluated in closed form
    (state_n = a^n s0 + c (a^(n-1) + ... + 1) mod 2^32) so large operands are quick."""
    n = int(np.prod(shape))
    a, c = np.uint64(1664525), np.uint64(1013904223)
    s0 = np.uint64((0x9E3779B9 ^ seed) & 0xFFFFFFFF)
    with np.errstate(over="ignore"):
        pw = np.cumprod(np.full(n, a, np.uint64))                       # a^1 .. a^n (mod 2^64)
        geo = np.cumsum(np.concatenate([[np.uint64(1)], pw[:-1]]))      # a^0 + .. + a^(n-1)
        st = (pw * s0 + c * geo) & np.uint64(0xFFFFFFFF)
    u = ((st >> np.uint64(8)) & np.uint64(0xFFFF)).astype(np.float32) / np.float32(65535.0)
    v = (u * np.float32(2.0) - np.float32(1.0)) * np.float32(amp)
    return v.astype(np.float16).view(np.uint16).reshape(shape)


def cosine(got16, ref):
    g = got16.view(np.float16).astype(np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    ng, nr = g @ g, r @ r
    return 1.0 if ng == 0 and nr == 0 else float(g @ r / np.sqrt(ng * nr))


def ulp16(a, b):
    def ordered(h):
        h = h.astype(np.int32)
        return np.where(h & 0x8000, -(h & 0x7FFF), h)
    return np.abs(ordered(a) - ordered(b))


def test_lcg_fill_matches_the_recurrence():
    st, want = 0x9E3779B9 ^ 7, []
    for _ in range(300):
        st = (st * 1664525 + 1013904223) & 0xFFFFFFFF
        want.append(np.float16((np.float32((st >> 8) & 0xFFFF) / np.float32(65535) * np.float32(2)
                                - np.float32(1)) * np.float32(2.5)))
    assert np.array_equal(lcg_fill(300, 2.5, 7), np.array(want, np.float16).view(np.uint16))


@pytest.mark.parametrize("n", [4096, 65536, 100000, 100003])
@pytest.mark.parametrize("kind", [R.ROCKET_ACTIVATION_SILU, R.ROCKET_ACTIVATION_GELU])
def test_geglu(lib, orc, fd, n, kind):
    say(f"geglu n={n} kind={kind}")
    gate = lcg_fill(n + 1, 6.0, 11 + kind)        # logits in [-6, 6] (tests/ffn_rocket.c:71-72)
    up = lcg_fill(n + 1, 2.5, 99 + kind)
    want = orc.geglu_f16(gate[:n], up[:n], kind)
    got = np.empty(n + 1, np.uint16)
    assert lib.rocket_geglu_fp16(fd, R.ptr(gate), R.ptr(up), kind, R.ptr(got), n) == 0
    # fp32 arithmetic, one rounding: within one fp16 step of the double-rounded oracle
    assert ulp16(got[:n], want).max() <= 1 and np.mean(got[:n] == want) > 0.99
    assert cosine(got[:n], want.view(np.float16)) >= 0.999
    # operands two bytes off 16-byte alignment take the per-element path: same bits
    g1 = np.empty(n, np.uint16)
    assert lib.rocket_geglu_fp16(fd, R.ptr(gate[1:]), R.ptr(up[1:]), kind, R.ptr(g1), n) == 0
    want1 = orc.geglu_f16(gate[1:], up[1:], kind)
    assert ulp16(g1, want1).max() <= 1


def ffn_operands(M, H, I, kind, scaled):
    if scaled:   # tests/ffn_fused_rocket.c:118-123: amplitudes by 1/sqrt(H), 1/sqrt(I)
        a = np.float32(3.0) / np.sqrt(np.float32(H))
        return (lcg_fill((M, H), 1.0, 1 + kind), lcg_fill((I, H), a, 2 + kind),
                lcg_fill((I, H), a, 3 + kind), lcg_fill((H, I), np.float32(1.5) / np.sqrt(np.float32(I)), 4 + kind))
    # tests/ffn_rocket.c:90-92
    return (lcg_fill((M, H), 0.35, 1), lcg_fill((I, H), 0.35, 2), lcg_fill((I, H), 0.35, 3),
            lcg_fill((H, I), 0.35, 4))


def ffn_run(lib, fd, f, M, H, I, x, Wg, Wu, Wd, kind):
    out = np.full((M, H), 0x7FFF, np.uint16)      # NaN sentinel: no finite result equals it
    assert f(fd, M, H, I, R.ptr(x), R.ptr(Wg), R.ptr(Wu), R.ptr(Wd), kind, R.ptr(out)) == 0
    assert not np.any(out == 0x7FFF)
    return out


S_, G_ = R.ROCKET_ACTIVATION_SILU, R.ROCKET_ACTIVATION_GELU


# the reference's rocket_ffn_fp16 shapes (tests/ffn_rocket.c:117-120) plus partial tiles
@pytest.mark.parametrize("M,H,I,kind", [(16, 128, 256, S_), (64, 512, 512, S_), (128, 1024, 1024, S_),
                                        (128, 2048, 1024, S_), (128, 1024, 1024, G_), (1, 96, 160, G_),
                                        (12, 160, 96, S_), (300, 544, 1056, G_), (1024, 256, 8160, G_)])
def test_ffn(lib, orc, fd, M, H, I, kind):
    say(f"ffn M={M} H={H} I={I} kind={kind}")
    x, Wg, Wu, Wd = ffn_operands(M, H, I, kind, scaled=False)
    want = orc.ffn_f16(x, Wg, Wu, Wd, kind)
    got = ffn_run(lib, fd, lib.rocket_ffn_fp16, M, H, I, x, Wg, Wu, Wd, kind)
    assert cosine(got, want.view(np.float16)) >= 0.998           # tests/ffn_rocket.c:98
    assert orc.norm_err(orc.f16_bits_to_f32(got), orc.f16_bits_to_f32(want)) <= 1e-2
    fused = ffn_run(lib, fd, lib.rocket_ffn_fp16_fused, M, H, I, x, Wg, Wu, Wd, kind)
    assert np.array_equal(fused, got)                            # one computation on this device


# the reference's rocket_ffn_fp16_fused shapes (tests/ffn_fused_rocket.c:166-170)
# (2048, 512, 8192) and (2048, 512, 8160): the gate+up product on 256x256 tiles, the second
# with a partial last tile of gate / up column pairs
@pytest.mark.parametrize("M,H,I,kind", [(128, 256, 512, S_), (512, 2048, 1024, S_), (256, 768, 3072, G_),
                                        (1024, 768, 3072, S_), (2048, 512, 8192, S_), (2048, 512, 8160, G_)])
def test_ffn_fused(lib, orc, fd, M, H, I, kind):
    say(f"ffn_fused M={M} H={H} I={I} kind={kind}")
    x, Wg, Wu, Wd = ffn_operands(M, H, I, kind, scaled=True)
    want = orc.ffn_f16(x, Wg, Wu, Wd, kind)
    fused = ffn_run(lib, fd, lib.rocket_ffn_fp16_fused, M, H, I, x, Wg, Wu, Wd, kind)
    host = ffn_run(lib, fd, lib.rocket_ffn_fp16, M, H, I, x, Wg, Wu, Wd, kind)
    assert cosine(fused, want.view(np.float16)) >= 0.999         # tests/ffn_fused_rocket.c:151
    assert cosine(fused, host.view(np.float16)) >= 0.9995
    assert orc.norm_err(orc.f16_bits_to_f32(fused), orc.f16_bits_to_f32(want)) <= 1e-2


@pytest.mark.parametrize("M,Din,Dff,Dout,kind,bias", [(256, 768, 3072, 768, G_, True), (4, 64, 96, 48, S_, False),
                                                      (1, 256, 512, 128, S_, True), (100, 320, 160, 80, G_, False),
                                                      (2048, 256, 4096, 256, S_, True)])
def test_mlp(lib, orc, fd, M, Din, Dff, Dout, kind, bias):
    say(f"mlp M={M} Din={Din} Dff={Dff} Dout={Dout} kind={kind} bias={bias}")
    x = lcg_fill((M, Din), 1.0, 5)
    W1 = lcg_fill((Dff, Din), np.float32(3.0) / np.sqrt(np.float32(Din)), 6)
    b1 = lcg_fill(Dff, 1.0, 7) if bias else None
    W2 = lcg_fill((Dout, Dff), np.float32(1.5) / np.sqrt(np.float32(Dff)), 8)
    want = orc.mlp_f16(x, W1, b1, W2, kind)
    out = np.full((M, Dout), 0x7FFF, np.uint16)
    assert lib.rocket_mlp_fp16_fused(fd, M, Din, Dff, Dout, R.ptr(x), R.ptr(W1),
                                     R.ptr(b1) if bias else None, R.ptr(W2), kind, R.ptr(out)) == 0
    assert not np.any(out == 0x7FFF)
    assert cosine(out, want.view(np.float16)) >= 0.999
    assert orc.norm_err(orc.f16_bits_to_f32(out), orc.f16_bits_to_f32(want)) <= 1e-2


@pytest.mark.parametrize("M,H,I", [(512, 3072, 8192), (512, 3840, 15360)])
def test_ffn_split_k_down_product(lib, orc, fd, M, H, I):
    """At M = 512 the down product has too few 256x128 tiles and runs as K slices; at the
    Gemma-12B shape (H = 3840, I = 15360) the gate+up product runs on 256x256 tiles with the
    gated epilogue. Checked against a float64 numpy evaluation of the block (the oracle's
    formula, pinned against it in the oracle tests; the oracle itself is too slow at this
    size)."""
    from scipy.special import ndtr
    say(f"ffn split-K down M={M} H={H} I={I}")
    x, Wg, Wu, Wd = ffn_operands(M, H, I, G_, scaled=True)
    X, G, U, D = (orc.f16_bits_to_f32(t).astype(np.float64) for t in (x, Wg, Wu, Wd))
    g, u = X @ G.T, X @ U.T
    want = (g * ndtr(g) * u) @ D.T
    got = ffn_run(lib, fd, lib.rocket_ffn_fp16_fused, M, H, I, x, Wg, Wu, Wd, G_)
    assert cosine(got, want) >= 0.999
    assert orc.norm_err(orc.f16_bits_to_f32(got), want) <= 1e-2
    again = ffn_run(lib, fd, lib.rocket_ffn_fp16, M, H, I, x, Wg, Wu, Wd, G_)
    assert np.array_equal(again, got)


def test_ffn_device_operands_and_rejections(lib, orc, fd):
    import torch
    M, H, I = 64, 256, 512
    x, Wg, Wu, Wd = ffn_operands(M, H, I, S_, scaled=True)
    host = ffn_run(lib, fd, lib.rocket_ffn_fp16, M, H, I, x, Wg, Wu, Wd, S_)
    dev = [torch.from_numpy(t.view(np.int16)).cuda() for t in (x, Wg, Wu, Wd)]
    dout = torch.empty((M, H), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()
    assert lib.rocket_ffn_fp16(fd, M, H, I, *[R.ptr(t) for t in dev], S_, R.ptr(dout)) == 0
    assert np.array_equal(dout.cpu().numpy().view(np.uint16), host)
    # GPU-path limits are shape errors on an open handle as on a closed one
    p = R.ptr(x)
    assert lib.rocket_ffn_fp16(fd, M, H, I, p, p, p, p, 1, p) == R.ROCKET_E_SHAPE
    assert lib.rocket_ffn_fp16(fd, M, 48, I, p, p, p, p, S_, p) == R.ROCKET_E_SHAPE
    assert lib.rocket_ffn_fp16(fd, 6, H, I, p, p, p, p, S_, p) == R.ROCKET_E_SHAPE
