"""Committed fixtures (tests/golden/golden.npz, written by numpy alone in make_golden.py):
the CPU oracle must reproduce them, and so must librocketnpu on the GPU through its C-ABI.
"""
import os

import numpy as np
import pytest

import rocketnpu as R

G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz"))


# ---- oracle (CPU) ----------------------------------------------------------------------

def test_oracle_integer_fixtures(orc):
    for tag in ("int8_a", "int8_m1"):
        assert np.array_equal(orc.matmul_int8(G[f"{tag}_A"], G[f"{tag}_B"]), G[f"{tag}_C"])
    assert np.array_equal(orc.matmul_int16_exact(G["int16_A"], G["int16_B"]), G["int16_C"])
    for tag in ("gw8", "gw4"):
        grp = int(G[f"{tag}_group"])
        assert np.array_equal(orc.gw_partials(G[f"{tag}_A"], G[f"{tag}_B"], grp), G[f"{tag}_P"])
        f64 = orc.matmul_gw_f64(G[f"{tag}_A"], G[f"{tag}_B"], G[f"{tag}_as"], G[f"{tag}_bs"], grp)
        assert np.allclose(f64, G[f"{tag}_ref64"], rtol=1e-12, atol=1e-12)
        f32 = orc.matmul_gw_f32(G[f"{tag}_A"], G[f"{tag}_B"], G[f"{tag}_as"], G[f"{tag}_bs"], grp)
        assert orc.rms_err(f32, G[f"{tag}_ref64"]) <= 1e-5


def test_oracle_float_fixtures(orc):
    c16 = orc.f16_bits_to_f32(orc.matmul_fp16(G["fp16_A"], G["fp16_B"]))
    ref = G["fp16_ref64"]
    # one fp32 sum rounded once to fp16: within an fp16 half-ulp of the exact product plus the
    # fp32 accumulation error
    assert np.all(np.abs(c16 - ref) <= np.abs(ref) * 2 ** -11 + 1e-3)
    assert np.allclose(orc.matmul_bf16(G["flt_A"], G["flt_B"]), G["bf16_ref64"], rtol=1e-6, atol=1e-7)
    assert np.allclose(orc.matmul_tf32(G["flt_A"], G["flt_B"]), G["tf32_ref64"], rtol=1e-6, atol=1e-7)
    assert np.allclose(orc.matmul_f32(G["flt_A"], G["flt_B"]), G["f32_ref64"], rtol=1e-6, atol=1e-7)


# ---- librocketnpu (GPU) ----------------------------------------------------------------

@pytest.mark.gpu
def test_gpu_integer_fixtures(lib, fd):
    for tag in ("int8_a", "int8_m1"):
        A, B = G[f"{tag}_A"], G[f"{tag}_B"]
        M, K = A.shape
        N = B.shape[0]
        C = np.empty((M, N), np.int32)
        assert lib.rocket_matmul_int8(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(C)) == 0
        assert np.array_equal(C, G[f"{tag}_C"])
    A, B = G["int16_A"], G["int16_B"]
    C = np.empty((A.shape[0], B.shape[0]), np.int64)
    assert lib.rocket_matmul_int16_exact(fd, A.shape[0], A.shape[1], B.shape[0], R.ptr(A), R.ptr(B), R.ptr(C)) == 0
    assert np.array_equal(C, G["int16_C"])


@pytest.mark.gpu
@pytest.mark.parametrize("tag,entry", [("gw8", "rocket_matmul_int8_groupwise_dump"),
                                       ("gw4", "rocket_matmul_int4_groupwise_dump")])
def test_gpu_groupwise_fixtures(lib, orc, fd, tag, entry):
    A, B, asc, bsc = G[f"{tag}_A"], G[f"{tag}_B"], G[f"{tag}_as"], G[f"{tag}_bs"]
    grp = int(G[f"{tag}_group"])
    M, K = A.shape
    N = B.shape[0]
    Cf = np.empty((M, N), np.float32)
    P = np.empty((M, K // grp, N), np.int32)
    assert getattr(lib, entry)(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(asc), R.ptr(bsc), R.ptr(Cf), grp,
                               0, M, R.ptr(P)) == 0
    assert np.array_equal(P, G[f"{tag}_P"])
    assert orc.rms_err(Cf, G[f"{tag}_ref64"]) <= 1e-5


@pytest.mark.gpu
def test_gpu_float_fixtures(lib, orc, fd):
    A16, B16 = G["fp16_A"], G["fp16_B"]
    M, K = A16.shape
    N = B16.shape[0]
    C16 = np.empty((M, N), np.uint16)
    assert lib.rocket_matmul_fp16(fd, M, K, N, R.ptr(A16), R.ptr(B16), R.ptr(C16)) == 0
    assert orc.norm_err(orc.f16_bits_to_f32(C16), G["fp16_ref64"]) <= 1e-2
    A, B = G["flt_A"], G["flt_B"]
    M, K = A.shape
    N = B.shape[0]
    # bf16: exact products of the truncated operands, fp32 accumulation. tf32 runs as three
    # bf16 products of an exact hi/lo split (hi*hi + lo*hi + hi*lo); the dropped lo*lo term is
    # below 2^-16 of each product, so its bound here is 5e-5 (the configuration gate is 5e-3).
    for entry, key, tol in (("rocket_matmul_bf16", "bf16_ref64", 1e-5), ("rocket_matmul_tf32", "tf32_ref64", 5e-5)):
        C = np.empty((M, N), np.float32)
        assert getattr(lib, entry)(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(C)) == 0
        assert orc.norm_err(C, G[key]) <= tol
