"""numpy front-end of the C oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker and as the timed CPU baseline. The shipped library never
imports it. Every function mirrors one in oracle.h, which names the reference file:line
it restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "-B"], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, i32, u64, sz, fl = C.c_void_p, C.c_int, C.c_uint64, C.c_size_t, C.c_float
        protos = {
            "rko_splitmix64_next": (u64, [C.POINTER(C.c_uint64)]),
            "rko_splitmix64_at": (u64, [u64, u64]),
            "rko_gen_i8": (None, [vp, sz, u64, i32, i32]),
            "rko_gen_i16": (None, [vp, sz, u64, i32, i32]),
            "rko_gen_f32_uniform": (None, [vp, sz, u64, fl, fl]),
            "rko_gen_f32_normal": (None, [vp, sz, u64, fl, fl]),
            "rko_f32_to_f16": (C.c_uint16, [fl]), "rko_f16_to_f32": (fl, [C.c_uint16]),
            "rko_f32_to_f16_n": (None, [vp, vp, sz]), "rko_f16_to_f32_n": (None, [vp, vp, sz]),
            "rko_f32_to_bf16_trunc": (C.c_uint16, [fl]), "rko_bf16_to_f32": (fl, [C.c_uint16]),
            "rko_tf32_trunc": (fl, [fl]),
            "rko_int16_split": (None, [C.c_int16, C.POINTER(C.c_int8), C.POINTER(C.c_int8)]),
            "rko_matmul_fp16": (None, [i32, i32, i32, vp, vp, vp]),
            "rko_matmul_fp16_naive": (None, [i32, i32, i32, vp, vp, vp]),
            "rko_matmul_fp16_f32out": (None, [i32, i32, i32, vp, vp, vp]),
            "rko_matmul_int8": (None, [i32, i32, i32, vp, vp, vp]),
            "rko_matmul_int16_exact": (None, [i32, i32, i32, vp, vp, vp]),
            "rko_gw_partials": (None, [i32, i32, i32, i32, vp, vp, vp]),
            "rko_matmul_gw_f32": (None, [i32, i32, i32, i32, vp, vp, vp, vp, vp]),
            "rko_matmul_gw_f64": (None, [i32, i32, i32, i32, vp, vp, vp, vp, vp]),
            "rko_matmul_gw_rowscale_f32": (None, [i32, i32, i32, i32, vp, vp, vp, vp, vp]),
            "rko_matmul_bf16": (None, [i32, i32, i32, vp, vp, vp]),
            "rko_matmul_tf32": (None, [i32, i32, i32, vp, vp, vp]),
            "rko_matmul_f32": (None, [i32, i32, i32, vp, vp, vp]),
            "rko_set_threads": (i32, [i32]),
            "rko_f64_to_f16": (C.c_uint16, [C.c_double]), "rko_act_exact": (C.c_double, [i32, C.c_double]),
            "rko_geglu_f16": (None, [vp, vp, i32, vp, sz]),
            "rko_quant_rows_f32": (None, [i32, i32, vp, vp, vp]),
            "rko_flash_attn_f16": (None, [i32, i32, i32, i32, i32, i32, C.c_float, C.c_float, vp, vp, vp, vp, vp]),
            "rko_mha_self_f16": (None, [i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
            "rko_ffn_f16": (None, [i32, i32, i32, vp, vp, vp, vp, i32, vp]),
            "rko_mlp_f16": (None, [i32, i32, i32, i32, vp, vp, vp, vp, i32, vp]),
        }
        for n, (r, a) in protos.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle operands must be C-contiguous"
    return C.c_void_p(a.ctypes.data)


# ---- generators ------------------------------------------------------------------------

def gen_i8(shape, seed, lo=-128, hi=127) -> np.ndarray:
    out = np.empty(shape, np.int8)
    lib().rko_gen_i8(_p(out), out.size, seed, lo, hi)
    return out


def gen_i16(shape, seed, lo=-32768, hi=32767) -> np.ndarray:
    out = np.empty(shape, np.int16)
    lib().rko_gen_i16(_p(out), out.size, seed, lo, hi)
    return out


def gen_uniform(shape, seed, lo=-1.0, hi=1.0) -> np.ndarray:
    out = np.empty(shape, np.float32)
    lib().rko_gen_f32_uniform(_p(out), out.size, seed, lo, hi)
    return out


def gen_normal(shape, seed, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(shape, np.float32)
    lib().rko_gen_f32_normal(_p(out), out.size, seed, mean, std)
    return out


# ---- conversions -----------------------------------------------------------------------

def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().rko_f32_to_f16_n(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().rko_f16_to_f32_n(_p(h), _p(out), h.size)
    return out


def int16_split(x: int):
    hi, lo = C.c_int8(0), C.c_int8(0)
    lib().rko_int16_split(x, C.byref(hi), C.byref(lo))
    return hi.value, lo.value


# ---- references ------------------------------------------------------------------------

def matmul_fp16(A16: np.ndarray, B16: np.ndarray) -> np.ndarray:
    """A16 [M,K], B16 [N,K] as uint16 fp16 bits -> C fp16 bits [M,N]."""
    M, K = A16.shape
    N = B16.shape[0]
    C16 = np.empty((M, N), np.uint16)
    lib().rko_matmul_fp16(M, K, N, _p(A16), _p(B16), _p(C16))
    return C16


def matmul_fp16_naive(A16: np.ndarray, B16: np.ndarray) -> np.ndarray:
    """The reference tests' single-thread loop (tests/matmul_fp16_rocket.c:43-50): same bits as
    matmul_fp16, no threads, each fp16 operand converted where it is read."""
    M, K = A16.shape
    N = B16.shape[0]
    C16 = np.empty((M, N), np.uint16)
    lib().rko_matmul_fp16_naive(M, K, N, _p(A16), _p(B16), _p(C16))
    return C16


def matmul_fp16_f32out(A16, B16):
    M, K = A16.shape
    N = B16.shape[0]
    out = np.empty((M, N), np.float32)
    lib().rko_matmul_fp16_f32out(M, K, N, _p(A16), _p(B16), _p(out))
    return out


def matmul_int8(A, B):
    M, K = A.shape
    N = B.shape[0]
    out = np.empty((M, N), np.int32)
    lib().rko_matmul_int8(M, K, N, _p(A), _p(B), _p(out))
    return out


def matmul_int16_exact(A, B):
    M, K = A.shape
    N = B.shape[0]
    out = np.empty((M, N), np.int64)
    lib().rko_matmul_int16_exact(M, K, N, _p(A), _p(B), _p(out))
    return out


def gw_partials(A, B, group):
    M, K = A.shape
    N = B.shape[0]
    out = np.empty((M, K // group, N), np.int32)
    lib().rko_gw_partials(M, K, N, group, _p(A), _p(B), _p(out))
    return out


def matmul_gw_f32(A, B, a_scale, b_scale, group):
    M, K = A.shape
    N = B.shape[0]
    out = np.empty((M, N), np.float32)
    lib().rko_matmul_gw_f32(M, K, N, group, _p(A), _p(B), _p(np.ascontiguousarray(a_scale, np.float32)),
                            _p(np.ascontiguousarray(b_scale, np.float32)), _p(out))
    return out


def quant_rows(A):
    """Per-row int8 quantisation of fp32 A[M, K] -> (Aq int8, row_scale fp32)
    (reference tools/rk3576-w8a8-hostterm.c:51-68)."""
    A = np.ascontiguousarray(A, np.float32)
    M, K = A.shape
    q = np.empty((M, K), np.int8)
    rs = np.empty(M, np.float32)
    lib().rko_quant_rows_f32(M, K, _p(A), _p(q), _p(rs))
    return q, rs


def flash_attn_f16(Q16, K16, V16, mask16, scale, softcap):
    """Q [nh][T][dk], K [nkvh][n_kv][dk], V [nkvh][dv][n_kv], mask [T][n_kv] or None (fp16
    bits) -> out [nh][T][dv] (reference rocket_attn.c:181-228)."""
    nh, T, dk = Q16.shape
    nkvh, n_kv, _ = K16.shape
    dv = V16.shape[1]
    out = np.empty((nh, T, dv), np.uint16)
    q, k, v = (np.ascontiguousarray(a, np.uint16) for a in (Q16, K16, V16))
    m = None if mask16 is None else np.ascontiguousarray(mask16, np.uint16)
    lib().rko_flash_attn_f16(T, n_kv, dk, dv, nh, nkvh, scale, softcap, _p(q), _p(k), _p(v),
                             _p(m) if m is not None else None, _p(out))
    return out


def mha_self_f16(x16, Wq, bq, Wk, bk, Wv, bv, Wo, bo, n_head):
    """Encoder self-attention sublayer on fp16 bits (reference rocket_attn.c:41-84)."""
    T, d = x16.shape
    out = np.empty((T, d), np.uint16)
    # contiguous copies held for the duration of the call
    keep = [None if a is None else np.ascontiguousarray(a, np.uint16) for a in (x16, Wq, bq, Wk, bk, Wv, bv, Wo, bo)]
    ptrs = [None if a is None else _p(a) for a in keep]
    lib().rko_mha_self_f16(T, d, n_head, *ptrs, _p(out))
    return out


def geglu_f16(gate16, up16, kind):
    """fp16 bits in and out: f16(act(gate) * up) in double (reference rocket_ffn.c:33-38)."""
    g = np.ascontiguousarray(gate16, np.uint16)
    u = np.ascontiguousarray(up16, np.uint16)
    out = np.empty(g.shape, np.uint16)
    lib().rko_geglu_f16(_p(g), _p(u), kind, _p(out), g.size)
    return out


def ffn_f16(x16, Wg16, Wu16, Wd16, kind):
    """Gated FFN on fp16 bits (reference rocket_ffn.c:58-82)."""
    M, H = x16.shape
    I = Wg16.shape[0]
    out = np.empty((M, H), np.uint16)
    lib().rko_ffn_f16(M, H, I, _p(np.ascontiguousarray(x16)), _p(np.ascontiguousarray(Wg16)),
                      _p(np.ascontiguousarray(Wu16)), _p(np.ascontiguousarray(Wd16)), kind, _p(out))
    return out


def mlp_f16(x16, W116, b116, W216, kind):
    """Non-gated MLP host path on fp16 bits (reference rocket_ffn.c:236-254); b116 may be None."""
    M, Din = x16.shape
    Dff, Dout = W116.shape[0], W216.shape[0]
    out = np.empty((M, Dout), np.uint16)
    b = None if b116 is None else np.ascontiguousarray(b116, np.uint16)
    lib().rko_mlp_f16(M, Din, Dff, Dout, _p(np.ascontiguousarray(x16)), _p(np.ascontiguousarray(W116)),
                      _p(b) if b is not None else None, _p(np.ascontiguousarray(W216)), kind, _p(out))
    return out


def matmul_gw_rowscale_f32(A, B, a_row, b_scale, group):
    M, K = A.shape
    N = B.shape[0]
    out = np.empty((M, N), np.float32)
    lib().rko_matmul_gw_rowscale_f32(M, K, N, group, _p(A), _p(B), _p(np.ascontiguousarray(a_row, np.float32)),
                                     _p(np.ascontiguousarray(b_scale, np.float32)), _p(out))
    return out


def matmul_gw_f64(A, B, a_scale, b_scale, group):
    M, K = A.shape
    N = B.shape[0]
    out = np.empty((M, N), np.float64)
    lib().rko_matmul_gw_f64(M, K, N, group, _p(A), _p(B), _p(np.ascontiguousarray(a_scale, np.float32)),
                            _p(np.ascontiguousarray(b_scale, np.float32)), _p(out))
    return out


def _f32mm(fn, A, B):
    M, K = A.shape
    N = B.shape[0]
    out = np.empty((M, N), np.float32)
    getattr(lib(), fn)(M, K, N, _p(A), _p(B), _p(out))
    return out


def matmul_bf16(A, B):
    return _f32mm("rko_matmul_bf16", A, B)


def matmul_tf32(A, B):
    return _f32mm("rko_matmul_tf32", A, B)


def matmul_f32(A, B):
    return _f32mm("rko_matmul_f32", A, B)


def set_threads(n: int) -> int:
    return lib().rko_set_threads(n)


# ---- error measures (as the reference tests state them) --------------------------------

def norm_err(act: np.ndarray, ref: np.ndarray) -> float:
    """max|act - ref| / max|ref| (tests/matmul_bf16_tiled_rocket.c:84-111)."""
    act = act.astype(np.float64)
    ref = ref.astype(np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(act - ref)) / (den if den > 0 else 1.0))


def rms_err(act, ref) -> float:
    """max|act - ref| / rms(ref) (tests/matmul_int8_groupwise_rocket.c:65-84)."""
    act = act.astype(np.float64)
    ref = ref.astype(np.float64)
    rms = float(np.sqrt(np.mean(ref * ref)))
    return float(np.max(np.abs(act - ref)) / (rms if rms > 0 else 1.0))
