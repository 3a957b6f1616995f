"""Writes tests/golden/golden.npz: small fixed cases for every arithmetic of the matmul
path, with expected outputs computed by numpy alone (int64 / float64 matmuls of the
operands after the reference's own input transforms), independently of oracle/.

Inputs come from numpy's PCG64 with fixed seeds. The transforms restated here are the
reference's: int16 clamp to [-32768, 32639] (rocket_matmul.c:3400,3404), bf16 truncation
(rocket_matmul.c:3444-3446), tf32 13-bit truncation (tests/matmul_tf32_tiled_rocket.c:52-56),
per-group exact partials combined with a*b scales (rocket_matmul.c:2842-2856).

Run:  python tests/golden/make_golden.py   (rewrites golden.npz deterministically)
"""
import os

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")


def i8(rng, shape, lo=-128, hi=127):
    return rng.integers(lo, hi + 1, shape, dtype=np.int64).astype(np.int8)


def main():
    rng = np.random.default_rng(0x52434B47)
    g = {}
    # int8 -> int32 (incl. extremes in the first row)
    for tag, (M, K, N) in {"int8_a": (4, 64, 32), "int8_m1": (1, 32, 32)}.items():
        A, B = i8(rng, (M, K)), i8(rng, (N, K))
        A[0, :4] = [-128, 127, -128, 127]
        g[f"{tag}_A"], g[f"{tag}_B"] = A, B
        g[f"{tag}_C"] = (A.astype(np.int64) @ B.astype(np.int64).T).astype(np.int32)
    # int16 exact with clamp boundaries
    M, K, N = 4, 64, 32
    A = rng.integers(-32768, 32768, (M, K), dtype=np.int64).astype(np.int16)
    B = rng.integers(-32768, 32768, (N, K), dtype=np.int64).astype(np.int16)
    A[0, :6] = [32767, 32640, 32639, -32768, 32641, -1]
    B[1, :4] = [32767, -32768, 32700, 32639]
    g["int16_A"], g["int16_B"] = A, B
    g["int16_C"] = np.minimum(A.astype(np.int64), 32639) @ np.minimum(B.astype(np.int64), 32639).T
    # fp16: configs[0] shape, U[-1,1] rounded to fp16 by numpy (IEEE RNE)
    M, K, N = 64, 256, 128
    A16 = rng.uniform(-1, 1, (M, K)).astype(np.float16)
    B16 = rng.uniform(-1, 1, (N, K)).astype(np.float16)
    g["fp16_A"], g["fp16_B"] = A16.view(np.uint16), B16.view(np.uint16)
    g["fp16_ref64"] = A16.astype(np.float64) @ B16.astype(np.float64).T
    # group-wise int8 (group 64) and int4-weight (group 128) with exact per-group partials
    for tag, (M, K, N, grp, blo, bhi) in {"gw8": (8, 256, 64, 64, -128, 127),
                                          "gw4": (8, 256, 64, 128, -8, 7)}.items():
        nG = K // grp
        A, B = i8(rng, (M, K)), i8(rng, (N, K), blo, bhi)
        asc = rng.uniform(0.5, 1.5, (M, nG)).astype(np.float32)
        bsc = rng.uniform(0.005, 0.02, (N, nG)).astype(np.float32)
        P = np.stack([A[:, j * grp:(j + 1) * grp].astype(np.int64) @ B[:, j * grp:(j + 1) * grp].astype(np.int64).T
                      for j in range(nG)], axis=1)
        g[f"{tag}_A"], g[f"{tag}_B"], g[f"{tag}_as"], g[f"{tag}_bs"] = A, B, asc, bsc
        g[f"{tag}_group"] = np.array(grp)
        g[f"{tag}_P"] = P.astype(np.int32)
        g[f"{tag}_ref64"] = np.einsum("mg,ng,mgn->mn", asc.astype(np.float64), bsc.astype(np.float64),
                                      P.astype(np.float64))
    # bf16 / tf32 on fp32 operands
    M, K, N = 4, 64, 32
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    trunc = lambda X, m: (X.view(np.uint32) & np.uint32(m)).view(np.float32).astype(np.float64)
    g["flt_A"], g["flt_B"] = A, B
    g["bf16_ref64"] = trunc(A, 0xFFFF0000) @ trunc(B, 0xFFFF0000).T
    g["tf32_ref64"] = trunc(A, 0xFFFFE000) @ trunc(B, 0xFFFFE000).T
    g["f32_ref64"] = A.astype(np.float64) @ B.astype(np.float64).T
    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT}: {len(g)} arrays")


if __name__ == "__main__":
    main()
