"""The fp32 order in which the group-wise kernels fold a product with per-group activation
scales a_scale[M][nG] (the reference layout), for the parity tests.

Each row is decided on its own scales: a row that carries one scale for all its groups (a
per-row scale passed in the reference's layout), with 4 <= nG <= 64, folds in the row-scale
order, fmaf(b_scale, P_g, acc) over g times the row's scale (oracle matmul_gw_rowscale_f32);
every other row folds in the reference's order, fmaf(a_scale * b_scale, P_g, acc) (oracle
matmul_gw_f32). A row's bits therefore do not depend on the rows batched with it.
"""
import numpy as np


def row_kinds(asc):
    """Per row: True when it folds in the row-scale order."""
    a = np.ascontiguousarray(asc, dtype=np.float32).view(np.int32)
    nG = a.shape[1]
    return np.all(a == a[:, :1], axis=1) & (4 <= nG <= 64)


def rows_constant(asc):
    """Every row of a_scale holds the same bits in all its groups."""
    a = np.ascontiguousarray(asc, dtype=np.float32).view(np.int32)
    return bool(np.all(a == a[:, :1]))


def row_order(asc):
    """Every row folds in the row-scale order."""
    return bool(np.all(row_kinds(asc)))


def gw_f32(orc, A, B, asc, bsc, group):
    """The kernels' fp32 result for rows A with per-group scales asc, each row in its own order."""
    kinds = row_kinds(asc)
    out = np.empty((A.shape[0], B.shape[0]), np.float32)
    if kinds.any():
        out[kinds] = orc.matmul_gw_rowscale_f32(np.ascontiguousarray(A[kinds]), B,
                                                np.ascontiguousarray(asc[kinds, 0]), bsc, group)
    if (~kinds).any():
        out[~kinds] = orc.matmul_gw_f32(np.ascontiguousarray(A[~kinds]), B, np.ascontiguousarray(asc[~kinds]),
                                        bsc, group)
    return out
