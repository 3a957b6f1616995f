"""The fp32 order in which the group-wise kernels fold a product with per-group activation
scales a_scale[M][nG] (the reference layout), for the parity tests.

A row tile whose rows each carry one scale for all their groups (a per-row scale passed in the
reference's layout), with 4 <= nG <= 64, folds in the row-scale order: fmaf(b_scale, P_g, acc)
over g, times the row's scale (oracle matmul_gw_rowscale_f32). Every other tile folds in the
reference's order, fmaf(a_scale * b_scale, P_g, acc) (oracle matmul_gw_f32). The kernel decides
per row tile, so a helper that sees the whole matrix is exact when its rows are all constant
or none of them is tile-aligned otherwise; mixed matrices are checked row by row against both.
"""
import numpy as np


def rows_constant(asc):
    """Every row of a_scale holds the same bits in all its groups."""
    a = np.ascontiguousarray(asc, dtype=np.float32).view(np.int32)
    return bool(np.all(a == a[:, :1]))


def row_order(asc):
    """The kernels fold in the row-scale order for this a_scale (all rows constant)."""
    nG = asc.shape[1]
    return 4 <= nG <= 64 and rows_constant(asc)


def gw_f32(orc, A, B, asc, bsc, group, row=None):
    """The kernels' fp32 result for rows A with per-group scales asc (row: the order, decided on
    the whole problem's scales; None: decided on asc)."""
    if row is None:
        row = row_order(asc)
    if row:
        return orc.matmul_gw_rowscale_f32(A, B, np.ascontiguousarray(asc[:, 0]), bsc, group)
    return orc.matmul_gw_f32(A, B, asc, bsc, group)
