"""GPU parity of the group-wise products at the BASELINE workloads, through the C-ABI.

* config 5 (MoE, resident int8 group-32 weights, 8 experts, 4096 tokens routed top-2) at
  its real size, on the grouped per-row-scale launch the bench times, on the grouped
  per-group-scale launch and on the reference's per-expert rocket_matmul_int8_prepacked_gw;
* config 3 (W4A8, group 128) through the reference's rocket_matmul_int4_prepacked_gw, whose
  per-group activation scales now run on the same 8-wave 256 x 128 tiles as the per-row
  entry, and through the benched per-row entry with its partials dumped;
* 8-wave tiles whose last row tile leaves waves without rows (M = 260), group 32 and 64, and
  a grouped launch whose light last-row tiles run after the heavy ones.

Bars (reference tests/matmul_int8_groupwise_rocket.c:65-84,
tests/matmul_int8_prepacked_gw_rocket.c:46-240): per-group int32 partials bit-exact, taken
from the launch under test (the dump is a run-time switch of that kernel); fp32 results
bit-identical to the oracle's fmaf order for the launch's formula; within 1e-5 rms of the
fp64 combine (config 3 also within its 1e-3 normalised gate).
"""
import ctypes as C
import sys

import numpy as np
import pytest

import gworder
import rocketnpu as R

pytestmark = pytest.mark.gpu

SEED = 0x52434C00


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def quantise_groups(w, group):
    """Symmetric per-(row, group) int8 quantisation of fp32 weights [N, K]: scale = amax/127,
    code = round(w / scale) (the config-5 weight recipe)."""
    N, K = w.shape
    g = w.reshape(N, K // group, group)
    amax = np.abs(g).max(axis=2)
    scale = np.where(amax > 0, amax / 127.0, 1.0).astype(np.float32)
    q = np.clip(np.rint(g / scale[:, :, None]), -127, 127).astype(np.int8).reshape(N, K)
    return np.ascontiguousarray(q), np.ascontiguousarray(scale)


def check_rows(orc, got, A, B, a_row, bsc, group, rows, a_group=None):
    """got[rows] against the oracle: bit-identical to the kernels' fp32 order for the entry
    (per-row scales: the row-scale order; per-group scales: each row's own order, as gworder
    decides it from the row's scales), and within 1e-5 rms of the fp64 combine."""
    Ar = np.ascontiguousarray(A[rows])
    if a_group is None:
        ar = np.ascontiguousarray(a_row[rows])
        want = orc.matmul_gw_rowscale_f32(Ar, B, ar, bsc, group)
        a64 = np.ascontiguousarray(np.repeat(ar[:, None], A.shape[1] // group, axis=1))
    else:
        a64 = np.ascontiguousarray(a_group[rows])
        want = gworder.gw_f32(orc, Ar, B, a64, bsc, group)
    assert np.array_equal(got[rows], want)
    ref = orc.matmul_gw_f64(Ar, B, a64, bsc, group)
    if np.any(ref != 0):
        assert orc.rms_err(got[rows], ref) <= 1e-5


# ---------------------------------------------------------------------------------------
# config 5: the MoE expert FFN at its real size
# ---------------------------------------------------------------------------------------
E, T, H, I, G = 8, 4096, 2048, 1408, 32


@pytest.fixture(scope="module")
def moe(lib, orc):
    """Eight experts' resident weights (gate and up stacked as one [2I, H] weight, down
    [H, I]), int8 group-32 codes of N(0, 0.02) values, packed once on one context."""
    say("config 5: packing 8 experts")
    ctx = lib.rocket_i8_ctx_create(1)
    assert ctx
    rng = np.random.default_rng(SEED)
    ex = []
    for e in range(E):
        gu, sgu = quantise_groups(rng.normal(0, 0.02, (2 * I, H)).astype(np.float32), G)
        dn, sdn = quantise_groups(rng.normal(0, 0.02, (H, I)).astype(np.float32), G)
        wgu = lib.rocket_i8_weights_pack_gw(ctx, 4, H, 2 * I, R.ptr(gu), G)
        wdn = lib.rocket_i8_weights_pack_gw(ctx, 4, I, H, R.ptr(dn), G)
        assert wgu and wdn
        assert lib.rocket_i8_weights_bytes(wgu) <= 1.2 * 2 * I * H
        ex.append(dict(gu=gu, sgu=sgu, dn=dn, sdn=sdn, wgu=wgu, wdn=wdn))
    yield ctx, ex
    for x in ex:
        lib.rocket_i8_weights_free(ctx, x["wgu"])
        lib.rocket_i8_weights_free(ctx, x["wdn"])
    lib.rocket_i8_ctx_free(ctx)


def route(orc, seed):
    """4096 fp16 N(0,1) tokens quantised to int8 per row, each sent to two distinct experts
    uniformly at random; returns per expert the gathered rows, padded with zero rows to a
    multiple of 4 (API contract, reference rocket_prepacked_int8.c:678-682)."""
    x16 = orc.f32_to_f16_bits(orc.gen_normal((T, H), seed))
    Aq, rs = orc.quant_rows(orc.f16_bits_to_f32(x16))
    rng = np.random.default_rng(seed)
    top2 = np.argsort(rng.random((T, E)), axis=1)[:, :2]
    out = []
    for e in range(E):
        idx = np.nonzero((top2 == e).any(axis=1))[0]
        m = len(idx)
        mp = (m + 3) // 4 * 4
        A = np.zeros((mp, H), np.int8)
        a = np.zeros(mp, np.float32)
        A[:m], a[:m] = Aq[idx], rs[idx]
        out.append((A, a, m))
    return out


def sample_rows(mp):
    """First rows, a middle row, the first rows of the last 256-row tile and the last rows."""
    t0 = (mp - 1) // 256 * 256
    return np.unique(np.r_[0:2, mp // 2, t0:t0 + 2, mp - 8:mp])


def grouped(lib, ctx, entry, Ms, As, scales, bss, Cs, ws, dump=None):
    pM, k0 = R.int_array(Ms)
    pA, k1 = R.ptr_array(As)
    pa, k2 = R.ptr_array(scales)
    pb, k3 = R.ptr_array(bss)
    pC, k4 = R.ptr_array(Cs)
    pW = (C.c_void_p * len(ws))(*ws)
    args = [ctx, len(Ms), pM, As[0].shape[1], Cs[0].shape[1], pA, pa, pb, pC, C.cast(pW, R.pp)]
    if dump is None:
        return getattr(lib, entry)(*args)
    r0, k5 = R.int_array(dump[0])
    nr, k6 = R.int_array(dump[1])
    pP, k7 = R.ptr_array(dump[2])
    return getattr(lib, entry + "_dump")(*args, r0, nr, pP)


@pytest.mark.parametrize("routing", [0, 1, 2])
def test_moe_config5_grouped_rowscale(lib, orc, moe, routing):
    """The bench's launches: gate+up (N = 2816, K = 2048) then down (N = 2048, K = 1408),
    each one grouped per-row-scale launch over the 8 experts, on gathered routed rows. The
    down product's input is act(gate) * up of the first product, re-quantised per row."""
    ctx, ex = moe
    say(f"config 5 routing {routing}")
    per = route(orc, 0x52434B05 + 17 * routing)
    Ms = [A.shape[0] for A, _, _ in per]
    say(f"  per-expert rows {[m for _, _, m in per]} (padded {Ms})")
    for stage in ("gate_up", "down"):
        if stage == "gate_up":
            As = [A for A, _, _ in per]
            ars = [a for _, a, _ in per]
            Bs = [x["gu"] for x in ex]
            bss = [x["sgu"] for x in ex]
            ws = [x["wgu"] for x in ex]
            N = 2 * I
        else:
            As, ars = [], []
            for e in range(E):
                g, u = Cgu[e][:, :I], Cgu[e][:, I:]
                h = (g / (1.0 + np.exp(-g.astype(np.float64)))).astype(np.float32) * u
                q, r = orc.quant_rows(h)
                As.append(q)
                ars.append(r)
            Bs = [x["dn"] for x in ex]
            bss = [x["sdn"] for x in ex]
            ws = [x["wdn"] for x in ex]
            N = H
        K = As[0].shape[1]
        nG = K // G
        Cs = [np.full((m, N), np.nan, np.float32) for m in Ms]
        row0 = [m - 8 for m in Ms]
        Ps = [np.full((8, nG, N), -7, np.int32) for _ in Ms]
        assert grouped(lib, ctx, "rocket_matmul_int8_prepacked_gw_grouped_rowscale", Ms, As, ars, bss, Cs, ws,
                       (row0, [8] * E, Ps)) == 0
        C2 = [np.full((m, N), np.nan, np.float32) for m in Ms]
        assert grouped(lib, ctx, "rocket_matmul_int8_prepacked_gw_grouped_rowscale", Ms, As, ars, bss, C2, ws) == 0
        for e in range(E):
            assert np.array_equal(Cs[e], C2[e]), (stage, e)     # the dump changes nothing else
            assert np.array_equal(Ps[e], orc.gw_partials(np.ascontiguousarray(As[e][row0[e]:]), Bs[e], G)), (stage, e)
            check_rows(orc, Cs[e], As[e], Bs[e], ars[e], bss[e], G, sample_rows(Ms[e]))
        say(f"  {stage}: 8 experts, partials and sampled rows exact")
        if stage == "gate_up":
            Cgu = Cs


def test_grouped_light_tiles_run_last(lib, orc, moe):
    """A grouped group-32 launch on 256 x 128 tiles numbers the light last-row tiles (at most
    128 of a tile's 256 rows) after every heavy tile: products whose only tile is light
    (M = 4, 68, 128), an empty product (M = 0), last tiles just above and at the half (132 and
    128 rows) and a one-tile-plus-4-rows product (260) all land on the right rows."""
    ctx, ex = moe
    Ms = [260, 0, 4, 1024, 132, 128, 388, 68]
    say(f"grouped light tiles last: M = {Ms}")
    rng = np.random.default_rng(SEED + 91)
    As = [np.ascontiguousarray(rng.integers(-128, 128, (max(m, 4), H), dtype=np.int8)[:m]) for m in Ms]
    As = [a if a.shape[0] else np.zeros((4, H), np.int8) for a in As]
    ars = [np.ascontiguousarray(rng.uniform(0.001, 0.05, max(m, 4)).astype(np.float32)) for m in Ms]
    N = 2 * I
    Cs = [np.full((max(m, 4), N), np.nan, np.float32) for m in Ms]
    assert grouped(lib, ctx, "rocket_matmul_int8_prepacked_gw_grouped_rowscale", Ms, As, ars,
                   [x["sgu"] for x in ex], Cs, [x["wgu"] for x in ex]) == 0
    for e, m in enumerate(Ms):
        if m == 0:
            assert np.isnan(Cs[e]).all()     # an empty product writes nothing
            continue
        rows = np.unique(np.r_[0:2, m // 2, max(m - 4, 0):m])
        check_rows(orc, Cs[e], As[e], ex[e]["gu"], ars[e], ex[e]["sgu"], G, rows)
    say("  every product's sampled rows exact")


def test_moe_config5_reference_layout(lib, orc, moe):
    """The reference's own resident entry, one expert at a time (reference
    tests/matmul_int8_prepacked_gw_rocket.c:46-240, tests/matmul_int8_crossm_gw_rocket.c:74-120),
    with the row scale repeated over the groups as a reference caller passes it, and the
    grouped per-group-scale launch with scales that differ per group, partials dumped."""
    ctx, ex = moe
    per = route(orc, 0x52434B05)
    Ms = [A.shape[0] for A, _, _ in per]
    nG = H // G
    ascs = []
    for e, (A, a, m) in enumerate(per):
        asc = np.ascontiguousarray(np.repeat(a[:, None], nG, axis=1))
        Cf = np.empty((A.shape[0], 2 * I), np.float32)
        assert lib.rocket_matmul_int8_prepacked_gw(ctx, A.shape[0], H, 2 * I, R.ptr(A), R.ptr(asc),
                                                   R.ptr(ex[e]["sgu"]), R.ptr(Cf), ex[e]["wgu"]) == 0
        check_rows(orc, Cf, A, ex[e]["gu"], None, ex[e]["sgu"], G, sample_rows(A.shape[0]), a_group=asc)
        # per-group activation scales that differ per group, for the grouped launch below
        ascs.append(orc.gen_uniform((A.shape[0], nG), SEED + 40 + e, 0.5, 1.5))
    say("  reference-layout per-expert calls exact")
    As = [A for A, _, _ in per]
    Cs = [np.empty((m, 2 * I), np.float32) for m in Ms]
    row0 = [m - 12 for m in Ms]
    Ps = [np.empty((12, nG, 2 * I), np.int32) for _ in Ms]
    assert grouped(lib, ctx, "rocket_matmul_int8_prepacked_gw_grouped", Ms, As, ascs,
                   [x["sgu"] for x in ex], Cs, [x["wgu"] for x in ex], (row0, [12] * E, Ps)) == 0
    for e in range(E):
        assert np.array_equal(Ps[e], orc.gw_partials(np.ascontiguousarray(As[e][row0[e]:]), ex[e]["gu"], G))
        check_rows(orc, Cs[e], As[e], ex[e]["gu"], None, ex[e]["sgu"], G, sample_rows(Ms[e]), a_group=ascs[e])
    say("  grouped per-group-scale launch exact")


# ---------------------------------------------------------------------------------------
# config 3 through the reference's entries, and the benched entry's partials
# ---------------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def cfg3(lib, orc):
    M, K, N, group = 512, 3840, 15360, 128
    nG = K // group
    x = orc.gen_normal((M, K), 0x52434B03)
    A = np.clip(np.round(x * 32), -128, 127).astype(np.int8)
    arow = (np.abs(x).max(axis=1) / 127).astype(np.float32)
    B = orc.gen_i8((N, K), 0x52434B03 + 1, -8, 7)
    bsc = orc.f16_bits_to_f32(orc.f32_to_f16_bits(orc.gen_uniform((N, nG), 0x52434B03 + 2, 0.005, 0.02)))
    ctx = lib.rocket_i4_ctx_create(1)
    w = lib.rocket_i4_weights_pack_gw(ctx, M, K, N, R.ptr(B), group)
    assert w
    yield dict(M=M, K=K, N=N, group=group, nG=nG, A=A, arow=arow, B=B, bsc=bsc, ctx=ctx, w=w)
    lib.rocket_i4_weights_free(ctx, w)
    lib.rocket_i4_ctx_free(ctx)


CFG3_ROWS = np.r_[0:4, 127:129, 250:262, 380, 508:512]


def test_config3_rowscale_partials_from_the_benched_kernel(lib, orc, cfg3):
    """rocket_matmul_int4_prepacked_gw_rowscale (the bench's entry) with rows 250..261 of its
    partials dumped: they straddle the boundary of the two 256-row tiles."""
    c = cfg3
    M, K, N, group, nG = c["M"], c["K"], c["N"], c["group"], c["nG"]
    say("config 3 rowscale dump")
    Cd = np.full((M, N), np.nan, np.float32)
    P = np.full((12, nG, N), -7, np.int32)
    assert lib.rocket_matmul_int4_prepacked_gw_rowscale_dump(c["ctx"], M, K, N, R.ptr(c["A"]), R.ptr(c["arow"]),
                                                             R.ptr(c["bsc"]), R.ptr(Cd), c["w"], 250, 12,
                                                             R.ptr(P)) == 0
    assert np.array_equal(P, orc.gw_partials(np.ascontiguousarray(c["A"][250:262]), c["B"], group))
    Cf = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_int4_prepacked_gw_rowscale(c["ctx"], M, K, N, R.ptr(c["A"]), R.ptr(c["arow"]),
                                                        R.ptr(c["bsc"]), R.ptr(Cf), c["w"]) == 0
    assert np.array_equal(Cf, Cd)
    check_rows(orc, Cf, c["A"], c["B"], c["arow"], c["bsc"], group, CFG3_ROWS)


@pytest.mark.parametrize("scales", ["row_repeated", "per_group"])
def test_config3_reference_entry(lib, orc, cfg3, scales):
    """rocket_matmul_int4_prepacked_gw (reference include/rocket_matmul.h:739-775, the call
    ggml-rocket makes) at the config-3 shape on the 8-wave 256 x 128 tiles: per-group
    activation scales a_scale[M * nG], either the row scale repeated (what a per-token
    quantised caller passes) or scales that differ per group. Rows 252..259 of its partials
    are dumped from the same launch."""
    c = cfg3
    M, K, N, group, nG = c["M"], c["K"], c["N"], c["group"], c["nG"]
    say(f"config 3 reference entry, {scales} activation scales")
    if scales == "row_repeated":
        asc = np.ascontiguousarray(np.repeat(c["arow"][:, None], nG, axis=1))
    else:
        asc = orc.gen_uniform((M, nG), SEED + 60, 0.002, 0.03)
    Cf = np.full((M, N), np.nan, np.float32)
    P = np.full((8, nG, N), -7, np.int32)
    assert lib.rocket_matmul_int4_prepacked_gw_dump(c["ctx"], M, K, N, R.ptr(c["A"]), R.ptr(asc), R.ptr(c["bsc"]),
                                                    R.ptr(Cf), c["w"], 252, 8, R.ptr(P)) == 0
    assert np.array_equal(P, orc.gw_partials(np.ascontiguousarray(c["A"][252:260]), c["B"], group))
    C2 = np.empty((M, N), np.float32)
    assert lib.rocket_matmul_int4_prepacked_gw(c["ctx"], M, K, N, R.ptr(c["A"]), R.ptr(asc), R.ptr(c["bsc"]),
                                               R.ptr(C2), c["w"]) == 0
    assert np.array_equal(C2, Cf)
    check_rows(orc, Cf, c["A"], c["B"], None, c["bsc"], group, CFG3_ROWS, a_group=asc)
    Ar = np.ascontiguousarray(c["A"][CFG3_ROWS])
    rel = orc.norm_err(Cf[CFG3_ROWS], orc.matmul_gw_f64(Ar, c["B"], np.ascontiguousarray(asc[CFG3_ROWS]),
                                                        c["bsc"], group))
    say(f"  norm rel err vs fp64 {rel:.3g}")
    assert rel <= 1e-3


# ---------------------------------------------------------------------------------------
# 8-wave tiles with waves past M (the dead-wave skip of the group-32 / 64 kernels)
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("bfmt", ["int8", "int4"])
def test_eight_wave_dead_waves(lib, orc, fd, group, bfmt):
    """M = 260: the second 256-row tile holds 4 rows, so three of its four wave rows lie
    past M and skip their fragment reads, MFMAs and folds. N = 12288 gives 192 tiles, which
    selects the 8-wave 256 x 128 tile. Per-row and per-group activation scales; partials of
    rows 250..259 dumped across the tile boundary."""
    M, K, N = 260, 1024, 12288
    nG = K // group
    say(f"dead waves {bfmt} g{group}")
    A = orc.gen_i8((M, K), SEED + 70 + group)
    B = orc.gen_i8((N, K), SEED + 71 + group, *((-8, 7) if bfmt == "int4" else (-128, 127)))
    arow = orc.gen_uniform((M,), SEED + 72, 0.5, 1.5)
    asc = orc.gen_uniform((M, nG), SEED + 73, 0.5, 1.5)
    bsc = orc.gen_uniform((N, nG), SEED + 74, 0.005, 0.02)
    rows = np.r_[0:4, 63:66, 191:193, 250:260]
    if bfmt == "int8":
        ctx = lib.rocket_i8_ctx_create(1)
        w = lib.rocket_i8_weights_pack_gw(ctx, M, K, N, R.ptr(B), group)
        rs_dump, pg_dump = lib.rocket_matmul_int8_prepacked_gw_rowscale_dump, lib.rocket_matmul_int8_prepacked_gw_dump
    else:
        ctx = lib.rocket_i4_ctx_create(1)
        w = lib.rocket_i4_weights_pack_gw(ctx, M, K, N, R.ptr(B), group)
        rs_dump, pg_dump = lib.rocket_matmul_int4_prepacked_gw_rowscale_dump, lib.rocket_matmul_int4_prepacked_gw_dump
    assert w
    want_P = orc.gw_partials(np.ascontiguousarray(A[250:260]), B, group)
    for name, fn, sc in (("rowscale", rs_dump, arow), ("per-group", pg_dump, asc)):
        Cf = np.full((M, N), np.nan, np.float32)
        P = np.full((10, nG, N), -7, np.int32)
        assert fn(ctx, M, K, N, R.ptr(A), R.ptr(sc), R.ptr(bsc), R.ptr(Cf), w, 250, 10, R.ptr(P)) == 0
        assert np.array_equal(P, want_P), name
        assert np.all(np.isfinite(Cf)), name
        if name == "rowscale":
            check_rows(orc, Cf, A, B, arow, bsc, group, rows)
        else:
            check_rows(orc, Cf, A, B, None, bsc, group, rows, a_group=asc)
    if bfmt == "int8":
        lib.rocket_i8_weights_free(ctx, w)
        lib.rocket_i8_ctx_free(ctx)
    else:
        lib.rocket_i4_weights_free(ctx, w)
        lib.rocket_i4_ctx_free(ctx)


@pytest.mark.parametrize("K,group", [(2048, 32), (2080, 32), (96, 32), (3840, 128)])
def test_per_group_scales_fold_order(lib, orc, fd, K, group):
    """Per-group activation scales whose rows are constant in the first 256 rows and random in
    the rest: the constant rows fold in the row-scale order when 4 <= nG <= 64 (nG = 64 and
    30 here; 65 and 3 keep the reference order), the others in the reference order; the
    one-shot and the resident entries give the same bits."""
    M, N = 512, 1024
    nG = K // group
    say(f"fold order K={K} g={group} nG={nG}")
    A = orc.gen_i8((M, K), SEED + 90 + nG)
    B = orc.gen_i8((N, K), SEED + 91 + nG)
    asc = orc.gen_uniform((M, nG), SEED + 92 + nG, 0.5, 1.5)
    asc[:256] = asc[:256, :1]
    asc = np.ascontiguousarray(asc)
    bsc = orc.gen_uniform((N, nG), SEED + 93 + nG, 0.005, 0.02)
    Co = np.full((M, N), np.nan, np.float32)
    assert lib.rocket_matmul_int8_groupwise(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(asc), R.ptr(bsc), R.ptr(Co), group) == 0
    ctx = lib.rocket_i8_ctx_create(1)
    w = lib.rocket_i8_weights_pack_gw(ctx, M, K, N, R.ptr(B), group)
    assert w
    Cr = np.full((M, N), np.nan, np.float32)
    assert lib.rocket_matmul_int8_prepacked_gw(ctx, M, K, N, R.ptr(A), R.ptr(asc), R.ptr(bsc), R.ptr(Cr), w) == 0
    lib.rocket_i8_weights_free(ctx, w)
    lib.rocket_i8_ctx_free(ctx)
    assert np.array_equal(Co, Cr)
    for lo, hi, row in ((0, 256, 4 <= nG <= 64), (256, 512, False)):
        rows = np.r_[lo:lo + 3, hi - 3:hi]
        Ar, ar = np.ascontiguousarray(A[rows]), np.ascontiguousarray(asc[rows])
        assert np.array_equal(Co[rows], gworder.gw_f32(orc, Ar, B, ar, bsc, group)), (lo, row)
        assert orc.rms_err(Co[rows], orc.matmul_gw_f64(Ar, B, ar, bsc, group)) <= 1e-5


@pytest.mark.parametrize("K,group", [(2048, 32), (3840, 128)])
def test_fold_order_is_per_row(lib, orc, fd, K, group):
    """A row's fp32 bits depend on its own activation scales only: one row whose scales vary
    over its groups, placed among rows that each carry one scale, leaves every other row with
    the bits it has when all rows carry one scale (the row-scale order), and itself folds in
    the reference order; rows of both kinds sit in every row tile of the launch."""
    M, N = 512, 1024
    nG = K // group
    say(f"per-row fold order K={K} g={group}")
    A = orc.gen_i8((M, K), SEED + 100 + nG)
    B = orc.gen_i8((N, K), SEED + 101 + nG)
    bsc = orc.gen_uniform((N, nG), SEED + 102 + nG, 0.005, 0.02)
    arow = orc.gen_uniform((M, 1), SEED + 103 + nG, 0.5, 1.5)
    uni = np.ascontiguousarray(np.repeat(arow, nG, axis=1))
    odd = np.array([5, 129, 300, 511])   # one row in each 128-row tile, two 256-row tiles
    mixed = uni.copy()
    mixed[odd] = orc.gen_uniform((len(odd), nG), SEED + 104 + nG, 0.5, 1.5)
    outs = []
    for asc in (uni, mixed):
        C = np.full((M, N), np.nan, np.float32)
        assert lib.rocket_matmul_int8_groupwise(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(asc), R.ptr(bsc), R.ptr(C),
                                                group) == 0
        outs.append(C)
    keep = np.setdiff1d(np.arange(M), odd)
    assert np.array_equal(outs[0][keep], outs[1][keep])
    rows = np.r_[0:3, 254:258, M - 3:M]
    rows = np.setdiff1d(rows, odd)
    Ar = np.ascontiguousarray(A[rows])
    assert np.array_equal(outs[1][rows], orc.matmul_gw_rowscale_f32(Ar, B, np.ascontiguousarray(arow[rows, 0]),
                                                                     bsc, group))
    Ao, ao = np.ascontiguousarray(A[odd]), np.ascontiguousarray(mixed[odd])
    assert np.array_equal(outs[1][odd], orc.matmul_gw_f32(Ao, B, ao, bsc, group))
    assert np.array_equal(outs[1][odd], gworder.gw_f32(orc, Ao, B, ao, bsc, group))
    assert orc.rms_err(outs[1][odd], orc.matmul_gw_f64(Ao, B, ao, bsc, group)) <= 1e-5


def test_dump_rejections(lib, orc, cfg3):
    """Dump windows outside the problem are refused before any launch."""
    c = cfg3
    M, K, N = c["M"], c["K"], c["N"]
    P = np.empty(8, np.int32)
    Cf = np.empty(8, np.float32)
    for row0, nrows in ((-1, 4), (510, 4), (0, -1)):
        assert lib.rocket_matmul_int4_prepacked_gw_rowscale_dump(c["ctx"], M, K, N, R.ptr(c["A"]), R.ptr(c["arow"]),
                                                                 R.ptr(c["bsc"]), R.ptr(Cf), c["w"], row0, nrows,
                                                                 R.ptr(P)) == R.ROCKET_E_SHAPE
    assert lib.rocket_matmul_int4_prepacked_gw_rowscale_dump(c["ctx"], M, K, N, R.ptr(c["A"]), R.ptr(c["arow"]),
                                                             R.ptr(c["bsc"]), R.ptr(Cf), c["w"], 0, 4,
                                                             None) == R.ROCKET_E_SHAPE
