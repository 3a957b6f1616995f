"""The C-ABI boundary on the CPU: every symbol include/*.h declares is exported, and every
contract that needs no device holds (planner validation and counts, shape rejections
before any device call, stub entries, logging, the machine profile).

Reference contracts: rocket_matmul.h:38-45 (planner return), rocket_matmul.c:486-568,
2383-2437, 2671-2714, 2917-2956, 3320-3359, 3797-3838 (alignment), :3139 (int4 group
bound), rocket_npu.h:41-48 (status values), rocket_log.h:14-66.
"""
import ctypes as C
import os
import re

import numpy as np

import pytest

import rocketnpu as R


def test_every_header_function_is_exported(lib):
    names = R.header_functions()
    assert len(names) > 100
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the binding declares exactly the header surface
    assert set(names) == set(R.PROTOS), set(names) ^ set(R.PROTOS)
    for sym in R.DATA_SYMBOLS:
        assert C.c_void_p.in_dll(lib, sym) is not None


def test_library_resolves_every_symbol_at_load(lib):
    # ctypes binds lazily; a kernel whose launch stub was not emitted only shows up as an
    # unresolved symbol when every relocation is processed at load time
    C.CDLL(R.LIB_PATH, mode=os.RTLD_NOW | os.RTLD_LOCAL)


def test_status_values_match_reference():
    text = open(os.path.join(R.INCLUDE, "rocket_npu.h")).read()
    vals = dict(re.findall(r"(ROCKET_E?_?\w+)\s*=\s*(-?\d+)", text))
    assert vals["ROCKET_OK"] == "0" and vals["ROCKET_E_SHAPE"] == "-1" and vals["ROCKET_E_TILING"] == "-2"
    assert vals["ROCKET_E_NOMEM"] == "-3" and vals["ROCKET_E_DEVICE"] == "-4" and vals["ROCKET_E_UNSUPPORTED"] == "-5"


PLANS = [
    # name, (K align, N align), extra args
    ("rocket_matmul_plan", 32, 16),
    ("rocket_matmul_plan_int8", 32, 32),
    ("rocket_matmul_plan_int4", 32, 64),
    ("rocket_matmul_plan_int16", 32, 16),
    ("rocket_matmul_plan_bf16", 32, 16),
    ("rocket_matmul_plan_tf32", 16, 16),
]


@pytest.mark.parametrize("name,kal,nal", PLANS)
def test_planner_alignment_and_positive_count(lib, name, kal, nal):
    n, mt, kt, nt = R.plan(name, 512, 4096, 4096)
    assert n > 0 and 0 < mt <= 512 and kt == 4096 and 0 < nt <= 4096
    assert n == ((512 + mt - 1) // mt) * ((4096 + nt - 1) // nt)      # one workgroup per tile
    assert R.plan(name, 512, 4096 + kal // 2, 4096)[0] == R.ROCKET_E_SHAPE    # K misaligned
    assert R.plan(name, 512, 4096, 4096 + nal // 2)[0] == R.ROCKET_E_SHAPE    # N misaligned
    for m in (1, 2, 3, 5, 6):                                                  # plans reject M%4 != 0
        assert R.plan(name, m, 4096, 4096)[0] == R.ROCKET_E_SHAPE
    assert R.plan(name, 0, 4096, 4096)[0] == R.ROCKET_E_SHAPE
    assert R.plan(name, 4, (1 << 24) + kal, 4096)[0] == R.ROCKET_E_SHAPE      # dimension cap
    assert R.plan(name, 4, kal, nal)[0] > 0                                   # the smallest legal shape


def test_groupwise_planner_pins_kt_to_group(lib):
    n, mt, kt, nt = R.plan("rocket_matmul_plan_int8_gw", 512, 2880, 512, 576)
    assert n > 0 and kt == 576
    for bad in (0, 16, 48, 100, 640):              # < 32, not %32, does not divide K
        assert R.plan("rocket_matmul_plan_int8_gw", 512, 2880, 512, bad)[0] == R.ROCKET_E_SHAPE
    assert R.plan("rocket_matmul_plan_int8_gw", 6, 2880, 512, 576)[0] == R.ROCKET_E_SHAPE


def test_rk3576_entries_are_unsupported_stubs(lib):
    assert R.plan("rocket_matmul_plan_int8_rk3576", 512, 1024, 1024)[0] == R.ROCKET_E_UNSUPPORTED
    assert lib.rocket_matmul_int8_rk3576(0, 4, 32, 32, None, None, None, 1.0, None) == R.ROCKET_E_UNSUPPORTED
    out = C.c_void_p(1234)
    assert lib.rocket_rk3576_wbo_create(0, 32, 32, None, C.byref(out)) == R.ROCKET_E_UNSUPPORTED
    assert out.value is None
    st = R.I32Stats(submits=7, refused=3)
    lib.rocket_rk3576_i32_last_stats(C.byref(st))
    assert st.submits == 0 and st.refused == 0


def test_shape_rejections_happen_before_the_device(lib):
    # an invalid handle would fail with ROCKET_E_DEVICE; a bad shape must be reported first
    bad = -1
    assert lib.rocket_matmul_fp16(bad, 5, 32, 16, None, None, None) == R.ROCKET_E_SHAPE
    assert lib.rocket_matmul_fp16(bad, 4, 48, 16, None, None, None) == R.ROCKET_E_SHAPE
    assert lib.rocket_matmul_int8(bad, 4, 32, 48, None, None, None) == R.ROCKET_E_SHAPE
    assert lib.rocket_matmul_int4(bad, 4, 32, 96, None, None, None) == R.ROCKET_E_SHAPE
    assert lib.rocket_matmul_int16_exact(bad, 4, 32, 16, None, None, None) == R.ROCKET_E_SHAPE
    assert lib.rocket_matmul_bf16(bad, 4, 16, 16, None, None, None) == R.ROCKET_E_SHAPE
    assert lib.rocket_matmul_tf32(bad, 4, 8, 16, None, None, None) == R.ROCKET_E_SHAPE
    # group-wise one-shot entries do not pad M==1 (rocket_matmul.c:2676, :3139)
    assert lib.rocket_matmul_int8_groupwise(bad, 1, 64, 32, None, None, None, None, None, 32) == R.ROCKET_E_SHAPE
    assert lib.rocket_matmul_int4_groupwise(bad, 1, 64, 64, None, None, None, None, None, 32) == R.ROCKET_E_SHAPE
    # int4 group-wise keeps the reference's 49*group < 32767 bound
    assert lib.rocket_matmul_int4_groupwise(bad, 4, 1344, 64, None, None, None, None, None, 672) == R.ROCKET_E_SHAPE
    # a legal shape on a closed handle is a device error, not a crash
    assert lib.rocket_matmul_int8(bad, 4, 32, 32, None, None, None) < 0


def test_resident_constructors_reject_bad_shapes_without_a_device(lib):
    assert lib.rocket_i8_weights_pack(None, 4, 32, 32, None) is None
    assert lib.rocket_matmul_int8_prepacked(None, 4, 32, 32, None, None, None) == R.ROCKET_E_SHAPE
    assert lib.rocket_matmul_int4_prepacked_gw(None, 4, 32, 64, None, None, None, None, None) == R.ROCKET_E_SHAPE
    assert lib.rocket_matmul_fp16_prepacked(None, 4, 32, 16, None, None, None) == R.ROCKET_E_SHAPE
    assert lib.rocket_i8_weights_bytes(None) == 0 and lib.rocket_i4_weights_bytes(None) == 0
    # the gated MoE down entry takes SILU or GELU and an up array, checked before anything else
    glu = lib.rocket_matmul_int8_prepacked_gw_grouped_glu_f32in
    M1, keep = R.int_array([4])
    one = (C.c_void_p * 1)(None)
    for act in (0, R.ROCKET_ACTIVATION_TANH, 99):
        assert glu(None, 1, M1, 32, 32, one, one, act, one, one, one) == R.ROCKET_E_SHAPE
    assert glu(None, 1, M1, 32, 32, one, None, R.ROCKET_ACTIVATION_SILU, one, one, one) == R.ROCKET_E_SHAPE
    assert glu(None, 1, M1, 32, 32, one, one, R.ROCKET_ACTIVATION_GELU, one, one, one) == R.ROCKET_E_SHAPE


def test_submit_entries_and_probes(lib):
    assert lib.rocket_batched_submit_supported() == 0
    assert lib.rocket_ppu_done_supported() == 0
    assert lib.rocket_batch_completion_tracked() == 0
    assert lib.rocket_bo_ranges_supported() == 1
    EBADF = 9
    assert lib.rocket_submit_tasks(77, None, 0, None, 0, None, 0) == -EBADF
    assert lib.rocket_submit_jobs(-3, None, 0) == -EBADF
    assert lib.rocket_submit_scratch_size(10) >= 10
    bo = R.RocketBO()
    assert lib.rocket_bo_alloc(-1, 4096, C.byref(bo)) < 0
    assert lib.rocket_bo_fini(-1, C.byref(bo)) < 0        # never allocated
    lib.rocket_submit_counters_reset()
    assert lib.rocket_submit_ioctl_count() == 0 and lib.rocket_submit_task_count() == 0


def test_affinity_hints(lib):
    lib.rocket_affinity_set_base(3)
    assert lib.rocket_affinity_get_base() == 3
    lib.rocket_affinity_set_base(0)
    lib.rocket_pin_worker(2)
    assert lib.rocket_num_big_cores() == 0


def test_log_channel_callback_and_level(lib):
    got = []
    cb = R.LOG_CB(lambda lvl, text, ud: got.append((lvl, text.decode())))
    lib.rocket_log_set_callback(cb, None)
    try:
        old = lib.rocket_log_get_level()
        lib.rocket_log_set_level(2)
        lib.rocket_log(0, b"error line\n")
        lib.rocket_log(3, b"debug line\n")           # above the threshold: dropped
        assert lib.rocket_matmul_int8(-1, 5, 32, 32, None, None, None) == R.ROCKET_E_SHAPE
        assert any("rocket_matmul_int8: unsupported shape" in t for _, t in got)
        assert not any("debug line" in t for _, t in got)
        lib.rocket_log_set_level(old)
    finally:
        lib.rocket_log_set_callback(R.LOG_CB(0), None)


def test_hw_profile(lib):
    p = lib.rocket_hw_current().contents
    assert p.name == b"mi355x"
    assert p.cbuf_banks * p.cbuf_bank_size == 160 * 1024        # LDS per CU
    assert p.dtype_supported & 0xFF == 0xFF
    assert lib.rocket_hw_by_name(b"rk3588").contents.name == b"rk3588"
    assert not lib.rocket_hw_by_name(b"nope")


def test_rocket_open_without_a_gpu_is_a_negative_errno(lib):
    # runs in the CPU container: no HIP device
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    assert lib.rocket_open() < 0


def test_ffn_host_references_equal_the_oracle(lib, orc):
    # fd < 0 selects the reference's own host path (rocket_ffn.c:33-38, :58-82, :236-254)
    M, H, I = 4, 64, 96
    a = 3.0 / np.sqrt(H)
    x = orc.f32_to_f16_bits(orc.gen_uniform((M, H), 71, -1, 1))
    Wg = orc.f32_to_f16_bits(orc.gen_uniform((I, H), 72, -a, a))
    Wu = orc.f32_to_f16_bits(orc.gen_uniform((I, H), 73, -a, a))
    Wd = orc.f32_to_f16_bits(orc.gen_uniform((H, I), 74, -0.15, 0.15))
    for kind in (R.ROCKET_ACTIVATION_SILU, R.ROCKET_ACTIVATION_GELU):
        want = orc.ffn_f16(x, Wg, Wu, Wd, kind)
        for f in (lib.rocket_ffn_fp16, lib.rocket_ffn_fp16_fused):
            out = np.empty((M, H), np.uint16)
            assert f(-1, M, H, I, R.ptr(x), R.ptr(Wg), R.ptr(Wu), R.ptr(Wd), kind, R.ptr(out)) == 0
            assert np.array_equal(out, want)
        out = np.empty((M, H), np.uint16)
        lib.rocket_ffn_ref_fp16(M, H, I, R.ptr(x), R.ptr(Wg), R.ptr(Wu), R.ptr(Wd), kind, R.ptr(out))
        assert np.array_equal(out, want)
        g, u = Wg[:2].ravel().copy(), Wu[:2].ravel().copy()
        p = np.empty_like(g)
        assert lib.rocket_geglu_fp16(-1, R.ptr(g), R.ptr(u), kind, R.ptr(p), g.size) == 0
        assert np.array_equal(p, orc.geglu_f16(g, u, kind))
        p2 = np.empty_like(g)
        lib.rocket_geglu_ref_fp16(R.ptr(g), R.ptr(u), kind, R.ptr(p2), g.size)
        assert np.array_equal(p2, p)
        W1, W2 = Wg, Wd
        b1 = orc.f32_to_f16_bits(orc.gen_uniform(I, 75, -1, 1))
        for bias in (None, b1):
            out = np.empty((M, H), np.uint16)
            assert lib.rocket_mlp_fp16_fused(-1, M, H, I, H, R.ptr(x), R.ptr(W1),
                                             None if bias is None else R.ptr(bias), R.ptr(W2), kind,
                                             R.ptr(out)) == 0
            assert np.array_equal(out, orc.mlp_f16(x, W1, bias, W2, kind))


def test_ffn_rejections_happen_before_the_device(lib):
    S, G = R.ROCKET_ACTIVATION_SILU, R.ROCKET_ACTIVATION_GELU
    closed = 77
    # the reference's own argument checks (rocket_ffn.c:42, :89-93, :272-273), any fd
    assert lib.rocket_geglu_fp16(closed, None, None, S, None, 0) == R.ROCKET_E_SHAPE
    assert lib.rocket_ffn_fp16(-1, 0, 32, 32, None, None, None, None, S, None) == R.ROCKET_E_SHAPE
    assert lib.rocket_ffn_fp16_fused(closed, 4, 32, 0, None, None, None, None, S, None) == R.ROCKET_E_SHAPE
    assert lib.rocket_ffn_fp16(closed, 65536, 32, 65536, None, None, None, None, S, None) == R.ROCKET_E_SHAPE
    assert lib.rocket_mlp_fp16_fused(closed, 4, 32, 32, 0, None, None, None, None, S, None) == R.ROCKET_E_SHAPE
    buf = np.zeros(4 * 4096, np.uint16)
    p = R.ptr(buf)
    # GPU-path limits: SiLU/GELU only; H, I multiples of 32; M a multiple of 4 or 1
    assert lib.rocket_ffn_fp16(closed, 4, 32, 32, p, p, p, p, 1, p) == R.ROCKET_E_SHAPE
    assert lib.rocket_ffn_fp16(closed, 4, 48, 32, p, p, p, p, S, p) == R.ROCKET_E_SHAPE
    assert lib.rocket_ffn_fp16(closed, 6, 32, 32, p, p, p, p, G, p) == R.ROCKET_E_SHAPE
    assert lib.rocket_mlp_fp16_fused(closed, 4, 32, 32, 24, p, p, None, p, S, p) == R.ROCKET_E_SHAPE
    assert lib.rocket_geglu_fp16(closed, p, p, 0, p, 64) == R.ROCKET_E_SHAPE
    # a legal call on a closed handle is a device error
    assert lib.rocket_ffn_fp16(closed, 4, 32, 32, p, p, p, p, S, p) == R.ROCKET_E_DEVICE
    assert lib.rocket_geglu_fp16(closed, p, p, G, p, 64) == R.ROCKET_E_DEVICE


# ---- serialised resident weights (rocket_weights_io.h) -----------------------------

def _fixtures():
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "make_weights_fixture", os.path.join(os.path.dirname(__file__), "golden", "make_weights_fixture.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def test_xxh64_matches_the_xxhash_package(lib):
    import xxhash
    # the specification's empty-input value, then every tail length and a few long inputs
    assert lib.rocket_weights_xxh64(None, 0) == 0xEF46DB3751D8E999
    rng = np.random.default_rng(5)
    data = rng.integers(0, 256, 5000, dtype=np.uint8).tobytes()
    buf = C.create_string_buffer(data, len(data))
    for n in list(range(0, 131)) + [255, 256, 1000, 4093, 5000]:
        assert lib.rocket_weights_xxh64(buf, n) == xxhash.xxh64(data[:n], seed=0).intdigest(), n


def test_weights_fixtures_are_stable_and_read_back(lib):
    fx = _fixtures()
    here = os.path.join(os.path.dirname(__file__), "golden")
    B4, sc, blob4 = fx.int4_fixture()
    B8, blob8 = fx.int8_fixture()
    assert open(os.path.join(here, "weights_int4_g32.rktw"), "rb").read() == blob4
    assert open(os.path.join(here, "weights_int8_pc.rktw"), "rb").read() == blob8
    info = R.WeightsInfo()
    buf = C.create_string_buffer(blob4, len(blob4))
    assert lib.rocket_weights_info_read(buf, len(blob4), C.byref(info)) == 0
    assert (info.kind, info.flags, info.N, info.K, info.group, info.M) == (2, 1, 64, 128, 32, 4)
    assert info.code_bytes == 64 * 64 and info.scale_bytes == 64 * 4 * 4
    buf8 = C.create_string_buffer(blob8, len(blob8))
    assert lib.rocket_weights_info_read(buf8, len(blob8), C.byref(info)) == 0
    assert (info.kind, info.flags, info.N, info.K, info.group, info.M) == (1, 0, 32, 64, 0, 8)
    # the int4 codes are the documented nibble layout of the fixture's values
    assert blob4[64:64 + 4] == bytes([((int(B4[0, j]) & 15) << 4) | (int(B4[0, 4 + j]) & 15) for j in range(4)])


def test_weights_reader_rejects_malformed(lib):
    fx = _fixtures()
    blob = bytearray(fx.int4_fixture()[2])
    info = R.WeightsInfo()

    def ok(b):
        return lib.rocket_weights_info_read(C.create_string_buffer(bytes(b), len(b)), len(b), C.byref(info)) == 0

    assert ok(blob)
    assert not ok(blob[:-1])                       # truncated payload
    assert not ok(blob[:63])                       # truncated header
    assert lib.rocket_weights_info_read(None, 0, C.byref(info)) == R.ROCKET_E_SHAPE
    for pos in (0, 4, 8, 16, 24, 33, 44, 50, 60, 64, 64 + 4096, len(blob) - 1):
        bad = bytearray(blob)
        bad[pos] ^= 0x01                           # any flipped bit: a checksum or a field check fails
        assert not ok(bad), pos
    # a consistent header (checksums recomputed) that describes a bad shape is refused too
    B, sc, _ = fx.int4_fixture()
    assert not ok(fx.serialise(2, 64, 128, 48, 4, fx.pack_int4(B), sc))      # group does not divide K
    assert not ok(fx.serialise(3, 64, 128, 32, 4, fx.pack_int4(B), sc))      # unknown kind
    assert not ok(fx.serialise(2, 64, 128, 32, 4, fx.pack_int4(B)[:-1], sc))  # codes of the wrong size
    assert not ok(fx.serialise(2, 64, 128, 0, 4, fx.pack_int4(B), sc))       # scales without groups


def test_attention_host_references_equal_the_oracle(lib, orc):
    # fd < 0 selects the reference's fp64 host paths (rocket_attn.c:41-84, :189-228)
    rng = np.random.default_rng(17)
    h = lambda a: np.asarray(a, np.float32).astype(np.float16).view(np.uint16)
    nh, nkvh, T, n_kv, dk, dv = 4, 2, 5, 37, 64, 32
    Q = h(rng.uniform(-1, 1, (nh, T, dk)))
    K = h(rng.uniform(-1, 1, (nkvh, n_kv, dk)))
    V = h(rng.uniform(-1, 1, (nkvh, dv, n_kv)))
    mask = h(np.where(rng.random((T, n_kv)) < 0.3, -np.inf, 0.0))
    for m, cap in ((mask, 0.0), (None, 20.0)):
        want = orc.flash_attn_f16(Q, K, V, m, 0.125, cap)
        out = np.empty_like(want)
        assert lib.rocket_flash_attn_fp16(-1, T, n_kv, dk, dv, nh, nkvh, 0.125, cap, R.ptr(Q), R.ptr(K), R.ptr(V),
                                          None if m is None else R.ptr(m), R.ptr(out)) == 0
        assert np.array_equal(out, want)
        out2 = np.empty_like(want)
        lib.rocket_flash_attn_ref_fp16(T, n_kv, dk, dv, nh, nkvh, 0.125, cap, R.ptr(Q), R.ptr(K), R.ptr(V),
                                       None if m is None else R.ptr(m), R.ptr(out2))
        assert np.array_equal(out2, want)
    T, d, n_head = 6, 64, 2
    x = h(rng.uniform(-1, 1, (T, d)))
    W = [h(rng.uniform(-0.1, 0.1, (d, d))) for _ in range(4)]
    b = [h(rng.uniform(-0.1, 0.1, d)) for _ in range(4)]
    want = orc.mha_self_f16(x, W[0], b[0], W[1], None, W[2], b[2], W[3], b[3], n_head)
    out = np.empty_like(want)
    assert lib.rocket_mha_self_fp16(-1, T, d, n_head, R.ptr(x), R.ptr(W[0]), R.ptr(b[0]), R.ptr(W[1]), None,
                                    R.ptr(W[2]), R.ptr(b[2]), R.ptr(W[3]), R.ptr(b[3]), R.ptr(out)) == 0
    assert np.array_equal(out, want)
    out2 = np.empty_like(want)
    lib.rocket_mha_self_ref_fp16(T, d, n_head, R.ptr(x), R.ptr(W[0]), R.ptr(b[0]), R.ptr(W[1]), None,
                                 R.ptr(W[2]), R.ptr(b[2]), R.ptr(W[3]), R.ptr(b[3]), R.ptr(out2))
    assert np.array_equal(out2, want)


def test_attention_rejections(lib):
    S = R.ROCKET_E_SHAPE
    # the reference's checks (rocket_attn.c:98, :733-734), before any device use
    assert lib.rocket_flash_attn_fp16(77, 4, 4, 48, 16, 2, 2, 1.0, 0.0, None, None, None, None, None) == S
    assert lib.rocket_flash_attn_fp16(77, 4, 4, 64, 24, 2, 2, 1.0, 0.0, None, None, None, None, None) == S
    assert lib.rocket_flash_attn_fp16(77, 4, 4, 64, 16, 3, 2, 1.0, 0.0, None, None, None, None, None) == S
    assert lib.rocket_flash_attn_fp16_mt(77, 0, 4, 64, 16, 2, 2, 1.0, 0.0, None, None, None, None, None, 4) == S
    assert lib.rocket_flash_attn_fp16_ctx(None, 4, 4, 64, 16, 2, 2, 1.0, 0.0, None, None, None, None, None) == S
    assert lib.rocket_mha_self_fp16(77, 4, 60, 8, *([None] * 10)) == S
    # GPU limits: head dims above 256
    buf = np.zeros(8, np.uint16)
    p = R.ptr(buf)
    assert lib.rocket_flash_attn_fp16(77, 4, 4, 288, 16, 2, 2, 1.0, 0.0, p, p, p, None, p) == S
    assert lib.rocket_flash_attn_fp16(77, 4, 4, 64, 16, 2, 2, 1.0, 0.0, p, p, p, None, p) == R.ROCKET_E_DEVICE
    fd = lib.rocket_open()
    if fd < 0:
        assert lib.rocket_fa_ctx_create(2) is None     # no device: no context (reference: NULL)
    else:
        lib.rocket_close(fd)
