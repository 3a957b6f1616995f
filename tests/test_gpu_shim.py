"""The HIP device shim behind rocket_npu.h on a real MI355X: buffer objects on an open
handle, the bounded wait (ROCKET_WAIT_MS, reference src/rocket_matmul.c:53-69 and
src/rocket_npu.c:612-739), the per-phase profile (ROCKET_MM_PROFILE, rocket_matmul.c:71-125)
and handle lifetime under threads (the reference's uapi / prep robustness tests,
tests/uapi_selftest_rocket.c, tests/prep_signal_robust_rocket.c)."""
import ctypes as C
import errno
import json
import os
import subprocess
import sys
import threading
import time

import numpy as np
import pytest

import rocketnpu as R

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def child(mode, **env):
    e = dict(os.environ, **env)
    p = subprocess.run([sys.executable, os.path.join(HERE, "shim_child.py"), mode], env=e, capture_output=True,
                       text=True, timeout=240)
    assert p.returncode == 0, p.stderr[-2000:]
    return json.loads(p.stdout.strip().splitlines()[-1]), p.stderr


def test_bo_alloc_prep_fini_on_a_gpu_handle(lib, orc):
    import torch
    fd = lib.rocket_open()
    assert fd >= 0
    bo = R.RocketBO()
    assert lib.rocket_bo_alloc(fd, 100000, C.byref(bo)) == 0
    assert bo.ptr and bo.dma_address and bo.size >= 100000 and bo.size % 4096 == 0
    # the CPU mapping is writable and the device view feeds a product
    M, K, N = 64, 256, 128
    A = orc.gen_i8((M, K), 0x52434E30)
    B = orc.gen_i8((N, K), 0x52434E31)
    view = np.ctypeslib.as_array((C.c_int8 * (M * K)).from_address(bo.ptr))
    view[:] = A.ravel()
    Cg = np.zeros((M, N), np.int32)
    assert lib.rocket_matmul_int8(fd, M, K, N, C.c_void_p(bo.dma_address), R.ptr(B), R.ptr(Cg)) == 0
    assert np.array_equal(Cg, orc.matmul_int8(A, B))
    # a zero timeout polls: busy while queued work runs, then complete
    dev = torch.device("cuda:0")
    X = torch.randint(-128, 127, (8192, 8192), dtype=torch.int8, device=dev)
    Y = torch.empty((8192, 8192), dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    assert lib.rocket_hip_set_mode(fd, R.ROCKET_HIP_ASYNC | R.ROCKET_HIP_DEVICE_OPERANDS) == 0
    for _ in range(8):
        assert lib.rocket_matmul_int8(fd, 8192, 8192, 8192, R.ptr(X), R.ptr(X), R.ptr(Y)) == 0
    assert lib.rocket_bo_prep(fd, C.byref(bo), 0, 0) == -errno.EBUSY
    assert lib.rocket_bo_prep(fd, C.byref(bo), 0, 2 ** 64 - 1) == 0    # saturated, waits
    assert lib.rocket_bo_prep(fd, C.byref(bo), 0, 0) == 0
    assert lib.rocket_bo_fini(fd, C.byref(bo)) == 0
    assert lib.rocket_hip_set_mode(fd, 0) == 0
    # ranges: ascending, disjoint, inside the object
    good = (R.RocketBORange * 2)(R.RocketBORange(0, 4096), R.RocketBORange(8192, 4096))
    bad = (R.RocketBORange * 2)(R.RocketBORange(8192, 4096), R.RocketBORange(0, 4096))
    past = (R.RocketBORange * 1)(R.RocketBORange(bo.size - 4096, 8192))
    assert lib.rocket_bo_prep_ranges(fd, C.byref(bo), good, 2, 10 ** 9) == 0
    assert lib.rocket_bo_fini_ranges(fd, C.byref(bo), good, 2) == 0
    assert lib.rocket_bo_prep_ranges(fd, C.byref(bo), bad, 2, 10 ** 9) == -errno.EINVAL
    assert lib.rocket_bo_fini_ranges(fd, C.byref(bo), past, 1) == -errno.EINVAL
    lib.rocket_bo_free(fd, C.byref(bo))
    assert not bo.ptr and bo.size == 0
    assert lib.rocket_bo_prep(fd, C.byref(bo), 0, 0) == -errno.EINVAL
    lib.rocket_close(fd)
    bo2 = R.RocketBO()
    assert lib.rocket_bo_alloc(fd, 4096, C.byref(bo2)) == -errno.EBADF     # closed handle


def test_wait_deadline_gives_up_then_drains():
    """ROCKET_WAIT_MS=1: the call whose queued work outlasts the deadline returns
    ROCKET_E_DEVICE while its kernels complete; the next call on the handle drains that
    work first and computes a correct result."""
    out, err = child("wait", ROCKET_WAIT_MS="1")
    assert out["fd"] >= 0
    assert out["long_rc"] == R.ROCKET_E_DEVICE, out
    assert "WAIT TIMEOUT" in err
    rc, ok = out["next"][-1]
    assert rc == 0 and ok, out


def test_mm_profile_summary():
    """ROCKET_MM_PROFILE=1: one INFO line at exit with the phase totals over every call."""
    out, err = child("profile", ROCKET_MM_PROFILE="1")
    assert all(rc == 0 and ok for rc, ok in out["calls"])
    lines = [l for l in err.splitlines() if l.startswith("ROCKET profile total(ms):")]
    assert len(lines) == 1, err[-2000:]
    fields = dict(kv.split("=") for kv in lines[0].split(":", 1)[1].split() if "=" in kv)
    assert lines[0].rstrip().endswith("over 3 calls")
    assert all(float(fields[k]) >= 0 for k in ("stage", "submit", "wait", "read"))
    assert float(fields["stage"]) > 0 and float(fields["wait"]) > 0
    out, err = child("profile")
    assert "ROCKET profile" not in err          # off unless asked for


def test_handles_across_threads(lib, orc):
    """Threads opening, using and closing handles at once (the _mt entries open and close
    one per call), and a close racing calls on the same handle: every call returns 0 with a
    correct result, or ROCKET_E_DEVICE once the handle is closed; nothing faults."""
    M, K, N = 64, 256, 128
    A = orc.gen_i8((M, K), 0x52434E40)
    B = orc.gen_i8((N, K), 0x52434E41)
    want = orc.matmul_int8(A, B)
    A16 = orc.f32_to_f16_bits(orc.gen_uniform((M, K), 0x52434E42))
    B16 = orc.f32_to_f16_bits(orc.gen_uniform((N, K), 0x52434E43))
    want16 = np.empty((M, N), np.uint16)
    fd0 = lib.rocket_open()
    assert lib.rocket_matmul_fp16(fd0, M, K, N, R.ptr(A16), R.ptr(B16), R.ptr(want16)) == 0
    errors = []

    def worker(i):
        try:
            for _ in range(15):
                fd = lib.rocket_open()
                assert fd >= 0
                Cg = np.zeros((M, N), np.int32)
                assert lib.rocket_matmul_int8(fd, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg)) == 0
                assert np.array_equal(Cg, want)
                lib.rocket_close(fd)
                C16 = np.zeros((M, N), np.uint16)
                assert lib.rocket_matmul_fp16_mt(M, K, N, R.ptr(A16), R.ptr(B16), R.ptr(C16), 2) == 0
                assert np.array_equal(C16, want16)
        except AssertionError as e:   # reported by the main thread
            errors.append((i, repr(e)))

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors

    rcs = []

    def caller():
        for _ in range(200):
            Cg = np.zeros((M, N), np.int32)
            rc = lib.rocket_matmul_int8(fd0, M, K, N, R.ptr(A), R.ptr(B), R.ptr(Cg))
            rcs.append((rc, rc == 0 and bool(np.array_equal(Cg, want))))

    t = threading.Thread(target=caller)
    t.start()
    while len(rcs) < 20:
        time.sleep(0.0005)
    lib.rocket_close(fd0)
    t.join()
    assert all(rc in (0, R.ROCKET_E_DEVICE) for rc, _ in rcs)
    assert all(ok for rc, ok in rcs if rc == 0)
    assert rcs[-1][0] == R.ROCKET_E_DEVICE and rcs[0][0] == 0


def test_handle_getters_stream_binding_and_weight_views(lib, orc):
    """The rocket_hip.h getters: each context's handle, the handle's stream (a bound caller
    stream, then its own again), the bounded sync (and ROCKET_E_DEVICE for a bad handle),
    and the device views of resident weights in their documented layouts (int8 rows [N, K];
    int4: byte j of packed word d holds k = 8d + j high and k = 8d + 4 + j low)."""
    import torch
    hip = C.CDLL("libamdhip64.so.7")   # the runtime librocketnpu itself loaded
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    hip.hipMemcpy.restype = C.c_int
    for make, free, fdof in ((lib.rocket_ctx_create, lib.rocket_ctx_free, lib.rocket_ctx_fd),
                             (lib.rocket_stream_create, lib.rocket_stream_free, lib.rocket_stream_fd),
                             (lib.rocket_bf16_stream_create, lib.rocket_bf16_stream_free, lib.rocket_bf16_stream_fd)):
        obj = make(1)
        assert obj
        fd = fdof(obj)
        assert fd >= 0 and lib.rocket_hip_stream(fd)
        assert lib.rocket_hip_sync(fd) == 0
        free(obj)
    assert lib.rocket_hip_sync(-1) == R.ROCKET_E_DEVICE
    lib.rocket_busy_poll_set_us(50)
    lib.rocket_busy_poll_set_us(0)

    N, K = 64, 256
    B8 = orc.gen_i8((N, K), 0x52434E40)
    B4 = (orc.gen_i8((N, K), 0x52434E41) % 16 - 8).astype(np.int8)
    c8, c4 = lib.rocket_i8_ctx_create(1), lib.rocket_i4_ctx_create(1)
    fd8 = lib.rocket_i8_ctx_fd(c8)
    assert fd8 >= 0 and lib.rocket_i4_ctx_fd(c4) >= 0
    own = lib.rocket_hip_stream(fd8)
    st = torch.cuda.Stream()
    assert lib.rocket_hip_set_stream(fd8, C.c_void_p(st.cuda_stream)) == 0
    assert lib.rocket_hip_stream(fd8) == st.cuda_stream
    assert lib.rocket_hip_set_stream(fd8, None) == 0
    assert lib.rocket_hip_stream(fd8) == own
    w8 = lib.rocket_i8_weights_pack(c8, 4, K, N, R.ptr(B8))
    w4 = lib.rocket_i4_weights_pack(c4, 4, K, N, R.ptr(B4))
    assert w8 and w4
    got8 = np.empty((N, K), np.int8)
    got4 = np.empty((N, K // 2), np.uint8)
    assert hip.hipMemcpy(got8.ctypes.data, lib.rocket_i8_weights_device(w8), got8.nbytes, 2) == 0
    assert hip.hipMemcpy(got4.ctypes.data, lib.rocket_i4_weights_device(w4), got4.nbytes, 2) == 0
    assert np.array_equal(got8, B8)
    nib = (B4.astype(np.int32) & 15).reshape(N, K // 8, 2, 4)   # [n][word d][half][byte j]
    want4 = ((nib[:, :, 0, :] << 4) | nib[:, :, 1, :]).astype(np.uint8).reshape(N, K // 2)
    assert np.array_equal(got4, want4)
    lib.rocket_i8_weights_free(c8, w8)
    lib.rocket_i4_weights_free(c4, w4)
    lib.rocket_i8_ctx_free(c8)
    lib.rocket_i4_ctx_free(c4)
