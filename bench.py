#!/usr/bin/env python3
"""Throughput of librocketnpu's MI355X matmul path on the BASELINE.json configurations.

A "step" is one call of the matmul entry on inputs already resident in HBM (torch device
tensors, used in place by the library), queued on torch's current stream with the handle
in async mode. W warm-up steps, then K timed steps bracketed by a device synchronisation;
HIP events on that same stream give the average time per step, which is the kernel's
launch duration when the steps run back to back.

Default workload: configs[2], the Gemma-12B prefill GEMM the metric is quoted on (W4A8
group-wise, M=512 K=3840 N=15360, resident int4 weights, per-row activation scales).
--config picks another; --all measures every config and adds a "per_config" summary to the
one JSON line.
The CPU baseline times the repository's C oracle (oracle/, OpenMP) on a bounded row
sample of the same workload on this host.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for sub in ("rocket-userspace_amd", "oracle"):
    sys.path.insert(0, os.path.join(REPO, sub))

import numpy as np  # noqa: E402

# TOPS / TFLOPS; GB/s for HBM and for the host link (PCIe 5.0 x16, one direction)
PEAK = {"int8": 5000.0, "fp16": 2500.0, "bf16": 2500.0, "fp32": 157.3, "hbm": 8000.0, "pcie": 64.0}


CONFIGS = ["fp16", "int8", "int16", "int4gw", "int4gw_ref", "int8gemma", "bf16", "tf32", "moe", "moe_fwd", "moe_ref", "ffn",
           "int4gw_f32in", "weights_load", "attn"]


def traffic(config):
    """HBM bytes per launch of the config's dominant kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE measurement (profiles/traffic.json, each counter scaled by what it
    reads for a plain 256 MiB copy), or None when none is recorded."""
    try:
        with open(os.path.join(REPO, "profiles", "traffic.json")) as f:
            t = json.load(f)[config]
        return int(t["fetch_bytes"] + t["write_bytes"])
    except (OSError, KeyError, ValueError):
        return None


def cpu_host():
    """The host CPUs the baseline may use: the CPUs this process is allowed to run on
    (sched_getaffinity), capped by OMP_NUM_THREADS when the environment sets it (the GPU box
    sets it to its CPU share per GPU), with the machine's CPU count and model for the record."""
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = os.cpu_count() or 1
    try:
        omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    except ValueError:
        omp = 0
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    threads = max(1, min(aff, omp) if omp > 0 else aff)
    return dict(threads=threads, nproc=os.cpu_count(), affinity_cpus=aff, omp_num_threads=omp or None,
                cpu_model=model)


def cpu_threads():
    return cpu_host()["threads"]


# The vendor library's own product at a config's shape (hipBLASLt through torch), timed beside
# ours as a reference point for what this GPU sustains there. Group-wise configs get the plain
# int8 x int8 -> int32 product of the same shape (the library has no W4A8 group-wise GEMM).
VENDOR_SHAPES = {"int8": (512, 4096, 4096, "int8"), "int4gw": (512, 3840, 15360, "int8"),
                 "int4gw_ref": (512, 3840, 15360, "int8"), "int8gemma": (512, 3840, 15360, "int8"),
                 "bf16": (2048, 15360, 3840, "bf16"), "fp16": (64, 256, 128, "fp16")}


def vendor_baseline(config, reps=20):
    import torch
    if config not in VENDOR_SHAPES:
        return None
    M, K, N, kind = VENDOR_SHAPES[config]
    try:
        if kind == "int8":
            a = torch.randint(-128, 128, (M, K), dtype=torch.int8, device="cuda")
            w = torch.randint(-128, 128, (N, K), dtype=torch.int8, device="cuda")
            fn = lambda: torch._int_mm(a, w.t())   # B as [N, K] rows, like ours
            lib = "hipBLASLt (torch._int_mm), int8 x int8 -> int32"
        else:
            dt = torch.bfloat16 if kind == "bf16" else torch.float16
            a = torch.randn(M, K, dtype=dt, device="cuda")
            w = torch.randn(N, K, dtype=dt, device="cuda")
            fn = lambda: a @ w.t()
            lib = f"hipBLASLt (torch.matmul), {kind} -> {kind}"
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
    except Exception as ex:   # the library path is a reference only
        return {"lib": "unavailable", "error": str(ex)[:120]}
    return {"lib": lib, "shape_mkn": [M, K, N], "us": round(us, 2),
            "value": round(2.0 * M * N * K / (us * 1e-6) / 1e12, 3), "unit": "TOPS" if kind == "int8" else "TFLOP/s"}


class Bench:
    def __init__(self, steps, warmup):
        import torch
        import rocketnpu as R
        import oracle
        self.torch, self.R, self.orc = torch, R, oracle
        self.lib = R.load()
        self.steps, self.warmup = steps, warmup
        self.flush_buf = None
        self.per_step = {}
        self.cur = None
        self.dev = torch.device("cuda:0")
        # a real stream (torch's default is the legacy null stream, which cannot be bound)
        self.stream = torch.cuda.Stream()
        torch.cuda.set_stream(self.stream)

    def bind(self, fd):
        lib = self.lib
        assert lib.rocket_hip_set_stream(fd, C.c_void_p(self.stream.cuda_stream)) == 0
        assert lib.rocket_hip_set_mode(fd, self.R.ROCKET_HIP_ASYNC | self.R.ROCKET_HIP_DEVICE_OPERANDS) == 0

    def up(self, a):
        return self.torch.from_numpy(np.ascontiguousarray(a)).to(self.dev)

    def time_steps(self, step):
        import gc
        torch = self.torch
        for _ in range(self.warmup):
            rc = step()
            assert rc == 0, rc
        torch.cuda.synchronize()
        # no collector pass inside the timed region: a full pass over torch's object graph
        # takes milliseconds and stalls the host while the GPU queue drains
        gc.collect()
        gc.disable()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(self.stream)
        for _ in range(self.steps):
            rc = step()
            assert rc == 0, rc
        e1.record(self.stream)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / self.steps * 1e3
        ms = e0.elapsed_time(e1) / self.steps
        # per-step kernel times, median of 20: inputs warm in L2/MALL (as in the timed loop),
        # and with a 512 MiB write before each step that evicts them (HBM-cold). Either way
        # the GPU is kept busy (a spin, or the eviction write) while the host queues the
        # step, so no launch latency falls between the events.
        if self.flush_buf is None:
            self.flush_buf = torch.empty(128 << 20, dtype=torch.float32, device=self.dev)
        per = {"warm": [], "cold": []}
        for kind in ("warm", "cold"):
            for _ in range(20):
                if kind == "cold":
                    self.flush_buf.zero_()
                else:
                    torch.cuda._sleep(200000)
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record(self.stream)
                rc = step()
                assert rc == 0, rc
                b.record(self.stream)
                b.synchronize()
                per[kind].append(a.elapsed_time(b))
        gc.enable()
        self.per_step[self.cur] = {k: float(np.median(v)) for k, v in per.items()}
        return ms, wall

    # ---- configurations --------------------------------------------------------------
    def cfg_fp16(self):
        o, R, lib = self.orc, self.R, self.lib
        M, K, N = 64, 256, 128
        A = o.f32_to_f16_bits(o.gen_uniform((M, K), 0x52434B01))
        B = o.f32_to_f16_bits(o.gen_uniform((N, K), 0x52434B02))
        dA, dB = self.up(A), self.up(B)
        dC = self.torch.empty((M, N), dtype=self.torch.float16, device=self.dev)
        fd = lib.rocket_open()
        self.bind(fd)
        ms, wall = self.time_steps(lambda: lib.rocket_matmul_fp16(fd, M, K, N, R.ptr(dA), R.ptr(dB), R.ptr(dC)))
        ops = 2.0 * M * N * K
        nbytes = 2 * (M * K + N * K + M * N)
        return dict(workload="fp16 matmul 64x256x128 (configs[0])", ops=ops, nbytes=nbytes, ms=ms, wall=wall,
                    dtype="fp16", peak=PEAK["hbm"], bound="hbm", fd=fd,
                    cpu=lambda: self.cpu_rows(lambda m: o.matmul_fp16(A[:m].copy(), B), M, ops))

    def cfg_int8(self):
        o, R, lib = self.orc, self.R, self.lib
        M, K, N = 512, 4096, 4096
        A = o.gen_i8((M, K), 0x52434B02)
        B = o.gen_i8((N, K), 0x52434B03)
        dA, dB = self.up(A), self.up(B)
        dC = self.torch.empty((M, N), dtype=self.torch.int32, device=self.dev)
        fd = lib.rocket_open()
        self.bind(fd)
        ms, wall = self.time_steps(lambda: lib.rocket_matmul_int8(fd, M, K, N, R.ptr(dA), R.ptr(dB), R.ptr(dC)))
        ops = 2.0 * M * N * K
        return dict(workload="int8 matmul 512x4096x4096 -> int32 (configs[1])", ops=ops,
                    nbytes=M * K + N * K + 4 * M * N, ms=ms, wall=wall, dtype="int8", peak=PEAK["int8"],
                    bound="mfma", fd=fd,
                    cpu=lambda: self.cpu_rows(lambda m: o.matmul_int8(A[:m].copy(), B), M, ops))

    def cfg_int16(self):
        o, R, lib = self.orc, self.R, self.lib
        M, K, N = 512, 4096, 4096
        A = o.gen_i16((M, K), 0x52434B12, -32768, 32639)
        B = o.gen_i16((N, K), 0x52434B13, -32768, 32639)
        dA, dB = self.up(A), self.up(B)
        dC = self.torch.empty((M, N), dtype=self.torch.int64, device=self.dev)
        fd = lib.rocket_open()
        self.bind(fd)
        ms, wall = self.time_steps(lambda: lib.rocket_matmul_int16_exact(fd, M, K, N, R.ptr(dA), R.ptr(dB), R.ptr(dC)))
        ops = 4 * 2.0 * M * N * K          # int8-equivalent MFMA work
        return dict(workload="int16_exact 512x4096x4096 -> int64 (configs[1], int8-equivalent ops)", ops=ops,
                    nbytes=2 * (M * K + N * K) + 8 * M * N, ms=ms, wall=wall, dtype="int16", peak=PEAK["int8"],
                    bound="mfma", fd=fd,
                    cpu=lambda: self.cpu_rows(lambda m: o.matmul_int16_exact(A[:m].copy(), B), M, ops))

    def cfg_int4gw(self):
        o, R, lib = self.orc, self.R, self.lib
        M, K, N, group = 512, 3840, 15360, 128
        nG = K // group
        x = o.gen_normal((M, K), 0x52434B03)
        A = np.clip(np.round(x * 32), -128, 127).astype(np.int8)
        row_scale = (np.abs(x).max(axis=1) / 127).astype(np.float32)
        B = o.gen_i8((N, K), 0x52434B04, -8, 7)
        bsc = o.f16_bits_to_f32(o.f32_to_f16_bits(o.gen_uniform((N, nG), 0x52434B05, 0.005, 0.02)))
        ctx = lib.rocket_i4_ctx_create(1)
        w = lib.rocket_i4_weights_pack_gw(ctx, M, K, N, R.ptr(B), group)
        assert w
        fd = lib.rocket_i4_ctx_fd(ctx)
        dA, dar, dbs = self.up(A), self.up(row_scale), self.up(bsc)
        dC = self.torch.empty((M, N), dtype=self.torch.float32, device=self.dev)
        self.bind(fd)
        ms, wall = self.time_steps(lambda: lib.rocket_matmul_int4_prepacked_gw_rowscale(
            ctx, M, K, N, R.ptr(dA), R.ptr(dar), R.ptr(dbs), R.ptr(dC), w))
        ops = 2.0 * M * N * K
        nbytes = M * K + 4 * M + N * K // 2 + 4 * N * nG + 4 * M * N
        return dict(workload="W4A8 group-wise (g=128) resident int4 512x3840x15360, per-row activation scale "
                             "(configs[2], Gemma-12B FFN up-projection)", ops=ops,
                    nbytes=nbytes, ms=ms, wall=wall, dtype="int8", peak=PEAK["int8"], bound="mfma", fd=fd,
                    cpu=lambda: self.cpu_rows(lambda m: o.matmul_gw_rowscale_f32(A[:m].copy(), B, row_scale[:m].copy(),
                                                                                 bsc, group), M, ops))

    def cfg_int4gw_ref(self):
        """Config 3 through the reference's own resident entry, rocket_matmul_int4_prepacked_gw
        (reference include/rocket_matmul.h:739-775, what ggml-rocket calls): activation scales
        a_scale[M * nG], each row's scale repeated over its groups (so every tile folds in the
        row-scale order)."""
        o, R, lib = self.orc, self.R, self.lib
        M, K, N, group = 512, 3840, 15360, 128
        nG = K // group
        x = o.gen_normal((M, K), 0x52434B03)
        A = np.clip(np.round(x * 32), -128, 127).astype(np.int8)
        row_scale = (np.abs(x).max(axis=1) / 127).astype(np.float32)
        asc = np.ascontiguousarray(np.repeat(row_scale[:, None], nG, axis=1))
        B = o.gen_i8((N, K), 0x52434B04, -8, 7)
        bsc = o.f16_bits_to_f32(o.f32_to_f16_bits(o.gen_uniform((N, nG), 0x52434B05, 0.005, 0.02)))
        ctx = lib.rocket_i4_ctx_create(1)
        w = lib.rocket_i4_weights_pack_gw(ctx, M, K, N, R.ptr(B), group)
        assert w
        fd = lib.rocket_i4_ctx_fd(ctx)
        dA, das, dbs = self.up(A), self.up(asc), self.up(bsc)
        dC = self.torch.empty((M, N), dtype=self.torch.float32, device=self.dev)
        self.bind(fd)
        ms, wall = self.time_steps(lambda: lib.rocket_matmul_int4_prepacked_gw(
            ctx, M, K, N, R.ptr(dA), R.ptr(das), R.ptr(dbs), R.ptr(dC), w))
        ops = 2.0 * M * N * K
        nbytes = M * K + 4 * M * nG + N * K // 2 + 4 * N * nG + 4 * M * N
        return dict(workload="W4A8 group-wise (g=128) resident int4 512x3840x15360 through the reference entry "
                             "rocket_matmul_int4_prepacked_gw, per-group activation scales (configs[2])", ops=ops,
                    nbytes=nbytes, ms=ms, wall=wall, dtype="int8", peak=PEAK["int8"], bound="mfma", fd=fd,
                    cpu=lambda: self.cpu_rows(lambda m: o.matmul_gw_f32(A[:m].copy(), B, asc[:m].copy(), bsc, group),
                                              M, ops))

    def cfg_int4gw_f32in(self):
        o, R, lib = self.orc, self.R, self.lib
        M, K, N, group = 512, 3840, 15360, 128
        nG = K // group
        x = o.gen_normal((M, K), 0x52434B03)
        B = o.gen_i8((N, K), 0x52434B04, -8, 7)
        bsc = o.f16_bits_to_f32(o.f32_to_f16_bits(o.gen_uniform((N, nG), 0x52434B05, 0.005, 0.02)))
        ctx = lib.rocket_i4_ctx_create(1)
        w = lib.rocket_i4_weights_pack_gw(ctx, M, K, N, R.ptr(B), group)
        assert w
        fd = lib.rocket_i4_ctx_fd(ctx)
        dx, dbs = self.up(x), self.up(bsc)
        dC = self.torch.empty((M, N), dtype=self.torch.float32, device=self.dev)
        self.bind(fd)
        ms, wall = self.time_steps(lambda: lib.rocket_matmul_int4_prepacked_gw_f32in(
            ctx, M, K, N, R.ptr(dx), R.ptr(dbs), R.ptr(dC), w))
        ops = 2.0 * M * N * K
        nbytes = 4 * M * K + N * K // 2 + 4 * N * nG + 4 * M * N
        def cpu(m):
            q, rs = o.quant_rows(x[:m].copy())
            return o.matmul_gw_rowscale_f32(q, B, rs, bsc, group)
        return dict(workload="W4A8 group-wise (g=128) resident int4 512x3840x15360 on fp32 activations: step = "
                             "per-row int8 quantisation pre-pass + the configs[2] GEMM", ops=ops,
                    nbytes=nbytes, ms=ms, wall=wall, dtype="int8", peak=PEAK["int8"], bound="mfma", fd=fd,
                    cpu=lambda: self.cpu_rows(cpu, M, ops))

    def cfg_int8gemma(self):
        o, R, lib = self.orc, self.R, self.lib
        M, K, N = 512, 3840, 15360
        A = o.gen_i8((M, K), 0x52434B22)
        B = o.gen_i8((N, K), 0x52434B23)
        dA, dB = self.up(A), self.up(B)
        dC = self.torch.empty((M, N), dtype=self.torch.int32, device=self.dev)
        fd = lib.rocket_open()
        self.bind(fd)
        ms, wall = self.time_steps(lambda: lib.rocket_matmul_int8(fd, M, K, N, R.ptr(dA), R.ptr(dB), R.ptr(dC)))
        ops = 2.0 * M * N * K
        return dict(workload="int8 matmul 512x3840x15360 -> int32 (W8A8 at the configs[2] Gemma-12B shape)", ops=ops,
                    nbytes=M * K + N * K + 4 * M * N, ms=ms, wall=wall, dtype="int8", peak=PEAK["int8"],
                    bound="mfma", fd=fd,
                    cpu=lambda: self.cpu_rows(lambda m: o.matmul_int8(A[:m].copy(), B), M, ops))

    def _cfg_float(self, name, entry, oref, peak, bound):
        o, R, lib = self.orc, self.R, self.lib
        M, K, N = 2048, 15360, 3840
        A = o.gen_normal((M, K), 0x52434B06)
        B = o.gen_normal((N, K), 0x52434B07, 0.0, 0.02)
        dA, dB = self.up(A), self.up(B)
        dC = self.torch.empty((M, N), dtype=self.torch.float32, device=self.dev)
        fd = lib.rocket_open()
        self.bind(fd)
        fn = getattr(lib, entry)
        ms, wall = self.time_steps(lambda: fn(fd, M, K, N, R.ptr(dA), R.ptr(dB), R.ptr(dC)))
        ops = 2.0 * M * N * K
        # a step is the whole library call: the fp32 operands' conversion pass (bf16, or tf32
        # hi/lo pairs) and the GEMM; the roofline figure is that whole step's rate
        return dict(workload=f"{name} matmul 2048x15360x3840 fp32 in/out (configs[3]); step = conversion pass + GEMM",
                    ops=ops,
                    nbytes=4 * (M * K + N * K + M * N), ms=ms, wall=wall, dtype=name, peak=peak, bound=bound, fd=fd,
                    cpu=lambda: self.cpu_rows(lambda m: oref(A[:m].copy(), B), M, ops))

    def cfg_bf16(self):
        return self._cfg_float("bf16", "rocket_matmul_bf16", self.orc.matmul_bf16, PEAK["bf16"], "mfma")

    def cfg_tf32(self):
        return self._cfg_float("tf32", "rocket_matmul_tf32", self.orc.matmul_tf32, PEAK["bf16"], "mfma")

    # ---- config 5: the MoE expert FFN -------------------------------------------------
    def _moe_data(self):
        """Eight experts' resident int8 group-32 weights (gate, up [1408, 2048], down [2048,
        1408], per-(row, group) symmetric codes of N(0, 0.02) values) and 100 routings of 4096
        fp16 N(0,1) tokens, each top-2 over distinct experts uniformly at random. For every
        routing the routed rows are gathered per expert in HBM (padded with zero rows to a
        multiple of 4) and the down product's input is act(gate) * up of that routing's first
        product, quantised per row by the library: all of it before timing, so a timed step is
        the expert GEMMs of one forward on its own routed data."""
        if getattr(self, "_moe", None) is not None:
            return self._moe
        o, R, lib, torch = self.orc, self.R, self.lib, self.torch
        E, T, H, F, group, calls = 8, 4096, 2048, 1408, 32, 100
        ctx = lib.rocket_i8_ctx_create(1)
        fd = lib.rocket_i8_ctx_fd(ctx)
        W, S, hostw = {}, {}, {}
        for e in range(E):
            for j, (kind, (n, k)) in enumerate((("gate", (F, H)), ("up", (F, H)), ("down", (H, F)))):
                w = o.gen_normal((n, k), 0x52434B10 + 16 * e + j, 0.0, 0.02).reshape(n, k // group, group)
                amax = np.abs(w).max(axis=2)
                sc = np.where(amax > 0, amax / 127.0, 1.0).astype(np.float32)
                q = np.clip(np.rint(w / sc[:, :, None]), -127, 127).astype(np.int8).reshape(n, k)
                W[kind, e] = lib.rocket_i8_weights_pack_gw(ctx, 4, k, n, R.ptr(np.ascontiguousarray(q)), group)
                assert W[kind, e]
                S[kind, e] = self.up(sc)
                if e == 0:   # host copies for the CPU baseline
                    hostw[kind] = (np.ascontiguousarray(q), np.ascontiguousarray(sc))
        x16 = o.f32_to_f16_bits(o.gen_normal((T, H), 0x52434B05))
        xq, xs = o.quant_rows(o.f16_bits_to_f32(x16))
        # one zero row (scale 0) past the tokens: the padding rows of every expert gather it
        dxq = self.up(np.concatenate([xq, np.zeros((1, H), np.int8)]))
        dxs = self.up(np.concatenate([xs, np.zeros(1, np.float32)]))
        rng = np.random.default_rng(0x52434B05)
        self.bind(fd)
        routes = []
        for i in range(calls):
            top2 = rng.random((T, E)).argsort(axis=1)[:, :2]
            A, a, Ms, Mreal = [], [], [], 0
            for e in range(E):
                idx = np.nonzero((top2 == e).any(axis=1))[0]
                m = len(idx)
                mp = (m + 3) // 4 * 4
                sel = torch.from_numpy(np.concatenate([idx, np.full(mp - m, T)]).astype(np.int64)).to(self.dev)
                A.append(dxq.index_select(0, sel).contiguous())
                a.append(dxs.index_select(0, sel).contiguous())
                Ms.append(mp)
                Mreal += m
            routes.append(dict(A=A, a=a, M=Ms, rows=Mreal))
        Mmax = max(max(r["M"]) for r in routes)
        Cg = [torch.empty((Mmax, F), dtype=torch.float32, device=self.dev) for _ in range(2 * E)]
        Cd = [torch.empty((Mmax, H), dtype=torch.float32, device=self.dev) for _ in range(E)]
        up_fn = lib.rocket_matmul_int8_prepacked_gw_grouped_rowscale
        kW = (C.c_void_p * (2 * E))(*([W["gate", e] for e in range(E)] + [W["up", e] for e in range(E)]))
        jW = (C.c_void_p * E)(*[W["down", e] for e in range(E)])
        pbs, kb = R.ptr_array([S["gate", e] for e in range(E)] + [S["up", e] for e in range(E)])
        qbs, jb = R.ptr_array([S["down", e] for e in range(E)])
        pC, kc = R.ptr_array(Cg)
        qC, jc = R.ptr_array(Cd)
        keep = [kW, jW, kb, jb, kc, jc]
        for r in routes:
            pA, k1 = R.ptr_array(r["A"] + r["A"])
            pa, k2 = R.ptr_array(r["a"] + r["a"])
            pM, k3 = R.int_array(r["M"] + r["M"])
            qM, k4 = R.int_array(r["M"])
            # this routing's down input: act(gate) * up of its gate/up product, per-row int8
            assert up_fn(ctx, 2 * E, pM, H, F, pA, pa, pbs, pC, C.cast(kW, R.pp)) == 0
            Ah, ah = [], []
            for e in range(E):
                m = r["M"][e]
                g, u = Cg[e][:m], Cg[E + e][:m]
                h = (torch.nn.functional.silu(g) * u).contiguous()
                q = torch.empty((m, F), dtype=torch.int8, device=self.dev)
                s = torch.empty(m, dtype=torch.float32, device=self.dev)
                if m:
                    assert lib.rocket_quantize_rows_int8(fd, m, F, R.ptr(h), R.ptr(q), R.ptr(s)) == 0
                Ah.append(q)
                ah.append(s)
            qA, k5 = R.ptr_array(Ah)
            qa, k6 = R.ptr_array(ah)
            r.update(Ah=Ah, ah=ah, pA=pA, pa=pa, pM=pM, qA=qA, qa=qa, qM=qM)
            keep += [k1, k2, k3, k4, k5, k6]
        torch.cuda.synchronize()
        r0, m0 = routes[0], routes[0]["M"][0]
        host = dict(A=r0["A"][0][:m0].cpu().numpy(), a=r0["a"][0][:m0].cpu().numpy(),
                    Ah=r0["Ah"][0][:m0].cpu().numpy(), ah=r0["ah"][0][:m0].cpu().numpy(),
                    Wg=hostw["gate"][0], sg=hostw["gate"][1], Wd=hostw["down"][0], sd=hostw["down"][1])
        self._moe = dict(ctx=ctx, fd=fd, W=W, S=S, routes=routes, E=E, H=H, F=F, group=group, calls=calls,
                         pbs=pbs, qbs=qbs, pC=pC, qC=qC, pW=C.cast(kW, R.pp), qW=C.cast(jW, R.pp), Cg=Cg, Cd=Cd,
                         keep=keep, host=host)
        return self._moe

    def _moe_result(self, d, ms, wall, workload, per_group=False):
        rows = float(np.mean([r["rows"] for r in d["routes"]]))
        H, F, E, group = d["H"], d["F"], d["E"], d["group"]
        ops = rows * 3 * 2.0 * H * F
        mpad = float(np.mean([sum(r["M"]) for r in d["routes"]]))
        # weights and scales once, the routed activations (int8) and their scales, fp32 outputs
        nbytes = 3 * E * H * F + 4 * 3 * E * F * H // group + mpad * (H + F) + 4 * 2 * mpad + 4 * mpad * (2 * F + H)
        return dict(workload=workload, ops=ops, nbytes=nbytes, ms=ms, wall=wall, dtype="int8", peak=PEAK["int8"],
                    bound="mfma", fd=d["fd"], cpu=lambda: self._moe_cpu(d, per_group))

    def _moe_cpu(self, d, per_group):
        """The oracle on a row sample of the first routing's expert 0: its gate product
        (2048 -> 1408) and its down product (1408 -> 2048) on the first m routed rows, with
        per-row scales (the grouped entry) or the same scales repeated per group (the reference
        entry, reference fold order). The rate of these two products stands for the forward's:
        the gate, up and down products of every expert have the same cost per operation."""
        o, H, F, group = self.orc, d["H"], d["F"], d["group"]
        h = d["host"]
        A, a, Ah, ah = h["A"], h["a"], h["Ah"], h["ah"]
        M = A.shape[0]
        if per_group:
            ag = np.ascontiguousarray(np.repeat(a[:, None], H // group, axis=1))
            ahg = np.ascontiguousarray(np.repeat(ah[:, None], F // group, axis=1))

            def fn(m):
                o.matmul_gw_f32(A[:m].copy(), h["Wg"], ag[:m].copy(), h["sg"], group)
                o.matmul_gw_f32(Ah[:m].copy(), h["Wd"], ahg[:m].copy(), h["sd"], group)
        else:
            def fn(m):
                o.matmul_gw_rowscale_f32(A[:m].copy(), h["Wg"], a[:m].copy(), h["sg"], group)
                o.matmul_gw_rowscale_f32(Ah[:m].copy(), h["Wd"], ah[:m].copy(), h["sd"], group)
        r = self.cpu_rows(fn, M, 2 * 2.0 * M * H * F)
        r["sample"] = "expert 0 of the first routing, gate and down products: " + r["sample"]
        return r

    def cfg_moe(self):
        d = self._moe_data()
        lib = self.lib
        ctx, E, H, F, routes = d["ctx"], d["E"], d["H"], d["F"], d["routes"]
        up_fn = lib.rocket_matmul_int8_prepacked_gw_grouped_rowscale
        self.bind(d["fd"])

        def forward(i):
            r = routes[i]
            rc = up_fn(ctx, 2 * E, r["pM"], H, F, r["pA"], r["pa"], d["pbs"], d["pC"], d["pW"])
            if rc:
                return rc
            return up_fn(ctx, E, r["qM"], F, H, r["qA"], r["qa"], d["qbs"], d["qC"], d["qW"])

        it = iter(range(10 ** 9))
        ms, wall = self.time_steps(lambda: forward(next(it) % d["calls"]))
        return self._moe_result(d, ms, wall, "MoE resident int8 group-wise (g=32), 8 experts, 4096 tok top-2 over "
                                "gathered routed rows, per-row activation scales (configs[4]); a step = one forward's "
                                "expert GEMMs: the grouped gate+up launch and the grouped down launch")

    def cfg_moe_fwd(self):
        """Config 5's whole expert FFN forward per step: the gate and up products of all experts
        in one grouped launch with fp16 results (rocket_matmul_int8_prepacked_gw_grouped_rowscale_
        f16out: each fp32 result rounded once), then the down products through
        rocket_matmul_int8_prepacked_gw_grouped_glu_f16in, whose one pre-pass launch forms
        SiLU(gate) * up in fp32 from those rows and quantises every expert's rows per row
        before its grouped launch. Checked once against the precomputed forward of the same
        routing, whose gated rows torch formed in fp32 from fp32 gate and up products: within
        1e-2 normalised error (the fp16 gate and up values, 2^-11 relative, move some codes of
        the int8 re-quantisation by one step)."""
        d = self._moe_data()
        R, lib, torch, o = self.R, self.lib, self.torch, self.orc
        ctx, E, H, F, routes = d["ctx"], d["E"], d["H"], d["F"], d["routes"]
        Mmax = max(max(r["M"]) for r in routes)
        G = torch.zeros((2 * E, Mmax, F), dtype=torch.float16, device=self.dev)
        Dn = torch.empty((E, Mmax, H), dtype=torch.float32, device=self.dev)
        pG, k1 = R.ptr_array([G[i] for i in range(2 * E)])
        pGg, k2 = R.ptr_array([G[e] for e in range(E)])
        pGu, k3 = R.ptr_array([G[E + e] for e in range(E)])
        pD, k4 = R.ptr_array([Dn[e] for e in range(E)])
        up_fn = lib.rocket_matmul_int8_prepacked_gw_grouped_rowscale_f16out
        dn_fn = lib.rocket_matmul_int8_prepacked_gw_grouped_glu_f16in
        silu = R.ROCKET_ACTIVATION_SILU
        self.bind(d["fd"])

        def forward(i):
            r = routes[i]
            rc = up_fn(ctx, 2 * E, r["pM"], H, F, r["pA"], r["pa"], d["pbs"], pG, d["pW"])
            if rc:
                return rc
            return dn_fn(ctx, E, r["qM"], F, H, pGg, pGu, silu, d["qbs"], pD, d["qW"])

        assert forward(0) == 0
        r = routes[0]
        assert lib.rocket_matmul_int8_prepacked_gw_grouped_rowscale(ctx, E, r["qM"], F, H, r["qA"], r["qa"],
                                                                    d["qbs"], d["qC"], d["qW"]) == 0
        torch.cuda.synchronize()
        for e in range(E):
            m = r["M"][e]
            if m:
                err = o.norm_err(Dn[e][:m].cpu().numpy(), d["Cd"][e][:m].cpu().numpy())
                assert err <= 1e-2, f"moe_fwd expert {e}: {err}"
        it = iter(range(10 ** 9))
        ms, wall = self.time_steps(lambda: forward(next(it) % d["calls"]))
        del k1, k2, k3, k4
        return self._moe_result(d, ms, wall, "configs[4] whole expert FFN forward: gate+up grouped launch with fp16 "
                                "results, then one pre-pass launch forming SiLU(gate)*up in fp32 and quantising it "
                                "per row, and the down grouped launch (rocket_matmul_int8_prepacked_gw_grouped_"
                                "rowscale_f16out + _glu_f16in); ops = the three GEMMs")

    def cfg_moe_ref(self):
        """Config 5 through the reference's own resident entry, rocket_matmul_int8_prepacked_gw,
        one call per expert and weight (24 calls a forward), activation scales a_scale[M * nG]
        (each row's scale repeated over its groups, as a per-token quantising caller passes, so
        every tile folds in the row-scale order)."""
        d = self._moe_data()
        R, lib, torch = self.R, self.lib, self.torch
        ctx, E, H, F, group, routes = d["ctx"], d["E"], d["H"], d["F"], d["group"], d["routes"]
        for r in routes:
            if "ag" not in r:
                r["ag"] = [a[:, None].expand(-1, H // group).contiguous() for a in r["a"]]
                r["ahg"] = [a[:, None].expand(-1, F // group).contiguous() for a in r["ah"]]
        fn = lib.rocket_matmul_int8_prepacked_gw
        W, S, Cg, Cd = d["W"], d["S"], d["Cg"], d["Cd"]
        calls = []
        for r in routes:
            cs = []
            for e in range(E):
                m = r["M"][e]
                if not m:
                    continue
                for kind, A, a, Cout, k, n in (("gate", r["A"][e], r["ag"][e], Cg[e], H, F),
                                               ("up", r["A"][e], r["ag"][e], Cg[E + e], H, F),
                                               ("down", r["Ah"][e], r["ahg"][e], Cd[e], F, H)):
                    cs.append((m, k, n, R.ptr(A), R.ptr(a), R.ptr(S[kind, e]), R.ptr(Cout), W[kind, e]))
            calls.append(cs)
        self.bind(d["fd"])

        def forward(i):
            for m, k, n, A, a, b, Cout, w in calls[i]:
                rc = fn(ctx, m, k, n, A, a, b, Cout, w)
                if rc:
                    return rc
            return 0

        it = iter(range(10 ** 9))
        ms, wall = self.time_steps(lambda: forward(next(it) % d["calls"]))
        return self._moe_result(d, ms, wall, "configs[4] through the reference entry rocket_matmul_int8_prepacked_gw: "
                                "24 per-expert calls a forward (gate, up, down), per-group activation scales",
                                per_group=True)

    def cfg_ffn(self):
        o, R, lib = self.orc, self.R, self.lib
        M, H, I, kind = 512, 3840, 15360, R.ROCKET_ACTIVATION_GELU
        a = 3.0 / np.sqrt(H)
        x = o.f32_to_f16_bits(o.gen_uniform((M, H), 0x52434B30))
        Wg = o.f32_to_f16_bits(o.gen_uniform((I, H), 0x52434B31, -a, a))
        Wu = o.f32_to_f16_bits(o.gen_uniform((I, H), 0x52434B32, -a, a))
        Wd = o.f32_to_f16_bits(o.gen_uniform((H, I), 0x52434B33, -1.5 / np.sqrt(I), 1.5 / np.sqrt(I)))
        dx, dg, du, dd = self.up(x), self.up(Wg), self.up(Wu), self.up(Wd)
        dout = self.torch.empty((M, H), dtype=self.torch.float16, device=self.dev)
        fd = lib.rocket_open()
        self.bind(fd)
        ms, wall = self.time_steps(lambda: lib.rocket_ffn_fp16_fused(fd, M, H, I, R.ptr(dx), R.ptr(dg), R.ptr(du),
                                                                     R.ptr(dd), kind, R.ptr(dout)))
        ops = 3 * 2.0 * M * H * I
        nbytes = 2 * (M * H + 3 * I * H + M * H) + 2 * 2 * M * I     # + the [M, I] product written, read
        return dict(workload="gated FFN block fp16 (GeGLU) M=512 H=3840 I=15360 (Gemma-12B, the configs[2] "
                             "caller); step = gate/up launch with the activation epilogue + down launch",
                    ops=ops, nbytes=nbytes, ms=ms, wall=wall, dtype="fp16", peak=PEAK["fp16"], bound="mfma", fd=fd,
                    cpu=lambda: self.cpu_rows(lambda m: o.ffn_f16(x[:m].copy(), Wg, Wu, Wd, kind), M, ops))

    def cfg_attn(self):
        """Masked grouped-query attention at a Gemma-12B layer shape: 512-token prefill chunk
        over a 4096-key cache (causal: query t sees keys <= 3584 + t), head_dim 256, 16 query
        heads on 8 kv heads. Work counted densely (every (query, key) pair), as the kernel
        computes it."""
        o, R, lib, torch = self.orc, self.R, self.lib, self.torch
        T, n_kv, dh, nh, nkvh = 512, 4096, 256, 16, 8
        rng = np.random.default_rng(0x52434B40)
        Q = rng.uniform(-1, 1, (nh, T, dh)).astype(np.float16)
        K = rng.uniform(-1, 1, (nkvh, n_kv, dh)).astype(np.float16)
        V = rng.uniform(-1, 1, (nkvh, dh, n_kv)).astype(np.float16)
        pos = n_kv - T + np.arange(T)[:, None]
        M = np.where(np.arange(n_kv)[None, :] <= pos, 0.0, -np.inf).astype(np.float16)
        dQ, dK, dV, dM = (self.up(a.view(np.int16)) for a in (Q, K, V, M))
        dO = torch.empty((nh, T, dh), dtype=torch.float16, device=self.dev)
        fd = lib.rocket_open()
        self.bind(fd)
        scale = float(1.0 / np.sqrt(dh))
        ms, wall = self.time_steps(lambda: lib.rocket_flash_attn_fp16(fd, T, n_kv, dh, dh, nh, nkvh, scale, 0.0,
                                                                      R.ptr(dQ), R.ptr(dK), R.ptr(dV), R.ptr(dM),
                                                                      R.ptr(dO)))
        ops = 4.0 * nh * T * n_kv * dh
        nbytes = 2 * (nh * T * dh + 2 * nkvh * n_kv * dh + T * n_kv + nh * T * dh)
        Qb, Kb, Vb, Mb = (a.view(np.uint16) for a in (Q, K, V, M))
        def cpu(m):   # the first m query rows of every head
            return o.flash_attn_f16(np.ascontiguousarray(Qb[:, :m]), Kb, Vb, np.ascontiguousarray(Mb[:m]), scale, 0.0)
        return dict(workload="flash attention fp16, 512 queries x 4096 keys (causal, cached prefix), head_dim 256, "
                             "16 q-heads / 8 kv-heads (Gemma-12B local layer shape)",
                    ops=ops, nbytes=nbytes, ms=ms, wall=wall, dtype="fp16", peak=PEAK["fp16"], bound="mfma", fd=fd,
                    cpu=lambda: self.cpu_rows(cpu, T, ops))

    def cfg_weights_load(self):
        """Loading the config-3 int4 weight (with its scales) from a serialised file into HBM,
        against packing it again from int8 values: host wall time per call, file in the page
        cache."""
        import tempfile
        o, R, lib = self.orc, self.R, self.lib
        M, K, N, group = 512, 3840, 15360, 128
        B = o.gen_i8((N, K), 0x52434B04, -8, 7)
        bsc = o.gen_uniform((N, K // group), 0x52434B05, 0.005, 0.02)
        ctx = lib.rocket_i4_ctx_create(1)
        fd = lib.rocket_i4_ctx_fd(ctx)
        w = lib.rocket_i4_weights_pack_gw(ctx, M, K, N, R.ptr(B), group)
        assert w
        path = os.path.join(tempfile.mkdtemp(), "gemma_ffn_up_int4_g128.rktw")
        assert lib.rocket_i4_weights_save(ctx, w, R.ptr(bsc), path.encode()) == 0
        nbytes = os.path.getsize(path)
        sc = np.empty_like(bsc)

        def timed(fn, reps):
            t = []
            for _ in range(reps):
                t0 = time.perf_counter()
                ww = fn()
                t.append(time.perf_counter() - t0)
                assert ww
                lib.rocket_i4_weights_free(ctx, ww)
            return float(np.median(t)) * 1e3

        timed(lambda: lib.rocket_i4_weights_load(ctx, path.encode(), R.ptr(sc)), 3)
        ms = timed(lambda: lib.rocket_i4_weights_load(ctx, path.encode(), R.ptr(sc)), max(5, self.steps // 5))
        repack = timed(lambda: lib.rocket_i4_weights_pack_gw(ctx, M, K, N, R.ptr(B), group), max(5, self.steps // 5))
        assert np.array_equal(sc, bsc)
        lib.rocket_i4_weights_free(ctx, w)
        os.remove(path)
        self.per_step[self.cur] = {"load_ms": ms, "repack_from_int8_ms": repack}
        return dict(workload=f"load the configs[2] int4 weight + scales from a {nbytes} B serialised file into HBM "
                             "(median host wall per call; step = one rocket_i4_weights_load)",
                    ops=float(nbytes), nbytes=nbytes, ms=ms, wall=ms, dtype="u8", peak=PEAK["pcie"], bound="pcie",
                    fd=fd, cpu=None)

    # ---- CPU baseline ----------------------------------------------------------------
    def cpu_naive_config1(self, budget_s=2.0):
        """The comparability row: the reference tests' single-thread fp16 loop
        (tests/matmul_fp16_rocket.c:43-50, oracle matmul_fp16_naive) on config 1, 64x256x128,
        repeated for about budget_s seconds."""
        o = self.orc
        M, K, N = 64, 256, 128
        A = o.f32_to_f16_bits(o.gen_uniform((M, K), 0x52434B01))
        B = o.f32_to_f16_bits(o.gen_uniform((N, K), 0x52434B02))
        reps, total = 0, 0.0
        while total < budget_s and reps < 100000:
            t0 = time.perf_counter()
            o.matmul_fp16_naive(A, B)
            total += time.perf_counter() - t0
            reps += 1
        ms = total / reps * 1e3
        return {"value": round(2.0 * M * N * K / (ms * 1e-3) / 1e9, 3), "unit": "GFLOP/s", "cores": 1,
                "ms_per_call": round(ms, 4), "sample": f"configs[0] 64x256x128 fp16, {reps} calls ({total:.1f} s)"}

    def cpu_rows(self, fn, M, ops_full, budget_s=10.0):
        """Oracle on the first m rows (doubling m while a run takes under a quarter of the
        budget), then repeated until about budget_s seconds of CPU work; scaled to ops/s."""
        threads = self.orc.set_threads(cpu_threads())
        m = 4
        while True:
            t0 = time.perf_counter()
            fn(m)
            dt = time.perf_counter() - t0
            if dt > budget_s / 4 or m >= M:
                break
            m = min(M, m * 2)
        reps, total = 1, dt
        while total < budget_s and reps < 1000:
            t0 = time.perf_counter()
            fn(m)
            total += time.perf_counter() - t0
            reps += 1
        ops = ops_full * m / M * reps
        return dict(value=ops / total / 1e12, cores=threads,
                    sample=f"first {m} of {M} rows x {reps} runs ({total:.1f} s)")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="int4gw", choices=CONFIGS)
    ap.add_argument("--all", action="store_true", help="also measure every other config")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain device copy of 256 MiB (calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.copy_probe:
        import torch
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")      # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": src.numel() * 4}))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the matmul path is built and measured per GPU "
              "(multi-GPU sharding is a design note, not part of this build)", file=sys.stderr)
        sys.exit(2)

    b = Bench(args.steps, args.warmup)
    names = [args.config] + ([n for n in CONFIGS if n != args.config] if args.all else [])
    results = {}
    for n in names:
        b.cur = n
        r = getattr(b, "cfg_" + n)()
        results[n] = r
        print(f"[bench] {n}: {r['ms'] * 1e3:.1f} us/step, {r['ops'] / r['ms'] / 1e9:.1f} TOPS", file=sys.stderr, flush=True)

    r = results[args.config]
    value = r["ops"] / (r["ms"] * 1e-3) / 1e12
    if r["bound"] in ("hbm", "pcie"):
        ach, unit = r["nbytes"] / (r["ms"] * 1e-3) / 1e9, "GB/s"
    else:
        ach, unit = value, "TFLOP/s"
    if r["bound"] == "pcie":
        value = ach
    line = {
        "metric": "TOPS int8/int4, TFLOPS fp16 per GEMM at Gemma-12B prefill; % MFMA peak",
        "value": round(value, 3),
        "unit": "GB/s" if r["bound"] == "pcie" else ("TFLOP/s" if r["dtype"] in ("fp16", "bf16", "tf32") else "TOPS"),
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(r["ms"], 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": r["dtype"], "data": "synthetic (splitmix64-seeded, BASELINE.json distributions)",
        "config": {"workload": r["workload"]},
        "roofline": {"bound": r["bound"], "achieved": round(ach, 3), "peak": r["peak"], "unit": unit,
                     "frac": round(ach / r["peak"], 4), "traffic": traffic(args.config)},
        # median single-step times (20 each): warm = as in the timed loop; cold = after a
        # 512 MiB write that evicts the inputs from L2 and MALL
        "per_step_median_ms": {k: round(v, 6) for k, v in b.per_step.get(args.config, {}).items()},
    }
    vb = vendor_baseline(args.config)
    if vb:
        line["vendor_baseline"] = vb
    if not args.no_cpu and r.get("cpu"):
        cb = r["cpu"]()
        hostinfo = cpu_host()
        line["cpu_baseline"] = {"value": round(cb["value"], 4), "unit": line["unit"], "cores": cb["cores"],
                                "kind": "port", "sample": cb["sample"], "nproc": hostinfo["nproc"],
                                "affinity_cpus": hostinfo["affinity_cpus"],
                                "omp_num_threads": hostinfo["omp_num_threads"], "cpu_model": hostinfo["cpu_model"],
                                # the comparability row: the reference tests' single-thread loop on configs[0]
                                "naive_1t_config1": b.cpu_naive_config1()}
    if args.all:
        line["per_config"] = {n: {"us_per_step": round(x["ms"] * 1e3, 2),
                                  "value": round(x["ops"] / (x["ms"] * 1e-3) / (1e9 if x["bound"] == "pcie" else 1e12), 3),
                                  "frac_of_peak": round(x["ops"] / (x["ms"] * 1e-3) / 1e12 / x["peak"], 4)
                                  if x["bound"] == "mfma" else
                                  round(x["nbytes"] / (x["ms"] * 1e-3) / 1e9 / x["peak"], 4),
                                  "unit": "GB/s" if x["bound"] == "pcie" else "TOPS / TFLOP/s",
                                  "host_wall_us": round(x["wall"] * 1e3, 2),
                                  "median_us": {k: round(v * 1e3, 2) for k, v in b.per_step.get(n, {}).items()}}
                              for n, x in results.items()}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
