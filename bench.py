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


CONFIGS = ["fp16", "int8", "int16", "int4gw", "int8gemma", "bf16", "tf32", "moe", "ffn", "int4gw_f32in",
           "weights_load", "attn"]


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


def cpu_threads():
    return max(1, min(16, os.cpu_count() or 1))


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

    def cfg_moe(self):
        o, R, lib, torch = self.orc, self.R, self.lib, self.torch
        E, T, H, F, group, calls = 8, 4096, 2048, 1408, 32, 100
        ctx = lib.rocket_i8_ctx_create(1)
        fd = lib.rocket_i8_ctx_fd(ctx)
        W = {}
        scales = {}
        for e in range(E):
            for kind, (n, k) in (("gate", (F, H)), ("up", (F, H)), ("down", (H, F))):
                w = np.clip(np.round(o.gen_normal((n, k), 0x52434B10 + 16 * e + len(kind)) / 0.02 * 16), -127, 127).astype(np.int8)
                W[kind, e] = lib.rocket_i8_weights_pack_gw(ctx, 4, k, n, R.ptr(w), group)
                assert W[kind, e]
                scales[kind, e] = self.up(o.gen_uniform((n, k // group), 0x52434B90 + 16 * e + len(kind), 0.001, 0.002))
        x = o.gen_normal((T, H), 0x52434B05)
        xq = np.clip(np.round(x / (np.abs(x).max(axis=1, keepdims=True) / 127)), -127, 127).astype(np.int8)
        rng = np.random.default_rng(0x52434B05)
        routes = []
        for _ in range(calls):
            r = rng.random((T, E)).argsort(axis=1)[:, :2]          # top-2 distinct experts, uniform
            cnt = np.bincount(r.ravel(), minlength=E)
            routes.append([int((c + 3) // 4 * 4) for c in cnt])    # per-expert M padded to %4
        Mmax = max(max(r) for r in routes)
        Ain = [self.up(np.resize(xq, (Mmax, H))) for _ in range(E)]
        Ah = [self.up(o.gen_i8((Mmax, F), 0x52434C00 + e, -127, 127)) for e in range(E)]
        # activations quantised per row (per token): one fp32 scale per row
        xs = (np.abs(x).max(axis=1) / 127).astype(np.float32)
        a_in = [self.up(np.resize(xs, Mmax)) for _ in range(E)]
        a_h = [self.up(np.full(Mmax, 1.0 / 127, np.float32)) for _ in range(E)]
        Cg = [torch.empty((Mmax, F), dtype=torch.float32, device=self.dev) for _ in range(2 * E)]
        Cd = [torch.empty((Mmax, H), dtype=torch.float32, device=self.dev) for _ in range(E)]
        self.bind(fd)
        # every argument array is built before timing: a step is the two library calls
        pA, kA = R.ptr_array(Ain + Ain)
        pas, ka = R.ptr_array(a_in + a_in)
        pbs, kb = R.ptr_array([scales["gate", e] for e in range(E)] + [scales["up", e] for e in range(E)])
        pC, kc = R.ptr_array(Cg)
        kW = (C.c_void_p * (2 * E))(*([W["gate", e] for e in range(E)] + [W["up", e] for e in range(E)]))
        pW = C.cast(kW, R.pp)
        qA, jA = R.ptr_array(Ah)
        qas, ja = R.ptr_array(a_h)
        qbs, jb = R.ptr_array([scales["down", e] for e in range(E)])
        qC, jc = R.ptr_array(Cd)
        jW = (C.c_void_p * E)(*[W["down", e] for e in range(E)])
        qW = C.cast(jW, R.pp)
        Mup = [R.int_array(r + r) for r in routes]
        Mdown = [R.int_array(r) for r in routes]
        up_fn = lib.rocket_matmul_int8_prepacked_gw_grouped_rowscale

        def forward(i):
            rc = up_fn(ctx, 2 * E, Mup[i][0], H, F, pA, pas, pbs, pC, pW)
            if rc:
                return rc
            return up_fn(ctx, E, Mdown[i][0], F, H, qA, qas, qbs, qC, qW)

        it = iter(range(10 ** 9))
        ms, wall = self.time_steps(lambda: forward(next(it) % calls))
        ops = float(np.mean([sum(r) for r in routes])) * 3 * 2.0 * H * F
        mavg = float(np.mean([sum(r) for r in routes]))
        nbytes = 3 * E * H * F + 4 * 3 * E * F * H // group + mavg * (2 * H + F) + 4 * mavg * (2 * F + H)
        return dict(workload="MoE resident int8 group-wise (g=32), 8 experts, 4096 tok top-2, per-row activation "
                             "scales (configs[4]); a step = one forward (gate+up launch, down launch)",
                    ops=ops, nbytes=nbytes, ms=ms, wall=wall, dtype="int8", peak=PEAK["int8"], bound="mfma", fd=fd,
                    cpu=None)

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
    if not args.no_cpu and r.get("cpu"):
        cb = r["cpu"]()
        line["cpu_baseline"] = {"value": round(cb["value"], 4), "unit": line["unit"], "cores": cb["cores"],
                                "kind": "port", "sample": cb["sample"]}
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
