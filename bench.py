"""Benchmark of the int8 block-stack forward path on one MI355X (prints ONE JSON line).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]

Workloads:
    stack   config[3]: the Ava-0.4-shaped int8 block stack, teacher-forced, B=64, T=2048, d=1024
    stack_heads  config[3] with the engram at the reference's geometry (32 heads of 32, f32 store)
    greedy  config[0]: one stream, a 512-token prompt and 128 greedy steps, d=512
    decode  config[4]: batched stateful decode, B=256 streams, 32768-token state
    lif     config[1]: the standalone LIF scan, B=64, T=2048, C=2048
    delta   config[2]: the plain delta rule, chunked, B=32, H=8, T=4096, d=64
    kwta    the kWTA + relu2 of config[3]'s wide layer (131072 rows of 4096, k=1024)
    gemm    one config[3] dense int8 product (131072 x 1024 x 4096)
    copy    a plain device copy of 1 GiB (the traffic-counter calibration kernel)

A "step" is one pass of the path over one batch of synthetic input resident in HBM. The timed
region is K steps between two synchronisations; the dominant kernel's average duration comes from
HIP events recorded on the stream the kernels are launched on (torch's current stream, which is the
stream every ava_* call receives). The CPU baseline is the oracle (a C restatement of the
reference's CPU loops) timed on a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "tokens/sec int8 block-stack forward @B=64,T=2048, 1 GPU; % HBM / MFMA roofline"
HBM_PEAK_GBS = 8000.0
WARM_S = 0.25  # minimum warm-up time, seconds (the stack's three default warm-up steps take longer)
I8_PEAK_TOPS = 5000.0  # dense int8 MFMA, TOP/s
F32_MFMA_PEAK_TFLOPS = 157.3  # dense fp32 MFMA
FP32_PEAK_TFLOPS = 157.3


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_threads():
    n = os.cpu_count() or 1
    return max(1, min(n, 16))


# ----------------------------------------------------------------------------- workloads


class Lif:
    """config[1]: cur ~N(0,1) [64, 2048, 2048]; beta = sigmoid(U(1.5, 4.5)); theta 1, rho 0.95,
    gain 0.05; int2 spikes, subtract reset; outputs int8 spikes, final v and theta."""

    name = "lif"
    metric = "tokens/sec LIF scan @B=64,T=2048,C=2048 (config[1]), int2 spikes, ALIF, 1 GPU; % HBM roofline"
    warm_extend = True  # short, repeatable steps: warm up for WARM_S seconds
    kernel = "lif_scan_buf_kernel"  # the scan for D a multiple of 64 (lif_scan_kernel otherwise)

    def __init__(self, B=64, T=2048, D=2048):
        import torch
        from ava_amd import _lib

        self.B, self.T, self.D = B, T, D
        self.L = _lib.lib()
        g = torch.Generator(device="cuda").manual_seed(1)
        self.cur = torch.randn((B, T, D), device="cuda", generator=g, dtype=torch.float32)
        beta = torch.sigmoid(torch.rand(D, device="cuda", generator=g) * 3.0 + 1.5)
        self.ps = torch.cat([beta, torch.ones(D, dtype=torch.float32, device="cuda"), torch.full((D,), 0.95, dtype=torch.float32, device="cuda"),
                             torch.full((D,), 0.05, dtype=torch.float32, device="cuda")]).contiguous()
        self.v = torch.zeros((B, D), dtype=torch.float32, device="cuda")
        self.s = torch.zeros((B, D), dtype=torch.float32, device="cuda")
        self.a = torch.zeros((B, D), dtype=torch.float32, device="cuda")
        self.th = torch.empty((B, D), dtype=torch.float32, device="cuda")
        self.spikes = torch.empty((B, T, D), dtype=torch.int8, device="cuda")
        self.tokens = B * T
        # algorithmic bytes: read cur, write spikes, write v_T and theta_T, read the 4 parameter rows
        self.bytes = B * T * D * (4 + 1) + B * D * (4 + 4) + 4 * D * 4
        self.config = {"workload": "lif_scan config[1]", "B": B, "T": T, "C": D, "spikes": "int2",
                       "alif": True, "rho": 0.95, "gain": 0.05}
        self.dtype = "f32"

    def step(self, stream, ev=None):
        from ava_amd._lib import check
        import ctypes as C

        # the state carries over from step to step (a stream read in pieces, state.rs:4-12)
        args = (C.c_void_p(self.cur.data_ptr()), self.B, self.T, self.D, C.c_void_p(self.ps.data_ptr()),
                C.c_void_p(self.v.data_ptr()), C.c_void_p(self.s.data_ptr()), C.c_void_p(self.a.data_ptr()), 2, 1, 1,
                C.c_void_p(self.spikes.data_ptr()), C.c_void_p(self.th.data_ptr()))
        if ev: ev[0].record()
        check(self.L.ava_lif_scan(*args, stream))
        if ev: ev[1].record()

    def roofline(self, kernel_s):
        a = self.bytes / kernel_s / 1e9
        return {"bound": "hbm", "achieved": a, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": a / HBM_PEAK_GBS}

    def cpu_baseline(self):
        from oracle import oracle as O

        O.set_threads(1)  # the reference's CPU scan is one loop on one thread (lif_gen.rs:198-212)
        B = 32
        rng = np.random.default_rng(1)
        cur = rng.standard_normal((B, self.T, self.D), dtype=np.float32)
        beta = (1.0 / (1.0 + np.exp(-rng.uniform(1.5, 4.5, self.D)))).astype(np.float32)
        ps = np.concatenate([beta, np.ones(self.D), np.full(self.D, 0.95), np.full(self.D, 0.05)]).astype(np.float32)
        t0 = time.perf_counter()
        O.lif_scan(cur, ps, levels=2, signed=True, alif=True)
        dt = time.perf_counter() - t0
        return {"value": B * self.T / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
                "sample": f"oracle lif_scan (the reference's lif_gen.rs:191-214 loop), B={B} of 64, "
                          f"T={self.T}, C={self.D}, one thread, {dt:.2f} s"}


class Kwta:
    """kWTA + relu2 over config[3]'s wide layer: u [131072, 4096] ~N(0,1), k = 1024."""

    name = "kwta"
    metric = "tokens/sec kWTA + relu2 planes @131072 rows (tokens) x 4096, k=1024 (config[3] wide layer), 1 GPU; % HBM roofline"
    warm_extend = True  # short, repeatable steps: warm up for WARM_S seconds
    kernel = "kwta_kernel"

    def __init__(self, n=131072, h=4096, k=1024):
        import torch
        from ava_amd import _lib

        self.n, self.h, self.k = n, h, k
        self.L = _lib.lib()
        g = torch.Generator(device="cuda").manual_seed(2)
        self.u = torch.randn((n, h), device="cuda", generator=g)
        self.a = torch.empty_like(self.u)
        self.kth = torch.empty(n, dtype=torch.float32, device="cuda")
        self.tokens = n
        self.bytes = n * h * 8 + n * 4
        self.config = {"workload": "kwta_relu2 config[3] wide layer", "rows": n, "H": h, "k": k}
        self.dtype = "f32"

    def step(self, stream, ev=None):
        from ava_amd._lib import check
        import ctypes as C

        if ev: ev[0].record()
        check(self.L.ava_kwta(C.c_void_p(self.u.data_ptr()), self.n, self.h, self.k, 1,
                              C.c_void_p(self.a.data_ptr()), C.c_void_p(self.kth.data_ptr()), stream))
        if ev: ev[1].record()

    def roofline(self, kernel_s):
        a = self.bytes / kernel_s / 1e9
        return {"bound": "hbm", "achieved": a, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": a / HBM_PEAK_GBS}

    def cpu_baseline(self):
        from oracle import oracle as O

        O.set_threads(1)
        rows = 2048
        u = np.random.default_rng(2).standard_normal((rows, self.h)).astype(np.float32)
        t0 = time.perf_counter()
        O.kwta(u, self.k, True)
        dt = time.perf_counter() - t0
        return {"value": rows / dt, "unit": "rows/s", "cores": 1, "kind": "port",
                "sample": f"oracle kwta (sort per row, lif.rs:248-263), {rows} rows of {self.h}, {dt:.2f} s"}


class Gemm:
    """One dense int8 product of config[3]: x [131072, 1024] f32 -> 3 planes -> i8 MFMA -> y [131072, 4096]."""

    name = "gemm"
    metric = "tokens/sec int8 product @131072 rows (tokens) x 1024 -> 4096, 3 activation planes (config[3] W1), 1 GPU; % i8 MFMA roofline"
    warm_extend = True  # short, repeatable steps: warm up for WARM_S seconds
    kernel = "q8_gemm_kernel"

    def __init__(self, m=131072, k=1024, n=4096, planes=3):
        import torch
        from ava_amd import ops

        self.m, self.k, self.n, self.planes = m, k, n, planes
        g = torch.Generator(device="cuda").manual_seed(3)
        w = torch.randn((k, n), device="cuda", generator=g) * 0.02
        self.qw = ops.QW.from_tensor(w)
        self.x = torch.randn((m, k), device="cuda", generator=g)
        self.xq, self.xe = ops.quant_rows(self.x, planes)
        self.y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        self.tokens = m
        self.ops = 2.0 * m * k * n * planes  # int8 OPs per launch
        self.config = {"workload": "q8 product config[3] W1", "m": m, "k": k, "n": n, "planes": planes}
        self.dtype = "i8"

    def step(self, stream, ev=None):
        import ctypes as C
        from ava_amd import _lib

        L = _lib.lib()
        _lib.check(L.ava_q8_quant_rows(C.c_void_p(self.x.data_ptr()), self.m, self.k, self.planes,
                                       C.c_void_p(self.xq.data_ptr()), C.c_void_p(self.xe.data_ptr()), stream))
        if ev: ev[0].record()
        _lib.check(L.ava_q8_matmul_planes(C.c_void_p(self.xq.data_ptr()), C.c_void_p(self.xe.data_ptr()),
                                          self.planes, self.m, C.byref(self.qw.c), C.c_void_p(self.y.data_ptr()),
                                          stream))
        if ev: ev[1].record()

    def roofline(self, kernel_s):
        a = self.ops / kernel_s / 1e12
        return {"bound": "mfma", "achieved": a, "peak": I8_PEAK_TOPS, "unit": "TOP/s", "frac": a / I8_PEAK_TOPS}

    def extra(self):
        """The same integer work through the platform's library GEMM (torch._int_mm, hipBLASLt on ROCm):
        the planes stacked as rows, [P m, k] x [k, n] int8 -> int32 (no plane combine, no f32 output
        scaling), 5 launches; and its 8192-cube rate. A reference point for the product kernel only."""
        import torch

        out = {}
        try:
            a = self.xq.reshape(self.planes * self.m, -1)[:, :self.k].contiguous()
            b = self.qw.qt[:, :self.k].t() if hasattr(self.qw, "qt") else None
            if b is None:
                g = torch.Generator(device="cuda").manual_seed(4)
                b = torch.randint(-127, 128, (self.n, self.k), dtype=torch.int8, device="cuda", generator=g).t()
            for name, (x, y) in (("library_int_mm", (a, b)),
                                 ("library_int_mm_8192", (torch.ones((8192, 8192), dtype=torch.int8, device="cuda"),
                                                          torch.ones((8192, 8192), dtype=torch.int8,
                                                                     device="cuda").t()))):
                torch._int_mm(x, y)
                torch.cuda.synchronize()
                s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s0.record()
                for _ in range(5):
                    torch._int_mm(x, y)
                s1.record()
                torch.cuda.synchronize()
                ms = s0.elapsed_time(s1) / 5
                ops = 2.0 * x.shape[0] * x.shape[1] * y.shape[1]
                out[name] = {"ms": ms, "tops": ops / ms / 1e9, "shape": [x.shape[0], x.shape[1], y.shape[1]]}
        except Exception as ex:  # the reference point is optional
            out["library_int_mm_error"] = str(ex)
        return out

    def cpu_baseline(self):
        from oracle import oracle as O

        rng = np.random.default_rng(3)
        x = rng.standard_normal((1024, self.k)).astype(np.float32)
        q, s = O.quantize_int8((rng.standard_normal((self.k, self.n)) * 0.02).astype(np.float32))
        th = cpu_threads()
        rows, t0 = 0, time.perf_counter()
        while rows == 0 or time.perf_counter() - t0 < 3.0:  # calls of 1024 rows for about 3 s
            O.q8_matmul_ref(x, q, s, threads=th)
            rows += x.shape[0]
        dt = time.perf_counter() - t0
        return {"value": rows / dt, "unit": "rows/s", "cores": th, "kind": "port",
                "sample": f"oracle W8A32 product (int8.rs:301-331 fma chain, in int8/block.rs's 6 x 16 register blocks), "
                          f"{rows} rows, {dt:.2f} s"}


class Delta:
    """config[2]: the plain delta rule W += beta (v - W k) k^T, y = W q, chunks of 64: B=32, H=8, T=4096,
    d_k = d_v = 64; keys and queries N(0,1) then unit length, values N(0,1), beta = sigmoid(N(0,1)) per
    token and head, W_0 = 0."""

    name = "delta"
    metric = "tokens/sec chunked delta rule @B=32,H=8,T=4096,d=64, chunks of 64 (config[2]), 1 GPU; % fp32 MFMA roofline"
    warm_extend = True  # short, repeatable steps: warm up for WARM_S seconds
    kernel = "delta_inv_kernel + delta_seq_bf_kernel"  # the two-phase form (see __init__)

    def __init__(self, B=32, H=8, T=4096):
        import torch
        from ava_amd import _lib

        self.L = _lib.lib()
        BH = B * H
        self.BH, self.T = BH, T
        g = torch.Generator(device="cuda").manual_seed(5)
        n = lambda: torch.randn((BH, T, 64), device="cuda", generator=g)
        self.q, self.k, self.v = n(), n(), n()
        self.q /= self.q.norm(dim=2, keepdim=True)
        self.k /= self.k.norm(dim=2, keepdim=True)
        self.beta = torch.sigmoid(torch.randn((BH, T), device="cuda", generator=g))
        self.F = torch.zeros((BH, 64, 64), dtype=torch.float32, device="cuda")
        self.y = torch.empty_like(self.q)
        # the two-phase form's workspace (the chunks' inverses); AVA_DELTA_ONE_KERNEL=1 times the
        # single-kernel walk instead
        one = os.environ.get("AVA_DELTA_ONE_KERNEL", "0") != "0"
        self.work_bytes = 0 if one else self.L.ava_delta_chunk_workspace(BH, T)
        self.work = torch.empty(self.work_bytes, dtype=torch.uint8, device="cuda") if self.work_bytes else None
        self.kernel = "delta_plain_kernel" if one else "delta_inv_kernel + delta_seq_bf_kernel"
        self.tokens = B * T
        # read q, k, v, beta; write y and the final state
        self.bytes = 3 * BH * T * 64 * 4 + BH * T * 4 + BH * T * 64 * 4 + BH * 64 * 64 * 4
        self.config = {"workload": "delta rule chunked config[2]", "B": B, "H": H, "T": T, "d": 64, "chunk": 64,
                       "form": "one kernel" if one else "two-phase"}
        self.dtype = "f32"

    def step(self, stream, ev=None):
        import ctypes as C
        from ava_amd._lib import check

        p = lambda t: C.c_void_p(t.data_ptr())
        self.F.zero_()
        if ev: ev[0].record()
        check(self.L.ava_delta_chunk(p(self.q), p(self.k), p(self.v), None, p(self.beta), self.BH, self.T, 64,
                                     p(self.F), p(self.y), p(self.work) if self.work is not None else None,
                                     self.work_bytes, stream))
        if ev: ev[1].record()

    def roofline(self, kernel_s):
        # fp32-MFMA bound: the chunked form's work, 6 hs^2 + (5 c - 1) hs FLOPs per token and head
        # (c = 64), against the dense fp32 MFMA peak; the HBM rate of the same launch beside it
        hs, c = 64, 64
        flops = (6 * hs * hs + (5 * c - 1) * hs) * self.BH * self.T
        a = flops / kernel_s / 1e12
        return {"bound": "mfma", "achieved": a, "peak": F32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": a / F32_MFMA_PEAK_TFLOPS, "flops_per_launch": flops, "hbm_bytes_per_launch": self.bytes,
                "hbm_gbs": self.bytes / kernel_s / 1e9}

    def cpu_baseline(self):
        from oracle import oracle as O

        O.set_threads(1)
        BH, T = 8, 4096
        rng = np.random.default_rng(5)
        q, k, v = (rng.standard_normal((BH, T, 64)).astype(np.float32) for _ in range(3))
        q /= np.linalg.norm(q, axis=2, keepdims=True)
        k /= np.linalg.norm(k, axis=2, keepdims=True)
        beta = (1.0 / (1.0 + np.exp(-rng.standard_normal((BH, T, 1))))).astype(np.float32)
        t0 = time.perf_counter()
        O.mem_rec(q, k, k, v, np.zeros_like(beta), beta)
        dt = time.perf_counter() - t0
        return {"value": BH * T / dt / 8, "unit": "tokens/s (B x T per second, 8 heads per token)", "cores": 1,
                "kind": "port", "sample": f"oracle recurrence (mem_gen.rs:220-273 loop), {BH} of 256 heads, T={T}, "
                                          f"{dt:.2f} s"}


class LifBwd:
    """The LIF scan's backward at config[1]'s shape: cur ~N(0,1) [64, 2048, 2048] and dL/dspikes ~N(0,1),
    beta = sigmoid(U(1.5, 4.5)), theta 1, rho 0.95, gain 0.05; int2 spikes, ALIF, surrogate slope 4
    (gpu/model.rs:39 LIF_SLOPE), the reset gradient on. Outputs dL/dcur [64, 2048, 2048] and the
    per-stream state and parameter gradients."""

    name = "lif_bwd"
    metric = "tokens/sec LIF scan backward @B=64,T=2048,C=2048 (config[1] shape), 1 GPU; % HBM roofline"
    warm_extend = True  # short, repeatable steps: warm up for WARM_S seconds
    kernel = "lif_bwd_kernel"

    def __init__(self, B=64, T=2048, D=2048):
        import torch
        from ava_amd import _lib

        self.B, self.T, self.D = B, T, D
        self.L = _lib.lib()
        g = torch.Generator(device="cuda").manual_seed(11)
        self.cur = torch.randn((B, T, D), device="cuda", generator=g, dtype=torch.float32)
        self.g = torch.randn((B, T, D), device="cuda", generator=g, dtype=torch.float32)
        beta = torch.sigmoid(torch.rand(D, device="cuda", generator=g) * 3.0 + 1.5)
        self.ps = torch.cat([beta, torch.ones(D, dtype=torch.float32, device="cuda"), torch.full((D,), 0.95, dtype=torch.float32, device="cuda"),
                             torch.full((D,), 0.05, dtype=torch.float32, device="cuda")]).contiguous()
        self.z = torch.zeros((B, D), dtype=torch.float32, device="cuda")
        self.out = [torch.empty((B, D), dtype=torch.float32, device="cuda") for _ in range(5)]
        self.dI = torch.empty_like(self.cur)
        self.tokens = B * T
        # algorithmic bytes: read cur and dL/dspikes, write dL/dcur; per (b, c) the initial state and the
        # final-state gradients in, five gradients out; the parameter rows
        self.bytes = B * T * D * 12 + B * D * 4 * (5 + 5) + 4 * D * 4
        self.config = {"workload": "lif_scan backward config[1]", "B": B, "T": T, "C": D, "spikes": "int2",
                       "alif": True, "slope": 4.0, "reset_grad": True}
        self.dtype = "f32"

    def step(self, stream, ev=None):
        from ava_amd._lib import check
        import ctypes as C

        p = lambda t: C.c_void_p(t.data_ptr())
        z = p(self.z)
        if ev: ev[0].record()
        check(self.L.ava_lif_scan_bwd(p(self.cur), self.B, self.T, self.D, p(self.ps), z, z, z, 2, 1, 1, 4.0, 1,
                                      p(self.g), z, z, p(self.dI), *(p(o) for o in self.out), stream))
        if ev: ev[1].record()

    def roofline(self, kernel_s):
        a = self.bytes / kernel_s / 1e9
        return {"bound": "hbm", "achieved": a, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": a / HBM_PEAK_GBS,
                "note": "algorithmic 12 B per element; the kernel reads the currents twice (16 B)"}

    def cpu_baseline(self):
        from oracle import oracle as O

        O.set_threads(1)
        B = self.B  # the whole workload: about 5 s on one thread
        rng = np.random.default_rng(11)
        cur = rng.standard_normal((B, self.T, self.D), dtype=np.float32)
        g = rng.standard_normal((B, self.T, self.D), dtype=np.float32)
        beta = (1.0 / (1.0 + np.exp(-rng.uniform(1.5, 4.5, self.D)))).astype(np.float32)
        ps = np.concatenate([beta, np.ones(self.D), np.full(self.D, 0.95), np.full(self.D, 0.05)]).astype(np.float32)
        t0 = time.perf_counter()
        O.lif_bwd(cur, ps, g, levels=2, signed=True, alif=True, slope=4.0, reset_grad=True)
        dt = time.perf_counter() - t0
        return {"value": B * self.T / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
                "sample": f"oracle lif_bwd (lifg_bwd's recurrence, gpu/lif.cu:3228-3290, restated), B={B} of {self.B}, "
                          f"T={self.T}, C={self.D}, one thread, {dt:.2f} s"}


class MemBwd:
    """The fast-weight memory's backward at config[3]'s block shape: 64 streams x 16 heads of 64 over
    T = 2048, per-channel gates, momentum 0.5; unit q, k, e, v ~N(0,1), alpha ~U(0.85, 0.999),
    b ~U(0.1, 1.9), dL/dy ~N(0,1), from a zero state."""

    name = "mem_bwd"
    metric = "tokens/sec fast-weight memory backward @64 streams x 16 heads x 2048 (config[3] block), 1 GPU"
    warm_extend = True  # short, repeatable steps: warm up for WARM_S seconds
    kernel = "mem_bwd_kernel"

    def __init__(self, B=64, H=16, T=2048):
        import torch
        from ava_amd import _lib

        BH = B * H
        self.BH, self.T = BH, T
        self.L = _lib.lib()
        g = torch.Generator(device="cuda").manual_seed(12)

        def unit():
            x = torch.randn((BH, T, 64), device="cuda", generator=g)
            return (x / x.norm(dim=2, keepdim=True)).contiguous()

        self.q, self.k, self.e = unit(), unit(), unit()
        self.v = torch.randn((BH, T, 64), device="cuda", generator=g)
        self.la = torch.log(torch.rand((BH, T, 64), device="cuda", generator=g) * 0.149 + 0.85)
        self.b = torch.rand((BH, T, 64), device="cuda", generator=g) * 1.8 + 0.1
        self.dy = torch.randn((BH, T, 64), device="cuda", generator=g)
        self.out = [torch.empty((BH, T, 64), dtype=torch.float32, device="cuda") for _ in range(6)]
        self.dF0 = torch.empty((BH, 64, 64), dtype=torch.float32, device="cuda")
        self.dS0 = torch.empty((BH, 64, 64), dtype=torch.float32, device="cuda")
        self.work_bytes = self.L.ava_mem_scan_bwd_workspace(BH, T, 1)
        self.work = torch.empty(self.work_bytes, dtype=torch.uint8, device="cuda")
        self.tokens = B * T
        # algorithmic bytes per (head, token): q, k, e, v, log alpha, b, dy in; dq, dk, de, dv, dla, db out
        self.bytes = BH * T * 64 * 4 * 13
        # FLOPs per (head, token, element): the step replayed (~9) and walked back (~21)
        self.flops = BH * T * 64 * 64 * 30
        self.config = {"workload": "memory backward config[3] block", "B": B, "heads": H, "T": T, "hs": 64,
                       "gates": "per channel", "momentum": 0.5}
        self.dtype = "f32"

    def step(self, stream, ev=None):
        from ava_amd._lib import check
        import ctypes as C

        p = lambda t: C.c_void_p(t.data_ptr())
        if ev: ev[0].record()
        check(self.L.ava_mem_scan_bwd(p(self.q), p(self.k), p(self.e), p(self.v), p(self.la), p(self.b), self.BH,
                                      self.T, 64, 64, 0.5, 1e5, None, None, p(self.dy), None, None,
                                      *(p(o) for o in self.out), p(self.dF0), p(self.dS0), p(self.work),
                                      self.work_bytes, stream))
        if ev: ev[1].record()

    def roofline(self, kernel_s):
        a = self.bytes / kernel_s / 1e9
        return {"bound": "hbm", "achieved": a, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": a / HBM_PEAK_GBS,
                "vector_tflops": self.flops / kernel_s / 1e12, "vector_peak_tflops": FP32_PEAK_TFLOPS,
                "workspace_bytes": self.work_bytes,
                "note": "a recurrence walked twice per head: latency-bound, not bandwidth-bound"}

    def cpu_baseline(self):
        from oracle import oracle as O

        O.set_threads(1)
        BH, T = 256, self.T  # a quarter of the heads: about 12 s on one thread
        rng = np.random.default_rng(12)

        def unit():
            x = rng.standard_normal((BH, T, 64)).astype(np.float32)
            return x / np.linalg.norm(x, axis=2, keepdims=True)

        q, k, e = unit(), unit(), unit()
        v = rng.standard_normal((BH, T, 64)).astype(np.float32)
        la = np.log(rng.uniform(0.85, 0.999, (BH, T, 64))).astype(np.float32)
        b = rng.uniform(0.1, 1.9, (BH, T, 64)).astype(np.float32)
        dy = rng.standard_normal((BH, T, 64)).astype(np.float32)
        t0 = time.perf_counter()
        O.mem_rec_bwd(q, k, e, v, la, b, dy, m=0.5)
        dt = time.perf_counter() - t0
        return {"value": BH * T / dt / 16, "unit": "tokens/s (B x T per second, 16 heads per token)", "cores": 1,
                "kind": "port", "sample": f"oracle memory backward (delta_rec's gradient, float64), {BH} of {self.BH} "
                                          f"heads, T={T}, one thread, {dt:.2f} s"}


class Train:
    """The float32 training step (ava_train_step) on config[3]'s model: the loss and every parameter's
    gradient of a teacher-forced batch of B x T random tokens from a zero state (the reference's
    hand-written step, gpu/model/fwin.rs). Random-init f32 weights N(0, 0.02) as synth.params."""

    name = "train"
    kernel = "whole training step"
    metric = "tokens/sec f32 training step (loss and gradients) of config[3]'s model, 1 GPU; % fp32 MFMA roofline"
    default_steps = 3

    def __init__(self, B=4, T=2048):
        import torch
        from ava_amd import synth
        from ava_amd.train import Trainer

        self.cfg = c = synth.config("ava04_d1024")
        self.B, self.T = B, T
        log("bench: building weights")
        prm = synth.params(c, seed=0)
        self.tr = Trainer(c, slope=4.0)
        self.flat = self.tr.pack(prm)
        self.grads = torch.empty_like(self.flat)
        g = torch.Generator(device="cuda").manual_seed(6)
        self.ids = torch.randint(0, c["vocab"], (B, T), device="cuda", generator=g, dtype=torch.int32)
        self.tgt = torch.randint(0, c["vocab"], (B, T), device="cuda", generator=g, dtype=torch.int32)
        self.tokens = B * T
        d, H, V, L, r = c["d"], c["hidden"], c["vocab"], c["layers"], c["gate_rank"]
        nh = d // c["head_size"]
        # the step's product FLOPs: forward 2 N P, backward 4 N P over the matrices' P multiply-adds per
        # token (8 d^2 + 2 d H + 2 d nh + 4 d r per block, the engram's 4 d de, the head d V)
        P = L * (8 * d * d + 2 * d * H + 2 * d * nh + 4 * d * r) + 4 * d * c["eng_dim"] + d * V
        self.flops = 6.0 * self.tokens * P
        self.config = {"workload": "f32 training step config[3] model", "B": B, "T": T, "d": d, "blocks": L,
                       "hidden": H, "vocab": V, "engram_block": c["eng_block"]}
        self.dtype = "f32"

    def step(self, stream, ev=None):
        if ev: ev[0].record()
        self.tr.step(self.flat, self.ids, self.tgt, self.grads)
        if ev: ev[1].record()

    def roofline(self, kernel_s):
        a = self.flops / kernel_s / 1e12
        return {"bound": "mfma", "achieved": a, "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": a / FP32_PEAK_TFLOPS, "scope": "the step's product FLOPs over the whole step's time",
                "product_flops_per_step": self.flops}

    def cpu_baseline(self):
        return None


class MemChunk:
    """The chunked fast-weight memory (ava_mem_chunk, delta_chunk / chunk_core) at config[3]'s per-block
    shape: 64 streams x 16 heads x 2048 tokens, unit q, k, e, v ~N(0,1), per-channel log alpha =
    log U(0.85, 0.999), b ~U(0.1, 1.9), momentum 0.5, from a zero state. The token loop (ava_mem_scan) on
    the same inputs is timed beside it. The state contractions run as bf16 products of three-term splits
    (mem_chunk_bf_kernel); AVA_MEM_CHUNK_FP32=1 runs them on the f32 matrix cores (mem_chunk_kernel). The
    FLOPs are priced at the fp32 peak either way: the arithmetic is f32's."""

    name = "mem_chunk"
    metric = "tokens/sec chunked fast-weight memory @64 streams x 16 heads x 2048 (config[3] block), 1 GPU; % fp32 MFMA roofline"
    warm_extend = True  # short, repeatable steps: warm up for WARM_S seconds
    kernel = "mem_chunk_kernel" if os.environ.get("AVA_MEM_CHUNK_FP32") == "1" else "mem_chunk_bf_kernel"

    def __init__(self, B=64, H=16, T=2048):
        import torch
        from ava_amd import _lib

        BH = B * H
        self.BH, self.T = BH, T
        self.L = _lib.lib()
        g = torch.Generator(device="cuda").manual_seed(13)

        def unit():
            x = torch.randn((BH, T, 64), device="cuda", generator=g)
            return (x / x.norm(dim=2, keepdim=True)).contiguous()

        self.q, self.k, self.e = unit(), unit(), unit()
        self.v = torch.randn((BH, T, 64), device="cuda", generator=g)
        self.la = torch.log(torch.rand((BH, T, 64), device="cuda", generator=g) * 0.149 + 0.85)
        self.b = torch.rand((BH, T, 64), device="cuda", generator=g) * 1.8 + 0.1
        self.F = torch.zeros((BH, 64, 64), dtype=torch.float32, device="cuda")
        self.S = torch.zeros_like(self.F)
        self.y = torch.empty_like(self.q)
        self.tokens = B * T
        # per chunk of 16 and head: the contractions with F and S (32 x 128 x 64 and 128 x 32 x 64 MACs)
        # and the intra-chunk products Ke V, Qw V, Qa R (3 x 16 x 16 x 64), 2 FLOPs per MAC
        self.flops = BH * (T // 16) * 2 * (2 * 32 * 128 * 64 + 3 * 16 * 16 * 64)
        self.bytes = BH * T * 64 * 4 * 7 + 2 * 2 * BH * 64 * 64 * 4  # 6 inputs + y; F, S in and out
        self.config = {"workload": "memory forward chunked config[3] block", "B": B, "heads": H, "T": T, "hs": 64,
                       "gates": "per channel", "momentum": 0.5, "chunk": 16,
                       "contractions": "f32 MFMA" if MemChunk.kernel == "mem_chunk_kernel" else "bf16 MFMA, 3-term splits"}
        self.dtype = "f32"

    def _run(self, fn, stream):
        import ctypes as C
        from ava_amd._lib import check

        p = lambda t: C.c_void_p(t.data_ptr())
        self.F.zero_()
        self.S.zero_()
        check(fn(p(self.q), p(self.k), p(self.e), p(self.v), p(self.la), p(self.b), self.BH, self.T, 64, 64, 0.5, 1e5,
                 p(self.F), p(self.S), p(self.y), stream))

    def step(self, stream, ev=None):
        # the events bracket the launch only (the state is cleared before)
        import ctypes as C
        from ava_amd._lib import check

        p = lambda t: C.c_void_p(t.data_ptr())
        self.F.zero_()
        self.S.zero_()
        if ev: ev[0].record()
        check(self.L.ava_mem_chunk(p(self.q), p(self.k), p(self.e), p(self.v), p(self.la), p(self.b), self.BH,
                                   self.T, 64, 64, 0.5, 1e5, p(self.F), p(self.S), p(self.y), stream))
        if ev: ev[1].record()

    def roofline(self, kernel_s):
        a = self.flops / kernel_s / 1e12
        return {"bound": "mfma", "achieved": a, "peak": F32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": a / F32_MFMA_PEAK_TFLOPS, "flops_per_launch": self.flops, "hbm_bytes_per_launch": self.bytes,
                "hbm_gbs": self.bytes / kernel_s / 1e9}

    def extra(self):
        # the token loop on the same inputs, same stream, 5 launches
        import torch

        st = torch.cuda.current_stream()
        sp = __import__("ctypes").c_void_p(st.cuda_stream)
        self._run(self.L.ava_mem_scan, sp)
        torch.cuda.synchronize()
        ms = []
        for _ in range(5):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            self._run(self.L.ava_mem_scan, sp)
            b.record()
            torch.cuda.synchronize()
            ms.append(a.elapsed_time(b))
        return {"token_loop_ms": float(np.median(ms)), "token_loop_kernel": "mem_scan_kernel"}

    def cpu_baseline(self):
        from oracle import oracle as O

        O.set_threads(1)
        BH, T = 256, self.T  # a quarter of the 1024 heads: about 12 s on one thread
        rng = np.random.default_rng(13)

        def unit():
            x = rng.standard_normal((BH, T, 64)).astype(np.float32)
            return x / np.linalg.norm(x, axis=2, keepdims=True)

        q, k, e = unit(), unit(), unit()
        v = rng.standard_normal((BH, T, 64)).astype(np.float32)
        la = np.log(rng.uniform(0.85, 0.999, (BH, T, 64))).astype(np.float32)
        b = rng.uniform(0.1, 1.9, (BH, T, 64)).astype(np.float32)
        t0 = time.perf_counter()
        O.mem_chunk(q, k, e, v, la, b, m=0.5)
        dt = time.perf_counter() - t0
        return {"value": BH * T / dt / 16, "unit": "tokens/s (B x T per second, 16 heads per token)", "cores": 1,
                "kind": "port", "sample": f"oracle chunked memory (chunk_core, arch.rs:1243-1327), {BH} of {self.BH} "
                                          f"heads, T={T}, one thread, {dt:.2f} s"}


class Copy:
    """A plain 1 GiB device-to-device copy: the calibration kernel for the FETCH/WRITE_SIZE counters."""

    name = "copy"
    metric = "calls/sec 1 GiB device copy (counter calibration), 1 GPU; % HBM roofline"
    unit = "calls/s"
    warm_extend = True  # short, repeatable steps: warm up for WARM_S seconds
    kernel = "copy"

    def __init__(self, nbytes=1 << 30):
        import torch

        self.src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
        self.dst = torch.empty_like(self.src)
        self.tokens = 1
        self.bytes = 2 * nbytes
        self.config = {"workload": "device copy calibration", "bytes": nbytes}
        self.dtype = "f32"

    def step(self, stream, ev=None):
        if ev: ev[0].record()
        self.dst.copy_(self.src)
        if ev: ev[1].record()

    def roofline(self, kernel_s):
        a = self.bytes / kernel_s / 1e9
        return {"bound": "hbm", "achieved": a, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": a / HBM_PEAK_GBS}

    def cpu_baseline(self):
        return None


class Stack:
    """config[3]: the Ava-0.4-shaped int8 block stack, teacher-forced prefill of B=64 x T=2048 token
    ids (uniform over vocab 8192) from a fresh state; d=1024, 8 blocks, wide 4096 with kWTA 1024,
    16 memory heads of 64 (per-channel gates, erase key, momentum 0.5), the engram read in block 4;
    random-init weights N(0, 0.02) quantized to int8 per output column. Outputs: logits [B*T, 8192]
    f32, the final membranes and fast-weight states."""

    name = "stack"
    kernel = "q8_gemm"

    def __init__(self, B=64, T=2048, cfg_name="ava04_d1024", planes=3):
        import torch
        from ava_amd import synth
        from ava_amd.model import Model

        self.cfg = synth.config(cfg_name)
        c = self.cfg
        self.B, self.T, self.planes = B, T, planes
        log("bench: building weights")
        self.params = synth.params(c, seed=0)
        self.model = Model(c, self.params, planes=planes)
        self.st = self.model.state(B, eng_cap=T)
        g = torch.Generator(device="cuda").manual_seed(4)
        self.ids = torch.randint(0, c["vocab"], (B, T), device="cuda", generator=g, dtype=torch.int32)
        self.logits = torch.empty((B * T, c["vocab"]), dtype=torch.float32, device="cuda")
        self.tokens = B * T
        d, H, V, L = c["d"], c["hidden"], c["vocab"], c["layers"]
        # algorithmic int8 work per forward (2 ops per multiply-add): 16 d^2 per token per block
        # (Win, Wout, Wq, Wk, Wv, We, Wg, Wo: 8 d^2; W1, W2: 8 d^2), the engram's 4 d de, the head d V
        self.ops = 2.0 * self.tokens * (L * 16 * d * d + 4 * d * c["eng_dim"] + d * V)
        self.config = {"workload": "int8 block stack config[3]", "B": B, "T": T, "d": d, "blocks": L, "hidden": H,
                       "kwta_k": c["kwta_k"], "heads": d // c["head_size"], "head_size": c["head_size"], "vocab": V,
                       "engram_block": c["eng_block"], "momentum": c["momentum"], "act_planes": planes}
        self.dtype = "i8"
        self.breakdown = None
        # MFMA work actually executed: the dense products run their activations as `planes` int8
        # planes (one i8 pass each), the spike product (Wout) one pass
        P = planes
        self.exec_ops = 2.0 * self.tokens * (L * (P * 15 + 1) * d * d + P * 4 * d * c["eng_dim"] + P * d * V)
        # HBM bytes per q8 product launch, the mean over one forward's 51 launches, measured with
        # rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE on this workload (2.0 x FETCH_SIZE + WRITE_SIZE,
        # KiB; the factor from the 1 GiB copy kernel of --workload copy)
        self.traffic = 2.746e9

    def _reset(self):
        st = self.st
        for t in (st.lif_v, st.lif_s, st.lif_a, st.mem_f, st.mem_s):
            t.zero_()
        st.eng_len = 0

    def step(self, stream, ev=None):
        self._reset()
        self.model.forward_with_state(self.ids, self.st, self.logits)

    def start_timed(self):
        self.model.timing(reset=True)
        self.model.set_timing(True)

    def kernel_ms(self):
        t = self.model.timing(reset=True)
        self.model.set_timing(False)
        self.breakdown = {k: {"calls": v[0], "ms": round(v[1], 3)} for k, v in sorted(t.items(), key=lambda kv: -kv[1][1])}
        calls, ms = t["q8_gemm"]
        self.gemm_calls, self.gemm_ms_total = calls, ms
        return [ms]  # summed over the timed steps; divided by steps in roofline()

    def roofline(self, kernel_s):
        per_fwd = kernel_s / self.nsteps
        a = self.ops / per_fwd / 1e12
        x = self.exec_ops / per_fwd / 1e12
        return {"bound": "mfma", "achieved": a, "peak": I8_PEAK_TOPS, "unit": "TOP/s", "frac": a / I8_PEAK_TOPS,
                "executed": x, "executed_frac": x / I8_PEAK_TOPS, "executed_ops_per_forward": self.exec_ops,
                "algorithmic_ops_per_forward": self.ops, "gemm_ms_per_forward": per_fwd * 1e3,
                "kernel_calls_per_forward": self.gemm_calls // self.nsteps,
                "kernel_avg_us": self.gemm_ms_total * 1e3 / self.gemm_calls}

    def extra(self):
        return {"breakdown_ms_total": self.breakdown}

    def cpu_baseline(self):
        from oracle import oracle as O

        B, T = 2, 2048  # 4096 tokens: a few seconds on the box's 16 threads
        th = cpu_threads()
        O.set_threads(th)
        om = O.OracleModel(self.cfg, self.params)
        ids = np.random.default_rng(4).integers(0, self.cfg["vocab"], (B, T)).astype(np.int32)
        t0 = time.perf_counter()
        om.forward(ids, state=om.new_state(B, eng_cap=T), planes=0, threads=th)
        dt = time.perf_counter() - t0
        return {"value": B * T / dt, "unit": "tokens/s", "cores": th, "kind": "port",
                "sample": f"oracle block-stack forward with the reference's W8A32 products (int8.rs:301-331 fma chain, "
                          f"int8/block.rs's 6 x 16 register blocks from 6 rows) on "
                          f"config[3]'s model, B={B}, T={T}, {th} threads for the products, {dt:.2f} s"}


class Greedy:
    """config[0]: the reference's own CPU-runnable case. Ava-0.4-shaped int8 model with d=512 (8 blocks,
    wide 2048 with kWTA 512, 8 memory heads of 64, the single-head engram read in block 4), vocab 8192,
    random-init weights; one stream: a prompt of 512 ids, then 128 greedy steps (argmax, the lowest id
    on ties) with carried state (Model.generate, generate in gpu/state.rs:1392-1458). A step is the
    whole generation; value = generated tokens per second. Latency-bound: one token's int8 weights
    and state are ~46 MB, under 6 µs of HBM time, against ~110 launches per token."""

    name = "greedy"
    kernel = "whole_step"
    metric = "tokens/sec greedy decode @B=1, 512-token prompt + 128 steps (config[0]), 1 GPU; % HBM roofline"
    default_steps = 3

    def __init__(self, prompt=512, new=128, planes=3):
        from ava_amd import synth
        from ava_amd.model import Model

        self.cfg = c = synth.config("ava04_d512")
        self.prompt_len, self.new = prompt, new
        log("bench: building weights")
        self.params = synth.params(c, seed=0)
        self.model = Model(c, self.params, planes=planes)
        self.prompt = np.random.default_rng(7).integers(0, c["vocab"], prompt).tolist()
        self.tokens = new
        d, H, V, L, nh = c["d"], c["hidden"], c["vocab"], c["layers"], c["d"] // c["head_size"]
        # bytes per generated token: the int8 weights (16 d^2 per block, the engram's 4 d 64, the head
        # d V, each with 4-byte column scales), LIF state r/w (3 [d] f32), F and S r/w ([nh][64][64] f32
        # each), the engram's keys and values read (prompt + half the steps on average, 64 f32 each),
        # the logits row written
        w = L * 16 * d * d + 4 * d * c["eng_dim"] + d * V
        self.bytes_per_token = (w + 4 * (L * 16 * d + 4 * c["eng_dim"] + V) + L * 3 * d * 4 * 2
                                + L * nh * 64 * 64 * 4 * 2 * 2 + (prompt + new // 2) * 64 * 4 * 2 + V * 4)
        self.config = {"workload": "greedy generation config[0]", "B": 1, "prompt": prompt, "steps": new, "d": d,
                       "blocks": L, "hidden": H, "kwta_k": c["kwta_k"], "vocab": V, "act_planes": planes}
        self.dtype = "i8"
        self.out = None

    def step(self, stream, ev=None):
        self.out = self.model.generate([self.prompt], self.new, eos=None)[0]  # config[0]: 128 steps

    def kernel_ms(self):
        return [self.wall * 1e3 / self.nsteps]  # the whole generation, per step

    def roofline(self, kernel_s):
        per_token = kernel_s / self.new
        a = self.bytes_per_token / per_token / 1e9
        return {"bound": "hbm", "achieved": a, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": a / HBM_PEAK_GBS,
                "bytes_per_token": self.bytes_per_token, "ms_per_token": per_token * 1e3,
                "note": "whole generation (prefill included) over its wall time; latency-bound"}

    def cpu_baseline(self):
        from oracle import oracle as O

        new = self.new  # the same generation: the prompt's pass and 128 greedy steps
        th = cpu_threads()
        O.set_threads(th)
        om = O.OracleModel(self.cfg, self.params)
        t0 = time.perf_counter()
        st = om.new_state(1, eng_cap=self.prompt_len + new)
        lg, st, _ = om.forward(np.asarray([self.prompt], np.int32), state=st, planes=0, threads=th)
        last = lg[-1]
        for _ in range(new - 1):
            lg, st, _ = om.forward(np.asarray([[int(np.argmax(last))]], np.int32), state=st, planes=0, threads=th)
            last = lg[-1]
        dt = time.perf_counter() - t0
        return {"value": new / dt, "unit": "tokens/s", "cores": th, "kind": "port",
                "sample": f"oracle greedy loop with the reference's W8A32 products (int8.rs:301-331; the prompt in "
                          f"int8/block.rs's 6 x 16 register blocks) on config[0]'s "
                          f"model: the {self.prompt_len}-token prompt and {new} steps, {th} threads, {dt:.2f} s "
                          f"(prefill included, as in the GPU figure; the same tokens are not checked here)"}


class StackHeads(Stack):
    """config[3] with the engram read at the reference's geometry (gpu/memory.rs:610-700): 32 heads of
    32 over the whole width (Wq, Wk, Wv, Wo 1024 x 1024) and an f32 store, instead of BASELINE's one
    head of 64. Not the headline line: it shows what the reference's own engram costs on this path."""

    name = "stack_heads"
    metric = "tokens/sec int8 block-stack forward @B=64,T=2048, engram of 32 heads of 32, 1 GPU; % HBM / MFMA roofline"

    def __init__(self, B=64, T=2048, planes=3):
        super().__init__(B=B, T=T, cfg_name="ava04_d1024_heads", planes=planes)
        self.config.update(workload="int8 block stack config[3], engram of 32 heads of 32",
                           engram_heads=self.cfg["eng_heads"], engram_dim=self.cfg["eng_dim"])
        self.traffic = None  # the counter runs cover the headline workload


class Decode:
    """config[4]: batched stateful decode. B=256 streams of config[3]'s model with the cerebellum head
    (12,288 granule units, 384 kept, per-stream online table with a 256-token half-life). Each stream's
    state (membranes, thresholds, fast weights and momentum, the engram store) comes from a
    teacher-forced prefill of `prefill` random tokens (32,768 as config[4]; untimed, in pieces of
    `piece` tokens). A step is one token per stream: the forward (T = 1) to logits [256, 8192] and
    one online table step on each stream's next token (random ids: a teacher-forced continuation)."""

    name = "decode"
    kernel = "attend_split"
    metric = "tokens/sec batched stateful int8 decode @B=256 streams, 32768-token state (config[4]), 1 GPU; % HBM roofline"
    default_steps = 256

    def __init__(self, B=256, prefill=32768, piece=512, steps_cap=1100, planes=3):
        import torch
        from ava_amd import synth
        from ava_amd.model import Model

        self.cfg = c = synth.config("ava04_d1024_decode")
        self.prefill = prefill = int(os.environ.get("AVA_DECODE_PREFILL", prefill))
        self.B, self.planes = B, planes
        log("bench: building weights")
        self.params = synth.params(c, seed=0)
        self.model = Model(c, self.params, planes=planes)
        self.st = self.model.state(B, eng_cap=prefill + steps_cap, device_len=True)
        g = torch.Generator(device="cuda").manual_seed(5)
        V = c["vocab"]
        self.toks = torch.randint(0, V, (steps_cap + 1, B, 1), device="cuda", generator=g, dtype=torch.int32)
        self.nexts = self.toks[1:, :, 0].contiguous()
        # the step's inputs live in fixed buffers so that it can be captured and replayed; the logits
        # and next buffers alternate between steps, as the overlapped step learns from the previous
        # step's pair while this step's forward writes the other
        self.logits2 = [torch.empty((B, V), dtype=torch.float32, device="cuda") for _ in range(2)]
        self.nxt2 = [torch.empty(B, dtype=torch.int32, device="cuda") for _ in range(2)]
        self.logits, self.nxt_buf = self.logits2[0], self.nxt2[0]
        self.nats = torch.empty(B, dtype=torch.float64, device="cuda")
        self.ids_buf = torch.empty((B, 1), dtype=torch.int32, device="cuda")
        # AVA_DECODE_GRAPH=1 replays the step as a captured HIP graph (the same bits; measured about 1%
        # slower than eager launches on this ROCm, so off by default)
        self.use_graph = os.environ.get("AVA_DECODE_GRAPH", "0") != "0"
        # AVA_DECODE_OVERLAP=1: overlapped steps (Model.decode_step), step t running the table step of
        # token t - 1 beside the forward of token t. Off by default: on this box the two streams'
        # kernels land on one hardware queue and run in turn (measured 1% slower than in order).
        self.overlap = os.environ.get("AVA_DECODE_OVERLAP", "0") != "0"
        self.graph = None
        self.graphs = None
        self.t = 0
        self.steps_cap = steps_cap
        t0 = time.perf_counter()
        done = 0
        while done < prefill:
            n = min(piece, prefill - done)
            ids = torch.randint(0, V, (B, n), device="cuda", generator=g, dtype=torch.int32)
            self.model.forward_with_state(ids, self.st, want_logits=False)
            done += n
        torch.cuda.synchronize()
        log(f"bench: prefill of {prefill} tokens x {B} streams in {time.perf_counter() - t0:.1f} s")
        self.tokens = B
        d, H, L, de = c["d"], c["hidden"], c["layers"], c["eng_dim"]
        nh = d // c["head_size"]
        self.config = {"workload": "stateful decode config[4]", "streams": B, "prefill": prefill, "d": d,
                       "blocks": L, "hidden": H, "kwta_k": c["kwta_k"], "heads": nh, "vocab": V,
                       "engram_block": c["eng_block"], "engram_store": "fp16" if c.get("eng_half") else "f32",
                       "cb_units": c["cb_units"], "cb_half": c["cb_half"], "momentum": c["momentum"],
                       "act_planes": planes, "hip_graph": self.use_graph, "overlapped_table_step": self.overlap}
        self.dtype = "i8"
        self.breakdown = None

    def step_bytes(self):
        """Algorithmic HBM bytes of one step at the current store length: int8 weights, the carried
        state read and written (LIF v, s, a; F and S), the engram keys and values read, the step's keys
        and values written, the online table rows of the kept units read (apply) and read + written
        (learn), the code, the logits, E read by the learning step."""
        c, B = self.cfg, self.B
        d, H, L, V, de, G = c["d"], c["hidden"], c["layers"], c["vocab"], c["eng_dim"], c["cb_units"]
        w = L * 16 * d * d + 4 * d * de + d * V
        lif = L * B * d * 4 * 3 * 2
        fs = L * B * d * c["head_size"] * 4 * 2 * 2
        n = self.st.eng_len
        ek = 2 if c.get("eng_half") else 4  # the store's element (fp16 for config[4])
        kv = B * (n + 1) * de * ek * 2 + B * de * ek * 2
        kept = G // 32
        cb = B * kept * d * 4 * 3 + B * G * 4 * 2
        out = B * V * 4 * 2 + V * d * 4
        return w + lif + fs + kv + cb + out

    def step(self, stream, ev=None, eager=False):
        if self.t >= self.steps_cap:
            raise RuntimeError("decode: more steps than the store was sized for")
        if self.overlap:
            return self.step_overlapped(eager)
        self.ids_buf.copy_(self.toks[self.t])
        self.nxt_buf.copy_(self.nexts[self.t])
        if self.graph is not None and not eager:
            self.graph.replay()
        else:
            self.model.forward_with_state(self.ids_buf, self.st, self.logits)
            self.model.cb_learn(self.logits, self.nxt_buf, self.st, nats=self.nats)
            if self.use_graph and self.graph is None:
                # captured after the first eager step (scratch allocated): every later step replays it
                self.graph = self.model.capture_decode(self.st, self.ids_buf, self.logits, self.nxt_buf, self.nats)
        self.t += 1

    def step_overlapped(self, eager):
        """Token t's forward with token t - 1's table step beside it (none at t = 0). Both graphs are
        captured after two eager steps (the second allocates the table step's scratch)."""
        t, m = self.t, self.model
        cur, prev = t % 2, (t - 1) % 2
        self.ids_buf.copy_(self.toks[t])
        self.nxt2[cur].copy_(self.nexts[t])
        if self.graphs is not None and not eager:
            self.graphs[prev].replay()  # graph p learns from buffer p and writes buffer 1 - p
        elif t == 0:
            m.decode_step(self.ids_buf, self.st, self.logits2[cur])
        else:
            m.decode_step(self.ids_buf, self.st, self.logits2[cur], self.logits2[prev], self.nxt2[prev], self.nats)
            if self.use_graph and self.graphs is None:
                self.graphs = [m.capture_decode_step(self.st, self.ids_buf, self.logits2[1 - p], self.logits2[p],
                                                     self.nxt2[p], self.nats) for p in (0, 1)]
        self.t += 1

    prof_steps = 8

    def start_timed(self):
        self.bytes0 = self.step_bytes()

    def kernel_ms(self):
        # A step is ~150 short launches, so the per-launch event pairs of the launch timer would
        # lengthen it: the timed steps run without them, and the breakdown comes from prof_steps more
        # steps with the timer on, after the timed region.
        import torch
        self.model.timing(reset=True)
        self.model.set_timing(True)
        for _ in range(self.prof_steps):
            self.step(None, eager=True)
        torch.cuda.synchronize()
        t = self.model.timing(reset=True)
        self.model.set_timing(False)
        self.breakdown = {k: {"calls": v[0], "ms_per_step": round(v[1] / self.prof_steps, 4)}
                          for k, v in sorted(t.items(), key=lambda kv: -kv[1][1])}
        calls, ms = t.get("attend", (1, 0.0))
        self.att_calls, self.att_ms = calls, ms
        return [ms]

    def roofline(self, kernel_s):
        # the whole step is HBM-bound: algorithmic bytes per step over the measured step time
        per = self.wall / self.nsteps
        b = 0.5 * (self.bytes0 + self.step_bytes())
        a = b / per / 1e9
        return {"bound": "hbm", "achieved": a, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": a / HBM_PEAK_GBS,
                "algorithmic_bytes_per_step": b, "scope": "whole decode step",
                "kernel_avg_us": self.att_ms * 1e3 / max(self.att_calls, 1)}

    def extra(self):
        return {"breakdown": self.breakdown, "breakdown_note": f"launch-timer sums over {self.prof_steps} steps "
                "after the timed region, per step"}

    def cpu_baseline(self):
        """The oracle's decode step (forward of one token with the reference's W8A32 products, then the
        table's learning step) on a subset of the streams, from the GPU's state after the prefill and
        the timed steps, reported per stream-step (the reference's talking engine runs one stream per
        call, gpu/model/fstep/arch.rs:525-1073)."""
        import torch
        from oracle import oracle as O

        S = 4
        th = cpu_threads()
        O.set_threads(th)
        sub = self.st.select(list(range(S)))
        om = O.OracleModel(self.cfg, self.params)
        n = self.st.eng_len
        so = om.new_state(S, eng_cap=n + 64)
        for k in ("lif_v", "lif_s", "lif_a", "mem_f", "mem_s"):
            so[k][...] = getattr(sub, k).cpu().numpy()
        for k in ("eng_k", "eng_v"):
            so[k][:, :n] = getattr(sub, k)[:, :n].float().cpu().numpy()
        so["eng_len"] = n
        so["cb_tab"][...] = sub.cb_tab.cpu().numpy()
        so["cb_scale"][...] = sub.cb_scale.cpu().numpy()
        so["cb_code"][...] = sub.cb_code.cpu().numpy()
        del sub
        toks = self.toks[:, :S, 0].cpu().numpy()
        steps, t0 = 0, time.perf_counter()
        while steps < 64 and (steps < 2 or time.perf_counter() - t0 < 15.0):
            lo, so, _ = om.forward(toks[steps][:, None].astype(np.int32), state=so, planes=0, threads=th)
            om.cb_learn(lo, toks[steps + 1], so)
            steps += 1
        dt = time.perf_counter() - t0
        return {"value": S * steps / dt, "unit": "tokens/s (stream-steps per second)", "cores": th, "kind": "port",
                "sample": f"oracle decode steps (forward with the reference's W8A32 products + the online table's "
                          f"step) of {S} streams from the GPU's state ({n} stored tokens), {steps} steps, {th} "
                          f"threads, {dt:.2f} s"}


WORKLOADS = {"stack": Stack, "stack_heads": StackHeads, "greedy": Greedy, "decode": Decode, "lif": Lif, "delta": Delta, "kwta": Kwta, "gemm": Gemm, "copy": Copy,
             "lif_bwd": LifBwd, "mem_bwd": MemBwd, "mem_chunk": MemChunk, "train": Train}
DEFAULT = "stack"


def extra_workloads():
    return DEFAULT


# ----------------------------------------------------------------------------- main


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 10; decode 256)")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default=None)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (every path shards with no exchange; "
              "see the sharding paragraph of the design notes); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)

    default = extra_workloads()
    wname = args.workload or default
    W = WORKLOADS[wname]()
    if args.steps is None:
        args.steps = getattr(W, "default_steps", 10)
    stream = torch.cuda.current_stream()
    sptr = __import__("ctypes").c_void_p(stream.cuda_stream)

    log(f"bench: workload={wname} warmup={args.warmup} steps={args.steps}")
    # untimed warm-up: W steps and, for the single-kernel workloads, more until the GPU has been busy
    # for WARM_S seconds (the clocks take a few hundred milliseconds of load to settle: a
    # sub-millisecond kernel timed right after three warm-up launches runs 15-25% slower than in
    # steady state)
    tw = time.perf_counter()
    for _ in range(args.warmup):
        W.step(sptr)
    torch.cuda.synchronize()
    warm_run = args.warmup
    while getattr(W, "warm_extend", False) and args.warmup > 0 and time.perf_counter() - tw < WARM_S:
        for _ in range(args.warmup):
            W.step(sptr)
        torch.cuda.synchronize()
        warm_run += args.warmup

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    W.nsteps = args.steps
    if hasattr(W, "start_timed"):
        W.start_timed()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        W.step(sptr, ev[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    W.wall = wall
    # the dominant kernel's launches: one event pair per step, or the workload's own launch timer
    kernel_ms = W.kernel_ms() if hasattr(W, "kernel_ms") else [a.elapsed_time(b) for a, b in ev]
    ms_per_step = wall * 1e3 / args.steps
    value = W.tokens * args.steps / wall
    kern_s = float(np.mean(kernel_ms)) / 1e3  # per launch, or (stack) summed over the timed steps
    roof = W.roofline(kern_s)
    roof["kernel"] = W.kernel
    roof.setdefault("kernel_avg_us", kern_s * 1e6)
    roof["traffic"] = getattr(W, "traffic", None)

    cpu = None
    if not args.no_cpu:
        log("bench: cpu baseline")
        cpu = W.cpu_baseline()
        if cpu is not None:
            # the host's core count beside the threads the baseline used (nproc = the CPUs this process
            # may run on; the machine may have more)
            cpu["threads"] = cpu["cores"]
            cpu["nproc"] = len(os.sched_getaffinity(0))
            cpu["host_cpus"] = os.cpu_count()

    out = {
        "metric": getattr(W, "metric", METRIC),
        "value": value,
        "unit": getattr(W, "unit", "tokens/s"),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": warm_run,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": W.dtype,
        "data": "synthetic (seeded random inputs and random-init weights)",
        "config": W.config,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    if hasattr(W, "extra"):
        out.update(W.extra())
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
