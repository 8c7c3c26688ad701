#!/usr/bin/env python3
"""Benchmark of KORE's fused layer ops on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME[,NAME]] [--no-cpu]

A step is one launch of a fused kernel over one full BASELINE.json config with
its inputs already resident in HBM.  The headline line is the largest
BASELINE.json config that runs on one GPU, configs[2]'s SwiGLU over gate and
up [16384, 14336] (2.8 GB per launch); every other config (RoPE Q+K, RMSNorm,
GELU, the embedding gather, the pre-quant step) is measured the same way and
reported under "kernels" and in the summary lines on stderr.

Per workload:
  * W untimed warmup launches (continued until 0.1 s of device time has
    passed, so clocks have settled), then K timed launches bracketed by
    torch.cuda.synchronize(); HIP events recorded on the stream the kernels are
    launched on give the average kernel duration;
  * algorithmic bytes = every input read once + every output written once;
    achieved GB/s = bytes / average duration; frac = achieved / 8000 GB/s;
  * inputs are rotated over enough buffer sets to exceed four times the 256 MB MALL, so
    HBM is measured, not cache;
  * cpu_baseline: the oracle (a C restatement of the reference's CPU
    functions) timed on this host on a bounded sample of the same workload.

Prints ONE JSON line (rank 0).  `--gpus N` with N > 1 exits: this build runs
on one GPU (every op is row- or element-independent, so a multi-GPU version
shards token rows across processes with no exchange).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

PEAK_GBS = 8000.0
MFMA_I8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POP/s
# MI355X vector fp32 FMA without packed math: 256 CUs x 4 SIMDs x 16 lanes x
# 2 flops x 2.4 GHz
VALU_F32_PEAK_TFLOPS = 78.6
# MI355X dense fp32 MFMA: 157.3 TFLOP/s
MFMA_F32_PEAK_TFLOPS = 157.3
MALL_BYTES = 256 << 20
# The headline workload: BASELINE.json's largest single-GPU config.
HEADLINE = "swiglu"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--only", type=str, default="")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-graph", action="store_true",
                   help="skip the graph-replay timing (profiler runs: only warmup + timed launches dispatch)")
    p.add_argument("--cpu-seconds", type=float, default=8.0, help="CPU work per baseline sample")
    return p.parse_args()


# ----------------------------------------------------------------- workloads
class Workload:
    name = ""
    desc = ""
    tokens = 1
    bytes = 0
    kernel = ""       # device kernel symbol prefix (for rocprof cross-checks)
    dtype = "f32"
    bound = "hbm"     # roofline of the dominant kernel: "hbm" or "mfma"
    ops = 0           # arithmetic operations per launch (MFMA-bound workloads)

    def setup(self, torch, lib):  # allocate inputs, return None
        raise NotImplementedError

    def launch(self, i: int, stream: int) -> int:
        raise NotImplementedError

    def cpu_sample(self):
        """-> (callable running the oracle once on the sample, sample_bytes,
        sample_tokens, threads, description)"""
        raise NotImplementedError

    def free(self):
        for k in list(self.__dict__):
            if k.startswith("_d"):
                delattr(self, k)


def n_sets(bytes_per_set: int, cap: int = 16) -> int:
    # four MALLs' worth: a buffer set is reused only after enough other
    # traffic to evict it even where some of that traffic bypasses the MALL
    return max(1, min(cap, math.ceil(4 * MALL_BYTES / max(bytes_per_set, 1))))


_DIAG = None


def diag_library():
    """libkore_bench_diag.so (bench_diag/): the floor probes, kept out of the
    product library.  Built by bench_diag/Makefile (__graft_entry__.build)."""
    global _DIAG
    if _DIAG is None:
        import ctypes

        path = os.path.join(ROOT, "bench_diag", "libkore_bench_diag.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} not found: run `make -C bench_diag`")
        lib = ctypes.CDLL(path)
        lib.kore_hip_diag_empty.argtypes = [ctypes.c_void_p]
        lib.kore_hip_diag_stream_rows.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_uint64] * 2 + [ctypes.c_void_p]
        _DIAG = lib
    return _DIAG


def randn(torch, shape, seed, mean=0.0, std=1.0):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    t = torch.randn(shape, generator=g, device="cuda", dtype=torch.float32)
    if std != 1.0:
        t.mul_(std)
    if mean != 0.0:
        t.add_(mean)
    return t


class RopeQK(Workload):
    name = "rope_qk"
    B, S, HQ, HK, D = 8, 2048, 32, 8, 128
    kernel = "rope_lane_kernel"

    def __init__(self, interleaved=False):
        self.interleaved = interleaved
        if interleaved:
            self.name = "rope_qk_interleaved"
        self.tokens = self.B * self.S
        self.bytes = 2 * self.B * self.S * (self.HQ + self.HK) * self.D * 4
        self.desc = (f"RoPE f32 in place, Q[{self.B},{self.S},{self.HQ},{self.D}] + K[{self.B},{self.S},{self.HK},"
                     f"{self.D}], theta 1e4, positions 0..{self.S - 1}, "
                     f"{'interleaved' if interleaved else 'half-split'} pairs, one Q+K launch")

    def setup(self, torch, lib):
        from kore_amd import rocm

        self.lib = lib
        self.k = n_sets(self.bytes // 2)
        self._dq = [randn(torch, (self.B, self.S, self.HQ, self.D), 2 * s) for s in range(self.k)]
        self._dk = [randn(torch, (self.B, self.S, self.HK, self.D), 2 * s + 1) for s in range(self.k)]
        self._dinv = torch.from_numpy(rocm.rope_inv_freq_host(self.D, 10000.0)).cuda()

    def launch(self, i, stream):
        j = i % self.k
        return self.lib.kore_hip_rope_qk_f32(self._dq[j].data_ptr(), self._dk[j].data_ptr(), self._dinv.data_ptr(),
                                             self.B, self.S, self.HQ, self.HK, self.D, 0, int(self.interleaved),
                                             stream)

    def cpu_sample(self):
        import oracle
        from inputs import normal

        q = normal((1, self.S, self.HQ, self.D), 0)
        k = normal((1, self.S, self.HK, self.D), 1)

        def run():
            oracle.rope(q, 0, 10000.0, self.interleaved)
            oracle.rope(k, 0, 10000.0, self.interleaved)

        return run, self.bytes // self.B, self.S, 1, "batch 0 of Q and K (1/8 of the config), single thread"


class RMSNorm(Workload):
    kernel = "row_norm_kernel"

    def __init__(self, rows, cols):
        self.rows, self.cols = rows, cols
        self.name = f"rms_norm_{rows}x{cols}"
        self.tokens = rows
        self.bytes = rows * cols * 4 * 2 + cols * 4
        self.desc = f"RMSNorm f32 x[{rows},{cols}] ~ N(0,1), w ~ N(1,0.02), eps 1e-6 (bit-exact)"

    def setup(self, torch, lib):
        self.lib = lib
        per = self.rows * self.cols * 8
        self.k = n_sets(per)
        self._dx = [randn(torch, (self.rows, self.cols), s) for s in range(self.k)]
        self._dy = [torch.empty_like(self._dx[0]) for _ in range(self.k)]
        self._dw = randn(torch, (self.cols,), 100, 1.0, 0.02)

    def launch(self, i, stream):
        j = i % self.k
        return self.lib.kore_hip_rms_norm_f32(self._dx[j].data_ptr(), self._dw.data_ptr(), self._dy[j].data_ptr(),
                                              self.rows, self.cols, 1e-6, stream)

    def cpu_sample(self):
        import oracle
        from inputs import rmsnorm_inputs

        rows = min(self.rows, 4096)
        x, g = rmsnorm_inputs(rows, self.cols, 0)
        return (lambda: oracle.rms_norm(x, g, 1e-6)), rows * self.cols * 8 + self.cols * 4, rows, 1, \
            f"{rows} rows, single thread"


class Swiglu(Workload):
    name = "swiglu"
    T, F = 16384, 14336
    kernel = "binary_vec_kernel"

    def __init__(self):
        self.tokens = self.T
        self.bytes = 3 * self.T * self.F * 4
        self.desc = f"SwiGLU f32 out = silu(gate) * up, gate/up/out [{self.T},{self.F}] ~ N(0,1)"

    def setup(self, torch, lib):
        self.lib = lib
        self._dg = randn(torch, (self.T, self.F), 0)
        self._du = randn(torch, (self.T, self.F), 1)
        self._do = torch.empty_like(self._dg)

    def launch(self, i, stream):
        return self.lib.kore_hip_swiglu_f32(self._dg.data_ptr(), self._du.data_ptr(), self._do.data_ptr(),
                                            self.T * self.F, stream)

    def cpu_sample(self):
        import oracle
        from inputs import normal

        rows = 512
        g, u = normal((rows, self.F), 0), normal((rows, self.F), 1)
        thr = os.cpu_count() or 1
        return (lambda: oracle.swiglu(g, u, threads=thr)), 3 * rows * self.F * 4, rows, thr, \
            f"{rows} of {self.T} rows; silu single thread, mul on {thr} threads (rayon in the reference)"


class Gelu(Workload):
    name = "gelu"
    T, F = 16384, 14336
    kernel = "unary_vec_kernel"

    def __init__(self):
        self.tokens = self.T
        self.bytes = 2 * self.T * self.F * 4
        self.desc = f"GELU (tanh form) f32 x[{self.T},{self.F}] ~ N(0,1)"

    def setup(self, torch, lib):
        self.lib = lib
        self._dx = randn(torch, (self.T, self.F), 0)
        self._dy = torch.empty_like(self._dx)

    def launch(self, i, stream):
        return self.lib.kore_hip_gelu_f32(self._dx.data_ptr(), self._dy.data_ptr(), self.T * self.F, stream)

    def cpu_sample(self):
        import oracle
        from inputs import normal

        rows = 256
        x = normal((rows, self.F), 0)
        return (lambda: oracle.gelu(x)), 2 * rows * self.F * 4, rows, 1, f"{rows} of {self.T} rows, single thread"


class Embedding(Workload):
    name = "embedding"
    V, D, N = 128256, 4096, 8192
    kernel = "embedding_vec1_kernel"

    def __init__(self):
        self.tokens = self.N
        self.bytes = self.N * self.D * 4 * 2 + self.N * 4
        self.desc = (f"Embedding gather f32 table[{self.V},{self.D}] ~ N(0,0.02), ids int32[{self.N}] "
                     "uniform with 5% repeats (bit-exact)")

    def setup(self, torch, lib):
        from inputs import embedding_ids

        self.lib = lib
        self._dt = randn(torch, (self.V, self.D), 0, 0.0, 0.02)
        self.k = n_sets(self.bytes)
        self._dids = [torch.from_numpy(embedding_ids(self.N, self.V, seed=s)).cuda() for s in range(self.k)]
        self._do = [torch.empty((self.N, self.D), device="cuda") for _ in range(self.k)]

    def launch(self, i, stream):
        j = i % self.k
        return self.lib.kore_hip_embedding_f32(self._dt.data_ptr(), self._dids[j].data_ptr(), self._do[j].data_ptr(),
                                               self.N, self.V, self.D, stream)

    def cpu_sample(self):
        import oracle
        from inputs import embedding_ids

        table = np.full((self.V, self.D), 0.5, np.float32)  # values do not change copy speed
        ids = embedding_ids(self.N, self.V, 0)
        return (lambda: oracle.embedding(table, ids)), self.bytes, self.N, 1, \
            "full config (values constant), single thread"


class Prequant(Workload):
    kernel = "row_norm_kernel"

    def __init__(self, rows, cols=2560):
        self.rows, self.cols = rows, cols
        self.name = f"prequant_{rows}x{cols}"
        self.tokens = rows
        self.bytes = rows * cols * 4 + rows * cols + rows * 4 + cols * 4
        self.desc = (f"BitLinear pre-quant x[{rows},{cols}] (1% outliers x20) -> RMSNorm -> int8 codes + f32 "
                     "scale per row (bit-exact)")

    def setup(self, torch, lib):
        self.lib = lib
        self.k = n_sets(self.rows * self.cols * 5, cap=16)
        self._dx = []
        for s in range(self.k):
            x = randn(torch, (self.rows, self.cols), s)
            g = torch.Generator(device="cuda")
            g.manual_seed(1000 + s)
            m = torch.rand((self.rows, self.cols), generator=g, device="cuda") < 0.01
            x[m] *= 20.0
            self._dx.append(x)
        self._dq = [torch.empty((self.rows, self.cols), dtype=torch.int8, device="cuda") for _ in range(self.k)]
        self._ds = [torch.empty((self.rows,), device="cuda") for _ in range(self.k)]
        self._dw = randn(torch, (self.cols,), 100, 1.0, 0.02)

    def launch(self, i, stream):
        j = i % self.k
        return self.lib.kore_hip_rms_norm_quant_i8(self._dx[j].data_ptr(), self._dw.data_ptr(),
                                                   self._dq[j].data_ptr(), self._ds[j].data_ptr(), self.rows,
                                                   self.cols, 1e-6, stream)

    def cpu_sample(self):
        import oracle
        from inputs import prequant_inputs

        x, g = prequant_inputs(self.rows, self.cols, 0)
        return (lambda: oracle.rms_norm_quant_i8(x, g, 1e-6)), self.bytes, self.rows, 1, \
            "full config, single thread"


class RmsNormSiluGate(Workload):
    """y = RMSNorm(x) * silu(z) (cuda/ops.rs:717-751) on the
    pre-quant activation shape."""
    kernel = "row_norm_kernel"

    def __init__(self, rows=4096, cols=2560):
        self.rows, self.cols = rows, cols
        self.name = f"rms_norm_silu_gate_{rows}x{cols}"
        self.tokens = rows
        self.bytes = rows * cols * 4 * 3 + cols * 4
        self.desc = f"RMSNorm(x) * silu(z) f32, x, z [{rows},{cols}] ~ N(0,1), w ~ N(1,0.02), eps 1e-6"

    def setup(self, torch, lib):
        self.lib = lib
        self.k = n_sets(self.rows * self.cols * 12)
        self._dx = [randn(torch, (self.rows, self.cols), s) for s in range(self.k)]
        self._dz = [randn(torch, (self.rows, self.cols), 50 + s) for s in range(self.k)]
        self._dy = [torch.empty_like(self._dx[0]) for _ in range(self.k)]
        self._dw = randn(torch, (self.cols,), 100, 1.0, 0.02)

    def launch(self, i, stream):
        j = i % self.k
        return self.lib.kore_hip_rms_norm_silu_gate_f32(self._dx[j].data_ptr(), self._dw.data_ptr(),
                                                        self._dz[j].data_ptr(), self._dy[j].data_ptr(), self.rows,
                                                        self.cols, 1e-6, stream)

    def cpu_sample(self):
        import oracle
        from inputs import normal, rmsnorm_inputs

        rows = min(self.rows, 1024)
        x, g = rmsnorm_inputs(rows, self.cols, 0)
        z = normal((rows, self.cols), 5)
        return (lambda: oracle.rms_norm_silu_gate(x, g, z, 1e-6)), rows * self.cols * 12 + self.cols * 4, rows, 1, \
            f"{rows} rows, single thread"


class Softmax(Workload):
    """row softmax (cuda/ops.rs:486-511, cpu_fused.rs:195-231)
    over attention-probability rows [16 heads x 2048 queries, 2048 keys]."""
    kernel = "softmax_reg_kernel"

    def __init__(self, rows=32768, cols=2048):
        self.rows, self.cols = rows, cols
        self.name = f"softmax_{rows}x{cols}"
        self.tokens = rows
        self.bytes = rows * cols * 8
        self.desc = f"softmax f32 over the last dim of x[{rows},{cols}] ~ N(0,4^2)"

    def setup(self, torch, lib):
        self.lib = lib
        self.k = n_sets(self.bytes)
        self._dx = [randn(torch, (self.rows, self.cols), 200 + s, 0.0, 4.0) for s in range(self.k)]
        self._dy = [torch.empty_like(self._dx[0]) for _ in range(self.k)]

    def launch(self, i, stream):
        j = i % self.k
        return self.lib.kore_hip_softmax_f32(self._dx[j].data_ptr(), self._dy[j].data_ptr(), self.rows, self.cols,
                                             stream)

    def cpu_sample(self):
        import oracle
        from inputs import normal

        rows = 2048
        x = normal((rows, self.cols), 0) * 4
        return (lambda: oracle.softmax(x)), rows * self.cols * 8, rows, 1, f"{rows} rows, single thread"


class SoftmaxBackward(Workload):
    """fused_softmax_backward (cpu_fused_backward.rs:86-115)."""
    kernel = "softmax_reg_kernel"

    def __init__(self, rows=32768, cols=2048):
        self.rows, self.cols = rows, cols
        self.name = f"softmax_backward_{rows}x{cols}"
        self.tokens = rows
        self.bytes = rows * cols * 12
        self.desc = f"softmax backward f32 dx = y*(dy - sum(y*dy)), y, dy, dx [{rows},{cols}]"

    def setup(self, torch, lib):
        self.lib = lib
        self.k = n_sets(self.bytes)
        self._dy_ = [torch.softmax(randn(torch, (self.rows, self.cols), 300 + s), dim=-1) for s in range(self.k)]
        self._dg = [randn(torch, (self.rows, self.cols), 400 + s) for s in range(self.k)]
        self._do = [torch.empty_like(self._dg[0]) for _ in range(self.k)]

    def launch(self, i, stream):
        j = i % self.k
        return self.lib.kore_hip_softmax_backward_f32(self._dg[j].data_ptr(), self._dy_[j].data_ptr(),
                                                      self._do[j].data_ptr(), self.rows, self.cols, stream)

    def cpu_sample(self):
        import oracle
        from inputs import normal

        rows = 2048
        y = oracle.softmax(normal((rows, self.cols), 0))
        dy = normal((rows, self.cols), 1)
        return (lambda: oracle.softmax_backward(dy, y)), rows * self.cols * 12, rows, 1, f"{rows} rows, single thread"


class RmsNormBackward(Workload):
    """fused_rms_norm_backward (cpu_fused_backward.rs:20-81):
    dx and dgamma; three launches (row pass, partial sums, final sum)."""
    kernel = "rms_bwd_rows_kernel"

    def __init__(self, rows=16384, cols=2048):
        self.rows, self.cols = rows, cols
        self.name = f"rms_norm_backward_{rows}x{cols}"
        self.tokens = rows
        self.bytes = rows * cols * 12 + cols * 8
        self.desc = (f"RMSNorm backward f32: dy, x [{rows},{cols}] -> dx [{rows},{cols}], dgamma [{cols}] "
                     f"(eps 1e-5, deterministic dgamma)")

    def setup(self, torch, lib):
        self.lib = lib
        self.k = n_sets(self.bytes)
        self._dx_ = [randn(torch, (self.rows, self.cols), 500 + s) for s in range(self.k)]
        self._ddy = [randn(torch, (self.rows, self.cols), 600 + s) for s in range(self.k)]
        self._dout = [torch.empty_like(self._dx_[0]) for _ in range(self.k)]
        self._dg = randn(torch, (self.cols,), 700, 1.0, 0.02)
        self._dgg = torch.empty_like(self._dg)
        self.wsb = lib.kore_hip_rms_norm_backward_workspace_bytes(self.rows, self.cols)
        self._dws = torch.empty(self.wsb, dtype=torch.uint8, device="cuda")

    def launch(self, i, stream):
        j = i % self.k
        return self.lib.kore_hip_rms_norm_backward_f32(self._ddy[j].data_ptr(), self._dx_[j].data_ptr(),
                                                       self._dg.data_ptr(), self._dout[j].data_ptr(),
                                                       self._dgg.data_ptr(), self._dws.data_ptr(), self.wsb,
                                                       self.rows, self.cols, 1e-5, stream)

    def cpu_sample(self):
        import oracle
        from inputs import normal, rmsnorm_inputs

        rows = 2048
        x, g = rmsnorm_inputs(rows, self.cols, 0)
        dy = normal((rows, self.cols), 1)
        return (lambda: oracle.rms_norm_backward(dy, x, g, 1e-5)), rows * self.cols * 12 + self.cols * 8, rows, 1, \
            f"{rows} rows, single thread"


class TernaryI8(Workload):
    """BitLinear int8 x ternary matmul (kore_hip_ternary_matmul_i8) on the
    pre-quant config's activations: 4096 tokens (also the decode batches of 64
    and 1) of 2560 codes against a 2560 -> 6912 base-243 ternary weight matrix
    (BitNet-2B4T FFN shape).  At 4096 tokens MFMA-bound, reported as int8 TOPS
    against MI355X's 5.0 POP/s dense; at 1 token bound by the packed weights'
    HBM bytes."""
    kernel = "ternary_i8_mfma_kernel"
    bound = "mfma"

    def __init__(self, m=6912, n=4096, k=2560, layer=False):
        self.m, self.n, self.k = m, n, k
        self.layer = layer
        self.kp = (k + 4) // 5
        self.name = f"{'bit_linear_i8' if layer else 'ternary_i8'}_{m}x{n}x{k}"
        if n <= 8:
            self.kernel = "ternary_i8_gemv_kernel"
        elif n <= 64:
            self.kernel = "ternary_i8_skinny_kernel"
        elif ((m + 255) // 256) * ((n + 255) // 256) >= 144:
            # the library's choice among its wide-path kernels: 256 x 192 tiles
            # when their rounds of 256 CUs are fewer (at >= 8 K steps), else
            # 256 x 128 tiles two workgroups per CU at <= 16 K steps
            t256 = ((m + 255) // 256) * ((n + 255) // 256)
            t192 = ((m + 255) // 256) * ((n + 191) // 192)
            steps = (k + 159) // 160
            n192 = 4 * ((t192 + 255) // 256) < 5 * ((t256 + 255) // 256) and steps >= 8
            self.kernel = "ternary_i8_w2_kernel" if not n192 and steps <= 16 else "ternary_i8_wide_kernel"
        self.tokens = n
        self.ops = 2 * m * n * k
        self.bytes = m * self.kp + n * k + 4 * m * n + 4 * (m + n) + (4 * m if layer else 0)
        self.desc = (f"BitLinear int8 x ternary matmul c[{m},{n}] = ((float)(trits[{m},{k}] . q[{n},{k}]) * "
                     f"a_scale) * q_scale, base-243 weights, int8 codes (bit-exact)")
        if layer:
            self.desc = (f"BitLinear layer on int8 codes (kore_hip_bit_linear_i8): y[{n},{m}] = c^T + bias, the "
                         f"layer's output layout, one launch (bit-exact)")

    def setup(self, torch, lib):
        self.lib = lib
        self.k_sets = 4
        g = torch.Generator(device="cuda")
        g.manual_seed(0)
        self._da = [torch.randint(0, 243, (self.m * self.kp,), generator=g, dtype=torch.uint8, device="cuda")
                    for _ in range(self.k_sets)]
        self._dq = [torch.randint(-128, 128, (self.n * self.k,), generator=g, dtype=torch.int8, device="cuda")
                    for _ in range(self.k_sets)]
        self._dsa = torch.rand(self.m, generator=g, device="cuda")
        self._dsq = torch.rand(self.n, generator=g, device="cuda")
        self._dbias = torch.randn(self.m, generator=g, device="cuda")
        self._dc = [torch.empty(self.m * self.n, device="cuda") for _ in range(self.k_sets)]

    def launch(self, i, stream):
        j = i % self.k_sets
        if self.layer:
            return self.lib.kore_hip_bit_linear_i8(self._da[j].data_ptr(), self._dsa.data_ptr(),
                                                   self._dq[j].data_ptr(), self._dsq.data_ptr(),
                                                   self._dbias.data_ptr(), self._dc[j].data_ptr(), self.m, self.n,
                                                   self.k, stream)
        return self.lib.kore_hip_ternary_matmul_i8(self._da[j].data_ptr(), self._dsa.data_ptr(),
                                                   self._dq[j].data_ptr(), self._dsq.data_ptr(),
                                                   self._dc[j].data_ptr(), self.m, self.n, self.k, stream)

    def library_reference(self, torch):
        """The vendor library's plain int8 GEMM on the same shape for context
        (torch._int_mm: hipBLASLt, int8 x int8 -> int32 [m, n], no trit
        decode, no scales): average of 20 launches after 3 warmups."""
        a = torch.randint(-128, 128, (self.m, self.k), dtype=torch.int8, device="cuda")
        b = torch.randint(-128, 128, (self.k, self.n), dtype=torch.int8, device="cuda")
        for _ in range(3):
            torch._int_mm(a, b)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(20):
            torch._int_mm(a, b)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / 20
        return {"op": "torch._int_mm int8 x int8 -> int32 (hipBLASLt)", "us": round(us, 3),
                "tops": round(self.ops / (us * 1e-6) / 1e12, 1)}

    def cpu_sample(self):
        import oracle
        from inputs import int8_codes, raw_packed

        m, n = 16, 256
        p, q = raw_packed(m, self.k, 1), int8_codes(n, self.k, 2)
        sa, sq = np.ones(m, np.float32), np.ones(n, np.float32)
        return (lambda: oracle.ternary_matmul_i8(p, sa, q, sq, m, n, self.k)), \
            m * self.kp + n * self.k + 4 * m * n, n * m / self.m, 1, \
            f"{m} weight rows x {n} tokens, single thread", 2 * m * n * self.k


class TernaryF32(Workload):
    """BitLinear matmul on f32 activations (kore_hip_ternary_matmul_f32, the
    reference's ternary_matmul as BitLinear::forward calls it): the same
    2560 -> 6912 weights on a decode batch.  Every output is the reference's
    sequential f32 fold over K (bit-exact).  Decode batches run one fma per
    term and lane on the vector unit; where the shape gives the matrix-core
    kernel enough waves (prefill, large batches) each fold step is one
    v_mfma_f32_16x16x1_4b_f32 step.  Reported as fp32 throughput (2 flops per
    term) against the vector fma or the fp32 MFMA peak, next to the bytes."""

    def __init__(self, m=6912, n=1, k=2560, layer=False):
        self.m, self.n, self.k = m, n, k
        self.layer = layer
        # the library's dispatch (ternary.hip: kRowsMinCols, kMfMinWaves)
        mfma = ((m + 63) // 64) * ((n + 15) // 16) >= 768
        # the library's dispatch: the 4 x 4 x 1 matrix-core kernel where the
        # 16 x 16 one does not run: 41-192 tokens, k >= 2560 (up to 7675), at
        # least 640 waves of 4 rows x 64 tokens for the layer's token-major
        # input, 1024 for [K, N] b
        slice_ok = ((3 + 32 * ((k + 4) // 5) + 3) // 4 + 4) * 4 <= 48 * 1024  # the workgroup's packed rows fit its LDS
        mf4 = (not mfma and slice_ok and k >= 2560 and 41 <= n <= 192
               and (m + 3) // 4 * ((n + 63) // 64) >= (640 if layer else 1024))
        self.bound = "mfma_f32" if mfma or mf4 else "valu"
        self.kernel = ("ternary_f32_mfma_kernel" if mfma else "ternary_f32_mf4_kernel" if mf4 else
                       "ternary_f32_pipe_kernel" if n <= 4 else "ternary_f32_rows_kernel")
        self.kp = (k + 4) // 5
        self.name = f"{'bit_linear_f32' if layer else 'ternary_f32'}_{m}x{n}x{k}"
        self.tokens = n
        self.ops = 2 * m * n * k
        self.bytes = m * self.kp + 4 * k * n + 4 * m * n + 4 * m
        self.desc = (f"BitLinear f32 x ternary matmul c[{m},{n}] = (sum_k trits[{m},{k}] * b[{k},{n}]) * a_scale, "
                     "sequential f32 fold in k order (bit-exact)")
        if layer:
            self.bytes += 4 * m
            self.desc = (f"BitLinear::forward (kore_hip_bit_linear_f32): y[{n},{m}] = ternary_matmul(W, s, x^T)^T + "
                         f"bias with x[{n},{k}] as stored, one launch (bit-exact)")

    def setup(self, torch, lib):
        self.lib = lib
        self.k_sets = 4
        g = torch.Generator(device="cuda")
        g.manual_seed(0)
        self._da = [torch.randint(0, 243, (self.m * self.kp,), generator=g, dtype=torch.uint8, device="cuda")
                    for _ in range(self.k_sets)]
        self._db = [torch.randn((self.k * self.n,), generator=g, device="cuda") for _ in range(self.k_sets)]
        self._dsa = torch.rand(self.m, generator=g, device="cuda")
        self._dbias = torch.randn(self.m, generator=g, device="cuda")
        self._dc = [torch.empty(self.m * self.n, device="cuda") for _ in range(self.k_sets)]

    def launch(self, i, stream):
        j = i % self.k_sets
        if self.layer:
            return self.lib.kore_hip_bit_linear_f32(self._da[j].data_ptr(), self._dsa.data_ptr(),
                                                    self._db[j].data_ptr(), self._dbias.data_ptr(),
                                                    self._dc[j].data_ptr(), self.m, self.n, self.k, stream)
        return self.lib.kore_hip_ternary_matmul_f32(self._da[j].data_ptr(), self._dsa.data_ptr(),
                                                    self._db[j].data_ptr(), self._dc[j].data_ptr(), self.m, self.n,
                                                    self.k, stream)

    def cpu_sample(self):
        import oracle
        from inputs import normal, raw_packed

        m = 512 if self.n <= 64 else max(8, 512 * 64 // self.n)
        p, b = raw_packed(m, self.k, 1), normal((self.k, self.n), 2)
        sa = np.ones(m, np.float32)
        return (lambda: oracle.ternary_matmul(p, sa, b, m, self.n, self.k)), \
            m * self.kp + 4 * self.k * self.n + 4 * m * self.n, self.n * m / self.m, 1, \
            f"{m} weight rows x {self.n} tokens, single thread", 2 * m * self.n * self.k


class PackTernary(Workload):
    """Weight packing (kore_hip_pack_weights_ternary, the reference's
    pack_weights_ternary): f32 weights of the 2560 -> 6912 BitLinear to
    base-243 bytes and per-row scales, bit-exact.  Reads 4 m k bytes, writes
    m ceil(k/5) + 4 m: HBM-bound."""
    kernel = "ternary_pack_kernel"

    def __init__(self, m=6912, k=2560):
        self.m, self.k = m, k
        self.kp = (k + 4) // 5
        self.name = f"pack_weights_ternary_{m}x{k}"
        self.tokens = m  # weight rows
        self.bytes = 4 * m * k + m * self.kp + 4 * m
        self.desc = f"ternary weight packing w[{m},{k}] f32 -> base-243 bytes [{m},{self.kp}] + scales, threshold 0.3"

    def setup(self, torch, lib):
        self.lib = lib
        self.k_sets = n_sets(self.bytes)
        g = torch.Generator(device="cuda")
        g.manual_seed(0)
        self._dw = [torch.randn((self.m * self.k,), generator=g, device="cuda") for _ in range(self.k_sets)]
        self._dp = [torch.empty(self.m * self.kp, dtype=torch.uint8, device="cuda") for _ in range(self.k_sets)]
        self._ds = [torch.empty(self.m, device="cuda") for _ in range(self.k_sets)]

    def launch(self, i, stream):
        j = i % self.k_sets
        return self.lib.kore_hip_pack_weights_ternary(self._dw[j].data_ptr(), self.m, self.k, 0.3,
                                                      self._dp[j].data_ptr(), self._ds[j].data_ptr(), stream)

    def cpu_sample(self):
        import oracle
        from inputs import normal

        m = 1024
        w = normal((m, self.k), 3)
        return (lambda: oracle.pack_weights_ternary(w, 0.3)), 4 * m * self.k + m * self.kp + 4 * m, m, 1, \
            f"{m} weight rows, single thread"


class Copy(Workload):
    """A plain 1 GiB device copy through the gather kernel with ids = 0..N-1;
    used to calibrate rocprof's FETCH_SIZE / WRITE_SIZE counters."""
    name = "copy_1gib"
    N, D = 65536, 4096
    kernel = "embedding_vec1_kernel"

    def __init__(self):
        self.tokens = self.N
        self.bytes = self.N * self.D * 4 * 2 + self.N * 4
        self.desc = "calibration copy: 1 GiB read + 1 GiB written (gather with ids 0..N-1)"

    def setup(self, torch, lib):
        self.lib = lib
        self._dt = randn(torch, (self.N, self.D), 0)
        self._dids = torch.arange(self.N, dtype=torch.int32, device="cuda")
        self._do = torch.empty_like(self._dt)

    def launch(self, i, stream):
        return self.lib.kore_hip_embedding_f32(self._dt.data_ptr(), self._dids.data_ptr(), self._do.data_ptr(),
                                               self.N, self.N, self.D, stream)

    def cpu_sample(self):
        return None


class LaunchFloor(Workload):
    """One empty workgroup per launch (kore_hip_diag_empty): the floor of a
    dependent kernel launch on a stream, against which the latency-bound
    configs (a few rows) are read."""
    name = "launch_floor"
    kernel = "diag_empty_kernel"
    tokens = 1
    bytes = 0
    desc = "empty kernel, one workgroup of 64 threads (launch floor)"

    def setup(self, torch, lib):
        self.lib = diag_library()

    def launch(self, i, stream):
        return self.lib.kore_hip_diag_empty(stream)

    def cpu_sample(self):
        return None


class StreamFloor(Workload):
    """The pre-quant kernel's bytes with a trivial body
    (kore_hip_diag_stream_rows): reads x[rows, cols] f32 once, writes one byte
    per value and one f32 per row, one wave per row.  The streaming ceiling of
    that shape, measured next to the real kernel."""
    kernel = "diag_stream_rows_kernel"

    def __init__(self, rows=4096, cols=2560):
        self.rows, self.cols = rows, cols
        self.name = f"stream_floor_{rows}x{cols}"
        self.tokens = rows
        self.bytes = rows * cols * 4 + rows * cols + rows * 4 + cols * 4
        self.desc = f"pre-quant traffic with a trivial body: x[{rows},{cols}] f32 -> one byte per value + f32 per row"

    def setup(self, torch, lib):
        self.lib = diag_library()
        self.k = n_sets(self.rows * self.cols * 5, cap=16)
        self._dx = [randn(torch, (self.rows, self.cols), s) for s in range(self.k)]
        self._dq = [torch.empty((self.rows, self.cols), dtype=torch.int8, device="cuda") for _ in range(self.k)]
        self._ds = [torch.empty((self.rows,), device="cuda") for _ in range(self.k)]

    def launch(self, i, stream):
        j = i % self.k
        return self.lib.kore_hip_diag_stream_rows(self._dx[j].data_ptr(), self._dq[j].data_ptr(),
                                                  self._ds[j].data_ptr(), self.rows, self.cols, stream)

    def cpu_sample(self):
        return None


def all_workloads():
    return [RopeQK(False), RopeQK(True), RMSNorm(32, 2048), RMSNorm(16384, 2048), Swiglu(), Gelu(), Embedding(),
            Prequant(4096), Prequant(64), Prequant(1), LaunchFloor(), StreamFloor(), StreamFloor(1, 2560),
            StreamFloor(64, 2560), StreamFloor(32, 2048), RmsNormSiluGate(), Softmax(),
            SoftmaxBackward(),
            RmsNormBackward(), TernaryI8(), TernaryI8(2560, 4096, 6912), TernaryI8(6912, 64, 2560),
            TernaryI8(6912, 1, 2560), TernaryI8(6912, 4096, 2560, layer=True), TernaryI8(2560, 4096, 6912, layer=True),
            TernaryI8(6912, 64, 2560, layer=True), TernaryF32(), TernaryF32(6912, 16, 2560), TernaryF32(6912, 64, 2560),
            TernaryF32(6912, 1, 2560, layer=True), TernaryF32(6912, 64, 2560, layer=True), TernaryF32(6912, 1024, 2560),
            TernaryF32(6912, 4096, 2560, layer=True), PackTernary(),
            PackTernary(2560, 6912), Copy()]


# ------------------------------------------------------------------ measure
MIN_WARM_S = 0.1


def time_gpu(torch, w: Workload, steps: int, warmup: int):
    """W warmup launches, continued in batches until at least MIN_WARM_S of
    device time has passed (clocks settle under a sustained load; a few cold
    launches of a compute-bound kernel run up to ~15% slower), then the timed
    launches.  Returns (ms per timed launch, wall seconds, warmup launches)."""
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    n_warm = 0
    t_warm = time.perf_counter()
    batch = max(warmup, 1)
    while True:
        for _ in range(batch):
            rc = w.launch(n_warm, sp)
            if rc != 0:
                raise RuntimeError(f"{w.name}: launch returned {rc}")
            n_warm += 1
        torch.cuda.synchronize()
        if n_warm >= warmup and time.perf_counter() - t_warm >= MIN_WARM_S:
            break
        batch = max(batch, 10)
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(steps):
        rc = w.launch(n_warm + i, sp)
        if rc != 0:
            raise RuntimeError(f"{w.name}: launch returned {rc}")
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = ev0.elapsed_time(ev1)
    return ev_ms / steps, wall, n_warm


def time_graph(torch, w: Workload, per_graph: int = 20, replays: int = 20):
    """Per-launch time with `per_graph` launches captured in one HIP graph and
    replayed: the kernels back to back without host launch overhead.  Every
    entry point is capturable (no allocation, synchronisation or memset)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(3):
            w.launch(i, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        sp = torch.cuda.current_stream().cuda_stream
        for i in range(per_graph):
            if w.launch(i, sp) != 0:
                raise RuntimeError(f"{w.name}: launch failed under capture")
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (replays * per_graph)
    del g
    return us


def time_cpu(w: Workload, budget_s: float):
    s = w.cpu_sample()
    if s is None:
        return None
    run, nbytes, ntok, threads, desc = s[:5]
    ops = s[5] if len(s) > 5 else 0
    run()  # warm (page-in, libm init)
    reps, t = 0, 0.0
    t0 = time.perf_counter()
    while True:
        run()
        reps += 1
        t = time.perf_counter() - t0
        if t >= budget_s or reps >= 1000:
            break
    per = t / reps
    out = {"value": round(nbytes / per / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
           "ns_per_token": round(per / ntok * 1e9, 1), "seconds": round(t, 2), "reps": reps,
           "sample": desc, "host_cores": os.cpu_count()}
    if ops:
        unit = "GOP/s (int8 multiply-adds x 2)" if w.bound == "mfma" else "GFLOP/s (f32 fold, 2 per term)"
        out.update({"value": round(ops / per / 1e9, 4), "unit": unit, "gbs": round(nbytes / per / 1e9, 4)})
    return out


def load_traffic():
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE and
    WRITE_SIZE, scaled by the copy-kernel calibration), if a committed summary
    exists: profiles/hbm_traffic.txt, lines `workload fetch_bytes write_bytes`."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.txt")
    out = {}
    if os.path.exists(path):
        for line in open(path):
            f = line.split()
            if len(f) == 3 and not line.startswith("#"):
                try:
                    out[f[0]] = int(float(f[1])) + int(float(f[2]))
                except ValueError:
                    pass
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested). The fused layer ops are "
              "row/element independent and shard by token rows with no exchange.", file=sys.stderr)
        sys.exit(2)
    import torch

    import kore_amd

    lib = kore_amd.load_library()
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    only = set(filter(None, args.only.split(",")))
    works = [w for w in all_workloads() if not only or w.name in only]
    if not works:
        sys.exit(f"--only {args.only}: no workload of that name "
                 f"(names: {', '.join(w.name for w in all_workloads())})")
    if not only:
        works = [w for w in works if w.name != "copy_1gib"]
    traffic = load_traffic()
    results = {}
    for w in works:
        print(f"[bench] {w.name}: setup", file=sys.stderr, flush=True)
        w.setup(torch, lib)
        torch.cuda.synchronize()
        steps = args.steps if w.bytes >= (64 << 20) else max(args.steps, 200)
        print(f"[bench] {w.name}: {args.warmup} warmup + {steps} timed launches", file=sys.stderr, flush=True)
        ms, wall, n_warm = time_gpu(torch, w, steps, args.warmup)
        graph_us = None
        if w.bytes < (16 << 20) and not args.no_graph:  # latency-bound launches: also without host launch overhead
            graph_us = round(time_graph(torch, w), 3)
        gbs = w.bytes / (ms * 1e-3) / 1e9
        r = {
            "workload": w.desc, "kernel": w.kernel, "bytes_per_launch": w.bytes, "tokens": w.tokens,
            "kernel_us": round(ms * 1e3, 3), "achieved_gbs": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_GBS, 4),
            "ns_per_token": round(ms * 1e6 / w.tokens, 3), "steps": steps, "warmup_launches": n_warm,
            "wall_s": round(wall, 7),
            "wall_gbs": round(w.bytes * steps / wall / 1e9, 1),
        }
        if graph_us is not None:
            r["graph_us"] = graph_us
        if w.ops:
            tops = w.ops / (ms * 1e-3) / 1e12
            r.update({"bound": w.bound, "ops_per_launch": w.ops, "achieved_tops": round(tops, 3)})
            if w.bound == "mfma":
                r["frac_of_mfma_peak"] = round(tops / MFMA_I8_PEAK_TOPS, 4)
            elif w.bound == "mfma_f32":
                r["frac_of_mfma_f32_peak"] = round(tops / MFMA_F32_PEAK_TFLOPS, 4)
            else:
                r["frac_of_valu_f32_peak"] = round(tops / VALU_F32_PEAK_TFLOPS, 4)
        if w.name in traffic:
            r["hbm_traffic_bytes"] = traffic[w.name]
        if hasattr(w, "library_reference") and getattr(w, "n", 8) % 8 != 0:
            r["library_reference"] = {"skipped": "torch._int_mm needs n % 8 == 0"}
        elif hasattr(w, "library_reference") and not getattr(w, "layer", False):
            try:
                r["library_reference"] = w.library_reference(torch)
            except Exception as ex:  # the reference is context only
                r["library_reference"] = {"error": str(ex)[:200]}
        w.free()
        torch.cuda.empty_cache()
        if not args.no_cpu:
            print(f"[bench] {w.name}: cpu baseline", file=sys.stderr, flush=True)
            r["cpu_baseline"] = time_cpu(w, args.cpu_seconds if w.name == HEADLINE else args.cpu_seconds / 3)
        results[w.name] = r
        extra = ""
        if w.ops and w.bound == "mfma":
            extra = f", {r['achieved_tops']} TOPS ({100 * r['frac_of_mfma_peak']:.1f}% of the int8 MFMA peak)"
        elif w.ops and w.bound == "mfma_f32":
            extra = f", {r['achieved_tops']} TFLOP/s ({100 * r['frac_of_mfma_f32_peak']:.1f}% of the fp32 MFMA peak)"
        elif w.ops:
            extra = f", {r['achieved_tops']} TFLOP/s ({100 * r['frac_of_valu_f32_peak']:.1f}% of the fp32 FMA peak)"
        print(f"[bench] {w.name}: {r['kernel_us']} us, {r['achieved_gbs']} GB/s ({100 * r['frac_of_peak']:.1f}% "
              f"of peak), {r['ns_per_token']} ns/token{extra}", file=sys.stderr, flush=True)

    head_name = HEADLINE if HEADLINE in results else next(iter(results))
    h = results[head_name]
    steps = h["steps"]
    line = {
        "metric": "achieved HBM GB/s and % of MI355X HBM peak per fused kernel; ns/token",
        "value": round(h["bytes_per_launch"] * steps / h["wall_s"] / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["wall_s"] / steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) inputs of the BASELINE shapes)",
        "config": {"workload": h["workload"], "kernel": h["kernel"], "bytes_per_step": h["bytes_per_launch"],
                   "tokens_per_step": h["tokens"], "ns_per_token": h["ns_per_token"]},
        "roofline": {"bound": "hbm", "achieved": h["achieved_gbs"], "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": h["frac_of_peak"], "traffic": h.get("hbm_traffic_bytes")},
        "cpu_baseline": h.get("cpu_baseline"),
        "kernels": results,
    }
    print(json.dumps(line), flush=True)
    print_summary(results)


# The floors and the "next" rows, then BASELINE.json's configs -> workloads
# (configs[2]'s SwiGLU is the headline): printed last, so that a captured tail
# of stderr holds every config.
SUMMARY = [("floor: empty launch", "launch_floor"),
           ("floor: pre-quant bytes, trivial body", "stream_floor_4096x2560"),
           ("floor: 1x2560 read + byte writes, one wave", "stream_floor_1x2560"),
           ("floor: 64x2560 read + byte writes", "stream_floor_64x2560"),
           ("floor: 32x2048 read + byte writes", "stream_floor_32x2048"),
           ("next: RMSNorm 16384x2048", "rms_norm_16384x2048"), ("next: norm+SiLU gate", "rms_norm_silu_gate_4096x2560"),
           ("next: softmax 32768x2048", "softmax_32768x2048"),
           ("next: ternary i8 6912x4096x2560", "ternary_i8_6912x4096x2560"),
           ("next: BitLinear layer i8 6912x4096x2560", "bit_linear_i8_6912x4096x2560"),
           ("next: ternary i8 2560x4096x6912", "ternary_i8_2560x4096x6912"),
           ("next: BitLinear layer f32 6912x4096x2560 (fp32 MFMA)", "bit_linear_f32_6912x4096x2560"),
           ("cfg0 RMSNorm 32x2048", "rms_norm_32x2048"), ("cfg1 RoPE Q+K half-split", "rope_qk"),
           ("cfg1 RoPE Q+K interleaved", "rope_qk_interleaved"), ("cfg2 SwiGLU 16384x14336", "swiglu"),
           ("cfg2 GELU 16384x14336", "gelu"), ("cfg3 Embedding 8192x4096", "embedding"),
           ("cfg4 pre-quant 4096x2560", "prequant_4096x2560"), ("cfg4 pre-quant 64x2560", "prequant_64x2560"),
           ("cfg4 pre-quant 1x2560", "prequant_1x2560")]


# Latency-bound configs -> the trivial-body kernel moving their rows (reads
# every value, writes a byte per value): any kernel that writes memory pays
# about 1 us more per launch than an empty one.
SAME_SHAPE_FLOOR = {"rms_norm_32x2048": "stream_floor_32x2048", "prequant_64x2560": "stream_floor_64x2560",
                    "prequant_1x2560": "stream_floor_1x2560"}


def print_summary(results):
    """Compact per-config lines on stderr (after the JSON line, so that a
    captured stderr tail holds every BASELINE config)."""
    floor = results.get("launch_floor", {}).get("kernel_us")
    out = ["[summary] config: us (graph us) | GB/s | % of 8 TB/s | ns/token | CPU baseline"]
    for label, name in SUMMARY:
        r = results.get(name)
        if not r:
            continue
        g = f" ({r['graph_us']})" if "graph_us" in r else ""
        cpu = r.get("cpu_baseline") or {}
        cpu_s = f"{cpu.get('value')} {cpu.get('unit', '')} x{cpu.get('cores', '')}" if cpu else "-"
        tail = ""
        if floor and "graph_us" in r and name != "launch_floor" and not name.startswith("stream_floor"):
            tail = f" | {r['kernel_us'] / floor:.2f}x launch floor"
            same = results.get(SAME_SHAPE_FLOOR.get(name, ""), {}).get("kernel_us")
            if same:
                tail += f", {r['kernel_us'] / same:.2f}x its shape's read/write floor per launch"
        if "achieved_tops" in r and r.get("bound") == "mfma":
            tail += f" | {r['achieved_tops']} TOPS ({100 * r['frac_of_mfma_peak']:.1f}% int8 MFMA)"
        elif "achieved_tops" in r and r.get("bound") == "mfma_f32":
            tail += f" | {r['achieved_tops']} TFLOP/s ({100 * r['frac_of_mfma_f32_peak']:.1f}% fp32 MFMA)"
        out.append(f"[summary] {label}: {r['kernel_us']}{g} | {r['achieved_gbs']} | {100 * r['frac_of_peak']:.1f}% | "
                   f"{r['ns_per_token']} | {cpu_s}{tail}")
    print("\n".join(out), file=sys.stderr, flush=True)


if __name__ == "__main__":
    main()
