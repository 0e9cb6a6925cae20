"""Benchmark of the MI355X tile-op path on BASELINE.json's configs (1 GPU).

  python bench.py [--config gemm|softmax|mlp|attn|decode|all|...] [--steps K] [--warmup W]
                  [--path library|emitted]

A step is one launch of the tile op over one batch of synthetic, seeded input
already resident in HBM (generated on the device by th_fill_random with seed
0x71130000 + config index).  The default workload is BASELINE config 2 — the
4096^3 bf16 GEMM, the configuration the metric is quoted on — and prints ONE
JSON line.  Bandwidth-bound configs rotate input/output sets totalling more
than 256 MB so the Infinity Cache cannot serve them.

Timing: a clock-settle phase (steps run until --settle-ms of wall time have
passed: MI355X ramps its clock over the first ~100 ms of sustained MFMA work, and
a cold 4096^3 GEMM step takes 140-160 us against ~123 us settled), then W untimed
steps, then K steps bracketed by stream synchronization, with HIP events on the
stream the kernels run on between groups of consecutive steps (about 1 ms of work
per group, at least ten groups; an event after every 10 us step would add its own
gap); ms_per_step is the median over groups of the per-step time (the mean over
all K steps is reported beside it).  --path emitted runs the same step through the
kernel the hip codegen target emits for the config (tilers_hip/examples).
roofline.achieved = algorithmic work per step / ms_per_step (the step is one
kernel launch except decode, which is the split kernel plus a small combine).
cpu_baseline times the CPU oracle (test infrastructure, never the measured
path) on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "tile-rs_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "GEMM/attention TFLOP/s, softmax GB/s, % of MI355X roofline (1 GPU)"
PEAK_MFMA_TFLOPS = 2500.0   # MI355X dense bf16/f16 MFMA
PEAK_MFMA_F32_TFLOPS = 157.3  # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
SEED0 = 0x71130000
MALL_BYTES = 256 << 20


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Workload:
    name = ""
    index = 0
    bound = "mfma"
    dtype = "bf16"
    unit = "TFLOP/s"
    peak = None  # TFLOP/s or GB/s; None = the bf16 MFMA or the HBM peak by unit

    def work(self) -> float:  # FLOP or bytes per step
        raise NotImplementedError

    def setup(self, th, dev, s):
        raise NotImplementedError

    def step(self, th, s, i: int):
        raise NotImplementedError

    def cpu_sample(self, th, s, seconds: float):
        raise NotImplementedError

    # The same step through the `hip` codegen target: the example module's kernel
    # (tilers_hip/examples/<stem>.mlir, emitted and compiled by the build) launched
    # by name on `tiles` logical tiles.
    emitted = None  # (module stem, kernel name)

    def emitted_args(self, i: int):
        raise NotImplementedError

    def emitted_step(self, th, s, i: int):
        import ctypes as C
        tiles, bufs, scalars = self.emitted_args(i)
        args = [C.c_void_p(b.as_raw_ptr()) for b in bufs] + [C.c_uint32(x) for x in scalars]
        self.launcher.launch(self.emitted[1], th.LaunchGrid.blocks_only(tiles), args, s)


def rotation_sets(bytes_per_set: int) -> int:
    return max(1, -(-2 * MALL_BYTES // bytes_per_set))


class Softmax(Workload):
    name, index, bound, dtype, unit = "softmax", 1, "hbm", "f32", "GB/s"
    rows, cols = 8192, 1024

    def work(self):
        return 2.0 * self.rows * self.cols * 4

    def config(self):
        return {"workload": "row softmax f32 8192x1024, X~N(0,2)", "rows": self.rows,
                "cols": self.cols}

    def setup(self, th, dev, s):
        D = th.TileDtype
        n = self.rows * self.cols
        self.sets = []
        for r in range(rotation_sets(2 * n * 4)):
            x = dev.alloc(n, D.F32)
            th.fill_random(x, n, D.F32, "normal", 0.0, 2.0, SEED0 + self.index + 1000 * r, s)
            self.sets.append((x, dev.alloc(n, D.F32)))

    def step(self, th, s, i):
        x, y = self.sets[i % len(self.sets)]
        th.softmax(x, y, self.rows, self.cols, th.TileDtype.F32, s)

    emitted = ("softmax_rows", "softmax_rows_f32")   # one 1 x 1024 row per tile

    def emitted_args(self, i):
        x, y = self.sets[i % len(self.sets)]
        return self.rows, [x, y], []

    def cpu_sample(self, th, s, seconds):
        from oracle import oracle as orc
        x = self.sets[0][0].copy_to_host(s).reshape(self.rows, self.cols)
        done, t0 = 0, time.perf_counter()
        while True:
            r0 = (done * 512) % self.rows
            orc.softmax(x[r0:r0 + 512], 512, self.cols)
            done += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                break
        rows = done * 512
        return rows * self.cols * 8 / el / 1e9, f"{rows} rows of the 8192x1024 softmax"


class Gemm(Workload):
    name, index, bound, dtype, unit = "gemm", 2, "mfma", "bf16", "TFLOP/s"
    M = N = K = 4096
    in_dt, out_dt = "BF16", "F32"

    def work(self):
        return 2.0 * self.M * self.N * self.K

    def config(self):
        return {"workload": "dense GEMM C=A*B, 4096^3, A,B bf16 U[-1,1], C f32 (f32 acc)",
                "M": self.M, "N": self.N, "K": self.K}

    def setup(self, th, dev, s):
        D = th.TileDtype
        self.a = dev.alloc(self.M * self.K, D.BF16)
        self.b = dev.alloc(self.K * self.N, D.BF16)
        self.c = dev.alloc(self.M * self.N, D.F32)
        th.fill_random(self.a, self.M * self.K, D.BF16, "uniform", -1.0, 1.0, SEED0 + 2, s)
        th.fill_random(self.b, self.K * self.N, D.BF16, "uniform", -1.0, 1.0, SEED0 + 102, s)

    def step(self, th, s, i):
        D = th.TileDtype
        th.matmul(self.a, self.b, self.c, self.M, self.K, self.N, getattr(D, self.in_dt),
                  getattr(D, self.out_dt), False, stream=s)

    emitted = ("config_gemms", "gemm_4096_bf16_acc_f32")

    def emitted_args(self, i):
        return 1, [self.a, self.b, self.c], []

    def cpu_sample(self, th, s, seconds):
        from oracle import oracle as orc
        import numpy as np
        dt = orc.BF16 if self.in_dt == "BF16" else orc.F16
        a = self.a.copy_to_host(s).reshape(self.M, self.K)
        b = self.b.copy_to_host(s)
        out = orc.F32 if self.out_dt == "F32" else orc.F16
        rows, t0, chunk = 0, time.perf_counter(), 64
        while True:
            r0 = rows % self.M
            orc.matmul(np.ascontiguousarray(a[r0:r0 + chunk]), b, chunk, self.K, self.N, dt, out)
            rows += chunk
            el = time.perf_counter() - t0
            if el >= seconds:
                break
        return 2.0 * rows * self.K * self.N / el / 1e12, (
            f"{rows} rows of C ({self.M}x{self.N}x{self.K}), oracle f32 FMA")


class Mlp(Gemm):
    name, index, dtype = "mlp", 3, "f16"
    M, K, N = 8192, 4096, 14336
    in_dt, out_dt = "F16", "F16"

    def config(self):
        return {"workload": "MLP GEMM M=8192 K=4096 N=14336, f16 in, f32 acc, f16 out",
                "M": self.M, "N": self.N, "K": self.K}

    emitted = ("config_gemms", "mlp_up_f16")

    def setup(self, th, dev, s):
        D = th.TileDtype
        self.a = dev.alloc(self.M * self.K, D.F16)
        self.b = dev.alloc(self.K * self.N, D.F16)
        self.c = dev.alloc(self.M * self.N, D.F16)
        th.fill_random(self.a, self.M * self.K, D.F16, "normal", 0.0, 1.0, SEED0 + 3, s)
        th.fill_random(self.b, self.K * self.N, D.F16, "normal", 0.0, 0.02, SEED0 + 103, s)


class GemmF32(Gemm):
    """__tile_matmul_f32 on the fp32 MFMA: 4096^3, A, B and C f32."""
    name, index, dtype = "gemm_f32", 7, "f32"
    in_dt, out_dt = "F32", "F32"
    peak = PEAK_MFMA_F32_TFLOPS
    emitted = None

    def config(self):
        return {"workload": "dense GEMM C=A*B, 4096^3, A,B f32 U[-1,1], C f32 (fp32 MFMA)",
                "M": self.M, "N": self.N, "K": self.K}

    def setup(self, th, dev, s):
        D = th.TileDtype
        self.a = dev.alloc(self.M * self.K, D.F32)
        self.b = dev.alloc(self.K * self.N, D.F32)
        self.c = dev.alloc(self.M * self.N, D.F32)
        th.fill_random(self.a, self.M * self.K, D.F32, "uniform", -1.0, 1.0, SEED0 + 7, s)
        th.fill_random(self.b, self.K * self.N, D.F32, "uniform", -1.0, 1.0, SEED0 + 107, s)

    def cpu_sample(self, th, s, seconds):
        from oracle import oracle as orc
        import numpy as np
        a = self.a.copy_to_host(s).reshape(self.M, self.K)
        b = self.b.copy_to_host(s)
        rows, t0, chunk = 0, time.perf_counter(), 64
        while True:
            r0 = rows % self.M
            orc.matmul(np.ascontiguousarray(a[r0:r0 + chunk]), b, chunk, self.K, self.N, orc.F32,
                       orc.F32)
            rows += chunk
            el = time.perf_counter() - t0
            if el >= seconds:
                break
        return 2.0 * rows * self.K * self.N / el / 1e12, (
            f"{rows} rows of C ({self.M}x{self.N}x{self.K}), oracle f32 FMA")


class Swiglu(Mlp):
    """Config 3's MLP shape with the gate epilogue fused: C = silu(A.B) * UP (f16)."""
    name = "swiglu"
    emitted = ("config_gemms", "mlp_gate_f16")

    def emitted_args(self, i):
        return 1, [self.a, self.b, self.up, self.c], []

    def config(self):
        return {"workload": "MLP gate GEMM M=8192 K=4096 N=14336 with fused silu*mul "
                            "epilogue, f16 in, f32 acc, f16 UP and out",
                "M": self.M, "N": self.N, "K": self.K}

    def setup(self, th, dev, s):
        super().setup(th, dev, s)
        D = th.TileDtype
        self.up = dev.alloc(self.M * self.N, D.F16)
        th.fill_random(self.up, self.M * self.N, D.F16, "normal", 0.0, 1.0, SEED0 + 203, s)

    def step(self, th, s, i):
        D = th.TileDtype
        th.matmul_silu_mul(self.a, self.b, self.up, self.c, self.M, self.K, self.N, D.F16, D.F16,
                           False, stream=s)

    def cpu_sample(self, th, s, seconds):
        from oracle import oracle as orc
        import numpy as np
        a = self.a.copy_to_host(s).reshape(self.M, self.K)
        b, up = self.b.copy_to_host(s), self.up.copy_to_host(s).reshape(self.M, self.N)
        rows, t0, chunk = 0, time.perf_counter(), 32
        while True:
            r0 = rows % self.M
            orc.matmul_silu_mul(np.ascontiguousarray(a[r0:r0 + chunk]), b,
                                np.ascontiguousarray(up[r0:r0 + chunk]), chunk, self.K, self.N,
                                orc.F16, orc.F16)
            rows += chunk
            el = time.perf_counter() - t0
            if el >= seconds:
                break
        return 2.0 * rows * self.K * self.N / el / 1e12, (
            f"{rows} rows of the gate GEMM + silu*mul, oracle f32")


class RmsNorm(Workload):
    """Row RMSNorm on an LLM hidden-state shape: 8192 tokens x 4096, bf16."""
    name, index, bound, dtype, unit = "rmsnorm", 6, "hbm", "bf16", "GB/s"
    rows, cols, eps = 8192, 4096, 1e-6

    def work(self):
        return 2.0 * self.rows * self.cols * 2

    def config(self):
        return {"workload": "row RMSNorm bf16 8192x4096 (f32 math), X~N(0,1), eps 1e-6",
                "rows": self.rows, "cols": self.cols}

    def setup(self, th, dev, s):
        D = th.TileDtype
        n = self.rows * self.cols
        self.sets = []
        for r in range(rotation_sets(2 * n * 2)):
            x = dev.alloc(n, D.BF16)
            th.fill_random(x, n, D.BF16, "normal", 0.0, 1.0, SEED0 + self.index + 1000 * r, s)
            self.sets.append((x, dev.alloc(n, D.BF16)))

    def step(self, th, s, i):
        x, y = self.sets[i % len(self.sets)]
        th.rms_norm(x, y, self.rows, self.cols, self.eps, th.TileDtype.BF16, s)

    def cpu_sample(self, th, s, seconds):
        from oracle import oracle as orc
        import numpy as np
        x = self.sets[0][0].copy_to_host(s).reshape(self.rows, self.cols)
        done, t0 = 0, time.perf_counter()
        while True:
            r0 = (done * 256) % self.rows
            orc.rms_norm(np.ascontiguousarray(x[r0:r0 + 256]), 256, self.cols, self.eps, orc.BF16)
            done += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                break
        rows = done * 256
        return rows * self.cols * 4 / el / 1e9, f"{rows} rows of the 8192x4096 RMSNorm"


class Attn(Workload):
    name, index, bound, dtype, unit = "attn", 4, "mfma", "bf16", "TFLOP/s"
    B, H, S, Dh = 4, 32, 4096, 128

    def work(self):
        return 4.0 * self.B * self.H * self.S * self.S * self.Dh / 2

    def config(self):
        return {"workload": "causal attention fwd bf16 B=4 H=32 S=4096 D=128",
                "batch": self.B, "heads": self.H, "seq_len": self.S, "head_dim": self.Dh}

    def setup(self, th, dev, s):
        D = th.TileDtype
        n = self.B * self.S * self.H * self.Dh
        self.bufs = []
        for j in range(3):
            b = dev.alloc(n, D.BF16)
            th.fill_random(b, n, D.BF16, "normal", 0.0, 1.0, SEED0 + 4 + 100 * j, s)
            self.bufs.append(b)
        self.o = dev.alloc(n, D.BF16)

    def step(self, th, s, i):
        q, k, v = self.bufs
        th.attention_prefill(q, k, v, self.o, self.B, self.S, 0, self.S, self.Dh, self.H, self.H,
                             th.TileDtype.BF16, s)

    emitted = ("prefill_bf16", "prefill_bf16")   # one tile per batch element

    def emitted_args(self, i):
        return self.B, self.bufs + [self.o], [self.S, 0, self.S, self.Dh, self.H, self.H]

    def cpu_sample(self, th, s, seconds):
        from oracle import oracle as orc
        q, k, v = (b.copy_to_host(s) for b in self.bufs)
        t0, flops, bh = time.perf_counter(), 0.0, 0
        while True:
            # last 64 query rows of one (b, h): the rows with the most keys
            q0 = self.S - 64
            orc.attention_prefill(q, k, v, orc.BF16, self.B, self.S, 0, self.S, self.Dh, self.H,
                                  self.H, bh0=bh % (self.B * self.H), nbh=1, q0=q0, nq=64)
            flops += sum(4.0 * (p + 1) * self.Dh for p in range(q0, self.S))
            bh += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                break
        return flops / el / 1e12, f"{bh} x 64 query rows (last rows of a head), oracle f32"


class AttnF32(Workload):
    """__tile_attention_f32 on the fp32 MFMA: 32 single-head S=4096 D=128 problems."""
    name, index, bound, dtype, unit = "attn_f32", 8, "mfma", "f32", "TFLOP/s"
    peak = PEAK_MFMA_F32_TFLOPS
    tiles, S, Dh = 32, 4096, 128

    def work(self):
        return 4.0 * self.tiles * self.S * self.S * self.Dh

    def config(self):
        return {"workload": "single-head attention f32 (non-causal), 32 problems S=4096 D=128",
                "tiles": self.tiles, "seq_len": self.S, "head_dim": self.Dh}

    def setup(self, th, dev, s):
        D = th.TileDtype
        n = self.tiles * self.S * self.Dh
        self.bufs = []
        for j in range(3):
            b = dev.alloc(n, D.F32)
            th.fill_random(b, n, D.F32, "normal", 0.0, 1.0, SEED0 + 8 + 100 * j, s)
            self.bufs.append(b)
        self.o = dev.alloc(n, D.F32)

    def step(self, th, s, i):
        q, k, v = self.bufs
        th.attention(q, k, v, self.o, self.S, self.Dh, self.tiles, th.TileDtype.F32, s)

    def cpu_sample(self, th, s, seconds):
        from oracle import oracle as orc
        q, k, v = (b.copy_to_host(s) for b in self.bufs)
        n = self.S * self.Dh
        t0, done = time.perf_counter(), 0
        while True:
            t = done % self.tiles
            sl = slice(t * n, (t + 1) * n)
            orc.attention_f32(q[sl], k[sl], v[sl], self.S, self.Dh)
            done += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                break
        return (done * 4.0 * self.S * self.S * self.Dh / el / 1e12,
                f"{done} whole problem(s) (S=4096 D=128), oracle f32")


class Decode(Workload):
    name, index, bound, dtype, unit = "decode", 5, "hbm", "bf16", "GB/s"
    B, NH, NKV, L, Dh = 64, 32, 8, 8192, 128

    def work(self):
        return 2.0 * self.B * self.NKV * self.L * self.Dh * 2

    def config(self):
        return {"workload": "GQA decode bf16 B=64 NH=32 NKV=8 L=8192 D=128", "batch": self.B,
                "heads": self.NH, "kv_heads": self.NKV, "kv_len": self.L, "head_dim": self.Dh}

    def setup(self, th, dev, s):
        D = th.TileDtype
        nq, nkv = self.B * self.NH * self.Dh, self.B * self.NKV * self.L * self.Dh
        self.q = dev.alloc(nq, D.BF16)
        self.k = dev.alloc(nkv, D.BF16)
        self.v = dev.alloc(nkv, D.BF16)
        self.o = dev.alloc(nq, D.BF16)
        th.fill_random(self.q, nq, D.BF16, "normal", 0.0, 1.0, SEED0 + 5, s)
        th.fill_random(self.k, nkv, D.BF16, "normal", 0.0, 1.0, SEED0 + 105, s)
        th.fill_random(self.v, nkv, D.BF16, "normal", 0.0, 1.0, SEED0 + 205, s)
        wsz = th.attention_decode_workspace_size(self.B, self.L, self.Dh, self.NH, self.NKV)
        self.ws = dev.alloc(wsz // 4, D.F32)
        self.wsz = wsz

    def step(self, th, s, i):
        th.attention_decode(self.q, self.k, self.v, self.o, self.B, self.L, self.L, self.Dh,
                            self.NH, self.NKV, th.TileDtype.BF16, self.ws, self.wsz, s)

    emitted = ("decode_bf16", "decode_bf16")   # one tile per batch element

    def emitted_args(self, i):
        return self.B, [self.q, self.k, self.v, self.o], [self.L, self.L, self.Dh, self.NH, self.NKV]

    def cpu_sample(self, th, s, seconds):
        from oracle import oracle as orc
        q, k, v = (b.copy_to_host(s) for b in (self.q, self.k, self.v))
        t0, bh = time.perf_counter(), 0
        while True:
            orc.attention_decode(q, k, v, orc.BF16, self.B, self.L, self.L, self.Dh, self.NH,
                                 self.NKV, bh0=bh % (self.B * self.NH), nbh=self.NH // self.NKV)
            bh += self.NH // self.NKV
            el = time.perf_counter() - t0
            if el >= seconds:
                break
        kv_bytes = (bh // (self.NH // self.NKV)) * self.L * self.Dh * 2 * 2
        return kv_bytes / el / 1e9, f"{bh} query heads ({bh // 4} kv heads x 8192 positions)"


class Copy(Workload):
    """Calibration only: a 1 GiB device-to-device copy of known size, whose HBM
    counters (FETCH_SIZE / WRITE_SIZE) scale the counters of the tile kernels."""
    name, index, bound, dtype, unit = "copy", 0, "hbm", "u8", "GB/s"
    nbytes = 1 << 30

    def work(self):
        return 2.0 * self.nbytes

    def config(self):
        return {"workload": "device-to-device copy, 1 GiB (counter calibration)"}

    def setup(self, th, dev, s):
        self.src = dev.alloc(self.nbytes // 4, th.TileDtype.F32)
        self.dst = dev.alloc(self.nbytes // 4, th.TileDtype.F32)
        th.lib().th_memset_async(self.src.as_raw_ptr(), 1, self.nbytes, s.handle)

    def step(self, th, s, i):
        from tilers_hip._lib import check
        check(th.lib().th_memcpy_dtod_async(self.dst.as_raw_ptr(), self.src.as_raw_ptr(),
                                            self.nbytes, s.handle))

    def cpu_sample(self, th, s, seconds):
        return 0.0, "none"


WORKLOADS = {w.name: w for w in (Softmax, Gemm, Mlp, Attn, Decode, Swiglu, RmsNorm, GemmF32,
                                  AttnF32, Copy)}
BENCH_LINES = ("attn", "decode", "gemm", "mlp", "softmax")


def measured_traffic(name: str):
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes (profiles/hbm_traffic.json), or None."""
    try:
        t = json.loads((ROOT / "profiles" / "hbm_traffic.json").read_text())
        return round(t[name]["traffic_bytes"])
    except (OSError, KeyError, ValueError):
        return None


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def run(name: str, steps: int, warmup: int, cpu_seconds: float, settle_ms: float,
        path: str = "library") -> dict:
    import tilers_hip as th
    w = WORKLOADS[name]()
    dev = th.HipDevice(0)
    s = dev.create_stream()
    log(f"[bench] {name}: setup on {dev.name()} ({dev.arch()}), {path} path")
    w.setup(th, dev, s)
    if path == "emitted":
        from tilers_hip import _build
        if w.emitted is None:
            raise SystemExit(f"bench.py: no emitted kernel for --config {name}")
        w.launcher = dev.create_launcher()
        w.launcher.load(_build.example_path(w.emitted[0]), th.KernelMode.GENERAL)
        w.step = lambda th_, s_, i: w.emitted_step(th_, s_, i)
    s.synchronize()
    settle_steps, t0 = 0, time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < settle_ms:
        for _ in range(10):
            w.step(th, s, settle_steps)
            settle_steps += 1
        s.synchronize()
    settle_wall = (time.perf_counter() - t0) * 1e3
    for i in range(warmup):
        w.step(th, s, i)
    s.synchronize()
    # Events go between groups of consecutive steps (about 1 ms of work each, at least
    # ten groups): an event between every step of a ~10 us kernel adds a few us of gap.
    est_ms = settle_wall / max(settle_steps, 1)
    group = max(1, min(max(steps // 10, 1), int(round(1.0 / max(est_ms, 1e-3)))))
    bounds = list(range(0, steps, group)) + [steps]
    ev = [th.HipEvent() for _ in bounds]
    ev[0].record(s)
    for g in range(len(bounds) - 1):
        for i in range(bounds[g], bounds[g + 1]):
            w.step(th, s, warmup + i)
        ev[g + 1].record(s)
    ev[-1].synchronize()
    s.synchronize()
    per = sorted(ev[g].elapsed_ms(ev[g + 1]) / (bounds[g + 1] - bounds[g])
                 for g in range(len(bounds) - 1))
    n = len(per)
    ms = per[n // 2] if n % 2 else 0.5 * (per[n // 2 - 1] + per[n // 2])
    ms_mean = ev[0].elapsed_ms(ev[-1]) / steps
    work = w.work()
    if w.unit == "TFLOP/s":
        value, peak = work / (ms * 1e-3) / 1e12, w.peak or PEAK_MFMA_TFLOPS
    else:
        value, peak = work / (ms * 1e-3) / 1e9, w.peak or PEAK_HBM_GBS
    log(f"[bench] {name}: median {ms * 1e3:.1f} us/step (mean {ms_mean * 1e3:.1f}, settle "
        f"{settle_steps} steps / {settle_wall:.0f} ms), {value:.1f} {w.unit} ({value / peak:.1%} of peak)")
    cpu = None
    if cpu_seconds > 0:
        from oracle import oracle as orc
        log(f"[bench] {name}: timing the CPU oracle for ~{cpu_seconds:.0f} s")
        cv, sample = w.cpu_sample(th, s, cpu_seconds)
        cpu = {"value": round(cv, 6), "unit": w.unit, "cores": orc.num_threads(), "kind": "port",
               "sample": sample, "cpu_model": cpu_model()}
    return {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": w.unit,
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 6),
        "ms_per_step_mean": round(ms_mean, 6),
        "timing": {"statistic": "median over groups of consecutive steps (HIP events)",
                   "steps_per_group": group, "groups": n, "settle_steps": settle_steps,
                   "settle_ms": round(settle_wall, 1)},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": "synthetic (seeded on-device PRNG, inputs resident in HBM)",
        "config": dict(w.config(), **({"path": "emitted: " + w.emitted[1]} if path == "emitted" else {})),
        "roofline": {"bound": w.bound, "achieved": round(value, 3), "peak": peak, "unit": w.unit,
                     "frac": round(value / peak, 4), "traffic": measured_traffic(name)},
        "cpu_baseline": cpu,
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # enough untimed steps for the GPU clock to settle (tens of ms of MFMA work)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--config", default="gemm", choices=sorted(WORKLOADS) + ["all"])
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--settle-ms", type=float, default=300.0,
                    help="wall time of untimed steps before the warmup (clock ramp)")
    ap.add_argument("--path", default="library", choices=("library", "emitted"),
                    help="library: the C-ABI tile op; emitted: the tile_std kernel from the "
                         "hip codegen target (tilers_hip/examples), launched by name")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: the tile ops shard with no exchange step "
              "(rows / tiles / heads per GPU), and this build runs on a single GPU only; "
              "use --gpus 1.", file=sys.stderr)
        return 2
    names = list(BENCH_LINES) if args.config == "all" else [args.config]
    for n in names:
        print(json.dumps(run(n, args.steps, args.warmup, args.cpu_seconds, args.settle_ms,
                             args.path)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
