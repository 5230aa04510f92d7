"""Benchmark of the GGUF quantized-matmul path on one MI355X.

Headline (BASELINE.json metric "GEMV HBM GB/s & GEMM TFLOPS per quant
format, % of MI355X roofline", configs[1]): Q4_0 decode GEMV, weight
11008x4096 N(0,0.02) quantized to Q4_0, activation batch 1 of 4096 f32
N(0,1).  A step is one GEMV over device-resident inputs; weights rotate
over enough copies (> 2 x 256 MB) that each step streams its weight from
HBM rather than the Infinity Cache.  `value` is algorithmic bytes per step
(weight bytes + 4 k + 4 n) / time per step.  Other formats/configs are
reported under "per_format".  The CPU baseline is the oracle (a C
restatement of the reference's mm_1d, one task per output row over the
host cores) timed on a bounded sample of the same workload.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--mode q8|exact] [--no-cpu] [--quick]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense bf16/fp16
INFINITY_CACHE = 256 << 20


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Hip:
    """The few HIP runtime calls the timing needs (events on a stream)."""

    def __init__(self):
        self.L = ctypes.CDLL("libamdhip64.so.7")
        for n in ("hipEventCreate", "hipEventRecord", "hipEventSynchronize", "hipEventElapsedTime",
                  "hipEventDestroy", "hipDeviceSynchronize"):
            getattr(self.L, n).restype = ctypes.c_int
        self.L.hipEventCreate.argtypes = [ctypes.c_void_p]
        self.L.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.L.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.L.hipEventElapsedTime.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        self.L.hipEventDestroy.argtypes = [ctypes.c_void_p]
        for n in ("hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate", "hipGraphLaunch",
                  "hipGraphExecDestroy", "hipGraphDestroy"):
            getattr(self.L, n).restype = ctypes.c_int
        self.L.hipStreamBeginCapture.argtypes = [ctypes.c_void_p, ctypes.c_int]
        self.L.hipStreamEndCapture.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.L.hipGraphInstantiate.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                               ctypes.c_char_p, ctypes.c_size_t]
        self.L.hipGraphLaunch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.L.hipGraphExecDestroy.argtypes = [ctypes.c_void_p]
        self.L.hipGraphDestroy.argtypes = [ctypes.c_void_p]

    def capture(self, stream, body):
        """Record body() (launches on `stream`) into an executable graph, so
        the timed replay is not bound by host launch overhead."""
        assert self.L.hipStreamBeginCapture(ctypes.c_void_p(stream), 1) == 0  # thread-local mode
        try:
            body()
        finally:
            g = ctypes.c_void_p()
            rc = self.L.hipStreamEndCapture(ctypes.c_void_p(stream), ctypes.byref(g))
        assert rc == 0, f"hipStreamEndCapture rc={rc}"
        ex = ctypes.c_void_p()
        assert self.L.hipGraphInstantiate(ctypes.byref(ex), g, None, None, 0) == 0
        return g, ex

    def launch(self, ex, stream):
        assert self.L.hipGraphLaunch(ex, ctypes.c_void_p(stream)) == 0

    def destroy(self, g, ex):
        self.L.hipGraphExecDestroy(ex)
        self.L.hipGraphDestroy(g)

    def event(self):
        e = ctypes.c_void_p()
        assert self.L.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def record(self, e, stream):
        assert self.L.hipEventRecord(e, ctypes.c_void_p(stream)) == 0

    def elapsed_ms(self, a, b) -> float:
        assert self.L.hipEventSynchronize(b) == 0
        ms = ctypes.c_float()
        assert self.L.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value

    def sync(self):
        assert self.L.hipDeviceSynchronize() == 0


def gemv_bytes(dt, n, k, t=1):
    import oracle as O
    return O.tensor_byte_size(dt, n * k) + 4 * k * t + 4 * n * t


def make_weight(seed, dt, n, k):
    import oracle as O
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    return O.quantize(w, dt)


def time_gemv(hip, ctx, dt, n, k, t_rows, mode, steps, warmup, seed):
    """Time `steps` device-resident GEMVs rotating over weight copies."""
    import rce_amd
    b = make_weight(seed, dt, n, k)
    copies = max(2, min(64, (2 * INFINITY_CACHE) // b.size + 1))
    ws = [rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k) for _ in range(copies)]
    rng = np.random.default_rng(seed + 1)
    x = rng.standard_normal((t_rows, k)).astype(np.float32)
    xa = rce_amd.DeviceBuffer.from_numpy(ctx, x)
    out = rce_amd.DeviceBuffer(ctx, 4 * n * t_rows)
    stream = ctx.stream

    def run(count):
        for i in range(count):
            rce_amd.mm_batched_dev(ctx, xa.ptr, rce_amd.GgufDtype.F32, t_rows, ws[i % copies], out.ptr, mode)

    run(max(1, warmup))  # untimed, eager (also sizes any scratch before capture)
    ctx.synchronize()
    g, ex = hip.capture(stream, lambda: run(steps))
    hip.launch(ex, stream)  # untimed replay
    ctx.synchronize()
    e0, e1 = hip.event(), hip.event()
    hip.record(e0, stream)
    hip.launch(ex, stream)
    hip.record(e1, stream)
    ms = hip.elapsed_ms(e0, e1) / steps
    ctx.synchronize()
    hip.destroy(g, ex)
    res = out.download(np.float32, n * t_rows).reshape(t_rows, n)
    for w in ws:
        w.close()
    xa.free(); out.free()
    return ms, b, x, res, copies


def cpu_baseline(b, x, dt, n, k, budget_s=10.0):
    """Oracle (C restatement of mm_1d, OpenMP over rows) on the same workload."""
    import oracle as O
    threads = O.max_threads()
    O.mm_batched(x, b, dt, n, k, threads)  # warm
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        O.mm_batched(x, b, dt, n, k, threads)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return med, threads, len(times)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--mode", choices=["q8", "exact"], default="q8")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline only, no per-format sweep")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import oracle as O
    import rce_amd
    from rce_amd import Mode
    hip = Hip()
    ctx = rce_amd.Context(0)
    mode = Mode.Q8 if args.mode == "q8" else Mode.EXACT

    # ---- headline: configs[1], Q4_0 11008x4096, batch 1 -------------------------
    dt, n, k = O.Q4_0, 11008, 4096
    log(f"headline Q4_0 GEMV {n}x{k} batch 1 mode={args.mode} steps={args.steps} warmup={args.warmup}")
    ms, b, x, res, copies = time_gemv(hip, ctx, dt, n, k, 1, mode, args.steps, args.warmup, 11)
    nbytes = gemv_bytes(dt, n, k, 1)
    gbs = nbytes / (ms * 1e-3) / 1e9
    ref = O.mm_batched(x, b, dt, n, k) if mode == Mode.EXACT else O.mm_batched_q8(x, b, dt, n, k)
    exact_ok = bool(np.array_equal(res.view(np.uint32), ref.view(np.uint32)))
    log(f"  {ms * 1e3:.2f} us/step  {gbs:.0f} GB/s  ({gbs / HBM_PEAK_GBS:.1%} of HBM peak)  parity={exact_ok}")

    line = {
        "metric": "GEMV HBM GB/s (Q4_0 decode, 11008x4096, batch 1)",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 dot (Q8 activations) -> f32" if mode == Mode.Q8 else "f32 (reference order)",
        "data": "synthetic: W~N(0,0.02) seeded then GGUF-quantized, x~N(0,1); weights rotated over "
                f"{copies} HBM copies",
        "config": {"workload": "configs[1] Q4_0 GEMV 11008x4096 batch 1", "mode": args.mode,
                   "bytes_per_step": nbytes, "parity_bit_exact": exact_ok},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
    }

    # ---- per-format sweep (BASELINE metric is per quant format) ------------------
    per = {}
    if not args.quick:
        sweep = [
            ("Q8_0 4096x4096 b1", O.Q8_0, 4096, 4096, 1),
            ("Q4_0 11008x4096 b1", O.Q4_0, 11008, 4096, 1),
            ("Q4_0 11008x4096 b8", O.Q4_0, 11008, 4096, 8),
            ("Q4_K 4096x4096 b1", O.Q4_K, 4096, 4096, 1),
            ("Q4_K 5632x2048 b1", O.Q4_K, 5632, 2048, 1),
            ("Q6_K 32000x2048 b1", O.Q6_K, 32000, 2048, 1),
        ]
        for name, sdt, sn, sk, st in sweep:
            for m in (Mode.EXACT, Mode.Q8):
                steps = max(20, args.steps // 2)
                sms, sb, sx, sres, _ = time_gemv(hip, ctx, sdt, sn, sk, st, m, steps, 5, 100 + sdt)
                sbytes = gemv_bytes(sdt, sn, sk, st)
                sg = sbytes / (sms * 1e-3) / 1e9
                key = f"{name} {m.name.lower()}"
                per[key] = {"us": round(sms * 1e3, 2), "GB/s": round(sg, 1), "hbm_frac": round(sg / HBM_PEAK_GBS, 4)}
                log(f"  {key}: {sms * 1e3:.2f} us  {sg:.0f} GB/s ({sg / HBM_PEAK_GBS:.1%})")
    line["per_format"] = per

    # ---- CPU baseline (oracle, same workload, bounded sample) ---------------------
    if not args.no_cpu:
        log("cpu baseline: oracle mm_1d on the headline workload (~10 s sample)")
        med, threads, calls = cpu_baseline(b, x, dt, n, k)
        cpu_gbs = nbytes / med / 1e9
        line["cpu_baseline"] = {"value": round(cpu_gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
                                "sample": f"{calls} calls of mm_1d Q4_0 11008x4096 batch 1 (median {med * 1e3:.1f} ms)"}
        log(f"  cpu {cpu_gbs:.2f} GB/s on {threads} threads")
    ctx.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
