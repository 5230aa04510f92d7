"""Benchmark of the GGUF quantized-matmul path on one MI355X.

Headline (BASELINE.json metric "GEMV HBM GB/s & GEMM TFLOPS per quant
format, % of MI355X roofline", configs[1]): Q4_0 decode GEMV, weight
11008x4096 N(0,0.02) quantized to Q4_0, activation batch 1 of 4096 f32
N(0,1), Q8-activation mode.  A step is one GEMV launch over device-resident
inputs; weights rotate over enough copies (> 2 x 256 MB) that each step
streams its weight from HBM rather than the Infinity Cache, and the steps
are replayed from a HIP graph.  `value` is algorithmic bytes per launch
(GGUF weight bytes + 4 k + 4 n per token) / time per launch, the time
taken with HIP events on the stream the kernels run on.  Other formats
and configs are reported under "per_format".  The CPU baseline is the
oracle (a C restatement of the reference's mm_1d, one task per output row
over the host cores) timed on a bounded sample of the same workload.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--mode q8|exact] [--no-cpu] [--quick]
python bench.py --copy-calibration   # device copies of known size (PMC scaling)
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFS = 2500.0     # MI355X dense fp16 MFMA, TFLOP/s
INFINITY_CACHE = 256 << 20
HEADLINE_PROFILE = os.path.join(ROOT, "profiles", "gemv_q4_0_11008x4096_q8_traffic.md")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Hip:
    """The few HIP runtime calls the timing needs (events, graphs, copies)."""

    def __init__(self):
        self.L = ctypes.CDLL("libamdhip64.so")
        P, S = ctypes.c_void_p, ctypes.c_size_t
        sig = {
            "hipEventCreate": [P], "hipEventRecord": [P, P], "hipEventSynchronize": [P],
            "hipEventElapsedTime": [P, P, P], "hipEventDestroy": [P], "hipDeviceSynchronize": [],
            "hipStreamBeginCapture": [P, ctypes.c_int], "hipStreamEndCapture": [P, P],
            "hipGraphInstantiate": [P, P, P, ctypes.c_char_p, S], "hipGraphLaunch": [P, P],
            "hipGraphExecDestroy": [P], "hipGraphDestroy": [P], "hipMalloc": [P, S], "hipFree": [P],
            "hipMemcpyAsync": [P, P, S, ctypes.c_int, P], "hipMemset": [P, ctypes.c_int, S],
        }
        for n, args in sig.items():
            fn = getattr(self.L, n)
            fn.restype = ctypes.c_int
            fn.argtypes = args

    def ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed with hipError {rc}")

    def capture(self, stream, body):
        """Record body() (launches on `stream`) into an executable graph, so
        the timed replay is not bound by host launch overhead."""
        self.ok(self.L.hipStreamBeginCapture(ctypes.c_void_p(stream), 1), "hipStreamBeginCapture")
        try:
            body()
        finally:
            g = ctypes.c_void_p()
            rc = self.L.hipStreamEndCapture(ctypes.c_void_p(stream), ctypes.byref(g))
        self.ok(rc, "hipStreamEndCapture")
        ex = ctypes.c_void_p()
        self.ok(self.L.hipGraphInstantiate(ctypes.byref(ex), g, None, None, 0), "hipGraphInstantiate")
        return g, ex

    def launch(self, ex, stream):
        self.ok(self.L.hipGraphLaunch(ex, ctypes.c_void_p(stream)), "hipGraphLaunch")

    def destroy(self, g, ex):
        self.L.hipGraphExecDestroy(ex)
        self.L.hipGraphDestroy(g)

    def event(self):
        e = ctypes.c_void_p()
        self.ok(self.L.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e

    def record(self, e, stream):
        self.ok(self.L.hipEventRecord(e, ctypes.c_void_p(stream)), "hipEventRecord")

    def elapsed_ms(self, a, b) -> float:
        self.ok(self.L.hipEventSynchronize(b), "hipEventSynchronize")
        ms = ctypes.c_float()
        self.ok(self.L.hipEventElapsedTime(ctypes.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value

    def timed_graph(self, stream, body, steps):
        """Capture `body` (steps launches), replay once untimed, then time one
        replay with events on `stream`; returns ms per launch."""
        g, ex = self.capture(stream, body)
        self.launch(ex, stream)
        e0, e1 = self.event(), self.event()
        self.ok(self.L.hipDeviceSynchronize(), "hipDeviceSynchronize")
        self.record(e0, stream)
        self.launch(ex, stream)
        self.record(e1, stream)
        ms = self.elapsed_ms(e0, e1) / steps
        self.destroy(g, ex)
        self.L.hipEventDestroy(e0)
        self.L.hipEventDestroy(e1)
        return ms


def make_weight(seed, dt, n, k):
    import oracle as O
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    return O.quantize(w, dt)


def gemv_bytes(dt, n, k, t=1):
    import oracle as O
    return O.tensor_byte_size(dt, n * k) + 4 * k * t + 4 * n * t


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
    ms = hip.timed_graph(stream, lambda: run(steps), steps)
    ctx.synchronize()
    res = out.download(np.float32, n * t_rows).reshape(t_rows, n)
    for w in ws:
        w.close()
    xa.free()
    out.free()
    return ms, b, x, res, copies


def time_gemm(hip, ctx, dt, n, k, m, steps, warmup, seed):
    """configs[2]-style prefill GEMM in F16_MFMA mode: A [m, k] f16 resident,
    weights rotated over HBM copies; returns ms per launch and a normwise
    check of the first 16 output rows against the oracle's exact order."""
    import oracle as O
    import rce_amd
    b = make_weight(seed, dt, n, k)
    copies = max(2, min(64, (2 * INFINITY_CACHE) // b.size + 1))
    ws = [rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k) for _ in range(copies)]
    rng = np.random.default_rng(seed + 1)
    x = rng.standard_normal((m, k)).astype(np.float16)
    xa = rce_amd.DeviceBuffer.from_numpy(ctx, x)
    out = rce_amd.DeviceBuffer(ctx, 4 * n * m)

    def run(count):
        for i in range(count):
            rce_amd.mm_batched_dev(ctx, xa.ptr, rce_amd.GgufDtype.F16, m, ws[i % copies], out.ptr,
                                   rce_amd.Mode.F16_MFMA)

    run(max(1, warmup))
    ctx.synchronize()
    ms = hip.timed_graph(ctx.stream, lambda: run(steps), steps)
    ctx.synchronize()
    res = out.download(np.float32, 16 * n).reshape(16, n)
    ref = O.mm_batched(x[:16].astype(np.float32), b, dt, n, k)
    err = float(np.max(np.abs(res.astype(np.float64) - ref)) / np.max(np.abs(ref)))
    for w in ws:
        w.close()
    xa.free()
    out.free()
    return ms, err


def time_moe(hip, ctx, steps, warmup, seed, mode):
    """8 Q4_0 experts (w1 14336x4096, w2 4096x14336), 256 tokens,
    top-2 of N(0,1) router logits; ms per grouped-FFN call (all 8 experts'
    528 MB stream from HBM each call), the touched weight bytes, and a
    normwise check of the first 8 tokens against the oracle's moe_ffn."""
    import oracle as O
    import rce_amd
    E, dm, dff, T, K = 8, 4096, 14336, 256, 2
    rng = np.random.default_rng(seed)
    w1b, w2b = [], []
    for _ in range(E):
        w1b.append(O.quantize(rng.standard_normal((dff, dm), dtype=np.float32) * np.float32(0.02), O.Q4_0))
        w2b.append(O.quantize(rng.standard_normal((dm, dff), dtype=np.float32) * np.float32(0.02), O.Q4_0))
    x = rng.standard_normal((T, dm), dtype=np.float32)
    logits = rng.standard_normal((T, E), dtype=np.float32)
    ids, gw = rce_amd.moe_router(logits, K)
    W1 = [rce_amd.QuantWeight.from_owned_bytes(ctx, b, O.Q4_0, dff, dm) for b in w1b]
    W2 = [rce_amd.QuantWeight.from_owned_bytes(ctx, b, O.Q4_0, dm, dff) for b in w2b]
    bx = rce_amd.DeviceBuffer.from_numpy(ctx, x)
    bi = rce_amd.DeviceBuffer.from_numpy(ctx, ids)
    bw = rce_amd.DeviceBuffer.from_numpy(ctx, gw)
    bo = rce_amd.DeviceBuffer(ctx, T * dm * 4)

    def run(count):
        for _ in range(count):
            rce_amd.moe_ffn_dev(ctx, W1, W2, bx.ptr, T, bi.ptr, bw.ptr, K, bo.ptr, mode)

    run(max(1, warmup))  # sizes scratch and uploads the expert tables before capture
    ctx.synchronize()
    ms = hip.timed_graph(ctx.stream, lambda: run(steps), steps)
    ctx.synchronize()
    got = bo.download(np.float32, T * dm).reshape(T, dm)[:8]
    ref = O.moe_ffn(x[:8], w1b, w2b, O.Q4_0, dff, ids[:8], gw[:8])
    err = float(np.max(np.abs(got.astype(np.float64) - ref)) / np.max(np.abs(ref)))
    touched = sorted(set(int(e) for e in ids.reshape(-1)))
    wbytes = sum(w1b[e].size + w2b[e].size for e in touched)
    for w in W1 + W2:
        w.close()
    for bb in (bx, bi, bw, bo):
        bb.free()
    return ms, err, wbytes + 2 * T * dm * 4


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
    return float(np.median(times)), threads, len(times)


def headline_traffic():
    """HBM bytes per launch of the headline kernel from the committed PMC
    summary (FETCH_SIZE + WRITE_SIZE, scaled by a copy kernel), or None."""
    try:
        text = open(HEADLINE_PROFILE).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", text)
    return int(m.group(1)) if m else None


def copy_calibration(hip, nbytes=256 << 20, reps=8):
    """Device-to-device copies of a known size: the reference reading for the
    FETCH_SIZE / WRITE_SIZE counters (bytes read = bytes written = nbytes)."""
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    hip.ok(hip.L.hipMalloc(ctypes.byref(src), nbytes), "hipMalloc")
    hip.ok(hip.L.hipMalloc(ctypes.byref(dst), nbytes), "hipMalloc")
    hip.ok(hip.L.hipMemset(src, 1, nbytes), "hipMemset")
    hip.ok(hip.L.hipMemset(dst, 0, nbytes), "hipMemset")
    hip.ok(hip.L.hipDeviceSynchronize(), "hipDeviceSynchronize")
    for _ in range(reps):
        hip.ok(hip.L.hipMemcpyAsync(dst, src, nbytes, 3, None), "hipMemcpyAsync")
    hip.ok(hip.L.hipDeviceSynchronize(), "hipDeviceSynchronize")
    hip.L.hipFree(src)
    hip.L.hipFree(dst)
    print(json.dumps({"copy_calibration_bytes": nbytes, "copies": reps}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--mode", choices=["q8", "exact"], default="q8")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline only, no per-format sweep")
    ap.add_argument("--copy-calibration", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every GPU box here has one, and this build has no multi-GPU "
              f"path (asked for --gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    hip = Hip()
    if args.copy_calibration:
        copy_calibration(hip)
        return

    import oracle as O
    import rce_amd
    from rce_amd import Mode
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
    log(f"  {ms * 1e3:.2f} us/launch  {gbs:.0f} GB/s  ({gbs / HBM_PEAK_GBS:.1%} of HBM peak)  "
        f"bit-identical to the oracle: {exact_ok}")

    line = {
        "metric": "GEMV HBM GB/s (Q4_0 decode 11008x4096, batch 1, Q8 activations)",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8" if mode == Mode.Q8 else "f32",
        "data": "synthetic: W~N(0,0.02) seeded then GGUF-quantized, x~N(0,1); weights rotated over "
                f"{copies} HBM copies",
        "config": {"workload": "configs[1]: Q4_0 GEMV 11008x4096 batch 1", "mode": args.mode,
                   "bytes_per_launch": nbytes, "parity_bit_exact": exact_ok},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": headline_traffic() if mode == Mode.Q8 else None},
    }

    # ---- per-format sweep (the metric is per quant format) -----------------------
    per = {}
    if not args.quick:
        sweep = [
            ("Q8_0 4096x4096 b1", O.Q8_0, 4096, 4096, 1),      # configs[0] shape
            ("Q4_0 11008x4096 b1", O.Q4_0, 11008, 4096, 1),    # configs[1]
            ("Q4_0 11008x4096 b8", O.Q4_0, 11008, 4096, 8),    # configs[1], batch 8
            ("Q4_K 4096x4096 b1", O.Q4_K, 4096, 4096, 1),
            ("Q4_K 5632x2048 b1", O.Q4_K, 5632, 2048, 1),      # configs[4] FFN shapes
            ("Q4_K 2048x5632 b1", O.Q4_K, 2048, 5632, 1),
            ("Q6_K 32000x2048 b1", O.Q6_K, 32000, 2048, 1),    # configs[4] head
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
        # Q4_K prefill GEMM 512x4096x4096 on f16 MFMA
        gms, gerr = time_gemm(hip, ctx, O.Q4_K, 4096, 4096, 512, max(20, args.steps // 4), 5, 300)
        gtf = 2.0 * 512 * 4096 * 4096 / (gms * 1e-3) / 1e12
        per["Q4_K GEMM 512x4096x4096 f16_mfma"] = {
            "us": round(gms * 1e3, 2), "TFLOP/s": round(gtf, 1), "mfma_frac": round(gtf / MFMA_F16_PEAK_TFS, 4),
            "normwise_err_vs_oracle": float(f"{gerr:.3g}")}
        log(f"  Q4_K GEMM 512x4096x4096: {gms * 1e3:.2f} us  {gtf:.0f} TFLOP/s ({gtf / MFMA_F16_PEAK_TFS:.1%} of "
            f"f16 MFMA peak), normwise err {gerr:.2e}")
        # grouped MoE, 8 Q4_0 experts, 256 tokens, top-2
        mms, merr, mbytes = time_moe(hip, ctx, 5, 2, 400, Mode.F16_MFMA)
        mtf = 120259084288 / (mms * 1e-3) / 1e12
        mgb = mbytes / (mms * 1e-3) / 1e9
        per["MoE 8x(14336x4096, 4096x14336) Q4_0 T256 top2 f16_mfma"] = {
            "us": round(mms * 1e3, 2), "TFLOP/s": round(mtf, 1), "mfma_frac": round(mtf / MFMA_F16_PEAK_TFS, 4),
            "GB/s": round(mgb, 1), "hbm_frac": round(mgb / HBM_PEAK_GBS, 4),
            "normwise_err_vs_oracle": float(f"{merr:.3g}")}
        log(f"  MoE configs[3]: {mms * 1e3:.1f} us  {mtf:.0f} TFLOP/s ({mtf / MFMA_F16_PEAK_TFS:.1%}), "
            f"{mgb:.0f} GB/s ({mgb / HBM_PEAK_GBS:.1%}), normwise err {merr:.2e}")
    line["per_format"] = per

    # ---- CPU baseline (oracle, same workload, bounded sample) ---------------------
    if not args.no_cpu:
        log("cpu baseline: oracle mm_1d on the headline workload (~10 s sample)")
        med, threads, calls = cpu_baseline(b, x, dt, n, k)
        cpu_gbs = nbytes / med / 1e9
        line["cpu_baseline"] = {"value": round(cpu_gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
                                "sample": f"{calls} calls of mm_1d (f32 activations, reference order) on the "
                                          f"headline Q4_0 11008x4096 batch-1 workload, median {med * 1e3:.2f} ms"}
        log(f"  cpu {cpu_gbs:.2f} GB/s on {threads} threads")
    ctx.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
