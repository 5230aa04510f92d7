"""Benchmark of the GGUF quantized-matmul path on one MI355X.

Headline (BASELINE.json metric "GEMV HBM GB/s & GEMM TFLOPS per quant
format, % of MI355X roofline", configs[1]): Q4_0 decode GEMV, weight
11008x4096 N(0,0.02) quantized to Q4_0, activation batch 1 of 4096 f32
N(0,1), in the reference's own f32 order (EXACT mode, bit-identical to
mm_1d; --mode q8 for the Q8-activation mode).  A step is one GEMV launch over device-resident
inputs; weights rotate over enough copies (> 2 x 256 MB) that each step
streams its weight from HBM rather than the Infinity Cache, and the steps
are replayed from a HIP graph.  `value` is algorithmic bytes per launch
(GGUF weight bytes + 4 k + 4 n per token) / time per launch, the time
taken with HIP events on the stream the kernels run on.  Next to the
8 TB/s datasheet peak the line reports the measured read ceiling: the
fastest single launch that only reads the same number of bytes
(rce_qmm_read_ceiling_dev, weights rotated the same way).  Other formats
and configs are reported under "per_format".  The CPU baseline is the
oracle (a C restatement of the reference's mm_1d, one task per output row
over the host cores) timed on a bounded sample of the same workload.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--mode exact|q8] [--no-cpu] [--quick]
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
# Committed HBM-traffic summaries of the headline kernel, per mode; each
# records the SHA-256 of the kernel sources it was measured on.
TRAFFIC_PROFILE = {"exact": os.path.join(ROOT, "profiles", "gemv_q4_0_11008x4096_exact_traffic.md"),
                   "q8": os.path.join(ROOT, "profiles", "gemv_q4_0_11008x4096_q8_traffic.md")}
KERNEL_SOURCES = ("rce_amd/csrc/qmm_gemv_kernels.h", "rce_amd/csrc/gemv_q4_0.hip", "rce_amd/csrc/qmm_gemv.hip",
                  "rce_amd/csrc/qmm_internal.h")


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


# F32, F16, BF16, I2_S, Q1_0, Q2_0, STQ1_0: no Q8 form, the same kernel in both modes
FLOAT_DTYPES = (0, 1, 30, 36, 41, 42, 0x8000002A)


def make_weight(seed, dt, n, k):
    """N(0, 0.02) f32 weights (seeded) as GGUF bytes: by the library's
    quantizer (the reference's encoders) where it has one, as the values
    themselves for F32 / F16 / BF16, and as random blocks (random bit
    fields, f16 scales of about 0.002) for Q5_0 / Q4_1 / Q3_K, which the
    reference ships no encoder for."""
    import rce_amd
    rng = np.random.default_rng(seed)
    if int(dt) in (36, 41, 42, 0x8000002A):  # multiply-free formats: random codes, scales about 0.02
        qk, bb = {36: (128, 32), 41: (128, 18), 42: (128, 34), 0x8000002A: (256, 42)}[int(dt)]
        b = rng.integers(0, 256, size=n * (k // qk) * bb + (4 if int(dt) == 36 else 0), dtype=np.uint8)
        if int(dt) == 36:
            b[-4:] = np.frombuffer(np.float32(0.02).tobytes(), np.uint8)
        else:
            bl = b.reshape(-1, bb)
            at = 40 if int(dt) == 0x8000002A else 0
            bl[:, at:at + 2] = np.frombuffer(np.float16(0.02).tobytes(), np.uint8)
        return b
    if int(dt) in (3, 6, 11):
        qk, bb = (256, 110) if int(dt) == 11 else (32, 20 if int(dt) == 3 else 22)
        b = rng.integers(0, 256, size=(n * (k // qk), bb), dtype=np.uint8)
        d = rng.uniform(0.0005, 0.004, b.shape[0]).astype(np.float16).view(np.uint8).reshape(-1, 2)
        if int(dt) == 11:
            b[:, 108:110] = d
        else:
            b[:, 0:2] = d
        if int(dt) == 3:  # Q4_1's f16 min: finite, of the size of the values
            b[:, 2:4] = rng.uniform(-0.03, 0.03, b.shape[0]).astype(np.float16).view(np.uint8).reshape(-1, 2)
        return b.reshape(-1)
    w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
    if int(dt) == 0:
        return w.view(np.uint8).reshape(-1)
    if int(dt) == 1:
        return w.astype(np.float16).view(np.uint8).reshape(-1)
    if int(dt) == 30:
        return (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1)
    return rce_amd.quantize(w, dt)


def gemv_bytes(dt, n, k, t=1):
    import rce_amd
    return n * rce_amd.row_bytes(dt, k) + 4 * k * t + 4 * n * t


def time_gemv(hip, ctx, dt, n, k, t_rows, mode, steps, warmup, seed, settle_s=0.0):
    """Time `steps` device-resident GEMVs rotating over weight copies.
    settle_s: seconds of untimed launches first (see settle)."""
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

    settle(ctx, run, settle_s)
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


def settle(ctx, run, settle_s):
    """settle_s seconds of untimed launches: an idle GPU's clocks ramp up
    over the first tens of milliseconds of work (measured: the Q4_K GEMM
    takes 32 us per launch on a freshly idle GPU, 27 us once warm)."""
    t0 = time.time()
    while time.time() - t0 < settle_s:
        run(16)
        ctx.synchronize()


def time_gemm(hip, ctx, dt, n, k, m, steps, warmup, seed, settle_s=0.2):
    """configs[2]-style prefill GEMM in F16_MFMA mode: A [m, k] f16 resident,
    weights rotated over HBM copies; returns ms per launch and the first 16
    output rows (checked in the CPU leg)."""
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

    settle(ctx, run, settle_s)
    run(max(1, warmup))
    ctx.synchronize()
    ms = hip.timed_graph(ctx.stream, lambda: run(steps), steps)
    ctx.synchronize()
    res = out.download(np.float32, 16 * n).reshape(16, n)
    for w in ws:
        w.close()
    xa.free()
    out.free()
    # the first 16 rows, for the parity check of the CPU leg
    return ms, {"b": b, "x": x[:16].astype(np.float32), "got": res, "dt": dt, "n": n, "k": k}


def time_moe(hip, ctx, steps, warmup, seed, mode, settle_s=0.2, dtype=None):
    """8 Q4_0 experts (w1 14336x4096, w2 4096x14336), 256 tokens,
    top-2 of N(0,1) router logits; ms per grouped-FFN call (all 8 experts'
    weights stream from HBM each call), the touched weight bytes, and a
    sample of the first 8 tokens (checked in the CPU leg).  dtype: the same
    workload with experts of another format (per-format rows)."""
    import rce_amd
    dt = rce_amd.GgufDtype.Q4_0 if dtype is None else dtype
    E, dm, dff, T, K = 8, 4096, 14336, 256, 2
    rng = np.random.default_rng(seed)
    w1b, w2b = [], []
    for _ in range(E):
        w1b.append(rce_amd.quantize(rng.standard_normal((dff, dm), dtype=np.float32) * np.float32(0.02), dt))
        w2b.append(rce_amd.quantize(rng.standard_normal((dm, dff), dtype=np.float32) * np.float32(0.02), dt))
    x = rng.standard_normal((T, dm), dtype=np.float32)
    logits = rng.standard_normal((T, E), dtype=np.float32)
    ids, gw = rce_amd.moe_router(logits, K)
    W1 = [rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, dff, dm) for b in w1b]
    W2 = [rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, dm, dff) for b in w2b]
    bx = rce_amd.DeviceBuffer.from_numpy(ctx, x)
    bi = rce_amd.DeviceBuffer.from_numpy(ctx, ids)
    bw = rce_amd.DeviceBuffer.from_numpy(ctx, gw)
    bo = rce_amd.DeviceBuffer(ctx, T * dm * 4)

    def run(count):
        for _ in range(count):
            rce_amd.moe_ffn_dev(ctx, W1, W2, bx.ptr, T, bi.ptr, bw.ptr, K, bo.ptr, mode)

    run(max(1, warmup))  # sizes scratch and uploads the expert tables before capture
    ctx.synchronize()
    settle(ctx, run, settle_s)
    ms = hip.timed_graph(ctx.stream, lambda: run(steps), steps)
    ctx.synchronize()
    got = bo.download(np.float32, T * dm).reshape(T, dm)[:8]
    touched = sorted(set(int(e) for e in ids.reshape(-1)))
    wbytes = sum(w1b[e].size + w2b[e].size for e in touched)
    for w in W1 + W2:
        w.close()
    for bb in (bx, bi, bw, bo):
        bb.free()
    sample = {"x": x[:8], "w1": w1b, "w2": w2b, "dff": dff, "ids": ids[:8], "gw": gw[:8], "got": got, "dtype": int(dt)}
    return ms, wbytes + 2 * T * dm * 4, sample


LLAMA_CFG = dict(d_model=2048, vocab=32000, n_layers=22, n_q_heads=32, n_kv_heads=4, d_head=64, rope_dim=64,
                 rope_freq_base=10000.0, d_ff=5632, context_length=2048, eps=1e-5)
LLAMA_WEIGHT_BYTES = 598_757_376  # 22 x 24,772,608 B of Q4_K linears + the 53,760,000 B Q6_K head


def llama_weights(seed):
    """TinyLlama-shaped random decoder, every weight N(0, 0.02)
    quantized (Q4_K linears and token_embd, Q6_K head), norms = 1."""
    import rce_amd
    G = rce_amd.GgufDtype
    c = LLAMA_CFG
    rng = np.random.default_rng(seed)
    dm, qd, kvd, ff = c["d_model"], c["n_q_heads"] * c["d_head"], c["n_kv_heads"] * c["d_head"], c["d_ff"]
    shapes = {"wq": (qd, dm), "wk": (kvd, dm), "wv": (kvd, dm), "wo": (dm, qd),
              "ffn_gate": (ff, dm), "ffn_up": (ff, dm), "ffn_down": (dm, ff)}

    def q(n, k, dt):
        return rce_amd.quantize(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02), dt), dt

    ones = np.ones(dm, np.float32)
    blocks = [dict({"attn_norm": ones, "ffn_norm": ones}, **{nm: q(*sh, G.Q4K) for nm, sh in shapes.items()})
              for _ in range(c["n_layers"])]
    return {"cfg": dict(c), "token_embd": q(c["vocab"], dm, G.Q4K), "output_norm": ones,
            "lm_head": q(c["vocab"], dm, G.Q6K), "blocks": blocks, "shapes": shapes}


def time_llama(hip, ctx, W, mode, steps, warmup, seed):
    """Batch-1 decode of `warmup` then `steps` tokens from position 0 through
    the device-resident decoder (one embed kernel + one graph replay per
    token, on the context's stream); ms per token over the timed tokens and
    the first 4 tokens' logits (checked in the CPU leg)."""
    import rce_amd
    c = W["cfg"]
    qw = lambda bd, n, k: rce_amd.QuantWeight.from_owned_bytes(ctx, bd[0], bd[1], n, k)  # noqa: E731
    blocks = [rce_amd.TinyLlamaBlock(b["attn_norm"], b["ffn_norm"],
                                     **{nm: qw(b[nm], *W["shapes"][nm]) for nm in W["shapes"]}) for b in W["blocks"]]
    weights = rce_amd.TinyLlamaWeights(qw(W["token_embd"], c["vocab"], c["d_model"]), W["output_norm"],
                                       qw(W["lm_head"], c["vocab"], c["d_model"]), blocks)
    dec = rce_amd.TinyLlamaRuntime(ctx, rce_amd.TinyLlamaConfig(**c), weights, mode)
    del blocks, weights  # the decoder holds the device weights
    toks = np.random.default_rng(seed).integers(0, c["vocab"], warmup + steps).astype(np.int32)
    first = [dec.forward_logits(int(t)) for t in toks[:4]]  # host entry point, also records the graph
    dec.new_state()
    tb = rce_amd.DeviceBuffer.from_numpy(ctx, toks)
    lo = rce_amd.DeviceBuffer(ctx, 4 * c["vocab"])
    for i in range(warmup):
        dec.forward_token_dev(tb.ptr + 4 * i, lo.ptr)
    ctx.synchronize()
    e0, e1 = hip.event(), hip.event()
    hip.record(e0, ctx.stream)
    h0 = time.perf_counter()
    for i in range(warmup, warmup + steps):
        dec.forward_token_dev(tb.ptr + 4 * i, lo.ptr)
    host_ms = (time.perf_counter() - h0) * 1e3 / steps  # submission only
    hip.record(e1, ctx.stream)
    ms = hip.elapsed_ms(e0, e1) / steps
    log(f"  decode: {ms * 1e3:.1f} us/token on the stream, host submission {host_ms * 1e3:.1f} us/token")
    dec.check()
    dec.close()
    tb.free()
    lo.free()
    return ms, {"tokens": [int(t) for t in toks[:4]], "got": first}


def cpu_model() -> str:
    """The host CPU's model name (what lscpu reports as "Model name")."""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_leg(line, head, rows, budget_s=10.0):
    """The CPU baseline and the parity checks (the only part of the bench
    that uses the oracle, the C restatement of the reference path).

    Baseline: the oracle's mm_1d (OpenMP over rows, the reference's rayon
    decomposition) timed on the headline workload for about budget_s
    seconds.  Checks: the headline GEMV result against the oracle's (bit
    identity), and each per-format row's kept sample against the oracle's
    reference order (normwise error)."""
    import oracle as O
    threads = O.max_threads()
    b, x, dt, n, k, res, mode = (head[key] for key in ("b", "x", "dt", "n", "k", "res", "mode"))
    want = O.mm_batched(x, b, dt, n, k, threads)  # also the warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        O.mm_batched(x, b, dt, n, k, threads)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    cpu_gbs = gemv_bytes(dt, n, k, 1) / med / 1e9
    line["cpu_baseline"] = {"value": round(cpu_gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
                            "cpu_model": cpu_model(),
                            "sample": f"{len(times)} calls of mm_1d (f32 activations, reference order) on the "
                                      f"headline Q4_0 11008x4096 batch-1 workload, median {med * 1e3:.2f} ms"}
    log(f"  cpu {cpu_gbs:.2f} GB/s on {threads} threads")
    ref = want if mode == 0 else O.mm_batched_q8(x, b, dt, n, k, threads)
    line["config"]["parity_bit_exact"] = bool(np.array_equal(res.view(np.uint32), ref.view(np.uint32)))
    log(f"  headline bit-identical to the oracle: {line['config']['parity_bit_exact']}")

    def normwise(got, want):
        return float(f"{np.max(np.abs(got.astype(np.float64) - want)) / np.max(np.abs(want)):.3g}")

    per = line["per_format"]
    for gk in [r for r in rows if r.startswith("gemm")]:
        g = rows[gk]
        per[g["key"]]["normwise_err_vs_oracle"] = normwise(g["got"], O.mm_batched(g["x"], g["b"], g["dt"], g["n"], g["k"]))
    for mk in [r for r in rows if r.startswith("moe")]:
        m = rows[mk]
        ref = O.moe_ffn(m["x"], m["w1"], m["w2"], m["dtype"], m["dff"], m["ids"], m["gw"])
        per[m["key"]]["normwise_err_vs_oracle"] = normwise(m["got"], ref)
    for lk in [r for r in rows if r.startswith("llama")]:
        L = rows[lk]
        W = L["W"]
        om = O.Llama(W["cfg"], W["token_embd"], W["output_norm"], W["lm_head"], W["blocks"], q8=L["q8"], threads=threads)
        t0 = time.perf_counter()
        errs = [normwise(got, om.forward_token(t)) for t, got in zip(L["tokens"], L["got"])]
        cpu_tok_s = len(errs) / (time.perf_counter() - t0)
        per[L["key"]]["normwise_err_vs_oracle_max"] = max(errs)
        per[L["key"]]["cpu_baseline_tok_s"] = round(cpu_tok_s, 2)
        log(f"  decoder ({lk}): normwise vs oracle {max(errs):.2e} over {len(errs)} tokens; oracle {cpu_tok_s:.2f} tok/s")
    for key, row in per.items():
        if "normwise_err_vs_oracle" in row:
            log(f"  {key}: normwise vs oracle {row['normwise_err_vs_oracle']:.2e}")


def kernel_sources_sha256() -> str:
    """SHA-256 over the headline kernel's source files (the stamp a traffic
    summary must carry to be used for this build)."""
    import hashlib
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def headline_traffic(mode_name: str):
    """HBM bytes per launch of the headline kernel from the committed PMC
    summary (FETCH_SIZE + WRITE_SIZE, scaled by a copy kernel), or None
    when there is none for this mode or it was measured on other kernel
    sources than the ones built here."""
    try:
        text = open(TRAFFIC_PROFILE[mode_name]).read()
    except (OSError, KeyError):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", text)
    h = re.search(r"kernel_sources_sha256:\s*([0-9a-f]{64})", text)
    if not m or not h or h.group(1) != kernel_sources_sha256():
        log(f"  traffic summary for {mode_name} missing or measured on other kernel sources: traffic null")
        return None
    return int(m.group(1))


def read_ceiling(hip, ctx, nbytes, steps):
    """The fastest single launch that only reads nbytes (every variant of
    rce_qmm_read_ceiling_dev), over the same rotation of HBM copies as the
    GEMV: (us per launch, variant); also the empty-launch time."""
    import rce_amd
    from rce_amd import _lib
    L = _lib.lib()
    nb = (nbytes + 4095) // 4096 * 4096
    copies = max(2, min(64, (2 * INFINITY_CACHE) // nb + 1))
    buf = rce_amd.DeviceBuffer(ctx, nb * copies)
    sink = rce_amd.DeviceBuffer(ctx, 256)
    hip.ok(hip.L.hipMemset(ctypes.c_void_p(buf.ptr), 1, nb * copies), "hipMemset")
    hip.ok(hip.L.hipDeviceSynchronize(), "hipDeviceSynchronize")
    stream = ctx.stream

    def run(variant, count, n):
        for i in range(count):
            _lib.check(L.rce_qmm_read_ceiling_dev(ctx.handle, ctypes.c_void_p(buf.ptr + (i % copies) * nb), n,
                                                  ctypes.c_void_p(sink.ptr), variant, None))

    best = None
    for v in range(9):
        run(v, 3, nbytes)
        ms = hip.timed_graph(stream, lambda: run(v, steps, nbytes), steps)
        if best is None or ms < best[0]:
            best = (ms, v)
    run(9, 3, 0)
    empty_ms = hip.timed_graph(stream, lambda: run(9, steps, 0), steps)
    buf.free()
    sink.free()
    return best[0] * 1e3, best[1], empty_ms * 1e3


def cache_warmth(hip, ctx, steps=200):
    """The decode step's GEMV shapes timed three ways: weights rotated over
    copies beyond 2 x the Infinity Cache (every read from HBM), over copies
    within about 96 MB (Infinity Cache), and one copy (L2 and Infinity
    Cache warm).  Equal times mean a launch is bound by its own latency, not
    by where its bytes come from."""
    import rce_amd
    from rce_amd import GgufDtype as G, Mode
    shapes = ((G.Q4K, 2048, 2048, "Q4_K 2048x2048 (wq, wo)"), (G.Q4K, 2560, 2048, "Q4_K 2560x2048 (q|k|v)"),
              (G.Q4K, 11264, 2048, "Q4_K 11264x2048 (gate|up)"), (G.Q4K, 2048, 5632, "Q4_K 2048x5632 (down)"),
              (G.Q4_0, 11008, 4096, "Q4_0 11008x4096 (headline)"))
    out = {}
    for dt, n, k, name in shapes:
        size = make_weight(3, dt, n, k).size
        plan = (("hbm", max(2, min(64, (2 * INFINITY_CACHE) // size + 1))), ("infinity_cache", max(2, (96 << 20) // size + 1)),
                ("one_copy", 1))
        for mode, mname in ((Mode.Q8, "q8"), (Mode.EXACT, "exact")):
            row = {}
            for where, copies in plan:
                b = make_weight(3, dt, n, k)
                ws = [rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k) for _ in range(copies)]
                x = np.random.default_rng(4).standard_normal((1, k)).astype(np.float32)
                xa = rce_amd.DeviceBuffer.from_numpy(ctx, x)
                o = rce_amd.DeviceBuffer(ctx, 4 * n)

                def run(c):
                    for i in range(c):
                        rce_amd.mm_batched_dev(ctx, xa.ptr, G.F32, 1, ws[i % copies], o.ptr, mode)
                settle(ctx, run, 0.1)
                run(10)
                ctx.synchronize()
                ms = hip.timed_graph(ctx.stream, lambda: run(steps), steps)
                for w in ws:
                    w.close()
                xa.free()
                o.free()
                row[where] = {"us": round(ms * 1e3, 3), "copies": copies}
            out[f"{name} {mname}"] = row
            log(f"  cache warmth {name} {mname}: " + "  ".join(f"{k2} {v['us']:.2f} us" for k2, v in row.items()))
    return out


def read_ceilings(hip, ctx, steps=200):
    """The read ceiling (read_ceiling) at the byte counts of the decode step's
    weights and of the headline: what a single launch that only streams
    that many bytes takes, launch cost included."""
    out = {}
    for name, nbytes in (("Q4_K 2048x2048", 2359296), ("Q4_K 2560x2048", 2949120), ("Q4_K 2048x5632", 6488064),
                         ("Q4_K 4096x4096", 9469952),
                         ("Q4_K 11264x2048", 12976128), ("Q4_0 11008x4096 (headline)", 25422848),
                         ("Q6_K 32000x2048", 53760000)):
        us, var, empty = read_ceiling(hip, ctx, nbytes, steps)
        out[name] = {"bytes": nbytes, "us": round(us, 3), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "variant": var, "empty_launch_us": round(empty, 3)}
        log(f"  read ceiling {name} ({nbytes} B): {us:.2f} us ({nbytes / (us * 1e-6) / 1e9:.0f} GB/s)")
    return out


def vendor_gemm(steps=40):
    """AMD's library on the prefill shapes, no dequantization: torch.matmul
    (hipBLASLt) of f16 and bf16 operands in this path's layout, A [m, k]
    times W^T with W [n, k] row-major (a transposed 2-D view, which the
    library takes as its transpose flag), weights rotated over copies
    beyond 2 x the Infinity Cache, timed with events on torch's stream."""
    import torch
    out = {}
    for m, n, k in ((512, 4096, 4096), (2048, 4096, 4096), (4096, 4096, 4096), (64, 14336, 4096)):
        for dt, dname in ((torch.float16, "f16"), (torch.bfloat16, "bf16")):
            g = torch.Generator(device="cuda").manual_seed(1)
            a = torch.randn(m, k, device="cuda", dtype=dt, generator=g)
            copies = max(2, min(32, (2 * INFINITY_CACHE) // (2 * n * k) + 1))
            ws = [torch.randn(n, k, device="cuda", dtype=dt, generator=g) for _ in range(copies)]
            for i in range(5):
                torch.matmul(a, ws[i % copies].t())
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(steps):
                torch.matmul(a, ws[i % copies].t())
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / steps
            tf = 2.0 * m * n * k / (us * 1e-6) / 1e12
            out[f"{m}x{n}x{k} {dname}"] = {"us": round(us, 2), "tflops": round(tf, 1),
                                            "frac_of_dense_peak": round(tf / MFMA_F16_PEAK_TFS, 4)}
            log(f"  vendor GEMM {m}x{n}x{k} {dname}: {us:.2f} us  {tf:.0f} TFLOP/s")
            del ws, a
    return out


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
    ap.add_argument("--mode", choices=["exact", "q8"], default="exact")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline only, no per-format rows")
    ap.add_argument("--rows", default="sweep,gemm,moe,llama",
                    help="per-format rows: comma-separated subset of sweep,gemm,moe,llama")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--no-ceiling", action="store_true", help="skip the read-ceiling launches (profiling runs)")
    ap.add_argument("--cache-warmth", action="store_true",
                    help="also time the decode-step GEMV shapes with weights from HBM, the Infinity Cache and one copy")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="also time AMD's library (torch.matmul, f16 / bf16) on the prefill shapes")
    ap.add_argument("--read-ceilings", action="store_true",
                    help="also measure the read ceiling at the decode step's weight sizes")
    ap.add_argument("--sweep-only", default="",
                    help="run only the sweep rows whose name contains this text (e.g. 'b8'; profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every GPU box here has one, and this build has no multi-GPU "
              f"path (asked for --gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    hip = Hip()
    if args.copy_calibration:
        copy_calibration(hip)
        return

    import rce_amd
    from rce_amd import GgufDtype as G, Mode
    ctx = rce_amd.Context(0)
    mode = Mode.Q8 if args.mode == "q8" else Mode.EXACT
    rows = set() if args.quick else set(r for r in args.rows.split(",") if r)

    # ---- headline: configs[1], Q4_0 11008x4096, batch 1 -------------------------
    dt, n, k = G.Q4_0, 11008, 4096
    log(f"headline Q4_0 GEMV {n}x{k} batch 1 mode={args.mode} steps={args.steps} warmup={args.warmup}")
    ms, b, x, res, copies = time_gemv(hip, ctx, dt, n, k, 1, mode, args.steps, args.warmup, 11, settle_s=0.3)
    nbytes = gemv_bytes(dt, n, k, 1)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"  {ms * 1e3:.2f} us/launch  {gbs:.0f} GB/s  ({gbs / HBM_PEAK_GBS:.1%} of HBM peak)")
    head = {"b": b, "x": x, "dt": int(dt), "n": n, "k": k, "res": res, "mode": int(mode)}

    if args.no_ceiling:
        ceil_us, ceil_var, empty_us = float("nan"), -1, float("nan")
    else:
        ceil_us, ceil_var, empty_us = read_ceiling(hip, ctx, nbytes, args.steps)
    ceil_gbs = nbytes / (ceil_us * 1e-6) / 1e9
    log(f"  read ceiling at {nbytes} B: {ceil_us:.2f} us ({ceil_gbs:.0f} GB/s, variant {ceil_var}); "
        f"empty launch {empty_us:.2f} us")
    line = {
        "metric": "GEMV HBM GB/s (Q4_0 decode 11008x4096, batch 1, "
                  + ("Q8 activations)" if mode == Mode.Q8 else "f32 activations, reference order)"),
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
                   "bytes_per_launch": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": headline_traffic(args.mode),
                     "read_ceiling": {"GB/s": round(ceil_gbs, 1), "us": round(ceil_us, 3), "variant": ceil_var,
                                      "frac": round(gbs / ceil_gbs, 4), "empty_launch_us": round(empty_us, 3)}},
    }

    # ---- per-format rows (the metric is per quant format) ------------------------
    per = {}
    kept = {}
    if "sweep" in rows:
        sweep = [
            ("Q8_0 4096x4096 b1", G.Q8_0, 4096, 4096, 1),      # configs[0] shape
            ("Q4_0 11008x4096 b1", G.Q4_0, 11008, 4096, 1),    # configs[1]
            ("Q4_0 11008x4096 b8", G.Q4_0, 11008, 4096, 8),    # configs[1], batch 8
            ("Q4_K 4096x4096 b1", G.Q4K, 4096, 4096, 1),
            ("Q4_K 5632x2048 b1", G.Q4K, 5632, 2048, 1),       # configs[4] FFN shapes
            ("Q4_K 2048x5632 b1", G.Q4K, 2048, 5632, 1),
            ("Q5_K 4096x4096 b1", G.Q5K, 4096, 4096, 1),       # Q5_K_M models' linears
            ("Q6_K 32000x2048 b1", G.Q6K, 32000, 2048, 1),     # configs[4] head
            ("Q5_0 4096x4096 b1", G.Q5_0, 4096, 4096, 1),
            ("Q4_1 4096x4096 b1", G.Q4_1, 4096, 4096, 1),
            ("Q3_K 4096x4096 b1", G.Q3K, 4096, 4096, 1),
            ("F16 2048x2048 b1", G.F16, 2048, 2048, 1),
            ("F16 32000x2048 b1", G.F16, 32000, 2048, 1),      # an F16 head
            ("Q1_0 2048x2048 b1", G.Q1_0, 2048, 2048, 1),
            ("Q2_0 2048x2048 b1", G.Q2_0, 2048, 2048, 1),
            ("STQ1_0 2048x2048 b1", G.STQ1_0, 2048, 2048, 1),
            ("I2_S 6912x2560 b1", G.I2S, 6912, 2560, 1),       # BitNet b1.58 2B FFN up
        ]
        sweep = [r for r in sweep if args.sweep_only in r[0]]
        for name, sdt, sn, sk, st in sweep:
            for m in ((Mode.EXACT,) if int(sdt) in FLOAT_DTYPES else (Mode.EXACT, Mode.Q8)):
                steps = max(20, args.steps // 2)
                sms, _, _, _, _ = time_gemv(hip, ctx, sdt, sn, sk, st, m, steps, 5, 100 + int(sdt))
                sbytes = gemv_bytes(sdt, sn, sk, st)
                sg = sbytes / (sms * 1e-3) / 1e9
                key = f"{name} {m.name.lower()}"
                per[key] = {"us": round(sms * 1e3, 2), "GB/s": round(sg, 1), "hbm_frac": round(sg / HBM_PEAK_GBS, 4)}
                log(f"  {key}: {sms * 1e3:.2f} us  {sg:.0f} GB/s ({sg / HBM_PEAK_GBS:.1%})")
    if "gemm" in rows:  # configs[2]: Q4_K prefill GEMM 512x4096x4096 on f16 MFMA, then the other formats
        for gdt in (G.Q4K, G.Q6K, G.Q8_0, G.Q5K, G.Q5_0, G.Q4_1, G.BF16, G.F32):
            gms, gs = time_gemm(hip, ctx, gdt, 4096, 4096, 512, max(20, args.steps // 4), 5, 300)
            gtf = 2.0 * 512 * 4096 * 4096 / (gms * 1e-3) / 1e12
            mname = "bf16_mfma" if gdt in (G.BF16, G.F32) else "f16_mfma"
            key = f"{G(gdt).name.replace('Q4K', 'Q4_K').replace('Q5K', 'Q5_K').replace('Q6K', 'Q6_K')} GEMM 512x4096x4096 {mname}"
            per[key] = {"us": round(gms * 1e3, 2), "TFLOP/s": round(gtf, 1), "mfma_frac": round(gtf / MFMA_F16_PEAK_TFS, 4)}
            kept[f"gemm {int(gdt)}"] = dict(gs, key=key)
            log(f"  {key}: {gms * 1e3:.2f} us  {gtf:.0f} TFLOP/s ({gtf / MFMA_F16_PEAK_TFS:.1%} of f16 MFMA peak)")
        # a short prompt: 64 tokens (one row tile; the 64-column tiles)
        gms, _ = time_gemm(hip, ctx, G.Q4K, 4096, 4096, 64, max(20, args.steps // 4), 5, 310)
        gtf = 2.0 * 64 * 4096 * 4096 / (gms * 1e-3) / 1e12
        key = "Q4_K GEMM 64x4096x4096 f16_mfma"
        per[key] = {"us": round(gms * 1e3, 2), "TFLOP/s": round(gtf, 1), "mfma_frac": round(gtf / MFMA_F16_PEAK_TFS, 4)}
        log(f"  {key}: {gms * 1e3:.2f} us  {gtf:.0f} TFLOP/s ({gtf / MFMA_F16_PEAK_TFS:.1%} of f16 MFMA peak)")
    if "moe" in rows:  # configs[3]: grouped MoE, 8 Q4_0 experts, 256 tokens, top-2
        mms, mbytes, msample = time_moe(hip, ctx, 5, 2, 400, Mode.F16_MFMA)
        mtf = 120259084288 / (mms * 1e-3) / 1e12
        mgb = mbytes / (mms * 1e-3) / 1e9
        key = "MoE 8x(14336x4096, 4096x14336) Q4_0 T256 top2 f16_mfma"
        per[key] = {"us": round(mms * 1e3, 2), "TFLOP/s": round(mtf, 1), "mfma_frac": round(mtf / MFMA_F16_PEAK_TFS, 4),
                    "GB/s": round(mgb, 1), "hbm_frac": round(mgb / HBM_PEAK_GBS, 4)}
        kept["moe"] = dict(msample, key=key)
        log(f"  MoE configs[3]: {mms * 1e3:.1f} us  {mtf:.0f} TFLOP/s ({mtf / MFMA_F16_PEAK_TFS:.1%}), "
            f"{mgb:.0f} GB/s ({mgb / HBM_PEAK_GBS:.1%})")
        # the same workload with the expert formats Q4_K_M / Q5_K_M / Q8_0 models ship
        for mdt, mname in ((G.Q6K, "Q6_K"), (G.Q5K, "Q5_K"), (G.Q8_0, "Q8_0")):
            mms, mbytes, msample = time_moe(hip, ctx, 5, 2, 410 + int(mdt), Mode.F16_MFMA, dtype=mdt)
            mtf = 120259084288 / (mms * 1e-3) / 1e12
            mgb = mbytes / (mms * 1e-3) / 1e9
            key = f"MoE 8x(14336x4096, 4096x14336) {mname} T256 top2 f16_mfma"
            per[key] = {"us": round(mms * 1e3, 2), "TFLOP/s": round(mtf, 1),
                        "mfma_frac": round(mtf / MFMA_F16_PEAK_TFS, 4), "GB/s": round(mgb, 1),
                        "hbm_frac": round(mgb / HBM_PEAK_GBS, 4)}
            kept[f"moe {mname}"] = dict(msample, key=key)
            log(f"  {key}: {mms * 1e3:.1f} us  {mtf:.0f} TFLOP/s ({mtf / MFMA_F16_PEAK_TFS:.1%}), "
                f"{mgb:.0f} GB/s ({mgb / HBM_PEAK_GBS:.1%})")
    if "llama" in rows:  # configs[4]: TinyLlama-shaped decode, batch 1
        log("  building the configs[4] decoder (22 layers, Q4_K + Q6_K head)")
        W = llama_weights(500)
        lsteps, lwarm = 128, 16
        # Q8, then the reference-order EXACT mode
        for lmode in (Mode.Q8, Mode.EXACT):
            lms, lsample = time_llama(hip, ctx, W, lmode, lsteps, lwarm, 501)
            lgb = LLAMA_WEIGHT_BYTES / (lms * 1e-3) / 1e9
            key = f"TinyLlama-shape decode 22L Q4_K/Q6_K b1 {lmode.name.lower()}"
            per[key] = {"us_per_token": round(lms * 1e3, 2), "tok/s": round(1e3 / lms, 1),
                        "weight_GB/s": round(lgb, 1), "hbm_frac": round(lgb / HBM_PEAK_GBS, 4),
                        "positions": f"{lwarm}..{lwarm + lsteps - 1}", "weight_bytes_per_token": LLAMA_WEIGHT_BYTES}
            kept[f"llama_{lmode.name.lower()}"] = dict(lsample, key=key, W=W, q8=(lmode == Mode.Q8))
            log(f"  {key}: {lms * 1e3:.1f} us/token  {1e3 / lms:.0f} tok/s  weights {lgb:.0f} GB/s "
                f"({lgb / HBM_PEAK_GBS:.1%} of HBM peak; floor {LLAMA_WEIGHT_BYTES / 8e12 * 1e6:.1f} us)")
    line["per_format"] = per
    if args.cache_warmth:
        line["cache_warmth"] = cache_warmth(hip, ctx)
    if args.read_ceilings:
        line["read_ceilings"] = read_ceilings(hip, ctx)
    if args.vendor_gemm:
        line["vendor_gemm"] = vendor_gemm()

    # ---- CPU baseline + parity checks (oracle) -------------------------------------
    if not args.no_cpu:
        log("cpu leg: oracle mm_1d on the headline workload (~10 s sample) and parity checks")
        cpu_leg(line, head, kept)
    ctx.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
