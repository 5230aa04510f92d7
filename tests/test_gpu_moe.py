"""GPU parity of the grouped-expert FFN (rce_qmm_moe_ffn_dev).

Reference semantics (rce-qwen36-moe/src/lib.rs L667-710, rce-op-moe
L35-110): for every token t and routing decision j, e = ids[t, j],
h = silu(W1[e] x_t), y_j = W2[e] h, out_t = sum_j w[t, j] * y_j in decision
order from +0.0.  The oracle restates that loop on the CPU (orc_moe_ffn).

Tolerances: the expert products of EXACT mode are the reference's own f32
order (bit-exact on their own; tests/test_gpu_gemv.py); the silu between
them calls the platform exp in the reference (host libm) and the library's
own exp on the GPU, which may differ in the last bit, so the MoE output is
compared normwise at 1e-5 with the reference, and bit for bit with the
oracle's restatement that takes the library's exp (moe_ffn(silu_dev=True)).
Q8 mode is compared bit for bit with the oracle's Q8 restatement
(moe_ffn(q8=True, silu_dev=True)); F16_MFMA mode with the reference order at
the fp16-dequant budget, 3e-3 normwise (two f16-rounded products in series).
Every mode must be run-to-run bit identical (fixed grouping and combine
order).
"""
import numpy as np
import pytest

import oracle as O
import rce_amd
from rce_amd import GgufDtype as G, Mode

pytestmark = pytest.mark.gpu
F32 = np.float32


def note(msg):
    print(msg, flush=True)


def make_case(seed, n_expert, d_model, d_ff, t_rows, top_k, dt):
    rng = np.random.default_rng(seed)
    w1 = [O.quantize((rng.standard_normal((d_ff, d_model)) * 0.02).astype(F32), dt) for _ in range(n_expert)]
    w2 = [O.quantize((rng.standard_normal((d_model, d_ff)) * 0.02).astype(F32), dt) for _ in range(n_expert)]
    x = rng.standard_normal((t_rows, d_model)).astype(F32)
    logits = rng.standard_normal((t_rows, n_expert)).astype(F32)
    ids, gw = rce_amd.moe_router(logits, top_k)
    return w1, w2, x, ids, gw


def run_moe(ctx, w1b, w2b, dt, d_model, d_ff, x, ids, gw, mode):
    t_rows, top_k = ids.shape
    W1 = [rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, d_ff, d_model) for b in w1b]
    W2 = [rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, d_model, d_ff) for b in w2b]
    bx = rce_amd.DeviceBuffer.from_numpy(ctx, x)
    bi = rce_amd.DeviceBuffer.from_numpy(ctx, ids.astype(np.int32))
    bw = rce_amd.DeviceBuffer.from_numpy(ctx, gw.astype(F32))
    bo = rce_amd.DeviceBuffer(ctx, t_rows * d_model * 4)
    outs = []
    for _ in range(2):
        rce_amd.moe_ffn_dev(ctx, W1, W2, bx.ptr, t_rows, bi.ptr, bw.ptr, top_k, bo.ptr, mode)
        ctx.synchronize()
        outs.append(bo.download(F32, t_rows * d_model).reshape(t_rows, d_model))
    for b in (bx, bi, bw, bo):
        b.free()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), "not run-to-run deterministic"
    return outs[0]


def q8_reference(x, w1b, w2b, dt, d_model, d_ff, ids, gw):
    """The Q8-activation path per (token, decision) in the device's order:
    the oracle's Q8 products (mm_batched_q8), silu with the library's exp,
    moe_combine."""
    return O.moe_ffn(x, w1b, w2b, dt, d_ff, ids, gw, q8=True, silu_dev=True)


def bit_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a, F32).view(np.uint32), np.ascontiguousarray(b, F32).view(np.uint32))


def normwise(got, want):
    return float(np.max(np.abs(got.astype(np.float64) - want)) / np.max(np.abs(want)))


CASES = [
    # (n_expert, d_model, d_ff, t_rows, top_k, dtype)
    (4, 512, 1024, 16, 2, O.Q4_0),
    (8, 256, 512, 3, 2, O.Q4_0),     # most experts get no token
    (4, 512, 768, 40, 1, O.Q4_0),    # top-1, ragged slots
    (4, 512, 1024, 24, 2, O.Q4_K),
    (40, 256, 512, 50, 3, O.Q4_0),   # more experts than the single-scan grouping takes
    (32, 256, 512, 300, 2, O.Q4_K),  # its largest expert count, several pairs per thread
]


@pytest.mark.parametrize("E,dm,dff,t,k,dt", CASES)
def test_moe_exact(ctx, E, dm, dff, t, k, dt):
    note(f"moe exact E={E} d={dm} ff={dff} t={t} k={k} dt={dt}")
    w1, w2, x, ids, gw = make_case(100 + E + t, E, dm, dff, t, k, dt)
    got = run_moe(ctx, w1, w2, dt, dm, dff, x, ids, gw, Mode.EXACT)
    ref = O.moe_ffn(x, w1, w2, dt, dff, ids, gw)
    assert normwise(got, ref) < 1e-5
    assert bit_equal(got, O.moe_ffn(x, w1, w2, dt, dff, ids, gw, silu_dev=True))


@pytest.mark.parametrize("E,dm,dff,t,k,dt", CASES)
def test_moe_q8(ctx, E, dm, dff, t, k, dt):
    note(f"moe q8 E={E} d={dm} ff={dff} t={t} k={k} dt={dt}")
    w1, w2, x, ids, gw = make_case(200 + E + t, E, dm, dff, t, k, dt)
    got = run_moe(ctx, w1, w2, dt, dm, dff, x, ids, gw, Mode.Q8)
    assert bit_equal(got, q8_reference(x, w1, w2, dt, dm, dff, ids, gw))


@pytest.mark.parametrize("E,dm,dff,t,k,dt", CASES)
def test_moe_f16_mfma(ctx, E, dm, dff, t, k, dt):
    note(f"moe f16-mfma E={E} d={dm} ff={dff} t={t} k={k} dt={dt}")
    w1, w2, x, ids, gw = make_case(300 + E + t, E, dm, dff, t, k, dt)
    got = run_moe(ctx, w1, w2, dt, dm, dff, x, ids, gw, Mode.F16_MFMA)
    ref = O.moe_ffn(x, w1, w2, dt, dff, ids, gw)
    assert normwise(got, ref) < 3e-3


def test_moe_mixtral_shapes(ctx):
    """configs[3] expert shapes (w1 14336x4096, w2 4096x14336, Q4_0) on two
    experts and a few tokens: the full-size tiles and long K of both GEMMs."""
    E, dm, dff, t, k, dt = 2, 4096, 14336, 6, 2, O.Q4_0
    note(f"moe mixtral-shaped E={E} t={t}")
    w1, w2, x, ids, gw = make_case(400, E, dm, dff, t, k, dt)
    ref = O.moe_ffn(x, w1, w2, dt, dff, ids, gw)
    got = run_moe(ctx, w1, w2, dt, dm, dff, x, ids, gw, Mode.F16_MFMA)
    assert normwise(got, ref) < 3e-3
    got = run_moe(ctx, w1, w2, dt, dm, dff, x, ids, gw, Mode.EXACT)
    assert normwise(got, ref) < 1e-5
    assert bit_equal(got, O.moe_ffn(x, w1, w2, dt, dff, ids, gw, silu_dev=True))
    # Q8: each expert's six tokens through the pre-quantized multi-token
    # GEMV (K 4096, then 14336), bit for bit with the oracle's Q8 path.
    note("  mode=Q8")
    got = run_moe(ctx, w1, w2, dt, dm, dff, x, ids, gw, Mode.Q8)
    assert bit_equal(got, q8_reference(x, w1, w2, dt, dm, dff, ids, gw))


def test_moe_bad_ids(ctx):
    """An out-of-range expert id is an error in the synchronous modes."""
    E, dm, dff, t, k, dt = 4, 256, 512, 4, 2, O.Q4_0
    w1, w2, x, ids, gw = make_case(500, E, dm, dff, t, k, dt)
    ids = ids.copy()
    ids[1, 0] = E  # out of range
    with pytest.raises(rce_amd.QmmError):
        run_moe(ctx, w1, w2, dt, dm, dff, x, ids, gw, Mode.EXACT)


# ---- SwiGLU experts (rce-qwen36-moe's form) ---------------------------------

def run_swiglu(ctx, gb, ub, db, dt, d_model, d_ff, x, ids, gw, mode):
    t_rows, top_k = ids.shape
    G = [rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, d_ff, d_model) for b in gb]
    U = [rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, d_ff, d_model) for b in ub]
    D = [rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, d_model, d_ff) for b in db]
    bx = rce_amd.DeviceBuffer.from_numpy(ctx, x)
    bi = rce_amd.DeviceBuffer.from_numpy(ctx, ids.astype(np.int32))
    bw = rce_amd.DeviceBuffer.from_numpy(ctx, gw.astype(F32))
    bo = rce_amd.DeviceBuffer(ctx, t_rows * d_model * 4)
    outs = []
    for _ in range(2):
        rce_amd.moe_swiglu_dev(ctx, G, U, D, bx.ptr, t_rows, bi.ptr, bw.ptr, top_k, bo.ptr, mode)
        ctx.synchronize()
        outs.append(bo.download(F32, t_rows * d_model).reshape(t_rows, d_model))
    for b in (bx, bi, bw, bo):
        b.free()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), "not run-to-run deterministic"
    return outs[0]


@pytest.mark.parametrize("mode,tol", [(Mode.EXACT, 1e-5), (Mode.F16_MFMA, 3e-3)])
@pytest.mark.parametrize("E,dm,dff,t,k,dt", [(4, 512, 1024, 16, 2, O.Q4_0), (6, 256, 512, 9, 3, O.Q4_K),
                                              (4, 512, 1024, 40, 2, O.Q8_0), (3, 256, 768, 30, 2, O.Q6_K)])
def test_moe_swiglu(ctx, mode, tol, E, dm, dff, t, k, dt):
    """rce_qmm_moe_swiglu_dev against the oracle's swiglu_expert_serial +
    combine (orc_moe_swiglu_ffn); tolerances as the two-matrix form."""
    note(f"moe swiglu mode={mode.name} E={E} d={dm} ff={dff} t={t} k={k} dt={dt}")
    rng = np.random.default_rng(600 + E + t)
    mk = lambda n, kk: O.quantize((rng.standard_normal((n, kk)) * 0.02).astype(F32), dt)  # noqa: E731
    gb = [mk(dff, dm) for _ in range(E)]
    ub = [mk(dff, dm) for _ in range(E)]
    db = [mk(dm, dff) for _ in range(E)]
    x = rng.standard_normal((t, dm)).astype(F32)
    ids, gw = rce_amd.moe_router(rng.standard_normal((t, E)).astype(F32), k)
    got = run_swiglu(ctx, gb, ub, db, dt, dm, dff, x, ids, gw, mode)
    ref = O.moe_swiglu_ffn(x, gb, ub, db, dt, dff, ids, gw)
    assert normwise(got, ref) < tol


def test_moe_f16_mfma_declines_formats_without_a_grouped_form(ctx):
    """Q3_K has no matrix-core form: Q3_K experts in F16_MFMA are refused on
    the host (no launch), while EXACT takes them."""
    from rand_blocks import rand_blocks
    E, dm, dff, T, K = 2, 256, 512, 4, 1
    rng = np.random.default_rng(77)
    w1 = [rand_blocks(rng, O.Q3_K, dff, dm, dmax=0.05 / 32) for _ in range(E)]
    w2 = [rand_blocks(rng, O.Q3_K, dm, dff, dmax=0.05 / 32) for _ in range(E)]
    x = rng.standard_normal((T, dm)).astype(np.float32)
    ids = np.zeros((T, K), np.int32)
    gw = np.ones((T, K), np.float32)
    with pytest.raises(rce_amd.QmmError, match="no GPU kernel"):
        run_moe(ctx, w1, w2, O.Q3_K, dm, dff, x, ids, gw, Mode.F16_MFMA)
    got = run_moe(ctx, w1, w2, O.Q3_K, dm, dff, x, ids, gw, Mode.EXACT)
    want = O.moe_ffn(x, w1, w2, O.Q3_K, dff, ids, gw)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))


# ---- grouped experts of the other formats on the matrix cores (gemm_gen.hip
# with tiles, gather and the silu epilogue) -----------------------------------

def expert_bytes(rng, dt, n, k, sigma=0.02):
    from rand_blocks import float_bytes, rand_blocks
    if dt in (O.F16, O.BF16, O.F32):
        return float_bytes(rng, dt, n, k, sigma)
    if dt in (O.Q5_0, O.Q4_1):  # no quantizer in the reference: random blocks
        return rand_blocks(rng, dt, n, k, dmax=sigma / 8)
    return O.quantize((rng.standard_normal((n, k)) * sigma).astype(F32), dt)


def run_moe2(ctx, w1b, w2b, dt1, dt2, d_model, d_ff, x, ids, gw, mode):
    """run_moe with a dtype per matrix."""
    t_rows, top_k = ids.shape
    W1 = [rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt1, d_ff, d_model) for b in w1b]
    W2 = [rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt2, d_model, d_ff) for b in w2b]
    bx = rce_amd.DeviceBuffer.from_numpy(ctx, x)
    bi = rce_amd.DeviceBuffer.from_numpy(ctx, ids.astype(np.int32))
    bw = rce_amd.DeviceBuffer.from_numpy(ctx, gw.astype(F32))
    bo = rce_amd.DeviceBuffer(ctx, t_rows * d_model * 4)
    outs = []
    for _ in range(2):
        rce_amd.moe_ffn_dev(ctx, W1, W2, bx.ptr, t_rows, bi.ptr, bw.ptr, top_k, bo.ptr, mode)
        ctx.synchronize()
        outs.append(bo.download(F32, t_rows * d_model).reshape(t_rows, d_model))
    for b in (bx, bi, bw, bo):
        b.free()
    for w in W1 + W2:
        w.close()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), "not run-to-run deterministic"
    return outs[0]


def f16_weights(b, dt, n, k):
    """The binary16 weights the F16_MFMA kernels form: the oracle's
    dequantized value rounded once (gemm_gen.hip), or for Q4_K the nibble
    kernel's f16(f16(d*sc)*q + f16(-dmin*m)) (gemm_f16.hip), for Q4_K and
    Q5_K, its f16(f16(d*sc)*q) for Q6_K, and f16(d*q + m) for Q4_1 at K % 256
    == 0."""
    if dt in (O.Q4_K, O.Q5_K):
        from test_gpu_gemm import q4k_f16_weights
        return q4k_f16_weights(b, n, k, q5=dt == O.Q5_K)
    if dt == O.Q6_K:
        from test_gpu_gemm import q6k_f16_weights
        return q6k_f16_weights(b, n, k)
    if dt == O.Q4_1 and k % 256 == 0:
        from test_gpu_gemm import q41_f16_weights
        return q41_f16_weights(b, n, k)
    from test_gpu_gemm import mfma_weights
    return mfma_weights(b, dt, n, k)


def f16_restatement(x, w1b, w2b, dt1, dt2, d_model, d_ff, ids, gw):
    """The grouped F16_MFMA path restated in numpy: x and every weight
    rounded to binary16 as the kernels form them, products summed in
    float64, h = binary16(silu(W1 x)), y = W2 h, combined in decision order."""
    x16 = x.astype(np.float16).astype(np.float64)
    out = np.zeros((x.shape[0], d_model))
    cache = {}
    for t in range(x.shape[0]):
        for j in range(ids.shape[1]):
            e = int(ids[t, j])
            if e not in cache:
                cache[e] = (f16_weights(w1b[e], dt1, d_ff, d_model), f16_weights(w2b[e], dt2, d_model, d_ff))
            a1, a2 = cache[e]
            h = a1 @ x16[t]
            h = (h / (1.0 + np.exp(-h))).astype(np.float16).astype(np.float64)
            out[t] += float(gw[t, j]) * (a2 @ h)
    return out


GEN_MOE_CASES = [
    # (n_expert, d_model, d_ff, t_rows, top_k, dtype of W1, dtype of W2)
    (4, 512, 1024, 40, 2, O.Q6_K, O.Q6_K),
    (4, 512, 1024, 40, 2, O.Q5_K, O.Q5_K),
    (4, 512, 1024, 40, 2, O.Q8_0, O.Q8_0),
    (6, 256, 512, 100, 2, O.Q4_K, O.Q6_K),   # Q4_K_M: Q4_K gate/up, Q6_K down (both kernels in one call)
    (3, 256, 768, 17, 1, O.Q5_0, O.Q4_1),
    (5, 256, 512, 300, 3, O.F16, O.Q8_0),    # experts past 128 rows: two tiles each
    # 128-row tiles holding 65-96 rows and at most 64 (the 96- and 64-row
    # bodies): Q8_0 / Q6_K experts at about 64 rows, Q4_K at about 100
    (8, 256, 512, 256, 2, O.Q8_0, O.Q6_K),
    (4, 256, 512, 200, 2, O.Q4_K, O.Q4_K),
    (4, 256, 512, 40, 2, O.BF16, O.F32),     # the bf16 forms
]


@pytest.mark.parametrize("E,dm,dff,t,k,dt1,dt2", GEN_MOE_CASES)
def test_moe_f16_mfma_other_formats(ctx, E, dm, dff, t, k, dt1, dt2):
    note(f"moe f16-mfma other formats E={E} d={dm} ff={dff} t={t} k={k} dt={dt1}/{dt2}")
    rng = np.random.default_rng(800 + E + t + dt1)
    w1 = [expert_bytes(rng, dt1, dff, dm) for _ in range(E)]
    w2 = [expert_bytes(rng, dt2, dm, dff) for _ in range(E)]
    x = rng.standard_normal((t, dm)).astype(F32)
    ids, gw = rce_amd.moe_router(rng.standard_normal((t, E)).astype(F32), k)
    got = run_moe2(ctx, w1, w2, dt1, dt2, dm, dff, x, ids, gw, Mode.F16_MFMA)
    assert normwise(got, f16_restatement(x, w1, w2, dt1, dt2, dm, dff, ids, gw)) < 1e-4, \
        "differs from the binary16 restatement of the same path"
    ref = O.moe_ffn(x, w1, w2, dt1, dff, ids, gw, dtype2=dt2)
    assert normwise(got, ref) < 3e-3
    if dt1 == dt2:  # EXACT takes the same experts, within 1e-5 of the reference
        assert normwise(run_moe2(ctx, w1, w2, dt1, dt2, dm, dff, x, ids, gw, Mode.EXACT), ref) < 1e-5


@pytest.mark.parametrize("dt", [O.Q6_K, O.Q5_K, O.Q8_0])
def test_moe_f16_mfma_other_formats_mixtral_shapes(ctx, dt):
    """Real expert shapes (w1 14336 x 4096, w2 4096 x 14336) in the formats
    Q4_K_M / Q5_K_M / Q8_0 models ship, 4 experts, 64 tokens top-2: every
    token against the reference order within the fp16-dequant budget."""
    E, dm, dff, t, k = 4, 4096, 14336, 64, 2
    note(f"moe f16-mfma mixtral-shaped dt={dt}")
    rng = np.random.default_rng(900 + dt)
    q = lambda n, kk: rce_amd.quantize(rng.standard_normal((n, kk), dtype=F32) * F32(0.02), dt)  # noqa: E731
    w1 = [q(dff, dm) for _ in range(E)]
    w2 = [q(dm, dff) for _ in range(E)]
    x = rng.standard_normal((t, dm)).astype(F32)
    ids, gw = rce_amd.moe_router(rng.standard_normal((t, E)).astype(F32), k)
    got = run_moe2(ctx, w1, w2, dt, dt, dm, dff, x, ids, gw, Mode.F16_MFMA)
    err = normwise(got, O.moe_ffn(x, w1, w2, dt, dff, ids, gw))
    note(f"  normwise {err:.3e}")
    assert err < 3e-3
