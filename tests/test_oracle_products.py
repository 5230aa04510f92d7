"""Pins the oracle's products (mm_1d / mm_batched, exact order; the Q8
activation path; MoE router/combine) with checks a plausible mistake would
fail: two independent restatements of the same order must agree bit for bit
(the reference's own 0-ulp judgement, spec/checker/tests/lift_gguf.rs
L288-291 and lift_llama.rs L283-288), the reference tests' kernel-vs-dequant
relations, an f64 error bound, and closed-form integer dots.  CPU only."""
import numpy as np
import pytest

import oracle as O

F32 = np.float32


# ---- independent numpy restatements (vectorized over rows, sequential order) ----

def _blocks(b, n, nb, bb):
    return b.reshape(n, nb, bb)


def np_values_q8_0_q4_0(b, dt, n, k):
    """(q int, d f32) of GGUF Q8_0/Q4_0 bytes, decoded with numpy."""
    nb = k // 32
    bl = _blocks(b, n, nb, 34 if dt == O.Q8_0 else 18)
    d = bl[:, :, :2].copy().view(np.float16)[:, :, 0].astype(F32)
    if dt == O.Q8_0:
        q = bl[:, :, 2:].view(np.int8).astype(np.int64)
    else:
        qs = bl[:, :, 2:].astype(np.int64)
        q = np.concatenate([(qs & 0xF) - 8, (qs >> 4) - 8], axis=2)
    return q.reshape(n, k), d


def np_mm_q8_0_q4_0(a, b, dt, n, k):
    """mm_1d_q8_0 / mm_1d_q4_0 order: sub over the block's positions (Q4_0:
    0,16,1,17,...), sumf += d * sub, in float32."""
    q, d = np_values_q8_0_q4_0(b, dt, n, k)
    order = list(range(32)) if dt == O.Q8_0 else [t for p in range(16) for t in (p, p + 16)]
    sumf = np.zeros(n, F32)
    for ib in range(k // 32):
        sub = np.zeros(n, F32)
        for t in order:
            sub = sub + q[:, 32 * ib + t].astype(F32) * a[32 * ib + t]
        sumf = sumf + d[:, ib] * sub
    return sumf


def np_mm_k(a, b, fmt, n, k):
    """dot_row_q4_k / dot_row_q5_k / dot_row_q6_k order from unpacked super-blocks."""
    nsb = k // 256
    bb = O.BLOCK[fmt][1]
    Q = np.zeros((n, k), np.int64)
    S = np.zeros((n, k // (16 if fmt == O.Q6_K else 32)), F32)
    M = np.zeros((n, k // 32), F32)
    for j in range(n):
        for s in range(nsb):
            q, sc, mn, d, dmin = O.unpack_k(b[(j * nsb + s) * bb:(j * nsb + s + 1) * bb], fmt)
            Q[j, 256 * s:256 * s + 256] = q
            ns = 16 if fmt == O.Q6_K else 8
            S[j, ns * s:ns * s + ns] = F32(d) * sc.astype(F32)
            if fmt != O.Q6_K:
                M[j, 8 * s:8 * s + 8] = F32(dmin) * mn.astype(F32)
    y = np.zeros(n, F32)
    if fmt == O.Q6_K:
        for s in range(nsb):
            for half in range(2):
                base = 256 * s + 128 * half
                for l in range(32):
                    for c in range(4):
                        p = base + l + 32 * c
                        y = y + (S[:, p // 16] * Q[:, p].astype(F32)) * a[p]
        return y
    for g in range(k // 64):
        b1, b2 = 2 * g, 2 * g + 1
        u1 = np.zeros(n, F32); a1 = F32(0); u2 = np.zeros(n, F32); a2 = F32(0)
        for t in range(32):
            p1, p2 = 32 * b1 + t, 32 * b2 + t
            u1 = u1 + Q[:, p1].astype(F32) * a[p1]
            a1 = F32(a1 + a[p1])
            u2 = u2 + Q[:, p2].astype(F32) * a[p2]
            a2 = F32(a2 + a[p2])
        y = y + (((S[:, b1] * u1 - M[:, b1] * a1) + S[:, b2] * u2) - M[:, b2] * a2)
    return y


def rand_weight(rng, dt, n, k, sigma=0.02):
    w = (rng.standard_normal((n, k)) * sigma).astype(F32)
    return w, O.quantize(w, dt)


FORMATS = [O.Q8_0, O.Q4_0, O.Q4_K, O.Q5_K, O.Q6_K]


@pytest.mark.parametrize("dt", FORMATS)
def test_mm_1d_equals_numpy_restatement(dt):
    rng = np.random.default_rng(10 + dt)
    n, k = 24, 512
    _, b = rand_weight(rng, dt, n, k)
    a = rng.standard_normal(k).astype(F32)
    got = O.mm_1d(a, b, dt, n, k)
    want = np_mm_q8_0_q4_0(a, b, dt, n, k) if dt in (O.Q8_0, O.Q4_0) else np_mm_k(a, b, dt, n, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dt", FORMATS)
def test_mm_1d_equals_value_form(dt):
    # The value-form products (nn.rs matmul_q, kquant.rs matmul_k) on the
    # unpacked values equal the kernel form bit for bit.
    rng = np.random.default_rng(20 + dt)
    n, k, m = 9, 768, 2
    _, b = rand_weight(rng, dt, n, k)
    x = rng.standard_normal((m, k)).astype(F32)
    got = O.mm_batched(x, b, dt, n, k)
    if dt in (O.Q8_0, O.Q4_0):
        q, d = np_values_q8_0_q4_0(b, dt, n, k)
        want = O.matmul_q(x, q.astype(np.int32), d, dt == O.Q4_0)
    else:
        nsb, bb = k // 256, O.BLOCK[dt][1]
        qs, ss, os_ = [], [], []
        for j in range(n):
            qr, sr, orow = [], [], []
            for s in range(nsb):
                q, sc, mn, d, dmin = O.unpack_k(b[(j * nsb + s) * bb:(j * nsb + s + 1) * bb], dt)
                qr.append(q); sr.append(F32(d) * sc.astype(F32))
                if dt != O.Q6_K:
                    orow.append(F32(dmin) * mn.astype(F32))
            qs.append(np.concatenate(qr)); ss.append(np.concatenate(sr))
            os_.append(np.concatenate(orow) if orow else np.zeros(1, F32))
        want = O.matmul_k(x, np.stack(qs), np.stack(ss), None if dt == O.Q6_K else np.stack(os_), dt)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _ref_bytes(n, nb, bb, mul, add, scale_at, scales):
    """The reference tests' synthetic bytes (rce-op-qmm lib.rs L2429-2500):
    byte i = (i*mul + add) & 0xFF with f16 scales forced per block."""
    b = ((np.arange(n * nb * bb) * mul + add) & 0xFF).astype(np.uint8).reshape(n * nb, bb)
    for off, val in zip(scale_at, scales):
        b[:, off:off + 2] = np.frombuffer(np.float16(val).tobytes(), np.uint8)
    return b.reshape(-1)


REF_CASES = [
    # (dtype, k, n, mul, add, scale offsets, scales, activation)
    (O.Q4_K, 512, 5, 17, 3, (0, 2), (0.0625, 0.03125), lambda i: np.cos(F32(i) * F32(0.021) + F32(0.5))),
    (O.Q4_0, 128, 6, 11, 1, (0,), (0.125,), lambda i: np.sin(F32(i) * F32(0.05) - F32(1.0))),
    (O.Q5_K, 512, 7, 31, 7, (0, 2), (0.0625, 0.03125), lambda i: np.sin(F32(i) * F32(0.013) - F32(0.7))),
    (O.Q3_K, 512, 6, 23, 11, (108,), (0.0625,), lambda i: np.sin(F32(i) * F32(0.017) - F32(0.3))),
]


@pytest.mark.parametrize("case", REF_CASES, ids=lambda c: str(c[0]))
def test_kernel_matches_dequant_then_dot(case):
    # q4_k_/q4_0_/q5_k_/q3_k_matmul_matches_dequant_then_dot (lib.rs L2358-2500):
    # rel err < 1e-5 against dequantize_to_f32 then a scalar dot.
    dt, k, n, mul, add, offs, scales, act = case
    qk, bb = O.BLOCK[dt]
    b = _ref_bytes(n, k // qk, bb, mul, add, offs, scales)
    a = np.array([act(i) for i in range(k)], F32)
    got = O.mm_1d(a, b, dt, n, k)
    rb = O.row_bytes(dt, k)
    for j in range(n):
        w = O.dequantize(b[j * rb:(j + 1) * rb], dt, k)
        acc = F32(0)
        for i in range(k):
            acc = F32(acc + a[i] * w[i])
        assert abs(got[j] - acc) / max(abs(acc), 1e-6) < 1e-5


@pytest.mark.parametrize("dt", FORMATS)
def test_mm_1d_error_bound_against_f64(dt):
    # |fl(sum) - sum| <= (K + 3) u sum|terms| for any order of K f32
    # roundings: a wrong term (index, sign, scale) breaks it by orders.
    rng = np.random.default_rng(30 + dt)
    n, k = 32, 1024
    _, b = rand_weight(rng, dt, n, k)
    a = rng.standard_normal(k).astype(F32)
    got = O.mm_1d(a, b, dt, n, k).astype(np.float64)
    w = O.dequantize(b, dt, n * k).reshape(n, k).astype(np.float64)
    exact = w @ a.astype(np.float64)
    bound = (k + 3) * 2.0 ** -24 * (np.abs(w) @ np.abs(a.astype(np.float64)))
    assert np.all(np.abs(got - exact) <= bound)


@pytest.mark.parametrize("dt", FORMATS)
def test_batched_is_per_row_and_thread_independent(dt):
    # mm_batched == t_rows x mm_1d (lib.rs L2575); serial == parallel (L3630).
    rng = np.random.default_rng(40 + dt)
    n, k, t = 40, 512, 3
    _, b = rand_weight(rng, dt, n, k)
    x = rng.standard_normal((t, k)).astype(F32)
    batched = O.mm_batched(x, b, dt, n, k, threads=4)
    for r in range(t):
        one = O.mm_1d(x[r], b, dt, n, k, threads=1)
        assert np.array_equal(batched[r].view(np.uint32), one.view(np.uint32))


# ---- Q8-activation path -------------------------------------------------------

def np_quantize_act(x):
    """quantize_block(x, false) per block of 32, restated in numpy."""
    xb = x.reshape(-1, 32)
    amax = np.max(np.abs(xb), axis=1).astype(F32)
    d = (amax / F32(127.0)).astype(F32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, F32(1.0) / d, F32(0.0)).astype(F32)
    v = (xb * idv[:, None]).astype(F32).astype(np.float64)
    q = (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int64)   # half away from zero
    dx = d.astype(np.float16).astype(F32)
    return q.reshape(-1), dx


def test_quantize_act_matches_numpy():
    rng = np.random.default_rng(50)
    x = rng.standard_normal(4096).astype(F32)
    x[:32] = 0.0  # an all-zero block: d = 0, id = 0, q = 0
    xq, dx, xs = O.quantize_act_q8(x)
    q, d = np_quantize_act(x)
    assert np.array_equal(xq.astype(np.int64), q)
    assert np.array_equal(dx, d)
    assert np.array_equal(xs, q.reshape(-1, 32).sum(axis=1))


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4_0])
def test_q8_block_isums_closed_form(dt):
    # Integer block dots are exact: compare with an int64 matrix product.
    rng = np.random.default_rng(60 + dt)
    n, k = 16, 1024
    _, b = rand_weight(rng, dt, n, k)
    x = rng.standard_normal(k).astype(F32)
    xq, _, _ = O.quantize_act_q8(x)
    isum = O.block_isums(xq, b, dt, n, k)
    q, _ = np_values_q8_0_q4_0(b, dt, n, k)
    want = (q.reshape(n, k // 32, 32) * xq.astype(np.int64).reshape(1, k // 32, 32)).sum(axis=2)
    assert np.array_equal(isum.astype(np.int64), want)
    assert np.abs(want).max() < 2 ** 24   # exact as f32 (32*127*127 < 2^24)


@pytest.mark.parametrize("dt", FORMATS)
def test_q8_path_equals_numpy_restatement(dt):
    rng = np.random.default_rng(70 + dt)
    n, k = 20, 512
    _, b = rand_weight(rng, dt, n, k)
    a = rng.standard_normal(k).astype(F32)
    got = O.mm_batched_q8(a, b, dt, n, k)[0]
    xq, dx = np_quantize_act(a)
    if dt in (O.Q8_0, O.Q4_0):
        q, d = np_values_q8_0_q4_0(b, dt, n, k)
        sumf = np.zeros(n, F32)
        for ib in range(k // 32):
            isum = (q[:, 32 * ib:32 * ib + 32] * xq[32 * ib:32 * ib + 32]).sum(axis=1)
            sub = (dx[ib] * isum.astype(F32)).astype(F32)
            sumf = sumf + d[:, ib] * sub
        want = sumf
    else:
        nsb, bb = k // 256, O.BLOCK[dt][1]
        want = np.zeros(n, F32)
        for j in range(n):
            sumf = F32(0)
            for s in range(nsb):
                q, sc, mn, d, dmin = O.unpack_k(b[(j * nsb + s) * bb:(j * nsb + s + 1) * bb], dt)
                xs = xq[256 * s:256 * s + 256]
                if dt in (O.Q4_K, O.Q5_K):
                    for g in range(4):
                        bl, bh = 8 * s + 2 * g, 8 * s + 2 * g + 1
                        il = int((q[64 * g:64 * g + 32] * xs[64 * g:64 * g + 32]).sum())
                        ih = int((q[64 * g + 32:64 * g + 64] * xs[64 * g + 32:64 * g + 64]).sum())
                        sl = int(xs[64 * g:64 * g + 32].sum()); sh = int(xs[64 * g + 32:64 * g + 64].sum())
                        d1, m1 = F32(d) * F32(sc[2 * g]), F32(dmin) * F32(mn[2 * g])
                        d2, m2 = F32(d) * F32(sc[2 * g + 1]), F32(dmin) * F32(mn[2 * g + 1])
                        t = F32(d1 * F32(dx[bl] * F32(il)))
                        t = F32(t - F32(m1 * F32(dx[bl] * F32(sl))))
                        t = F32(t + F32(d2 * F32(dx[bh] * F32(ih))))
                        t = F32(t - F32(m2 * F32(dx[bh] * F32(sh))))
                        sumf = F32(sumf + t)
                else:
                    ssb = F32(0)
                    for bsub in range(16):
                        isum = int((q[16 * bsub:16 * bsub + 16] * xs[16 * bsub:16 * bsub + 16]).sum())
                        ds = F32(F32(d) * F32(sc[bsub]))
                        ab = F32(dx[(256 * s + 16 * bsub) // 32] * F32(isum))
                        ssb = F32(ssb + F32(ds * ab))
                    sumf = F32(sumf + ssb)
            want[j] = sumf
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q8_path_close_to_exact_path():
    # The Q8 path differs from the reference only by the activation rounding.
    rng = np.random.default_rng(80)
    n, k = 256, 4096
    _, b = rand_weight(rng, O.Q4_0, n, k)
    a = rng.standard_normal(k).astype(F32)
    ex = O.mm_1d(a, b, O.Q4_0, n, k)
    q8 = O.mm_batched_q8(a, b, O.Q4_0, n, k)[0]
    rel = np.max(np.abs(q8 - ex)) / np.max(np.abs(ex))
    assert 0 < rel < 2e-2


# ---- MoE ----------------------------------------------------------------------

def test_moe_router_top_k_sorted_normalized():
    # rce-op-moe tests L145-165 shape: top-2 of 8, weights sum to 1, sorted,
    # distinct indices; plus the softmax values themselves.
    rng = np.random.default_rng(90)
    for _ in range(50):
        lg = rng.standard_normal(8).astype(F32)
        idx, w = O.moe_router(lg, 2, True)
        assert idx[0] != idx[1] and w[0] >= w[1]
        assert abs(float(w.sum()) - 1.0) < 1e-6
        order = np.argsort(-lg, kind="stable")[:2]
        assert list(idx) == list(order)
    idx, w = O.moe_router(np.array([0.0, 0.0, 1.0, -1.0], F32), 1, True)
    assert idx[0] == 2 and w[0] == 1.0
    # unnormalized: the raw softmax probabilities (sum < 1 when K < N)
    idx, w = O.moe_router(np.zeros(32, F32), 2, False)
    assert list(idx) == [0, 1] and np.allclose(w, 1 / 32)


def test_moe_combine_known_answer():
    # rce-op-moe combine_weights_correctly (L172-188): 0.5*1 + 0.3*2 + 0.2*3.
    ys = np.stack([np.full(32, 1.0, F32), np.full(32, 2.0, F32), np.full(32, 3.0, F32)])
    out = O.moe_combine(np.array([0.5, 0.3, 0.2], F32), ys)
    assert np.all(np.abs(out - 1.7) < 1e-5)
    want = F32(F32(F32(0) + F32(F32(0.5) * F32(1))) + F32(F32(0.3) * F32(2)))
    want = F32(want + F32(F32(0.2) * F32(3)))
    assert np.all(out == want)


def test_silu_branches():
    # tinyllama L164-166: x/(1+exp(-x)) for x >= 0, x e/(1+e) below.
    for x in (0.0, 1.5, -2.25, 10.0, -30.0):
        e = np.exp(np.float64(-x)) if x >= 0 else np.exp(np.float64(x))
        want = x / (1 + e) if x >= 0 else x * e / (1 + e)
        assert abs(O.silu(x) - want) <= 1e-6 * max(1.0, abs(want))


def test_moe_swiglu_ffn_independent():
    """orc_moe_swiglu_ffn (rce-qwen36-moe L667-703) against an f64 numpy
    restatement over the dequantized experts: silu on the gate product,
    times the up product, down, combined in decision order.  Swapping gate
    and up, or dropping the up factor, is far outside the bound."""
    rng = np.random.default_rng(77)
    E, dm, dff, T, K = 3, 64, 96, 5, 2
    dt = O.Q8_0
    mk = lambda n, k: O.quantize((rng.standard_normal((n, k)) * 0.05).astype(np.float32), dt)  # noqa: E731
    gate = [mk(dff, dm) for _ in range(E)]
    up = [mk(dff, dm) for _ in range(E)]
    down = [mk(dm, dff) for _ in range(E)]
    x = rng.standard_normal((T, dm)).astype(np.float32)
    ids = np.array([[0, 2], [1, 0], [2, 1], [2, 0], [1, 2]], np.int32)
    gw = rng.random((T, K)).astype(np.float32)
    got = O.moe_swiglu_ffn(x, gate, up, down, dt, dff, ids, gw)
    deq = lambda b, n, k: O.dequantize(b, dt, n * k).reshape(n, k).astype(np.float64)  # noqa: E731
    want = np.zeros((T, dm))
    for t in range(T):
        for j in range(K):
            e = ids[t, j]
            g = deq(gate[e], dff, dm) @ x[t]
            u = deq(up[e], dff, dm) @ x[t]
            h = g / (1 + np.exp(-g)) * u
            want[t] += gw[t, j] * (deq(down[e], dm, dff) @ h)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
