"""Pins of the oracle's Llama-2 decode step (oracle/qmm_oracle.c: orc_rms_norm,
orc_rope, orc_attend_head, orc_llama_forward), each against something that
does not restate the same code:

  * rms_norm (rce-tinyllama L158-163): a closed form (x = 2 everywhere,
    eps = 0 -> out == w exactly) and an f64 evaluation;
  * RoPE (rce-op-attn L115-151): pos 0 is the identity bit for bit; the
    rotation angle of pair i is pos * base^(-2i/rope_dim) (f64), pairs are
    (i, i + half) (a wrong pairing or sign fails), and every pair keeps its
    norm;
  * attention (rce-op-attn L185-251): one key returns v exactly; equal keys
    give the mean of the values; otherwise the three-pass softmax in f64
    (the reference's own test compares these two at 1e-4,
    rce-op-attn tests `fused_attend_matches_three_pass`);
  * the whole step (rce-tinyllama L252-330): an independent numpy f64
    decoder over the dequantized weights (norm placement, GQA head mapping
    h // (n_q / n_kv), residuals, silu(g) * u, lm_head) within 1e-4
    normwise over several positions, and the token path equal to the
    embedding path.
The libm functions themselves (expf, sinf, cosf, logf) are the host C
library's, as the reference's f32 methods on Linux; their last bits are not
pinned here ("parity unpinned" for those bits only).
"""
import math

import numpy as np
import pytest

import oracle as O
from llama_case import LIN, make_weights, normwise, oracle_model, shapes, tiny_cfg

F32 = np.float32


def test_rms_norm_closed_form():
    w = np.random.default_rng(0).standard_normal(256).astype(F32)
    x = np.full(256, 2.0, F32)
    out = O.rms_norm(x, w, 0.0)  # mean_sq = 4, inv = 0.5, (2 * 0.5) * w = w
    assert np.array_equal(out, w)


def test_rms_norm_f64():
    rng = np.random.default_rng(1)
    for n in (7, 256, 2048, 5632):
        x = rng.standard_normal(n).astype(F32) * F32(3.0)
        w = rng.standard_normal(n).astype(F32)
        want = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5) * w
        assert np.max(np.abs(O.rms_norm(x, w, 1e-5) - want)) <= 1e-5 * np.max(np.abs(want))


def test_rope_identity_at_pos0():
    x = np.random.default_rng(2).standard_normal(64).astype(F32)
    y, cs = O.rope(x, 64, 10000.0, 0)
    assert np.array_equal(y, x)
    assert np.all(cs[:, 0] == 1.0) and np.all(cs[:, 1] == 0.0)


@pytest.mark.parametrize("rope_dim,d,base,pos", [(64, 64, 10000.0, 1), (64, 64, 10000.0, 37),
                                                 (128, 128, 500000.0, 1000), (32, 64, 10000.0, 5)])
def test_rope_angles_and_pairs(rope_dim, d, base, pos):
    x = np.random.default_rng(3 + pos).standard_normal(d).astype(F32)
    y, cs = O.rope(x, rope_dim, base, pos)
    half = rope_dim // 2
    i = np.arange(half)
    theta = pos * base ** (-2.0 * i / rope_dim)
    # the reference forms theta in f32 (inv_freq and pos * inv_freq each
    # rounded): its angle is within a few ulp(theta) of the exact one
    tol = 4.0 * theta * 2.0 ** -24 + 1e-6
    assert np.all(np.abs(cs[:, 0] - np.cos(theta)) <= tol)
    assert np.all(np.abs(cs[:, 1] - np.sin(theta)) <= tol)
    a, b = x[:half].astype(np.float64), x[half:rope_dim].astype(np.float64)
    c, s = cs[:, 0].astype(np.float64), cs[:, 1].astype(np.float64)
    assert np.allclose(y[:half], a * c - b * s, atol=1e-6)
    assert np.allclose(y[half:rope_dim], a * s + b * c, atol=1e-6)
    assert np.array_equal(y[rope_dim:], x[rope_dim:])  # dims past rope_dim untouched
    assert np.allclose(np.hypot(y[:half], y[half:rope_dim]), np.hypot(a, b), rtol=1e-6)


def test_attend_single_key_is_v():
    rng = np.random.default_rng(4)
    q, k, v = (rng.standard_normal(64).astype(F32) for _ in range(3))
    out = O.attend_head(q, k, v, 0, 1, 64, 64, 0.125)
    assert np.array_equal(out, v)


def test_attend_equal_keys_mean():
    rng = np.random.default_rng(5)
    seq, kvd, dh = 9, 128, 64
    q = rng.standard_normal(dh).astype(F32)
    k1 = rng.standard_normal(dh).astype(F32)
    K = np.zeros((seq, kvd), F32)
    V = rng.standard_normal((seq, kvd)).astype(F32)
    K[:, dh:] = k1  # kv head 1: every key equal
    out = O.attend_head(q, K, V, 1, seq, kvd, dh, 0.125)
    assert np.allclose(out, V[:, dh:].astype(np.float64).mean(0), atol=1e-6)


@pytest.mark.parametrize("seq", [2, 17, 300])
def test_attend_three_pass(seq):
    rng = np.random.default_rng(6 + seq)
    nkv, dh = 4, 64
    kvd = nkv * dh
    q = rng.standard_normal(dh).astype(F32) * F32(2.0)
    K = rng.standard_normal((seq, kvd)).astype(F32)
    V = rng.standard_normal((seq, kvd)).astype(F32)
    for g in range(nkv):
        s = K[:, g * dh:(g + 1) * dh].astype(np.float64) @ q.astype(np.float64) / 8.0
        p = np.exp(s - s.max())
        want = (p / p.sum()) @ V[:, g * dh:(g + 1) * dh].astype(np.float64)
        got = O.attend_head(q, K, V, g, seq, kvd, dh, F32(1.0 / math.sqrt(dh)))
        assert np.max(np.abs(got - want)) <= 1e-5 * max(1.0, np.max(np.abs(want)))


def numpy_decoder(W: dict):
    """Independent f64 decode step over dequantized weights (generator of
    per-position logits from embeddings)."""
    c = W["cfg"]
    dm, nq, nkv, dh, ff = c["d_model"], c["n_q_heads"], c["n_kv_heads"], c["d_head"], c["d_ff"]
    rd, base, eps = c["rope_dim"], c["rope_freq_base"], c["eps"]
    sh = shapes(c)
    deq = lambda bd, n, k: O.dequantize(bd[0], bd[1], n * k).reshape(n, k).astype(np.float64)  # noqa: E731
    layers = [{n: deq(b[n], *sh[n]) for n in LIN} for b in W["blocks"]]
    head = deq(W["lm_head"], c["vocab"], dm)
    Kc = [[] for _ in layers]
    Vc = [[] for _ in layers]

    def norm(x, w):
        return x / np.sqrt(np.mean(x * x) + eps) * w

    def rope(v, pos):
        v = v.reshape(-1, dh).copy()
        half = rd // 2
        th = pos * base ** (-2.0 * np.arange(half) / rd)
        a, b = v[:, :half].copy(), v[:, half:rd].copy()
        v[:, :half] = a * np.cos(th) - b * np.sin(th)
        v[:, half:rd] = a * np.sin(th) + b * np.cos(th)
        return v

    def step(x, pos):
        x = x.astype(np.float64)
        for il, (L, b) in enumerate(zip(layers, W["blocks"])):
            xn = norm(x, b["attn_norm"])
            q, k, v = rope(L["wq"] @ xn, pos), rope(L["wk"] @ xn, pos), (L["wv"] @ xn).reshape(nkv, dh)
            Kc[il].append(k)
            Vc[il].append(v)
            K, V = np.stack(Kc[il]), np.stack(Vc[il])
            att = np.zeros((nq, dh))
            for h in range(nq):
                g = h // (nq // nkv)
                s = K[:, g] @ q[h] / math.sqrt(dh)
                p = np.exp(s - s.max())
                att[h] = (p / p.sum()) @ V[:, g]
            x = x + L["wo"] @ att.reshape(-1)
            xn = norm(x, b["ffn_norm"])
            gg, uu = L["ffn_gate"] @ xn, L["ffn_up"] @ xn
            x = x + L["ffn_down"] @ (gg / (1 + np.exp(-gg)) * uu)
        return head @ norm(x, W["output_norm"])
    return step


def test_llama_forward_matches_independent_decoder():
    W = make_weights(tiny_cfg(), seed=11)
    om = oracle_model(W)
    ref = numpy_decoder(W)
    for pos, tok in enumerate([3, 100, 7, 319, 3, 42]):
        e = om.embed(tok)
        got = om.forward_embedding(e)
        assert normwise(got, ref(e, pos)) < 1e-4, f"position {pos}"
    assert om.pos == 6


def test_llama_token_path_and_reset():
    W = make_weights(tiny_cfg(n_layers=1), seed=12)
    a = oracle_model(W)
    b = oracle_model(W)
    for tok in (5, 6, 7):
        la = a.forward_token(tok)
        lb = b.forward_embedding(b.embed(tok))
        assert np.array_equal(la, lb)
    a.reset()
    assert a.pos == 0
    assert np.array_equal(a.forward_token(5), oracle_model(W).forward_token(5))


def test_llama_q8_mode_close_to_exact():
    W = make_weights(tiny_cfg(), seed=13)
    e, q = oracle_model(W), oracle_model(W, q8=True)
    for tok in (1, 2, 3):
        le, lq = e.forward_token(tok), q.forward_token(tok)
        assert 0 < normwise(lq, le) < 5e-2  # Q8 activations: a different, nearby result


def test_llama_cache_full():
    W = make_weights(tiny_cfg(n_layers=1, context_length=2), seed=14)
    m = oracle_model(W)
    m.forward_token(1)
    m.forward_token(2)
    with pytest.raises(ValueError):
        m.forward_token(3)


# ---- the device's own orders (orc_exp_dev, orc_silu_dev, orc_rms_norm_dev,
# orc_attend_head_dev): what the GPU decode step is compared with bit for bit

def _bits(x: float) -> int:
    return int(np.array([x], F32).view(np.uint32)[0])


def test_exp_dev_within_one_ulp_everywhere():
    """Every float in [-104, 88.75]: within 1 ulp of the correctly rounded
    exp (double exp rounded to float), subnormal results included.  A wrong
    coefficient, a dropped Taylor term or a wrong ln 2 split fails this."""
    pos_ulp, _ = O.exp_dev_max_ulp(0, _bits(88.75))
    neg_ulp, _ = O.exp_dev_max_ulp(_bits(-0.0), _bits(-104.0))
    assert pos_ulp <= 1.0 and neg_ulp <= 1.0


def test_exp_dev_special_values():
    assert O.exp_dev(0.0) == 1.0 and O.exp_dev(-0.0) == 1.0
    assert O.exp_dev(float("-inf")) == 0.0 and O.exp_dev(-104.5) == 0.0
    assert O.exp_dev(89.0) == float("inf") and O.exp_dev(float("inf")) == float("inf")
    assert math.isnan(O.exp_dev(float("nan")))
    assert O.exp_dev(1.0) == float(np.float32(math.e))


def test_silu_dev_close_to_silu():
    for x in np.linspace(-90, 90, 2001).astype(F32):
        a, b = O.silu_dev(float(x)), O.silu(float(x))
        assert abs(a - b) <= 4 * np.spacing(F32(abs(b))) + 1e-44, (x, a, b)


@pytest.mark.parametrize("n,nt", [(2048, 256), (4096, 256), (256, 256), (2048, -256), (5632, -256), (300, -256),
                                  (8192, 512)])
def test_rms_norm_dev_is_the_same_sum(n, nt):
    """Squares that are small integers sum exactly in any order, so the
    device's trees must give the reference's bits: a dropped, doubled or
    misplaced term (a task past its end, a wave skipped) fails.  Random
    values: within rounding of the sequential sum."""
    rng = np.random.default_rng(n + nt)
    if nt > 0 and n // 8 > 2 * nt:
        pytest.skip("the fused form covers at most 2 nt tasks")
    w = rng.standard_normal(n).astype(F32)
    x = rng.integers(-7, 8, n).astype(F32)
    assert np.array_equal(O.rms_norm_dev(x, w, 1e-5, nt).view(np.uint32), O.rms_norm(x, w, 1e-5).view(np.uint32))
    x = rng.standard_normal(n).astype(F32)
    a, b = O.rms_norm_dev(x, w, 1e-5, nt), O.rms_norm(x, w, 1e-5)
    assert np.max(np.abs(a - b)) <= 2e-6 * np.max(np.abs(b))


@pytest.mark.parametrize("seq", [1, 2, 3, 4, 5, 63, 64, 65, 200, 257, 300])
@pytest.mark.parametrize("d_head", [64, 128])
def test_attend_head_dev_is_the_same_softmax(seq, d_head):
    """Equal scores make every p_j = 1 exactly; with small integer values
    every partial sum is exact, so the parallel order must give the mean of
    the values exactly as the reference's recurrence does (a key dropped or
    counted twice, a wrong run bound or a lost wave fails).  Random inputs:
    within 1e-6 of the reference's order.  Seq lengths cover waves without
    keys (fewer than four runs), one partial run, several runs per wave
    (more than four runs: 257 and 300 keys), and the 32-key runs of
    d_head 128."""
    rng = np.random.default_rng(seq * 7 + d_head)
    kvd = 2 * d_head
    q = np.zeros(d_head, F32)
    k = rng.standard_normal((seq, kvd)).astype(F32)
    v = rng.integers(-8, 9, (seq, kvd)).astype(F32)
    ref = O.attend_head(q, k, v, 1, seq, kvd, d_head, 0.125)
    got = O.attend_head_dev(q, k, v, 1, seq, kvd, d_head, 0.125)
    if seq & (seq - 1) == 0:  # 1 / seq exact
        assert np.array_equal(got, v[:, d_head:].mean(axis=0).astype(F32))
    assert np.max(np.abs(got - ref)) <= 1e-6 * max(1.0, np.max(np.abs(ref)))
    q = rng.standard_normal(d_head).astype(F32)
    v = rng.standard_normal((seq, kvd)).astype(F32)
    ref = O.attend_head(q, k, v, 1, seq, kvd, d_head, 0.125)
    got = O.attend_head_dev(q, k, v, 1, seq, kvd, d_head, 0.125)
    assert np.max(np.abs(got - ref)) <= 1e-6 * np.max(np.abs(ref))


def test_llama_device_order_close_to_reference_order():
    """The whole step in the device's orders stays within rounding of the
    reference's orders (EXACT linears), and the trace is the residual stream
    the step really adds to."""
    W = make_weights(tiny_cfg(), seed=61)
    a = oracle_model(W)
    b = O.Llama(W["cfg"], W["token_embd"], W["output_norm"], W["lm_head"], W["blocks"], device_order=(256, -256))
    for t in (3, 100, 7, 319, 3):
        la, xa = a.forward_token(t, trace=True)
        lb = b.forward_token(t)
        assert normwise(lb, la) < 1e-5
    # the trace's last row is what the output norm and head see
    head_in = O.rms_norm(xa[-1], W["output_norm"], W["cfg"]["eps"])
    bb, dt = W["lm_head"]
    assert np.array_equal(O.mm_1d(head_in, bb, dt, W["cfg"]["vocab"], W["cfg"]["d_model"]).view(np.uint32),
                          la.view(np.uint32))
