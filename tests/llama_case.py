"""Synthetic Llama-2 decoders for the decode-step tests: random N(0, sigma)
weights quantized to GGUF bytes by the library's quantizer (checked against
the oracle's in test_quantize.py), norm weights near 1, and the matching
oracle model (oracle.Llama) and device runtime (rce_amd.TinyLlamaRuntime)."""
from __future__ import annotations

import numpy as np

import oracle as O

LIN = ("wq", "wk", "wv", "wo", "ffn_gate", "ffn_up", "ffn_down")


def tiny_cfg(**kw) -> dict:
    c = dict(d_model=256, vocab=320, n_layers=2, n_q_heads=4, n_kv_heads=2, d_head=64, rope_dim=64,
             rope_freq_base=10000.0, d_ff=512, context_length=32, eps=1e-5)
    c.update(kw)
    return c


def shapes(c: dict) -> dict:
    qd, kvd = c["n_q_heads"] * c["d_head"], c["n_kv_heads"] * c["d_head"]
    dm, ff = c["d_model"], c["d_ff"]
    return {"wq": (qd, dm), "wk": (kvd, dm), "wv": (kvd, dm), "wo": (dm, qd),
            "ffn_gate": (ff, dm), "ffn_up": (ff, dm), "ffn_down": (dm, ff)}


def make_weights(c: dict, seed: int, lin_dtype=O.Q4_K, head_dtype=O.Q6_K, embd_dtype=O.Q4_K,
                 dtype_of=None, sigma: float = 0.05, unit_norms: bool = False) -> dict:
    """Host weights: GGUF bytes + dtypes and f32 norms.  dtype_of(layer,
    name) overrides the linear format per weight."""
    import rce_amd
    rng = np.random.default_rng(seed)

    def q(n, k, dt):
        if dt in (O.F32, O.F16, O.BF16):
            from rand_blocks import float_bytes
            return float_bytes(rng, dt, n, k, sigma), dt
        if dt in (O.Q5_0, O.Q4_1, O.Q3_K):  # no quantizer in the reference: random blocks of about sigma
            from rand_blocks import rand_blocks
            return rand_blocks(rng, dt, n, k, dmax=sigma / (32 if dt == O.Q3_K else 8)), dt
        w = (rng.standard_normal((n, k)) * sigma).astype(np.float32)
        return rce_amd.quantize(w, dt), dt

    def norm():
        if unit_norms:
            return np.ones(c["d_model"], np.float32)
        return (1.0 + 0.1 * rng.standard_normal(c["d_model"])).astype(np.float32)

    sh = shapes(c)
    blocks = []
    for il in range(c["n_layers"]):
        b = {"attn_norm": norm(), "ffn_norm": norm()}
        for n in LIN:
            dt = dtype_of(il, n) if dtype_of else lin_dtype
            b[n] = q(*sh[n], dt)
        blocks.append(b)
    return {"cfg": dict(c), "token_embd": q(c["vocab"], c["d_model"], embd_dtype), "output_norm": norm(),
            "lm_head": q(c["vocab"], c["d_model"], head_dtype), "blocks": blocks}


def oracle_model(W: dict, q8: bool = False) -> O.Llama:
    return O.Llama(W["cfg"], W["token_embd"], W["output_norm"], W["lm_head"], W["blocks"], q8=q8)


def device_model(ctx, W: dict, mode):
    import rce_amd
    c = W["cfg"]
    qw = lambda bd, n, k: rce_amd.QuantWeight.from_owned_bytes(ctx, bd[0], bd[1], n, k)  # noqa: E731
    sh = shapes(c)
    blocks = []
    for b in W["blocks"]:
        ws = {n: qw(b[n], *sh[n]) for n in LIN}
        blocks.append(rce_amd.TinyLlamaBlock(b["attn_norm"], b["ffn_norm"], **ws))
    weights = rce_amd.TinyLlamaWeights(qw(W["token_embd"], c["vocab"], c["d_model"]), W["output_norm"],
                                       qw(W["lm_head"], c["vocab"], c["d_model"]), blocks)
    cfg = rce_amd.TinyLlamaConfig(**c)
    return rce_amd.TinyLlamaRuntime(ctx, cfg, weights, mode)


# Formats whose decode GEMV has the fused forms (rms_norm inside the GEMV);
# Q6_K only in Q8 mode (its EXACT kernel is a row chain).
_FX = {O.Q4_0: 32, O.Q8_0: 32, O.Q5_0: 32, O.Q4_1: 32, O.Q3_K: 32, O.Q4_K: 64, O.Q5_K: 64, O.Q6_K: 256}


def _fused_nt(dt, n_cols, q8):
    """Threads of the fused GEMV whose blocks form rms_norm (None: no fused
    norm for this weight): 256 / 512 / 1024 by the row's column units."""
    if dt not in _FX or (dt == O.Q6_K and not q8):
        return None
    u = n_cols // _FX[dt]
    nt = 256 if u <= 256 else (512 if u <= 512 else 1024)
    return nt if n_cols // 8 <= 2 * nt else None


def device_order(W: dict, q8: bool, separate_norms: bool = False):
    """(nt_layers, nt_head) of oracle.Llama's device-order mode for the
    device decoder of W: the fused forms' thread count where the decoder
    forms rms_norm inside the q|k|v, gate/up and head GEMVs, -256 where it
    runs the separate norm kernel.  None where the layers' norms do not all
    take one form (mixed linear formats)."""
    dm = W["cfg"]["d_model"]
    forms = set()
    for b in W["blocks"]:
        qkv = {b[n][1] for n in ("wq", "wk", "wv")}
        gu = {b[n][1] for n in ("ffn_gate", "ffn_up")}
        for grp in (qkv, gu):
            nt = _fused_nt(next(iter(grp)), dm, q8) if len(grp) == 1 else None
            forms.add(-256 if separate_norms or nt is None else nt)
    if len(forms) != 1:
        return None
    nt_head = _fused_nt(W["lm_head"][1], dm, q8)
    return forms.pop(), (-256 if separate_norms or nt_head is None else nt_head)


def oracle_model_dev(W: dict, q8: bool = False, separate_norms: bool = False):
    """The oracle's decoder in the device's own orders (bit-identical
    target), or None where device_order has no single form."""
    order = device_order(W, q8, separate_norms)
    if order is None:
        return None
    return O.Llama(W["cfg"], W["token_embd"], W["output_norm"], W["lm_head"], W["blocks"], q8=q8,
                   device_order=order)


def normwise(got, want) -> float:
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - want)) / np.max(np.abs(want)))
