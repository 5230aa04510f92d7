"""CPU restatement of the reference's GGUF quantized-matmul path.

TEST INFRASTRUCTURE ONLY.  This package is the parity checker and the CPU
baseline; only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it, and never as the thing measured or
shipped.  The product (``rce_amd``, ``include/``) does not depend on it.

The C source ``qmm_oracle.c`` restates, in the reference's operation
order, the kernels of ``compute/crates/rce-op-qmm/src/lib.rs``, the
dequantizers of ``compute/crates/rce-ingest-gguf/src/dequant.rs``, the
quantizers and value-form products of
``compute/crates/rce-vm-backend-cpu/src/ml/{nn,kquant}.rs`` and the MoE
router/combine of ``compute/crates/rce-op-moe/src/lib.rs`` and the Llama-2
decode step of ``compute/crates/rce-tinyllama/src/lib.rs`` with the RoPE and
attention of ``compute/crates/rce-op-attn/src/lib.rs``; each C function
cites the file:line it follows.  The reference itself is Rust and cannot be
built here, so there is no ``oracle/_ref`` build.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_qmm.so")

# GGUF type tags (rce-ingest-gguf/src/parser.rs L306-341).
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 = 0, 1, 2, 3, 6, 7, 8
Q3_K, Q4_K, Q5_K, Q6_K, BF16 = 11, 12, 13, 14, 30
I2_S, Q1_0, Q2_0 = 36, 41, 42
STQ1_0 = 0x8000002A  # file tag 42 (shared with Q2_0) read as STQ1_0: this build's name for it
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20),
         Q5_0: (32, 22), Q8_0: (32, 34), Q3_K: (256, 110), Q4_K: (256, 144),
         Q5_K: (256, 176), Q6_K: (256, 210), I2_S: (128, 32), Q1_0: (128, 18), Q2_0: (128, 34),
         STQ1_0: (256, 42)}

_lib = None


def build() -> str:
    """Compile liboracle_qmm.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P, S, U32, I, F = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_int, ctypes.c_float
        sig = {
            "orc_f16_to_f32": (F, [ctypes.c_uint16]),
            "orc_round_to_f16": (F, [F]),
            "orc_f16_bits": (ctypes.c_uint16, [F]),
            "orc_block_geometry": (I, [U32, P, P]),
            "orc_tensor_byte_size": (S, [U32, S]),
            "orc_quantize_block": (None, [P, I, P, P]),
            "orc_quantize_q8_0_q4_0": (None, [P, S, I, P]),
            "orc_quantize_k": (None, [P, U32, P, P, P, P, P]),
            "orc_pack_k": (None, [P, P, P, F, F, U32, P]),
            "orc_unpack_k": (None, [P, U32, P, P, P, P, P]),
            "orc_quantize_tensor_k": (None, [P, S, U32, P]),
            "orc_dequantize": (I, [P, U32, S, P]),
            "orc_mm_batched": (I, [P, S, P, U32, S, S, P, I]),
            "orc_mm_1d": (I, [P, P, U32, S, S, P, I]),
            "orc_matmul_q": (None, [P, S, S, P, S, P, I, P]),
            "orc_matmul_k": (None, [P, S, S, P, S, P, P, U32, P]),
            "orc_quantize_act_q8": (None, [P, S, P, P, P]),
            "orc_mm_batched_q8": (I, [P, S, P, U32, S, S, P, I]),
            "orc_block_isums": (I, [P, P, U32, S, S, P]),
            "orc_silu": (F, [F]),
            "orc_moe_router": (None, [P, S, S, I, P, P]),
            "orc_moe_combine": (None, [P, P, S, S, P]),
            "orc_moe_ffn": (I, [P, S, S, S, P, P, U32, P, P, S, P, I, I]),
            "orc_moe_ffn2": (I, [P, S, S, S, P, P, U32, U32, P, P, S, P, I, I]),
            "orc_max_threads": (I, []),
            "orc_moe_swiglu_ffn": (I, [P, S, S, S, P, P, P, U32, P, P, S, P, I]),
            "orc_rms_norm": (None, [P, P, S, F, P]),
            "orc_rope": (None, [P, S, F, S, P]),
            "orc_attend_head": (None, [P, P, P, S, S, S, S, F, P]),
            "orc_llama_forward": (I, [P, F, F, I, P, P, P, P, P, P, P, U32, P, P, S, P, I, P, P]),
            "orc_exp_dev": (F, [F]),
            "orc_exp_dev_max_ulp": (ctypes.c_double, [U32, U32, P, I]),
            "orc_silu_dev": (F, [F]),
            "orc_rms_norm_dev": (None, [P, P, S, F, I, P]),
            "orc_attend_head_dev": (None, [P, P, P, S, S, S, S, F, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def max_threads() -> int:
    return int(lib().orc_max_threads())


def f16_to_f32(h: int) -> float:
    return float(lib().orc_f16_to_f32(int(h)))


def round_to_f16(x: float) -> float:
    return float(lib().orc_round_to_f16(float(x)))


def f16_bits(x: float) -> int:
    return int(lib().orc_f16_bits(float(x)))


def row_bytes(dtype: int, n_cols: int) -> int:
    qk, bb = BLOCK[dtype]
    return n_cols // qk * bb


def tensor_byte_size(dtype: int, n: int) -> int:
    return int(lib().orc_tensor_byte_size(dtype, n))


def quantize_block(x, q4: bool):
    x = _c(x, np.float32)
    assert x.size == 32
    q = np.zeros(32, np.int32)
    d = np.zeros(1, np.float32)
    lib().orc_quantize_block(_p(x), int(q4), _p(q), _p(d))
    return q, float(d[0])


def quantize(w, dtype: int) -> np.ndarray:
    """GGUF bytes of a flat f32 array (rows of n_cols back to back)."""
    w = _c(w, np.float32).reshape(-1)
    out = np.zeros(tensor_byte_size(dtype, w.size), np.uint8)
    if dtype in (Q8_0, Q4_0):
        assert w.size % 32 == 0
        lib().orc_quantize_q8_0_q4_0(_p(w), w.size, int(dtype == Q4_0), _p(out))
    elif dtype in (Q4_K, Q5_K, Q6_K):
        assert w.size % 256 == 0
        lib().orc_quantize_tensor_k(_p(w), w.size, dtype, _p(out))
    else:
        raise ValueError(f"no quantizer for dtype {dtype}")
    return out


def quantize_k(x, fmt: int):
    x = _c(x, np.float32)
    q = np.zeros(256, np.int32); sc = np.zeros(16, np.int32); mn = np.zeros(8, np.int32)
    d = np.zeros(1, np.float32); dm = np.zeros(1, np.float32)
    lib().orc_quantize_k(_p(x), fmt, _p(q), _p(sc), _p(mn), _p(d), _p(dm))
    nsc = 16 if fmt == Q6_K else 8
    return q, sc[:nsc].copy(), (mn.copy() if fmt != Q6_K else np.zeros(0, np.int32)), float(d[0]), float(dm[0])


def pack_k(q, sc, mn, d, dmin, fmt: int) -> np.ndarray:
    bb = BLOCK[fmt][1]
    out = np.zeros(bb, np.uint8)
    sc16 = np.zeros(16, np.int32); sc16[: len(sc)] = sc
    mn8 = np.zeros(8, np.int32); mn8[: len(mn)] = mn
    lib().orc_pack_k(_p(_c(q, np.int32)), _p(sc16), _p(mn8), float(d), float(dmin), fmt, _p(out))
    return out


def unpack_k(b, fmt: int):
    b = _c(b, np.uint8)
    q = np.zeros(256, np.int32); sc = np.zeros(16, np.int32); mn = np.zeros(8, np.int32)
    d = np.zeros(1, np.float32); dm = np.zeros(1, np.float32)
    lib().orc_unpack_k(_p(b), fmt, _p(q), _p(sc), _p(mn), _p(d), _p(dm))
    nsc = 16 if fmt == Q6_K else 8
    return q, sc[:nsc].copy(), (mn.copy() if fmt != Q6_K else np.zeros(0, np.int32)), float(d[0]), float(dm[0])


def dequantize(b, dtype: int, n: int) -> np.ndarray:
    b = _c(b, np.uint8)
    out = np.zeros(n, np.float32)
    if lib().orc_dequantize(_p(b), dtype, n, _p(out)) != 0:
        raise ValueError(f"unsupported dtype {dtype}")
    return out


def mm_batched(a, w_bytes, dtype: int, n_rows: int, n_cols: int, threads: int = 0) -> np.ndarray:
    """Exact-order reference result: out[t, j] for a [t_rows, n_cols]."""
    a = _c(a, np.float32)
    t_rows = a.size // n_cols
    w_bytes = _c(w_bytes, np.uint8)
    out = np.zeros((t_rows, n_rows), np.float32)
    rc = lib().orc_mm_batched(_p(a), t_rows, _p(w_bytes), dtype, n_rows, n_cols, _p(out),
                              threads or max_threads())
    if rc:
        raise ValueError(f"orc_mm_batched rc={rc}")
    return out


def mm_1d(a, w_bytes, dtype: int, n_rows: int, n_cols: int, threads: int = 0) -> np.ndarray:
    return mm_batched(a, w_bytes, dtype, n_rows, n_cols, threads)[0]


def mm_batched_q8(a, w_bytes, dtype: int, n_rows: int, n_cols: int, threads: int = 0) -> np.ndarray:
    """The Q8-activation path restated on the CPU (same definition as the GPU's)."""
    a = _c(a, np.float32)
    t_rows = a.size // n_cols
    w_bytes = _c(w_bytes, np.uint8)
    out = np.zeros((t_rows, n_rows), np.float32)
    rc = lib().orc_mm_batched_q8(_p(a), t_rows, _p(w_bytes), dtype, n_rows, n_cols, _p(out),
                                 threads or max_threads())
    if rc:
        raise ValueError(f"orc_mm_batched_q8 rc={rc}")
    return out


def quantize_act_q8(x):
    x = _c(x, np.float32)
    k = x.size
    xq = np.zeros(k, np.int8); dx = np.zeros(k // 32, np.float32); xs = np.zeros(k // 32, np.int32)
    lib().orc_quantize_act_q8(_p(x), k, _p(xq), _p(dx), _p(xs))
    return xq, dx, xs


def block_isums(xq, w_bytes, dtype: int, n_rows: int, n_cols: int) -> np.ndarray:
    out = np.zeros((n_rows, n_cols // 32), np.int32)
    rc = lib().orc_block_isums(_p(_c(xq, np.int8)), _p(_c(w_bytes, np.uint8)), dtype, n_rows, n_cols, _p(out))
    if rc:
        raise ValueError("unsupported")
    return out


def matmul_q(x, q, d, q4: bool) -> np.ndarray:
    x = _c(x, np.float32); q = _c(q, np.int32); d = _c(d, np.float32)
    m, k = x.shape; n = q.shape[0]
    out = np.zeros((m, n), np.float32)
    lib().orc_matmul_q(_p(x), m, k, _p(q), n, _p(d), int(q4), _p(out))
    return out


def matmul_k(x, q, s, o, fmt: int) -> np.ndarray:
    x = _c(x, np.float32); q = _c(q, np.int32); s = _c(s, np.float32)
    o = _c(o if o is not None else np.zeros(1, np.float32), np.float32)
    m, k = x.shape; n = q.shape[0]
    out = np.zeros((m, n), np.float32)
    lib().orc_matmul_k(_p(x), m, k, _p(q), n, _p(s), _p(o), fmt, _p(out))
    return out


def silu(x: float) -> float:
    return float(lib().orc_silu(float(x)))


def moe_router(logits, top_k: int, normalize: bool = True):
    logits = _c(logits, np.float32)
    idx = np.zeros(top_k, np.int32); w = np.zeros(top_k, np.float32)
    lib().orc_moe_router(_p(logits), logits.size, top_k, int(normalize), _p(idx), _p(w))
    return idx, w


def moe_combine(w, ys) -> np.ndarray:
    w = _c(w, np.float32); ys = _c(ys, np.float32)
    k, d = ys.shape
    out = np.zeros(d, np.float32)
    lib().orc_moe_combine(_p(w), _p(ys), k, d, _p(out))
    return out


def moe_ffn(x, w1_list, w2_list, dtype, d_ff, ids, gate_w, threads: int = 0, q8: bool = False,
            silu_dev: bool = False, dtype2: int | None = None) -> np.ndarray:
    """The grouped-expert FFN per (token, decision) in the reference's order;
    q8: the Q8-activation products; silu_dev: silu with exp_dev (the
    device's order); dtype2: the second matrices' dtype when it differs
    (a Q4_K_M model's Q6_K ffn_down_exps)."""
    x = _c(x, np.float32)
    t_rows, d_model = x.shape
    ids = _c(ids, np.int32); gate_w = _c(gate_w, np.float32)
    top_k = ids.shape[1]
    w1 = [_c(b, np.uint8) for b in w1_list]; w2 = [_c(b, np.uint8) for b in w2_list]
    P1 = (ctypes.c_void_p * len(w1))(*[b.ctypes.data for b in w1])
    P2 = (ctypes.c_void_p * len(w2))(*[b.ctypes.data for b in w2])
    out = np.zeros((t_rows, d_model), np.float32)
    rc = lib().orc_moe_ffn2(_p(x), t_rows, d_model, d_ff, ctypes.cast(P1, ctypes.c_void_p),
                            ctypes.cast(P2, ctypes.c_void_p), dtype, dtype if dtype2 is None else dtype2, _p(ids),
                            _p(gate_w), top_k, _p(out), threads or max_threads(), int(silu_dev) | (2 * int(q8)))
    if rc:
        raise ValueError(f"orc_moe_ffn rc={rc}")
    return out


def moe_swiglu_ffn(x, gate_list, up_list, down_list, dtype, d_ff, ids, gate_w, threads: int = 0) -> np.ndarray:
    """rce-qwen36-moe's routed SwiGLU experts (orc_moe_swiglu_ffn)."""
    x = _c(x, np.float32)
    t_rows, d_model = x.shape
    ids = _c(ids, np.int32); gate_w = _c(gate_w, np.float32)
    top_k = ids.shape[1]
    keep = [[_c(b, np.uint8) for b in L] for L in (gate_list, up_list, down_list)]
    ptrs = [(ctypes.c_void_p * len(L))(*[b.ctypes.data for b in L]) for L in keep]
    out = np.zeros((t_rows, d_model), np.float32)
    rc = lib().orc_moe_swiglu_ffn(_p(x), t_rows, d_model, d_ff, *[ctypes.cast(p, ctypes.c_void_p) for p in ptrs],
                                  dtype, _p(ids), _p(gate_w), top_k, _p(out), threads or max_threads())
    if rc:
        raise ValueError(f"orc_moe_swiglu_ffn rc={rc}")
    return out


# ---- Llama-2 decode step (rce-tinyllama L158-330, rce-op-attn L107-251) ----

def exp_dev(x: float) -> float:
    """The device library's exp (Cody-Waite reduction, Taylor degree 7)."""
    return float(lib().orc_exp_dev(float(x)))


def exp_dev_max_ulp(lo_bits: int, hi_bits: int, threads: int = 0):
    """Largest ulp error of exp_dev against the correctly rounded exp over
    the floats with bits in [lo_bits, hi_bits]; returns (ulps, worst input)."""
    wb = ctypes.c_uint32(0)
    u = lib().orc_exp_dev_max_ulp(lo_bits, hi_bits, ctypes.byref(wb), threads)
    return float(u), float(np.array([wb.value], np.uint32).view(np.float32)[0])


def silu_dev(x: float) -> float:
    return float(lib().orc_silu_dev(float(x)))


def rms_norm_dev(x, w, eps: float, nt: int) -> np.ndarray:
    """rms_norm with the device's sum-of-squares tree (nt > 0: the fused
    form's tasks of 8 over nt threads; nt < 0: the separate kernel's)."""
    x = _c(x, np.float32); w = _c(w, np.float32)
    out = np.zeros_like(x)
    lib().orc_rms_norm_dev(_p(x), _p(w), x.size, float(eps), int(nt), _p(out))
    return out


def attend_head_dev(q, k_cache, v_cache, kv_head: int, seq_len: int, kv_dim: int, d_head: int, scale: float):
    """One head's attention in the device's parallel order."""
    q = _c(q, np.float32); k_cache = _c(k_cache, np.float32); v_cache = _c(v_cache, np.float32)
    out = np.zeros(d_head, np.float32)
    lib().orc_attend_head_dev(_p(q), _p(k_cache), _p(v_cache), kv_head, seq_len, kv_dim, d_head, float(scale),
                              _p(out))
    return out


def rms_norm(x, w, eps: float) -> np.ndarray:
    x = _c(x, np.float32); w = _c(w, np.float32)
    out = np.zeros_like(x)
    lib().orc_rms_norm(_p(x), _p(w), x.size, float(eps), _p(out))
    return out


def rope(x, rope_dim: int, base: float, pos: int):
    """One head rotated in place (returns the new head and the (cos, sin)
    pairs used, shape [rope_dim // 2, 2])."""
    x = _c(x, np.float32).copy()
    cs = np.zeros((rope_dim // 2, 2), np.float32)
    lib().orc_rope(_p(x), rope_dim, float(base), pos, _p(cs))
    return x, cs


def attend_head(q, k_cache, v_cache, kv_head: int, seq_len: int, kv_dim: int, d_head: int, scale: float):
    q = _c(q, np.float32); k_cache = _c(k_cache, np.float32); v_cache = _c(v_cache, np.float32)
    out = np.zeros(d_head, np.float32)
    lib().orc_attend_head(_p(q), _p(k_cache), _p(v_cache), kv_head, seq_len, kv_dim, d_head, float(scale), _p(out))
    return out


class Llama:
    """The reference's TinyLlama decode (forward_embedding / forward_token)
    over GGUF weight bytes: cfg is a dict with d_model, vocab, n_layers,
    n_q_heads, n_kv_heads, d_head, rope_dim, rope_freq_base, d_ff,
    context_length, eps.  blocks: per layer a dict with attn_norm, ffn_norm
    (f32 arrays) and wq, wk, wv, wo, ffn_gate, ffn_up, ffn_down as
    (bytes, dtype).  token_embd and lm_head: (bytes, dtype).  q8: every
    linear uses the Q8-activation path instead of mm_1d.  device_order:
    None (the reference's order) or (nt_layers, nt_head), the GPU decode
    step's own orders (rms_norm_dev with those thread layouts,
    attend_head_dev, silu_dev)."""

    LIN = ("wq", "wk", "wv", "wo", "ffn_gate", "ffn_up", "ffn_down")

    def __init__(self, cfg, token_embd, output_norm, lm_head, blocks, q8: bool = False, threads: int = 0,
                 device_order=None):
        self.cfg = dict(cfg)
        c = self.cfg
        self.dims = np.array([c["d_model"], c["vocab"], c["n_layers"], c["n_q_heads"], c["n_kv_heads"],
                              c["d_head"], c["rope_dim"], c["d_ff"], c["context_length"]], np.uint64)
        self.token_embd = (_c(token_embd[0], np.uint8), int(token_embd[1]))
        self.output_norm = _c(output_norm, np.float32)
        self.lm_head = (_c(lm_head[0], np.uint8), int(lm_head[1]))
        self.attn_norm = _c(np.stack([b["attn_norm"] for b in blocks]), np.float32)
        self.ffn_norm = _c(np.stack([b["ffn_norm"] for b in blocks]), np.float32)
        self._bytes = [_c(b[n][0], np.uint8) for b in blocks for n in self.LIN]
        self._ptrs = (ctypes.c_void_p * len(self._bytes))(*[b.ctypes.data for b in self._bytes])
        self._types = np.array([int(b[n][1]) for b in blocks for n in self.LIN], np.uint32)
        self.q8 = q8
        self.threads = threads or max_threads()
        self.dev_order = None if device_order is None else np.array(device_order, np.int32)
        self.reset()

    def reset(self):
        c = self.cfg
        kv = c["n_kv_heads"] * c["d_head"]
        self.k_cache = np.zeros((c["n_layers"], c["context_length"], kv), np.float32)
        self.v_cache = np.zeros_like(self.k_cache)
        self.pos = 0

    def embed(self, token_id: int) -> np.ndarray:
        """QuantWeight::dequant_row (rce-op-qmm L150-167) of token_embd."""
        b, dt = self.token_embd
        dm = self.cfg["d_model"]
        rb = row_bytes(dt, dm)
        return dequantize(b[token_id * rb:(token_id + 1) * rb], dt, dm)

    def forward_embedding(self, embedding, trace: bool = False):
        """Logits of one step; with trace, also the residual stream entering
        each layer and leaving the last ([n_layers + 1, d_model])."""
        c = self.cfg
        e = _c(embedding, np.float32)
        assert e.size == c["d_model"]
        logits = np.zeros(c["vocab"], np.float32)
        xt = np.zeros((c["n_layers"] + 1, c["d_model"]), np.float32) if trace else None
        rc = lib().orc_llama_forward(
            _p(self.dims), float(c["rope_freq_base"]), float(c["eps"]), int(self.q8), _p(e),
            _p(self.attn_norm), _p(self.ffn_norm), ctypes.cast(self._ptrs, ctypes.c_void_p), _p(self._types),
            _p(self.output_norm), _p(self.lm_head[0]), self.lm_head[1], _p(self.k_cache), _p(self.v_cache),
            self.pos, _p(logits), self.threads, _p(xt) if trace else None,
            _p(self.dev_order) if self.dev_order is not None else None)
        if rc:
            raise ValueError(f"orc_llama_forward rc={rc}")
        self.pos += 1
        return (logits, xt) if trace else logits

    def forward_token(self, token_id: int, trace: bool = False):
        return self.forward_embedding(self.embed(token_id), trace)
