"""Python mirror of the reference's TinyLlama decode runtime over the C ABI
(``rce_qmm_llama_*`` in include/rce_qmm.h).

Names follow ``compute/crates/rce-tinyllama/src/lib.rs``: ``TinyLlamaConfig``
(L28-41), ``TinyLlamaBlock`` (L94-99), ``TinyLlamaWeights`` (L101-106) and the
runtime's ``new_state`` / ``forward_logits`` / ``forward_logits_embed``
(L355-363; ``forward_token`` L289-294, ``forward_embedding`` L303-330).  Here
the weights are device-resident ``QuantWeight`` handles, the state (KV caches
and position) lives on the device inside the runtime object, and one decode
step runs on the GPU as a recorded HIP graph: every linear on the decode GEMV
kernels, rms_norm / RoPE / attention / silu / residual adds on device
kernels.  There is no CPU path.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from ._lib import check, lib
from .qmm import Context, Mode, QmmError, QuantWeight

__all__ = ["TinyLlamaConfig", "TinyLlamaBlock", "TinyLlamaWeights", "TinyLlamaRuntime"]


@dataclass
class TinyLlamaConfig:
    d_model: int
    vocab: int
    n_layers: int
    n_q_heads: int
    n_kv_heads: int
    d_head: int
    rope_dim: int
    rope_freq_base: float
    d_ff: int
    context_length: int
    eps: float

    def n_embd_q(self) -> int:
        return self.n_q_heads * self.d_head

    def n_embd_kv(self) -> int:
        return self.n_kv_heads * self.d_head


@dataclass
class TinyLlamaBlock:
    attn_norm: np.ndarray
    ffn_norm: np.ndarray
    wq: QuantWeight
    wk: QuantWeight
    wv: QuantWeight
    wo: QuantWeight
    ffn_gate: QuantWeight
    ffn_up: QuantWeight
    ffn_down: QuantWeight


@dataclass
class TinyLlamaWeights:
    token_embd: QuantWeight
    output_norm: np.ndarray
    lm_head: QuantWeight  # separate output.weight (not tied)
    blocks: list


class _Cfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in ("d_model", "vocab", "n_layers", "n_q_heads", "n_kv_heads", "d_head",
                                                 "rope_dim", "d_ff", "context_length")] + \
               [("rope_freq_base", ctypes.c_float), ("eps", ctypes.c_float)]


class _Block(ctypes.Structure):
    _fields_ = [("attn_norm", ctypes.c_void_p), ("ffn_norm", ctypes.c_void_p)] + \
               [(n, ctypes.c_void_p) for n in ("wq", "wk", "wv", "wo", "ffn_gate", "ffn_up", "ffn_down")]


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class TinyLlamaRuntime:
    """Device-resident decoder (rce_qmm_llama).  ``mode`` picks the decode
    GEMV numerics of every linear: Mode.EXACT (the reference's f32 order)
    or Mode.Q8 (Q8 activations)."""

    LINEARS = ("wq", "wk", "wv", "wo", "ffn_gate", "ffn_up", "ffn_down")

    def __init__(self, ctx: Context, cfg: TinyLlamaConfig, weights: TinyLlamaWeights, mode: Mode = Mode.EXACT):
        self.ctx, self.cfg, self.weights, self.mode = ctx, cfg, weights, Mode(mode)
        c = _Cfg(cfg.d_model, cfg.vocab, cfg.n_layers, cfg.n_q_heads, cfg.n_kv_heads, cfg.d_head, cfg.rope_dim,
                 cfg.d_ff, cfg.context_length, cfg.rope_freq_base, cfg.eps)
        norms = []
        blocks = (_Block * max(1, len(weights.blocks)))()
        for i, b in enumerate(weights.blocks):
            an, fn = _f32(b.attn_norm), _f32(b.ffn_norm)
            if an.size != cfg.d_model or fn.size != cfg.d_model:
                raise QmmError(2, f"norm weights of layer {i} must have d_model values")
            norms += [an, fn]
            blocks[i] = _Block(an.ctypes.data, fn.ctypes.data, *[getattr(b, n).handle.value for n in self.LINEARS])
        on = _f32(weights.output_norm)
        if on.size != cfg.d_model:
            raise QmmError(2, "output_norm must have d_model values")
        h = ctypes.c_void_p()
        check(lib().rce_qmm_llama_create(ctx.handle, ctypes.byref(c), weights.token_embd.handle, on.ctypes.data,
                                         weights.lm_head.handle, ctypes.cast(blocks, ctypes.c_void_p), int(self.mode),
                                         ctypes.byref(h)))
        self._h = h

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise QmmError(1, "decoder is closed")
        return self._h

    def new_state(self) -> None:
        """TinyLlamaRuntime::new_state: back to position 0, empty caches."""
        check(lib().rce_qmm_llama_reset(self.handle))

    @property
    def pos(self) -> int:
        p = ctypes.c_size_t()
        check(lib().rce_qmm_llama_pos(self.handle, ctypes.byref(p)))
        return p.value

    def forward_logits(self, token_id: int) -> np.ndarray:
        """forward_token: logits [vocab] of token_id at the current position."""
        out = np.empty(self.cfg.vocab, np.float32)
        check(lib().rce_qmm_llama_forward_token(self.handle, int(token_id), out.ctypes.data_as(ctypes.c_void_p)))
        return out

    def forward_logits_embed(self, embedding) -> np.ndarray:
        """forward_embedding from a [d_model] input embedding."""
        e = _f32(embedding)
        if e.size != self.cfg.d_model:
            raise QmmError(2, f"embedding length {e.size} must equal d_model={self.cfg.d_model}")
        out = np.empty(self.cfg.vocab, np.float32)
        check(lib().rce_qmm_llama_forward_embedding(self.handle, e.ctypes.data_as(ctypes.c_void_p),
                                                    out.ctypes.data_as(ctypes.c_void_p)))
        return out

    def forward_token_dev(self, token_dev: int, logits_dev: int, stream: int | None = None) -> None:
        """Asynchronous step on device memory (token id int32, logits f32)."""
        check(lib().rce_qmm_llama_forward_token_dev(self.handle, ctypes.c_void_p(token_dev),
                                                    ctypes.c_void_p(logits_dev),
                                                    ctypes.c_void_p(stream) if stream else None))

    def check(self) -> None:
        """Wait and raise for an error found on the device (bad token id)."""
        check(lib().rce_qmm_llama_check(self.handle))

    def close(self) -> None:
        if self._h is not None:
            lib().rce_qmm_llama_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
