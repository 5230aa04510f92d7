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

__all__ = ["TinyLlamaConfig", "TinyLlamaBlock", "TinyLlamaWeights", "TinyLlamaRuntime", "load_weights"]


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

    @classmethod
    def from_gguf(cls, gguf) -> "TinyLlamaConfig":
        """TinyLlamaConfig::from_gguf (rce-tinyllama/src/lib.rs L44-89): the
        llama.* metadata of a GgufFile (rce_amd.gguf), with the reference's
        defaults and fallbacks; QmmError(BAD_SHAPE) naming a missing key."""
        arch = gguf.get_string("general.architecture")
        if arch is None:
            raise QmmError(2, "missing general.architecture")
        if arch != "llama":
            raise QmmError(2, f"expected llama, got {arch}")
        u32 = lambda k: gguf.get_u32(f"llama.{k}")  # noqa: E731
        f32 = lambda k: gguf.get_f32(f"llama.{k}")  # noqa: E731

        def need(k):
            v = u32(k)
            if v is None:
                raise QmmError(2, k)
            return v

        d_model = need("embedding_length")
        vocab = u32("vocab_size")
        if vocab is None:  # the token embedding's second dimension
            t = gguf.tensor("token_embd.weight")
            vocab = t.dims[1] if t is not None and len(t.dims) > 1 else None
        if vocab is None:
            raise QmmError(2, "vocab_size")
        n_layers = need("block_count")
        n_q = need("attention.head_count")
        n_kv = u32("attention.head_count_kv")
        n_kv = n_q if n_kv is None else n_kv
        d_head = d_model // n_q
        rope_dim = u32("rope.dimension_count")
        rope_base = f32("rope.freq_base")
        ctx_len = u32("context_length")
        eps = f32("attention.layer_norm_rms_epsilon")
        return cls(d_model=d_model, vocab=vocab, n_layers=n_layers, n_q_heads=n_q, n_kv_heads=n_kv, d_head=d_head,
                   rope_dim=d_head if rope_dim is None else rope_dim,
                   rope_freq_base=10000.0 if rope_base is None else rope_base, d_ff=need("feed_forward_length"),
                   context_length=2048 if ctx_len is None else ctx_len, eps=1e-5 if eps is None else eps)

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


def load_weights(ctx: Context, gguf, cfg: TinyLlamaConfig) -> TinyLlamaWeights:
    """load_weights (rce-tinyllama/src/lib.rs L108-145): every linear as a
    device-resident QuantWeight (QuantWeight::from_gguf), the norms read as
    f32 (read_tensor_f32); errors name the tensor."""
    def qw(name, n_rows, n_cols):
        try:
            return QuantWeight.from_gguf(ctx, gguf, name, n_rows, n_cols)
        except QmmError as e:
            raise QmmError(e.status, f"{name}: {e}") from None

    def f32n(name):
        try:
            return gguf.read_tensor_f32(name)
        except QmmError as e:
            raise QmmError(e.status, f"{name}: {e}") from None

    token_embd = qw("token_embd.weight", cfg.vocab, cfg.d_model)
    output_norm = f32n("output_norm.weight")
    lm_head = qw("output.weight", cfg.vocab, cfg.d_model)
    blocks = []
    for il in range(cfg.n_layers):
        bn = f"blk.{il}"
        blocks.append(TinyLlamaBlock(
            attn_norm=f32n(f"{bn}.attn_norm.weight"), ffn_norm=f32n(f"{bn}.ffn_norm.weight"),
            wq=qw(f"{bn}.attn_q.weight", cfg.n_embd_q(), cfg.d_model),
            wk=qw(f"{bn}.attn_k.weight", cfg.n_embd_kv(), cfg.d_model),
            wv=qw(f"{bn}.attn_v.weight", cfg.n_embd_kv(), cfg.d_model),
            wo=qw(f"{bn}.attn_output.weight", cfg.d_model, cfg.n_embd_q()),
            ffn_gate=qw(f"{bn}.ffn_gate.weight", cfg.d_ff, cfg.d_model),
            ffn_up=qw(f"{bn}.ffn_up.weight", cfg.d_ff, cfg.d_model),
            ffn_down=qw(f"{bn}.ffn_down.weight", cfg.d_model, cfg.d_ff)))
    return TinyLlamaWeights(token_embd=token_embd, output_norm=output_norm, lm_head=lm_head, blocks=blocks)


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

    @classmethod
    def load(cls, ctx: Context, path, mode: Mode = Mode.EXACT) -> "TinyLlamaRuntime":
        """TinyLlamaRuntime::load (rce-tinyllama/src/lib.rs L339-354): map and
        parse the GGUF file, read the config and upload every weight once;
        the file is closed again when the weights are on the device."""
        from .gguf import GgufFile
        with GgufFile.open(path) as g:
            cfg = TinyLlamaConfig.from_gguf(g)
            weights = load_weights(ctx, g, cfg)
        return cls(ctx, cfg, weights, mode)

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
