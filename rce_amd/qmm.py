"""Python mirror of the reference's quantized-matmul operator API over the
C ABI of librce_qmm.so.

Names follow ``compute/crates/rce-op-qmm/src/lib.rs``: ``GgufDtype``
(``rce-ingest-gguf/src/parser.rs`` L227-378), ``QuantWeight`` (L60-210,
here device-resident), ``mm_1d`` (L216-270), ``mm_1d_serial`` (L281-304),
``mm_batched`` (L967-1023), plus ``moe_router``/``moe_combine``-based grouped
experts (``rce-op-moe/src/lib.rs``).  The arithmetic runs in the HIP kernels
of ``rce_amd/csrc``; this module only marshals arguments.  Where the
reference panics (unsupported dtype, L268) the library returns
``RCE_QMM_UNSUPPORTED_DTYPE`` and this module raises ``QmmError``.
"""
from __future__ import annotations

import ctypes
import enum

import numpy as np

from ._lib import QmmError, check, lib

__all__ = [
    "GgufDtype", "Mode", "Context", "QuantWeight", "DeviceBuffer", "QmmError",
    "block_geometry", "row_bytes", "supports", "mm_1d", "mm_1d_serial", "mm_batched",
    "mm_batched_dev", "moe_router", "moe_ffn_dev", "moe_swiglu_dev", "quantize",
]


class GgufDtype(enum.IntEnum):
    """GGUF type tags (GgufDtype::from_u32 / to_u32, parser.rs L306-378)."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2K = 10
    Q3K = 11
    Q4K = 12
    Q5K = 13
    Q6K = 14
    BF16 = 30
    I2S = 36      # BitNet b1.58 (parser.rs L336)
    Q1_0 = 41     # PrismML Bonsai
    Q2_0 = 42     # PrismML Ternary-Bonsai
    # Tencent STQ1_0 shares file tag 42 with Q2_0 (parser.rs L376-377);
    # the library names it tag 42 with bit 31 set (RCE_QMM_DTYPE_STQ1_0).
    STQ1_0 = 0x8000002A

    @classmethod
    def from_u32(cls, v: int) -> "GgufDtype":
        return cls(v)

    def to_u32(self) -> int:
        return 42 if self is GgufDtype.STQ1_0 else int(self)


class Mode(enum.IntEnum):
    EXACT = 0
    Q8 = 1
    F16_MFMA = 2


# (values per block, bytes per block): dequant.rs L18-60 tensor_byte_size.
_GEOMETRY = {
    GgufDtype.F32: (1, 4), GgufDtype.F16: (1, 2), GgufDtype.BF16: (1, 2),
    GgufDtype.Q4_0: (32, 18), GgufDtype.Q4_1: (32, 20), GgufDtype.Q5_0: (32, 22),
    GgufDtype.Q5_1: (32, 24), GgufDtype.Q8_0: (32, 34), GgufDtype.Q8_1: (32, 36),
    GgufDtype.Q2K: (256, 84), GgufDtype.Q3K: (256, 110), GgufDtype.Q4K: (256, 144),
    GgufDtype.Q5K: (256, 176), GgufDtype.Q6K: (256, 210),
    GgufDtype.I2S: (128, 32),  # plus one f32 scale per tensor
    GgufDtype.Q1_0: (128, 18), GgufDtype.Q2_0: (128, 34), GgufDtype.STQ1_0: (256, 42),
}


def block_geometry(dtype) -> tuple[int, int]:
    return _GEOMETRY[GgufDtype(dtype)]


def row_bytes(dtype, n_cols: int) -> int:
    qk, bb = block_geometry(dtype)
    return n_cols // qk * bb


def supports(dtype, n_cols: int, mode: Mode = Mode.EXACT) -> bool:
    """MetalQmmContext::supports (rce-op-qmm-metal/src/lib.rs L127-139)."""
    return bool(lib().rce_qmm_supports(int(dtype), int(n_cols), int(mode)))


def _ptr(a: np.ndarray) -> ctypes.c_void_p:
    return a.ctypes.data_as(ctypes.c_void_p)


class Context:
    """One device + one HIP stream + scratch (rce_qmm_context)."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        check(lib().rce_qmm_context_create(int(device), ctypes.byref(h)))
        self._h = h
        self.device = device

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise QmmError(1, "context is closed")
        return self._h

    @property
    def stream(self) -> int:
        s = ctypes.c_void_p()
        check(lib().rce_qmm_context_stream(self.handle, ctypes.byref(s)))
        return s.value or 0

    def synchronize(self) -> None:
        check(lib().rce_qmm_synchronize(self.handle))

    def close(self) -> None:
        if self._h is not None:
            lib().rce_qmm_context_destroy(self._h)
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


class QuantWeight:
    """Device-resident QuantWeight (rce-op-qmm/src/lib.rs L76-91)."""

    def __init__(self, ctx: Context, handle: ctypes.c_void_p, parent: "QuantWeight | None" = None):
        self.ctx = ctx
        self._h = handle
        self._parent = parent
        dt, nr, nc, ln = ctypes.c_uint32(), ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
        check(lib().rce_qmm_weight_info(handle, ctypes.byref(dt), ctypes.byref(nr), ctypes.byref(nc),
                                        ctypes.byref(ln)))
        self.dtype = GgufDtype(dt.value)
        self.n_rows = nr.value
        self.n_cols = nc.value
        self.len = ln.value

    @classmethod
    def from_owned_bytes(cls, ctx: Context, data, dtype, n_rows: int, n_cols: int) -> "QuantWeight":
        """QuantWeight::from_owned_bytes (L123-138): uploads once to HBM."""
        b = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray))
                                 else data, dtype=np.uint8).reshape(-1)
        h = ctypes.c_void_p()
        check(lib().rce_qmm_weight_from_bytes(ctx.handle, int(dtype), n_rows, n_cols, _ptr(b), b.size,
                                              ctypes.byref(h)))
        return cls(ctx, h)

    @classmethod
    def from_gguf(cls, ctx: Context, gguf, name: str, n_rows: int, n_cols: int) -> "QuantWeight":
        """QuantWeight::from_gguf (L173-209): tensor `name` of a GgufFile
        (rce_amd.gguf) as a device-resident weight of the declared
        [n_rows, n_cols] (n_rows * n_cols must be its element count)."""
        h = ctypes.c_void_p()
        check(lib().rce_qmm_weight_from_gguf(ctx.handle, gguf.handle, name.encode("utf-8"), n_rows, n_cols,
                                             ctypes.byref(h)))
        return cls(ctx, h)

    def sub_view(self, byte_offset: int, byte_len: int, n_rows: int, n_cols: int) -> "QuantWeight":
        """QuantWeight::sub_view (L99-118): shares the device copy."""
        h = ctypes.c_void_p()
        check(lib().rce_qmm_weight_sub_view(self._h, byte_offset, byte_len, n_rows, n_cols,
                                            ctypes.byref(h)))
        return QuantWeight(self.ctx, h, parent=self)

    def dequant_row(self, row: int) -> np.ndarray:
        """QuantWeight::dequant_row (L150-167)."""
        out = np.empty(self.n_cols, np.float32)
        check(lib().rce_qmm_dequant_row(self.ctx.handle, self._h, row, _ptr(out)))
        return out

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def close(self) -> None:
        if self._h is not None:
            lib().rce_qmm_weight_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _host_call(fn, ctx: Context, a, t_rows: int, w: QuantWeight, out):
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    if a.size != t_rows * w.n_cols:
        raise QmmError(2, f"activation size {a.size} != {t_rows}x{w.n_cols}")
    res = np.empty(t_rows * w.n_rows, np.float32) if out is None else out
    if res.dtype != np.float32 or not res.flags.c_contiguous or res.size < t_rows * w.n_rows:
        raise QmmError(2, "out must be a contiguous float32 array of at least t_rows*n_rows")
    if fn is lib().rce_qmm_mm_batched:
        check(fn(ctx.handle, _ptr(a), t_rows, w.handle, _ptr(res)))
    else:
        check(fn(ctx.handle, _ptr(a), w.handle, _ptr(res)))
    return res


def mm_1d(a, w: QuantWeight, out: np.ndarray | None = None) -> np.ndarray:
    """out[j] = sum_i a[i] W[j, i], bit-identical to rce_op_qmm::mm_1d."""
    return _host_call(lib().rce_qmm_mm_1d, w.ctx, a, 1, w, out)


def mm_1d_serial(a, w: QuantWeight, out: np.ndarray | None = None) -> np.ndarray:
    """rce_op_qmm::mm_1d_serial: same result as mm_1d."""
    return _host_call(lib().rce_qmm_mm_1d_serial, w.ctx, a, 1, w, out)


def mm_batched(a, t_rows: int, w: QuantWeight, out: np.ndarray | None = None) -> np.ndarray:
    """rce_op_qmm::mm_batched: a [t_rows, n_cols] -> [t_rows, n_rows]."""
    r = _host_call(lib().rce_qmm_mm_batched, w.ctx, a, t_rows, w, out)
    return r.reshape(t_rows, w.n_rows) if out is None else r


def quantize(w, dtype) -> np.ndarray:
    """GGUF bytes of f32 weights [n_rows, n_cols] (rce_qmm_quantize: the
    reference's quantize_block / quantize_k encoders; host only)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    if w.ndim == 1:
        w = w.reshape(1, -1)
    n_rows, n_cols = w.shape
    out = np.empty(n_rows * row_bytes(dtype, n_cols), np.uint8)
    check(lib().rce_qmm_quantize(int(dtype), _ptr(w), n_rows, n_cols, _ptr(out), out.size))
    return out


class DeviceBuffer:
    """A device allocation made through the library (rce_qmm_dev_alloc)."""

    def __init__(self, ctx: Context, nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().rce_qmm_dev_alloc(ctx.handle, self.nbytes, ctypes.byref(p)))
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, ctx: Context, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(ctx, a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise QmmError(2, "upload larger than buffer")
        check(lib().rce_qmm_memcpy_h2d(self.ctx.handle, ctypes.c_void_p(self.ptr), _ptr(a), a.nbytes))

    def download(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype)
        if out.nbytes > self.nbytes:
            raise QmmError(2, "download larger than buffer")
        check(lib().rce_qmm_memcpy_d2h(self.ctx.handle, _ptr(out), ctypes.c_void_p(self.ptr), out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            check(lib().rce_qmm_dev_free(self.ctx.handle, ctypes.c_void_p(self.ptr)))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def mm_batched_dev(ctx: Context, a_dev: int, a_dtype, t_rows: int, w: QuantWeight, out_dev: int,
                   mode: Mode = Mode.EXACT, stream: int | None = None) -> None:
    """Asynchronous mm_batched on device buffers (a_dtype F32 or F16)."""
    check(lib().rce_qmm_mm_batched_dev(ctx.handle, ctypes.c_void_p(a_dev), int(a_dtype), t_rows, w.handle,
                                       ctypes.c_void_p(out_dev), int(mode),
                                       ctypes.c_void_p(stream) if stream else None))


def mm_batched_dev_noalloc(ctx: Context, a_dev: int, a_dtype, t_rows: int, w: QuantWeight, out_dev: int,
                           mode: Mode = Mode.EXACT, stream: int | None = None) -> None:
    """mm_batched_dev with its scratch in the library's fixed per-GPU array
    (rce_qmm_mm_batched_dev_noalloc): no device allocation."""
    check(lib().rce_qmm_mm_batched_dev_noalloc(ctx.handle, ctypes.c_void_p(a_dev), int(a_dtype), t_rows, w.handle,
                                               ctypes.c_void_p(out_dev), int(mode),
                                               ctypes.c_void_p(stream) if stream else None))


NOALLOC_SCRATCH_BYTES = 16 << 20  # RCE_QMM_NOALLOC_SCRATCH_BYTES


def moe_router(logits, top_k: int, normalize: bool = True):
    """rce_op_moe::moe_router from logits [n_tokens, n_expert]."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    if lg.ndim == 1:
        lg = lg.reshape(1, -1)
    n_tokens, n_expert = lg.shape
    ids = np.empty((n_tokens, top_k), np.int32)
    wts = np.empty((n_tokens, top_k), np.float32)
    check(lib().rce_qmm_moe_router(_ptr(lg), n_tokens, n_expert, top_k, int(normalize), _ptr(ids), _ptr(wts)))
    return ids, wts


def moe_ffn_dev(ctx: Context, w1: list[QuantWeight], w2: list[QuantWeight], x_dev: int, t_rows: int,
                ids_dev: int, weights_dev: int, top_k: int, out_dev: int, mode: Mode = Mode.F16_MFMA,
                stream: int | None = None) -> None:
    """Grouped-expert FFN (rce_qmm_moe_ffn_dev) on device buffers."""
    n = len(w1)
    A1 = (ctypes.c_void_p * n)(*[w.handle.value for w in w1])
    A2 = (ctypes.c_void_p * n)(*[w.handle.value for w in w2])
    check(lib().rce_qmm_moe_ffn_dev(ctx.handle, ctypes.cast(A1, ctypes.c_void_p), ctypes.cast(A2, ctypes.c_void_p),
                                    n, ctypes.c_void_p(x_dev), t_rows, ctypes.c_void_p(ids_dev),
                                    ctypes.c_void_p(weights_dev), top_k, ctypes.c_void_p(out_dev), int(mode),
                                    ctypes.c_void_p(stream) if stream else None))


def moe_swiglu_dev(ctx: Context, gate: list[QuantWeight], up: list[QuantWeight], down: list[QuantWeight], x_dev: int,
                   t_rows: int, ids_dev: int, weights_dev: int, top_k: int, out_dev: int,
                   mode: Mode = Mode.F16_MFMA, stream: int | None = None) -> None:
    """SwiGLU grouped experts (rce_qmm_moe_swiglu_dev): rce-qwen36-moe's
    routed experts down . (silu(gate . x) * (up . x)), combined in decision
    order."""
    n = len(gate)
    arr = lambda ws: (ctypes.c_void_p * n)(*[w.handle.value for w in ws])  # noqa: E731
    G, U, D = arr(gate), arr(up), arr(down)
    check(lib().rce_qmm_moe_swiglu_dev(ctx.handle, ctypes.cast(G, ctypes.c_void_p), ctypes.cast(U, ctypes.c_void_p),
                                       ctypes.cast(D, ctypes.c_void_p), n, ctypes.c_void_p(x_dev), t_rows,
                                       ctypes.c_void_p(ids_dev), ctypes.c_void_p(weights_dev), top_k,
                                       ctypes.c_void_p(out_dev), int(mode),
                                       ctypes.c_void_p(stream) if stream else None))
