"""The "hip:op-qmm" priced backend for rce-placement-adapter
(compute/crates/rce-placement-adapter/src/lib.rs): the Python mirror of the
backend a Rust caller registers next to CpuQmm and MetalQmm (L205-283).

``HipQmm`` implements both halves of the adapter's split trait surface:
``PricedBackend`` (``id``, ``handles``, ``cost``, ``execute``; cost is the
library's rce_qmm_hip_cost) and ``QmmDispatch`` (``qmm_1d``, bit-identical
to rce_op_qmm::mm_1d).  A weight is uploaded once per distinct GGUF byte
buffer and reused (the Metal twin copies per call, rce-op-qmm-metal L773).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import numpy as np

from ._lib import check, lib
from .qmm import Context, GgufDtype, QuantWeight, mm_1d

# rce-placement-adapter/src/lib.rs L80-90
QMM_DTYPE_UNKNOWN, QMM_DTYPE_Q8_0, QMM_DTYPE_Q4_K, QMM_DTYPE_Q5_K, QMM_DTYPE_Q6_K = 0, 1, 2, 3, 4
QMM_DTYPE_Q4_0, QMM_DTYPE_Q5_0, QMM_DTYPE_Q4_1, QMM_DTYPE_Q1_0, QMM_DTYPE_Q2_0, QMM_DTYPE_Q3_K = 5, 6, 7, 8, 9, 10

_ID_OF = {GgufDtype.Q8_0: QMM_DTYPE_Q8_0, GgufDtype.Q3K: QMM_DTYPE_Q3_K, GgufDtype.Q4K: QMM_DTYPE_Q4_K,
          GgufDtype.Q5K: QMM_DTYPE_Q5_K, GgufDtype.Q6K: QMM_DTYPE_Q6_K, GgufDtype.Q4_0: QMM_DTYPE_Q4_0,
          GgufDtype.Q5_0: QMM_DTYPE_Q5_0, GgufDtype.Q4_1: QMM_DTYPE_Q4_1, GgufDtype.Q1_0: QMM_DTYPE_Q1_0,
          GgufDtype.Q2_0: QMM_DTYPE_Q2_0}


def qmm_dtype_id(dtype) -> int:
    """qmm_dtype_id (L101-116): the adapter's wire id of a GGUF dtype."""
    try:
        return _ID_OF.get(GgufDtype(int(dtype)), QMM_DTYPE_UNKNOWN)
    except ValueError:
        return QMM_DTYPE_UNKNOWN


def dtype_for_qmm_id(qmm_id: int) -> int:
    """The GGUF tag of an adapter dtype id (0: unknown), from the library."""
    return int(lib().rce_qmm_dtype_for_qmm_id(int(qmm_id)))


def qmm_1d_flops_bytes(n: int, k: int, weight_bytes: int) -> tuple[int, int]:
    """qmm_1d_flops_bytes (L141-145)."""
    return 2 * n * k, weight_bytes + 4 * k + 4 * n


@dataclass(frozen=True)
class LinearCoeffs:
    """rce-placement LinearCoeffs (L231-242): pJ = a*flops + b*bytes + c."""
    a_pj_per_flop: float
    b_pj_per_byte: float
    c_pj_overhead: float

    def estimate_pj(self, flops: int, bytes_: int) -> float:
        return self.a_pj_per_flop * flops + self.b_pj_per_byte * bytes_ + self.c_pj_overhead


def hip_cost_prior() -> LinearCoeffs:
    """The library's analytical prior for the ("qmm", "hip:op-qmm") cell."""
    a, b, c = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    lib().rce_qmm_hip_cost_prior(ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
    return LinearCoeffs(a.value, b.value, c.value)


@dataclass
class HostQuantWeight:
    """The reference's QuantWeight as the adapter hands it over: GGUF bytes
    in host memory, dtype, [n_rows, n_cols]."""
    data: np.ndarray
    dtype: int
    n_rows: int
    n_cols: int


class HipQmm:
    """PricedBackend + QmmDispatch for the MI355X (adapter L205-283's CpuQmm /
    MetalQmm shape).  ``coeffs`` is the cost cell (the caller's CostTable may
    calibrate it); the library's prior by default."""

    def __init__(self, ctx: Context, coeffs: LinearCoeffs | None = None):
        self.ctx = ctx
        self.coeffs = coeffs or hip_cost_prior()
        self._dev: dict = {}

    # ---- PricedBackend ----
    def id(self) -> str:
        return "hip:op-qmm"

    def handles(self) -> list:
        return ["qmm"]

    def cost(self, op: str, shapes) -> tuple[float, str]:
        """(picojoules, basis): +inf declines (pick_priced then picks CpuQmm)."""
        if op != "qmm" or len(shapes) < 2:
            return math.inf, "est"
        a_shape = np.asarray(shapes[0], np.uintp)
        w_shape = np.asarray(shapes[1], np.uintp)
        pj = ctypes.c_double()
        c = self.coeffs
        check(lib().rce_qmm_hip_cost(a_shape.ctypes.data_as(ctypes.c_void_p), a_shape.size,
                                     w_shape.ctypes.data_as(ctypes.c_void_p), w_shape.size,
                                     c.a_pj_per_flop, c.b_pj_per_byte, c.c_pj_overhead, ctypes.byref(pj)))
        return pj.value, "est"

    def execute(self, op, inputs):
        raise RuntimeError("HipQmm: qmm dispatch uses QmmDispatch::qmm_1d, not PricedBackend::execute")

    # ---- QmmDispatch ----
    def _device_weight(self, w: HostQuantWeight) -> QuantWeight:
        key = (w.data.ctypes.data, w.data.nbytes, int(w.dtype), w.n_rows, w.n_cols)
        dw = self._dev.get(key)
        if dw is None:
            dw = self._dev[key] = QuantWeight.from_owned_bytes(self.ctx, w.data, w.dtype, w.n_rows, w.n_cols)
        return dw

    def qmm_1d(self, a, w: HostQuantWeight) -> np.ndarray:
        """mm_1d on the GPU (EXACT: bit-identical to rce_op_qmm::mm_1d)."""
        return mm_1d(np.asarray(a, np.float32), self._device_weight(w))

    def close(self) -> None:
        for dw in self._dev.values():
            dw.close()
        self._dev.clear()


class GpuEnergyMeter:
    """EnergyMeter (adapter L48-74) over the GPU's energy counter
    (rce_qmm_energy_read), the MI355X counterpart of SubstrateEnergyMeter
    (substrate_meter.rs L60-130): start() snapshots the counter under a
    token, end(token) returns the picojoules since, basis "reported".
    The counter advances once a second on MI355X, so windows shorter than
    that read 0 (the reference's meter expects that of tiny dispatches).
    ``open`` returns None where no counter can be read."""

    def __init__(self, device: int):
        self.device = device
        self._windows: dict = {}
        self._next = 0

    @classmethod
    def open(cls, device: int = 0) -> "GpuEnergyMeter | None":
        m = cls(device)
        return m if m._read() is not None else None

    def _read(self):
        uj = ctypes.c_uint64()
        return uj.value if lib().rce_qmm_energy_read(self.device, ctypes.byref(uj), None) == 0 else None

    def basis(self) -> str:
        return "reported"

    def start(self):
        uj = self._read()
        if uj is None:
            return None
        self._next += 1
        self._windows[self._next] = uj
        return self._next

    def end(self, token):
        prior = self._windows.pop(token, None)
        now = self._read()
        if prior is None or now is None:
            return None
        return max(0, now - prior) * 1_000_000  # uJ -> pJ

    def windows_open(self) -> int:
        return len(self._windows)


def pick_priced(backends, op: str, shapes):
    """rce-vm-scheduler pick_priced (L98-115): the first backend with the
    strictly lowest cost among those that handle `op`; None if none does."""
    best = None
    for be in backends:
        if op not in be.handles():
            continue
        pj, basis = be.cost(op, shapes)
        if best is None or pj < best[1]:
            best = (be, pj, basis)
    return best
