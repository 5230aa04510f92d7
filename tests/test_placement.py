"""The "hip:op-qmm" priced backend's cost side (rce_amd.placement over
rce_qmm_hip_cost / rce_qmm_dtype_for_qmm_id / rce_qmm_hip_cost_prior),
against rce-placement-adapter's own rules (src/lib.rs): the dtype id table
(L80-116), qmm_1d_flops_bytes (L141-145), the cost = +inf decline that
routes a format a backend lacks to CpuQmm (L253-266), and pick_priced's
choice between the reference's CPU prior (default_qmm_cost_table
L163-182) and this backend.  Host only: cost needs no GPU."""
import math

import pytest

import rce_amd.placement as P
from rce_amd import GgufDtype as G

CPU_PRIOR = P.LinearCoeffs(10.0, 0.05, 500_000.0)  # cpu:op-qmm (adapter L170-175)


class CpuQmmCost:
    """CpuQmm's cost (adapter L214-226): the generalist, never declines."""

    def id(self):
        return "cpu:op-qmm"

    def handles(self):
        return ["qmm"]

    def cost(self, op, shapes):
        if op != "qmm" or len(shapes) < 2:
            return math.inf, "est"
        k, n = shapes[0][0], shapes[1][0]
        wb = shapes[1][2] if len(shapes[1]) > 2 else 0
        return CPU_PRIOR.estimate_pj(*P.qmm_1d_flops_bytes(n, k, wb)), "est"


def shapes_of(dt, n, k):
    import rce_amd
    return [[k], [n, k, n * rce_amd.row_bytes(dt, k), P.qmm_dtype_id(dt)]]


def test_dtype_id_table():
    # QMM_DTYPE_* (L80-90) and qmm_dtype_id (L101-116)
    want = {G.Q8_0: 1, G.Q4K: 2, G.Q5K: 3, G.Q6K: 4, G.Q4_0: 5, G.Q5_0: 6, G.Q4_1: 7, G.Q1_0: 8, G.Q2_0: 9,
            G.Q3K: 10}
    for dt, i in want.items():
        assert P.qmm_dtype_id(dt) == i
        assert P.dtype_for_qmm_id(i) == int(dt)
    for dt in (G.F32, G.F16, G.BF16, G.I2S, G.STQ1_0, G.Q2K, 99):
        assert P.qmm_dtype_id(dt) == P.QMM_DTYPE_UNKNOWN
    assert P.dtype_for_qmm_id(0) == 0 and P.dtype_for_qmm_id(11) == 0 and P.dtype_for_qmm_id(1 << 40) == 0


def test_cost_formula_known_answer():
    hip = P.HipQmm(None, P.LinearCoeffs(1.0, 2.0, 3.0))
    n, k, wb = 11008, 4096, 25_362_432
    pj, basis = hip.cost("qmm", [[k], [n, k, wb, P.QMM_DTYPE_Q4_0]])
    assert pj == 2 * n * k + 2.0 * (wb + 4 * k + 4 * n) + 3.0 and basis == "est"


@pytest.mark.parametrize("op,shapes", [
    ("matmul", [[4096], [4096, 4096, 1, 5]]),          # another op
    ("qmm", [[4096]]),                                  # too few shapes
    ("qmm", [[4096], [4096, 4096, 1]]),                 # no dtype id: unknown
    ("qmm", [[4096], [4096, 4096, 1, 0]]),              # QMM_DTYPE_UNKNOWN
    ("qmm", [[4096 + 32], [4096, 4096 + 32, 1, 2]]),    # Q4_K with K not a multiple of 256
    ("qmm", [[4096], [4096, 4096, 1, 11]]),             # an id past the table
])
def test_declines(op, shapes):
    assert P.HipQmm(None).cost(op, shapes)[0] == math.inf


def test_prior_is_on_the_reference_scale():
    c = P.hip_cost_prior()
    assert (c.a_pj_per_flop, c.b_pj_per_byte, c.c_pj_overhead) == (10.0 / 9.0, 0.05, 5e5 * 42)
    # crossover with the CPU prior near 2.3 MFLOP (a 1024 x 1024 GEMV is 2.1)
    f = (c.c_pj_overhead - CPU_PRIOR.c_pj_overhead) / (CPU_PRIOR.a_pj_per_flop - c.a_pj_per_flop)
    assert 2.2e6 < f < 2.4e6


@pytest.mark.parametrize("dt,n,k,want", [
    (G.Q8_0, 64, 64, "cpu:op-qmm"),          # tiny: the per-call overhead decides
    (G.Q4_0, 512, 1024, "cpu:op-qmm"),
    (G.Q4_0, 11008, 4096, "hip:op-qmm"),     # configs[1]
    (G.Q4K, 4096, 4096, "hip:op-qmm"),
    (G.Q3K, 2048, 2048, "hip:op-qmm"),
    (G.F16, 4096, 4096, "cpu:op-qmm"),       # no adapter id for F16: declined
    (G.Q4K, 4096, 4096 + 32, "cpu:op-qmm"),  # no kernel for the shape: declined
])
def test_pick_priced_routes_by_shape_and_format(dt, n, k, want):
    # hybrid_routes_small_to_cpu_large_to_metal (adapter L745-787), with HipQmm
    be, pj, basis = P.pick_priced([CpuQmmCost(), P.HipQmm(None)], "qmm", shapes_of(dt, n, k))
    assert be.id() == want and basis == "est" and math.isfinite(pj)


def test_execute_is_not_the_dispatch_path():
    with pytest.raises(RuntimeError):
        P.HipQmm(None).execute("qmm", [])
