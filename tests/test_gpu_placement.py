"""HipQmm's dispatch half (QmmDispatch::qmm_1d) on the GPU: bit-identical to
the reference's mm_1d (the oracle), one upload per distinct weight buffer,
and the adapter's flow -- pick_priced, then the winner's qmm_1d -- running
the large shape here (rce-placement-adapter L420-470)."""
import numpy as np
import pytest

import oracle as O
import rce_amd.placement as P
from rce_amd import GgufDtype as G

pytestmark = pytest.mark.gpu


def test_qmm_1d_bit_identical_and_cached(ctx):
    print("HipQmm.qmm_1d Q4_0 11008x4096", flush=True)
    rng = np.random.default_rng(90)
    n, k = 11008, 4096
    import rce_amd
    b = rce_amd.quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32), G.Q4_0)
    w = P.HostQuantWeight(b, G.Q4_0, n, k)
    hip = P.HipQmm(ctx)
    shapes = [[k], [n, k, b.size, P.qmm_dtype_id(G.Q4_0)]]
    be, _, _ = P.pick_priced([hip], "qmm", shapes)
    assert be is hip
    for seed in (1, 2):
        a = np.random.default_rng(seed).standard_normal(k).astype(np.float32)
        got = be.qmm_1d(a, w)
        assert np.array_equal(got.view(np.uint32), O.mm_1d(a, b, O.Q4_0, n, k).view(np.uint32))
    assert len(hip._dev) == 1  # uploaded once, reused
    hip.close()


def test_gpu_energy_meter_brackets_dispatches(ctx):
    """EnergyMeter over the GPU's counter (the adapter's calibration input,
    L48-74): a window of dispatches spanning more than the counter's 1 s
    update period reads a power between 50 W and 2 kW; an unknown token
    reads None; windows close.  Skipped where the box exposes no counter
    (ROCm SMI absent or not permitted)."""
    print("GPU energy meter", flush=True)
    meter = P.GpuEnergyMeter.open(0)
    if meter is None:
        import rce_amd
        pytest.skip(f"no GPU energy counter here: {rce_amd._lib.lib().rce_qmm_last_error().decode()}")
    import rce_amd
    rng = np.random.default_rng(91)
    n, k = 11008, 4096
    b = rce_amd.quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32), G.Q4_0)
    hip = P.HipQmm(ctx)
    w = P.HostQuantWeight(b, G.Q4_0, n, k)
    a = rng.standard_normal(k).astype(np.float32)
    import time
    tok = meter.start()
    t0 = time.perf_counter()
    calls = 0
    while time.perf_counter() - t0 < 2.5:  # more than two counter updates
        hip.qmm_1d(a, w)
        calls += 1
    pj = meter.end(tok)
    watts = pj / 1e12 / (time.perf_counter() - t0)
    print(f"  {calls} host-entry GEMVs: {pj / 1e12:.1f} J, {watts:.0f} W", flush=True)
    assert pj is not None and meter.basis() == "reported"
    assert 50.0 < watts < 2000.0
    assert meter.end(12345) is None and meter.windows_open() == 0
    hip.close()
