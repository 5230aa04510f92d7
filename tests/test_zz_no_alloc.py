"""rce_qmm_mm_batched_dev_noalloc through the C ABI: the same bits as
rce_qmm_mm_batched_dev on two calls in a row (the second smaller, so it runs
on what the first left in the shared fixed scratch), in every mode that uses
scratch, and a clear error for a call whose scratch exceeds the fixed array."""
import sys

import numpy as np
import pytest

import oracle as O
import rce_amd
from rce_amd import GgufDtype as G, Mode

pytestmark = pytest.mark.gpu
F32 = np.float32


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run_pair(ctx, qw, a, a_dtype, t, n, mode):
    """Outputs of the allocating and the no-allocation entry points for the
    first t rows of a (device-resident), each into a NaN-filled buffer."""
    xa = rce_amd.DeviceBuffer.from_numpy(ctx, a)
    nan = np.full(t * n, np.nan, F32)
    o1 = rce_amd.DeviceBuffer.from_numpy(ctx, nan)
    o2 = rce_amd.DeviceBuffer.from_numpy(ctx, nan)
    rce_amd.mm_batched_dev(ctx, xa.ptr, a_dtype, t, qw, o1.ptr, mode)
    rce_amd.mm_batched_dev_noalloc(ctx, xa.ptr, a_dtype, t, qw, o2.ptr, mode)
    ctx.synchronize()
    want = o1.download(F32, t * n)
    got = o2.download(F32, t * n)
    xa.free(); o1.free(); o2.free()
    return want, got


CASES = [
    # (dtype, n_rows, n_cols, activation dtype, mode, first t, second t): the
    # scratch each uses -- Q8 with several tokens: the quantized activations;
    # F16 activations in EXACT / Q8: the widened f32 copy; F16_MFMA with F32
    # activations: the f16 copy.
    (O.Q4_0, 2048, 4096, G.F32, Mode.Q8, 8, 3),
    (O.Q4_K, 1024, 4096, G.F16, Mode.Q8, 6, 2),
    (O.Q8_0, 512, 2048, G.F16, Mode.EXACT, 4, 1),
    (O.Q4_K, 1024, 4096, G.F32, Mode.F16_MFMA, 128, 32),
    (O.Q4_0, 512, 4096, G.F32, Mode.F16_MFMA, 64, 16),
]


@pytest.mark.parametrize("dt,n,k,adt,mode,t1,t2", CASES)
def test_noalloc_equals_allocating_entry(ctx, dt, n, k, adt, mode, t1, t2):
    note(f"noalloc case dtype={dt} {n}x{k} a={adt.name} mode={mode.name} t={t1},{t2}")
    rng = np.random.default_rng(0xA110C + dt + t1)
    w = (rng.standard_normal((n, k)) * 0.02).astype(F32)
    qw = rce_amd.QuantWeight.from_owned_bytes(ctx, O.quantize(w, dt), dt, n, k)
    for t in (t1, t2):
        a = rng.standard_normal((t, k)).astype(F32)
        if adt == G.F16:
            a = a.astype(np.float16)
        want, got = run_pair(ctx, qw, a, adt, t, n, mode)
        assert not np.isnan(want).any()
        assert np.array_equal(want.view(np.uint32), got.view(np.uint32)), f"t={t}: differs from mm_batched_dev"
    qw.close()


def test_noalloc_rejects_scratch_beyond_the_fixed_array(ctx):
    # F16_MFMA with F32 activations needs 2 * t * k bytes for the f16 copy:
    # 4096 x 4096 is 32 MiB, twice the fixed array.  The call is refused
    # before any launch.
    n, k, t = 256, 4096, 4096
    assert 2 * t * k > rce_amd.NOALLOC_SCRATCH_BYTES
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((n, k)) * 0.02).astype(F32)
    qw = rce_amd.QuantWeight.from_owned_bytes(ctx, O.quantize(w, O.Q4_K), O.Q4_K, n, k)
    xa = rce_amd.DeviceBuffer(ctx, 4 * t * k)
    out = rce_amd.DeviceBuffer(ctx, 4 * t * n)
    with pytest.raises(rce_amd.QmmError) as e:
        rce_amd.mm_batched_dev_noalloc(ctx, xa.ptr, G.F32, t, qw, out.ptr, Mode.F16_MFMA)
    assert e.value.status == 2 and "scratch" in str(e.value)
    # an empty call is fine and touches nothing
    rce_amd.mm_batched_dev_noalloc(ctx, xa.ptr, G.F32, 0, qw, out.ptr, Mode.Q8)
    ctx.synchronize()
    xa.free(); out.free(); qw.close()
