"""Pins the oracle's whole-element rows (mm_1d_f32 / mm_1d_f16 /
mm_1d_bf16, rce-op-qmm/src/lib.rs L458-490: acc += a[i] * w[i] over the
row, i ascending, from +0.0) and dequantizers (dequant.rs L343-356), and
that their Q8 mode is the same order (no activation quantization for
float weights).  CPU only."""
import numpy as np
import pytest

import oracle as O
from rand_blocks import float_bytes

F32 = np.float32
FMTS = [O.F32, O.F16, O.BF16]


def np_values(b, dt, n, k):
    """Independent decode: f32 as is, f16 by numpy's IEEE binary16, bf16 as
    the high half of an f32."""
    if dt == O.F32:
        return b.view(F32).reshape(n, k)
    u = b.view(np.uint16).reshape(n, k)
    if dt == O.F16:
        return u.view(np.float16).astype(F32)
    return (u.astype(np.uint32) << 16).view(F32)


@pytest.mark.parametrize("dt", FMTS)
def test_dequant_equals_numpy(dt):
    rng = np.random.default_rng(500 + dt)
    n, k = 4, 300
    b = float_bytes(rng, dt, n, k)
    got = O.dequantize(b, dt, n * k).reshape(n, k)
    assert np.array_equal(got.view(np.uint32), np_values(b, dt, n, k).view(np.uint32))


def test_bf16_known_answers():
    # 0x3F80 = 1.0, 0xC000 = -2.0, 0x7F80 = inf, 0x0001 = the smallest subnormal 2^-133
    b = np.array([0x3F80, 0xC000, 0x7F80, 0x0001], np.uint16).view(np.uint8)
    v = O.dequantize(b, O.BF16, 4)
    assert v[0] == 1.0 and v[1] == -2.0 and np.isinf(v[2]) and v[3] == np.float32(2.0 ** -133)


@pytest.mark.parametrize("dt", FMTS)
@pytest.mark.parametrize("k", [1, 7, 256, 1000])
def test_mm_1d_equals_sequential_numpy(dt, k):
    rng = np.random.default_rng(510 + dt + k)
    n = 9
    b = float_bytes(rng, dt, n, k)
    a = rng.standard_normal(k).astype(F32)
    w = np_values(b, dt, n, k)
    acc = np.zeros(n, F32)
    for i in range(k):
        acc = acc + a[i] * w[:, i]
    got = O.mm_1d(a, b, dt, n, k)
    assert np.array_equal(got.view(np.uint32), acc.view(np.uint32))


@pytest.mark.parametrize("dt", FMTS)
def test_mm_1d_error_bound_against_f64(dt):
    rng = np.random.default_rng(520 + dt)
    n, k = 16, 2048
    b = float_bytes(rng, dt, n, k)
    a = rng.standard_normal(k).astype(F32)
    w = np_values(b, dt, n, k).astype(np.float64)
    got = O.mm_1d(a, b, dt, n, k).astype(np.float64)
    exact = w @ a.astype(np.float64)
    bound = (k + 1) * 2.0 ** -24 * (np.abs(w) @ np.abs(a.astype(np.float64)))
    assert np.all(np.abs(got - exact) <= bound)


@pytest.mark.parametrize("dt", FMTS)
def test_q8_mode_is_the_reference_order(dt):
    rng = np.random.default_rng(530 + dt)
    n, k, t = 11, 200, 3
    b = float_bytes(rng, dt, n, k)
    x = rng.standard_normal((t, k)).astype(F32)
    assert np.array_equal(O.mm_batched_q8(x, b, dt, n, k).view(np.uint32),
                          O.mm_batched(x, b, dt, n, k).view(np.uint32))
