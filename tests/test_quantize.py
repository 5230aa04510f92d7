"""The library's GGUF quantizer (rce_qmm_quantize, host only) produces the
same bytes as the oracle's restatement of the reference's encoders
(nn.rs L541-563 quantize_block, toy_gpt2.rs L46-58, kquant.rs L193-346),
which test_oracle_formats.py pins to the reference's known answers."""
import numpy as np
import pytest

import oracle as O
import rce_amd

F32 = np.float32


@pytest.mark.parametrize("dt,k", [(O.Q8_0, 4096), (O.Q4_0, 4096), (O.Q4_K, 2048), (O.Q5_K, 2048), (O.Q6_K, 2048),
                                  (O.Q4_0, 32), (O.Q4_K, 256), (O.Q5_K, 256)])
def test_quantize_matches_oracle(dt, k):
    rng = np.random.default_rng(dt * 1000 + k)
    for n, sigma in ((1, 1.0), (37, 0.02), (200, 3.0)):
        w = (rng.standard_normal((n, k)) * sigma).astype(F32)
        assert np.array_equal(rce_amd.quantize(w, dt), O.quantize(w, dt)), (dt, k, n, sigma)


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4_0, O.Q4_K, O.Q5_K, O.Q6_K])
def test_quantize_edge_blocks(dt):
    """Zero blocks (d = 0 branches), constant blocks, the reference's known
    answer input x = i - 16 (nn.rs L751-765), ties and large magnitudes."""
    k = 256
    rows = [np.zeros(k), np.full(k, 0.75), np.tile(np.arange(32) - 16.0, k // 32),
            np.tile(np.arange(32) * 0.5 - 8.0, k // 32), np.linspace(-6e4, 6e4, k),
            np.where(np.arange(k) % 2, 1.0, -1.0) * 1e-6]
    w = np.stack(rows).astype(F32)
    assert np.array_equal(rce_amd.quantize(w, dt), O.quantize(w, dt))


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4_0, O.Q4_K, O.Q5_K, O.Q6_K])
def test_quantize_nonfinite_blocks_match_oracle(dt):
    """Blocks holding +-inf, NaN, subnormal maxima (1/d overflows) and huge
    values: the library writes the oracle's bytes (the reference's
    saturating casts, wrapping adds and f16_bits; the known answers are in
    test_oracle_formats.py)."""
    rng = np.random.default_rng(40 + dt)
    k, n = 256, 64
    w = (rng.standard_normal((n, k)) * 0.02).astype(F32)
    specials = np.array([np.inf, -np.inf, np.nan, 2.0 ** -130, -(2.0 ** -131), 1e-45, 3e38, -3e38, 7e4], F32)
    for r in range(n):
        m = rng.random(k) < (0.02 + 0.3 * (r % 4 == 0))
        w[r, m] = rng.choice(specials, int(m.sum()))
        if r % 8 == 1:
            w[r] = w[r] * F32(1e-38)  # subnormal blocks
    with np.errstate(all="ignore"):
        assert np.array_equal(rce_amd.quantize(w, dt), O.quantize(w, dt))


def test_quantize_threaded_rows_identical():
    """Large inputs are split over threads by row ranges; the bytes equal a
    row-by-row quantization."""
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((512, 4096)) * 0.02).astype(F32)
    whole = rce_amd.quantize(w, O.Q4_K)
    rb = rce_amd.row_bytes(O.Q4_K, 4096)
    for r in (0, 1, 255, 511):
        assert np.array_equal(whole[r * rb:(r + 1) * rb], rce_amd.quantize(w[r:r + 1], O.Q4_K))


def test_quantize_errors():
    with pytest.raises(rce_amd.QmmError):
        rce_amd.quantize(np.zeros((1, 100), F32), O.Q4_0)  # not a block multiple
    with pytest.raises(rce_amd.QmmError):
        rce_amd.quantize(np.zeros((1, 256), F32), O.Q3_K)  # no encoder
