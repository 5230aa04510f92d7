"""Pins the oracle's Q5_0 and Q4_1 rows (mm_1d_q5_0 / dot_row_q5_0 and
mm_1d_q4_1, rce-op-qmm/src/lib.rs L331-352, L525-561, L615-645), their
dequantizers (rce-ingest-gguf dequant.rs L385-433) and the Q8-activation
path over them.  The reference ships no quantizer for either format, so the
weights are random bytes (every bit pattern of qs/qh, scales of both signs).

Checks: an independent vectorized numpy decode (bit positions taken from
the GGUF block definitions: qs byte q holds positions q (low nibble) and
q + 16 (high nibble); Q5_0 qh bit j is the fifth bit of position j),
planted single bits, the reference's own synthetic Q5_0 case
(lib.rs L3750-3790, |mm - dequant-then-dot| < 1e-4), an f64 error bound
and closed-form integer dots for the Q8 path.  CPU only."""
import numpy as np
import pytest

import oracle as O
from rand_blocks import rand_blocks

F32 = np.float32
FMTS = [O.Q5_0, O.Q4_1]


def np_decode(b, dt, n, k):
    """(v int64 [n, k], d f32 [n, nb], m f32 [n, nb] or None): v = the 5-bit
    value - 16 (Q5_0) or the raw nibble (Q4_1)."""
    nb = k // 32
    bl = b.reshape(n, nb, O.BLOCK[dt][1])
    d = bl[:, :, 0:2].copy().view(np.float16)[:, :, 0].astype(F32)
    if dt == O.Q5_0:
        qh = bl[:, :, 2:6].copy().view("<u4")[:, :, 0].astype(np.int64)
        qs = bl[:, :, 6:22].astype(np.int64)
        pos = np.arange(32)
        nib = np.concatenate([qs & 0xF, qs >> 4], axis=2)              # positions 0..15, 16..31
        hib = (qh[:, :, None] >> pos[None, None, :]) & 1               # bit j -> position j
        return ((nib | (hib << 4)) - 16).reshape(n, k), d, None
    m = bl[:, :, 2:4].copy().view(np.float16)[:, :, 0].astype(F32)
    qs = bl[:, :, 4:20].astype(np.int64)
    return np.concatenate([qs & 0xF, qs >> 4], axis=2).reshape(n, k), d, m


def np_mm(a, b, dt, n, k):
    """The reference's fold orders, vectorized over rows."""
    v, d, m = np_decode(b, dt, n, k)
    vf = v.astype(F32)
    sumf = np.zeros(n, F32)
    for ib in range(k // 32):
        o = 32 * ib
        if dt == O.Q5_0:  # sub += v0 a[q]; sub += v1 a[q+16]; sumf += scale*sub
            sub = np.zeros(n, F32)
            for q in range(16):
                sub = sub + vf[:, o + q] * a[o + q]
                sub = sub + vf[:, o + q + 16] * a[o + q + 16]
            sumf = sumf + d[:, ib] * sub
        else:  # va += v0 alo + v1 ahi; asum += alo + ahi; sumf += scale*va + min*asum
            va = np.zeros(n, F32)
            asum = F32(0)
            for q in range(16):
                va = va + (vf[:, o + q] * a[o + q] + vf[:, o + q + 16] * a[o + q + 16])
                asum = F32(asum + F32(a[o + q] + a[o + q + 16]))
            sumf = sumf + (d[:, ib] * va + m[:, ib] * asum)
    return sumf


@pytest.mark.parametrize("dt", FMTS)
def test_dequant_equals_numpy_decode(dt):
    rng = np.random.default_rng(300 + dt)
    n, k = 6, 256
    b = rand_blocks(rng, dt, n, k)
    v, d, m = np_decode(b, dt, n, k)
    want = v.astype(F32) * np.repeat(d, 32, axis=1)
    if dt == O.Q4_1:
        want = want + np.repeat(m, 32, axis=1)
    got = O.dequantize(b, dt, n * k).reshape(n, k)
    assert np.array_equal(got.view(np.uint32), want.astype(F32).view(np.uint32))


@pytest.mark.parametrize("j", [0, 5, 15, 16, 22, 31])
def test_q5_0_planted_high_bit(j):
    # scale 1, qs all zero, only qh bit j set: position j is 16 - 16 = 0,
    # every other position 0 - 16.
    blk = np.zeros(22, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:6] = np.frombuffer(np.uint32(1 << j).tobytes(), np.uint8)
    want = np.full(32, -16.0, F32)
    want[j] = 0.0
    assert np.array_equal(O.dequantize(blk, O.Q5_0, 32), want)


@pytest.mark.parametrize("dt", FMTS)
@pytest.mark.parametrize("q", [0, 9, 15])
def test_planted_nibbles(dt, q):
    # qs byte q = 0x3A: low nibble 10 at position q, high nibble 3 at q + 16.
    bb = O.BLOCK[dt][1]
    blk = np.zeros(bb, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    off = 6 if dt == O.Q5_0 else 4
    blk[off + q] = 0x3A
    base = -16.0 if dt == O.Q5_0 else 0.0
    want = np.full(32, base, F32)
    want[q], want[q + 16] = base + 10, base + 3
    assert np.array_equal(O.dequantize(blk, dt, 32), want)


@pytest.mark.parametrize("dt", FMTS)
def test_mm_1d_equals_numpy_restatement(dt):
    rng = np.random.default_rng(310 + dt)
    n, k = 24, 512
    b = rand_blocks(rng, dt, n, k)
    a = rng.standard_normal(k).astype(F32)
    got = O.mm_1d(a, b, dt, n, k)
    assert np.array_equal(got.view(np.uint32), np_mm(a, b, dt, n, k).view(np.uint32))


def test_q5_0_reference_case():
    # rce-op-qmm lib.rs L3750-3790 mm_1d_q5_0_matches_dequant: k 64, n 3,
    # scale 0.0625 + r*0.01 + blk*0.003, qh = 0x13579BDF ^ (r << (blk & 7)),
    # qs byte q = ((r+blk+q) % 16) | ((r*2+q) % 16) << 4; a_i = cos(0.023 i - 0.4).
    k, n = 64, 3
    nbl = k // 32
    b = np.zeros((n, nbl, 22), np.uint8)
    for r in range(n):
        for blk in range(nbl):
            sc = F32(F32(0.0625) + F32(r) * F32(0.01)) + F32(blk) * F32(0.003)
            b[r, blk, 0:2] = np.frombuffer(np.float16(sc).tobytes(), np.uint8)
            qh = 0x13579BDF ^ ((r << (blk & 7)) & 0xFFFFFFFF)
            b[r, blk, 2:6] = np.frombuffer(np.uint32(qh).tobytes(), np.uint8)
            for q in range(16):
                b[r, blk, 6 + q] = ((r + blk + q) % 16) | (((r * 2 + q) % 16) << 4)
    b = b.reshape(-1)
    a = np.cos(np.arange(k, dtype=F32) * F32(0.023) - F32(0.4)).astype(F32)
    got = O.mm_1d(a, b, O.Q5_0, n, k)
    rb = O.row_bytes(O.Q5_0, k)
    for r in range(n):
        w = O.dequantize(b[r * rb:(r + 1) * rb], O.Q5_0, k)
        dot = F32(0)
        for i in range(k):
            dot = F32(dot + a[i] * w[i])
        assert abs(got[r] - dot) < 1e-4


@pytest.mark.parametrize("dt", FMTS)
def test_mm_1d_error_bound_against_f64(dt):
    rng = np.random.default_rng(320 + dt)
    n, k = 32, 1024
    b = rand_blocks(rng, dt, n, k)
    a = rng.standard_normal(k).astype(F32)
    got = O.mm_1d(a, b, dt, n, k).astype(np.float64)
    w = O.dequantize(b, dt, n * k).reshape(n, k).astype(np.float64)
    exact = w @ a.astype(np.float64)
    # Q4_1 splits each term into scale*v + min (two roundings per term of the
    # form plus the per-block products): bound the sum of |scale v a| + |min a|.
    v, d, m = np_decode(b, dt, n, k)
    mag = np.abs(v.astype(np.float64) * np.repeat(d, 32, axis=1).astype(np.float64))
    if m is not None:
        mag = mag + np.abs(np.repeat(m, 32, axis=1).astype(np.float64))
    bound = (k + 8) * 2.0 ** -24 * (mag @ np.abs(a.astype(np.float64)))
    assert np.all(np.abs(got - exact) <= bound)


@pytest.mark.parametrize("dt", FMTS)
def test_q8_path_closed_form(dt):
    # Integer block dots in int64, then the path's float steps.
    rng = np.random.default_rng(330 + dt)
    n, k = 20, 512
    b = rand_blocks(rng, dt, n, k)
    a = rng.standard_normal(k).astype(F32)
    got = O.mm_batched_q8(a, b, dt, n, k)[0]
    xq, dx, _ = O.quantize_act_q8(a)
    xq = xq.astype(np.int64)
    v, d, m = np_decode(b, dt, n, k)
    sumf = np.zeros(n, F32)
    for ib in range(k // 32):
        isum = (v[:, 32 * ib:32 * ib + 32] * xq[32 * ib:32 * ib + 32]).sum(axis=1)
        if dt == O.Q5_0:
            sub = (dx[ib] * isum.astype(F32)).astype(F32)
            sumf = sumf + d[:, ib] * sub
        else:
            xs = int(xq[32 * ib:32 * ib + 32].sum())
            va = (dx[ib] * isum.astype(F32)).astype(F32)
            asum = F32(dx[ib] * F32(xs))
            sumf = sumf + (d[:, ib] * va + m[:, ib] * asum)
    assert np.array_equal(got.view(np.uint32), sumf.view(np.uint32))


@pytest.mark.parametrize("dt", FMTS)
def test_batched_is_per_row(dt):
    rng = np.random.default_rng(340 + dt)
    n, k, t = 40, 256, 3
    b = rand_blocks(rng, dt, n, k)
    x = rng.standard_normal((t, k)).astype(F32)
    batched = O.mm_batched(x, b, dt, n, k, threads=4)
    for r in range(t):
        assert np.array_equal(batched[r].view(np.uint32), O.mm_1d(x[r], b, dt, n, k, threads=1).view(np.uint32))
