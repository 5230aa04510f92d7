"""Pins the oracle's Q3_K row (mm_1d_q3_k, rce-op-qmm/src/lib.rs
L840-928), its dequantizer (dequant.rs L460-543) and the Q8-activation path
over it.  The reference ships no Q3_K quantizer, so weights are random
super-blocks (every bit pattern of hmask, qs and the packed scales).

The super-block definition (llama.cpp's block_q3_K, restated in the
reference's comments): [hmask 32 B][qs 64 B][scales 12 B][d f16]; value p =
128 o + 32 j + 16 h + l (o < 2, j < 4, h < 2, l < 16) has low bits
(qs[32 o + 16 h + l] >> 2 j) & 3 and high bit (hmask[16 h + l] >> (4 o + j)) & 1
(set: +0, clear: -4); its scale is sixteen-group 2 (4 o + j) + h, a 6-bit
number whose low 4 bits are nibble (g // 8) of byte g % 8 and whose high
2 bits are bits 2 (g // 4) of byte 8 + g % 4, minus 32.

Checks: an independent numpy decode written from that definition (bit
for bit against dequantize), planted single bits and scales, an
independent numpy fold in the reference's order, the reference's own
dequant-then-dot case (in test_oracle_products), an f64 bound, and
closed-form integer dots for the Q8 path.  CPU only."""
import numpy as np
import pytest

import oracle as O
from rand_blocks import rand_blocks

F32 = np.float32


def np_scales(sb12):
    """[..., 12] packed bytes -> [..., 16] signed scales (6-bit minus 32)."""
    g = np.arange(16)
    lo = np.where(g < 8, sb12[..., g % 8] & 0xF, sb12[..., g % 8] >> 4).astype(np.int64)
    hi = (sb12[..., 8 + g % 4].astype(np.int64) >> (2 * (g // 4))) & 3
    return (lo | (hi << 4)) - 32


def np_decode(b, n, k):
    """(v int64 [n, k] in -4..3, scale index per value, sc int64 [n, nsb, 16], d f32 [n, nsb])."""
    nsb = k // 256
    bl = b.reshape(n, nsb, 110).astype(np.int64)
    hmask, qs = bl[..., 0:32], bl[..., 32:96]
    sc = np_scales(bl[..., 96:108].astype(np.uint8))
    d = bl[..., 108:110].astype(np.uint8).copy().view(np.float16)[..., 0].astype(F32)
    p = np.arange(256)
    o, j, h, l = p // 128, (p % 128) // 32, (p % 32) // 16, p % 16
    low = (qs[..., 32 * o + 16 * h + l] >> (2 * j)) & 3
    high = (hmask[..., 16 * h + l] >> (4 * o + j)) & 1
    v = low - 4 * (1 - high)
    gidx = 2 * (4 * o + j) + h
    return v.reshape(n, k), gidx, sc, d


def test_dequant_equals_numpy_decode():
    rng = np.random.default_rng(400)
    n, k = 5, 512
    b = rand_blocks(rng, O.Q3_K, n, k)
    v, gidx, sc, d = np_decode(b, n, k)
    dl = (d[..., None] * sc.astype(F32)).astype(F32)           # [n, nsb, 16] = d * (sc - 32)
    want = (dl[..., gidx] * v.reshape(n, k // 256, 256).astype(F32)).reshape(n, k)
    got = O.dequantize(b, O.Q3_K, n * k).reshape(n, k)
    assert np.array_equal(got.view(np.uint32), want.astype(F32).view(np.uint32))


def _block(scales16=None, d=1.0):
    blk = np.zeros(110, np.uint8)
    blk[108:110] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    s = np.full(16, 33) if scales16 is None else np.asarray(scales16) + 32   # stored 6-bit values
    for g in range(16):  # pack per the definition in the module docstring
        blk[96 + g % 8] |= (s[g] & 0xF) << (4 * (g // 8))
        blk[104 + g % 4] |= (s[g] >> 4) << (2 * (g // 4))
    return blk


@pytest.mark.parametrize("g", [0, 3, 7, 8, 11, 15])
def test_planted_scale(g):
    # every scale 1 except group g = -29: values all -4 (no high bits)
    sc = np.ones(16, np.int64)
    sc[g] = -29
    v = O.dequantize(_block(sc), O.Q3_K, 256)
    want = np.full(256, -4.0, F32)
    want[16 * g:16 * g + 16] = 116.0
    assert np.array_equal(v, want)


@pytest.mark.parametrize("o,j,h,l", [(0, 0, 0, 0), (0, 3, 1, 15), (1, 0, 0, 7), (1, 2, 1, 4), (1, 3, 0, 9)])
def test_planted_bits(o, j, h, l):
    # scale 1 everywhere; one high bit and low bits 3 at (o, j, h, l): that
    # value is 3, every other -4.
    blk = _block()
    blk[16 * h + l] |= 1 << (4 * o + j)
    blk[32 + 32 * o + 16 * h + l] |= 3 << (2 * j)
    want = np.full(256, -4.0, F32)
    want[128 * o + 32 * j + 16 * h + l] = 3.0
    assert np.array_equal(O.dequantize(blk, O.Q3_K, 256), want)


def np_mm(a, b, n, k):
    """lib.rs L890-925 order: per (o, j), s1 and s2 over l ascending, then
    sumf += dl1 * s1 + dl2 * s2."""
    v, gidx, sc, d = np_decode(b, n, k)
    vf = v.astype(F32)
    sumf = np.zeros(n, F32)
    for s in range(k // 256):
        for o in range(2):
            for j in range(4):
                base = 256 * s + 128 * o + 32 * j
                s1 = np.zeros(n, F32)
                s2 = np.zeros(n, F32)
                for l in range(16):
                    s1 = s1 + vf[:, base + l] * a[base + l]
                    s2 = s2 + vf[:, base + 16 + l] * a[base + 16 + l]
                dl1 = (d[:, s] * sc[:, s, 2 * (4 * o + j)].astype(F32)).astype(F32)
                dl2 = (d[:, s] * sc[:, s, 2 * (4 * o + j) + 1].astype(F32)).astype(F32)
                sumf = sumf + (dl1 * s1 + dl2 * s2)
    return sumf


def test_mm_1d_equals_numpy_restatement():
    rng = np.random.default_rng(410)
    n, k = 16, 512
    b = rand_blocks(rng, O.Q3_K, n, k)
    a = rng.standard_normal(k).astype(F32)
    got = O.mm_1d(a, b, O.Q3_K, n, k)
    assert np.array_equal(got.view(np.uint32), np_mm(a, b, n, k).view(np.uint32))


def test_mm_1d_error_bound_against_f64():
    rng = np.random.default_rng(420)
    n, k = 24, 1024
    b = rand_blocks(rng, O.Q3_K, n, k)
    a = rng.standard_normal(k).astype(F32)
    got = O.mm_1d(a, b, O.Q3_K, n, k).astype(np.float64)
    w = O.dequantize(b, O.Q3_K, n * k).reshape(n, k).astype(np.float64)
    exact = w @ a.astype(np.float64)
    bound = (k + 8) * 2.0 ** -24 * (np.abs(w) @ np.abs(a.astype(np.float64)))
    assert np.all(np.abs(got - exact) <= bound)


def test_q8_path_closed_form():
    rng = np.random.default_rng(430)
    n, k = 12, 512
    b = rand_blocks(rng, O.Q3_K, n, k)
    a = rng.standard_normal(k).astype(F32)
    got = O.mm_batched_q8(a, b, O.Q3_K, n, k)[0]
    xq, dx, _ = O.quantize_act_q8(a)
    xq = xq.astype(np.int64)
    v, gidx, sc, d = np_decode(b, n, k)
    sumf = np.zeros(n, F32)
    for blk in range(k // 32):  # block blk = (super-block, o, j)
        s, u = divmod(blk, 8)
        base = 32 * blk
        i1 = (v[:, base:base + 16] * xq[base:base + 16]).sum(axis=1)
        i2 = (v[:, base + 16:base + 32] * xq[base + 16:base + 32]).sum(axis=1)
        dl1 = (d[:, s] * sc[:, s, 2 * u].astype(F32)).astype(F32)
        dl2 = (d[:, s] * sc[:, s, 2 * u + 1].astype(F32)).astype(F32)
        s1 = (dx[blk] * i1.astype(F32)).astype(F32)
        s2 = (dx[blk] * i2.astype(F32)).astype(F32)
        sumf = sumf + (dl1 * s1 + dl2 * s2)
    assert np.array_equal(got.view(np.uint32), sumf.view(np.uint32))


def test_batched_is_per_row():
    rng = np.random.default_rng(440)
    n, k, t = 30, 512, 3
    b = rand_blocks(rng, O.Q3_K, n, k)
    x = rng.standard_normal((t, k)).astype(F32)
    batched = O.mm_batched(x, b, O.Q3_K, n, k, threads=4)
    for r in range(t):
        assert np.array_equal(batched[r].view(np.uint32), O.mm_1d(x[r], b, O.Q3_K, n, k, threads=1).view(np.uint32))
