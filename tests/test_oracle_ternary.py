"""Pins the oracle's multiply-free formats: Q1_0 and Q2_0 (PrismML, blocks
of 128), STQ1_0 (Tencent, super-blocks of 256 through a 32-entry
codebook) and I2_S (BitNet b1.58: 2-bit codes, one f32 scale per tensor)
-- rows of mm_1d (rce-op-qmm/src/lib.rs L1478-1537, L1716-1875), their
dequantizers (dequant.rs L141-340) and tensor sizes.

Checks: the reference's own round-trip known answers (dequant.rs
t1_i2_s, t41_q1_0, t42_q2_0, t42_stq1_0: positions and values bit for
bit), the codebook's defining properties, the reference's
kernel-versus-dequant-dot tests (lib.rs L3008-3065, L3294-3470, their
tolerances), an independent numpy fold in the reference's order over
random codes, an f64 bound, and the Q8 mode being the reference order.
CPU only."""
import numpy as np
import pytest

import oracle as O
from rand_blocks import rand_ternary

F32 = np.float32
FMTS = [O.Q1_0, O.Q2_0, O.STQ1_0, O.I2_S]
CB = np.array([0xA9, 0x89, 0x29, 0x09, 0xA6, 0x86, 0x26, 0x06, 0x9A, 0x92, 0x1A, 0x12, 0x6A, 0x62, 0x4A, 0x42,
               0x01, 0x21, 0x81, 0xA1, 0x04, 0x24, 0x84, 0xA4, 0x10, 0x18, 0x90, 0x98, 0x40, 0x48, 0x60, 0x68])


def lanes(qp):
    return [((int(qp) >> (2 * p)) & 3) - 1 for p in range(4)]


def test_codebook_properties():
    # dequant.rs L141-161: every group is one zero and three +-1 lanes; the
    # 16 sign-0 entries are exactly the patterns whose first non-zero lane
    # is +1; entry 16 + i is entry i with its non-zero lanes negated.
    assert [int(lib_cb) for lib_cb in (O.lib().orc_stq1_0_codebook(i) for i in range(32))] == CB.tolist()
    pats = set()
    for i in range(16):
        v = lanes(CB[i])
        assert sorted(x == 0 for x in v) == [False, False, False, True]
        assert all(x in (-1, 0, 1) for x in v)
        assert [x for x in v if x][0] == 1
        pats.add(tuple(v))
        assert lanes(CB[16 + i]) == [-x for x in v]
    assert len(pats) == 16


def test_q1_0_roundtrip_known_answer():
    # dequant.rs L910-953: n 256, d 0.0625, sign + iff (i*5 + 1) % 2 == 0, bit 1 = +.
    n = 256
    want = np.array([1 if (i * 5 + 1) % 2 == 0 else -1 for i in range(n)])
    b = np.zeros((2, 18), np.uint8)
    for i in range(2):
        b[i, 0:2] = np.frombuffer(np.float16(0.0625).tobytes(), np.uint8)
        for j in range(128):
            if want[i * 128 + j] >= 0:
                b[i, 2 + j // 8] |= 1 << (j % 8)
    got = O.dequantize(b.reshape(-1), O.Q1_0, n)
    assert np.array_equal(got, (F32(0.0625) * want).astype(F32))
    assert O.tensor_byte_size(O.Q1_0, n) == 36


def test_q2_0_roundtrip_known_answer():
    # dequant.rs L956-998: d 0.125, q = (i % 4) - 1 covers all four codes.
    n = 256
    want = np.arange(n) % 4 - 1
    b = np.zeros((2, 34), np.uint8)
    for i in range(2):
        b[i, 0:2] = np.frombuffer(np.float16(0.125).tobytes(), np.uint8)
        for j in range(128):
            b[i, 2 + j // 4] |= (want[i * 128 + j] + 1) << ((j % 4) * 2)
    got = O.dequantize(b.reshape(-1), O.Q2_0, n)
    assert np.array_equal(got, (F32(0.125) * want).astype(F32))
    assert O.tensor_byte_size(O.Q2_0, n) == 68


def test_i2_s_roundtrip_known_answer():
    # dequant.rs L768-842: 256 values (i*31 + 7) % 3 -> 0, +1, -1; codes
    # -1 -> 00, 0 -> 01, +1 -> 10; scale 0.0625 after the codes, then 28
    # bytes of 0xAB padding that must be ignored.
    n = 256
    want = np.array([{0: 0, 1: 1, 2: -1}[(i * 31 + 7) % 3] for i in range(n)])
    code = {-1: 0, 0: 1, 1: 2}
    b = np.full(n // 4 + 32, 0xAB, np.uint8)
    for blk in range(2):
        for gp in range(32):
            c = [code[int(want[blk * 128 + 32 * s + gp])] for s in range(4)]
            b[blk * 32 + gp] = (c[0] << 6) | (c[1] << 4) | (c[2] << 2) | c[3]
    b[n // 4:n // 4 + 4] = np.frombuffer(np.float32(0.0625).tobytes(), np.uint8)
    got = O.dequantize(b, O.I2_S, n)
    assert np.array_equal(got.view(np.uint32), (F32(0.0625) * want.astype(F32)).view(np.uint32))
    assert O.tensor_byte_size(O.I2_S, n) == n // 4 + 4


def stq1_pack(nb, d):
    """dequant.rs L1107-1140: group g of block i takes codebook index
    (g + i) * 7 + 1 mod 32 (sign = bit 4, slot = low 4 bits)."""
    b = np.zeros((nb, 42), np.uint8)
    idx = np.zeros((nb, 64), np.int64)
    for i in range(nb):
        for g in range(64):
            ix = ((g + i) * 7 + 1) % 32
            idx[i, g] = ix
            b[i, g // 2] |= (ix & 0xF) << (4 * (g & 1))
            if ix >> 4:
                b[i, 32 + g // 8] |= 1 << (g % 8)
        b[i, 40:42] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    return b.reshape(-1), idx


def test_stq1_0_roundtrip_known_answer():
    b, idx = stq1_pack(2, 0.0625)
    got = O.dequantize(b, O.STQ1_0, 512).reshape(2, 64, 4)
    for i in range(2):
        for g in range(64):
            assert [float(x) for x in got[i, g]] == [0.0625 * q for q in lanes(CB[idx[i, g]])]
    assert O.tensor_byte_size(O.STQ1_0, 512) == 84


def _naive(a, w):
    acc = F32(0)
    for i in range(a.size):
        acc = F32(acc + a[i] * w[i])
    return acc


@pytest.mark.parametrize("dt,k,n,d", [(O.Q1_0, 256, 3, 0.0625), (O.Q2_0, 256, 3, 0.125), (O.STQ1_0, 512, 3, 0.0625)])
def test_kernel_matches_dequant_dot(dt, k, n, d):
    # lib.rs L3294-3470: |mm - dequant-then-dot| <= 1e-4 max(|dot|, 1).
    if dt == O.Q1_0:  # sign + iff (i*7 + 3) % 2 == 0, a_i = sin(0.011 i - 0.3)
        b = np.zeros((n * 2, 18), np.uint8)
        for r in range(n * 2):
            b[r, 0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
            for j in range(128):
                if (((r * 128 + j) * 7 + 3) % 2) == 0:
                    b[r, 2 + j // 8] |= 1 << (j % 8)
        a = np.sin(np.arange(k, dtype=F32) * F32(0.011) - F32(0.3)).astype(F32)
    elif dt == O.Q2_0:  # q = (i % 4) - 1, a_i = sin(0.013 i - 0.4)
        b = np.zeros((n * 2, 34), np.uint8)
        for r in range(n * 2):
            b[r, 0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
            for j in range(128):
                b[r, 2 + j // 4] |= ((r * 128 + j) % 4) << ((j % 4) * 2)
        a = np.sin(np.arange(k, dtype=F32) * F32(0.013) - F32(0.4)).astype(F32)
    else:
        b, _ = stq1_pack(n * 2, d)
        a = np.sin(np.arange(k, dtype=F32) * F32(0.017) - F32(0.5)).astype(F32)
    b = b.reshape(-1)
    got = O.mm_1d(a, b, dt, n, k)
    rb = O.row_bytes(dt, k)
    for j in range(n):
        dot = _naive(a, O.dequantize(b[j * rb:(j + 1) * rb], dt, k))
        assert abs(got[j] - dot) <= 1e-4 * max(abs(dot), 1.0)


def test_i2_s_kernel_matches_dequant_dot():
    # lib.rs L3008-3065: 2 rows x 256, ternary (i*17 + 3) % 3, scale 0.125,
    # a_i = sin(0.011 i - 0.3): rel err < 1e-4 against the row's dequant dot.
    n, k = 2, 256
    wt = np.array([{0: 0, 1: 1, 2: -1}[(i * 17 + 3) % 3] for i in range(n * k)]).reshape(n, k)
    code = {-1: 0, 0: 1, 1: 2}
    b = np.zeros(n * k // 4 + 4, np.uint8)
    for j in range(n):
        for blk in range(k // 128):
            for gp in range(32):
                c = [code[int(wt[j, blk * 128 + 32 * s + gp])] for s in range(4)]
                b[j * k // 4 + blk * 32 + gp] = (c[0] << 6) | (c[1] << 4) | (c[2] << 2) | c[3]
    b[-4:] = np.frombuffer(np.float32(0.125).tobytes(), np.uint8)
    a = np.sin(np.arange(k, dtype=F32) * F32(0.011) - F32(0.3)).astype(F32)
    got = O.mm_1d(a, b, O.I2_S, n, k)
    for j in range(n):
        row = np.concatenate([b[j * k // 4:(j + 1) * k // 4], b[-4:]])
        dot = _naive(a, O.dequantize(row, O.I2_S, k))
        assert abs(got[j] - dot) / max(abs(dot), 1e-6) < 1e-4


def np_values(b, dt, n, k):
    """Independent decode of the lane values (int) and scales, vectorized."""
    if dt == O.I2_S:
        codes = b[:n * k // 4].reshape(n, k // 128, 32).astype(np.int64)
        c = np.stack([(codes >> s) & 3 for s in (6, 4, 2, 0)], axis=2)   # [n, blk, 4(slot), 32(gp)]
        v = np.array([-1, 0, 1, 0])[c].reshape(n, k)                      # position 128 blk + 32 slot + gp
        return v, b[n * k // 4:n * k // 4 + 4].copy().view(F32)[0]
    qk, bb = O.BLOCK[dt]
    bl = b.reshape(n, k // qk, bb).astype(np.int64)
    if dt == O.Q1_0:
        bits = (bl[:, :, 2 + np.arange(128) // 8] >> (np.arange(128) % 8)) & 1
        return (2 * bits - 1).reshape(n, k), bl[:, :, 0:2].astype(np.uint8).copy().view(np.float16)[..., 0]
    if dt == O.Q2_0:
        q = (bl[:, :, 2 + np.arange(128) // 4] >> (2 * (np.arange(128) % 4))) & 3
        return (q - 1).reshape(n, k), bl[:, :, 0:2].astype(np.uint8).copy().view(np.float16)[..., 0]
    g = np.arange(64)
    code = (bl[:, :, g // 2] >> (4 * (g & 1))) & 0xF
    sg = (bl[:, :, 32 + g // 8] >> (g % 8)) & 1
    qp = CB[(sg << 4) | code]                                             # [n, nb, 64]
    v = np.stack([((qp >> (2 * p)) & 3) - 1 for p in range(4)], axis=3)  # [n, nb, 64, 4]
    return v.reshape(n, k), bl[:, :, 40:42].astype(np.uint8).copy().view(np.float16)[..., 0]


def np_mm(a, b, dt, n, k):
    """The reference's chains: a value +1 adds a to pos, -1 to neg (Q2_0: +2
    to plus2), 0 nothing; the visiting order is position order except I2_S
    (byte gp, then its four slots)."""
    v, d = np_values(b, dt, n, k)
    if dt == O.I2_S:
        order = [blk * 128 + 32 * s + gp for blk in range(k // 128) for gp in range(32) for s in range(4)]
        pos = np.zeros(n, F32); neg = np.zeros(n, F32)
        for i in order:
            pos = np.where(v[:, i] == 1, pos + a[i], pos).astype(F32)
            neg = np.where(v[:, i] == -1, neg + a[i], neg).astype(F32)
        return (F32(d) * (pos - neg)).astype(F32)
    qk = O.BLOCK[dt][0]
    sumf = np.zeros(n, F32)
    for blk in range(k // qk):
        pos = np.zeros(n, F32); neg = np.zeros(n, F32); p2 = np.zeros(n, F32)
        for i in range(blk * qk, blk * qk + qk):
            pos = np.where(v[:, i] == 1, pos + a[i], pos).astype(F32)
            neg = np.where(v[:, i] == -1, neg + a[i], neg).astype(F32)
            p2 = np.where(v[:, i] == 2, p2 + a[i], p2).astype(F32)
        t = (pos - neg).astype(F32)
        if dt == O.Q2_0:
            t = (t + F32(2.0) * p2).astype(F32)
        sumf = (sumf + d[:, blk].astype(F32) * t).astype(F32)
    return sumf


@pytest.mark.parametrize("dt", FMTS)
def test_mm_1d_equals_numpy_restatement(dt):
    rng = np.random.default_rng(600 + (dt & 0xFF))
    n, k = 12, 512
    b = rand_ternary(rng, dt, n, k)
    a = rng.standard_normal(k).astype(F32)
    got = O.mm_1d(a, b, dt, n, k)
    assert np.array_equal(got.view(np.uint32), np_mm(a, b, dt, n, k).view(np.uint32))


@pytest.mark.parametrize("dt", FMTS)
def test_dequant_equals_numpy_decode(dt):
    rng = np.random.default_rng(610 + (dt & 0xFF))
    n, k = 3, 512
    b = rand_ternary(rng, dt, n, k)
    v, d = np_values(b, dt, n, k)
    if dt == O.I2_S:  # one tensor: all rows' codes, then the scale
        want = (F32(d) * v.astype(F32)).reshape(-1)
        assert np.array_equal(O.dequantize(b, dt, n * k).view(np.uint32), want.view(np.uint32))
        return
    qk = O.BLOCK[dt][0]
    want = (v.astype(F32) * np.repeat(d.astype(F32), qk, axis=1)).astype(F32)
    assert np.array_equal(O.dequantize(b, dt, n * k).reshape(n, k).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dt", FMTS)
def test_mm_1d_error_bound_against_f64(dt):
    rng = np.random.default_rng(620 + (dt & 0xFF))
    n, k = 16, 1024
    b = rand_ternary(rng, dt, n, k)
    a = rng.standard_normal(k).astype(F32)
    v, d = np_values(b, dt, n, k)
    qk = 1 if dt == O.I2_S else O.BLOCK[dt][0]
    scale = np.full((n, k), float(d)) if dt == O.I2_S else np.repeat(d.astype(np.float64), qk, axis=1)
    w = v.astype(np.float64) * scale
    got = O.mm_1d(a, b, dt, n, k).astype(np.float64)
    exact = w @ a.astype(np.float64)
    bound = (k + 8) * 2.0 ** -24 * (np.abs(w) @ np.abs(a.astype(np.float64)))
    assert np.all(np.abs(got - exact) <= bound)


@pytest.mark.parametrize("dt", FMTS)
def test_q8_mode_is_the_reference_order(dt):
    rng = np.random.default_rng(630 + (dt & 0xFF))
    n, k, t = 8, 256, 2
    b = rand_ternary(rng, dt, n, k)
    x = rng.standard_normal((t, k)).astype(F32)
    assert np.array_equal(O.mm_batched_q8(x, b, dt, n, k).view(np.uint32),
                          O.mm_batched(x, b, dt, n, k).view(np.uint32))
