"""Pins the oracle's binary16 conversions, quantizers, packers and
dequantizers against the reference's own known answers and against what the
mathematics fixes (IEEE binary16, round trips).  CPU only."""
import os

import numpy as np
import pytest

import oracle as O
from conftest import lcg_uniform


# ---- binary16 ----------------------------------------------------------------

def test_f16_to_f32_exhaustive_against_ieee():
    # Every binary16 pattern widens exactly (half::f16::to_f32; kquant.rs
    # half_free L411-425); numpy's float16 is IEEE binary16.
    bits = np.arange(1 << 16, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(b)) for b in bits[::7]], np.float32)
    w = want[::7]
    nan = np.isnan(w)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), w[~nan].view(np.uint32))


def test_round_to_f16_known_answers():
    # nn.rs blocks_quantize_as_gguf_does L762-765.
    assert O.round_to_f16(65519.0) == 65504.0
    assert np.isinf(O.round_to_f16(65520.0))
    assert O.round_to_f16(2.0 ** -25) == 0.0
    assert O.round_to_f16(2.0 ** -24) == 2.0 ** -24


def test_round_to_f16_matches_ieee_rne():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(0.02),
        (rng.standard_normal(5000) * 1e-6).astype(np.float32),   # f16 subnormal range
        (rng.standard_normal(5000) * 3e4).astype(np.float32),
        np.array([0.5 + 2 ** -12, 1 + 2 ** -11, 1 + 3 * 2 ** -11, -(1 + 2 ** -11)], np.float32),  # ties
    ])
    with np.errstate(over="ignore"):  # values past 65504 round to infinity, as round_to_f16 does
        want = x.astype(np.float16).astype(np.float32)
    got = np.array([O.round_to_f16(float(v)) for v in x], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_f16_bits_inverts_widening():
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 1 << 16, 4000).astype(np.uint16)
    vals = bits.view(np.float16).astype(np.float32)
    ok = np.isfinite(vals)
    for b, v in zip(bits[ok], vals[ok]):
        if v == 0.0:
            continue  # +0/-0 both map to their own sign bit below
        assert O.f16_bits(float(v)) == int(b)
    assert O.f16_bits(0.0) == 0 and O.f16_bits(-0.0) == 0x8000


# ---- Q8_0 / Q4_0 quantizer (nn.rs quantize_block) ------------------------------

def test_quantize_block_known_answers():
    # nn.rs L751-761: x = i - 16.
    x = np.arange(32, dtype=np.float32) - 16
    q, d = O.quantize_block(x, False)
    assert d == O.round_to_f16(np.float32(16.0) / np.float32(127.0))
    assert q[0] == -127
    assert q[31] == int(np.round(np.float32(15.0) * np.float32(127.0 / 16.0)))
    q, d = O.quantize_block(x, True)
    assert d == 2.0 and q[0] == -8 and q.max() == 7


def test_q8_0_q4_0_pack_layout_round_trip():
    # quantize (toy_gpt2.rs L46-58) then dequantize (dequant.rs L360-454)
    # reproduces q * d position by position: pins the split-nibble order
    # (first 16 values = low nibbles, next 16 = high nibbles) and the sign of
    # the Q8_0 bytes.  A ramp makes every position distinct.
    x = (np.arange(64, dtype=np.float32) - 31.5) * np.float32(0.37)
    for dt in (O.Q8_0, O.Q4_0):
        b = O.quantize(x, dt)
        assert b.size == O.tensor_byte_size(dt, 64)
        got = O.dequantize(b, dt, 64)
        want = []
        for blk in range(2):
            q, d = O.quantize_block(x[32 * blk:32 * blk + 32], dt == O.Q4_0)
            want.extend(np.float32(v) * np.float32(d) for v in q)
        assert np.array_equal(got, np.array(want, np.float32))
        # and the values are close to x: |x - q d| <= d (Q8_0: d/2 + rounding)
        assert np.max(np.abs(got - x)) < 0.37 * 64 / 7


def test_dequant_q8_0_const_scale():
    # dequant.rs L748-760: scale 1.0, byte i = (i*2) as i8.
    b = np.zeros(34, np.uint8)
    b[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    b[2:] = (np.arange(32) * 2).astype(np.int8).view(np.uint8)
    assert np.array_equal(O.dequantize(b, O.Q8_0, 32), (np.arange(32) * 2).astype(np.int8).astype(np.float32))


def test_tensor_byte_size_known_answers():
    # dequant.rs tests L707-735 and quant.rs estimated_bytes_q4_0 (L295).
    assert O.tensor_byte_size(O.Q4_K, 256) == 144
    assert O.tensor_byte_size(O.Q4_K, 512) == 288
    assert O.tensor_byte_size(O.Q4_0, 32) == 18
    assert O.tensor_byte_size(O.F32, 100) == 400
    assert O.tensor_byte_size(O.Q6_K, 256) == 210
    assert O.tensor_byte_size(O.Q8_0, 4096 * 4096) == 17825792
    assert O.tensor_byte_size(O.Q4_0, 11008 * 4096) == 25362432


# ---- K-quants (kquant.rs quantize_k / pack / unpack, GT-10) ---------------------

KFMTS = [(O.Q4_K, 0), (O.Q5_K, 1), (O.Q6_K, 2)]


@pytest.mark.parametrize("fmt,disc", KFMTS)
def test_k_packing_round_trips_and_values_are_close(fmt, disc):
    # kquant.rs L425-437: x = lcg(7 + f as u64, 256) * 0.7; pack has the
    # format's byte count; unpack(pack(b)) == b; values within 0.1 of x.
    x = lcg_uniform(7 + disc, 256, 0.7)
    q, sc, mn, d, dmin = O.quantize_k(x, fmt)
    b = O.pack_k(q, sc, mn, d, dmin, fmt)
    assert b.size == O.BLOCK[fmt][1]
    q2, sc2, mn2, d2, dmin2 = O.unpack_k(b, fmt)
    assert np.array_equal(q, q2) and np.array_equal(sc, sc2) and np.array_equal(mn, mn2)
    assert d == d2 and dmin == dmin2
    # KBlock::values (kquant.rs L168-172) equals dequantize_to_f32 of the bytes
    sub = 16 if fmt == O.Q6_K else 32
    s = np.array([np.float32(d) * np.float32(c) for c in sc], np.float32)
    if fmt == O.Q6_K:
        vals = np.array([s[p // sub] * np.float32(q[p]) for p in range(256)], np.float32)
    else:
        o = np.array([np.float32(dmin) * np.float32(c) for c in mn], np.float32)
        vals = np.array([s[p // sub] * np.float32(q[p]) - o[p // sub] for p in range(256)], np.float32)
    if fmt != O.Q5_K:
        assert np.array_equal(O.dequantize(b, fmt, 256), vals)
    assert np.max(np.abs(vals - x)) < 0.1


@pytest.mark.parametrize("fmt", [O.Q4_K, O.Q6_K])
def test_k_quantizer_ranges_and_scales(fmt):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(256) * 0.02).astype(np.float32)
    q, sc, mn, d, dmin = O.quantize_k(x, fmt)
    if fmt == O.Q4_K:
        assert q.min() >= 0 and q.max() <= 15 and sc.max() <= 63 and mn.max() <= 63
        assert d == O.round_to_f16(d) and dmin == O.round_to_f16(dmin)
    else:
        assert q.min() >= -32 and q.max() <= 31 and sc.min() >= -128 and sc.max() <= 127
    # the element error is within one quantization step of its sub-block
    b = O.pack_k(q, sc, mn, d, dmin, fmt)
    err = np.abs(O.dequantize(b, fmt, 256) - x)
    assert err.max() < 0.02 * 6


def test_q4_k_dequant_layout_groups_of_64():
    # dequant.rs L546-589: group j of 64 = sc1*low nibbles of qs[32j..] -
    # min1, then sc2*high nibbles - min2 (the layout the comment at L554-557
    # says an earlier implementation got wrong).  Distinct q per position.
    q = np.array([(p * 7 + p // 64) % 16 for p in range(256)], np.int32)
    sc = np.array([1, 2, 3, 4, 5, 6, 7, 63], np.int32)
    mn = np.array([0, 1, 2, 3, 60, 61, 62, 63], np.int32)
    b = O.pack_k(q, sc, mn, 0.5, 0.25, O.Q4_K)
    v = O.dequantize(b, O.Q4_K, 256)
    want = np.array([np.float32(0.5 * sc[p // 32]) * np.float32(q[p]) - np.float32(0.25 * mn[p // 32])
                     for p in range(256)], np.float32)
    assert np.array_equal(v, want)


def test_q6_k_dequant_layout_quartets():
    # dequant.rs L658-701: per half, l in 0..32 produces positions l, l+32,
    # l+64, l+96 from ql[l], ql[l+32], qh[l]; scale index (l/16) + 2m.
    q = np.array([((p * 5) % 64) - 32 for p in range(256)], np.int32)
    sc = np.arange(16, dtype=np.int32) * 3 - 20
    b = O.pack_k(q, sc, np.zeros(0, np.int32), 0.125, 0.0, O.Q6_K)
    v = O.dequantize(b, O.Q6_K, 256)
    want = np.array([np.float32(0.125 * sc[p // 16]) * np.float32(q[p]) for p in range(256)], np.float32)
    assert np.array_equal(v, want)


# ---- GT-10 known answers (spec/book/08-steps-loops-concurrency.md L761-790,
# kquant.rs L193-245), derived by hand from the rule's text.  Each block is
# built so that one plausible mistake changes a named integer: round half to
# even instead of half away from zero, lo = the least value instead of
# min(0, least), a missing clamp of sc / m / q, the last instead of the first
# value of largest magnitude (Q6_K).

def _kat_q4k_ties_all_positive():
    """Q4_K, no negative value.  Sub-block 0: 59.0625, 9.84375, 1.96875, then
    zeros: hi - lo = 59.0625, w0 = 3.9375, d = f16(3.9375 / 63) = 0.0625,
    sc0 = 63, s0 = 3.9375, q = 59.0625 / s0 = 15, 9.84375 / s0 = 2.5 -> 3,
    1.96875 / s0 = 0.5 -> 1 (half to even: 2 and 0).  Sub-block 1: 9.84375
    then zeros: w1 = 0.65625, w1 / d = 10.5 -> sc1 = 11 (even: 10), s1 =
    0.6875, q = 14.318 -> 14.  Sub-block 2: 32 times 0.9375 (all positive):
    lo = min(0, 0.9375) = 0, w2 = 0.0625, sc2 = 1, q = 15 (lo = 0.9375 would
    give w2 = 0, sc2 = 0, q = 0).  All v_b = 0: dmin = 0, every m = 0."""
    x = np.zeros(256, np.float32)
    x[0], x[1], x[2], x[32] = 59.0625, 9.84375, 1.96875, 9.84375
    x[64:96] = 0.9375
    q = np.zeros(256, np.int32)
    q[0], q[1], q[2], q[32] = 15, 3, 1, 14
    q[64:96] = 15
    return x, q, [63, 11, 1, 0, 0, 0, 0, 0], [0] * 8, 0.0625, 0.0


def _kat_q4k_min_tie():
    """Q4_K with mins.  Sub-block 0: -7.875, 6.890625, then zeros: lo =
    -7.875, hi - lo = 14.765625, w0 = 0.984375 -> d = f16(0.984375 / 63) =
    2^-6, sc0 = 63, s0 = 0.984375; v0 = 7.875 -> dmin = f16(7.875 / 63) =
    0.125, m0 = 63, o0 = 7.875: q = 0 / s0 = 0, 14.765625 / s0 = 15, zeros
    7.875 / s0 = 8.  Sub-block 1: -2.5625, then zeros: w1 = 2.5625 / 15 ->
    w1 / d = 10.93 -> sc1 = 11, s1 = 0.171875; v1 / dmin = 20.5 -> m1 = 21
    (even: 20), o1 = 2.625: q = 0.0625 / s1 = 0.36 -> 0, zeros 2.625 / s1
    = 15.27 -> 15."""
    x = np.zeros(256, np.float32)
    x[0], x[1], x[32] = -7.875, 6.890625, -2.5625
    q = np.zeros(256, np.int32)
    q[1] = 15
    q[2:32] = 8
    q[33:64] = 15
    return x, q, [63, 11, 0, 0, 0, 0, 0, 0], [63, 21, 0, 0, 0, 0, 0, 0], 2.0 ** -6, 0.125


def _kat_q4k_clamps():
    """Q4_K of tiny values, where binary16 subnormal rounding makes the
    scales small.  Sub-block 0: 1323 * 2^-24, then zeros: w0 = 88.2 * 2^-24,
    d = f16(1.4 * 2^-24) = 2^-24, round(w0 / d) = 88 -> sc0 = 63 (clamp),
    s0 = 63 * 2^-24, q = 1323 / 63 = 21 -> 15 (clamp).  Sub-block 1:
    -88 * 2^-24, then zeros: v1 = 88 * 2^-24, dmin = f16(1.397 * 2^-24) =
    2^-24, m1 = 88 -> 63 (clamp), o1 = 63 * 2^-24; w1 = 88 / 15 * 2^-24 ->
    sc1 = round(5.87) = 6, s1 = 6 * 2^-24: q = -25 / 6 -> -4 -> 0 (clamp),
    zeros 63 / 6 = 10.5 -> 11 (even: 10)."""
    u = np.float32(2.0 ** -24)
    x = np.zeros(256, np.float32)
    x[0], x[32] = np.float32(1323) * u, np.float32(-88) * u
    q = np.zeros(256, np.int32)
    q[0] = 15
    q[33:64] = 11
    return x, q, [63, 6, 0, 0, 0, 0, 0, 0], [0, 63, 0, 0, 0, 0, 0, 0], 2.0 ** -24, 2.0 ** -24


def _kat_q6k_first_of_largest():
    """Q6_K.  Sub-block 0: 0.5, -0.5, then zeros: the first value of largest
    magnitude is 0.5, w0 = 0.5 / -32 = -2^-6; d = f16(2^-6 / 127) = 1032 *
    2^-23; sc0 = round(-127.008) = -127, s0 = -131064 * 2^-23: q = 0.5 / s0
    = -32.002 -> -32, -0.5 / s0 = 32.002 -> 31 (clamp).  The last value of
    largest magnitude would give sc0 = 127, q = 31 and -32.  Other
    sub-blocks: w = -0.0, sc = 0, s = 0, q = 0."""
    x = np.zeros(256, np.float32)
    x[0], x[1] = 0.5, -0.5
    q = np.zeros(256, np.int32)
    q[0], q[1] = -32, 31
    return x, q, [-127] + [0] * 15, [], 1032 * 2.0 ** -23, 0.0


def _kat_q5k_ties_all_positive():
    """Q5_K (nmax 31), no negative value.  Sub-block 0: 122.0625, 9.84375,
    1.96875, then zeros: w0 = 122.0625 / 31 = 3.9375 exactly, d = f16(3.9375
    / 63) = 0.0625, sc0 = 63, s0 = 3.9375: q = 31, 9.84375 / s0 = 2.5 -> 3,
    1.96875 / s0 = 0.5 -> 1 (half to even: 2 and 0).  Sub-block 1: 20.34375
    then zeros: w1 = 0.65625, w1 / d = 10.5 -> sc1 = 11 (even: 10), s1 =
    0.6875, q = 29.59 -> 30 (sc1 = 10 would give 32.55 -> 31).  Sub-block 2:
    32 times 1.9375: lo = min(0, 1.9375) = 0, w2 = 1.9375 / 31 = 0.0625,
    sc2 = 1, q = 31 (lo = 1.9375 would give w2 = 0, sc2 = 0, q = 0).  Every
    v_b = 0: dmin = 0, every m = 0."""
    x = np.zeros(256, np.float32)
    x[0], x[1], x[2], x[32] = 122.0625, 9.84375, 1.96875, 20.34375
    x[64:96] = 1.9375
    q = np.zeros(256, np.int32)
    q[0], q[1], q[2], q[32] = 31, 3, 1, 30
    q[64:96] = 31
    return x, q, [63, 11, 1, 0, 0, 0, 0, 0], [0] * 8, 0.0625, 0.0


def _kat_q5k_min_tie():
    """Q5_K with mins.  Sub-block 0: -7.875, 22.640625, then zeros: lo =
    -7.875, hi - lo = 30.515625, w0 = 0.984375 -> d = f16(0.984375 / 63) =
    2^-6, sc0 = 63, s0 = 0.984375; v0 = 7.875 -> dmin = f16(7.875 / 63) =
    0.125, m0 = 63, o0 = 7.875: q = 0, 30.515625 / s0 = 31, zeros 7.875 / s0
    = 8.  Sub-block 1: -2.5625, then zeros: w1 = 2.5625 / 31, w1 / d = 5.29
    -> sc1 = 5, s1 = 0.078125; v1 / dmin = 20.5 -> m1 = 21 (even: 20), o1 =
    2.625: q = 0.0625 / s1 = 0.8 -> 1 (m1 = 20: -0.8 -> 0), zeros 2.625 / s1
    = 33.6 -> 34 -> 31 (clamp)."""
    x = np.zeros(256, np.float32)
    x[0], x[1], x[32] = -7.875, 22.640625, -2.5625
    q = np.zeros(256, np.int32)
    q[1] = 31
    q[2:32] = 8
    q[32] = 1
    q[33:64] = 31
    return x, q, [63, 5, 0, 0, 0, 0, 0, 0], [63, 21, 0, 0, 0, 0, 0, 0], 2.0 ** -6, 0.125


KATS = [(O.Q4_K, _kat_q4k_ties_all_positive), (O.Q4_K, _kat_q4k_min_tie), (O.Q4_K, _kat_q4k_clamps),
        (O.Q5_K, _kat_q5k_ties_all_positive), (O.Q5_K, _kat_q5k_min_tie), (O.Q6_K, _kat_q6k_first_of_largest)]


@pytest.mark.parametrize("fmt,kat", KATS)
def test_quantize_k_known_answers(fmt, kat):
    x, q, sc, mn, d, dmin = kat()
    gq, gsc, gmn, gd, gdmin = O.quantize_k(x, fmt)
    assert gd == d and gdmin == dmin
    assert list(gsc) == sc
    if fmt != O.Q6_K:
        assert list(gmn) == mn
    assert np.array_equal(gq, q), np.nonzero(gq != q)[0][:8]


@pytest.mark.parametrize("fmt,kat", KATS)
def test_library_quantizer_bytes_on_known_answers(fmt, kat):
    """rce_qmm_quantize (the product's encoder) writes the oracle's bytes
    on the known-answer blocks (Q5_K too: same rule, nmax 31)."""
    import rce_amd
    x = kat()[0]
    assert np.array_equal(rce_amd.quantize(x.reshape(1, 256), fmt), O.quantize(x, fmt))


# ---- planted mistakes: copies of the oracle built with one mistake each
# (-DORC_PLANT=k in oracle/qmm_oracle.c) must each fail a known answer.

PLANTS = {1: "round half to even", 2: "lo = the least value", 3: "no clamp of sc", 4: "no clamp of m",
          5: "Q6_K: the last value of largest magnitude"}


@pytest.fixture(scope="module")
def planted_oracles(tmp_path_factory):
    import ctypes
    import shutil
    import subprocess
    if not shutil.which("gcc"):
        pytest.skip("gcc not available")
    src = os.path.join(os.path.dirname(O.__file__), "qmm_oracle.c")
    libs = {}
    for k in [0, *PLANTS]:  # 0: the shipped oracle, built the same way (the control)
        so = str(tmp_path_factory.mktemp("plant") / f"lib{k}.so")
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fPIC", "-shared", "-std=c11", f"-DORC_PLANT={k}", src,
                        "-o", so, "-lm"], check=True)
        L = ctypes.CDLL(so)
        L.orc_quantize_k.restype = None
        L.orc_quantize_k.argtypes = [ctypes.c_void_p, ctypes.c_uint32] + [ctypes.c_void_p] * 5
        libs[k] = L
    return libs


def _kat_holds(L, fmt, kat):
    x, q, sc, mn, d, dmin = kat()
    x = np.ascontiguousarray(x, np.float32)
    gq = np.zeros(256, np.int32); gsc = np.zeros(16, np.int32); gmn = np.zeros(8, np.int32)
    gd = np.zeros(1, np.float32); gdm = np.zeros(1, np.float32)
    L.orc_quantize_k(x.ctypes.data, fmt, gq.ctypes.data, gsc.ctypes.data, gmn.ctypes.data, gd.ctypes.data,
                     gdm.ctypes.data)
    nsc = 16 if fmt == O.Q6_K else 8
    ok = gd[0] == d and gdm[0] == dmin and list(gsc[:nsc]) == sc and np.array_equal(gq, q)
    return ok and (fmt == O.Q6_K or list(gmn) == mn)


def test_unplanted_copy_holds_every_known_answer(planted_oracles):
    assert all(_kat_holds(planted_oracles[0], fmt, kat) for fmt, kat in KATS)


@pytest.mark.parametrize("plant", sorted(PLANTS))
def test_each_planted_mistake_fails_a_known_answer(planted_oracles, plant):
    failed = [kat.__name__ for fmt, kat in KATS if not _kat_holds(planted_oracles[plant], fmt, kat)]
    assert failed, f"no known answer catches: {PLANTS[plant]}"


# ---- non-finite blocks: the reference's integer semantics (Rust `as i32`
# saturates, NaN -> 0; adds wrap in a release build; `as u8` / `as i8` keep
# the low bits; f16_bits (kquant.rs L267-281, toy_gpt2.rs L30-42) of an
# infinity keeps its exponent's low bits: (143 << 10) mod 2^16 = 0x3C00).
# Each byte string is derived by hand from nn.rs L541-563 / kquant.rs
# L193-245 and the packers.

def _nf_q8_inf():
    """Q8_0 [+inf, 1, NaN, -2, 0...]: amax = +inf (NaN fails amax < |v|), d =
    inf, id = 1/inf = 0; x * 0 is NaN (inf, NaN) or +-0: every q = 0.  The
    scale round_to_f16(inf) = inf is written 0x3C00."""
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2], x[3] = np.inf, 1.0, np.nan, -2.0
    return O.Q8_0, x, bytes([0x00, 0x3C] + [0] * 32)


def _nf_q8_tiny():
    """Q8_0 [2^-130, -2^-131, 0...]: d = 2^-130 / 127 (subnormal), 1/d
    overflows to inf: q0 = round(inf) as i32 = i32::MAX, as i8 = -1 (0xFF);
    q1 = i32::MIN as i8 = 0; 0 * inf = NaN -> 0.  round_to_f16(d) = 0."""
    x = np.zeros(32, np.float32)
    x[0], x[1] = 2.0 ** -130, -(2.0 ** -131)
    return O.Q8_0, x, bytes([0, 0, 0xFF, 0x00] + [0] * 30)


def _nf_q4_0_tiny():
    """Q4_0 [-2^-130, 2^-131, 0...]: m = -2^-130, d = m / -8 = 2^-133, id =
    2^133 = inf.  t0 = -inf: floor as i32 = i32::MIN, .min(15) - 8 and + 8
    wrap back to i32::MIN, as u8 = 0; t1 = +inf: i32::MAX -> 15; zeros: NaN
    -> 0 -> q = -8 -> 0.  Byte 1 = 15 | 0 << 4; round_to_f16(2^-133) = 0."""
    x = np.zeros(32, np.float32)
    x[0], x[1] = -(2.0 ** -130), 2.0 ** -131
    return O.Q4_0, x, bytes([0, 0, 0x00, 0x0F] + [0] * 14)


def _nf_q4k_inf():
    """Q4_K [+inf, 1.875, 0...]: w0 = inf, d = f16(inf) = inf (0x3C00), dmin
    = 0; sc0 = round(inf / inf) = NaN -> 0, the others 0 / inf = 0; s = inf
    * 0 = NaN != 0, so q = round(NaN) -> 0 everywhere."""
    x = np.zeros(256, np.float32)
    x[0], x[1] = np.inf, 1.875
    return O.Q4_K, x, bytes([0x00, 0x3C] + [0] * 142)


def _nf_q4k_nan_subblock():
    """Q4_K: sub-block 0 [1.875, 0...], sub-block 4 all NaN: there lo = 0 and
    hi = -inf (NaN fails both tests), w4 = -inf; w0 = 0.125, d = f16(0.125 /
    63) = 1040 * 2^-19 (0x1810), sc0 = round(63.015) = 63; sc4 = -inf / d as
    i32 = i32::MIN, .min(63) keeps it, and `as u8` packs 0: scale byte 0 =
    63 | (0 >> 4) << 6.  q0 = 1.875 / (63 d) = 15.004 -> 15; sub-block 4: s =
    d * -2^31, q = round(NaN) -> 0."""
    x = np.zeros(256, np.float32)
    x[0] = 1.875
    x[128:160] = np.nan
    b = [0x10, 0x18, 0, 0, 0x3F] + [0] * 11 + [0x0F] + [0] * 127
    return O.Q4_K, x, bytes(b)


NONFINITE = [_nf_q8_inf, _nf_q8_tiny, _nf_q4_0_tiny, _nf_q4k_inf, _nf_q4k_nan_subblock]


@pytest.mark.parametrize("kat", NONFINITE)
def test_quantize_nonfinite_known_answers(kat):
    fmt, x, want = kat()
    assert bytes(O.quantize(x, fmt)) == want


@pytest.mark.parametrize("kat", NONFINITE)
def test_library_quantizer_nonfinite_known_answers(kat):
    import rce_amd
    fmt, x, want = kat()
    assert bytes(rce_amd.quantize(x.reshape(1, -1), fmt)) == want
