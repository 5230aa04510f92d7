"""The Q8 activation quantizer's rounding shortcut, checked exhaustively.

The reference quantizer rounds x * (1/d) half away from zero (f32::round,
compute/crates/rce-vm-backend-cpu/src/ml/nn.rs L541-563 quantize_block).
The GPU kernel (rce_amd/csrc/qmm_gemv.hip, round_half_away) computes it as
trunc(v + copysign(pred(0.5), v)) with one round-to-nearest-even f32 add.
Every quantized value satisfies |v| <= 127, so checking every finite
binary32 with 0 <= v <= 128 proves the two agree wherever the kernel uses
it; negative v follow by symmetry (round-to-nearest-even, trunc and
half-away rounding are all odd functions).
"""
import numpy as np


def test_round_half_away_shortcut_matches_roundf_for_all_f32_up_to_128():
    h = np.nextafter(np.float32(0.5), np.float32(0))
    assert h == np.float32(0.5) - np.float32(2.0 ** -25)
    top = int(np.array(128.0, np.float32).view(np.uint32))  # 0x43000000
    step = 1 << 24
    checked = 0
    for lo in range(0, top + 1, step):
        v = np.arange(lo, min(lo + step, top + 1), dtype=np.uint32).view(np.float32)
        want = np.floor(v.astype(np.float64) + 0.5)  # exact: v + 0.5 fits f64
        got = np.trunc(v + h)  # one f32 RNE add, then truncation
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, f"v={v[bad[0]]!r}: {got[bad[0]]} != {want[bad[0]]}"
        checked += v.size
    assert checked == top + 1
    # the half-way points and their neighbours, both signs
    for x in (0.5, 1.5, 2.5, 126.5, 127.0):
        for v in (np.float32(x), np.nextafter(np.float32(x), np.float32(0)), np.nextafter(np.float32(x), np.float32(200))):
            for sgn in (1, -1):
                w = np.float32(sgn) * v
                want = np.sign(w) * np.floor(abs(float(w)) + 0.5)
                assert np.trunc(w + np.copysign(h, w)) == want
