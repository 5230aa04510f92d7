"""GPU parity of the prefill GEMM on the matrix cores (RCE_QMM_MODE_F16_MFMA).

The mode dequantizes the weights to binary16 and contracts them with f16
MFMA, f32 accumulation: Q4_K, Q5_K, Q4_0 (and Q8_0, Q6_K in a plain GEMM)
in registers, gemm_f16.hip; the other formats into LDS tiles,
gemm_gen.hip.  Two checks per case:
  * against a numpy restatement of the same f16 weights (f64 products):
    only accumulation order differs, so normwise error must be ~1e-6 --
    this catches a wrong fragment layout, K order or scale;
  * against the oracle's EXACT result (the reference's f32 order,
    rce-op-qmm mm_batched L967-1023): normwise max|gpu - ref| / max|ref|
    within 2e-3, the stated budget of the fp16-dequant path.
Elementwise relative error is not bounded near zero outputs by any f16
path; the tolerance is normwise, as the reference's own combined
tolerances are (rce-op-qmm L3462-3475).
"""
import numpy as np
import pytest

import oracle as O
import rce_amd
from rce_amd import GgufDtype as G, Mode

pytestmark = pytest.mark.gpu
F32 = np.float32
F16 = np.float16


def note(msg):
    print(msg, flush=True)


def q4k_f16_weights(b, n, k, q5=False):
    """Q4_K bytes -> the f16 weights the kernel forms: f16(f16(d*sc)*q + f16(-dmin*m))
    (one rounding of the fma), decoded with numpy from the GGUF layout
    (rce-ingest-gguf dequant.rs L546-589).  q5: Q5_K's 176-byte blocks, the
    32 qh bytes after the scales giving q's fifth bit (qh byte l, bit s =
    position 32 s + l; dequant.rs L591-636)."""
    nsb = k // 256
    blk = np.frombuffer(bytes(b), np.uint8).reshape(n, nsb, 176 if q5 else 144)
    d = blk[:, :, 0:2].copy().view(F16)[:, :, 0].astype(F32)
    dmin = blk[:, :, 2:4].copy().view(F16)[:, :, 0].astype(F32)
    s = blk[:, :, 4:16].astype(np.int32)
    sc = np.zeros((n, nsb, 8), np.int32)
    mn = np.zeros((n, nsb, 8), np.int32)
    for j in range(8):
        if j < 4:
            sc[:, :, j] = s[:, :, j] & 63
            mn[:, :, j] = s[:, :, j + 4] & 63
        else:
            sc[:, :, j] = (s[:, :, j + 4] & 0x0F) | ((s[:, :, j - 4] >> 6) << 4)
            mn[:, :, j] = (s[:, :, j + 4] >> 4) | ((s[:, :, j] >> 6) << 4)
    qs_at = 48 if q5 else 16
    qs = blk[:, :, qs_at:qs_at + 128].astype(np.int32).reshape(n, nsb, 4, 32)
    q = np.zeros((n, nsb, 8, 32), np.int32)
    q[:, :, 0::2, :] = qs & 0x0F
    q[:, :, 1::2, :] = qs >> 4
    if q5:
        qh = blk[:, :, 16:48].astype(np.int32)
        for sb in range(8):
            q[:, :, sb, :] |= ((qh >> sb) & 1) << 4
    d1 = (d[:, :, None] * sc.astype(F32)).astype(F16).astype(np.float64)
    m1 = (-(dmin[:, :, None] * mn.astype(F32))).astype(F16).astype(np.float64)
    w = (q.astype(np.float64) * d1[:, :, :, None] + m1[:, :, :, None]).astype(F16)
    return w.reshape(n, k).astype(np.float64)


def q40_f16_weights(b, n, k):
    """Q4_0 bytes -> f16(d * (q - 8)) (rce-ingest-gguf dequant.rs L360-382)."""
    nb = k // 32
    blk = b.reshape(n, nb, 18)
    d = blk[:, :, 0:2].copy().view(F16)[:, :, 0].astype(np.float64)
    qs = blk[:, :, 2:18].astype(np.int32)
    q = np.concatenate([(qs & 0x0F) - 8, (qs >> 4) - 8], axis=2).astype(np.float64)
    return (q * d[:, :, None]).astype(F16).reshape(n, k).astype(np.float64)


def q41_f16_weights(b, n, k):
    """Q4_1 bytes (d, m, qs[16] per block) -> the nibble kernel's weight
    f16(d * q + m), the product and sum exact, one rounding (the reference
    rounds d * q and the sum in f32 first, dequant.rs Q4_1; they differ in
    rare double-rounding cases only)."""
    nb = k // 32
    blk = np.frombuffer(bytes(b), np.uint8).reshape(n, nb, 20)
    d = blk[:, :, 0:2].copy().view(F16)[:, :, 0].astype(np.float64)
    m = blk[:, :, 2:4].copy().view(F16)[:, :, 0].astype(np.float64)
    qs = blk[:, :, 4:20].astype(np.int32)
    q = np.concatenate([qs & 0x0F, qs >> 4], axis=2).astype(np.float64)
    return (q * d[:, :, None] + m[:, :, None]).astype(F16).reshape(n, k).astype(np.float64)


def run_gemm(ctx, w, x, a_dtype):
    t = x.shape[0]
    xa = rce_amd.DeviceBuffer.from_numpy(ctx, x)
    out = rce_amd.DeviceBuffer(ctx, t * w.n_rows * 4)
    rce_amd.mm_batched_dev(ctx, xa.ptr, a_dtype, t, w, out.ptr, Mode.F16_MFMA)
    ctx.synchronize()
    r = out.download(F32, t * w.n_rows).reshape(t, w.n_rows)
    xa.free(); out.free()
    return r


def normwise(got, want):
    return float(np.max(np.abs(got.astype(np.float64) - want)) / np.max(np.abs(want)))


CASES = [
    # (dtype, n_rows, n_cols, tokens): the configs[2] shape, ragged M and N,
    # short K (split-K off), Q4_0 (the MoE experts' format)
    (O.Q4_K, 4096, 4096, 512),
    (O.Q4_K, 384, 1024, 100),
    (O.Q4_K, 200, 2048, 33),
    (O.Q4_K, 128, 256, 1),
    (O.Q4_0, 1024, 4096, 64),
    (O.Q4_0, 300, 512, 7),
    (O.Q4_0, 64, 14336, 5),
    # 65..96 rows: the 96 x 128 tile (RB = 3: three row blocks per wave)
    (O.Q4_K, 300, 1024, 80),
    (O.Q4_0, 256, 2048, 96),
    # a last 128-row tile holding 72 / 22 rows: the 96 x 64 / 64 x 64 body
    (O.Q4_K, 256, 1024, 200),
    (O.Q4_0, 128, 512, 150),
]


@pytest.mark.parametrize("dt,n,k,t", CASES)
@pytest.mark.parametrize("a16", [True, False])
def test_gemm_f16_mfma_parity(ctx, dt, n, k, t, a16):
    if not a16 and (n, k, t) == (4096, 4096, 512):
        pytest.skip("f32 activations covered at the smaller shapes")
    note(f"gemm f16-mfma dtype={dt} n={n} k={k} t={t} a16={a16}")
    rng = np.random.default_rng(9000 + dt + n + k + t)
    w32 = (rng.standard_normal((n, k)) * 0.02).astype(F32)
    b = O.quantize(w32, dt)
    x = rng.standard_normal((t, k)).astype(F16 if a16 else F32)
    xv = x.astype(F16).astype(np.float64)  # the kernel's f16 activations
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k)
    got = run_gemm(ctx, w, x, G.F16 if a16 else G.F32)
    wf = q4k_f16_weights(b, n, k) if dt == O.Q4_K else q40_f16_weights(b, n, k)
    same = xv @ wf.T
    assert normwise(got, same) < 1e-5, "kernel differs from the f16-weight restatement"
    ref = O.mm_batched(x.astype(F32), b, dt, n, k)  # reference order, f32 activations
    assert normwise(got, ref) < 2e-3
    again = run_gemm(ctx, w, x, G.F16 if a16 else G.F32)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "not run-to-run deterministic"


def test_gemm_supports_matrix():
    assert rce_amd.supports(G.Q4K, 4096, Mode.F16_MFMA)
    assert rce_amd.supports(G.Q4_0, 4096, Mode.F16_MFMA)
    assert not rce_amd.supports(G.Q4_0, 4096 + 64, Mode.F16_MFMA)  # whole groups of 8 blocks
    for dt in (G.Q6K, G.Q5K, G.Q8_0, G.Q5_0, G.Q4_1, G.F16):
        assert rce_amd.supports(dt, 4096, Mode.F16_MFMA), dt
    assert rce_amd.supports(G.Q8_0, 4096 + 64, Mode.F16_MFMA)
    assert not rce_amd.supports(G.Q8_0, 4096 + 32, Mode.F16_MFMA)  # whole chunks of 64
    assert not rce_amd.supports(G.Q6K, 4096 + 64, Mode.F16_MFMA)   # whole super-blocks
    for dt in (G.F32, G.BF16):                                     # the bf16 matrix-core forms
        assert rce_amd.supports(dt, 4096, Mode.F16_MFMA), dt
        assert not rce_amd.supports(dt, 4096 + 32, Mode.F16_MFMA), dt
    for dt in (G.Q3K, G.Q1_0, G.Q2_0, G.I2S):                      # no matrix-core form
        assert not rce_amd.supports(dt, 4096, Mode.F16_MFMA), dt


# ---- the other formats (gemm_gen.hip): every weight is the reference's f32
# dequantized value (rce-ingest-gguf dequant.rs) rounded once to binary16, so
# the restatement is the oracle's dequantize() rounded by numpy.

def gen_weight_bytes(rng, dt, n, k):
    from rand_blocks import float_bytes, rand_blocks
    if dt in (O.F16, O.BF16, O.F32):
        return float_bytes(rng, dt, n, k, 0.02)
    if dt in (O.Q5_0, O.Q4_1):  # no quantizer in the reference: random blocks
        return rand_blocks(rng, dt, n, k, dmax=0.02 / 8)
    return O.quantize((rng.standard_normal((n, k)) * 0.02).astype(F32), dt)


GEN_CASES = [
    # (dtype, n_rows, n_cols, tokens): configs[2]'s shape for the three
    # formats a Q4_K_M / Q5_K model's prefill needs besides Q4_K, then
    # ragged M and N (partial tiles, N not a multiple of the 64-row IL64
    # groups), chunk counts that are not multiples of the 6-deep load ring
    (O.Q6_K, 4096, 4096, 512),
    (O.Q8_0, 4096, 4096, 512),
    (O.Q5_K, 4096, 4096, 512),
    (O.Q6_K, 200, 2048, 33),
    (O.Q8_0, 300, 576, 7),
    (O.Q8_0, 64, 64, 1),
    (O.Q5_K, 130, 512, 129),
    (O.Q5_0, 256, 1024, 100),
    (O.Q4_1, 192, 1088, 65),
    (O.F16, 100, 640, 17),
    # a last 128-row tile holding 72 / 22 rows (the 96- / 64-row bodies)
    (O.Q8_0, 320, 1024, 200),
    (O.Q6_K, 256, 1024, 150),
    # K / 64 = 7 and 13 (= 1 mod 6): the pipeline's tail then holds DEPTH + 1
    # chunks, the last of which it must load itself
    (O.Q8_0, 128, 448, 40),
    (O.F16, 96, 832, 20),
    (O.Q4_1, 64, 1600, 9),
    # the bf16 forms (BF16 exact; F32 as two bf16 terms), configs[2]'s
    # shape and ragged ones
    (O.BF16, 4096, 4096, 512),
    (O.F32, 4096, 4096, 512),
    (O.BF16, 100, 640, 17),
    (O.F32, 130, 832, 65),
    # Q8_0 with K a multiple of 256 runs on the nibble kernel's 128 x 64 tile
    # (four 64-byte pieces per row and scale group, five A stages): one, two,
    # three and five groups, ragged M and N, one token, two row tiles
    (O.Q8_0, 64, 256, 1),
    (O.Q8_0, 300, 768, 37),
    (O.Q8_0, 130, 1280, 129),
    (O.Q8_0, 96, 512, 200),
    # Q6_K likewise (the 64-row groups of its interleaved layout, 13 chunks
    # per super-block, four scale sets per chunk): one and three super-blocks
    (O.Q6_K, 64, 256, 1),
    (O.Q6_K, 130, 768, 129),
    # Q5_K: Q4_K's tiles plus 32 bytes of fifth bits per row and group; the
    # 64-, 96- and 128-row tiles, ragged M and N
    (O.Q5_K, 64, 256, 1),
    (O.Q5_K, 200, 768, 80),
    (O.Q5_K, 130, 1280, 50),
    # Q4_1 ({d, m} words as the scale words) and Q5_0 (Q4_0 plus fifth-bit
    # words) with K a multiple of 256 on the same kernel, all three tiles
    (O.Q4_1, 130, 512, 37),
    (O.Q4_1, 200, 768, 80),
    (O.Q4_1, 64, 2048, 129),
    (O.Q5_0, 64, 256, 1),
    (O.Q5_0, 200, 768, 80),
    (O.Q5_0, 130, 1280, 129),
]


def bf16_round(v):
    """float32 -> the nearest bfloat16 (ties to even), as float64."""
    u = np.ascontiguousarray(v, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def q6k_f16_weights(b, n, k):
    """Q6_K bytes -> the f16 weights the nibble kernel forms:
    f16(f16(d*sc) * q), the scale rounded to binary16 first (GGUF block:
    ql 128, qh 64, 16 signed scales, f16 d; position P of a super-block: half
    n = P // 128, quarter qd, l: ql byte 64n + l + 32(qd & 1), high nibble
    for qd >= 2, qh byte 32n + l bits 2qd, scale 8n + l // 16 + 2qd)."""
    nsb = k // 256
    blk = np.frombuffer(bytes(b), np.uint8).reshape(n, nsb, 210)
    ql, qh = blk[:, :, :128].astype(np.int32), blk[:, :, 128:192].astype(np.int32)
    sc = blk[:, :, 192:208].view(np.int8).astype(np.float32)
    d = blk[:, :, 208:210].copy().view(np.float16).astype(np.float32)[:, :, 0]
    P = np.arange(256)
    hn, qd, l = P // 128, (P % 128) // 32, P % 32
    lo = ql[:, :, 64 * hn + l + 32 * (qd & 1)]
    nib = np.where(qd >= 2, lo >> 4, lo & 15)
    q = (nib | (((qh[:, :, 32 * hn + l] >> (2 * qd)) & 3) << 4)) - 32
    s16 = (d[:, :, None] * sc).astype(np.float16).astype(np.float64)  # f32 product, one rounding
    w = (s16[:, :, 8 * hn + l // 16 + 2 * qd] * q).astype(np.float16)
    return w.reshape(n, k).astype(np.float64)


def mfma_weights(b, dt, n, k):
    """The weights the F16_MFMA kernels contract: the reference's f32
    dequantized value rounded once to binary16; BF16 exactly; F32 as
    bf16(w) + bf16(w - bf16(w))."""
    v = O.dequantize(b, dt, n * k).reshape(n, k)
    if dt == O.BF16:
        return v.astype(np.float64)
    if dt == O.F32:
        hi = bf16_round(v)
        return hi + bf16_round((v.astype(np.float64) - hi).astype(np.float32))
    return v.astype(F16).astype(np.float64)


@pytest.mark.parametrize("dt,n,k,t", GEN_CASES)
def test_gemm_other_formats_parity(ctx, dt, n, k, t):
    note(f"gemm-gen f16-mfma dtype={dt} n={n} k={k} t={t}")
    rng = np.random.default_rng(7100 + dt + n + k + t)
    b = gen_weight_bytes(rng, dt, n, k)
    x = rng.standard_normal((t, k)).astype(F16)
    xv = x.astype(np.float64)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k)
    got = run_gemm(ctx, w, x, G.F16)
    # Q6_K and Q5_K run the nibble kernel (scale rounded to binary16 first),
    # as does Q4_1 at K % 256 == 0 (d q + m rounded once)
    if dt == O.Q6_K:
        wf = q6k_f16_weights(b, n, k)
    elif dt == O.Q5_K:
        wf = q4k_f16_weights(b, n, k, q5=True)
    elif dt == O.Q4_1 and k % 256 == 0:
        wf = q41_f16_weights(b, n, k)
    else:
        wf = mfma_weights(b, dt, n, k)
    assert np.all(np.isfinite(wf))
    assert normwise(got, xv @ wf.T) < 1e-5, "kernel differs from the f16-weight restatement"
    ref = O.mm_batched(x.astype(F32), b, dt, n, k)
    assert normwise(got, ref) < 2e-3
    again = run_gemm(ctx, w, x, G.F16)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "not run-to-run deterministic"
    w.close()


@pytest.mark.parametrize("dt", [O.BF16, O.F32])
def test_gemm_bf16_forms_beyond_binary16_range(ctx, dt):
    """BF16 / F32 weights whose magnitudes binary16 cannot hold (2^100 and
    2^-100 scales on alternate rows) keep their values on the bf16 matrix
    cores: the result equals the restatement of the same bf16 terms."""
    n, k, t = 192, 1024, 40
    note(f"gemm bf16 forms, range, dtype={dt}")
    rng = np.random.default_rng(7500 + dt)
    wv = rng.standard_normal((n, k)).astype(F32)
    wv[0::2] *= F32(2.0 ** 100)
    wv[1::2] *= F32(2.0 ** -100)
    b = wv.view(np.uint8).reshape(-1) if dt == O.F32 else (wv.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1)
    x = rng.standard_normal((t, k)).astype(F16)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k)
    got = run_gemm(ctx, w, x, G.F16)
    want = x.astype(np.float64) @ mfma_weights(b, dt, n, k).T
    for rows in (slice(0, None, 2), slice(1, None, 2)):  # each scale against its own rows
        assert np.all(np.isfinite(got[:, rows]))
        assert normwise(got[:, rows], want[:, rows]) < 1e-5
    w.close()


@pytest.mark.parametrize("dt", [O.Q6_K, O.Q8_0])
def test_gemm_other_formats_f32_activations(ctx, dt):
    """F32 activations are rounded to binary16 first (the library's
    conversion kernel); the result equals the F16 call on those values."""
    n, k, t = 192, 1024, 40
    note(f"gemm-gen f32 activations dtype={dt}")
    rng = np.random.default_rng(7200 + dt)
    b = gen_weight_bytes(rng, dt, n, k)
    x = rng.standard_normal((t, k)).astype(F32)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k)
    got32 = run_gemm(ctx, w, x, G.F32)
    got16 = run_gemm(ctx, w, x.astype(F16), G.F16)
    assert np.array_equal(got32.view(np.uint32), got16.view(np.uint32))
    assert normwise(got32, O.mm_batched(x, b, dt, n, k)) < 2e-3
    w.close()


@pytest.mark.parametrize("dt", [O.Q4_K, O.Q8_0])
def test_gemm_misaligned_f16_activations_rejected(ctx, dt):
    """The GEMM reads activations 16 bytes per lane: an F16 pointer off a
    16-byte boundary is refused on the host before any launch."""
    n, k, t = 64, 256, 4
    rng = np.random.default_rng(7300 + dt)
    b = O.quantize((rng.standard_normal((n, k)) * 0.02).astype(F32), dt)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k)
    xa = rce_amd.DeviceBuffer(ctx, 2 * t * k + 16)
    out = rce_amd.DeviceBuffer(ctx, 4 * t * n)
    with pytest.raises(rce_amd.QmmError, match="16-byte aligned"):
        rce_amd.mm_batched_dev(ctx, xa.ptr + 2, G.F16, t, w, out.ptr, Mode.F16_MFMA)
    xa.free(); out.free(); w.close()


def test_gemm_activations_past_4gib_sliced(ctx):
    """The nibble kernel's activation offsets are 32-bit, so a call whose
    f16 activations pass 2^32 bytes runs in slices of whole 128-row tiles
    (qmm_abi.cpp run_gemm).  Each output's sum does not depend on the
    slicing: rows on both sides of the slice boundary and the last rows
    equal, bit for bit, a separate call on just those rows, which in turn
    is within the f16 budget of the oracle."""
    n, k = 64, 256
    max_rows = ((2 ** 32 - 1) // (2 * k)) // 128 * 128  # the host's slice
    t = max_rows + 1000
    note(f"gemm f16-mfma sliced activations t={t} k={k} ({2 * t * k / 2 ** 30:.2f} GiB)")
    rng = np.random.default_rng(7400)
    b = O.quantize((rng.standard_normal((n, k)) * 0.02).astype(F32), O.Q4_0)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, O.Q4_0, n, k)
    base = rng.standard_normal((4099, k)).astype(F16)  # a period prime to the tile rows
    x = np.resize(base, (t, k))
    xa = rce_amd.DeviceBuffer.from_numpy(ctx, x)
    out = rce_amd.DeviceBuffer(ctx, t * n * 4)
    rce_amd.mm_batched_dev(ctx, xa.ptr, G.F16, t, w, out.ptr, Mode.F16_MFMA)
    ctx.synchronize()
    got = out.download(F32, t * n).reshape(t, n)
    xa.free(); out.free()
    rows = np.r_[0:200, max_rows - 300:max_rows + 300, t - 200:t]
    want = run_gemm(ctx, w, np.ascontiguousarray(x[rows]), G.F16)
    assert np.array_equal(got[rows].view(np.uint32), want.view(np.uint32))
    assert normwise(want, O.mm_batched(x[rows].astype(F32), b, O.Q4_0, n, k)) < 2e-3
    w.close()


@pytest.mark.parametrize("dt", [O.Q4_K, O.Q4_0, O.Q8_0])
def test_gemm_rows_independent_of_tile_shape(ctx, dt):
    """Each output's sum is formed the same way in every tile shape and body
    (a wave's k-step partial over the chunks in order, the four partials
    added in order), so a row's result does not depend on how many rows the
    call has: M 40 and 64 (a 64-row tile, 64 columns wide), 80 (96 rows),
    200 (128 rows, then a 72-row tile in the 96-row body) and 512 against
    the same rows of one another, bit for bit."""
    n, k = 512, 1024
    note(f"gemm tile-shape independence dtype={dt}")
    rng = np.random.default_rng(7500 + dt)
    b = O.quantize((rng.standard_normal((n, k)) * 0.02).astype(F32), dt)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k)
    x = rng.standard_normal((512, k)).astype(F16)
    full = run_gemm(ctx, w, x, G.F16)
    for m in (40, 64, 80, 200):
        got = run_gemm(ctx, w, np.ascontiguousarray(x[:m]), G.F16)
        assert np.array_equal(got.view(np.uint32), full[:m].view(np.uint32)), f"M={m}"
    tail = run_gemm(ctx, w, np.ascontiguousarray(x[440:]), G.F16)  # 72 rows
    assert np.array_equal(tail.view(np.uint32), full[440:].view(np.uint32))
    w.close()
