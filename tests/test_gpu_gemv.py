"""GPU parity of the decode kernels through the C ABI (librce_qmm.so).

EXACT mode must equal the oracle's restatement of rce_op_qmm::mm_1d /
mm_batched bit for bit; Q8 mode must equal the oracle's restatement of the
same Q8-activation algorithm bit for bit (the 1e-5 budget is not needed);
dequant_row must equal dequantize_to_f32 bit for bit."""
import sys

import numpy as np
import pytest

import oracle as O
import rce_amd
from rce_amd import GgufDtype as G, Mode
from rand_blocks import float_bytes, rand_blocks, rand_ternary

pytestmark = pytest.mark.gpu
F32 = np.float32


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make(rng, dt, n, k, sigma=0.02):
    if dt in (O.Q5_0, O.Q4_1, O.Q3_K):  # no quantizer in the reference: random blocks
        return rand_blocks(rng, dt, n, k)
    if dt in (O.F32, O.F16, O.BF16):
        return float_bytes(rng, dt, n, k, sigma)
    if dt in (O.Q1_0, O.Q2_0, O.STQ1_0, O.I2_S):  # multiply-free formats: random codes
        return rand_ternary(rng, dt, n, k)
    w = (rng.standard_normal((n, k)) * sigma).astype(F32)
    return O.quantize(w, dt)


def bits(x):
    return np.ascontiguousarray(x, F32).view(np.uint32)


SHAPES = {
    # (n_rows, n_cols): small, ragged and the configs' shapes
    O.Q8_0: [(1, 32), (16, 32), (3, 64), (65, 256), (1000, 2048), (4096, 4096)],
    O.Q4_0: [(1, 32), (6, 128), (77, 1024), (1024, 2048), (11008, 4096), (4096, 14336)],
    O.Q4_K: [(1, 256), (5, 512), (130, 2048), (2048, 5632), (4096, 4096)],
    O.Q5_K: [(1, 256), (7, 512), (129, 2048), (2048, 5632), (4096, 4096)],
    O.Q6_K: [(1, 256), (64, 256), (100, 512), (256, 2048), (32000, 2048)],
    O.Q5_0: [(1, 32), (5, 96), (77, 1024), (1024, 2048), (4096, 4096)],
    O.Q4_1: [(1, 32), (9, 160), (65, 1024), (2048, 2048), (4096, 4096)],
    O.Q3_K: [(1, 256), (6, 512), (99, 1024), (2048, 2048), (4096, 4096)],
    O.F16: [(1, 1), (5, 7), (64, 256), (65, 1000), (2048, 2048), (32000, 2048)],
    O.BF16: [(1, 8), (3, 100), (130, 2048), (4096, 4096)],
    O.F32: [(1, 4), (70, 333), (2048, 2048)],
    O.Q1_0: [(1, 128), (7, 384), (130, 2048), (2048, 2048), (4096, 4096)],
    O.Q2_0: [(1, 128), (9, 256), (65, 2048), (2048, 2048), (4096, 4096)],
    O.STQ1_0: [(1, 256), (5, 512), (100, 2048), (2048, 2048), (4096, 4096)],
    O.I2_S: [(1, 128), (3, 256), (64, 640), (129, 2048), (2560, 2560), (6912, 2560)],
}
CASES = [(dt, n, k) for dt, shapes in SHAPES.items() for (n, k) in shapes]


@pytest.mark.parametrize("dt,n,k", CASES)
def test_mm_1d_exact_bit_identical(ctx, dt, n, k):
    note(f"mm_1d exact dtype={dt} n={n} k={k}")
    rng = np.random.default_rng(1000 + dt * 7 + n + k)
    b = make(rng, dt, n, k)
    a = rng.standard_normal(k).astype(F32)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k)
    got = rce_amd.mm_1d(a, w)
    want = O.mm_1d(a, b, dt, n, k)
    assert np.array_equal(bits(got), bits(want)), f"{np.sum(bits(got) != bits(want))} rows differ"
    serial = rce_amd.mm_1d_serial(a, w)
    assert np.array_equal(bits(serial), bits(want))


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4_0, O.Q4_K, O.Q5_K, O.Q6_K, O.Q5_0, O.Q4_1, O.Q3_K, O.F16, O.BF16, O.F32,
                                O.Q1_0, O.Q2_0, O.STQ1_0, O.I2_S])
@pytest.mark.parametrize("t_rows", [2, 8])
def test_mm_batched_exact_bit_identical(ctx, dt, t_rows):
    n, k = (700, 2048) if dt != O.Q4_0 else (11008, 4096)
    note(f"mm_batched exact dtype={dt} t={t_rows} n={n} k={k}")
    rng = np.random.default_rng(2000 + dt + t_rows)
    b = make(rng, dt, n, k)
    x = rng.standard_normal((t_rows, k)).astype(F32)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k)
    got = rce_amd.mm_batched(x, t_rows, w)
    want = O.mm_batched(x, b, dt, n, k)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("dt", [O.F16, O.BF16, O.F32, O.Q6_K])
@pytest.mark.parametrize("n,t_rows", [(4100, 1), (4100, 3), (8200, 1), (8200, 3), (16448, 1)])
def test_row_chain_block_shapes(ctx, dt, n, t_rows):
    """The row-chain kernels (one chain lane per row, helper waves forming the
    addends): F32 / F16 / BF16 take 16, 32 or 64 rows per block by the count
    of 64-row groups times tokens (4100 x 1: 16; 4100 x 3 and 8200 x 1: 32;
    8200 x 3 and 16448 x 1: 64), Q6_K EXACT always 64; each case has a ragged
    last group, and all must equal the reference order bit for bit."""
    k = 256 if dt == O.Q6_K else 200
    note(f"row chain dtype={dt} n={n} t={t_rows} k={k}")
    rng = np.random.default_rng(2500 + dt + n + t_rows)
    b = make(rng, dt, n, k)
    x = rng.standard_normal((t_rows, k)).astype(F32)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k)
    got = rce_amd.mm_batched(x, t_rows, w)
    want = O.mm_batched(x, b, dt, n, k)
    assert np.array_equal(bits(got), bits(want)), f"{np.sum(bits(got) != bits(want))} values differ"


def run_dev(ctx, w, x, mode, a_dtype=G.F32):
    t_rows = x.shape[0]
    xa = rce_amd.DeviceBuffer.from_numpy(ctx, x)
    out = rce_amd.DeviceBuffer(ctx, t_rows * w.n_rows * 4)
    rce_amd.mm_batched_dev(ctx, xa.ptr, a_dtype, t_rows, w, out.ptr, mode)
    ctx.synchronize()
    r = out.download(F32, t_rows * w.n_rows).reshape(t_rows, w.n_rows)
    xa.free(); out.free()
    return r


Q8_CASES = [(O.Q8_0, 4096, 4096), (O.Q4_0, 11008, 4096), (O.Q4_0, 4096, 14336), (O.Q4_K, 4096, 4096),
            (O.Q4_K, 2048, 5632), (O.Q6_K, 32000, 2048), (O.Q4_0, 33, 64), (O.Q4_K, 7, 256), (O.Q6_K, 70, 256),
            (O.Q5_K, 4096, 4096), (O.Q5_K, 2048, 5632), (O.Q5_K, 9, 256), (O.Q5_0, 4096, 4096), (O.Q5_0, 13, 96),
            (O.Q4_1, 4096, 4096), (O.Q4_1, 11, 160), (O.Q3_K, 4096, 4096), (O.Q3_K, 5, 256), (O.F16, 2048, 2048),
            (O.BF16, 70, 96), (O.Q1_0, 300, 2048), (O.Q2_0, 33, 512), (O.STQ1_0, 70, 1024), (O.I2_S, 200, 2560)]


@pytest.mark.parametrize("dt,n,k", Q8_CASES)
@pytest.mark.parametrize("t_rows", [1, 5, 8])
def test_q8_path_bit_identical_to_its_restatement(ctx, dt, n, k, t_rows):
    note(f"q8 dtype={dt} n={n} k={k} t={t_rows}")
    rng = np.random.default_rng(3000 + dt + n + t_rows)
    b = make(rng, dt, n, k)
    x = rng.standard_normal((t_rows, k)).astype(F32)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k)
    got = run_dev(ctx, w, x, Mode.Q8)
    want = O.mm_batched_q8(x, b, dt, n, k)
    assert np.array_equal(bits(got), bits(want))
    # and it is the reference result up to the activation rounding
    ex = O.mm_batched(x, b, dt, n, k)
    assert np.max(np.abs(got - ex)) <= 2e-2 * np.max(np.abs(ex))


MFMA_Q8_CASES = [
    # (dtype, n_rows, n_cols, tokens): the int8 matrix-core form of the Q8
    # path (Q4_0 / Q8_0, K a multiple of 256, 2+ tokens): ragged row tiles
    # (n % 16), one stage (K 256), stage counts around the 4-stage unroll and
    # the 8-stage ring (K 768, 1280, 2304), the configs' K, token tiles of
    # 2, 16, 17 and 40 tokens
    (O.Q4_0, 77, 256, 2), (O.Q8_0, 300, 768, 16), (O.Q4_0, 130, 1280, 17), (O.Q8_0, 64, 2304, 3),
    (O.Q4_0, 11008, 4096, 8), (O.Q8_0, 4096, 4096, 8), (O.Q4_0, 4096, 14336, 40), (O.Q8_0, 33, 4096, 16),
]


@pytest.mark.parametrize("dt,n,k,t_rows", MFMA_Q8_CASES)
def test_q8_matrix_core_form_bit_identical(ctx, monkeypatch, dt, n, k, t_rows):
    """Forced on every case (RCE_QMM_Q8_MFMA=2; by default it runs where it
    is the faster form): the same bits as the Q8 restatement, which the
    decode kernels' form matches above; rows and tokens past the tile ends
    are not stored."""
    monkeypatch.setenv("RCE_QMM_Q8_MFMA", "2")
    note(f"q8 mfma dtype={dt} n={n} k={k} t={t_rows}")
    rng = np.random.default_rng(3100 + dt + n + t_rows)
    b = make(rng, dt, n, k)
    x = rng.standard_normal((t_rows, k)).astype(F32)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k)
    got = run_dev(ctx, w, x, Mode.Q8)
    want = O.mm_batched_q8(x, b, dt, n, k)
    assert np.array_equal(bits(got), bits(want)), f"{np.sum(bits(got) != bits(want))} values differ"
    w.close()


def test_f16_activations_are_widened_exactly(ctx):
    rng = np.random.default_rng(4000)
    n, k, t = 512, 4096, 4
    b = make(rng, O.Q4_K, n, k)
    x16 = rng.standard_normal((t, k)).astype(np.float16)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, O.Q4_K, n, k)
    got = run_dev(ctx, w, x16, Mode.EXACT, a_dtype=G.F16)
    want = O.mm_batched(x16.astype(F32), b, O.Q4_K, n, k)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("dt,n,k", [(O.Q8_0, 40, 256), (O.Q4_0, 70, 512), (O.Q4_K, 33, 1024), (O.Q5_K, 35, 1024),
                                    (O.Q6_K, 130, 512), (O.Q5_0, 21, 96), (O.Q4_1, 19, 160), (O.Q3_K, 17, 512),
                                    (O.F16, 70, 300), (O.BF16, 65, 64), (O.F32, 3, 5), (O.Q1_0, 9, 256),
                                    (O.Q2_0, 10, 384), (O.STQ1_0, 11, 512), (O.I2_S, 12, 384)])
def test_dequant_row_bit_identical(ctx, dt, n, k):
    rng = np.random.default_rng(5000 + dt)
    b = make(rng, dt, n, k)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k)
    rb = O.row_bytes(dt, k)
    for row in (0, 1, n // 2, n - 1):
        got = w.dequant_row(row)
        rowb = b[row * rb:(row + 1) * rb]
        if dt == O.I2_S:  # the row's codes and the tensor's scale
            rowb = np.concatenate([rowb, b[-4:]])
        want = O.dequantize(rowb, dt, k)
        assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("dt", [O.Q4_0, O.Q6_K, O.Q5_0, O.F16])
def test_sub_view_addresses_stacked_experts(ctx, dt):
    # split_experts (rce-qwen36-moe L216-223): sub_view(e*bpe, bpe, rows, cols)
    rng = np.random.default_rng(6000 + dt)
    E, rows, k = 4, 128, 512
    b = make(rng, dt, E * rows, k)
    stack = rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, E * rows, k)
    bpe = b.size // E
    a = rng.standard_normal(k).astype(F32)
    for e in range(E):
        v = stack.sub_view(e * bpe, bpe, rows, k)
        got = rce_amd.mm_1d(a, v)
        want = O.mm_1d(a, b[e * bpe:(e + 1) * bpe], dt, rows, k)
        assert np.array_equal(bits(got), bits(want))
    with pytest.raises(rce_amd.QmmError):
        stack.sub_view(7, bpe, rows, k)            # not on a row boundary
    with pytest.raises(rce_amd.QmmError):
        stack.sub_view(0, b.size + 1, E * rows, k)  # out of bounds


def test_runs_are_bit_identical(ctx):
    rng = np.random.default_rng(7000)
    n, k = 11008, 4096
    b = make(rng, O.Q4_0, n, k)
    x = rng.standard_normal((1, k)).astype(F32)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, O.Q4_0, n, k)
    for mode in (Mode.EXACT, Mode.Q8):
        r1 = run_dev(ctx, w, x, mode)
        r2 = run_dev(ctx, w, x, mode)
        assert np.array_equal(bits(r1), bits(r2))


def test_errors_and_empty_inputs(ctx):
    rng = np.random.default_rng(8000)
    b = make(rng, O.Q4_0, 8, 64)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, O.Q4_0, 8, 64)
    assert rce_amd.mm_batched(np.zeros((0, 64), F32), 0, w).shape == (0, 8)
    with pytest.raises(rce_amd.QmmError) as e:
        rce_amd.QuantWeight.from_owned_bytes(ctx, b[:-1], O.Q4_0, 8, 64)
    assert e.value.status == 2
    with pytest.raises(rce_amd.QmmError) as e:
        rce_amd.QuantWeight.from_owned_bytes(ctx, np.zeros(84, np.uint8), G.Q2K, 1, 256)  # not in mm_1d either
    assert e.value.status == 3
    with pytest.raises(rce_amd.QmmError):
        rce_amd.mm_1d(np.zeros(63, F32), w)


# The largest K each kernel family takes (rce_qmm_supports): 1024 column
# units per row (blocks of 1024 threads), the ternary blocks' 256 units,
# and the row chains' LDS staging (F16: 16 KB values padded to stages;
# Q6_K EXACT: 16384 is the longest row the LDS-staged chains take, longer
# rows read their activations from global memory).
MAX_K = [(O.Q4_0, 48, 32768), (O.Q8_0, 40, 32768), (O.Q5_0, 24, 32768), (O.Q4_K, 24, 65536),
         (O.Q6_K, 70, 65536), (O.Q6_K, 70, 16384), (O.Q3_K, 16, 32768), (O.F16, 80, 16320),
         (O.Q1_0, 24, 32768), (O.STQ1_0, 16, 65536), (O.I2_S, 70, 16384)]


@pytest.mark.parametrize("dt,n,k", MAX_K)
def test_largest_k(ctx, dt, n, k):
    note(f"largest k: dtype={dt} n={n} k={k}")
    assert rce_amd.supports(dt, k)
    rng = np.random.default_rng(9000 + (dt & 0xFF))
    b = make(rng, dt, n, k)
    a = rng.standard_normal(k).astype(F32)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, dt, n, k)
    assert np.array_equal(bits(rce_amd.mm_1d(a, w)), bits(O.mm_1d(a, b, dt, n, k)))
    if rce_amd.supports(dt, k, Mode.Q8):
        x = rng.standard_normal((3, k)).astype(F32)
        assert np.array_equal(bits(run_dev(ctx, w, x, Mode.Q8)), bits(O.mm_batched_q8(x, b, dt, n, k)))
    w.close()
