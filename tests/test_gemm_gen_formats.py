"""The generic prefill GEMM's weight forms, checked on the host (no GPU).

gemm_gen.hip's per-format policies (load: the raw bytes of 8 consecutive
weights from the format's device layout; dequant: the binary16 weights) are
compiled for the host by tests/gemm_gen_host.hip and run over a weight laid
out by the library's own relayout (plan_layout + relayout_host, as the
upload does).  Every weight must equal the oracle's f32 dequantized value
(rce-ingest-gguf dequant.rs, restated in oracle/qmm_oracle.c) rounded once
to binary16; a zero may carry the other sign (the kernels form (q - c) * d
as one fma, whose exact zero is +0).  A wrong plane, byte offset, nibble
half, fifth-bit or qh position, scale index or Q6_K quadrant fails here."""
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle as O
from rand_blocks import float_bytes, rand_blocks

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    from rce_amd import build as B
    lib = os.path.join(ROOT, "rce_amd", "lib", "librce_qmm.so")
    try:
        cc = B.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    if not os.path.exists(lib):
        pytest.skip("librce_qmm.so not built")
    exe = str(tmp_path_factory.mktemp("gg") / "gemm_gen_host")
    r = subprocess.run([cc, *B.FLAGS, os.path.join(HERE, "gemm_gen_host.hip"), "-L", os.path.dirname(lib),
                        "-lrce_qmm", f"-Wl,-rpath,{os.path.dirname(lib)}", "-o", exe],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


def weight_bytes(rng, dt, n, k):
    if dt == O.F16:
        return float_bytes(rng, dt, n, k, 0.02)
    if dt in (O.Q5_0, O.Q4_1):
        return rand_blocks(rng, dt, n, k, dmax=0.02 / 8)
    return O.quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32), dt)


# ragged rows (N not a multiple of the 64-row groups of the IL64 layouts),
# several super-blocks, both halves of every 64-group
CASES = [(O.Q8_0, 70, 576), (O.Q5_0, 33, 1024), (O.Q4_1, 20, 1088), (O.Q4_0, 20, 512), (O.F16, 100, 640),
         (O.Q5_K, 70, 512), (O.Q4_K, 20, 1024), (O.Q6_K, 130, 768)]


@pytest.mark.parametrize("dt,n,k", CASES)
def test_generic_gemm_weights_are_the_reference_values_in_binary16(harness, tmp_path, dt, n, k):
    rng = np.random.default_rng(900 + dt + n)
    b = weight_bytes(rng, dt, n, k)
    src, dst = tmp_path / "w.bin", tmp_path / "h.bin"
    b.tofile(src)
    subprocess.run([harness, str(dt), str(n), str(k), str(src), str(dst)], check=True)
    got = np.fromfile(dst, np.uint16).reshape(n, k)
    want = O.dequantize(b, dt, n * k).reshape(n, k).astype(np.float16).view(np.uint16)
    both_zero = ((got | want) & 0x7FFF) == 0
    assert np.array_equal(got[~both_zero], want[~both_zero])
    assert got.max() != 0  # not an all-zero output
