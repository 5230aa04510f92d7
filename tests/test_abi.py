"""The C-ABI library loads, exports every symbol include/rce_qmm.h declares,
and its host-only logic behaves (no GPU needed)."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle as O
import rce_amd
from rce_amd import _lib
from conftest import ROOT, gpu_available

HEADER = os.path.join(ROOT, "include", "rce_qmm.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rce_qmm_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), f"{n} missing from {_lib.LIB_PATH}"
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures drift from the header"


def test_abi_version_and_status_strings():
    L = _lib.lib()
    assert L.rce_qmm_abi_version() == 2
    assert L.rce_qmm_status_str(0) == b"ok"
    assert L.rce_qmm_status_str(3) == b"unsupported dtype"
    assert L.rce_qmm_status_str(8) == b"not found"
    assert L.rce_qmm_status_str(9) == b"parse error"
    assert L.rce_qmm_status_str(10) == b"i/o error"


def test_supports_matrix():
    G, M = rce_amd.GgufDtype, rce_amd.Mode
    assert rce_amd.supports(G.Q4_0, 4096) and rce_amd.supports(G.Q8_0, 4096)
    assert rce_amd.supports(G.Q4K, 4096) and rce_amd.supports(G.Q6K, 2048)
    assert rce_amd.supports(G.Q4_0, 4096, M.Q8)
    assert not rce_amd.supports(G.Q4_0, 4100)        # not a block multiple
    assert not rce_amd.supports(G.Q4K, 4096 + 32)     # K-quants need 256
    assert rce_amd.supports(G.Q5K, 4096) and rce_amd.supports(G.Q5K, 4096, M.Q8)
    assert rce_amd.supports(G.Q5_0, 96) and rce_amd.supports(G.Q4_1, 4096, M.Q8)
    assert rce_amd.supports(G.Q3K, 4096) and rce_amd.supports(G.Q3K, 512, M.Q8)
    assert not rce_amd.supports(G.Q3K, 4096 + 32)     # K-quants need 256
    assert not rce_amd.supports(G.Q2K, 4096)          # not in mm_1d's table either: reported unsupported
    for dt, k in ((G.Q1_0, 2048), (G.Q2_0, 2048), (G.STQ1_0, 2560), (G.I2S, 2560), (G.F16, 7), (G.BF16, 100)):
        assert rce_amd.supports(dt, k) and rce_amd.supports(dt, k, M.Q8)
    assert not rce_amd.supports(G.Q1_0, 2048 + 32) and not rce_amd.supports(G.I2S, 2560 + 64)
    assert G.STQ1_0.to_u32() == 42 and G.from_u32(42) is G.Q2_0
    assert not rce_amd.supports(99, 4096)


@pytest.mark.skipif(gpu_available(), reason="checks the no-device path")
def test_context_without_device_reports_no_device():
    with pytest.raises(rce_amd.QmmError) as e:
        rce_amd.Context(0)
    assert e.value.status == 4


def test_null_arguments_are_rejected():
    L = _lib.lib()
    assert L.rce_qmm_context_create(0, None) == 1
    assert L.rce_qmm_mm_1d(None, None, None, None) == 1
    assert L.rce_qmm_weight_from_bytes(None, 2, 1, 32, None, 18, None) == 1
    assert b"null" in L.rce_qmm_last_error()


def test_moe_router_matches_oracle_bit_for_bit():
    # Host-side router of the library vs the oracle's restatement of
    # rce-op-moe moe_router (both take exp from the platform libm).
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((256, 8)).astype(np.float32)
    ids, w = rce_amd.moe_router(logits, 2, True)
    for t in range(256):
        oi, ow = O.moe_router(logits[t], 2, True)
        assert list(ids[t]) == list(oi)
        assert np.array_equal(w[t].view(np.uint32), ow.view(np.uint32))
    ids1, w1 = rce_amd.moe_router(logits[:4], 3, False)
    for t in range(4):
        oi, ow = O.moe_router(logits[t], 3, False)
        assert list(ids1[t]) == list(oi) and np.array_equal(w1[t], ow)


def test_moe_router_rejects_bad_top_k():
    with pytest.raises(rce_amd.QmmError):
        rce_amd.moe_router(np.zeros((1, 4), np.float32), 5)


@pytest.mark.gpu
def test_size_checks_do_not_wrap(ctx):
    """Shape arguments whose products or sums overflow size_t are refused
    before any copy (the reference's slices would panic): n_rows * row_bytes
    wrapping to the buffer's length, and sub-views whose offset + length or
    n_rows * row_bytes wrap."""
    L = _lib.lib()
    SMAX = (1 << 64) - 1
    buf = np.zeros(64, np.uint8)
    out = ctypes.c_void_p()
    # Q4_0, 32 columns: 18 bytes per row; 2^64 / 18 + 1 rows wrap to 8 bytes
    n = (1 << 64) // 18 + 1
    wrapped = (n * 18) % (1 << 64)
    assert wrapped < 64
    st = L.rce_qmm_weight_from_bytes(ctx.handle, 2, n, 32, buf.ctypes.data, wrapped, ctypes.byref(out))
    assert st == 2 and not out.value
    rng = np.random.default_rng(3)
    b = O.quantize((rng.standard_normal((8, 64)) * 0.02).astype(np.float32), O.Q4_0)
    w = rce_amd.QuantWeight.from_owned_bytes(ctx, b, O.Q4_0, 8, 64)
    v = ctypes.c_void_p()
    assert L.rce_qmm_weight_sub_view(w.handle, SMAX - 5, 36, 1, 64, ctypes.byref(v)) == 2  # offset + len wraps
    assert L.rce_qmm_weight_sub_view(w.handle, 36, SMAX, 1, 64, ctypes.byref(v)) == 2
    n = (1 << 64) // 36 + 1  # n_rows * 36 wraps to 20
    assert L.rce_qmm_weight_sub_view(w.handle, 0, (n * 36) % (1 << 64), n, 64, ctypes.byref(v)) == 2
    assert not v.value
    assert L.rce_qmm_weight_sub_view(w.handle, 36, 72, 2, 64, ctypes.byref(v)) == 0  # a good view still works
    L.rce_qmm_weight_destroy(v)
    w.close()
