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


def scale_pairs(b, dt, n, k):
    """The nibble GEMM's binary16 {scale, bias} pairs restated from the GGUF
    bytes (rce-op-qmm/src/lib.rs L719-728 get_scale_min; dequant.rs L658-701
    for Q6_K): Q4_K / Q5_K sub-block j: {f16(d sc_j), f16(-(dmin m_j))};
    Q6_K scale j: {s = f16(d sc_j), f16(-32 s)}; [row][super-block][pair]
    as uint16 pairs."""
    nsb = k // 256
    bs = {O.Q4_K: 144, O.Q5_K: 176, O.Q6_K: 210}[dt]
    blk = np.frombuffer(bytes(b), np.uint8).reshape(n, nsb, bs)
    f16 = lambda a: a.copy().view(np.float16)[..., 0].astype(np.float32)  # noqa: E731
    if dt == O.Q6_K:
        d = f16(blk[:, :, 208:210])
        sc = blk[:, :, 192:208].view(np.int8).astype(np.float32)
        s = (d[:, :, None] * sc).astype(np.float16)
        bias = (np.float32(-32.0) * s.astype(np.float32)).astype(np.float16)
    else:
        d, dmin = f16(blk[:, :, 0:2]), f16(blk[:, :, 2:4])
        q = blk[:, :, 4:16].astype(np.int32)
        sc = np.zeros((n, nsb, 8), np.int32)
        m = np.zeros((n, nsb, 8), np.int32)
        for j in range(8):
            if j < 4:
                sc[:, :, j], m[:, :, j] = q[:, :, j] & 63, q[:, :, j + 4] & 63
            else:
                sc[:, :, j] = (q[:, :, j + 4] & 0x0F) | ((q[:, :, j - 4] >> 6) << 4)
                m[:, :, j] = (q[:, :, j + 4] >> 4) | ((q[:, :, j] >> 6) << 4)
        s = (d[:, :, None] * sc.astype(np.float32)).astype(np.float16)
        bias = (-(dmin[:, :, None] * m.astype(np.float32))).astype(np.float16)
    return np.stack([s.view(np.uint16), bias.view(np.uint16)], axis=-1)


@pytest.mark.parametrize("dt,n,k", [(O.Q4_K, 20, 1024), (O.Q5_K, 70, 512), (O.Q6_K, 130, 768)])
def test_upload_scale_pairs(harness, tmp_path, dt, n, k):
    """The pairs the upload adds to the Q4_K / Q5_K / Q6_K device layouts
    for the matrix-core GEMM equal their restatement from the file's bytes,
    bit for bit (a wrong sub-block index, a swapped scale / min or a
    rounding of the product in binary16 steps fails here)."""
    rng = np.random.default_rng(1300 + dt + n)
    b = weight_bytes(rng, dt, n, k)
    src, dst = tmp_path / "w.bin", tmp_path / "p.bin"
    b.tofile(src)
    subprocess.run([harness, "pairs", str(dt), str(n), str(k), str(src), str(dst)], check=True)
    nsb, npr = k // 256, 16 if dt == O.Q6_K else 8
    got = np.fromfile(dst, np.uint16).reshape(n, nsb, npr, 2)
    want = scale_pairs(b, dt, n, k)
    assert np.array_equal(got, want)
    assert np.any(got[..., 1] != 0)  # the biases are not all zero


def replay(ops, nchunks):
    """Check one printed schedule of gen_pipeline: every chunk is multiplied
    once, in order, from an LDS buffer that holds it and was stored before
    the last barrier; a store writes the register set that holds its chunk
    into a buffer no wave reads after the last barrier; a load never
    overwrites a register set whose chunk is not yet stored."""
    regs = {}        # slot -> (chunk, stored?)
    bufs = {}        # buf -> (chunk, epoch stored)
    read_epoch = {}  # buf -> epoch of its last read
    epoch, nxt, depth, cpb = 0, 0, None, None
    for line in ops:
        f = line.split()
        if f[0] == "S":
            epoch += 1
        elif f[0] == "L":
            slot, ch = int(f[1]), int(f[2])
            assert 0 <= ch < nchunks, line
            if slot in regs and regs[slot][0] >= nxt:
                assert regs[slot][1], f"load over unstored chunk {regs[slot][0]}: {line}"
            regs[slot] = (ch, False)
        elif f[0] == "T":
            slot, ch, buf = int(f[1]), int(f[2]), int(f[3])
            assert regs.get(slot, (None,))[0] == ch, f"register set {slot} does not hold chunk {ch}"
            assert read_epoch.get(buf, -1) < epoch, f"store into buffer {buf} read in this epoch: {line}"
            regs[slot] = (ch, True)
            bufs[buf] = (ch, epoch)
        elif f[0] == "M":
            ch, buf = int(f[1]), int(f[2])
            assert ch == nxt, f"chunk {ch} multiplied, {nxt} expected"
            held, when = bufs.get(buf, (None, None))
            assert held == ch, f"buffer {buf} holds chunk {held}, not {ch}"
            assert when < epoch, "multiplied before a barrier after its store"
            read_epoch[buf] = epoch
            nxt += 1
        elif f[0] == "E":
            depth, cpb = int(f[1]), int(f[2])
    assert nxt == nchunks, f"{nxt} of {nchunks} chunks multiplied"
    return depth, cpb


def test_generic_gemm_chunk_schedule(harness):
    """The kernel's own pipeline function, replayed for 1..64 chunks (K 64 ..
    4096): every residue of the load ring and the barrier pairs, including
    K/64 = 7, 13, 19, ... where DEPTH + 1 chunks are left for the tail."""
    for nchunks in range(1, 65):
        out = subprocess.run([harness, "sched", str(nchunks)], check=True, capture_output=True, text=True).stdout
        depth, cpb = replay(out.split("\n")[:-1], nchunks)
        assert depth and cpb


def test_schedule_replay_catches_a_stale_tail():
    """The replay itself fails the schedule the tail had before it loaded
    the chunks past c + DEPTH - 1 (7 chunks, DEPTH 6, CPB 2): chunk 6 is
    stored from the register set that still holds chunk 0."""
    ops = ["L %d %d" % (u, u) for u in range(6)] + ["T 0 0 0", "T 1 1 1"]
    ops += ["S", "M 0 0", "M 1 1", "T 2 2 2", "T 3 3 3",
            "S", "M 2 2", "M 3 3", "T 4 4 0", "T 5 5 1",
            "S", "M 4 0", "M 5 1", "T 0 6 2"]
    with pytest.raises(AssertionError, match="does not hold chunk 6"):
        replay(ops, 7)
