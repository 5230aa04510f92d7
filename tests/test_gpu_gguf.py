"""GGUF files to device weights (rce_qmm_weight_from_gguf, the
QuantWeight::from_gguf of rce-op-qmm/src/lib.rs L173-209), the TinyLlama
loader (TinyLlamaRuntime::load, rce-tinyllama/src/lib.rs L339-354) and
split_experts (rce-qwen36-moe/src/lib.rs L216-223), on files written by
tests/gguf_writer.py.  A weight read from a file must be the same weight
as the one uploaded from its bytes: products bit-identical."""
import numpy as np
import pytest

import oracle as O
import rce_amd
from rce_amd import GgufFile, Mode, QmmError, QuantWeight
from gguf_writer import STRING, U32, build_gguf, llama_gguf
from llama_case import device_model, make_weights, tiny_cfg
from rand_blocks import float_bytes, rand_blocks, rand_ternary

pytestmark = pytest.mark.gpu


def note(msg):
    print(msg, flush=True)


FORMATS = [(O.Q4_0, 96, 512), (O.Q8_0, 64, 256), (O.Q4_K, 80, 512), (O.Q5_K, 40, 512), (O.Q6_K, 48, 256),
           (O.Q5_0, 24, 96), (O.Q4_1, 24, 160), (O.Q3_K, 24, 512), (O.F16, 70, 100), (O.BF16, 64, 64),
           (O.F32, 3, 16), (O.Q1_0, 20, 256), (O.Q2_0, 20, 384), (O.I2_S, 20, 256)]


@pytest.mark.parametrize("align", [32, 64])
def test_weight_from_gguf_matches_bytes(ctx, align):
    note(f"weight_from_gguf, alignment {align}")
    rng = np.random.default_rng(50 + align)
    tens, keep = [], []
    for dt, n, k in FORMATS:
        b = (rand_blocks(rng, dt, n, k) if dt in (O.Q5_0, O.Q4_1, O.Q3_K)
             else rand_ternary(rng, dt, n, k) if dt in (O.Q1_0, O.Q2_0, O.I2_S)
             else float_bytes(rng, dt, n, k) if dt in (O.F32, O.F16, O.BF16)
             else rce_amd.quantize((rng.standard_normal((n, k)) * 0.05).astype(np.float32), dt))
        tens.append((f"w.{int(dt)}", (k, n), int(dt), bytes(b)))
        keep.append((dt, n, k, b))
    meta = [("general.alignment", U32, align)] if align != 32 else []
    f = GgufFile.parse(build_gguf(meta, tens, alignment=align))
    for dt, n, k, b in keep:
        wf = QuantWeight.from_gguf(ctx, f, f"w.{int(dt)}", n, k)
        wb = QuantWeight.from_owned_bytes(ctx, b, dt, n, k)
        assert (wf.dtype, wf.n_rows, wf.n_cols, wf.len) == (wb.dtype, wb.n_rows, wb.n_cols, wb.len)
        a = rng.standard_normal(k).astype(np.float32)
        assert np.array_equal(rce_amd.mm_1d(a, wf).view(np.uint32), rce_amd.mm_1d(a, wb).view(np.uint32))
        assert np.array_equal(wf.dequant_row(n - 1), wb.dequant_row(n - 1))
        wf.close()
        wb.close()
    f.close()


@pytest.mark.parametrize("arch", ["hunyuan-dense", "llama"])
def test_tag_42_follows_the_architecture(ctx, arch):
    """Tag 42 is STQ1_0 in hunyuan-dense files and Q2_0 otherwise
    (parser.rs L529-541); the file sizes it accordingly and the weight
    computes in that format."""
    note(f"tag 42 in a {arch} file")
    rng = np.random.default_rng(54)
    dt = O.STQ1_0 if arch == "hunyuan-dense" else O.Q2_0
    n, k = 40, 512
    b = rand_ternary(rng, dt, n, k)
    f = GgufFile.parse(build_gguf([("general.architecture", STRING, arch)], [("w", (k, n), 42, bytes(b))]))
    assert f.tensor("w").nbytes == b.size and f.tensor("w").dtype == 42
    w = QuantWeight.from_gguf(ctx, f, "w", n, k)
    assert w.dtype == dt
    a = rng.standard_normal(k).astype(np.float32)
    assert np.array_equal(rce_amd.mm_1d(a, w).view(np.uint32), O.mm_1d(a, b, dt, n, k).view(np.uint32))
    w.close()
    f.close()


def test_weight_from_gguf_errors(ctx):
    note("weight_from_gguf errors")
    b = rce_amd.quantize(np.ones((8, 64), np.float32), O.Q4_0)
    raw = build_gguf([], [("w", (64, 8), int(O.Q4_0), bytes(b)), ("f", (256,), 10, bytes(84))])
    f = GgufFile.parse(raw)
    with pytest.raises(QmmError) as e:
        QuantWeight.from_gguf(ctx, f, "w", 4, 64)  # declared 256 elements, the tensor has 512
    assert e.value.status == 2 and "numel" in str(e.value)
    with pytest.raises(QmmError) as e:
        QuantWeight.from_gguf(ctx, f, "nope", 8, 64)
    assert e.value.status == 8
    with pytest.raises(QmmError) as e:
        QuantWeight.from_gguf(ctx, f, "f", 1, 256)  # Q2_K: not in mm_1d's table
    assert e.value.status == 3
    short = GgufFile.parse(raw[:len(raw) - 130])  # the first tensor's bytes run past the end
    with pytest.raises(QmmError) as e:
        QuantWeight.from_gguf(ctx, short, "w", 8, 64)
    assert e.value.status == 2 and "out of bounds" in str(e.value)
    f.close()
    short.close()


@pytest.mark.parametrize("f16_norms", [False, True])
def test_tinyllama_load_matches_direct(ctx, tmp_path, f16_norms):
    """TinyLlamaRuntime.load(path) == the runtime built from the same
    weights in memory, logits bit for bit (EXACT and Q8)."""
    note(f"TinyLlamaRuntime.load, f16 norms {f16_norms}")
    W = make_weights(tiny_cfg(), seed=51)
    p = tmp_path / "tiny.gguf"
    p.write_bytes(llama_gguf(W, f16_norms=f16_norms))
    if f16_norms:  # the file holds f16 norms: compare with those values
        r16 = lambda v: np.asarray(v, np.float16).astype(np.float32)  # noqa: E731
        W["output_norm"] = r16(W["output_norm"])
        for b in W["blocks"]:
            b["attn_norm"], b["ffn_norm"] = r16(b["attn_norm"]), r16(b["ffn_norm"])
    for mode in (Mode.EXACT, Mode.Q8):
        a = rce_amd.TinyLlamaRuntime.load(ctx, p, mode)
        d = device_model(ctx, W, mode)
        c = W["cfg"]
        for k in ("d_model", "vocab", "n_layers", "n_q_heads", "n_kv_heads", "d_head", "rope_dim", "d_ff",
                  "context_length"):
            assert getattr(a.cfg, k) == c[k], k
        assert np.float32(a.cfg.eps) == np.float32(c["eps"])  # stored as F32 in the file
        for t in (3, 100, 7, 319):
            la, ld = a.forward_logits(t), d.forward_logits(t)
            assert np.array_equal(la.view(np.uint32), ld.view(np.uint32))
        a.close()
        d.close()


def test_tinyllama_load_missing_tensor(ctx, tmp_path):
    note("TinyLlamaRuntime.load, a missing tensor")
    W = make_weights(tiny_cfg(n_layers=1), seed=52)
    raw = llama_gguf(W)
    p = tmp_path / "bad.gguf"
    p.write_bytes(raw.replace(b"blk.0.ffn_up.weight", b"blk.0.ffn_XX.weight"))
    with pytest.raises(QmmError) as e:
        rce_amd.TinyLlamaRuntime.load(ctx, p)
    assert e.value.status == 8 and "blk.0.ffn_up.weight" in str(e.value)


def test_split_experts(ctx):
    """A stacked [n_expert, rows, cols] Q4_0 tensor (dims ne0 first: cols,
    rows, n_expert) loaded as one weight and split per expert equals each
    expert uploaded on its own."""
    note("split_experts")
    E, n, k = 4, 64, 256
    rng = np.random.default_rng(53)
    per = [rce_amd.quantize((rng.standard_normal((n, k)) * 0.05).astype(np.float32), O.Q4_0) for _ in range(E)]
    stacked = b"".join(bytes(b) for b in per)
    f = GgufFile.parse(build_gguf([("general.architecture", STRING, "qwen3moe")],
                                  [("blk.0.ffn_gate_exps.weight", (k, n, E), int(O.Q4_0), stacked)]))
    full = QuantWeight.from_gguf(ctx, f, "blk.0.ffn_gate_exps.weight", E * n, k)
    views = rce_amd.split_experts(full, E, n, k)
    a = rng.standard_normal(k).astype(np.float32)
    for e in range(E):
        own = QuantWeight.from_owned_bytes(ctx, per[e], O.Q4_0, n, k)
        assert (views[e].n_rows, views[e].n_cols) == (n, k)
        assert np.array_equal(rce_amd.mm_1d(a, views[e]).view(np.uint32), rce_amd.mm_1d(a, own).view(np.uint32))
        own.close()
    with pytest.raises(ValueError):  # the bytes do not divide by the expert count
        rce_amd.split_experts(full, 5, n, k)
    with pytest.raises(QmmError):  # they divide, but the views would cut rows (sub_view rejects them)
        rce_amd.split_experts(full, 3, n, k)
    f.close()
