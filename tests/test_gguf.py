"""GGUF parsing through the C ABI (rce_qmm_gguf_*; host code, no GPU).

The reference's parser tests (rce-ingest-gguf/src/parser.rs L699-969:
minimal header, bad magic, bad version, string / u32 / array metadata,
tensor infos, truncated input, dimension limit, version 2, the llama /
mistral accessors) restated on files from tests/gguf_writer.py, plus what
they leave open: every value type, the data-section alignment (default,
general.alignment as U32 / U64, the first entry wins), tag 42's two sizes,
tensor_byte_size's known answers (dequant.rs L719-745, quant.rs L295),
every truncation of a valid file failing cleanly, read_tensor_f32 of F32 /
F16 / BF16 against numpy, and TinyLlamaConfig::from_gguf's defaults
(rce-tinyllama/src/lib.rs L44-89).
"""
import struct

import numpy as np
import pytest

import rce_amd
from rce_amd import GgufFile, QmmError
from gguf_writer import (ARRAY, BOOL, F32, F64, I8, I16, I32, I64, STRING, U8, U16, U32, U64, build_gguf,
                         build_test_gguf, enc_value, llama_gguf)

PARSE_ERROR, NOT_FOUND, IO_ERROR, BAD_SHAPE, UNSUPPORTED = 9, 8, 10, 2, 3


def parse(b):
    return GgufFile.parse(b)


def parse_error(b) -> str:
    with pytest.raises(QmmError) as e:
        GgufFile.parse(b)
    assert e.value.status == PARSE_ERROR
    return str(e.value)


def test_minimal_header():
    f = parse(build_test_gguf([], []))
    assert f.version == 3 and f.metadata == [] and f.tensors == []
    assert f.alignment == 32 and f.data_offset == 32  # 24 header bytes padded to 32


def test_invalid_magic():
    b = bytearray(build_test_gguf([], []))
    b[0] = 0
    assert "invalid magic" in parse_error(bytes(b))


@pytest.mark.parametrize("v,ok", [(99, False), (1, False), (4, False), (2, True), (3, True)])
def test_versions(v, ok):
    b = build_test_gguf([], [], version=v)
    if ok:
        assert parse(b).version == v
    else:
        assert f"unsupported version {v}" in parse_error(b)


def test_string_u32_array_metadata():
    f = parse(build_test_gguf([("general.architecture", STRING, "llama"), ("llama.block_count", U32, 32),
                               ("test.array", ARRAY, (U32, [100, 200, 300]))], []))
    assert [m.key for m in f.metadata] == ["general.architecture", "llama.block_count", "test.array"]
    assert f.architecture() == "llama"
    assert f.metadata[1].value == rce_amd.GgufValue(U32, 32)
    arr = f.get_metadata("test.array")
    assert arr.type == ARRAY and [v.value for v in arr.value] == [100, 200, 300]
    assert all(v.type == U32 for v in arr.value)


def test_every_value_type_round_trips():
    vals = [("u8", U8, 250), ("i8", I8, -7), ("u16", U16, 65000), ("i16", I16, -30000), ("u32", U32, 4000000000),
            ("i32", I32, -2000000000), ("f32", F32, 1.5), ("bool", BOOL, True), ("str", STRING, "héllo ✓"),
            ("u64", U64, 2 ** 63 + 5), ("i64", I64, -2 ** 62), ("f64", F64, -2.25),
            ("strs", ARRAY, (STRING, ["a", "", "ßxy"])),
            ("nested", ARRAY, (ARRAY, [(I16, [1, -2]), (I16, []), (I16, [3])])),
            ("empty", ARRAY, (F32, []))]
    f = parse(build_test_gguf(vals, []))
    got = {m.key: m.value for m in f.metadata}
    for key, t, v in vals:
        assert got[key].type == t
        if t != ARRAY:
            assert got[key].value == v
    assert [x.value for x in got["strs"].value] == ["a", "", "ßxy"]
    assert [[y.value for y in x.value] for x in got["nested"].value] == [[1, -2], [], [3]]
    assert got["empty"].value == []
    assert f.get_u32("u32") == 4000000000 and f.get_u64("u64") == 2 ** 63 + 5 and f.get_u32("u64") is None


def test_tensor_infos_and_sizes():
    f = parse(build_test_gguf([], [("token_embd.weight", (4096, 32000), 1, 0),
                                   ("blk.0.attn_q.weight", (4096, 4096), 12, 65536),
                                   ("blk.0.ffn_gate.weight", (4096, 11008), 14, 131072),
                                   ("output_norm.weight", (4096,), 0, 0)]))
    t = f.tensors
    assert [x.name for x in t] == ["token_embd.weight", "blk.0.attn_q.weight", "blk.0.ffn_gate.weight",
                                   "output_norm.weight"]
    assert t[1].dims == (4096, 4096) and t[1].dtype == 12 and t[1].offset == 65536
    assert t[1].numel() == 4096 * 4096
    assert t[0].nbytes == 4096 * 32000 * 2                  # F16
    assert t[1].nbytes == 4096 * 4096 // 256 * 144         # Q4_K
    assert t[2].nbytes == 4096 * 11008 // 256 * 210        # Q6_K
    assert t[3].nbytes == 4096 * 4                          # F32


@pytest.mark.parametrize("tag,n,want", [
    (12, 256, 144), (12, 512, 288),   # tensor_byte_size_q4_k (dequant.rs L719)
    (2, 32, 18), (8, 32, 34),         # estimated_bytes_q4_0 = 18 (quant.rs L295); Q8_0 block
    (2, 33, 36),                      # partial blocks round up
    (3, 32, 20), (6, 32, 22), (7, 32, 24), (9, 32, 36), (10, 256, 84), (11, 256, 110), (13, 256, 176),
    (14, 256, 210), (30, 5, 10), (28, 3, 24), (24, 7, 7), (25, 7, 14), (26, 7, 28), (27, 7, 56),
    (36, 9, 3 + 4),                   # I2_S: ceil(n/4) bytes + a 4-byte scale
    (41, 128, 18), (42, 128, 34),     # Q1_0; tag 42 as PrismML Q2_0
    (20, 256, 0),                     # IQ4_NL: no size rule (0, as the reference)
])
def test_tensor_byte_size(tag, n, want):
    f = parse(build_test_gguf([], [("t", (n,), tag, 0)]))
    assert f.tensors[0].nbytes == want


def test_tag42_is_stq1_in_hunyuan_dense():
    f = parse(build_test_gguf([("general.architecture", STRING, "hunyuan-dense")], [("t", (512,), 42, 0)]))
    assert f.tensors[0].dtype == 42 and f.tensors[0].nbytes == 2 * 42  # STQ1_0: 42 B per 256


def test_data_offset_alignment():
    base = [("general.name", STRING, "x")]
    n0 = len(build_test_gguf(base, []))
    f = parse(build_test_gguf(base, []))
    assert f.data_offset == (n0 + 31) // 32 * 32
    for t in (U32, U64):
        meta = base + [("general.alignment", t, 64)]
        n = len(build_test_gguf(meta, []))
        f = parse(build_test_gguf(meta, []))
        assert f.alignment == 64 and f.data_offset == (n + 63) // 64 * 64
    meta = base + [("general.alignment", STRING, "64")]  # not U32/U64: the default
    assert parse(build_test_gguf(meta, [])).alignment == 32
    meta = base + [("general.alignment", U16, 64), ("general.alignment", U32, 128)]  # the first entry decides
    assert parse(build_test_gguf(meta, [])).alignment == 32
    assert "general.alignment is 0" in parse_error(build_test_gguf([("general.alignment", U32, 0)], []))


def test_truncation_eof_and_limits():
    assert "unexpected end of input at offset 4" in parse_error(b"GGUF")
    good = build_gguf([("general.architecture", STRING, "llama"), ("a", ARRAY, (STRING, ["x", "yz"]))],
                      [("w", (32, 2), 2, bytes(36))])
    parse(good)
    # every strict prefix that cuts the header, metadata or infos fails cleanly
    head = len(build_test_gguf([("general.architecture", STRING, "llama"), ("a", ARRAY, (STRING, ["x", "yz"]))],
                               [("w", (32, 2), 2, 0)]))
    for cut in range(head):
        parse_error(good[:cut])
    # counts larger than the input
    parse_error(b"GGUF" + struct.pack("<IQQ", 3, 0, 2 ** 62))
    parse_error(b"GGUF" + struct.pack("<IQQ", 3, 2 ** 62, 0))
    parse_error(build_test_gguf([("big", ARRAY, struct.pack("<IQ", U8, 2 ** 62))], []))


def test_too_many_dimensions():
    b = b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + enc_value(STRING, "bad") + struct.pack("<I", 9)
    assert "tensor dimension count 9 exceeds maximum (8)" in parse_error(b)


def test_bad_utf8_and_unknown_type():
    b = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 2) + b"\xc3\x28" + struct.pack("<I", U8) + b"\x01"
    assert "invalid utf-8" in parse_error(b)
    assert "unknown metadata value type tag 13" in parse_error(build_test_gguf([("k", 13, b"")], []))
    assert "unknown metadata value type tag 77" in parse_error(
        build_test_gguf([("k", ARRAY, struct.pack("<IQ", 77, 1))], []))


def test_full_model_header_and_accessors():
    meta = [("general.architecture", STRING, "llama"), ("general.name", STRING, "LLaMA-7B-Q4_K_M"),
            ("llama.block_count", U32, 32), ("llama.embedding_length", U32, 4096),
            ("llama.attention.head_count", U32, 32)]
    tens = [("token_embd.weight", (4096, 32000), 1, 0), ("output_norm.weight", (4096,), 0, 0),
            ("output.weight", (4096, 32000), 12, 0)]
    for blk in range(2):
        for n, d, t in (("attn_q", (4096, 4096), 12), ("attn_k", (4096, 4096), 12), ("attn_v", (4096, 4096), 12),
                        ("attn_output", (4096, 4096), 12), ("ffn_gate", (4096, 11008), 12),
                        ("ffn_up", (4096, 11008), 12), ("ffn_down", (11008, 4096), 12), ("attn_norm", (4096,), 0),
                        ("ffn_norm", (4096,), 0)):
            tens.append((f"blk.{blk}.{n}.weight", d, t, 0))
    f = parse(build_test_gguf(meta, tens))
    assert f.architecture() == "llama" and f.model_name() == "LLaMA-7B-Q4_K_M"
    assert f.block_count() == 32 and f.embedding_length() == 4096 and f.head_count() == 32
    assert f.head_count_kv() is None and len(f.tensors) == 3 + 2 * 9
    g = parse(build_test_gguf([("general.architecture", STRING, "mistral"), ("mistral.block_count", U32, 32),
                               ("mistral.attention.head_count_kv", U32, 8)], []))
    assert g.block_count() == 32 and g.head_count_kv() == 8


def test_read_tensor_f32():
    rng = np.random.default_rng(0)
    a = rng.standard_normal(37).astype(np.float32)
    h = np.array([0.0, -0.0, 1.0, 65504.0, 6e-8, -2.0 ** -24, np.inf, -np.inf, 0.333], np.float16)
    bf = (rng.standard_normal(11).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    q = bytes(18 * 2)
    f = parse(build_gguf([], [("a", (37,), 0, a.tobytes()), ("h", (9,), 1, h.tobytes()),
                              ("bf", (11,), 30, bf.tobytes()), ("q", (64,), 2, q)]))
    assert np.array_equal(f.read_tensor_f32("a").view(np.uint32), a.view(np.uint32))
    assert np.array_equal(f.read_tensor_f32("h"), h.astype(np.float32))
    assert np.array_equal(f.read_tensor_f32("h").view(np.uint32), h.astype(np.float32).view(np.uint32))  # -0.0
    assert np.array_equal(f.read_tensor_f32("bf").view(np.uint32), bf.astype(np.uint32) << 16)
    with pytest.raises(QmmError) as e:
        f.read_tensor_f32("q")
    assert e.value.status == UNSUPPORTED
    with pytest.raises(QmmError) as e:
        f.read_tensor_f32("nope")
    assert e.value.status == NOT_FOUND
    L = rce_amd._lib.lib()
    out = np.empty(36, np.float32)
    assert L.rce_qmm_gguf_read_f32(f.handle, b"a", out.ctypes.data, 36) == BAD_SHAPE


def test_read_out_of_bounds_tensor():
    """A tensor whose bytes run past the end of the file (QuantWeight::from_gguf's check)."""
    b = build_gguf([], [("a", (8,), 0, bytes(32))])
    f = parse(b[:-4])
    with pytest.raises(QmmError) as e:
        f.read_tensor_f32("a")
    assert e.value.status == BAD_SHAPE and "out of bounds" in str(e.value)
    f2 = parse(build_test_gguf([], [("far", (8,), 0, 2 ** 63)]))
    with pytest.raises(QmmError):
        f2.read_tensor_f32("far")


def test_find_and_open(tmp_path):
    b = build_gguf([("general.architecture", STRING, "llama")], [("w", (32, 4), 8, bytes(34 * 4))])
    p = tmp_path / "m.gguf"
    p.write_bytes(b)
    with GgufFile.open(p) as f:
        assert f.architecture() == "llama" and f.tensors[0].nbytes == 136
        L = rce_amd._lib.lib()
        import ctypes
        idx = ctypes.c_size_t()
        assert L.rce_qmm_gguf_find_tensor(f.handle, b"w", ctypes.byref(idx)) == 0 and idx.value == 0
        assert L.rce_qmm_gguf_find_tensor(f.handle, b"x", ctypes.byref(idx)) == NOT_FOUND
        assert L.rce_qmm_gguf_find_metadata(f.handle, b"general.architecture", ctypes.byref(idx)) == 0
        assert L.rce_qmm_gguf_find_metadata(f.handle, b"nope", ctypes.byref(idx)) == NOT_FOUND
    with pytest.raises(QmmError) as e:
        GgufFile.open(tmp_path / "missing.gguf")
    assert e.value.status == IO_ERROR
    empty = tmp_path / "empty.gguf"
    empty.write_bytes(b"")
    with pytest.raises(QmmError) as e:
        GgufFile.open(empty)
    assert e.value.status == PARSE_ERROR


def test_tinyllama_config_from_gguf():
    from llama_case import make_weights, tiny_cfg
    W = make_weights(tiny_cfg(), seed=40)
    f = parse(llama_gguf(W))
    cfg = rce_amd.TinyLlamaConfig.from_gguf(f)
    c = W["cfg"]
    for k in ("d_model", "vocab", "n_layers", "n_q_heads", "n_kv_heads", "d_head", "rope_dim", "d_ff",
              "context_length"):
        assert getattr(cfg, k) == c[k], k
    assert cfg.rope_freq_base == c["rope_freq_base"] and cfg.eps == np.float32(c["eps"])
    # defaults and fallbacks: kv heads = q heads, rope_dim = d_head, base 1e4,
    # context 2048, eps 1e-5, vocab from token_embd.weight's second dimension
    meta = [("general.architecture", STRING, "llama"), ("llama.embedding_length", U32, 256),
            ("llama.block_count", U32, 2), ("llama.attention.head_count", U32, 4),
            ("llama.feed_forward_length", U32, 512)]
    g = parse(build_test_gguf(meta, [("token_embd.weight", (256, 320), 12, 0)]))
    d = rce_amd.TinyLlamaConfig.from_gguf(g)
    assert (d.vocab, d.n_kv_heads, d.d_head, d.rope_dim, d.rope_freq_base, d.context_length) == \
        (320, 4, 64, 64, 10000.0, 2048)
    assert d.eps == pytest.approx(1e-5)
    for bad, msg in ((meta[1:], "missing general.architecture"),
                     ([("general.architecture", STRING, "gpt2")] + meta[1:], "expected llama, got gpt2"),
                     (meta[:1] + meta[2:], "embedding_length")):
        with pytest.raises(QmmError, match=msg):
            rce_amd.TinyLlamaConfig.from_gguf(parse(build_test_gguf(bad, [("token_embd.weight", (256, 320), 12, 0)])))


def test_mutated_files_never_crash():
    """Seeded mutations of a valid file (byte flips, count and length
    fields overwritten, truncations, splices) either parse or return a
    status: the parser bounds-checks every read."""
    good = build_gguf([("general.architecture", STRING, "llama"), ("arr", ARRAY, (STRING, ["ab", "c"])),
                       ("n", ARRAY, (ARRAY, [(U32, [1, 2]), (U8, [3])])), ("general.alignment", U32, 32)],
                      [("w", (32, 2), 2, bytes(36)), ("v", (4,), 0, bytes(16))])
    rng = np.random.default_rng(1234)
    ok = bad = 0
    for _ in range(3000):
        b = bytearray(good)
        kind = rng.integers(0, 4)
        if kind == 0:
            for _ in range(int(rng.integers(1, 4))):
                b[int(rng.integers(0, len(b)))] = int(rng.integers(0, 256))
        elif kind == 1:  # a u64 field somewhere set to a huge value
            i = int(rng.integers(0, len(b) - 8))
            big = [2 ** 63, 2 ** 40, 2 ** 64 - 1, 12345][int(rng.integers(0, 4))]
            b[i:i + 8] = struct.pack("<Q", big)
        elif kind == 2:
            b = b[:int(rng.integers(0, len(b)))]
        else:
            i, j = sorted(int(x) for x in rng.integers(0, len(b), 2))
            b = b[:i] + b[j:]
        try:
            f = GgufFile.parse(bytes(b))
            for t in f.tensors:
                if t.dtype in (0, 1, 30):
                    try:
                        f.read_tensor_f32(t.name)
                    except QmmError:
                        pass
            ok += 1
        except QmmError as e:
            assert e.status == PARSE_ERROR
            bad += 1
    assert ok > 100 and bad > 100
