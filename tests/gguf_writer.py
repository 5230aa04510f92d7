"""GGUF v2/v3 bytes for the tests: header, metadata, tensor infos and
(build_gguf) the aligned tensor-data section, in the layout GgufFile::parse
reads (rce-ingest-gguf/src/parser.rs L446-551; the reference's own fixture
builders are build_test_gguf / build_gguf, L617-697).  Values are encoded
from (type tag, python value); tensors name their GGUF dtype tag and dims
ne0 first."""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", U64: "<Q", I64: "<q",
        F64: "<d"}


def enc_string(s) -> bytes:
    b = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def enc_value(t: int, v) -> bytes:
    """A value of type t: scalars, strings, and arrays as (elem_type, [values])."""
    if t in _FMT:
        return struct.pack(_FMT[t], v)
    if t == BOOL:
        return bytes([1 if v else 0])
    if t == STRING:
        return enc_string(v)
    if t == ARRAY:
        et, vals = v
        return struct.pack("<IQ", et, len(vals)) + b"".join(enc_value(et, x) for x in vals)
    raise ValueError(t)


def build_test_gguf(metadata, tensors, version: int = 3, magic: bytes = b"GGUF") -> bytes:
    """Header + metadata [(key, type, value)] + tensor infos [(name, dims,
    dtype, offset)]; no data section."""
    out = bytearray(magic + struct.pack("<IQQ", version, len(tensors), len(metadata)))
    for key, t, v in metadata:
        out += enc_string(key) + struct.pack("<I", t) + (v if isinstance(v, (bytes, bytearray)) else enc_value(t, v))
    for name, dims, dtype, offset in tensors:
        out += enc_string(name) + struct.pack("<I", len(dims))
        out += b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", dtype, offset)
    return bytes(out)


def build_gguf(metadata, tensors, alignment: int = 32) -> bytes:
    """A whole file: tensors [(name, dims, dtype, data bytes)] placed at
    aligned offsets in a data section that starts at the aligned end of the
    infos (`alignment` must match general.alignment when that is set)."""
    up = lambda n: (n + alignment - 1) // alignment * alignment  # noqa: E731
    offs, off = [], 0
    for _, _, _, data in tensors:
        offs.append(off)
        off = up(off + len(data))
    head = build_test_gguf(metadata, [(n, d, t, o) for (n, d, t, _), o in zip(tensors, offs)])
    out = bytearray(head)
    start = up(len(out))
    out += bytes(start - len(out))
    for (_, _, _, data), o in zip(tensors, offs):
        out += bytes(start + o - len(out))
        out += bytes(data)
    return bytes(out)


def llama_gguf(W: dict, f16_norms: bool = False) -> bytes:
    """A llama GGUF of the decode-step test weights (llama_case.make_weights):
    the llama.* metadata TinyLlamaConfig::from_gguf reads and the tensors
    load_weights names; norms as F32, or rounded to F16 with f16_norms."""
    import numpy as np
    c = W["cfg"]
    meta = [("general.architecture", STRING, "llama"), ("general.name", STRING, "rce-amd test llama"),
            ("llama.embedding_length", U32, c["d_model"]), ("llama.block_count", U32, c["n_layers"]),
            ("llama.attention.head_count", U32, c["n_q_heads"]),
            ("llama.attention.head_count_kv", U32, c["n_kv_heads"]),
            ("llama.rope.dimension_count", U32, c["rope_dim"]), ("llama.rope.freq_base", F32, c["rope_freq_base"]),
            ("llama.feed_forward_length", U32, c["d_ff"]), ("llama.context_length", U32, c["context_length"]),
            ("llama.attention.layer_norm_rms_epsilon", F32, c["eps"]), ("llama.vocab_size", U32, c["vocab"])]

    def norm(v):
        v = np.asarray(v, np.float32)
        if f16_norms:
            return ((v.size,), 1, v.astype(np.float16).tobytes())
        return ((v.size,), 0, v.tobytes())

    def lin(bd, n_rows, n_cols):
        return ((n_cols, n_rows), int(bd[1]), bytes(bd[0]))

    qd, kvd = c["n_q_heads"] * c["d_head"], c["n_kv_heads"] * c["d_head"]
    dm, ff = c["d_model"], c["d_ff"]
    shapes = {"attn_q": ("wq", qd, dm), "attn_k": ("wk", kvd, dm), "attn_v": ("wv", kvd, dm),
              "attn_output": ("wo", dm, qd), "ffn_gate": ("ffn_gate", ff, dm), "ffn_up": ("ffn_up", ff, dm),
              "ffn_down": ("ffn_down", dm, ff)}
    tens = [("token_embd.weight",) + lin(W["token_embd"], c["vocab"], dm),
            ("output_norm.weight",) + norm(W["output_norm"]),
            ("output.weight",) + lin(W["lm_head"], c["vocab"], dm)]
    for il, b in enumerate(W["blocks"]):
        tens.append((f"blk.{il}.attn_norm.weight",) + norm(b["attn_norm"]))
        tens.append((f"blk.{il}.ffn_norm.weight",) + norm(b["ffn_norm"]))
        for gname, (key, nr, nc) in shapes.items():
            tens.append((f"blk.{il}.{gname}.weight",) + lin(b[key], nr, nc))
    return build_gguf(meta, tens)
