"""GGUF files over the C ABI (rce_qmm_gguf_*): the Python mirror of
rce-ingest-gguf's ``GgufFile`` (parser.rs L431-615) and ``read_tensor_f32``
(dequant.rs L85-112), and rce-qwen36-moe's ``split_experts`` (L216-223).
``QuantWeight.from_gguf`` (rce-op-qmm/src/lib.rs L173-209) takes a
GgufFile from here.

Parsing is the library's (native, bounds-checked); this module decodes the
metadata values it hands back, which are the file's own encoded bytes.
"""
from __future__ import annotations

import ctypes
import os
import struct
from dataclasses import dataclass

import numpy as np

from ._lib import QmmError, check, lib
from .qmm import QuantWeight

# GGUF metadata value type tags (parser.rs L187-199)
GGUF_TYPE_UINT8, GGUF_TYPE_INT8, GGUF_TYPE_UINT16, GGUF_TYPE_INT16 = 0, 1, 2, 3
GGUF_TYPE_UINT32, GGUF_TYPE_INT32, GGUF_TYPE_FLOAT32, GGUF_TYPE_BOOL = 4, 5, 6, 7
GGUF_TYPE_STRING, GGUF_TYPE_ARRAY, GGUF_TYPE_UINT64, GGUF_TYPE_INT64, GGUF_TYPE_FLOAT64 = 8, 9, 10, 11, 12

_SCALAR = {GGUF_TYPE_UINT8: "<B", GGUF_TYPE_INT8: "<b", GGUF_TYPE_UINT16: "<H", GGUF_TYPE_INT16: "<h",
           GGUF_TYPE_UINT32: "<I", GGUF_TYPE_INT32: "<i", GGUF_TYPE_FLOAT32: "<f", GGUF_TYPE_UINT64: "<Q",
           GGUF_TYPE_INT64: "<q", GGUF_TYPE_FLOAT64: "<d"}


@dataclass(frozen=True)
class GgufValue:
    """A metadata value with its type tag (the reference's GgufValue enum:
    ``type`` names the variant, ``value`` its payload; arrays hold a list
    of GgufValue)."""
    type: int
    value: object


@dataclass(frozen=True)
class GgufMetadata:
    key: str
    value: GgufValue


@dataclass(frozen=True)
class GgufTensorInfo:
    """A tensor descriptor (parser.rs L404-418): dims ne0 first, GGUF dtype
    tag, offset relative to ``data_offset``, and its size in the file."""
    name: str
    dims: tuple
    dtype: int
    offset: int
    nbytes: int

    def numel(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n


def _decode(buf: bytes, pos: int, t: int):
    """One encoded value at buf[pos:] -> (GgufValue, next position)."""
    if t in _SCALAR:
        fmt = _SCALAR[t]
        return GgufValue(t, struct.unpack_from(fmt, buf, pos)[0]), pos + struct.calcsize(fmt)
    if t == GGUF_TYPE_BOOL:
        return GgufValue(t, buf[pos] != 0), pos + 1
    if t == GGUF_TYPE_STRING:
        n = struct.unpack_from("<Q", buf, pos)[0]
        return GgufValue(t, buf[pos + 8:pos + 8 + n].decode("utf-8")), pos + 8 + n
    if t == GGUF_TYPE_ARRAY:
        et, count = struct.unpack_from("<IQ", buf, pos)
        pos += 12
        if et in _SCALAR:  # fixed-size elements in one step
            fmt = _SCALAR[et]
            vals = struct.unpack_from("<" + fmt[1] * count, buf, pos)
            return GgufValue(t, [GgufValue(et, v) for v in vals]), pos + struct.calcsize(fmt) * count
        out = []
        for _ in range(count):
            v, pos = _decode(buf, pos, et)
            out.append(v)
        return GgufValue(t, out), pos
    raise ValueError(f"unknown metadata value type tag {t}")  # the parser already rejected it


class GgufFile:
    """A parsed GGUF v2/v3 file (GgufFile::parse, parser.rs L446-551): the
    header, metadata and tensor infos; tensor data stays in the file."""

    def __init__(self, handle: ctypes.c_void_p, file_len: int, keepalive=None):
        self._h = handle
        self.file_len = file_len
        self._keep = keepalive  # the caller's bytes for parse(); None for open()
        L = lib()
        ver, nt, nm = ctypes.c_uint32(), ctypes.c_size_t(), ctypes.c_size_t()
        doff, align = ctypes.c_uint64(), ctypes.c_uint64()
        check(L.rce_qmm_gguf_header(handle, ctypes.byref(ver), ctypes.byref(nt), ctypes.byref(nm),
                                    ctypes.byref(doff), ctypes.byref(align)))
        self.version, self.data_offset, self.alignment = ver.value, doff.value, align.value
        self.metadata = []
        for i in range(nm.value):
            key, typ = ctypes.c_char_p(), ctypes.c_uint32()
            val, vlen = ctypes.c_void_p(), ctypes.c_size_t()
            check(L.rce_qmm_gguf_metadata(handle, i, ctypes.byref(key), ctypes.byref(typ), ctypes.byref(val),
                                          ctypes.byref(vlen)))
            raw = ctypes.string_at(val.value, vlen.value) if vlen.value else b""
            v, _ = _decode(raw, 0, typ.value)
            self.metadata.append(GgufMetadata(key.value.decode("utf-8"), v))
        self.tensors = []
        dims = (ctypes.c_uint64 * 8)()
        for i in range(nt.value):
            name, nd, dt = ctypes.c_char_p(), ctypes.c_uint32(), ctypes.c_uint32()
            off, nb = ctypes.c_uint64(), ctypes.c_uint64()
            check(L.rce_qmm_gguf_tensor(handle, i, ctypes.byref(name), ctypes.byref(nd), dims, ctypes.byref(dt),
                                        ctypes.byref(off), ctypes.byref(nb)))
            self.tensors.append(GgufTensorInfo(name.value.decode("utf-8"), tuple(dims[k] for k in range(nd.value)),
                                               dt.value, off.value, nb.value))

    @classmethod
    def parse(cls, data: bytes) -> "GgufFile":
        """GgufFile::parse over bytes (kept alive with the handle)."""
        buf = np.frombuffer(bytes(data), np.uint8)
        h = ctypes.c_void_p()
        check(lib().rce_qmm_gguf_parse(buf.ctypes.data_as(ctypes.c_void_p) if buf.size else None, buf.size,
                                       ctypes.byref(h)))
        return cls(h, buf.size, keepalive=buf)

    @classmethod
    def open(cls, path) -> "GgufFile":
        """mmap_load_sequential + parse: the file stays mapped until close()."""
        h = ctypes.c_void_p()
        check(lib().rce_qmm_gguf_open(os.fsencode(path), ctypes.byref(h)))
        return cls(h, os.path.getsize(path))

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise ValueError("GGUF file is closed")
        return self._h

    def close(self) -> None:
        if self._h is not None:
            lib().rce_qmm_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- convenience accessors (parser.rs L553-615) ----
    def get_metadata(self, key: str) -> GgufValue | None:
        for m in self.metadata:  # the first entry with the key
            if m.key == key:
                return m.value
        return None

    def _typed(self, key: str, t: int):
        v = self.get_metadata(key)
        return v.value if v is not None and v.type == t else None

    def get_string(self, key: str) -> str | None:
        return self._typed(key, GGUF_TYPE_STRING)

    def get_u32(self, key: str) -> int | None:
        return self._typed(key, GGUF_TYPE_UINT32)

    def get_u64(self, key: str) -> int | None:
        return self._typed(key, GGUF_TYPE_UINT64)

    def get_f32(self, key: str) -> float | None:
        return self._typed(key, GGUF_TYPE_FLOAT32)

    def architecture(self) -> str | None:
        return self.get_string("general.architecture")

    def model_name(self) -> str | None:
        return self.get_string("general.name")

    def _arch_u32(self, suffix: str) -> int | None:
        arch = self.architecture()
        return None if arch is None else self.get_u32(f"{arch}.{suffix}")

    def block_count(self) -> int | None:
        return self._arch_u32("block_count")

    def embedding_length(self) -> int | None:
        return self._arch_u32("embedding_length")

    def head_count(self) -> int | None:
        return self._arch_u32("attention.head_count")

    def head_count_kv(self) -> int | None:
        return self._arch_u32("attention.head_count_kv")

    def tensor(self, name: str) -> GgufTensorInfo | None:
        for t in self.tensors:
            if t.name == name:
                return t
        return None

    def read_tensor_f32(self, name: str) -> np.ndarray:
        """read_tensor_f32 (dequant.rs L85-112) for F32 / F16 / BF16 tensors."""
        t = self.tensor(name)
        if t is None:  # the library reports it
            check(lib().rce_qmm_gguf_read_f32(self.handle, name.encode("utf-8"), None, 0))
        # the library's checks, made before the output is allocated
        size = {0: 4, 1: 2, 30: 2}.get(t.dtype)
        if size is None:
            raise QmmError(3, f"{name}: dtype {t.dtype} (read_f32 takes F32, F16 and BF16 tensors)")
        n = t.numel()
        if n * size != t.nbytes:
            raise QmmError(2, f"{name}: element count overflows")
        if self.data_offset + t.offset + t.nbytes > self.file_len:
            raise QmmError(2, f"{name}: out of bounds [{self.data_offset + t.offset}, +{t.nbytes}) > file len "
                              f"{self.file_len}")
        out = np.empty(n, np.float32)
        check(lib().rce_qmm_gguf_read_f32(self.handle, name.encode("utf-8"),
                                          out.ctypes.data_as(ctypes.c_void_p) if n else None, n))
        return out


def split_experts(full: QuantWeight, n_expert: int, n_rows_per: int, n_cols_per: int) -> list:
    """split_experts (rce-qwen36-moe/src/lib.rs L216-223): per-expert views of
    a stacked [n_expert, n_rows_per, n_cols_per] tensor, byte stride
    total / n_expert (sharing the device copy)."""
    total = full.len
    if n_expert <= 0 or total % n_expert:
        raise ValueError(f"expert stack bytes {total} not divisible by n_expert {n_expert}")
    bpe = total // n_expert
    return [full.sub_view(e * bpe, bpe, n_rows_per, n_cols_per) for e in range(n_expert)]
