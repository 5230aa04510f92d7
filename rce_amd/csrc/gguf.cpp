// gguf.cpp -- GGUF files behind the rce_qmm_gguf_* entry points: the
// header / metadata / tensor-info parser (rce-ingest-gguf/src/parser.rs
// L446-551, GgufFile::parse), the read-only file mapping it runs over
// (mmap.rs, mmap_load_sequential), the on-disk size of a tensor
// (dequant.rs L18-60, tensor_byte_size), and the two ways a tensor leaves
// the file: QuantWeight::from_gguf (rce-op-qmm/src/lib.rs L173-209) as a
// device-resident weight, and read_tensor_f32 (dequant.rs L85-112) for the
// f32 / f16 / bf16 vectors (norm weights) a decoder keeps on the host.
//
// Host code only.  The parser never reads tensor data; every read is
// bounds-checked against the bytes it was given, so a truncated or
// malformed file is a status code, not a fault.
#include "abi_internal.h"

#include <cerrno>
#include <cstring>
#include <fcntl.h>
#include <new>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

using namespace rce_qmm;
using namespace rce_qmm_abi;

struct rce_qmm_gguf {
    const uint8_t *data = nullptr;  // the file's bytes (mapped, or the caller's)
    size_t len = 0;
    void *map = nullptr;  // owned mapping (rce_qmm_gguf_open)
    size_t map_len = 0;
    uint32_t version = 0;
    bool tag42_stq1 = false;  // hunyuan-dense: tag 42 is STQ1_0 (parser.rs L529-541)
    struct Meta {
        std::string key;
        uint32_t type = 0;
        size_t val_off = 0, val_len = 0;  // the encoded value inside data
    };
    struct Tensor {
        std::string name;
        uint32_t ndim = 0;
        uint64_t dims[8] = {};
        uint32_t dtype = 0;
        uint64_t offset = 0;  // relative to data_offset
        uint64_t nbytes = 0;  // tensor_byte_size; 0: no size rule for the dtype
        bool numel_ok = true; // the product of dims fits in 64 bits
    };
    std::vector<Meta> meta;
    std::vector<Tensor> tensors;
    uint64_t data_offset = 0, alignment = 32;
};

namespace {

// GGUF metadata value type tags (parser.rs L187-199).
enum : uint32_t {
    V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
    V_STRING = 8, V_ARRAY = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12
};
constexpr int MAX_NESTING = 64;  // arrays of arrays: a bound against hostile files

size_t scalar_size(uint32_t t) {
    switch (t) {
    case V_U8: case V_I8: case V_BOOL: return 1;
    case V_U16: case V_I16: return 2;
    case V_U32: case V_I32: case V_F32: return 4;
    case V_U64: case V_I64: case V_F64: return 8;
    default: return 0;
    }
}

// Strict UTF-8 (what Rust's String::from_utf8 accepts).
bool valid_utf8(const uint8_t *s, size_t n) {
    size_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) { i++; continue; }
        size_t k;
        uint32_t cp;
        if ((c & 0xE0) == 0xC0) { k = 1; cp = c & 0x1F; }
        else if ((c & 0xF0) == 0xE0) { k = 2; cp = c & 0x0F; }
        else if ((c & 0xF8) == 0xF0) { k = 3; cp = c & 0x07; }
        else return false;
        if (i + k >= n) return false;  // the sequence runs past the end
        for (size_t j = 1; j <= k; j++) {
            if ((s[i + j] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + j] & 0x3F);
        }
        if ((k == 1 && cp < 0x80) || (k == 2 && cp < 0x800) || (k == 3 && cp < 0x10000)) return false;  // overlong
        if (cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
        i += k + 1;
    }
    return true;
}

struct Cursor {
    const uint8_t *d;
    size_t n, pos = 0;
    std::string err;  // set on failure, in the reference's wording

    bool eof() {
        err = "unexpected end of input at offset " + std::to_string(pos);
        return false;
    }
    bool take(size_t k, const uint8_t *&p) {
        if (n - pos < k) return eof();
        p = d + pos;
        pos += k;
        return true;
    }
    bool u32(uint32_t &v) {
        const uint8_t *p;
        if (!take(4, p)) return false;
        v = (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
        return true;
    }
    bool u64(uint64_t &v) {
        const uint8_t *p;
        if (!take(8, p)) return false;
        v = 0;
        for (int i = 7; i >= 0; i--) v = v << 8 | p[i];
        return true;
    }
    // GGUF string: u64 length + UTF-8 bytes
    bool str(std::string *out) {
        uint64_t len;
        if (!u64(len)) return false;
        const size_t at = pos;
        if (len > n - pos) return eof();
        const uint8_t *p = d + pos;
        pos += (size_t)len;
        if (!valid_utf8(p, (size_t)len)) {
            err = "invalid utf-8 in string at offset " + std::to_string(at);
            return false;
        }
        if (out) out->assign(reinterpret_cast<const char *>(p), (size_t)len);
        return true;
    }
    // Step over one value of type t (read_value, parser.rs L201-226).
    bool skip_value(uint32_t t, int depth) {
        if (t == V_STRING) return str(nullptr);
        if (t == V_ARRAY) {
            if (depth >= MAX_NESTING) {
                err = "metadata arrays nested deeper than " + std::to_string(MAX_NESTING);
                return false;
            }
            uint32_t et;
            uint64_t count;
            if (!u32(et) || !u64(count)) return false;
            const size_t es = scalar_size(et);
            if (es) {  // fixed-size elements: one bounds check
                if (count > (n - pos) / es) {
                    pos = n;
                    return eof();
                }
                pos += (size_t)count * es;
                return true;
            }
            if (et != V_STRING && et != V_ARRAY) {
                err = "unknown metadata value type tag " + std::to_string(et);
                return false;
            }
            for (uint64_t i = 0; i < count; i++)
                if (!skip_value(et, depth + 1)) return false;
            return true;
        }
        const size_t s = scalar_size(t);
        if (!s) {
            err = "unknown metadata value type tag " + std::to_string(t);
            return false;
        }
        const uint8_t *p;
        return take(s, p);
    }
};

// tensor_byte_size (dequant.rs L18-60): bytes of n elements, per GGUF tag;
// tag 42 is PrismML Q2_0 unless the file's architecture says STQ1_0.
uint64_t dtype_bytes(uint32_t tag, uint64_t n, bool tag42_is_stq1, bool &known) {
    auto blocks = [&](uint64_t qk, uint64_t bb) { return (n / qk + (n % qk != 0)) * bb; };
    known = true;
    switch (tag) {
    case 0: return n * 4;              // F32
    case 28: return n * 8;             // F64
    case 1: case 30: return n * 2;     // F16, BF16
    case 24: return n;                 // I8
    case 25: return n * 2;             // I16
    case 26: return n * 4;             // I32
    case 27: return n * 8;             // I64
    case 2: return blocks(32, 18);     // Q4_0
    case 3: return blocks(32, 20);     // Q4_1
    case 6: return blocks(32, 22);     // Q5_0
    case 7: return blocks(32, 24);     // Q5_1
    case 8: return blocks(32, 34);     // Q8_0
    case 9: return blocks(32, 36);     // Q8_1
    case 10: return blocks(256, 84);   // Q2_K
    case 11: return blocks(256, 110);  // Q3_K
    case 12: return blocks(256, 144);  // Q4_K
    case 13: return blocks(256, 176);  // Q5_K
    case 14: return blocks(256, 210);  // Q6_K
    case 36: return n / 4 + (n % 4 != 0) + 4;  // I2_S: 2-bit codes + one f32 scale
    case 41: return blocks(128, 18);   // Q1_0
    case 42: return tag42_is_stq1 ? blocks(256, 42) : blocks(128, 34);  // STQ1_0 / Q2_0
    default: known = false; return 0;
    }
}

bool mul_overflows(uint64_t a, uint64_t b, uint64_t &r) { return __builtin_mul_overflow(a, b, &r); }

rce_qmm_status parse_into(rce_qmm_gguf *g) {
    Cursor c{g->data, g->len};
    auto perr = [&](const std::string &m) { return fail(RCE_QMM_PARSE_ERROR, "gguf: " + m); };
    const uint8_t *mg;
    if (!c.take(4, mg)) return perr(c.err);
    if (std::memcmp(mg, "GGUF", 4) != 0) {
        const uint32_t m = (uint32_t)mg[0] | (uint32_t)mg[1] << 8 | (uint32_t)mg[2] << 16 | (uint32_t)mg[3] << 24;
        char buf[80];
        std::snprintf(buf, sizeof buf, "invalid magic: expected GGUF (0x47475546), got %#010x", m);
        return perr(buf);
    }
    if (!c.u32(g->version)) return perr(c.err);
    if (g->version < 2 || g->version > 3)
        return perr("unsupported version " + std::to_string(g->version) + " (supported: 2..=3)");
    uint64_t n_tensors, n_meta;
    if (!c.u64(n_tensors) || !c.u64(n_meta)) return perr(c.err);
    // Each entry consumes bytes or fails, so a count larger than the file
    // ends in an end-of-input error after at most len / 12 entries (the
    // reference's error order: it reads entry by entry too).
    for (uint64_t i = 0; i < n_meta; i++) {
        rce_qmm_gguf::Meta m;
        if (!c.str(&m.key) || !c.u32(m.type)) return perr(c.err);
        m.val_off = c.pos;
        if (!c.skip_value(m.type, 0)) return perr(c.err);
        m.val_len = c.pos - m.val_off;
        g->meta.push_back(std::move(m));
    }
    // the architecture decides tag 42 (parser.rs L529-541)
    bool hunyuan = false;
    for (const auto &m : g->meta)
        if (m.key == "general.architecture" && m.type == V_STRING) {
            const uint8_t *v = g->data + m.val_off + 8;
            hunyuan = hunyuan || (m.val_len - 8 == 13 && std::memcmp(v, "hunyuan-dense", 13) == 0);
        }
    g->tag42_stq1 = hunyuan;
    for (uint64_t i = 0; i < n_tensors; i++) {
        rce_qmm_gguf::Tensor t;
        if (!c.str(&t.name) || !c.u32(t.ndim)) return perr(c.err);
        if (t.ndim > 8) return perr("tensor dimension count " + std::to_string(t.ndim) + " exceeds maximum (8)");
        for (uint32_t k = 0; k < t.ndim; k++)
            if (!c.u64(t.dims[k])) return perr(c.err);
        if (!c.u32(t.dtype) || !c.u64(t.offset)) return perr(c.err);
        uint64_t numel = 1;
        for (uint32_t k = 0; k < t.ndim && t.numel_ok; k++) t.numel_ok = !mul_overflows(numel, t.dims[k], numel);
        bool known = false;
        uint64_t nb = 0;
        if (t.numel_ok) {
            // sizes of at most 8 bytes per element, or blocks: overflow only
            // past 2^61 elements
            if (numel <= (UINT64_MAX >> 4)) nb = dtype_bytes(t.dtype, numel, hunyuan, known);
            else t.numel_ok = false;
        }
        t.nbytes = known ? nb : 0;
        g->tensors.push_back(std::move(t));
    }
    // data section: after the infos, padded to general.alignment (the first
    // entry with that key, when it is U32 or U64; else 32)
    g->alignment = 32;
    for (const auto &m : g->meta)
        if (m.key == "general.alignment") {
            const uint8_t *v = g->data + m.val_off;
            if (m.type == V_U32) {
                g->alignment = (uint64_t)v[0] | (uint64_t)v[1] << 8 | (uint64_t)v[2] << 16 | (uint64_t)v[3] << 24;
            } else if (m.type == V_U64) {
                uint64_t a = 0;
                for (int k = 7; k >= 0; k--) a = a << 8 | v[k];
                g->alignment = a;
            }
            break;
        }
    if (g->alignment == 0) return perr("general.alignment is 0");
    const uint64_t pos = c.pos;
    g->data_offset = pos % g->alignment == 0 ? pos : pos + (g->alignment - pos % g->alignment);
    return RCE_QMM_OK;
}

const rce_qmm_gguf::Tensor *find_tensor(const rce_qmm_gguf *g, const char *name, size_t *index = nullptr) {
    for (size_t i = 0; i < g->tensors.size(); i++)
        if (g->tensors[i].name == name) {
            if (index) *index = i;
            return &g->tensors[i];
        }
    return nullptr;
}

// The tensor's bytes inside the file, checked (QuantWeight::from_gguf and
// read_tensor_f32: start = data_offset + offset, end = start + size).
rce_qmm_status tensor_span(const rce_qmm_gguf *g, const rce_qmm_gguf::Tensor &t, const uint8_t *&p, size_t &n) {
    if (!t.numel_ok) return fail(RCE_QMM_BAD_SHAPE, t.name + ": element count overflows");
    uint64_t start;
    if (__builtin_add_overflow(g->data_offset, t.offset, &start) || start > g->len || t.nbytes > g->len - start)
        return fail(RCE_QMM_BAD_SHAPE, t.name + ": out of bounds [" + std::to_string(g->data_offset + t.offset) + ", +" +
                                           std::to_string(t.nbytes) + ") > file len " + std::to_string(g->len));
    p = g->data + start;
    n = (size_t)t.nbytes;
    return RCE_QMM_OK;
}

uint64_t numel_of(const rce_qmm_gguf::Tensor &t) {
    uint64_t n = 1;
    for (uint32_t k = 0; k < t.ndim; k++) n *= t.dims[k];
    return n;
}

float half_to_float(uint16_t h) {  // binary16 -> binary32, exact
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1F, m = h & 0x3FF;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else {  // subnormal: normalize
            int k = -1;
            uint32_t mm = m;
            do { k++; mm <<= 1; } while ((mm & 0x400) == 0);
            bits = s | (uint32_t)(127 - 15 - k) << 23 | (mm & 0x3FF) << 13;
        }
    } else if (e == 31) {
        bits = s | 0x7F800000u | m << 13;
    } else {
        bits = s | (e + 127 - 15) << 23 | m << 13;
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

}  // namespace

extern "C" {

rce_qmm_status rce_qmm_gguf_parse(const uint8_t *bytes, size_t len, rce_qmm_gguf **out) {
    if (!out || (!bytes && len)) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    *out = nullptr;
    rce_qmm_gguf *g = new (std::nothrow) rce_qmm_gguf();
    if (!g) return fail(RCE_QMM_OUT_OF_MEMORY, "gguf handle");
    g->data = bytes;
    g->len = len;
    rce_qmm_status st;
    try {
        st = parse_into(g);
    } catch (const std::bad_alloc &) {
        st = fail(RCE_QMM_OUT_OF_MEMORY, "gguf: metadata");
    }
    if (st) {
        delete g;
        return st;
    }
    *out = g;
    return RCE_QMM_OK;
}

rce_qmm_status rce_qmm_gguf_open(const char *path, rce_qmm_gguf **out) {
    if (!path || !out) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(RCE_QMM_IO_ERROR, std::string("open ") + path + ": " + std::strerror(errno));
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        const int e = errno;
        ::close(fd);
        return fail(RCE_QMM_IO_ERROR, std::string("stat ") + path + ": " + std::strerror(e));
    }
    const size_t len = (size_t)sb.st_size;
    void *map = nullptr;
    if (len) {
        map = mmap(nullptr, len, PROT_READ, MAP_PRIVATE, fd, 0);
        if (map == MAP_FAILED) {
            const int e = errno;
            ::close(fd);
            return fail(RCE_QMM_IO_ERROR, std::string("mmap ") + path + ": " + std::strerror(e));
        }
        (void)madvise(map, len, MADV_SEQUENTIAL);  // a hint; the load walks the file in order
    }
    ::close(fd);
    rce_qmm_gguf *g = nullptr;
    rce_qmm_status st = rce_qmm_gguf_parse(static_cast<const uint8_t *>(map), len, &g);
    if (st) {
        if (map) munmap(map, len);
        return st;
    }
    g->map = map;
    g->map_len = len;
    *out = g;
    return RCE_QMM_OK;
}

void rce_qmm_gguf_close(rce_qmm_gguf *g) {
    if (!g) return;
    if (g->map) munmap(g->map, g->map_len);
    delete g;
}

rce_qmm_status rce_qmm_gguf_header(const rce_qmm_gguf *g, uint32_t *version, size_t *n_tensors, size_t *n_metadata,
                                   uint64_t *data_offset, uint64_t *alignment) {
    if (!g) return fail(RCE_QMM_NULL_ARGUMENT, "null gguf");
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = g->tensors.size();
    if (n_metadata) *n_metadata = g->meta.size();
    if (data_offset) *data_offset = g->data_offset;
    if (alignment) *alignment = g->alignment;
    return RCE_QMM_OK;
}

rce_qmm_status rce_qmm_gguf_metadata(const rce_qmm_gguf *g, size_t i, const char **key, uint32_t *type,
                                     const uint8_t **value, size_t *value_len) {
    if (!g) return fail(RCE_QMM_NULL_ARGUMENT, "null gguf");
    if (i >= g->meta.size()) return fail(RCE_QMM_BAD_SHAPE, "metadata index " + std::to_string(i) + " out of range");
    const auto &m = g->meta[i];
    if (key) *key = m.key.c_str();
    if (type) *type = m.type;
    if (value) *value = g->data + m.val_off;
    if (value_len) *value_len = m.val_len;
    return RCE_QMM_OK;
}

rce_qmm_status rce_qmm_gguf_find_metadata(const rce_qmm_gguf *g, const char *key, size_t *index) {
    if (!g || !key || !index) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    for (size_t i = 0; i < g->meta.size(); i++)  // the first entry with the key (get_metadata)
        if (g->meta[i].key == key) {
            *index = i;
            return RCE_QMM_OK;
        }
    return fail(RCE_QMM_NOT_FOUND, std::string("metadata key not found: ") + key);
}

rce_qmm_status rce_qmm_gguf_tensor(const rce_qmm_gguf *g, size_t i, const char **name, uint32_t *ndim, uint64_t *dims,
                                   uint32_t *dtype, uint64_t *offset, uint64_t *nbytes) {
    if (!g) return fail(RCE_QMM_NULL_ARGUMENT, "null gguf");
    if (i >= g->tensors.size()) return fail(RCE_QMM_BAD_SHAPE, "tensor index " + std::to_string(i) + " out of range");
    const auto &t = g->tensors[i];
    if (name) *name = t.name.c_str();
    if (ndim) *ndim = t.ndim;
    if (dims)
        for (int k = 0; k < 8; k++) dims[k] = k < (int)t.ndim ? t.dims[k] : 0;
    if (dtype) *dtype = t.dtype;
    if (offset) *offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return RCE_QMM_OK;
}

rce_qmm_status rce_qmm_gguf_find_tensor(const rce_qmm_gguf *g, const char *name, size_t *index) {
    if (!g || !name || !index) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    if (!find_tensor(g, name, index)) return fail(RCE_QMM_NOT_FOUND, std::string("tensor not found: ") + name);
    return RCE_QMM_OK;
}

rce_qmm_status rce_qmm_weight_from_gguf(rce_qmm_context *ctx, const rce_qmm_gguf *g, const char *name, size_t n_rows,
                                        size_t n_cols, rce_qmm_weight **out) {
    if (!ctx || !g || !name || !out) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    *out = nullptr;
    const rce_qmm_gguf::Tensor *t = find_tensor(g, name);
    if (!t) return fail(RCE_QMM_NOT_FOUND, std::string("tensor not found: ") + name);
    uint64_t want;
    if (mul_overflows(n_rows, n_cols, want) || !t->numel_ok || numel_of(*t) != want)
        return fail(RCE_QMM_BAD_SHAPE, std::string(name) + ": declared shape " + std::to_string(n_rows) + "x" +
                                           std::to_string(n_cols) + " != tensor numel " +
                                           (t->numel_ok ? std::to_string(numel_of(*t)) : std::string("(overflow)")));
    const uint8_t *p;
    size_t n;
    rce_qmm_status st = tensor_span(g, *t, p, n);
    if (st) return st;
    const uint32_t dt = (t->dtype == 42 && g->tag42_stq1) ? RCE_QMM_DTYPE_STQ1_0 : t->dtype;
    return rce_qmm_weight_from_bytes(ctx, dt, n_rows, n_cols, p, n, out);
}

rce_qmm_status rce_qmm_gguf_read_f32(const rce_qmm_gguf *g, const char *name, float *out, size_t n) {
    if (!g || !name || (!out && n)) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    const rce_qmm_gguf::Tensor *t = find_tensor(g, name);
    if (!t) return fail(RCE_QMM_NOT_FOUND, std::string("tensor not found: ") + name);
    if (!t->numel_ok || numel_of(*t) != n)
        return fail(RCE_QMM_BAD_SHAPE, std::string(name) + ": " + std::to_string(n) + " values asked, tensor has " +
                                           (t->numel_ok ? std::to_string(numel_of(*t)) : std::string("(overflow)")));
    if (t->dtype != 0 && t->dtype != 1 && t->dtype != 30)
        return fail(RCE_QMM_UNSUPPORTED_DTYPE, std::string(name) + ": dtype " + std::to_string(t->dtype) +
                                                   " (read_f32 takes F32, F16 and BF16 tensors)");
    const uint8_t *p;
    size_t nb;
    rce_qmm_status st = tensor_span(g, *t, p, nb);
    if (st) return st;
    for (size_t i = 0; i < n; i++) {
        if (t->dtype == 0) {
            std::memcpy(&out[i], p + 4 * i, 4);  // little-endian host
        } else {
            const uint16_t h = (uint16_t)(p[2 * i] | p[2 * i + 1] << 8);
            if (t->dtype == 1) {
                out[i] = half_to_float(h);
            } else {
                const uint32_t bits = (uint32_t)h << 16;
                std::memcpy(&out[i], &bits, 4);
            }
        }
    }
    return RCE_QMM_OK;
}

}  // extern "C"
