// qmm_gemv_kernels.h -- device code of the decode-shaped kernels of the GGUF
// quantized-matmul path for gfx950 (CDNA4): GEMV / skinny GEMM in the reference's f32 order (EXACT),
// the Q8-activation GEMV (Q8), and row dequantization.
//
// Work mapping ("activation-stationary").  A row of the weight is U column
// units (a Q4_0 / Q8_0 block of 32, a Q4_K group of 64, a Q6_K super-block
// of 256).  Thread `tid` of a block of NT threads owns unit col = tid % U
// and the rows rsub, rsub + P, ... (rsub = tid / U, P = NT / U) of the
// block's tile of RT = P * RPL rows, for TB activation rows (tokens).  It
// keeps its slice of the activations in registers, issues the loads of all
// RPL rows before doing any arithmetic, and writes one addend per (token,
// row) -- the reference's per-unit term of the row sum -- to LDS.  After a
// barrier, one thread per (token, row) folds the U addends in unit order,
// which is the reference's sequential `sumf += ...` over blocks.  The
// device layouts (qmm_internal.h) make every wave-wide weight load a
// contiguous 1 KB read.
//
// Exactness (EXACT): every + - * of the reference is one binary32 operation
// in the same order.  Q4_0's product (n - 8) a is formed as fma(n, a, -8a)
// when a thread has one token (-8a is exact while |a| < 2^124, and the fma
// rounds (n - 8) a once) and as (float)(n) - 8 (exact) times a otherwise;
// Q5_0 and Q3_K likewise with -16a and -4a.  So EXACT is the reference's bit
// for bit for activations of magnitude below 2^123; larger or non-finite
// activations can give another overflow or NaN pattern.  All other code is built
// with -ffp-contract=off.  The Q6_K row sum of the reference is one chain
// over all positions of the row, so Q6_K EXACT runs one row per lane.
//
// Q8: the block quantizes its activation rows into LDS once (4 lanes per
// block of 32: max |x| by two quad exchanges, then quantize_block(x, false)
// semantics), every thread copies its units' words to registers, and each
// per-block sub-sum of the reference becomes dx * (exact int32 dot).
//
// This header holds the kernels and launch templates; gemv_<format>.hip
// instantiate them per weight format (one translation unit each, so they
// build in parallel) and qmm_gemv.hip holds the host-side planning.
#pragma once

#include "qmm_internal.h"

#include <cstdlib>
#include <type_traits>
#include <utility>

namespace rce_qmm {
namespace {


constexpr uint32_t NIB = 0x0F0F0F0Fu;

// Weight loads.  A launch reads each weight byte once, so the loads are
// non-temporal: they stream through the caches instead of displacing what
// is reused (measured on the headline shapes: 5-10 % faster per launch).
typedef unsigned v4u32 __attribute__((ext_vector_type(4)));
typedef unsigned v2u32 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ldw16(const uint8_t *p) {
    const v4u32 t = __builtin_nontemporal_load(reinterpret_cast<const v4u32 *>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ uint2 ldw8(const uint8_t *p) {
    const v2u32 t = __builtin_nontemporal_load(reinterpret_cast<const v2u32 *>(p));
    return make_uint2(t.x, t.y);
}
__device__ __forceinline__ uint32_t ldw4(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p));
}
__device__ __forceinline__ uint32_t ldw2(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(p));
}

// Buffer access to one weight's rows.  A row's byte offset splits into the
// lane's part (its row within the block's row pass, times the row stride;
// loop-invariant, one VGPR) and the row pass's part (block-uniform, an SGPR
// soffset), so the weight loads of every row after the first cost no vector
// address arithmetic.  Loads are non-temporal (aux bit 1 on gfx950) like
// the pointer forms above.  num_records is the maximum: the layouts'
// padding rows (layout_pad_bytes) back every offset a tile forms, as for the
// pointer loads.  Each block's buffer starts at its own first row, so its
// offsets span the block's rows only (far below 2^31 bytes).
struct WBuf {
    __amdgpu_buffer_rsrc_t r;
    uint32_t lane;
};
__device__ __forceinline__ WBuf make_wbuf(const uint8_t *base, uint32_t lane_off) {
    WBuf b;
    b.r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), (short)0, (int)0x7FFFFFFF, 0x00020000);
    b.lane = lane_off;
    return b;
}
constexpr int BUF_NT = 2;
__device__ __forceinline__ uint4 bld16(const WBuf &b, uint32_t off, uint32_t soff) {
    const v4u32 t = __builtin_amdgcn_raw_buffer_load_b128(b.r, (int)(b.lane + off), (int)soff, BUF_NT);
    return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ uint2 bld8(const WBuf &b, uint32_t off, uint32_t soff) {
    const v2u32 t = __builtin_amdgcn_raw_buffer_load_b64(b.r, (int)(b.lane + off), (int)soff, BUF_NT);
    return make_uint2(t.x, t.y);
}
__device__ __forceinline__ uint32_t bld4(const WBuf &b, uint32_t off, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(b.r, (int)(b.lane + off), (int)soff, BUF_NT);
}
__device__ __forceinline__ uint32_t bld2(const WBuf &b, uint32_t off, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b16(b.r, (int)(b.lane + off), (int)soff, BUF_NT);
}

// Two nibbles (bytes 2h and 2h + 1 of x, each 0..15) as exact floats.  A
// byte n < 16 read as an OCP FP8 E4M3 code is n * 2^-9 exactly (codes 0..7
// are the subnormals m * 2^-9, codes 8..15 the binade (1 + m/8) * 2^-6 =
// (8 + m) * 2^-9); the conversion's scale 2^9 makes it n.  One instruction
// per two values instead of one per value (v_cvt_f32_ubyte).
typedef float f32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ f32x2v nib2f(uint32_t x, bool h) {
    return h ? __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((int)x, 512.0f, true)
             : __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((int)x, 512.0f, false);
}
// The four byte values (each < 16) of x as floats: FP8 = two packed
// conversions (half rate, so the same issue time as four v_cvt_f32_ubyte;
// measured per format: Q4_K 2 % faster with them, Q4_0 2-3 % slower).
template <bool FP8>
__device__ __forceinline__ void nib4f(uint32_t x, float *v) {
    if constexpr (FP8) {
        const f32x2v a = nib2f(x, false), b = nib2f(x, true);
        v[0] = a.x; v[1] = a.y; v[2] = b.x; v[3] = b.y;
    } else {
        v[0] = (float)(x & 0xFFu); v[1] = (float)((x >> 8) & 0xFFu); v[2] = (float)((x >> 16) & 0xFFu);
        v[3] = (float)(x >> 24);
    }
}

// Rows of weight loads a thread keeps in flight ahead of its arithmetic:
// the next rows' loads go out before each row's addends, so a wave's data
// arrives in the order it is used (measured: 2 beats issuing all rows at
// once, 1 and 4).
constexpr int PREFETCH_ROWS = 2;

__device__ __forceinline__ float h2f(uint32_t bits) {
    _Float16 h;
    uint16_t b = (uint16_t)bits;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;  // v_cvt_f32_f16: exact, subnormals preserved
}

// x & m, opaque to the optimizer so that later byte extractions compile to
// v_cvt_f32_ubyte{0..3} instead of one bitfield extract per nibble.
__device__ __forceinline__ uint32_t and_opaque(uint32_t x, uint32_t m) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(m), "v"(x));
    return r;
}

template <int J>
__device__ __forceinline__ float ubyte(uint32_t x) {
    return (float)((x >> (8 * J)) & 0xFFu);
}

__device__ __forceinline__ uint32_t wrd(const uint4 &v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

__device__ __forceinline__ void load_f32x(const float *p, float *v, int n) {
    const float4 *q = reinterpret_cast<const float4 *>(p);
#pragma unroll
    for (int i = 0; i < n / 4; i++) {
        float4 t = q[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
}

// Lane exchanges inside a quad of lanes (DPP quad_perm).
__device__ __forceinline__ int quad_xor1(int x) { return __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false); }
__device__ __forceinline__ int quad_xor2(int x) { return __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false); }
__device__ __forceinline__ float quad_xor1f(float x) { return __int_as_float(quad_xor1(__float_as_int(x))); }
__device__ __forceinline__ float quad_xor2f(float x) { return __int_as_float(quad_xor2(__float_as_int(x))); }

// Byte i (0..11) of a Q4_K super-block's packed scales, the header being the
// super-block's first 16 bytes (d, dmin, scales[12]).
__device__ __forceinline__ int k4_sbyte(const uint4 &h, int i) {
    uint32_t w = i < 4 ? h.y : (i < 8 ? h.z : h.w);
    return (int)((w >> (8 * (i & 3))) & 0xFFu);
}

// q4_k_get_scale_min (rce-op-qmm/src/lib.rs L719-728) for the sub-block pair
// (2g, 2g+1) of group g, with selects instead of indexed byte access (an
// index that varies per lane would send the header through scratch).
// Bytes: g<2 reads scales[2g..2g+1] and [2g+4..2g+5]; g>=2 reads
// scales[2g+4..2g+5] (low/high nibbles) plus the top two bits of
// scales[2g-4..2g-3] and [2g..2g+1].
__device__ __forceinline__ void k4_scale_min_pair(const uint4 &h, int g, int &sc1, int &m1, int &sc2,
                                                  int &m2) {
    const int sh = 16 * (g & 1);
    const uint32_t Y = h.y >> sh, Z = h.z >> sh, W = h.w >> sh;  // low 16 bits: the byte pair
    const uint32_t y0 = Y & 0xFF, y1 = (Y >> 8) & 0xFF, z0 = Z & 0xFF, z1 = (Z >> 8) & 0xFF;
    const uint32_t w0 = W & 0xFF, w1 = (W >> 8) & 0xFF;
    if (g < 2) {
        sc1 = (int)(y0 & 63); sc2 = (int)(y1 & 63);
        m1 = (int)(z0 & 63); m2 = (int)(z1 & 63);
    } else {
        sc1 = (int)((w0 & 0x0F) | ((y0 >> 6) << 4)); sc2 = (int)((w1 & 0x0F) | ((y1 >> 6) << 4));
        m1 = (int)((w0 >> 4) | ((z0 >> 6) << 4)); m2 = (int)((w1 >> 4) | ((z1 >> 6) << 4));
    }
}

// q4_k_get_scale_min (rce-op-qmm/src/lib.rs L719-728), one sub-block j.
__device__ __forceinline__ void k4_scale_min(const uint4 &h, int j, int &sc, int &m) {
    if (j < 4) {
        sc = k4_sbyte(h, j) & 63;
        m = k4_sbyte(h, j + 4) & 63;
    } else {
        sc = (k4_sbyte(h, j + 4) & 0x0F) | ((k4_sbyte(h, j - 4) >> 6) << 4);
        m = (k4_sbyte(h, j + 4) >> 4) | ((k4_sbyte(h, j) >> 6) << 4);
    }
}

// ---------------------------------------------------------------------------
// Raw unit loads (one row, one column unit) from the device layouts.
// ---------------------------------------------------------------------------

struct RawQ4_0 { uint4 q; uint32_t s; };
struct RawQ8_0 { uint4 q0, q1; uint32_t s; };
struct RawQ4_K { uint4 h, q0, q1; };
struct RawQ6_K { uint4 c[13]; uint32_t d; };
struct RawQ5_K { uint4 h, q0, q1; uint2 hb; };
struct RawQ5_0 { uint4 q; uint32_t s, h; };
struct RawQ4_1 { uint4 q; uint32_t sm; };
struct RawQ3_K { uint2 q; uint32_t h; uint32_t sd; };  // sd: scales (bytes 0, 1), d (bits 16..31)

__device__ __forceinline__ RawQ4_0 ld_q4_0(const DevWeight &w, size_t row, int col) {
    const uint8_t *rp = w.base + row * w.row_stride;
    RawQ4_0 r;
    r.q = ldw16(rp + w.plane1 + 16 * (size_t)col);
    r.s = ldw2(rp + 2 * (size_t)col);
    return r;
}

__device__ __forceinline__ RawQ8_0 ld_q8_0(const DevWeight &w, size_t row, int col) {
    const uint8_t *rp = w.base + row * w.row_stride;
    RawQ8_0 r;
    r.q0 = ldw16(rp + w.plane1 + 16 * (size_t)col);
    r.q1 = ldw16(rp + w.plane2 + 16 * (size_t)col);
    r.s = ldw2(rp + 2 * (size_t)col);
    return r;
}

__device__ __forceinline__ RawQ4_K ld_q4_k(const DevWeight &w, size_t row, int col) {
    const uint8_t *rp = w.base + row * w.row_stride;
    RawQ4_K r;
    r.h = ldw16(rp + 16 * (size_t)(col >> 2));
    r.q0 = ldw16(rp + w.plane1 + 16 * (size_t)col);
    r.q1 = ldw16(rp + w.plane2 + 16 * (size_t)col);
    return r;
}

__device__ __forceinline__ RawQ5_K ld_q5_k(const DevWeight &w, size_t row, int col) {
    const uint8_t *rp = w.base + row * w.row_stride;
    RawQ5_K r;
    r.h = ldw16(rp + 16 * (size_t)(col >> 2));
    r.q0 = ldw16(rp + w.plane1 + 16 * (size_t)col);
    r.q1 = ldw16(rp + w.plane2 + 16 * (size_t)col);
    r.hb = ldw8(rp + w.plane3 + 8 * (size_t)col);
    return r;
}

__device__ __forceinline__ RawQ5_0 ld_q5_0(const DevWeight &w, size_t row, int col) {
    const uint8_t *rp = w.base + row * w.row_stride;
    RawQ5_0 r;
    r.q = ldw16(rp + w.plane1 + 16 * (size_t)col);
    r.s = ldw2(rp + 2 * (size_t)col);
    r.h = ldw4(rp + w.plane2 + 4 * (size_t)col);
    return r;
}

__device__ __forceinline__ RawQ4_1 ld_q4_1(const DevWeight &w, size_t row, int col) {
    const uint8_t *rp = w.base + row * w.row_stride;
    RawQ4_1 r;
    r.q = ldw16(rp + w.plane1 + 16 * (size_t)col);
    r.sm = ldw4(rp + 4 * (size_t)col);
    return r;
}

__device__ __forceinline__ RawQ3_K ld_q3_k(const DevWeight &w, size_t row, int col) {
    const uint8_t *rp = w.base + row * w.row_stride;
    RawQ3_K r;
    r.q = ldw8(rp + w.plane1 + 8 * (size_t)col);
    r.h = ldw4(rp + w.plane2 + 4 * (size_t)col);
    const uint32_t sc = ldw2(rp + w.plane3 + 2 * (size_t)col);
    const uint32_t d = ldw2(rp + 2 * (size_t)(col >> 3));
    r.sd = sc | (d << 16);
    return r;
}

// The same unit loads through a WBuf: soff is the row pass's byte offset
// (uniform), b.lane the lane's row offset within the pass.
__device__ __forceinline__ RawQ4_0 bl_q4_0(const DevWeight &w, const WBuf &b, uint32_t soff, int col) {
    RawQ4_0 r;
    r.q = bld16(b, (uint32_t)w.plane1 + 16u * col, soff);
    r.s = bld2(b, 2u * col, soff);
    return r;
}
__device__ __forceinline__ RawQ8_0 bl_q8_0(const DevWeight &w, const WBuf &b, uint32_t soff, int col) {
    RawQ8_0 r;
    r.q0 = bld16(b, (uint32_t)w.plane1 + 16u * col, soff);
    r.q1 = bld16(b, (uint32_t)w.plane2 + 16u * col, soff);
    r.s = bld2(b, 2u * col, soff);
    return r;
}
__device__ __forceinline__ RawQ4_K bl_q4_k(const DevWeight &w, const WBuf &b, uint32_t soff, int col) {
    RawQ4_K r;
    r.h = bld16(b, 16u * (col >> 2), soff);
    r.q0 = bld16(b, (uint32_t)w.plane1 + 16u * col, soff);
    r.q1 = bld16(b, (uint32_t)w.plane2 + 16u * col, soff);
    return r;
}
__device__ __forceinline__ RawQ5_K bl_q5_k(const DevWeight &w, const WBuf &b, uint32_t soff, int col) {
    RawQ5_K r;
    r.h = bld16(b, 16u * (col >> 2), soff);
    r.q0 = bld16(b, (uint32_t)w.plane1 + 16u * col, soff);
    r.q1 = bld16(b, (uint32_t)w.plane2 + 16u * col, soff);
    r.hb = bld8(b, (uint32_t)w.plane3 + 8u * col, soff);
    return r;
}
__device__ __forceinline__ RawQ5_0 bl_q5_0(const DevWeight &w, const WBuf &b, uint32_t soff, int col) {
    RawQ5_0 r;
    r.q = bld16(b, (uint32_t)w.plane1 + 16u * col, soff);
    r.s = bld2(b, 2u * col, soff);
    r.h = bld4(b, (uint32_t)w.plane2 + 4u * col, soff);
    return r;
}
__device__ __forceinline__ RawQ4_1 bl_q4_1(const DevWeight &w, const WBuf &b, uint32_t soff, int col) {
    RawQ4_1 r;
    r.q = bld16(b, (uint32_t)w.plane1 + 16u * col, soff);
    r.sm = bld4(b, 4u * col, soff);
    return r;
}
__device__ __forceinline__ RawQ3_K bl_q3_k(const DevWeight &w, const WBuf &b, uint32_t soff, int col) {
    RawQ3_K r;
    r.q = bld8(b, (uint32_t)w.plane1 + 8u * col, soff);
    r.h = bld4(b, (uint32_t)w.plane2 + 4u * col, soff);
    const uint32_t sc = bld2(b, (uint32_t)w.plane3 + 2u * col, soff);
    const uint32_t d = bld2(b, 2u * (col >> 3), soff);
    r.sd = sc | (d << 16);
    return r;
}

// Four bits b0..b3 of t (t < 16) to bit 2 of bytes 0..3 (see spread4_bit4).
__device__ __forceinline__ uint32_t spread4_bit2(uint32_t t) { return ((t * 0x00204081u) & 0x01010101u) << 2; }

// The 3-bit values (low | high << 2, the reference's value + 4) of
// positions 16 h + 4 i .. + 3 of a Q3_K unit, one per byte.
__device__ __forceinline__ uint32_t q3_vals(const RawQ3_K &r, int h, int i) {
    const uint32_t w = h ? r.q.y : r.q.x;
    return ((w >> (2 * i)) & 0x03030303u) | spread4_bit2((r.h >> (16 * h + 4 * i)) & 0xFu);
}

// Four bits b0..b3 of t (t < 16) to bit 4 of bytes 0..3: t * 0x00204081
// puts copies of t at bits 0, 7, 14 and 21 (no overlap, so no carries),
// and bit j of t then sits at bit 8j; shifted to 8j + 4.
__device__ __forceinline__ uint32_t spread4_bit4(uint32_t t) { return ((t * 0x00204081u) & 0x01010101u) << 4; }

// The 5-bit values of positions 4i..4i+3 of Q5_K group halves, one per
// byte: nibbles of qs word x (low or high) with the 5th bits from hb.
__device__ __forceinline__ uint32_t q5_lo(uint32_t x, uint32_t hb_lo, int i) {
    return (x & NIB) | spread4_bit4((hb_lo >> (4 * i)) & 0xFu);
}
__device__ __forceinline__ uint32_t q5_hi(uint32_t x, uint32_t hb_hi, int i) {
    return ((x >> 4) & NIB) | spread4_bit4((hb_hi >> (4 * i)) & 0xFu);
}

// Q6_K super-block sb of row `row` (LAYOUT_IL64_Q6_K: chunk c of rows
// r..r+63 contiguous, so a wave of 64 rows reads 1 KB per chunk).
__device__ __forceinline__ void ld_q6_k(const DevWeight &w, size_t row, int sb, RawQ6_K &r) {
    const uint8_t *sp = w.base + (row >> 6) * w.group_stride + (size_t)sb * IL64_Q6K_SB;
    const size_t lane = row & 63;
#pragma unroll
    for (int j = 0; j < 13; j++) r.c[j] = ldw16(sp + ((size_t)j * 64 + lane) * 16);
    r.d = ldw2(sp + IL64_Q6K_D + lane * 2);
}

// The four 6-bit value words (+32 offset, one byte per l) of positions
// l..l+3 (m = 0), +32 (m = 1), +64 (m = 2), +96 (m = 3) of half o,
// l = 4 * lq (rce-op-qmm/src/lib.rs L425-454 bit layout: ql = c[0..7],
// qh = c[8..11]).
__device__ __forceinline__ void q6_words(const RawQ6_K &b, int o, int lq, uint32_t &u1, uint32_t &u2,
                                         uint32_t &u3, uint32_t &u4) {
    const int c = lq >> 2, wi = lq & 3;
    const uint32_t qa = wrd(b.c[4 * o + c], wi), qb = wrd(b.c[4 * o + 2 + c], wi);
    const uint32_t qh = wrd(b.c[8 + 2 * o + c], wi);
    u1 = (qa & NIB) | ((qh & 0x03030303u) << 4);
    u2 = (qb & NIB) | ((qh & 0x0C0C0C0Cu) << 2);
    u3 = ((qa >> 4) & NIB) | (qh & 0x30303030u);
    u4 = ((qb >> 4) & NIB) | ((qh >> 2) & 0x30303030u);
}

__device__ __forceinline__ int q6_sc(const uint4 &s, int i) {
    return (int)(int8_t)((wrd(s, i >> 2) >> (8 * (i & 3))) & 0xFFu);
}

// ---------------------------------------------------------------------------
// Q8 activations in LDS: per token t, xq words [k/4], dx [k/32] (the block
// scale round_to_f16(amax/127)), s16 [k/16] (sums of xq over 16 values).
// ---------------------------------------------------------------------------

struct ActLds {
    int *xq;
    float *dx;
    int *s16;
    __device__ ActLds(unsigned char *lds, size_t k, int tb) {
        xq = reinterpret_cast<int *>(lds);
        dx = reinterpret_cast<float *>(lds + (size_t)tb * k);
        s16 = reinterpret_cast<int *>(lds + (size_t)tb * k + (size_t)tb * (k / 32) * 4);
    }
};

__host__ __device__ constexpr size_t act_lds_bytes(size_t k, int tb) { return (size_t)tb * (k + k / 8 + k / 4); }

// Round half away from zero (f32::round / C roundf) of |v| <= 2^22, as an
// integer: v + copysign(pred(0.5), v) in round-to-nearest-even, truncated.
// Identical to roundf for every finite f32 in that range (checked
// exhaustively on the CPU, tests/test_round_identity.py); 3 instructions
// instead of roundf's 6.
__device__ __forceinline__ int round_half_away(float v) {
    return (int)(v + __builtin_copysignf(0x1.fffffep-2f, v));
}

// One task = 8 consecutive activation values of one token; four
// consecutive tasks (one lane quad) form a block of 32.
struct QuantTask {
    float4 v0, v1;
    float4 g0, g1;  // FX_NORM: the norm weights of the same 8 positions
};

// FX_NORM: the norm weights of the task's positions (out-of-range tasks read
// task 0's, like quant_task_load).
__device__ __forceinline__ void quant_task_load_g(const float *gw, int kq, int total, int task, QuantTask &q) {
    const int tk = task < total ? task : 0;
    const int e = (tk % kq) * 8;
    const float4 *p = reinterpret_cast<const float4 *>(gw + e);
    q.g0 = p[0];
    q.g1 = p[1];
}

// Sequential sum of the squares of the task's 8 values (0 for a task past
// the end): one task's share of rms_norm's sum of squares.
__device__ __forceinline__ float quant_task_ssq(const QuantTask &q, bool valid) {
    const float v[8] = {q.v0.x, q.v0.y, q.v0.z, q.v0.w, q.v1.x, q.v1.y, q.v1.z, q.v1.w};
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float sq = v[i] * v[i];
        s = s + sq;
    }
    return valid ? s : 0.0f;
}

__device__ __forceinline__ void quant_task_load(const float *A, int kq, int t0, int total, int task, QuantTask &q) {
    // kq = k / 8 tasks per token.  Out-of-range tasks load task 0 (always
    // valid), so the loads stay unconditional; they come in whole quads
    // (total is a multiple of 4) and quant_task_finish writes nothing for
    // them, so their values never reach a valid block.
    const int tk = task < total ? task : 0;
    const int t = tk / kq, e = (tk - t * kq) * 8;
    const float4 *p = reinterpret_cast<const float4 *>(A + (size_t)(t0 + t) * ((size_t)kq * 8) + e);
    q.v0 = p[0];
    q.v1 = p[1];
}

// nn.rs L541-563 quantize_block(x, false) of the quad's block: d = amax/127,
// id = 1/d (0 when d = 0), q = round half away from zero of x*id; the scale
// kept is round_to_f16(d) (nn.rs L521-533 = the hardware's RNE conversion).
// Every lane of the wave must call this (quad exchanges).
// NORM: the values are first normalized, (x * inv) * g (rms_norm's order).
template <bool NORM = false>
__device__ __forceinline__ void quant_task_finish(const QuantTask &q, size_t k, int total, int task, const ActLds &L,
                                                  float inv = 0.0f) {
    float v[8] = {q.v0.x, q.v0.y, q.v0.z, q.v0.w, q.v1.x, q.v1.y, q.v1.z, q.v1.w};
    if constexpr (NORM) {
        const float g[8] = {q.g0.x, q.g0.y, q.g0.z, q.g0.w, q.g1.x, q.g1.y, q.g1.z, q.g1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float t = v[i] * inv;
            v[i] = t * g[i];
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, quad_xor1f(amax));
    amax = fmaxf(amax, quad_xor2f(amax));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int w0 = 0, w1 = 0, s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int qi = round_half_away(v[i] * id);  // |v * id| <= 127
        s += qi;
        if (i < 4) w0 |= (int)(((uint32_t)qi & 0xFFu) << (8 * i));
        else w1 |= (int)(((uint32_t)qi & 0xFFu) << (8 * (i - 4)));
    }
    s += quad_xor1(s);  // the sum over this lane's half-block of 16
    if (task < total) {
        const size_t e = (size_t)task * 8;  // token-major: t*k + position
        *reinterpret_cast<int2 *>(L.xq + e / 4) = make_int2(w0, w1);
        if ((task & 1) == 0) L.s16[e / 16] = s;
        if ((task & 3) == 0) L.dx[e / 32] = (float)(_Float16)d;
    }
}

// ---------------------------------------------------------------------------
// Column units.  TB = tokens per thread.  init_*: the thread's activation
// slice; addends(raw, out): out[t] = the reference's per-unit term of
// row sum of token t.
// ---------------------------------------------------------------------------

// Q4_0 block, EXACT (rce-op-qmm/src/lib.rs L496-522): sub over q in 0..16
// of (lo_q - 8) a[q] then (hi_q - 8) a[q+16]; addend = scale * sub.
template <int TB>
struct Q4_0Exact {
    static constexpr int NTOK = TB;
    using Raw = RawQ4_0;
    float av[TB][32];
    __device__ static Raw load(const DevWeight &w, size_t row, int col) { return ld_q4_0(w, row, col); }
    __device__ static Raw load_b(const DevWeight &w, const WBuf &b, uint32_t soff, int col) { return bl_q4_0(w, b, soff, col); }
    __device__ void init(const float *A, size_t k, int t0, int tv, int col) {
#pragma unroll
        for (int t = 0; t < TB; t++) {
            // Tokens past tv read token 0's slice (no branch: a load inside
            // a branch is waited for before the branch joins); their sums
            // are never folded or stored.
            load_f32x(A + ((size_t)t0 + (t < tv ? t : 0)) * k + 32 * (size_t)col, av[t], 32);
        }
    }
    __device__ void addends(const Raw &r, float *out) const {
        float sub[TB];
#pragma unroll
        for (int t = 0; t < TB; t++) sub[t] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t x = wrd(r.q, i);
            float nls[4], nhs[4];
            nib4f<false>(and_opaque(x, NIB), nls);
            nib4f<false>(and_opaque(x >> 4, NIB), nhs);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float nl = nls[j], nh = nhs[j];
                if constexpr (TB == 1) {
                    sub[0] = sub[0] + __builtin_fmaf(nl, av[0][4 * i + j], -8.0f * av[0][4 * i + j]);
                    sub[0] = sub[0] + __builtin_fmaf(nh, av[0][4 * i + j + 16], -8.0f * av[0][4 * i + j + 16]);
                } else {
                    const float vl = nl - 8.0f, vh = nh - 8.0f;  // exact
#pragma unroll
                    for (int t = 0; t < TB; t++) {
                        sub[t] = sub[t] + vl * av[t][4 * i + j];
                        sub[t] = sub[t] + vh * av[t][4 * i + j + 16];
                    }
                }
            }
        }
        const float scale = h2f(r.s);
#pragma unroll
        for (int t = 0; t < TB; t++) out[t] = scale * sub[t];
    }
    // FX_NORM: the slice becomes (x * inv) * g (one token).
    __device__ void normalize(const float *gw, int col, float inv) {
        float g[32];
        load_f32x(gw + 32 * (size_t)col, g, 32);
#pragma unroll
        for (int l = 0; l < 32; l++) { const float t = av[0][l] * inv; av[0][l] = t * g[l]; }
    }
};

// Q8_0 block, EXACT (rce-op-qmm/src/lib.rs L315-328, L648-670).
template <int TB>
struct Q8_0Exact {
    static constexpr int NTOK = TB;
    using Raw = RawQ8_0;
    float av[TB][32];
    __device__ static Raw load(const DevWeight &w, size_t row, int col) { return ld_q8_0(w, row, col); }
    __device__ static Raw load_b(const DevWeight &w, const WBuf &b, uint32_t soff, int col) { return bl_q8_0(w, b, soff, col); }
    __device__ void init(const float *A, size_t k, int t0, int tv, int col) {
#pragma unroll
        for (int t = 0; t < TB; t++) {
            // Tokens past tv read token 0's slice (no branch: a load inside
            // a branch is waited for before the branch joins); their sums
            // are never folded or stored.
            load_f32x(A + ((size_t)t0 + (t < tv ? t : 0)) * k + 32 * (size_t)col, av[t], 32);
        }
    }
    __device__ void addends(const Raw &r, float *out) const {
        float sub[TB];
#pragma unroll
        for (int t = 0; t < TB; t++) sub[t] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t x = i < 4 ? wrd(r.q0, i) : wrd(r.q1, i - 4);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float v = (float)(int8_t)(x >> (8 * j));
#pragma unroll
                for (int t = 0; t < TB; t++) sub[t] = sub[t] + v * av[t][4 * i + j];
            }
        }
        const float scale = h2f(r.s);
#pragma unroll
        for (int t = 0; t < TB; t++) out[t] = scale * sub[t];
    }
    __device__ void normalize(const float *gw, int col, float inv) {
        float g[32];
        load_f32x(gw + 32 * (size_t)col, g, 32);
#pragma unroll
        for (int l = 0; l < 32; l++) { const float t = av[0][l] * inv; av[0][l] = t * g[l]; }
    }
};

// Q5_0 block, EXACT (rce-op-qmm/src/lib.rs L331-352, L525-561): Q4_0's
// order with 5-bit values: position j (< 16: low nibble of qs byte j,
// else high nibble of byte j - 16) takes bit j of qh as its fifth bit, and
// the value is that minus 16.
template <int TB>
struct Q5_0Exact {
    static constexpr int NTOK = TB;
    using Raw = RawQ5_0;
    float av[TB][32];
    __device__ static Raw load(const DevWeight &w, size_t row, int col) { return ld_q5_0(w, row, col); }
    __device__ static Raw load_b(const DevWeight &w, const WBuf &b, uint32_t soff, int col) { return bl_q5_0(w, b, soff, col); }
    __device__ void init(const float *A, size_t k, int t0, int tv, int col) {
#pragma unroll
        for (int t = 0; t < TB; t++)
            load_f32x(A + ((size_t)t0 + (t < tv ? t : 0)) * k + 32 * (size_t)col, av[t], 32);
    }
    __device__ void addends(const Raw &r, float *out) const {
        float sub[TB];
#pragma unroll
        for (int t = 0; t < TB; t++) sub[t] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t x = wrd(r.q, i);
            const uint32_t lo = and_opaque(x, NIB) | spread4_bit4((r.h >> (4 * i)) & 0xFu);
            const uint32_t hi = and_opaque(x >> 4, NIB) | spread4_bit4((r.h >> (16 + 4 * i)) & 0xFu);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float nl = (float)((lo >> (8 * j)) & 0xFFu), nh = (float)((hi >> (8 * j)) & 0xFFu);
                if constexpr (TB == 1) {  // (n - 16) a as fma(n, a, -16a): one rounding, like the product
                    sub[0] = sub[0] + __builtin_fmaf(nl, av[0][4 * i + j], -16.0f * av[0][4 * i + j]);
                    sub[0] = sub[0] + __builtin_fmaf(nh, av[0][4 * i + j + 16], -16.0f * av[0][4 * i + j + 16]);
                } else {
                    const float vl = nl - 16.0f, vh = nh - 16.0f;  // exact
#pragma unroll
                    for (int t = 0; t < TB; t++) {
                        sub[t] = sub[t] + vl * av[t][4 * i + j];
                        sub[t] = sub[t] + vh * av[t][4 * i + j + 16];
                    }
                }
            }
        }
        const float scale = h2f(r.s);
#pragma unroll
        for (int t = 0; t < TB; t++) out[t] = scale * sub[t];
    }
    __device__ void normalize(const float *gw, int col, float inv) {
        float g[32];
        load_f32x(gw + 32 * (size_t)col, g, 32);
#pragma unroll
        for (int l = 0; l < 32; l++) { const float t = av[0][l] * inv; av[0][l] = t * g[l]; }
    }
};

// Q4_1 block, EXACT (rce-op-qmm/src/lib.rs L615-645): va over q in 0..16
// of (v0 a[q] + v1 a[q+16]) and asum of (a[q] + a[q+16]), both from +0.0;
// addend = scale va + min asum.  asum does not depend on the row and is
// formed once per thread, in the same order.
template <int TB>
struct Q4_1Exact {
    static constexpr int NTOK = TB;
    using Raw = RawQ4_1;
    float av[TB][32];
    float as[TB];
    __device__ static Raw load(const DevWeight &w, size_t row, int col) { return ld_q4_1(w, row, col); }
    __device__ static Raw load_b(const DevWeight &w, const WBuf &b, uint32_t soff, int col) { return bl_q4_1(w, b, soff, col); }
    __device__ void sums() {
#pragma unroll
        for (int t = 0; t < TB; t++) {
            as[t] = 0.0f;
#pragma unroll
            for (int q = 0; q < 16; q++) as[t] = as[t] + (av[t][q] + av[t][q + 16]);
        }
    }
    __device__ void init(const float *A, size_t k, int t0, int tv, int col) {
#pragma unroll
        for (int t = 0; t < TB; t++)
            load_f32x(A + ((size_t)t0 + (t < tv ? t : 0)) * k + 32 * (size_t)col, av[t], 32);
    }
    __device__ void prepare() { sums(); }  // after the weight loads are out
    __device__ void addends(const Raw &r, float *out) const {
        float va[TB];
#pragma unroll
        for (int t = 0; t < TB; t++) va[t] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t x = wrd(r.q, i);
            float nls[4], nhs[4];
            nib4f<false>(and_opaque(x, NIB), nls);
            nib4f<false>(and_opaque(x >> 4, NIB), nhs);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float nl = nls[j], nh = nhs[j];
#pragma unroll
                for (int t = 0; t < TB; t++) {
                    const float p = nl * av[t][4 * i + j], q = nh * av[t][4 * i + j + 16];
                    va[t] = va[t] + (p + q);
                }
            }
        }
        const float scale = h2f(r.sm & 0xFFFFu), mn = h2f(r.sm >> 16);
#pragma unroll
        for (int t = 0; t < TB; t++) {
            const float u = scale * va[t], v = mn * as[t];
            out[t] = u + v;
        }
    }
    __device__ void normalize(const float *gw, int col, float inv) {
        float g[32];
        load_f32x(gw + 32 * (size_t)col, g, 32);
#pragma unroll
        for (int l = 0; l < 32; l++) { const float t = av[0][l] * inv; av[0][l] = t * g[l]; }
    }
};

// Q3_K unit (outer o, j) of a super-block, EXACT (rce-op-qmm/src/lib.rs
// L840-928): s1 over l < 16 of q a[l], s2 over l < 16 of q a[16 + l], both
// from +0.0 with q = (low | high << 2) - 4; addend = dl1 s1 + dl2 s2 with
// dl = d * (scale - 32).
template <int TB>
struct Q3_KExact {
    static constexpr int NTOK = TB;
    using Raw = RawQ3_K;
    float av[TB][32];
    __device__ static Raw load(const DevWeight &w, size_t row, int col) { return ld_q3_k(w, row, col); }
    __device__ static Raw load_b(const DevWeight &w, const WBuf &b, uint32_t soff, int col) { return bl_q3_k(w, b, soff, col); }
    __device__ void init(const float *A, size_t k, int t0, int tv, int col) {
#pragma unroll
        for (int t = 0; t < TB; t++)
            load_f32x(A + ((size_t)t0 + (t < tv ? t : 0)) * k + 32 * (size_t)col, av[t], 32);
    }
    __device__ void addends(const Raw &r, float *out) const {
        float s1[TB], s2[TB];
#pragma unroll
        for (int t = 0; t < TB; t++) { s1[t] = 0.0f; s2[t] = 0.0f; }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float n1s[4], n2s[4];
            nib4f<false>(q3_vals(r, 0, i), n1s);  // values 0..7
            nib4f<false>(q3_vals(r, 1, i), n2s);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float n1 = n1s[j], n2 = n2s[j];
                const int p = 4 * i + j;
                if constexpr (TB == 1) {  // (n - 4) a as fma(n, a, -4a): one rounding, like the product
                    s1[0] = s1[0] + __builtin_fmaf(n1, av[0][p], -4.0f * av[0][p]);
                    s2[0] = s2[0] + __builtin_fmaf(n2, av[0][16 + p], -4.0f * av[0][16 + p]);
                } else {
                    const float q1 = n1 - 4.0f, q2 = n2 - 4.0f;  // exact
#pragma unroll
                    for (int t = 0; t < TB; t++) {
                        s1[t] = s1[t] + q1 * av[t][p];
                        s2[t] = s2[t] + q2 * av[t][16 + p];
                    }
                }
            }
        }
        const float d = h2f(r.sd >> 16);
        const float dl1 = d * (float)(int8_t)(r.sd & 0xFFu), dl2 = d * (float)(int8_t)((r.sd >> 8) & 0xFFu);
#pragma unroll
        for (int t = 0; t < TB; t++) {
            const float u = dl1 * s1[t], v = dl2 * s2[t];
            out[t] = u + v;
        }
    }
    __device__ void normalize(const float *gw, int col, float inv) {
        float g[32];
        load_f32x(gw + 32 * (size_t)col, g, 32);
#pragma unroll
        for (int l = 0; l < 32; l++) { const float t = av[0][l] * inv; av[0][l] = t * g[l]; }
    }
};

// Q4_K group g of a super-block, EXACT (rce-op-qmm/src/lib.rs L354-385,
// L730-781): va_lo, a_lo, va_hi, a_hi over l in 0..32 from +0.0, then
// ((d1 va_lo - min1 a_lo) + d2 va_hi) - min2 a_hi.  a_lo and a_hi do not
// depend on the row and are formed once per thread, in the same order.
template <int TB>
struct Q4_KExact {
    static constexpr int NTOK = TB;
    using Raw = RawQ4_K;
    float av[TB][64];
    float a_lo[TB], a_hi[TB];
    int g;
    __device__ static Raw load(const DevWeight &w, size_t row, int col) { return ld_q4_k(w, row, col); }
    __device__ static Raw load_b(const DevWeight &w, const WBuf &b, uint32_t soff, int col) { return bl_q4_k(w, b, soff, col); }
    __device__ void init(const float *A, size_t k, int t0, int tv, int col) {
        g = col & 3;
#pragma unroll
        for (int t = 0; t < TB; t++) {
            // Tokens past tv read token 0's slice (no branch: a load inside
            // a branch is waited for before the branch joins); their sums
            // are never folded or stored.
            load_f32x(A + ((size_t)t0 + (t < tv ? t : 0)) * k + 64 * (size_t)col, av[t], 64);
        }
    }
    // After the weight loads are out: the row-independent sums.
    __device__ void prepare() {
#pragma unroll
        for (int t = 0; t < TB; t++) {
            a_lo[t] = 0.0f;
            a_hi[t] = 0.0f;
#pragma unroll
            for (int l = 0; l < 32; l++) { a_lo[t] = a_lo[t] + av[t][l]; a_hi[t] = a_hi[t] + av[t][32 + l]; }
        }
    }
    __device__ void addends(const Raw &r, float *out) const {
        const float d = h2f(r.h.x & 0xFFFFu), dmin = h2f(r.h.x >> 16);
        int sc1, m1, sc2, m2;
        k4_scale_min_pair(r.h, g, sc1, m1, sc2, m2);
        const float d1 = d * (float)sc1, min1 = dmin * (float)m1;
        const float d2 = d * (float)sc2, min2 = dmin * (float)m2;
        float va_lo[TB], va_hi[TB];
#pragma unroll
        for (int t = 0; t < TB; t++) { va_lo[t] = 0.0f; va_hi[t] = 0.0f; }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t x = i < 4 ? wrd(r.q0, i) : wrd(r.q1, i - 4);
            float vls[4], vhs[4];
            nib4f<true>(and_opaque(x, NIB), vls);
            nib4f<true>(and_opaque(x >> 4, NIB), vhs);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float vl = vls[j], vh = vhs[j];
#pragma unroll
                for (int t = 0; t < TB; t++) {
                    va_lo[t] = va_lo[t] + vl * av[t][4 * i + j];
                    va_hi[t] = va_hi[t] + vh * av[t][32 + 4 * i + j];
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TB; t++) {
            float s = d1 * va_lo[t];
            s = s - min1 * a_lo[t];
            s = s + d2 * va_hi[t];
            s = s - min2 * a_hi[t];
            out[t] = s;
        }
    }
    // FX_NORM: the slice becomes (x * inv) * g (prepare forms the sums after).
    __device__ void normalize(const float *gw, int col, float inv) {
        float g[64];
        load_f32x(gw + 64 * (size_t)col, g, 64);
#pragma unroll
        for (int l = 0; l < 64; l++) { const float t = av[0][l] * inv; av[0][l] = t * g[l]; }
    }
};

// Q5_K group, EXACT (rce-op-qmm/src/lib.rs L388-422, L783-838): Q4_K's
// group formula with the 5-bit values (nibble | h << 4).
template <int TB>
struct Q5_KExact {
    static constexpr int NTOK = TB;
    using Raw = RawQ5_K;
    float av[TB][64];
    float a_lo[TB], a_hi[TB];
    int g;
    __device__ static Raw load(const DevWeight &w, size_t row, int col) { return ld_q5_k(w, row, col); }
    __device__ static Raw load_b(const DevWeight &w, const WBuf &b, uint32_t soff, int col) { return bl_q5_k(w, b, soff, col); }
    __device__ void init(const float *A, size_t k, int t0, int tv, int col) {
        g = col & 3;
#pragma unroll
        for (int t = 0; t < TB; t++)  // tokens past tv read token 0's slice (never folded)
            load_f32x(A + ((size_t)t0 + (t < tv ? t : 0)) * k + 64 * (size_t)col, av[t], 64);
    }
    // After the weight loads are out: the row-independent sums.
    __device__ void prepare() {
#pragma unroll
        for (int t = 0; t < TB; t++) {
            a_lo[t] = 0.0f;
            a_hi[t] = 0.0f;
#pragma unroll
            for (int l = 0; l < 32; l++) { a_lo[t] = a_lo[t] + av[t][l]; a_hi[t] = a_hi[t] + av[t][32 + l]; }
        }
    }
    __device__ void addends(const Raw &r, float *out) const {
        const float d = h2f(r.h.x & 0xFFFFu), dmin = h2f(r.h.x >> 16);
        int sc1, m1, sc2, m2;
        k4_scale_min_pair(r.h, g, sc1, m1, sc2, m2);
        const float d1 = d * (float)sc1, min1 = dmin * (float)m1;
        const float d2 = d * (float)sc2, min2 = dmin * (float)m2;
        float va_lo[TB], va_hi[TB];
#pragma unroll
        for (int t = 0; t < TB; t++) { va_lo[t] = 0.0f; va_hi[t] = 0.0f; }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t x = i < 4 ? wrd(r.q0, i) : wrd(r.q1, i - 4);
            const uint32_t lo = q5_lo(x, r.hb.x, i), hi = q5_hi(x, r.hb.y, i);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float vl = (float)((lo >> (8 * j)) & 0xFFu), vh = (float)((hi >> (8 * j)) & 0xFFu);
#pragma unroll
                for (int t = 0; t < TB; t++) {
                    va_lo[t] = va_lo[t] + vl * av[t][4 * i + j];
                    va_hi[t] = va_hi[t] + vh * av[t][32 + 4 * i + j];
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TB; t++) {
            float s = d1 * va_lo[t];
            s = s - min1 * a_lo[t];
            s = s + d2 * va_hi[t];
            s = s - min2 * a_hi[t];
            out[t] = s;
        }
    }
    __device__ void normalize(const float *gw, int col, float inv) {
        float gv[64];
        load_f32x(gw + 64 * (size_t)col, gv, 64);
#pragma unroll
        for (int l = 0; l < 64; l++) { const float t = av[0][l] * inv; av[0][l] = t * gv[l]; }
    }
};

// Blocks of 32, Q8.  Q4_0 / Q8_0 / Q5_0: sub = dx * isum, addend =
// scale * sub (the offsets 8 and 16 enter isum as -8 xs, -16 xs, with xs
// the sum of the block's xq).  Q4_1: va = dx * isum over the raw nibbles,
// a = dx * xs, addend = scale va + min a.
enum Blk32 { B32_Q8_0, B32_Q4_0, B32_Q5_0, B32_Q4_1 };
template <int KIND> struct Blk32Raw;
template <> struct Blk32Raw<B32_Q8_0> { using T = RawQ8_0; };
template <> struct Blk32Raw<B32_Q4_0> { using T = RawQ4_0; };
template <> struct Blk32Raw<B32_Q5_0> { using T = RawQ5_0; };
template <> struct Blk32Raw<B32_Q4_1> { using T = RawQ4_1; };

template <int TB, int KIND>
struct Q32Q8 {
    static constexpr int NTOK = TB;
    static constexpr bool IS_Q4 = KIND == B32_Q4_0;
    using Raw = typename Blk32Raw<KIND>::T;
    int xq[TB][8];
    float dx[TB];
    int xs[TB];
    __device__ static Raw load(const DevWeight &w, size_t row, int col) {
        if constexpr (KIND == B32_Q4_0) return ld_q4_0(w, row, col);
        else if constexpr (KIND == B32_Q5_0) return ld_q5_0(w, row, col);
        else if constexpr (KIND == B32_Q4_1) return ld_q4_1(w, row, col);
        else return ld_q8_0(w, row, col);
    }
    __device__ static Raw load_b(const DevWeight &w, const WBuf &b, uint32_t soff, int col) {
        if constexpr (KIND == B32_Q4_0) return bl_q4_0(w, b, soff, col);
        else if constexpr (KIND == B32_Q5_0) return bl_q5_0(w, b, soff, col);
        else if constexpr (KIND == B32_Q4_1) return bl_q4_1(w, b, soff, col);
        else return bl_q8_0(w, b, soff, col);
    }
    __device__ void init_q8(const ActLds &L, size_t k, int tv, int col) {
#pragma unroll
        for (int t = 0; t < TB; t++) {
            const bool ok = t < tv;
            const size_t tt = ok ? (size_t)t : 0;
            const int4 *p = reinterpret_cast<const int4 *>(L.xq + (tt * k + 32 * (size_t)col) / 4);
            const int4 a = p[0], b = p[1];
            const int v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 8; i++) xq[t][i] = ok ? v[i] : 0;
            dx[t] = ok ? L.dx[tt * (k / 32) + col] : 0.0f;
            xs[t] = ok ? L.s16[tt * (k / 16) + 2 * col] + L.s16[tt * (k / 16) + 2 * col + 1] : 0;
        }
    }
    __device__ void addends(const Raw &r, float *out) const {
        if constexpr (KIND == B32_Q5_0 || KIND == B32_Q4_1) {
            int lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                lo[i] = (int)(wrd(r.q, i) & NIB);
                hi[i] = (int)((wrd(r.q, i) >> 4) & NIB);
                if constexpr (KIND == B32_Q5_0) {
                    lo[i] |= (int)spread4_bit4((r.h >> (4 * i)) & 0xFu);
                    hi[i] |= (int)spread4_bit4((r.h >> (16 + 4 * i)) & 0xFu);
                }
            }
#pragma unroll
            for (int t = 0; t < TB; t++) {
                int acc = 0;  // the 5-bit values are 0..31: positive as signed bytes
#pragma unroll
                for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_sdot4(lo[i], xq[t][i], acc, false);
#pragma unroll
                for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_sdot4(hi[i], xq[t][4 + i], acc, false);
                if constexpr (KIND == B32_Q5_0) {
                    const float sub = dx[t] * (float)(acc - 16 * xs[t]);
                    out[t] = h2f(r.s) * sub;
                } else {
                    const float va = dx[t] * (float)acc, a = dx[t] * (float)xs[t];
                    const float u = h2f(r.sm & 0xFFFFu) * va, v = h2f(r.sm >> 16) * a;
                    out[t] = u + v;
                }
            }
        } else if constexpr (IS_Q4) {
            const float scale = h2f(r.s);
            int lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; i++) { lo[i] = (int)(wrd(r.q, i) & NIB); hi[i] = (int)((wrd(r.q, i) >> 4) & NIB); }
#pragma unroll
            for (int t = 0; t < TB; t++) {
                int acc = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_sdot4(lo[i], xq[t][i], acc, false);
#pragma unroll
                for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_sdot4(hi[i], xq[t][4 + i], acc, false);
                const float sub = dx[t] * (float)(acc - 8 * xs[t]);
                out[t] = scale * sub;
            }
        } else {
            const float scale = h2f(r.s);
#pragma unroll
            for (int t = 0; t < TB; t++) {
                int acc = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_sdot4((int)wrd(r.q0, i), xq[t][i], acc, false);
#pragma unroll
                for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_sdot4((int)wrd(r.q1, i), xq[t][4 + i], acc, false);
                const float sub = dx[t] * (float)acc;
                out[t] = scale * sub;
            }
        }
    }
};

// Q3_K unit, Q8: s1 = dx * isum1, s2 = dx * isum2 over the two halves of
// 16 (isum = dot of the 3-bit values with xq, minus 4 times the half's xq
// sum); addend = dl1 s1 + dl2 s2.
template <int TB>
struct Q3_KQ8 {
    static constexpr int NTOK = TB;
    using Raw = RawQ3_K;
    int xq[TB][8];
    float dx[TB];
    int xs1[TB], xs2[TB];
    __device__ static Raw load(const DevWeight &w, size_t row, int col) { return ld_q3_k(w, row, col); }
    __device__ static Raw load_b(const DevWeight &w, const WBuf &b, uint32_t soff, int col) { return bl_q3_k(w, b, soff, col); }
    __device__ void init_q8(const ActLds &L, size_t k, int tv, int col) {
#pragma unroll
        for (int t = 0; t < TB; t++) {
            const bool ok = t < tv;
            const size_t tt = ok ? (size_t)t : 0;
            const int4 *p = reinterpret_cast<const int4 *>(L.xq + (tt * k + 32 * (size_t)col) / 4);
            const int4 a = p[0], b = p[1];
            const int v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 8; i++) xq[t][i] = ok ? v[i] : 0;
            dx[t] = ok ? L.dx[tt * (k / 32) + col] : 0.0f;
            xs1[t] = ok ? L.s16[tt * (k / 16) + 2 * col] : 0;
            xs2[t] = ok ? L.s16[tt * (k / 16) + 2 * col + 1] : 0;
        }
    }
    __device__ void addends(const Raw &r, float *out) const {
        int v1[4], v2[4];
#pragma unroll
        for (int i = 0; i < 4; i++) { v1[i] = (int)q3_vals(r, 0, i); v2[i] = (int)q3_vals(r, 1, i); }
        const float d = h2f(r.sd >> 16);
        const float dl1 = d * (float)(int8_t)(r.sd & 0xFFu), dl2 = d * (float)(int8_t)((r.sd >> 8) & 0xFFu);
#pragma unroll
        for (int t = 0; t < TB; t++) {
            int a1 = 0, a2 = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) a1 = __builtin_amdgcn_sdot4(v1[i], xq[t][i], a1, false);
#pragma unroll
            for (int i = 0; i < 4; i++) a2 = __builtin_amdgcn_sdot4(v2[i], xq[t][4 + i], a2, false);
            const float s1 = dx[t] * (float)(a1 - 4 * xs1[t]), s2 = dx[t] * (float)(a2 - 4 * xs2[t]);
            const float u = dl1 * s1, v = dl2 * s2;
            out[t] = u + v;
        }
    }
};

// Q4_K group, Q8: va = dx * isum, a = dx * (sum of xq); then the EXACT
// group formula.
template <int TB>
struct Q4_KQ8 {
    static constexpr int NTOK = TB;
    using Raw = RawQ4_K;
    int xl[TB][8], xh[TB][8];
    float dl[TB], dh[TB];
    int sl[TB], sh[TB];
    int g;
    __device__ static Raw load(const DevWeight &w, size_t row, int col) { return ld_q4_k(w, row, col); }
    __device__ static Raw load_b(const DevWeight &w, const WBuf &b, uint32_t soff, int col) { return bl_q4_k(w, b, soff, col); }
    __device__ void init_q8(const ActLds &L, size_t k, int tv, int col) {
        g = col & 3;
#pragma unroll
        for (int t = 0; t < TB; t++) {
            // tokens past tv read token 0's slice and are zeroed (no branch)
            const bool ok = t < tv;
            const size_t tt = ok ? (size_t)t : 0;
            const int4 *p = reinterpret_cast<const int4 *>(L.xq + (tt * k + 64 * (size_t)col) / 4);
            const int4 a = p[0], b = p[1], c = p[2], e = p[3];
            const int v[16] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y, c.z, c.w, e.x, e.y, e.z, e.w};
#pragma unroll
            for (int i = 0; i < 8; i++) { xl[t][i] = ok ? v[i] : 0; xh[t][i] = ok ? v[8 + i] : 0; }
            const size_t b32 = tt * (k / 32) + 2 * (size_t)col, b16 = tt * (k / 16) + 4 * (size_t)col;
            dl[t] = ok ? L.dx[b32] : 0.0f;
            dh[t] = ok ? L.dx[b32 + 1] : 0.0f;
            sl[t] = ok ? L.s16[b16] + L.s16[b16 + 1] : 0;
            sh[t] = ok ? L.s16[b16 + 2] + L.s16[b16 + 3] : 0;
        }
    }
    __device__ void addends(const Raw &r, float *out) const {
        const float d = h2f(r.h.x & 0xFFFFu), dmin = h2f(r.h.x >> 16);
        int sc1, m1, sc2, m2;
        k4_scale_min_pair(r.h, g, sc1, m1, sc2, m2);
        const float d1 = d * (float)sc1, min1 = dmin * (float)m1;
        const float d2 = d * (float)sc2, min2 = dmin * (float)m2;
        int lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t x = i < 4 ? wrd(r.q0, i) : wrd(r.q1, i - 4);
            lo[i] = (int)(x & NIB);
            hi[i] = (int)((x >> 4) & NIB);
        }
#pragma unroll
        for (int t = 0; t < TB; t++) {
            int il = 0, ih = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                il = __builtin_amdgcn_sdot4(lo[i], xl[t][i], il, false);
                ih = __builtin_amdgcn_sdot4(hi[i], xh[t][i], ih, false);
            }
            const float va_lo = dl[t] * (float)il, a_lo = dl[t] * (float)sl[t];
            const float va_hi = dh[t] * (float)ih, a_hi = dh[t] * (float)sh[t];
            float s = d1 * va_lo;
            s = s - min1 * a_lo;
            s = s + d2 * va_hi;
            s = s - min2 * a_hi;
            out[t] = s;
        }
    }
};

// Q5_K group, Q8: Q4_KQ8 with the 5-bit values (0..31, so sdot4 applies).
template <int TB>
struct Q5_KQ8 {
    static constexpr int NTOK = TB;
    using Raw = RawQ5_K;
    int xl[TB][8], xh[TB][8];
    float dl[TB], dh[TB];
    int sl[TB], sh[TB];
    int g;
    __device__ static Raw load(const DevWeight &w, size_t row, int col) { return ld_q5_k(w, row, col); }
    __device__ static Raw load_b(const DevWeight &w, const WBuf &b, uint32_t soff, int col) { return bl_q5_k(w, b, soff, col); }
    __device__ void init_q8(const ActLds &L, size_t k, int tv, int col) {
        g = col & 3;
#pragma unroll
        for (int t = 0; t < TB; t++) {
            const bool ok = t < tv;
            const size_t tt = ok ? (size_t)t : 0;
            const int4 *p = reinterpret_cast<const int4 *>(L.xq + (tt * k + 64 * (size_t)col) / 4);
            const int4 a = p[0], b = p[1], c = p[2], e = p[3];
            const int v[16] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y, c.z, c.w, e.x, e.y, e.z, e.w};
#pragma unroll
            for (int i = 0; i < 8; i++) { xl[t][i] = ok ? v[i] : 0; xh[t][i] = ok ? v[8 + i] : 0; }
            const size_t b32 = tt * (k / 32) + 2 * (size_t)col, b16 = tt * (k / 16) + 4 * (size_t)col;
            dl[t] = ok ? L.dx[b32] : 0.0f;
            dh[t] = ok ? L.dx[b32 + 1] : 0.0f;
            sl[t] = ok ? L.s16[b16] + L.s16[b16 + 1] : 0;
            sh[t] = ok ? L.s16[b16 + 2] + L.s16[b16 + 3] : 0;
        }
    }
    __device__ void addends(const Raw &r, float *out) const {
        const float d = h2f(r.h.x & 0xFFFFu), dmin = h2f(r.h.x >> 16);
        int sc1, m1, sc2, m2;
        k4_scale_min_pair(r.h, g, sc1, m1, sc2, m2);
        const float d1 = d * (float)sc1, min1 = dmin * (float)m1;
        const float d2 = d * (float)sc2, min2 = dmin * (float)m2;
        int lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t x = i < 4 ? wrd(r.q0, i) : wrd(r.q1, i - 4);
            lo[i] = (int)q5_lo(x, r.hb.x, i);
            hi[i] = (int)q5_hi(x, r.hb.y, i);
        }
#pragma unroll
        for (int t = 0; t < TB; t++) {
            int il = 0, ih = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                il = __builtin_amdgcn_sdot4(lo[i], xl[t][i], il, false);
                ih = __builtin_amdgcn_sdot4(hi[i], xh[t][i], ih, false);
            }
            const float va_lo = dl[t] * (float)il, a_lo = dl[t] * (float)sl[t];
            const float va_hi = dh[t] * (float)ih, a_hi = dh[t] * (float)sh[t];
            float s = d1 * va_lo;
            s = s - min1 * a_lo;
            s = s + d2 * va_hi;
            s = s - min2 * a_hi;
            out[t] = s;
        }
    }
};

// Q6_K super-block, Q8: for sub-blocks b of 16 ascending,
// ssb += (d sc_b) (dx isum_b) from +0.0; the addend is ssb.
template <int TB>
struct Q6_KQ8 {
    static constexpr int NTOK = TB;
    using Raw = RawQ6_K;
    int xw[TB][64];
    float dx[TB][8];
    int s16[TB][16];
    __device__ static Raw load(const DevWeight &w, size_t row, int col) {
        Raw r;
        ld_q6_k(w, row, col, r);
        return r;
    }
    __device__ void init_q8(const ActLds &L, size_t k, int tv, int col) {
#pragma unroll
        for (int t = 0; t < TB; t++) {
            const bool ok = t < tv;
            const size_t tt = ok ? (size_t)t : 0;
            const int4 *p = reinterpret_cast<const int4 *>(L.xq + (tt * k + 256 * (size_t)col) / 4);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int4 v = p[i];
                xw[t][4 * i] = ok ? v.x : 0; xw[t][4 * i + 1] = ok ? v.y : 0;
                xw[t][4 * i + 2] = ok ? v.z : 0; xw[t][4 * i + 3] = ok ? v.w : 0;
            }
#pragma unroll
            for (int i = 0; i < 8; i++) dx[t][i] = ok ? L.dx[tt * (k / 32) + 8 * (size_t)col + i] : 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) s16[t][i] = ok ? L.s16[tt * (k / 16) + 16 * (size_t)col + i] : 0;
        }
    }
    __device__ void addends(const Raw &b, float *out) const {
        const float d = h2f(b.d);
        float ssb[TB];
#pragma unroll
        for (int t = 0; t < TB; t++) ssb[t] = 0.0f;
#pragma unroll
        for (int o = 0; o < 2; o++) {
            int acc[TB][8];  // sub-block 8o + 2m + c -> index 2m + c
#pragma unroll
            for (int t = 0; t < TB; t++)
#pragma unroll
                for (int i = 0; i < 8; i++) acc[t][i] = 0;
#pragma unroll
            for (int lq = 0; lq < 8; lq++) {
                uint32_t u[4];
                q6_words(b, o, lq, u[0], u[1], u[2], u[3]);
                const int c = lq >> 2, wi = lq & 3;
#pragma unroll
                for (int m = 0; m < 4; m++) {
#pragma unroll
                    for (int t = 0; t < TB; t++)
                        acc[t][2 * m + c] = __builtin_amdgcn_sdot4((int)u[m], xw[t][32 * o + 8 * m + 4 * c + wi],
                                                                   acc[t][2 * m + c], false);
                }
            }
#pragma unroll
            for (int bb = 0; bb < 8; bb++) {
                const int sbk = 8 * o + bb;
                const float ds = d * (float)q6_sc(b.c[12], sbk);
#pragma unroll
                for (int t = 0; t < TB; t++) {
                    const int isum = acc[t][bb] - 32 * s16[t][sbk];
                    const float ab = dx[t][sbk >> 1] * (float)isum;
                    ssb[t] = ssb[t] + ds * ab;
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TB; t++) out[t] = ssb[t];
    }
};

// ---------------------------------------------------------------------------
// The activation-stationary kernel.
// ---------------------------------------------------------------------------

__host__ __device__ constexpr int fold_ld(int U) { return ((U + 3) & ~3) + 4; }

// Units with prepare(): work on the activations (row-independent sums) done
// after the weight loads are issued, so it does not hold them back.
template <class U, class = void> struct HasPrepare : std::false_type {};
template <class U> struct HasPrepare<U, std::void_t<decltype(std::declval<U &>().prepare())>> : std::true_type {};
// Units whose weights load through a WBuf (every layout with whole rows at
// row_stride; LAYOUT_IL64_Q6_K interleaves 64 rows and keeps the pointer form).
template <class U, class = void> struct HasLoadB : std::false_type {};
template <class U>
struct HasLoadB<U, std::void_t<decltype(U::load_b(std::declval<const DevWeight &>(), std::declval<const WBuf &>(),
                                                   0u, 0))>> : std::true_type {};

// Dynamic LDS a block may use (the default per-block limit).
constexpr size_t LDS_MAX = 64 * 1024;

inline size_t gemv_lds_bytes(int U, int nt, int rpl, int tb, bool q8, size_t k) {
    // the tile's addends, plus (when nt is not a multiple of U) one tile of
    // dummy rows for the idle lanes' stores
    const size_t rt = (size_t)(nt / U) * rpl;
    const size_t fold = ((size_t)tb * rt + (nt % U ? rt : 0)) * fold_ld(U) * sizeof(float);
    const size_t act = q8 ? act_lds_bytes(k, tb) : 0;
    return fold > act ? fold : act;
}

// FX (qmm_internal.h): 0 = the plain GEMV; FX_SEG, FX_RESIDUAL, FX_SWIGLU =
// the decode step's fused forms (`fx` is read only by them).
template <class Unit, int NT, int RPL, bool Q8, int FX>
__global__ __launch_bounds__(NT) void k_gemv_as(DevWeight w, const float *__restrict__ A, float *__restrict__ out,
                                                int t_rows, int U, GemvFx fx) {
    constexpr int TB = Unit::NTOK;
    constexpr int KIND = FX & 7;
    constexpr bool NORM = (FX & FX_NORM) != 0;
    constexpr bool PREQ = (FX & FX_PREQ) != 0;
    static_assert(!PREQ || (Q8 && KIND == 0 && !NORM), "pre-quantized activations: plain Q8 launches");
    static_assert(!NORM || TB == 1, "the normalizing forms are single-token");
    extern __shared__ __align__(16) unsigned char lds[];
    const int tid = threadIdx.x;
    const int P = NT / U;
    const int col = tid % U, rsub = tid / U;
    const bool active = rsub < P;
    const int RT = P * RPL;
    unsigned bx = blockIdx.x;
    if constexpr (KIND == FX_SEG) {  // block-uniform choice of the segment
        if (fx.pos && bx == 0 && tid == 0 && fx.status[2] == 0) {  // the step's last kernel: advance the position
            const int p = fx.pos[0];
            if (p >= fx.ctx_len && fx.status[0] == 0) fx.status[0] = 2;
            fx.pos[0] = p + 1;
        }
        if (bx >= fx.blk3) { w = fx.w3; out = fx.out3; bx -= fx.blk3; }
        else if (bx >= fx.blk2) { w = fx.w2; out = fx.out2; bx -= fx.blk2; }
    }
    // FX_SWIGLU: loads u < RPL / 2 read gate rows, the others the same up
    // rows; tile rows [0, RTO) are gate rows, [RTO, RT) the matching up rows.
    constexpr int HALF = RPL / 2;
    static_assert(KIND != FX_SWIGLU || RPL % 2 == 0, "swiglu pairs need an even row count per lane");
    const int RTO = KIND == FX_SWIGLU ? RT / 2 : RT;  // output rows of the block
    const size_t row0 = (size_t)bx * RTO;
    const int t0 = blockIdx.y * TB;
    const int tv = min(TB, t_rows - t0);
    const size_t k = w.n_cols;

    Unit unit;
    // Phase 1: activation loads first (they are not behind the weights in
    // the in-order load counter), then every weight load of the thread.
    // No load sits in a branch (the compiler waits for a load made inside
    // a branch before the branch joins, which would serialize the rows):
    // rows past the end read the allocation's zero padding
    // (layout_pad_bytes) and idle lanes a valid row; neither is folded.
    QuantTask qt0, qt1;
    const int kq = (int)(k / 8);
    // Q8: the block's quantization tasks; FX_NORM: the tasks of the sum of
    // squares (the host guarantees kq <= 2 NT, so qt0 and qt1 cover the row)
    const int qtotal = ((Q8 && !PREQ) || NORM) ? tv * kq : 0;
    if constexpr ((Q8 && !PREQ) || NORM) {
        quant_task_load(A, kq, t0, qtotal, tid, qt0);
        quant_task_load(A, kq, t0, qtotal, tid + NT, qt1);
    }
    if constexpr (Q8 && NORM) {
        quant_task_load_g(fx.norm_w, kq, qtotal, tid, qt0);
        quant_task_load_g(fx.norm_w, kq, qtotal, tid + NT, qt1);
    }
    if constexpr (!Q8) unit.init(A, k, t0, tv, col);
    __builtin_amdgcn_sched_barrier(0);  // activation loads stay ahead of the weights'
    typename Unit::Raw raw[RPL];
    const int rs = active ? rsub : P - 1;
    // Buffer loads: the buffer starts at the block's first row, the lane's
    // row within a pass is a VGPR, the pass (u P rows) a uniform soffset:
    // offsets stay below the block's own span, whatever the weight's size.
    WBuf wb1, wb2;
    if constexpr (HasLoadB<Unit>::value) {
        wb1 = make_wbuf(w.base + row0 * w.row_stride, (uint32_t)((size_t)rs * w.row_stride));
        if constexpr (KIND == FX_SWIGLU)
            wb2 = make_wbuf(fx.w2.base + row0 * fx.w2.row_stride, (uint32_t)((size_t)rs * fx.w2.row_stride));
    }
    auto issue = [&](int u) {
        const bool up = KIND == FX_SWIGLU && u >= HALF;
        const int uu = up ? u - HALF : u;
        if constexpr (HasLoadB<Unit>::value) {
            const DevWeight &ww = up ? fx.w2 : w;
            const uint32_t soff = (uint32_t)((size_t)(uu * P) * ww.row_stride);
            raw[u] = Unit::load_b(ww, up ? wb2 : wb1, soff, col);
        } else {
            const size_t r = row0 + (size_t)(uu * P + rs);
            raw[u] = Unit::load(up ? fx.w2 : w, r, col);
        }
    };
    constexpr int PF = PREFETCH_ROWS < RPL ? PREFETCH_ROWS : RPL;  // rows loaded ahead of the arithmetic
#pragma unroll
    for (int u = 0; u < PF; u++) issue(u);
    // Keep every load above ahead of any arithmetic on loaded data.
    __builtin_amdgcn_sched_barrier(0);
    // FX_NORM: rms_norm's scale from the whole row, while the weights load.
    float inv = 0.0f;
    if constexpr (NORM) {
        __shared__ float red[NT / 64];
        float ss = quant_task_ssq(qt0, tid < qtotal);
        ss = ss + quant_task_ssq(qt1, tid + NT < qtotal);
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int i = 0; i < NT / 64; i++) tot = tot + red[i];
        const float mean_sq = tot / (float)k;
        inv = 1.0f / sqrtf(mean_sq + fx.eps);
        if constexpr (!Q8) unit.normalize(fx.norm_w, col, inv);
    }
    // Phase 2 (Q8): quantize the block's activation rows into LDS (or, with
    // FX_PREQ, read the block's tokens from the pre-quantized buffer).
    if constexpr (PREQ) {
        const size_t T = (size_t)fx.preq_t;
        ActLds L(const_cast<unsigned char *>(fx.preq), k, (int)T);
        L.xq += (size_t)t0 * k / 4;
        L.dx += (size_t)t0 * (k / 32);
        L.s16 += (size_t)t0 * (k / 16);
        if (active) unit.init_q8(L, k, tv, col);
    } else if constexpr (Q8) {
        ActLds L(lds, k, TB);
        quant_task_finish<NORM>(qt0, k, qtotal, tid, L, inv);
        quant_task_finish<NORM>(qt1, k, qtotal, tid + NT, L, inv);
        for (int base = 2 * NT; base < qtotal; base += NT) {
            QuantTask q;
            quant_task_load(A, kq, t0, qtotal, base + tid, q);
            quant_task_finish(q, k, qtotal, base + tid, L);
        }
        __syncthreads();
        if (active) unit.init_q8(L, k, tv, col);
        __syncthreads();  // the fold below reuses the LDS
    }
    if constexpr (!Q8 && HasPrepare<Unit>::value) unit.prepare();
    // Phase 3: per-unit addends of every (token, row) to LDS.
    float *part = reinterpret_cast<float *>(lds);
    const int ld = fold_ld(U);
    // Store address of (token t, pass u): lane part + u P ld (uniform) +
    // t RT ld.  Idle lanes (rsub == P, only when NT % U != 0) store into
    // the dummy tile past the TB tiles, the same slot for every token.
    int lane_fold = (active ? rsub : TB * RT) * ld + col;
    int tok_fold = active ? RT * ld : 0;
    // opaque, so the optimizer cannot fold the uniform offsets back into a
    // per-row multiply
    asm volatile("" : "+v"(lane_fold), "+v"(tok_fold));
#pragma unroll
    for (int u = 0; u < RPL; u++) {
        if constexpr (PF < RPL) {  // the next rows' loads go out before this row's arithmetic
            if (u + PF < RPL) issue(u + PF);
            __builtin_amdgcn_sched_barrier(0);
        }
        // Every lane computes and stores, so no load is sunk into a guarded
        // branch; rows past n_rows store sums the fold below never reads.
        float ad[TB];
        unit.addends(raw[u], ad);
#pragma unroll
        for (int t = 0; t < TB; t++) part[lane_fold + u * (P * ld) + t * tok_fold] = ad[t];
    }
    __syncthreads();
    // Phase 4: the reference's fold, one thread per (token, output row).
    auto fold = [&](int t, int r) {
        const float *pp = part + (t * RT + r) * ld;
        const float4 *p4 = reinterpret_cast<const float4 *>(pp);
        float s = 0.0f;
        const int U4 = U >> 2;
#pragma unroll 8
        for (int c = 0; c < U4; c++) {
            const float4 v = p4[c];
            s = s + v.x;
            s = s + v.y;
            s = s + v.z;
            s = s + v.w;
        }
        for (int c = U4 * 4; c < U; c++) s = s + pp[c];
        return s;
    };
    for (int j = tid; j < tv * RTO; j += NT) {
        const int t = j / RTO, r = j % RTO;
        if (row0 + r < w.n_rows) {
            const size_t o = ((size_t)t0 + t) * w.n_rows + row0 + r;
            if constexpr (KIND == FX_SWIGLU) {
                const float g = fold(t, r), u = fold(t, RTO + r);
                out[o] = silu_ref(g) * u;  // rce-tinyllama L320: h = silu(g) * u
            } else if constexpr (KIND == FX_RESIDUAL) {
                out[o] = fx.res[o] + fold(t, r);  // rce-tinyllama L318, L323: x += ...
            } else {
                out[o] = fold(t, r);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Launch geometry.
// ---------------------------------------------------------------------------

inline int units_per_row(uint32_t dtype, size_t n_cols) {
    switch (dtype) {
    case T_Q4_0: case T_Q8_0: case T_Q5_0: case T_Q4_1: case T_Q3_K: return (int)(n_cols / 32);
    case T_Q1_0: case T_Q2_0: return (int)(n_cols / 128);
    case T_STQ1_0: return (int)(n_cols / 256);
    case T_Q4_K: case T_Q5_K: return (int)(n_cols / 64);
    case T_Q6_K: return (int)(n_cols / 256);
    default: return 0;
    }
}

inline int nt_for(int U) { return U <= 256 ? 256 : (U <= 512 ? 512 : 1024); }

// The buffer loads' offsets are 32-bit and relative to the block's first
// row: one block's rows must span less than 2^31 bytes.
inline bool wbuf_span_ok(const DevWeight &w, size_t tile_rows) {
    return tile_rows * w.row_stride < ((size_t)1 << 31);
}

template <class Unit, int NT, int RPL, bool Q8>
hipError_t launch_as(const DevWeight &w, int U, const float *a, size_t t_rows, float *out, hipStream_t s) {
    constexpr int TB = Unit::NTOK;
    const int P = NT / U, RT = P * RPL;
    if (P < 1) return hipErrorInvalidConfiguration;
    if (!wbuf_span_ok(w, RT)) return hipErrorInvalidValue;
    const size_t lds = gemv_lds_bytes(U, NT, RPL, TB, Q8, w.n_cols);
    if (lds > LDS_MAX) return hipErrorInvalidConfiguration;
    dim3 grid((unsigned)((w.n_rows + RT - 1) / RT), (unsigned)((t_rows + TB - 1) / TB)), block(NT);
    hipLaunchKernelGGL((k_gemv_as<Unit, NT, RPL, Q8, 0>), grid, block, lds, s, w, a, out, (int)t_rows, U, GemvFx{});
    return hipGetLastError();
}

// The fused forms (one token).  The caller has checked that the weights
// share dtype and n_cols (FX_SWIGLU: and n_rows).
template <class Unit, int NT, int RPL, bool Q8>
hipError_t launch_as_fx(const FxLaunch &f, int U, const float *a, hipStream_t s) {
    static_assert(Unit::NTOK == 1, "the fused forms are single-token");
    const int P = NT / U, RT = P * RPL;
    if (P < 1) return hipErrorInvalidConfiguration;
    for (int i = 0; i < f.nw && i < 3; i++)
        if (!wbuf_span_ok(f.w[i], RT)) return hipErrorInvalidValue;
    const size_t lds = gemv_lds_bytes(U, NT, RPL, 1, Q8, f.w[0].n_cols);
    if (lds > LDS_MAX) return hipErrorInvalidConfiguration;
    auto nblk = [&](const DevWeight &w, int rows_per_block) {
        return (unsigned)((w.n_rows + rows_per_block - 1) / rows_per_block);
    };
    GemvFx fx{};
    fx.norm_w = f.norm_w;
    fx.eps = f.eps;
    if (f.pos && ((f.kind & 7) != FX_SEG || !f.status)) return hipErrorInvalidValue;
    fx.pos = f.pos;
    fx.status = f.status;
    fx.ctx_len = f.ctx_len;
    if ((f.kind & FX_NORM) && (f.w[0].n_cols / 8 > (size_t)(2 * NT) || !f.norm_w)) return hipErrorInvalidValue;
    unsigned blocks = 0;
    switch (f.kind & 7) {
    case FX_SEG: {
        if (f.nw < 1 || f.nw > 3) return hipErrorInvalidValue;
        blocks = nblk(f.w[0], RT);
        fx.blk2 = fx.blk3 = ~0u;
        if (f.nw >= 2) { fx.w2 = f.w[1]; fx.out2 = f.out[1]; fx.blk2 = blocks; blocks += nblk(f.w[1], RT); }
        if (f.nw >= 3) { fx.w3 = f.w[2]; fx.out3 = f.out[2]; fx.blk3 = blocks; blocks += nblk(f.w[2], RT); }
        if (f.kind & FX_NORM)
            hipLaunchKernelGGL((k_gemv_as<Unit, NT, RPL, Q8, FX_SEG | FX_NORM>), dim3(blocks), dim3(NT), lds, s, f.w[0], a,
                               f.out[0], 1, U, fx);
        else
            hipLaunchKernelGGL((k_gemv_as<Unit, NT, RPL, Q8, FX_SEG>), dim3(blocks), dim3(NT), lds, s, f.w[0], a,
                               f.out[0], 1, U, fx);
        break;
    }
    case FX_RESIDUAL:
        if (f.kind & FX_NORM) return hipErrorInvalidValue;
        fx.res = f.res;
        hipLaunchKernelGGL((k_gemv_as<Unit, NT, RPL, Q8, FX_RESIDUAL>), dim3(nblk(f.w[0], RT)), dim3(NT), lds, s, f.w[0],
                           a, f.out[0], 1, U, fx);
        break;
    case FX_SWIGLU:
        if constexpr (RPL % 2 != 0) {
            return hipErrorInvalidValue;  // gate and up rows come in pairs
        } else {
            if (f.nw != 2 || f.w[1].n_rows != f.w[0].n_rows) return hipErrorInvalidValue;
            fx.w2 = f.w[1];
            if (f.kind & FX_NORM)
                hipLaunchKernelGGL((k_gemv_as<Unit, NT, RPL, Q8, FX_SWIGLU | FX_NORM>), dim3(nblk(f.w[0], RT / 2)),
                                   dim3(NT), lds, s, f.w[0], a, f.out[0], 1, U, fx);
            else
                hipLaunchKernelGGL((k_gemv_as<Unit, NT, RPL, Q8, FX_SWIGLU>), dim3(nblk(f.w[0], RT / 2)), dim3(NT), lds,
                                   s, f.w[0], a, f.out[0], 1, U, fx);
        }
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Shapes of the fused forms: the plain GEMV's threads per block, rows per
// lane 1, 2, 4 or 8 (FX_SWIGLU: even).
template <class Unit, bool Q8>
hipError_t launch_as_fx_nt(const FxLaunch &f, const GemvGeom &g, const float *a, hipStream_t s) {
    const int U = units_per_row(f.w[0].dtype, f.w[0].n_cols);
#define RCE_RPL_FX(NT)                                                      \
    switch (g.rpl) {                                                        \
    case 1: return launch_as_fx<Unit, NT, 1, Q8>(f, U, a, s);               \
    case 2: return launch_as_fx<Unit, NT, 2, Q8>(f, U, a, s);               \
    case 4: return launch_as_fx<Unit, NT, 4, Q8>(f, U, a, s);               \
    case 8: return launch_as_fx<Unit, NT, 8, Q8>(f, U, a, s);               \
    default: return hipErrorInvalidValue;                                   \
    }
    switch (g.nt) {
    case 256: RCE_RPL_FX(256)
    case 512: RCE_RPL_FX(512)
    case 1024: RCE_RPL_FX(1024)
    default: return hipErrorInvalidValue;
    }
#undef RCE_RPL_FX
}

template <class Unit, bool Q8>
hipError_t launch_as_nt(const DevWeight &w, const GemvGeom &g, const float *a, size_t t_rows, float *out,
                        hipStream_t s) {
    const int U = units_per_row(w.dtype, w.n_cols);
#define RCE_RPL(NT)                                                                        \
    switch (g.rpl) {                                                                       \
    case 2: return launch_as<Unit, NT, 2, Q8>(w, U, a, t_rows, out, s);                    \
    case 4: return launch_as<Unit, NT, 4, Q8>(w, U, a, t_rows, out, s);                    \
    case 8: return launch_as<Unit, NT, 8, Q8>(w, U, a, t_rows, out, s);                    \
    case 12: return launch_as<Unit, NT, 12, Q8>(w, U, a, t_rows, out, s);                  \
    case 16: return launch_as<Unit, NT, 16, Q8>(w, U, a, t_rows, out, s);                  \
    default: return hipErrorInvalidValue;                                                  \
    }
    switch (g.nt) {
    case 256: RCE_RPL(256)
    case 512: RCE_RPL(512)
    case 1024: RCE_RPL(1024)
    default: return hipErrorInvalidValue;
    }
#undef RCE_RPL
}

// Plain Q8 launches on pre-quantized activations (FX_PREQ): no activation
// LDS, 256 threads, 2 / 4 / 8 / 16 rows per lane, 2 / 4 / 8 tokens per thread.
template <class Unit, int RPL>
hipError_t launch_as_preq(const DevWeight &w, int U, const float *a, size_t t_rows, float *out,
                          const unsigned char *preq, hipStream_t s) {
    constexpr int NT = 256, TB = Unit::NTOK;
    const int P = NT / U, RT = P * RPL;
    if (P < 1) return hipErrorInvalidConfiguration;
    if (!wbuf_span_ok(w, RT)) return hipErrorInvalidValue;
    const size_t lds = gemv_lds_bytes(U, NT, RPL, TB, false, w.n_cols);
    if (lds > LDS_MAX) return hipErrorInvalidConfiguration;
    GemvFx fx{};
    fx.preq = preq;
    fx.preq_t = (int)t_rows;
    dim3 grid((unsigned)((w.n_rows + RT - 1) / RT), (unsigned)((t_rows + TB - 1) / TB)), block(NT);
    hipLaunchKernelGGL((k_gemv_as<Unit, NT, RPL, true, FX_PREQ>), grid, block, lds, s, w, a, out, (int)t_rows, U, fx);
    return hipGetLastError();
}

template <template <int> class Unit, int MAXTB>
hipError_t launch_as_preq_tb(const DevWeight &w, const GemvGeom &g, const float *a, size_t t_rows, float *out,
                             const unsigned char *preq, hipStream_t s) {
    const int U = units_per_row(w.dtype, w.n_cols);
    if (g.nt != 256) return hipErrorInvalidValue;
#define RCE_PQ(TB)                                                                   \
    switch (g.rpl) {                                                                 \
    case 2: return launch_as_preq<Unit<TB>, 2>(w, U, a, t_rows, out, preq, s);       \
    case 4: return launch_as_preq<Unit<TB>, 4>(w, U, a, t_rows, out, preq, s);       \
    case 8: return launch_as_preq<Unit<TB>, 8>(w, U, a, t_rows, out, preq, s);       \
    case 16: return launch_as_preq<Unit<TB>, 16>(w, U, a, t_rows, out, preq, s);     \
    default: return hipErrorInvalidValue;                                            \
    }
    switch (g.tb) {
    case 2: RCE_PQ(2)
    case 4:
        if constexpr (MAXTB >= 4) { RCE_PQ(4) }
        return hipErrorInvalidValue;
    case 8:
        if constexpr (MAXTB >= 8) { RCE_PQ(8) }
        return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
#undef RCE_PQ
}

// MAXTB: the most tokens per thread the unit's registers allow.
template <template <int> class Unit, bool Q8, int MAXTB>
hipError_t launch_as_tb(const DevWeight &w, const GemvGeom &g, const float *a, size_t t_rows, float *out,
                        hipStream_t s) {
    switch (g.tb) {
    case 1: return launch_as_nt<Unit<1>, Q8>(w, g, a, t_rows, out, s);
    case 2:
        if constexpr (MAXTB >= 2) return launch_as_nt<Unit<2>, Q8>(w, g, a, t_rows, out, s);
        return hipErrorInvalidValue;
    case 4:
        if constexpr (MAXTB >= 4) return launch_as_nt<Unit<4>, Q8>(w, g, a, t_rows, out, s);
        return hipErrorInvalidValue;
    case 8:
        if constexpr (MAXTB >= 8) return launch_as_nt<Unit<8>, Q8>(w, g, a, t_rows, out, s);
        return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

template <int TB> using Q4_0Q8 = Q32Q8<TB, B32_Q4_0>;
template <int TB> using Q8_0Q8 = Q32Q8<TB, B32_Q8_0>;
template <int TB> using Q5_0Q8 = Q32Q8<TB, B32_Q5_0>;
template <int TB> using Q4_1Q8 = Q32Q8<TB, B32_Q4_1>;


}  // namespace
}  // namespace rce_qmm
