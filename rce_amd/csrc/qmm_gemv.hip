// qmm_gemv.hip -- decode-shaped kernels of the GGUF quantized-matmul path for
// gfx950 (CDNA4): exact-order GEMV, Q8-activation GEMV, activation
// quantization and row dequantization.
//
// Two work mappings are used:
//  * activation-stationary ("AS"): each lane owns one column unit (a Q4_0 /
//    Q8_0 block of 32, or a Q4_K group of 64) of the activation, keeps that
//    slice in registers and walks rows.  The wave's loads of one row are
//    contiguous 16-byte chunks.  Each unit's addend of the row sum goes to
//    LDS and one lane per row then folds the addends in block order, so the
//    fold is the reference's sequential `sumf += ...` loop.
//  * lane-per-row ("LPR", Q6_K): the reference's Q6_K row sum is a single
//    sequential chain over all positions, so one lane runs one row's chain
//    and the activation is wave-uniform (scalar registers).  The weight is
//    stored 64-row interleaved so those per-lane loads are still contiguous
//    across the wave.
//
// Exactness (MODE_EXACT): every + - * of the reference is one binary32
// operation here in the same order.  The product of a Q4_0 value (n - 8)
// and an activation a is formed as fma(n, a, -8a): -8a is exact and the fma
// rounds n*a - 8a = (n-8)*a once, which is the reference's rounded product
// (likewise fma(u, ds, -32 ds) = (u - 32) * ds for Q6_K).  Everything else
// is compiled with -ffp-contract=off so no other multiply-add is fused.
#include "qmm_internal.h"

namespace rce_qmm {
namespace {

constexpr uint32_t NIB = 0x0F0F0F0Fu;

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
// Column units, exact mode.
// ---------------------------------------------------------------------------

// Q4_0 block (rce-op-qmm/src/lib.rs L496-522): sub over q in 0..16 of
// (lo_q - 8) a[q] then (hi_q - 8) a[q+16]; addend = scale * sub.
struct UnitQ4_0Exact {
    static constexpr int ACT = 32;
    float av[32], an[32];
    struct Raw { uint4 q; uint32_t s; };
    __device__ void load_act(const float *a, int col) {
        load_f32x(a + 32 * col, av, 32);
#pragma unroll
        for (int i = 0; i < 32; i++) an[i] = -8.0f * av[i];
    }
    __device__ static Raw load(const DevWeight &w, size_t row, int col) {
        const uint8_t *rp = w.base + row * w.row_stride;
        Raw r;
        r.s = *reinterpret_cast<const uint16_t *>(rp + 2 * col);
        r.q = *reinterpret_cast<const uint4 *>(rp + w.qs_off + 16 * (size_t)col);
        return r;
    }
    __device__ float addend(const Raw &r) const {
        float sub = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t x = wrd(r.q, i);
            uint32_t lo = and_opaque(x, NIB), hi = and_opaque(x >> 4, NIB);
#define Q40_STEP(J)                                                                 \
    sub = sub + __builtin_fmaf(ubyte<J>(lo), av[4 * i + J], an[4 * i + J]);           \
    sub = sub + __builtin_fmaf(ubyte<J>(hi), av[4 * i + J + 16], an[4 * i + J + 16]);
            Q40_STEP(0) Q40_STEP(1) Q40_STEP(2) Q40_STEP(3)
#undef Q40_STEP
        }
        return h2f(r.s) * sub;
    }
};

// Q8_0 block (rce-op-qmm/src/lib.rs L315-328, L648-670).
struct UnitQ8_0Exact {
    static constexpr int ACT = 32;
    float av[32];
    struct Raw { uint4 q0, q1; uint32_t s; };
    __device__ void load_act(const float *a, int col) { load_f32x(a + 32 * col, av, 32); }
    __device__ static Raw load(const DevWeight &w, size_t row, int col) {
        const uint8_t *rp = w.base + row * w.row_stride;
        Raw r;
        r.s = *reinterpret_cast<const uint16_t *>(rp + 2 * col);
        const uint4 *qp = reinterpret_cast<const uint4 *>(rp + w.qs_off + 32 * (size_t)col);
        r.q0 = qp[0];
        r.q1 = qp[1];
        return r;
    }
    __device__ float addend(const Raw &r) const {
        float sub = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            uint32_t x = i < 4 ? wrd(r.q0, i) : wrd(r.q1, i - 4);
#pragma unroll
            for (int j = 0; j < 4; j++) sub = sub + (float)(int8_t)(x >> (8 * j)) * av[4 * i + j];
        }
        return h2f(r.s) * sub;
    }
};

// Q4_K group g of a super-block (rce-op-qmm/src/lib.rs L354-385, L730-781):
// va_lo, a_lo, va_hi, a_hi over l in 0..32 from +0.0, then
// ((d1 va_lo - min1 a_lo) + d2 va_hi) - min2 a_hi.  The activation sums
// a_lo, a_hi do not depend on the row and are formed once per lane.
struct UnitQ4_KExact {
    static constexpr int ACT = 64;
    float av[64];
    float a_lo, a_hi;
    int g;
    struct Raw { uint4 h, q0, q1; };
    __device__ void load_act(const float *a, int col) {
        load_f32x(a + 64 * col, av, 64);
        g = col & 3;
        a_lo = 0.0f; a_hi = 0.0f;
#pragma unroll
        for (int l = 0; l < 32; l++) { a_lo = a_lo + av[l]; a_hi = a_hi + av[32 + l]; }
    }
    __device__ static Raw load(const DevWeight &w, size_t row, int col) {
        const uint8_t *sp = w.base + row * w.row_stride + 144 * (size_t)(col >> 2);
        Raw r;
        r.h = *reinterpret_cast<const uint4 *>(sp);
        const uint4 *qp = reinterpret_cast<const uint4 *>(sp + 16 + 32 * (col & 3));
        r.q0 = qp[0];
        r.q1 = qp[1];
        return r;
    }
    __device__ float addend(const Raw &r) const {
        float d = h2f(r.h.x & 0xFFFFu), dmin = h2f(r.h.x >> 16);
        int sc1, m1, sc2, m2;
        k4_scale_min_pair(r.h, g, sc1, m1, sc2, m2);
        float d1 = d * (float)sc1, min1 = dmin * (float)m1;
        float d2 = d * (float)sc2, min2 = dmin * (float)m2;
        float va_lo = 0.0f, va_hi = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            uint32_t x = i < 4 ? wrd(r.q0, i) : wrd(r.q1, i - 4);
            uint32_t lo = and_opaque(x, NIB), hi = and_opaque(x >> 4, NIB);
#define Q4K_STEP(J)                                               \
    va_lo = va_lo + ubyte<J>(lo) * av[4 * i + J];                 \
    va_hi = va_hi + ubyte<J>(hi) * av[32 + 4 * i + J];
            Q4K_STEP(0) Q4K_STEP(1) Q4K_STEP(2) Q4K_STEP(3)
#undef Q4K_STEP
        }
        float t = d1 * va_lo;
        t = t - min1 * a_lo;
        t = t + d2 * va_hi;
        t = t - min2 * a_hi;
        return t;
    }
};

// ---------------------------------------------------------------------------
// Column units, Q8-activation mode.  TB activation rows (tokens) per pass.
// Each lane quantizes the activation blocks it owns straight from f32 (no
// separate quantization pass); the addends are the exact-mode formulas with
// each block sub-sum replaced by dx * (exact int32 dot of the block).
// ---------------------------------------------------------------------------

// nn.rs L541-563 quantize_block(x, false) of one block of 32: d = amax/127,
// id = 1/d (0 when d = 0), q = round half away from zero of x*id, packed
// four per word; the scale kept is round_to_f16(d) (nn.rs L521-533, the
// hardware's round-to-nearest-even conversion).  s_lo / s_hi: sums of the
// first / last 16 values of q.
__device__ __forceinline__ void quant_block32(const float *p, int *xq8, float &dx, int &s_lo, int &s_hi) {
    float v[32];
    load_f32x(p, v, 32);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) if (amax < fabsf(v[i])) amax = fabsf(v[i]);
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    s_lo = 0;
    s_hi = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) xq8[i] = 0;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const int qi = (int)roundf(v[i] * id);
        if (i < 16) s_lo += qi; else s_hi += qi;
        xq8[i >> 2] |= (int)(((uint32_t)qi & 0xFFu) << (8 * (i & 3)));
    }
    dx = (float)(_Float16)d;
}

template <int TB>
struct UnitQ4_0Q8 {
    int xq[TB][8];
    float dx[TB];
    int xs[TB];
    struct Raw { uint4 q; uint32_t s; };
    __device__ void load_act(const float *A, size_t k, int t0, int tv, int col) {
#pragma unroll
        for (int t = 0; t < TB; t++) {
            if (t < tv) {
                int lo, hi;
                quant_block32(A + (t0 + t) * k + 32 * (size_t)col, xq[t], dx[t], lo, hi);
                xs[t] = lo + hi;
            }
        }
    }
    __device__ static Raw load(const DevWeight &w, size_t row, int col) {
        const uint8_t *rp = w.base + row * w.row_stride;
        Raw r;
        r.s = *reinterpret_cast<const uint16_t *>(rp + 2 * col);
        r.q = *reinterpret_cast<const uint4 *>(rp + w.qs_off + 16 * (size_t)col);
        return r;
    }
    __device__ void addends(const Raw &r, float *out) const {
        int lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; i++) { lo[i] = (int)(wrd(r.q, i) & NIB); hi[i] = (int)((wrd(r.q, i) >> 4) & NIB); }
        float scale = h2f(r.s);
#pragma unroll
        for (int t = 0; t < TB; t++) {
            int acc = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_sdot4(lo[i], xq[t][i], acc, false);
#pragma unroll
            for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_sdot4(hi[i], xq[t][4 + i], acc, false);
            int isum = acc - 8 * xs[t];
            float sub = dx[t] * (float)isum;
            out[t] = scale * sub;
        }
    }
};

template <int TB>
struct UnitQ8_0Q8 {
    int xq[TB][8];
    float dx[TB];
    struct Raw { uint4 q0, q1; uint32_t s; };
    __device__ void load_act(const float *A, size_t k, int t0, int tv, int col) {
#pragma unroll
        for (int t = 0; t < TB; t++) {
            if (t < tv) {
                int lo, hi;
                quant_block32(A + (t0 + t) * k + 32 * (size_t)col, xq[t], dx[t], lo, hi);
            }
        }
    }
    __device__ static Raw load(const DevWeight &w, size_t row, int col) {
        const uint8_t *rp = w.base + row * w.row_stride;
        Raw r;
        r.s = *reinterpret_cast<const uint16_t *>(rp + 2 * col);
        const uint4 *qp = reinterpret_cast<const uint4 *>(rp + w.qs_off + 32 * (size_t)col);
        r.q0 = qp[0];
        r.q1 = qp[1];
        return r;
    }
    __device__ void addends(const Raw &r, float *out) const {
        float scale = h2f(r.s);
#pragma unroll
        for (int t = 0; t < TB; t++) {
            int acc = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_sdot4((int)wrd(r.q0, i), xq[t][i], acc, false);
#pragma unroll
            for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_sdot4((int)wrd(r.q1, i), xq[t][4 + i], acc, false);
            float sub = dx[t] * (float)acc;
            out[t] = scale * sub;
        }
    }
};

template <int TB>
struct UnitQ4_KQ8 {
    int xl[TB][8], xh[TB][8];
    float dl[TB], dh[TB];
    int sl[TB], sh[TB];
    int g;
    using Raw = UnitQ4_KExact::Raw;
    __device__ void load_act(const float *A, size_t k, int t0, int tv, int col) {
        g = col & 3;
#pragma unroll
        for (int t = 0; t < TB; t++) {
            if (t < tv) {
                // the activation blocks of sub-blocks 2g and 2g+1
                const float *p = A + (t0 + t) * k + 64 * (size_t)col;
                int a, b;
                quant_block32(p, xl[t], dl[t], a, b);
                sl[t] = a + b;
                quant_block32(p + 32, xh[t], dh[t], a, b);
                sh[t] = a + b;
            }
        }
    }
    __device__ static Raw load(const DevWeight &w, size_t row, int col) {
        return UnitQ4_KExact::load(w, row, col);
    }
    __device__ void addends(const Raw &r, float *out) const {
        float d = h2f(r.h.x & 0xFFFFu), dmin = h2f(r.h.x >> 16);
        int sc1, m1, sc2, m2;
        k4_scale_min_pair(r.h, g, sc1, m1, sc2, m2);
        float d1 = d * (float)sc1, min1 = dmin * (float)m1;
        float d2 = d * (float)sc2, min2 = dmin * (float)m2;
        int lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            uint32_t x = i < 4 ? wrd(r.q0, i) : wrd(r.q1, i - 4);
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
            float va_lo = dl[t] * (float)il, a_lo = dl[t] * (float)sl[t];
            float va_hi = dh[t] * (float)ih, a_hi = dh[t] * (float)sh[t];
            float tt = d1 * va_lo;
            tt = tt - min1 * a_lo;
            tt = tt + d2 * va_hi;
            tt = tt - min2 * a_hi;
            out[t] = tt;
        }
    }
};

// ---------------------------------------------------------------------------
// Activation-stationary kernels.
// Block of NT threads; U column units per row; P = NT / U rows per pass;
// RT rows per tile (multiple of P); RB rows loaded ahead per lane.
// LDS: the addends of a tile, [TB][RT][U + 1] floats.
// ---------------------------------------------------------------------------

constexpr int RB = 4;

template <class Unit, int NT>
__global__ __launch_bounds__(NT) void k_gemv_exact_as(DevWeight w, const float *__restrict__ A,
                                                      float *__restrict__ out, int U, int P, int RT,
                                                      int ntiles) {
    extern __shared__ float part[];
    const int tid = threadIdx.x;
    const int col = tid % U, rsub = tid / U;
    const bool active = rsub < P;
    const size_t tok = blockIdx.y;
    const float *a = A + tok * w.n_cols;
    float *o = out + tok * w.n_rows;
    const int ld = U + 1;
    Unit unit;
    if (active) unit.load_act(a, col);
    for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const size_t row0 = (size_t)tile * RT;
        if (active) {
            for (int r0 = rsub; r0 < RT; r0 += P * RB) {
                typename Unit::Raw raw[RB];
#pragma unroll
                for (int u = 0; u < RB; u++) {
                    const int r = r0 + u * P;
                    if (r < RT && row0 + r < w.n_rows) raw[u] = Unit::load(w, row0 + r, col);
                }
#pragma unroll
                for (int u = 0; u < RB; u++) {
                    const int r = r0 + u * P;
                    if (r < RT) part[r * ld + col] = row0 + r < w.n_rows ? unit.addend(raw[u]) : 0.0f;
                }
            }
        }
        __syncthreads();
        for (int r = tid; r < RT; r += NT) {
            if (row0 + r < w.n_rows) {
                float s = 0.0f;
                for (int c = 0; c < U; c++) s = s + part[r * ld + c];
                o[row0 + r] = s;
            }
        }
        __syncthreads();
    }
}

template <class Unit, int NT, int TB>
__global__ __launch_bounds__(NT) void k_gemv_q8_as(DevWeight w, const float *__restrict__ A, float *__restrict__ out,
                                                   int t_rows, int U, int P, int RT, int ntiles) {
    extern __shared__ float part[];
    const int tid = threadIdx.x;
    const int col = tid % U, rsub = tid / U;
    const bool active = rsub < P;
    const int t0 = blockIdx.y * TB;
    const int tv = min(TB, t_rows - t0);
    const int ld = U + 1;
    Unit unit;
    if (active) unit.load_act(A, w.n_cols, t0, tv, col);
    for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const size_t row0 = (size_t)tile * RT;
        if (active) {
            for (int r0 = rsub; r0 < RT; r0 += P * RB) {
                typename Unit::Raw raw[RB];
#pragma unroll
                for (int u = 0; u < RB; u++) {
                    const int r = r0 + u * P;
                    if (r < RT && row0 + r < w.n_rows) raw[u] = Unit::load(w, row0 + r, col);
                }
#pragma unroll
                for (int u = 0; u < RB; u++) {
                    const int r = r0 + u * P;
                    if (r < RT) {
                        float ad[TB];
                        if (row0 + r < w.n_rows) {
                            unit.addends(raw[u], ad);
                        } else {
#pragma unroll
                            for (int t = 0; t < TB; t++) ad[t] = 0.0f;
                        }
#pragma unroll
                        for (int t = 0; t < TB; t++) part[(t * RT + r) * ld + col] = ad[t];
                    }
                }
            }
        }
        __syncthreads();
        for (int j = tid; j < tv * RT; j += NT) {
            const int t = j / RT, r = j % RT;
            if (row0 + r < w.n_rows) {
                float s = 0.0f;
                const float *pp = part + (t * RT + r) * ld;
                for (int c = 0; c < U; c++) s = s + pp[c];
                out[(size_t)(t0 + t) * w.n_rows + row0 + r] = s;
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Q6_K, lane per row (LAYOUT_IL64).
// ---------------------------------------------------------------------------

struct Q6Block {
    uint4 ql[8], qh[4], sc;
    uint32_t d;
};

__device__ __forceinline__ void q6_load(const uint8_t *sbp, int lane, Q6Block &b) {
#pragma unroll
    for (int c = 0; c < 8; c++)
        b.ql[c] = *reinterpret_cast<const uint4 *>(sbp + IL64_Q6K_QL + (size_t)(c * 64 + lane) * 16);
#pragma unroll
    for (int c = 0; c < 4; c++)
        b.qh[c] = *reinterpret_cast<const uint4 *>(sbp + IL64_Q6K_QH + (size_t)(c * 64 + lane) * 16);
    b.sc = *reinterpret_cast<const uint4 *>(sbp + IL64_Q6K_SC + (size_t)lane * 16);
    b.d = *reinterpret_cast<const uint16_t *>(sbp + IL64_Q6K_D + (size_t)lane * 2);
}

__device__ __forceinline__ int q6_sc(const uint4 &s, int i) {
    return (int)(int8_t)((wrd(s, i >> 2) >> (8 * (i & 3))) & 0xFFu);
}

// The four 6-bit value words (+32 offset, one byte per l) of positions
// l..l+3 (q1), +32 (q2), +64 (q3), +96 (q4) of half o, l = 4*lq.
__device__ __forceinline__ void q6_words(const Q6Block &b, int o, int lq, uint32_t &u1, uint32_t &u2,
                                         uint32_t &u3, uint32_t &u4) {
    const int c = lq >> 2, wi = lq & 3;
    const uint32_t qa = wrd(b.ql[4 * o + c], wi), qb = wrd(b.ql[4 * o + 2 + c], wi);
    const uint32_t qh = wrd(b.qh[2 * o + c], wi);
    u1 = (qa & NIB) | ((qh & 0x03030303u) << 4);
    u2 = (qb & NIB) | ((qh & 0x0C0C0C0Cu) << 2);
    u3 = ((qa >> 4) & NIB) | (qh & 0x30303030u);
    u4 = ((qb >> 4) & NIB) | ((qh >> 2) & 0x30303030u);
}

// rce-op-qmm/src/lib.rs L425-454, L1667-1705: per half o, l in 0..32, the
// positions l, l+32, l+64, l+96 in order: sumf += ((d sc) q) a.
__global__ __launch_bounds__(256) void k_gemv_exact_q6k(DevWeight w, const float *__restrict__ A,
                                                        float *__restrict__ out) {
    const size_t row = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t grp = row >> 6;
    const int lane = threadIdx.x & 63;
    if (grp * 64 >= w.n_rows) return;  // wave-uniform
    const size_t tok = blockIdx.y;
    const float *a = A + tok * w.n_cols;
    const uint8_t *gb = w.base + grp * w.group_stride;
    const int nsb = (int)(w.n_cols / 256);
    float sumf = 0.0f;
    for (int sb = 0; sb < nsb; sb++) {
        Q6Block b;
        q6_load(gb + (size_t)sb * IL64_Q6K_SB, lane, b);
        const float d = h2f(b.d);
        const float *as = a + 256 * sb;
#pragma unroll
        for (int o = 0; o < 2; o++) {
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const float ds1 = d * (float)q6_sc(b.sc, 8 * o + c), ds2 = d * (float)q6_sc(b.sc, 8 * o + c + 2);
                const float ds3 = d * (float)q6_sc(b.sc, 8 * o + c + 4), ds4 = d * (float)q6_sc(b.sc, 8 * o + c + 6);
                const float n1 = -32.0f * ds1, n2 = -32.0f * ds2, n3 = -32.0f * ds3, n4 = -32.0f * ds4;
#pragma unroll
                for (int lq = 4 * c; lq < 4 * c + 4; lq++) {
                    uint32_t u1, u2, u3, u4;
                    q6_words(b, o, lq, u1, u2, u3, u4);
                    const float *al = as + 128 * o + 4 * lq;
#define Q6_STEP(J)                                                                   \
    sumf = sumf + __builtin_fmaf(ubyte<J>(u1), ds1, n1) * al[J];                       \
    sumf = sumf + __builtin_fmaf(ubyte<J>(u2), ds2, n2) * al[J + 32];                  \
    sumf = sumf + __builtin_fmaf(ubyte<J>(u3), ds3, n3) * al[J + 64];                  \
    sumf = sumf + __builtin_fmaf(ubyte<J>(u4), ds4, n4) * al[J + 96];
                    Q6_STEP(0) Q6_STEP(1) Q6_STEP(2) Q6_STEP(3)
#undef Q6_STEP
                }
            }
        }
    }
    if (row < w.n_rows) out[tok * w.n_rows + row] = sumf;
}

// Q8-activation Q6_K: per super-block, for sub-blocks b of 16 ascending,
// ssb += (d sc_b) (dx isum_b) from +0.0, then sumf += ssb.  The block first
// quantizes the activation row into LDS (xq words, dx, half-block sums);
// every lane then reads the same LDS word (a broadcast).
__global__ __launch_bounds__(256) void k_gemv_q8_q6k(DevWeight w, const float *__restrict__ A,
                                                     float *__restrict__ out) {
    extern __shared__ int lds_q[];
    const size_t k = w.n_cols;
    const int nb = (int)(k / 32);
    int *xq = lds_q;                                          // k/4 words
    float *dx = reinterpret_cast<float *>(lds_q + k / 4);     // k/32
    int *xs16 = lds_q + k / 4 + k / 32;                       // k/16
    const size_t tok = blockIdx.y;
    for (int b = threadIdx.x; b < nb; b += 256) {
        int q8[8], lo, hi;
        float d;
        quant_block32(A + tok * k + 32 * (size_t)b, q8, d, lo, hi);
#pragma unroll
        for (int i = 0; i < 8; i++) xq[8 * b + i] = q8[i];
        dx[b] = d;
        xs16[2 * b] = lo;
        xs16[2 * b + 1] = hi;
    }
    __syncthreads();
    const size_t row = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t grp = row >> 6;
    const int lane = threadIdx.x & 63;
    if (grp * 64 >= w.n_rows) return;  // wave-uniform, after the only barrier
    const uint8_t *gb = w.base + grp * w.group_stride;
    const int nsb = (int)(k / 256);
    float sumf = 0.0f;
    for (int sb = 0; sb < nsb; sb++) {
        Q6Block b;
        q6_load(gb + (size_t)sb * IL64_Q6K_SB, lane, b);
        const float d = h2f(b.d);
        float ssb = 0.0f;
#pragma unroll
        for (int o = 0; o < 2; o++) {
            int acc[8];  // sub-block 8o + 2m + c -> index 2m + c
#pragma unroll
            for (int i = 0; i < 8; i++) acc[i] = 0;
#pragma unroll
            for (int lq = 0; lq < 8; lq++) {
                uint32_t u[4];
                q6_words(b, o, lq, u[0], u[1], u[2], u[3]);
                const int c = lq >> 2, wi = lq & 3;
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    // positions 128o + 32m + 16c + 4wi .. +3
                    const int xw = (256 * sb + 128 * o + 32 * m + 16 * c + 4 * wi) >> 2;
                    acc[2 * m + c] = __builtin_amdgcn_sdot4((int)u[m], xq[xw], acc[2 * m + c], false);
                }
            }
#pragma unroll
            for (int bb = 0; bb < 8; bb++) {
                const int sbk = 8 * o + bb;              // sub-block within the super-block
                const int gsub = 16 * sb + sbk;          // sub-block of 16 within the row
                const int isum = acc[bb] - 32 * xs16[gsub];
                const float ds = d * (float)q6_sc(b.sc, sbk);
                const float ab = dx[gsub >> 1] * (float)isum;
                ssb = ssb + ds * ab;
            }
        }
        sumf = sumf + ssb;
    }
    if (row < w.n_rows) out[tok * w.n_rows + row] = sumf;
}

// ---------------------------------------------------------------------------
// f16 widening, row dequantization.
// ---------------------------------------------------------------------------

__global__ void k_f16_to_f32(const uint16_t *__restrict__ s, float *__restrict__ d, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) d[i] = h2f(s[i]);
}

// dequant.rs L360-382 (Q4_0), L438-454 (Q8_0), L546-589 (Q4_K), L658-701
// (Q6_K): one output value per thread.
__global__ void k_dequant_row(DevWeight w, size_t row, float *__restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= w.n_cols) return;
    float v = 0.0f;
    if (w.dtype == T_Q4_0 || w.dtype == T_Q8_0) {
        const uint8_t *rp = w.base + row * w.row_stride;
        const size_t b = i / 32;
        const int p = (int)(i % 32);
        const float scale = h2f(*reinterpret_cast<const uint16_t *>(rp + 2 * b));
        if (w.dtype == T_Q4_0) {
            const uint8_t byte = rp[w.qs_off + 16 * b + (p & 15)];
            const int n = p < 16 ? (byte & 0x0F) - 8 : ((byte >> 4) & 0x0F) - 8;
            v = (float)n * scale;
        } else {
            v = (float)(int8_t)rp[w.qs_off + 32 * b + p] * scale;
        }
    } else if (w.dtype == T_Q4_K) {
        const uint8_t *sp = w.base + row * w.row_stride + 144 * (i / 256);
        const int p = (int)(i % 256), g = p / 64, l = p % 32, hi = (p % 64) >= 32;
        const uint4 h = *reinterpret_cast<const uint4 *>(sp);
        int sc, m;
        k4_scale_min(h, 2 * g + hi, sc, m);
        const float d = h2f(h.x & 0xFFFFu), dmin = h2f(h.x >> 16);
        const float dd = d * (float)sc, mm = dmin * (float)m;
        const uint8_t byte = sp[16 + 32 * g + l];
        const int n = hi ? ((byte >> 4) & 0x0F) : (byte & 0x0F);
        v = dd * (float)n - mm;
    } else if (w.dtype == T_Q6_K) {
        const size_t grp = row >> 6;
        const int lane = (int)(row & 63);
        const uint8_t *sbp = w.base + grp * w.group_stride + (i / 256) * IL64_Q6K_SB;
        const int p = (int)(i % 256), o = p / 128, r = p % 128, m = r / 32, l = r % 32;
        // ql byte j of the super-block lives in chunk j/16, byte j%16.
        auto ql = [&](int j) { return sbp[IL64_Q6K_QL + (size_t)((j >> 4) * 64 + lane) * 16 + (j & 15)]; };
        auto qh = [&](int j) { return sbp[IL64_Q6K_QH + (size_t)((j >> 4) * 64 + lane) * 16 + (j & 15)]; };
        const int qhb = qh(32 * o + l);
        int q;
        if (m == 0) q = ((ql(64 * o + l) & 0x0F) | ((qhb & 3) << 4)) - 32;
        else if (m == 1) q = ((ql(64 * o + l + 32) & 0x0F) | (((qhb >> 2) & 3) << 4)) - 32;
        else if (m == 2) q = ((ql(64 * o + l) >> 4) | (((qhb >> 4) & 3) << 4)) - 32;
        else q = ((ql(64 * o + l + 32) >> 4) | (((qhb >> 6) & 3) << 4)) - 32;
        const int sc = (int)(int8_t)sbp[IL64_Q6K_SC + (size_t)lane * 16 + 8 * o + l / 16 + 2 * m];
        const float d = h2f(*reinterpret_cast<const uint16_t *>(sbp + IL64_Q6K_D + (size_t)lane * 2));
        const float t = d * (float)sc;
        v = t * (float)q;
    }
    out[i] = v;
}

// ---------------------------------------------------------------------------
// Launch geometry.
// ---------------------------------------------------------------------------

struct AsGeom { int nt, U, P, RT, ntiles, grid; size_t lds; };

// Threads per block: the smallest of 256/512/1024 holding one row's units.
// Rows per tile: 2*RB passes per lane (RT = 2*RB*P) keeps a lane's loads in
// flight while the tile count stays well above the CU count.
AsGeom as_geom(size_t n_rows, int U, int tb) {
    AsGeom g{};
    g.U = U;
    g.nt = U <= 256 ? 256 : (U <= 512 ? 512 : 1024);
    g.P = g.nt / U;
    int passes = tb > 1 ? RB : 2 * RB;
    g.RT = g.P * passes;
    g.ntiles = (int)((n_rows + g.RT - 1) / g.RT);
    g.grid = g.ntiles;
    g.lds = (size_t)tb * g.RT * (U + 1) * sizeof(float);
    return g;
}

template <class Unit>
hipError_t run_exact_as(const DevWeight &w, int U, const float *a, size_t t_rows, float *out,
                        hipStream_t s) {
    AsGeom g = as_geom(w.n_rows, U, 1);
    dim3 grid(g.grid, (unsigned)t_rows), block(g.nt);
    if (g.nt == 256)
        hipLaunchKernelGGL((k_gemv_exact_as<Unit, 256>), grid, block, g.lds, s, w, a, out, g.U, g.P, g.RT, g.ntiles);
    else if (g.nt == 512)
        hipLaunchKernelGGL((k_gemv_exact_as<Unit, 512>), grid, block, g.lds, s, w, a, out, g.U, g.P, g.RT, g.ntiles);
    else
        hipLaunchKernelGGL((k_gemv_exact_as<Unit, 1024>), grid, block, g.lds, s, w, a, out, g.U, g.P, g.RT, g.ntiles);
    return hipGetLastError();
}

template <template <int> class Unit, int TB>
hipError_t run_q8_as_tb(const DevWeight &w, int U, const float *q, size_t t_rows, float *out,
                        hipStream_t s) {
    AsGeom g = as_geom(w.n_rows, U, TB);
    dim3 grid(g.grid, (unsigned)((t_rows + TB - 1) / TB)), block(g.nt);
    int tr = (int)t_rows;
    if (g.nt == 256)
        hipLaunchKernelGGL((k_gemv_q8_as<Unit<TB>, 256, TB>), grid, block, g.lds, s, w, q, out, tr, g.U, g.P, g.RT, g.ntiles);
    else if (g.nt == 512)
        hipLaunchKernelGGL((k_gemv_q8_as<Unit<TB>, 512, TB>), grid, block, g.lds, s, w, q, out, tr, g.U, g.P, g.RT, g.ntiles);
    else
        hipLaunchKernelGGL((k_gemv_q8_as<Unit<TB>, 1024, TB>), grid, block, g.lds, s, w, q, out, tr, g.U, g.P, g.RT, g.ntiles);
    return hipGetLastError();
}

template <template <int> class Unit, int TBMAX>
hipError_t run_q8_as(const DevWeight &w, int U, const float *q, size_t t_rows, float *out,
                     hipStream_t s) {
    if (t_rows == 1) return run_q8_as_tb<Unit, 1>(w, U, q, t_rows, out, s);
    if (t_rows <= 4 || TBMAX == 4) return run_q8_as_tb<Unit, 4>(w, U, q, t_rows, out, s);
    return run_q8_as_tb<Unit, (TBMAX > 4 ? TBMAX : 4)>(w, U, q, t_rows, out, s);
}

}  // namespace

// Column units per row must fit one block of up to 1024 threads.
bool gpu_supports(uint32_t dtype, size_t n_cols, int mode) {
    if (n_cols == 0) return false;
    switch (dtype) {
    case T_Q4_0:
    case T_Q8_0:
        return n_cols % 32 == 0 && n_cols / 32 <= 1024 && (mode == 0 || mode == 1);
    case T_Q4_K:
        return n_cols % 256 == 0 && n_cols / 64 <= 1024 && (mode == 0 || mode == 1);
    case T_Q6_K:
        return n_cols % 256 == 0 && (mode == 0 || mode == 1);
    default:
        return false;
    }
}

hipError_t launch_f16_to_f32(const uint16_t *src, float *dst, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_f16_to_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, dst, n);
    return hipGetLastError();
}

hipError_t launch_gemv_exact(const DevWeight &w, const float *a, size_t t_rows, float *out,
                             hipStream_t s) {
    if (t_rows == 0 || w.n_rows == 0) return hipSuccess;
    switch (w.dtype) {
    case T_Q4_0: return run_exact_as<UnitQ4_0Exact>(w, (int)(w.n_cols / 32), a, t_rows, out, s);
    case T_Q8_0: return run_exact_as<UnitQ8_0Exact>(w, (int)(w.n_cols / 32), a, t_rows, out, s);
    case T_Q4_K: return run_exact_as<UnitQ4_KExact>(w, (int)(w.n_cols / 64), a, t_rows, out, s);
    case T_Q6_K: {
        dim3 grid((unsigned)((w.n_rows + 255) / 256), (unsigned)t_rows);
        hipLaunchKernelGGL(k_gemv_exact_q6k, grid, dim3(256), 0, s, w, a, out);
        return hipGetLastError();
    }
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_q8(const DevWeight &w, const float *a, size_t t_rows, float *out,
                          hipStream_t s) {
    if (t_rows == 0 || w.n_rows == 0) return hipSuccess;
    switch (w.dtype) {
    case T_Q4_0: return run_q8_as<UnitQ4_0Q8, 8>(w, (int)(w.n_cols / 32), a, t_rows, out, s);
    case T_Q8_0: return run_q8_as<UnitQ8_0Q8, 8>(w, (int)(w.n_cols / 32), a, t_rows, out, s);
    case T_Q4_K: return run_q8_as<UnitQ4_KQ8, 4>(w, (int)(w.n_cols / 64), a, t_rows, out, s);
    case T_Q6_K: {
        dim3 grid((unsigned)((w.n_rows + 255) / 256), (unsigned)t_rows);
        const size_t lds = w.n_cols + (w.n_cols / 32) * 4 + (w.n_cols / 16) * 4;
        hipLaunchKernelGGL(k_gemv_q8_q6k, grid, dim3(256), lds, s, w, a, out);
        return hipGetLastError();
    }
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_dequant_row(const DevWeight &w, size_t row, float *out, hipStream_t s) {
    hipLaunchKernelGGL(k_dequant_row, dim3((unsigned)((w.n_cols + 255) / 256)), dim3(256), 0, s, w,
                       row, out);
    return hipGetLastError();
}

}  // namespace rce_qmm
