// gemv_ternary.hip -- the multiply-free block formats Q1_0, Q2_0 (blocks of
// 128) and STQ1_0 (super-blocks of 256), one token per thread.  The
// reference keeps per-block chains of activation sums (pos: weights +1,
// neg: weights -1, Q2_0 also plus2: weights +2) in position order and adds
// d * (pos - neg [+ 2 plus2]) per block (rce-op-qmm/src/lib.rs
// L1716-1875), so a unit is one whole block.  A chain step adds the
// activation or +0.0 (the activation's bits masked to zero): the chains
// start at +0.0 and a sum of two floats is -0.0 only if both are, so
// adding +0.0 leaves every chain value unchanged, and the result equals
// the reference's conditional adds bit for bit.  There is no Q8 form:
// both modes run these kernels.
#include "qmm_gemv_kernels.h"

namespace rce_qmm {
namespace {

// a if (mask == all ones), else +0.0
__device__ __forceinline__ float keep(float a, uint32_t mask) { return __uint_as_float(__float_as_uint(a) & mask); }

// Q1_0 block (lib.rs L1716-1760): bit j of the 16 code bytes (LSB first)
// is position j; set: pos += a, clear: neg += a.
template <int TB>
struct Q1_0Unit {
    static_assert(TB == 1, "one token per thread");
    static constexpr int NTOK = 1;
    using Raw = RawQ4_0;  // 16 code bytes + the f16 d, Q4_0's layout
    float av[128];
    __device__ static Raw load(const DevWeight &w, size_t row, int col) { return ld_q4_0(w, row, col); }
    __device__ void init(const float *A, size_t k, int t0, int, int col) {
        load_f32x(A + (size_t)t0 * k + 128 * (size_t)col, av, 128);
    }
    __device__ void addends(const Raw &r, float *out) const {
        float pos = 0.0f, neg = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t x = wrd(r.q, i);
#pragma unroll
            for (int j = 0; j < 32; j++) {
                // bit j as a mask (one v_bfe_i32), the activation kept where it
                // is set (v_and_b32) and where it is clear (one v_bfi_b32:
                // (m & 0) | (~m & a)); volatile keeps each step's masks in place
                uint32_t m, nv;
                asm volatile("v_bfe_i32 %0, %1, %2, 1" : "=v"(m) : "v"(x), "n"(j));
                const uint32_t a = __float_as_uint(av[32 * i + j]);
                asm volatile("v_bfi_b32 %0, %1, 0, %2" : "=v"(nv) : "v"(m), "v"(a));
                pos = pos + __uint_as_float(a & m);
                neg = neg + __uint_as_float(nv);
            }
        }
        const float t = pos - neg;
        out[0] = h2f(r.s) * t;
    }
};

// Q2_0 block (lib.rs L1766-1815): 2-bit lane j % 4 of byte j / 4 is
// position j; code 0: neg += a, 2: pos += a, 3: plus2 += a, 1: nothing;
// addend d * ((pos - neg) + 2 plus2).
template <int TB>
struct Q2_0Unit {
    static_assert(TB == 1, "one token per thread");
    static constexpr int NTOK = 1;
    using Raw = RawQ8_0;  // 32 code bytes in two planes + the f16 d, Q8_0's layout
    float av[128];
    __device__ static Raw load(const DevWeight &w, size_t row, int col) { return ld_q8_0(w, row, col); }
    __device__ void init(const float *A, size_t k, int t0, int, int col) {
        load_f32x(A + (size_t)t0 * k + 128 * (size_t)col, av, 128);
    }
    __device__ void addends(const Raw &r, float *out) const {
        float pos = 0.0f, neg = 0.0f, p2 = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t x = i < 4 ? wrd(r.q0, i) : wrd(r.q1, i - 4);
#pragma unroll
            for (int l = 0; l < 16; l++) {
                const uint32_t c = (x >> (2 * l)) & 3u;
                const float a = av[16 * i + l];
                neg = neg + keep(a, c == 0 ? ~0u : 0u);
                pos = pos + keep(a, c == 2 ? ~0u : 0u);
                p2 = p2 + keep(a, c == 3 ? ~0u : 0u);
            }
        }
        float t = pos - neg;
        const float u = 2.0f * p2;
        t = t + u;
        out[0] = h2f(r.s) * t;
    }
};

// STQ1_0 super-block (lib.rs L1821-1875) with its codebook expanded at
// upload: lane code 2: pos += a, 0: neg += a.  The unit's 256 activations
// are read from global memory (L1) 16 at a time rather than held.
struct RawSTQ1_0 { uint4 c[4]; uint32_t d; };
template <int TB>
struct STQ1_0Unit {
    static_assert(TB == 1, "one token per thread");
    static constexpr int NTOK = 1;
    using Raw = RawSTQ1_0;
    const float *ap;
    __device__ static Raw load(const DevWeight &w, size_t row, int col) {
        const uint8_t *rp = w.base + row * w.row_stride;
        Raw r;
        const uint4 *p = reinterpret_cast<const uint4 *>(rp + w.plane1 + 64 * (size_t)col);
#pragma unroll
        for (int i = 0; i < 4; i++) r.c[i] = p[i];
        r.d = *reinterpret_cast<const uint16_t *>(rp + 2 * (size_t)col);
        return r;
    }
    __device__ void init(const float *A, size_t k, int t0, int, int col) { ap = A + (size_t)t0 * k + 256 * (size_t)col; }
    __device__ void addends(const Raw &r, float *out) const {
        float pos = 0.0f, neg = 0.0f;
        // Positions 64 seg .. 64 seg + 63: 16 code bytes, 64 activations;
        // the next segment's activations are loaded while this one is
        // summed (two segments live at a time; no reuse across rows).
        float a[2][64];
        load_f32x(ap, a[0], 64);
#pragma unroll
        for (int seg = 0; seg < 4; seg++) {
            const uint4 cw = r.c[seg];
            if (seg < 3) load_f32x(ap + 64 * (seg + 1), a[(seg + 1) & 1], 64);
            const float *as = a[seg & 1];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t x = wrd(cw, i);
#pragma unroll
                for (int l = 0; l < 16; l++) {
                    const uint32_t c = (x >> (2 * l)) & 3u;
                    pos = pos + keep(as[16 * i + l], c == 2 ? ~0u : 0u);
                    neg = neg + keep(as[16 * i + l], c == 0 ? ~0u : 0u);
                }
            }
        }
        const float t = pos - neg;
        out[0] = h2f(r.d) * t;
    }
};

}  // namespace

namespace {
// These units are compute-heavy (a chain step per value, 128 or 256 steps
// per unit) and light on bytes, so the launch maximizes (unit, row) pairs
// in flight: the smallest block that holds a row's units, one row per lane
// (two once there are more than 2048 blocks), one token per thread.
template <class Unit>
hipError_t launch_ternary(const DevWeight &w, const float *a, size_t t_rows, float *out, hipStream_t s) {
    const int U = units_per_row(w.dtype, w.n_cols);
    if (U < 1 || U > 256) return hipErrorInvalidValue;
    const int nt = U <= 64 ? 64 : (U <= 128 ? 128 : 256);
    const size_t blocks = (w.n_rows + (size_t)(nt / U) - 1) / (size_t)(nt / U);
    const bool two = blocks > 2048;
    switch (nt) {
    case 64: return two ? launch_as<Unit, 64, 2, false>(w, U, a, t_rows, out, s)
                        : launch_as<Unit, 64, 1, false>(w, U, a, t_rows, out, s);
    case 128: return two ? launch_as<Unit, 128, 2, false>(w, U, a, t_rows, out, s)
                         : launch_as<Unit, 128, 1, false>(w, U, a, t_rows, out, s);
    default: return two ? launch_as<Unit, 256, 2, false>(w, U, a, t_rows, out, s)
                        : launch_as<Unit, 256, 1, false>(w, U, a, t_rows, out, s);
    }
}
}  // namespace

hipError_t launch_gemv_ternary(const DevWeight &w, const GemvGeom &, const float *a, size_t t_rows, float *out,
                               hipStream_t s) {
    switch (w.dtype) {
    case T_Q1_0: return launch_ternary<Q1_0Unit<1>>(w, a, t_rows, out, s);
    case T_Q2_0: return launch_ternary<Q2_0Unit<1>>(w, a, t_rows, out, s);
    case T_STQ1_0: return launch_ternary<STQ1_0Unit<1>>(w, a, t_rows, out, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace rce_qmm
