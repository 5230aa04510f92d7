/*
 * qmm_oracle.c -- TEST INFRASTRUCTURE ONLY (parity checker + CPU baseline).
 *
 * A plain-C restatement of the reference's CPU implementation of the GGUF
 * block-quantized matmul path (openIE-dev/rce, compute/crates).  Nothing in
 * the product (rce_amd/, include/) links, loads or calls this file; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg do, and
 * only as the checker.
 *
 * Every function follows the reference in operation order: one IEEE-754
 * binary32 rounding per + - * /, no fused multiply-add (build with
 * -ffp-contract=off and without -ffast-math), sums from +0.0 in the order
 * the reference loops run.  Each function cites the reference file:line it
 * restates; paths are relative to the reference root.
 *
 * Parity pins (see tests/test_oracle_*.py):
 *   - f16 conversions: exhaustive against numpy's IEEE binary16.
 *   - quantizers: the reference's known answers (nn.rs L751-765,
 *     kquant.rs L425-437) and pack/unpack round trips.
 *   - dequant layouts: quantize->pack->dequant reproduces the quantizer's
 *     values (a wrong nibble/bit position fails), plus dequant.rs L748.
 *   - mm_1d kernels: bit-identical to the independent value-form
 *     restatement (nn.rs matmul_q, kquant.rs matmul_k), within 1e-5 of
 *     dequant-then-dot on the reference tests' synthetic bytes
 *     (rce-op-qmm lib.rs L2358-2500), and within a derived bound of an
 *     f64 brute-force dot.
 *   - Q8-activation path: the per-block integer dots are checked against
 *     numpy int64 dot products (closed form).
 *   - MoE router: known answers of rce-op-moe tests (L112-205).
 *   - expf/sinf/cosf come from the platform libm exactly as the
 *     reference's f32::exp etc. do on Linux; their last bits are
 *     "parity unpinned" (only used by router weights, silu, rope, softmax).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define EXPORT __attribute__((visibility("default")))

/* GGUF type tags (rce-ingest-gguf/src/parser.rs L306-341). */
enum {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7,
    T_Q8_0 = 8, T_Q8_1 = 9, T_Q2_K = 10, T_Q3_K = 11, T_Q4_K = 12,
    T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30, T_I2_S = 36, T_Q1_0 = 41, T_Q2_0 = 42
};
/* STQ1_0 shares the file tag 42 with Q2_0 (parser.rs L376-377); this build
 * names it tag 42 with bit 31 set. */
#define T_STQ1_0 0x8000002Au

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* ------------------------------------------------------------------ */
/* binary16 <-> binary32                                               */
/* ------------------------------------------------------------------ */

/* Exact binary16 -> binary32 (the `half` crate's f16::to_f32, as pinned
 * in-repo by kquant.rs L411-425 `half_free`). */
EXPORT float orc_f16_to_f32(uint16_t h) {
    uint32_t s = ((uint32_t)(h >> 15)) << 31;
    int e = (h >> 10) & 0x1f;
    uint32_t m = h & 0x3ff;
    if (e == 0x1f) return bits_f32(s | 0x7f800000u | (m << 13));
    float mag;
    if (e == 0) mag = (float)m * bits_f32(0x33800000u); /* m * 2^-24, exact */
    else mag = bits_f32(((uint32_t)(e - 15 + 127) << 23) | (m << 13));
    return bits_f32(f32_bits(mag) | s);
}

static inline float rd_f16(const uint8_t *p) {
    return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}

/* bfloat16 -> f32 (half::bf16::to_f32): the high half of the f32 bits. */
static inline float rd_bf16(const uint8_t *p) {
    return bits_f32(((uint32_t)(p[0] | (p[1] << 8))) << 16);
}

/* rce-vm-backend-cpu/src/ml/nn.rs L521-533 `round_to_f16`: x rounded once
 * to binary16, ties to even, returned as f32; |r| >= 65520 -> infinity. */
EXPORT float orc_round_to_f16(float x) {
    if (x == 0.0f || !isfinite(x)) return x;
    int e = (int)((f32_bits(fabsf(x)) >> 23) & 0xff) - 127;
    int qe = e >= -14 ? e - 10 : -24;
    double q = ldexp(1.0, qe);
    double r = nearbyint((double)x / q) * q; /* ties to even (default mode) */
    if (fabs(r) >= 65520.0) return r > 0 ? INFINITY : -INFINITY;
    return (float)r;
}

/* kquant.rs L267-281 / spec/checker/tests/support/toy_gpt2.rs L30-42
 * `f16_bits`: the binary16 bits of an f32 that is a binary16 value. */
EXPORT uint16_t orc_f16_bits(float x) {
    uint32_t b = f32_bits(x);
    uint16_t s = (uint16_t)((b >> 16) & 0x8000);
    float a = fabsf(x);
    if (a == 0.0f) return s;
    if (a < ldexpf(1.0f, -14)) return (uint16_t)(s | (uint16_t)(a / ldexpf(1.0f, -24)));
    int e = (int)(f32_bits(a) >> 23) - 127 + 15;
    return (uint16_t)(s | ((uint16_t)e << 10) | (uint16_t)((f32_bits(a) >> 13) & 0x3ff));
}

/* ------------------------------------------------------------------ */
/* Block geometry (dequant.rs L18-60 tensor_byte_size)                 */
/* ------------------------------------------------------------------ */

EXPORT int orc_block_geometry(uint32_t t, uint32_t *block, uint32_t *bytes) {
    uint32_t qk, bb;
    switch (t) {
    case T_F32: qk = 1; bb = 4; break;
    case T_F16: case T_BF16: qk = 1; bb = 2; break;
    case T_Q4_0: qk = 32; bb = 18; break;
    case T_Q4_1: qk = 32; bb = 20; break;
    case T_Q5_0: qk = 32; bb = 22; break;
    case T_Q5_1: qk = 32; bb = 24; break;
    case T_Q8_0: qk = 32; bb = 34; break;
    case T_Q8_1: qk = 32; bb = 36; break;
    case T_Q2_K: qk = 256; bb = 84; break;
    case T_Q3_K: qk = 256; bb = 110; break;
    case T_Q4_K: qk = 256; bb = 144; break;
    case T_Q5_K: qk = 256; bb = 176; break;
    case T_Q6_K: qk = 256; bb = 210; break;
    case T_I2_S: qk = 128; bb = 32; break;  /* plus one f32 scale per tensor */
    case T_Q1_0: qk = 128; bb = 18; break;
    case T_Q2_0: qk = 128; bb = 34; break;
    case T_STQ1_0: qk = 256; bb = 42; break;
    default: return -1;
    }
    *block = qk; *bytes = bb;
    return 0;
}

EXPORT size_t orc_tensor_byte_size(uint32_t t, size_t n) {
    uint32_t qk, bb;
    if (t == T_I2_S) return (n + 3) / 4 + 4;  /* dequant.rs L45-48: 2-bit codes + the f32 scale */
    if (orc_block_geometry(t, &qk, &bb)) return 0;
    return (n + qk - 1) / qk * bb;
}

/* ------------------------------------------------------------------ */
/* Quantizers (produce the configs' weights)                           */
/* ------------------------------------------------------------------ */

/* Rust's `f as i32` (saturating): NaN -> 0, values beyond the range -> the
 * nearest bound, else truncation toward zero.  A plain C cast of NaN or an
 * out-of-range float is undefined (x86 gives INT_MIN for all of them). */
static inline int32_t as_i32(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x <= -2147483648.0f) return INT32_MIN;
    return (int32_t)x;
}

/* Planted mistakes for the known-answer tests (tests/test_oracle_formats.py
 * compiles copies with -DORC_PLANT=k; the shipped build has 0):
 * 1 round half to even instead of away from zero; 2 lo = the least value
 * instead of min(0, least); 3 no clamp of sc at 63; 4 no clamp of m at 63;
 * 5 Q6_K's last instead of first value of largest magnitude. */
#ifndef ORC_PLANT
#define ORC_PLANT 0
#endif

/* nn.rs L541-563 `quantize_block`: GGUF reference quantizers of one block
 * of 32.  Q8_0: d = amax/127, q = round_half_away(x*id).  Q4_0: m = first
 * x of largest magnitude, d = m/-8, q = min(15, floor(x*id + 8.5)) - 8.
 * The scale returned is round_to_f16(d). */
EXPORT void orc_quantize_block(const float *x, int q4, int32_t *q, float *d_out) {
    float amax = 0.0f, max = 0.0f;
    for (int i = 0; i < 32; i++) {
        if (amax < fabsf(x[i])) { amax = fabsf(x[i]); max = x[i]; }
    }
    float d = q4 ? max / -8.0f : amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    for (int i = 0; i < 32; i++) {
        if (q4) {
            float t = x[i] * id;
            t = t + 8.5f;
            int32_t v = as_i32(floorf(t));
            /* `.min(15) - 8` wraps in a release build (only -inf reaches it) */
            q[i] = (int32_t)((uint32_t)(v < 15 ? v : 15) - 8u);
        } else {
            float t = x[i] * id;
            q[i] = as_i32(roundf(t));
        }
    }
    *d_out = orc_round_to_f16(d);
}

/* toy_gpt2.rs L46-58 `quantize`: GGUF Q8_0 / Q4_0 bytes of n values
 * (n a multiple of 32), blocks along the flat order. */
EXPORT void orc_quantize_q8_0_q4_0(const float *w, size_t n, int q4, uint8_t *out) {
    size_t nb = n / 32, bb = q4 ? 18 : 34;
#pragma omp parallel for schedule(static)
    for (size_t b = 0; b < nb; b++) {
        int32_t q[32]; float d;
        orc_quantize_block(w + b * 32, q4, q, &d);
        uint8_t *o = out + b * bb;
        uint16_t h = orc_f16_bits(d);
        o[0] = (uint8_t)(h & 0xff); o[1] = (uint8_t)(h >> 8);
        if (q4) {
            for (int t = 0; t < 16; t++)  /* (q + 8) as u8, the add wrapping */
                o[2 + t] = (uint8_t)((uint8_t)((uint32_t)q[t] + 8u) | (uint8_t)((uint8_t)((uint32_t)q[t + 16] + 8u) << 4));
        } else {
            for (int t = 0; t < 32; t++) o[2 + t] = (uint8_t)(int8_t)q[t];
        }
    }
}

/* f32::round (half away from zero) as i32 */
static inline int rnd_i(float x) { return ORC_PLANT == 1 ? as_i32(rintf(x)) : as_i32(roundf(x)); }
static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* kquant.rs L193-245 `quantize_k` (GT-10): RCE's reference quantizer of
 * one super-block of 256.  fmt: T_Q4_K, T_Q5_K or T_Q6_K.  q[256] in
 * position order; sc[8]/mn[8] (Q6_K: sc[16], mn unused). */
EXPORT void orc_quantize_k(const float *x, uint32_t fmt, int32_t *q, int32_t *sc,
                           int32_t *mn, float *d_out, float *dmin_out) {
    if (fmt == T_Q6_K) {
        float w[16];
        for (int b = 0; b < 16; b++) {
            float amax = 0.0f, m = 0.0f;
            for (int i = 0; i < 16; i++) {
                float v = x[b * 16 + i];
                if (ORC_PLANT == 5 ? amax <= fabsf(v) : amax < fabsf(v)) { amax = fabsf(v); m = v; }
            }
            w[b] = m / -32.0f;
        }
        float wmax = 0.0f;
        for (int b = 0; b < 16; b++) if (wmax < fabsf(w[b])) wmax = fabsf(w[b]);
        float d = orc_round_to_f16(wmax / 127.0f);
        for (int b = 0; b < 16; b++) sc[b] = d != 0.0f ? clampi(rnd_i(w[b] / d), -128, 127) : 0;
        for (int p = 0; p < 256; p++) {
            float s = d * (float)sc[p / 16];
            q[p] = s != 0.0f ? clampi(rnd_i(x[p] / s), -32, 31) : 0;
        }
        *d_out = d; *dmin_out = 0.0f;
        return;
    }
    float nmax = fmt == T_Q5_K ? 31.0f : 15.0f;
    float w[8], v[8];
    for (int b = 0; b < 8; b++) {
        float lo = ORC_PLANT == 2 ? INFINITY : 0.0f, hi = -INFINITY;
        for (int i = 0; i < 32; i++) {
            float t = x[b * 32 + i];
            if (t < lo) lo = t;
            if (t > hi) hi = t;
        }
        w[b] = (hi - lo) / nmax;
        v[b] = -lo;
    }
    float bw = 0.0f, bv = 0.0f;
    for (int b = 0; b < 8; b++) { if (w[b] > bw) bw = w[b]; if (v[b] > bv) bv = v[b]; }
    float d = orc_round_to_f16(bw / 63.0f);
    float dmin = orc_round_to_f16(bv / 63.0f);
    for (int b = 0; b < 8; b++) {
        int s = d != 0.0f ? rnd_i(w[b] / d) : 0;
        int m = dmin != 0.0f ? rnd_i(v[b] / dmin) : 0;
        sc[b] = d != 0.0f ? (s < 63 || ORC_PLANT == 3 ? s : 63) : 0;
        mn[b] = dmin != 0.0f ? (m < 63 || ORC_PLANT == 4 ? m : 63) : 0;
    }
    for (int p = 0; p < 256; p++) {
        float s = d * (float)sc[p / 32], o = dmin * (float)mn[p / 32];
        q[p] = s != 0.0f ? clampi(rnd_i((x[p] + o) / s), 0, (int)nmax) : 0;
    }
    *d_out = d; *dmin_out = dmin;
}

/* kquant.rs L284-292 `pack_scales`. */
static void pack_scales(const int32_t *sc, const int32_t *mn, uint8_t *s) {
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)(((uint8_t)sc[j] & 63) | ((uint8_t)(((uint8_t)sc[j + 4]) >> 4) << 6));
        s[j + 4] = (uint8_t)(((uint8_t)mn[j] & 63) | ((uint8_t)(((uint8_t)mn[j + 4]) >> 4) << 6));
        s[j + 8] = (uint8_t)(((uint8_t)sc[j + 4] & 15) | (((uint8_t)mn[j + 4] & 15) << 4));
    }
}

/* kquant.rs L295-302 `unpack_scale` == rce-op-qmm lib.rs L719-728
 * `q4_k_get_scale_min`. */
static inline void get_scale_min(const uint8_t *s, int j, int *sc, int *m) {
    if (j < 4) { *sc = s[j] & 63; *m = s[j + 4] & 63; }
    else {
        *sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* kquant.rs L304-346 `pack`: one super-block as GGUF bytes. */
EXPORT void orc_pack_k(const int32_t *q, const int32_t *sc, const int32_t *mn, float d,
                       float dmin, uint32_t fmt, uint8_t *out) {
    if (fmt == T_Q4_K || fmt == T_Q5_K) {
        uint16_t h = orc_f16_bits(d), hm = orc_f16_bits(dmin);
        out[0] = (uint8_t)h; out[1] = (uint8_t)(h >> 8);
        out[2] = (uint8_t)hm; out[3] = (uint8_t)(hm >> 8);
        pack_scales(sc, mn, out + 4);
        uint8_t *qs = out + 16;
        if (fmt == T_Q5_K) {
            uint8_t *qh = out + 16;
            memset(qh, 0, 32);
            for (int g = 0; g < 4; g++)
                for (int l = 0; l < 32; l++) {
                    qh[l] |= (uint8_t)(((q[g * 64 + l] >> 4) & 1) << (2 * g));
                    qh[l] |= (uint8_t)(((q[g * 64 + 32 + l] >> 4) & 1) << (2 * g + 1));
                }
            qs = out + 48;
        }
        for (int g = 0; g < 4; g++)
            for (int l = 0; l < 32; l++)
                qs[g * 32 + l] = (uint8_t)((q[g * 64 + l] & 15) | ((q[g * 64 + 32 + l] & 15) << 4));
        return;
    }
    /* Q6_K */
    uint8_t *ql = out, *qh = out + 128;
    for (int half = 0; half < 2; half++)
        for (int l = 0; l < 32; l++) {
            uint8_t q1 = (uint8_t)(q[half * 128 + l] + 32), q2 = (uint8_t)(q[half * 128 + l + 32] + 32);
            uint8_t q3 = (uint8_t)(q[half * 128 + l + 64] + 32), q4 = (uint8_t)(q[half * 128 + l + 96] + 32);
            ql[half * 64 + l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
            ql[half * 64 + l + 32] = (uint8_t)((q2 & 15) | ((q4 & 15) << 4));
            qh[half * 32 + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    for (int b = 0; b < 16; b++) out[192 + b] = (uint8_t)(int8_t)sc[b];
    uint16_t h = orc_f16_bits(d);
    out[208] = (uint8_t)h; out[209] = (uint8_t)(h >> 8);
}

/* kquant.rs L349-395 `unpack`: a super-block read back (value form). */
EXPORT void orc_unpack_k(const uint8_t *bytes, uint32_t fmt, int32_t *q, int32_t *sc,
                         int32_t *mn, float *d, float *dmin) {
    if (fmt == T_Q4_K || fmt == T_Q5_K) {
        *d = rd_f16(bytes); *dmin = rd_f16(bytes + 2);
        for (int j = 0; j < 8; j++) { int a, b; get_scale_min(bytes + 4, j, &a, &b); sc[j] = a; mn[j] = b; }
        const uint8_t *qh = bytes + 16, *qs = fmt == T_Q5_K ? bytes + 48 : bytes + 16;
        for (int g = 0; g < 4; g++)
            for (int l = 0; l < 32; l++) {
                int lo = qs[g * 32 + l] & 15, hi = qs[g * 32 + l] >> 4;
                if (fmt == T_Q5_K) {
                    lo |= ((qh[l] >> (2 * g)) & 1) << 4;
                    hi |= ((qh[l] >> (2 * g + 1)) & 1) << 4;
                }
                q[g * 64 + l] = lo; q[g * 64 + 32 + l] = hi;
            }
        return;
    }
    const uint8_t *ql = bytes, *qh = bytes + 128;
    for (int b = 0; b < 16; b++) sc[b] = (int8_t)bytes[192 + b];
    *d = rd_f16(bytes + 208); *dmin = 0.0f;
    for (int half = 0; half < 2; half++)
        for (int l = 0; l < 32; l++) {
            int a = ql[half * 64 + l], b = ql[half * 64 + l + 32], hb = qh[half * 32 + l];
            int at = half * 128;
            q[at + l] = ((a & 15) | ((hb & 3) << 4)) - 32;
            q[at + l + 32] = ((b & 15) | (((hb >> 2) & 3) << 4)) - 32;
            q[at + l + 64] = ((a >> 4) | (((hb >> 4) & 3) << 4)) - 32;
            q[at + l + 96] = ((b >> 4) | (((hb >> 6) & 3) << 4)) - 32;
        }
}

/* Whole tensors of n values (n a multiple of 256) quantized by quantize_k
 * and packed (spec/checker/tests/support/toy_llama.rs L26-29). */
EXPORT void orc_quantize_tensor_k(const float *w, size_t n, uint32_t fmt, uint8_t *out) {
    size_t nsb = n / 256, bb = fmt == T_Q6_K ? 210 : (fmt == T_Q5_K ? 176 : 144);
#pragma omp parallel for schedule(static)
    for (size_t b = 0; b < nsb; b++) {
        int32_t q[256], sc[16], mn[8]; float d, dmin;
        orc_quantize_k(w + b * 256, fmt, q, sc, mn, &d, &dmin);
        orc_pack_k(q, sc, mn, d, dmin, fmt, out + b * bb);
    }
}

/* ------------------------------------------------------------------ */
/* Dequantization (rce-ingest-gguf/src/dequant.rs)                     */
/* ------------------------------------------------------------------ */

/* dequant.rs L360-382 */
static void dq_q4_0(const uint8_t *x, size_t nb, float *out) {
    for (size_t b = 0; b < nb; b++, x += 18, out += 32) {
        float scale = rd_f16(x);
        for (int j = 0; j < 16; j++) {
            int v0 = (x[2 + j] & 0x0F) - 8, v1 = ((x[2 + j] >> 4) & 0x0F) - 8;
            out[j] = (float)v0 * scale;
            out[j + 16] = (float)v1 * scale;
        }
    }
}
/* dequant.rs L385-407 */
static void dq_q4_1(const uint8_t *x, size_t nb, float *out) {
    for (size_t b = 0; b < nb; b++, x += 20, out += 32) {
        float scale = rd_f16(x), min = rd_f16(x + 2);
        for (int j = 0; j < 16; j++) {
            float v0 = (float)(x[4 + j] & 0x0F), v1 = (float)((x[4 + j] >> 4) & 0x0F);
            out[j] = v0 * scale + min;
            out[j + 16] = v1 * scale + min;
        }
    }
}
/* dequant.rs L410-435 */
static void dq_q5_0(const uint8_t *x, size_t nb, float *out) {
    for (size_t b = 0; b < nb; b++, x += 22, out += 32) {
        float scale = rd_f16(x);
        uint32_t qh = (uint32_t)x[2] | ((uint32_t)x[3] << 8) | ((uint32_t)x[4] << 16) | ((uint32_t)x[5] << 24);
        for (int j = 0; j < 16; j++) {
            int h0 = (qh >> j) & 1, h1 = (qh >> (j + 16)) & 1;
            int v0 = ((x[6 + j] & 0x0F) | (h0 << 4)) - 16, v1 = ((x[6 + j] >> 4) | (h1 << 4)) - 16;
            out[j] = (float)v0 * scale;
            out[j + 16] = (float)v1 * scale;
        }
    }
}
/* dequant.rs L438-454 */
static void dq_q8_0(const uint8_t *x, size_t nb, float *out) {
    for (size_t b = 0; b < nb; b++, x += 34, out += 32) {
        float scale = rd_f16(x);
        for (int i = 0; i < 32; i++) out[i] = (float)(int8_t)x[2 + i] * scale;
    }
}
/* Q3_K sub-scale unpack (dequant.rs L488-503, rce-op-qmm lib.rs L877-894). */
static void q3k_scales(const uint8_t *sb, int8_t *scales) {
    const uint32_t K1 = 0x03030303u, K2 = 0x0f0f0f0fu;
    uint32_t aux[4];
    for (int k = 0; k < 3; k++)
        aux[k] = (uint32_t)sb[k * 4] | ((uint32_t)sb[k * 4 + 1] << 8) | ((uint32_t)sb[k * 4 + 2] << 16) | ((uint32_t)sb[k * 4 + 3] << 24);
    uint32_t tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & K2) | (((tmp >> 4) & K1) << 4);
    aux[3] = ((aux[1] >> 4) & K2) | (((tmp >> 6) & K1) << 4);
    aux[0] = (aux[0] & K2) | (((tmp) & K1) << 4);
    aux[1] = (aux[1] & K2) | (((tmp >> 2) & K1) << 4);
    for (int k = 0; k < 4; k++)
        for (int j = 0; j < 4; j++) scales[k * 4 + j] = (int8_t)((aux[k] >> (8 * j)) & 0xff);
}
/* dequant.rs L468-543 */
static void dq_q3_k(const uint8_t *x, size_t nb, float *out) {
    for (size_t b = 0; b < nb; b++, x += 110, out += 256) {
        const uint8_t *hmask = x, *qs = x + 32;
        float d_all = rd_f16(x + 108);
        int8_t scales[16];
        q3k_scales(x + 96, scales);
        uint8_t m = 1; int is = 0; int q_off = 0;
        for (int no = 0; no < 2; no++) {
            int shift = 0;
            for (int j = 0; j < 4; j++) {
                float dl1 = d_all * (float)(scales[is] - 32); is++;
                for (int l = 0; l < 16; l++) {
                    int ql = (qs[q_off + l] >> shift) & 3, hi = (hmask[l] & m) ? 0 : 4;
                    out[no * 128 + j * 32 + l] = dl1 * (float)(ql - hi);
                }
                float dl2 = d_all * (float)(scales[is] - 32); is++;
                for (int l = 0; l < 16; l++) {
                    int ql = (qs[q_off + l + 16] >> shift) & 3, hi = (hmask[l + 16] & m) ? 0 : 4;
                    out[no * 128 + j * 32 + 16 + l] = dl2 * (float)(ql - hi);
                }
                shift += 2; m = (uint8_t)(m << 1);
            }
            q_off += 32;
        }
    }
}
/* dequant.rs L546-589 */
static void dq_q4_k(const uint8_t *x, size_t nb, float *out) {
    for (size_t b = 0; b < nb; b++, x += 144, out += 256) {
        float d = rd_f16(x), dmin = rd_f16(x + 2);
        const uint8_t *scales = x + 4, *qs = x + 16;
        for (int j = 0; j < 4; j++) {
            int sc1, m1, sc2, m2;
            get_scale_min(scales, j * 2, &sc1, &m1);
            get_scale_min(scales, j * 2 + 1, &sc2, &m2);
            float d1 = d * (float)sc1, min1 = dmin * (float)m1;
            float d2 = d * (float)sc2, min2 = dmin * (float)m2;
            for (int l = 0; l < 32; l++) {
                uint8_t byte = qs[j * 32 + l];
                out[j * 64 + l] = d1 * (float)(byte & 0x0F) - min1;
                out[j * 64 + 32 + l] = d2 * (float)((byte >> 4) & 0x0F) - min2;
            }
        }
    }
}
/* dequant.rs L606-655 */
static void dq_q5_k(const uint8_t *x, size_t nb, float *out) {
    for (size_t b = 0; b < nb; b++, x += 176, out += 256) {
        float d = rd_f16(x), dmin = rd_f16(x + 2);
        const uint8_t *scales = x + 4, *qh = x + 16, *qs = x + 48;
        uint8_t u1 = 1, u2 = 2;
        for (int j = 0; j < 4; j++) {
            int sc1, m1, sc2, m2;
            get_scale_min(scales, j * 2, &sc1, &m1);
            get_scale_min(scales, j * 2 + 1, &sc2, &m2);
            float d1 = d * (float)sc1, min1 = dmin * (float)m1;
            float d2 = d * (float)sc2, min2 = dmin * (float)m2;
            for (int l = 0; l < 32; l++) {
                uint8_t byte = qs[j * 32 + l];
                uint32_t h1 = (qh[l] & u1) ? 16u : 0u, h2 = (qh[l] & u2) ? 16u : 0u;
                out[j * 64 + l] = d1 * (float)((byte & 0x0F) + h1) - min1;
                out[j * 64 + 32 + l] = d2 * (float)(((byte >> 4) & 0x0F) + h2) - min2;
            }
            u1 = (uint8_t)(u1 << 2); u2 = (uint8_t)(u2 << 2);
        }
    }
}
/* dequant.rs L658-701 */
static void dq_q6_k(const uint8_t *x, size_t nb, float *out) {
    for (size_t b = 0; b < nb; b++, x += 210, out += 256) {
        const uint8_t *ql = x, *qh = x + 128;
        const int8_t *sc = (const int8_t *)(x + 192);
        float d = rd_f16(x + 208);
        for (int o = 0; o < 2; o++) {
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = ((ql[o * 64 + l] & 0x0F) | ((qh[o * 32 + l] & 3) << 4)) - 32;
                int q2 = ((ql[o * 64 + l + 32] & 0x0F) | (((qh[o * 32 + l] >> 2) & 3) << 4)) - 32;
                int q3 = ((ql[o * 64 + l] >> 4) | (((qh[o * 32 + l] >> 4) & 3) << 4)) - 32;
                int q4 = ((ql[o * 64 + l + 32] >> 4) | (((qh[o * 32 + l] >> 6) & 3) << 4)) - 32;
                float *ob = out + o * 128;
                ob[l] = d * (float)sc[o * 8 + is] * (float)q1;
                ob[l + 32] = d * (float)sc[o * 8 + is + 2] * (float)q2;
                ob[l + 64] = d * (float)sc[o * 8 + is + 4] * (float)q3;
                ob[l + 96] = d * (float)sc[o * 8 + is + 6] * (float)q4;
            }
        }
    }
}

/* dequant.rs L141-148 STQ1_0_CODEBOOK: (sign << 4 | code) -> four 2-bit
 * lanes (lane p at bits 2p; 0 = -1, 1 = 0, 2 = +1).  A table of the
 * format, the same in every implementation. */
static const uint8_t STQ1_CB[32] = {
    0xA9, 0x89, 0x29, 0x09, 0xA6, 0x86, 0x26, 0x06, 0x9A, 0x92, 0x1A, 0x12, 0x6A, 0x62, 0x4A, 0x42,
    0x01, 0x21, 0x81, 0xA1, 0x04, 0x24, 0x84, 0xA4, 0x10, 0x18, 0x90, 0x98, 0x40, 0x48, 0x60, 0x68};
EXPORT uint8_t orc_stq1_0_codebook(int i) { return STQ1_CB[i & 31]; }

/* dequant.rs L222-256 dequant_i2_s: byte gp of block b holds positions
 * 128 b + {gp, 32 + gp, 64 + gp, 96 + gp} at bits 7:6, 5:4, 3:2, 1:0;
 * w = scale * map2bit[code], map2bit = {-1, 0, +1, 0}; the f32 scale
 * follows the ceil(n / 4) code bytes. */
static void dq_i2_s(const uint8_t *x, size_t n, float *out) {
    static const float MAP[4] = {-1.0f, 0.0f, 1.0f, 0.0f};
    float scale; memcpy(&scale, x + (n + 3) / 4, 4);
    for (size_t b = 0; b < (n + 127) / 128; b++)
        for (int gp = 0; gp < 32; gp++) {
            uint8_t byte = x[b * 32 + gp];
            for (int c = 0; c < 4; c++) {
                size_t i = b * 128 + (size_t)(32 * c + gp);
                if (i < n) out[i] = scale * MAP[(byte >> (6 - 2 * c)) & 3];
            }
        }
}
/* dequant.rs L272-299 dequant_q1_0: bit j of qs (LSB first) -> +d, else -d. */
static void dq_q1_0(const uint8_t *x, size_t nb, float *out) {
    for (size_t b = 0; b < nb; b++, x += 18, out += 128) {
        float d = rd_f16(x), nd = -d;
        for (int j = 0; j < 128; j++) out[j] = ((x[2 + j / 8] >> (j % 8)) & 1) ? d : nd;
    }
}
/* dequant.rs L317-340 dequant_q2_0: q = 2-bit lane j % 4 of qs[j / 4]; (q - 1) * d. */
static void dq_q2_0(const uint8_t *x, size_t nb, float *out) {
    for (size_t b = 0; b < nb; b++, x += 34, out += 128) {
        float d = rd_f16(x);
        for (int j = 0; j < 128; j++) out[j] = (float)(((x[2 + j / 4] >> ((j % 4) * 2)) & 3) - 1) * d;
    }
}
/* dequant.rs L162-196 dequant_stq1_0: group g of 4: code = nibble g & 1 of
 * qs[g / 2], sign = bit g % 8 of sign[g / 8], lanes from the codebook. */
static void dq_stq1_0(const uint8_t *x, size_t nb, float *out) {
    for (size_t b = 0; b < nb; b++, x += 42, out += 256) {
        float d = rd_f16(x + 40);
        for (int g = 0; g < 64; g++) {
            int code = (x[g / 2] >> (4 * (g & 1))) & 0xF, sg = (x[32 + g / 8] >> (g % 8)) & 1;
            uint8_t qp = STQ1_CB[(sg << 4) | code];
            for (int p = 0; p < 4; p++) out[4 * g + p] = (float)(((qp >> (2 * p)) & 3) - 1) * d;
        }
    }
}

/* dequant.rs L115-134 `dequantize_to_f32` for whole blocks (n a multiple
 * of the block size).  Returns 0, or -1 for an unsupported type. */
EXPORT int orc_dequantize(const uint8_t *bytes, uint32_t t, size_t n, float *out) {
    switch (t) {
    case T_F32: memcpy(out, bytes, n * 4); return 0;
    case T_F16: for (size_t i = 0; i < n; i++) out[i] = rd_f16(bytes + 2 * i); return 0;
    case T_BF16: for (size_t i = 0; i < n; i++) out[i] = rd_bf16(bytes + 2 * i); return 0;
    case T_Q4_0: dq_q4_0(bytes, n / 32, out); return 0;
    case T_Q4_1: dq_q4_1(bytes, n / 32, out); return 0;
    case T_Q5_0: dq_q5_0(bytes, n / 32, out); return 0;
    case T_Q8_0: dq_q8_0(bytes, n / 32, out); return 0;
    case T_Q3_K: dq_q3_k(bytes, n / 256, out); return 0;
    case T_Q4_K: dq_q4_k(bytes, n / 256, out); return 0;
    case T_Q5_K: dq_q5_k(bytes, n / 256, out); return 0;
    case T_Q6_K: dq_q6_k(bytes, n / 256, out); return 0;
    case T_I2_S: dq_i2_s(bytes, n, out); return 0;
    case T_Q1_0: dq_q1_0(bytes, n / 128, out); return 0;
    case T_Q2_0: dq_q2_0(bytes, n / 128, out); return 0;
    case T_STQ1_0: dq_stq1_0(bytes, n / 256, out); return 0;
    default: return -1;
    }
}

/* ------------------------------------------------------------------ */
/* Row dots of mm_1d (rce-op-qmm/src/lib.rs), exact reference order    */
/* ------------------------------------------------------------------ */

/* lib.rs L458-470 mm_1d_f32 */
static float row_f32(const float *a, const uint8_t *r, size_t k) {
    float acc = 0.0f;
    for (size_t i = 0; i < k; i++) { float w; memcpy(&w, r + 4 * i, 4); acc += a[i] * w; }
    return acc;
}
/* lib.rs L472-480 mm_1d_f16 */
static float row_f16(const float *a, const uint8_t *r, size_t k) {
    float acc = 0.0f;
    for (size_t i = 0; i < k; i++) acc += a[i] * rd_f16(r + 2 * i);
    return acc;
}
/* lib.rs L482-490 mm_1d_bf16 */
static float row_bf16(const float *a, const uint8_t *r, size_t k) {
    float acc = 0.0f;
    for (size_t i = 0; i < k; i++) acc += a[i] * rd_bf16(r + 2 * i);
    return acc;
}
/* lib.rs L496-522 mm_1d_q4_0: sub over q in 0..16 of v0*a[q] then
 * v1*a[q+16] (GT-4 order 0,16,1,17,...); sumf += scale*sub. */
static float row_q4_0(const float *a, const uint8_t *r, size_t k) {
    float sumf = 0.0f;
    for (size_t ib = 0; ib < k / 32; ib++) {
        const uint8_t *s = r + ib * 18;
        float scale = rd_f16(s);
        const float *ab = a + ib * 32;
        float sub = 0.0f;
        for (int q = 0; q < 16; q++) {
            int v0 = (s[2 + q] & 0x0F) - 8, v1 = ((s[2 + q] >> 4) & 0x0F) - 8;
            sub += (float)v0 * ab[q];
            sub += (float)v1 * ab[q + 16];
        }
        sumf += scale * sub;
    }
    return sumf;
}
/* lib.rs L615-645 mm_1d_q4_1 */
static float row_q4_1(const float *a, const uint8_t *r, size_t k) {
    float sumf = 0.0f;
    for (size_t ib = 0; ib < k / 32; ib++) {
        const uint8_t *s = r + ib * 20;
        float scale = rd_f16(s), min = rd_f16(s + 2);
        const float *ab = a + ib * 32;
        float va = 0.0f, asum = 0.0f;
        for (int q = 0; q < 16; q++) {
            float v0 = (float)(s[4 + q] & 0x0F), v1 = (float)((s[4 + q] >> 4) & 0x0F);
            float alo = ab[q], ahi = ab[q + 16];
            va += v0 * alo + v1 * ahi;
            asum += alo + ahi;
        }
        sumf += scale * va + min * asum;
    }
    return sumf;
}
/* lib.rs L331-352 dot_row_q5_0 (== mm_1d_q5_0 L525-561) */
static float row_q5_0(const float *a, const uint8_t *r, size_t k) {
    float sumf = 0.0f;
    for (size_t ib = 0; ib < k / 32; ib++) {
        const uint8_t *s = r + ib * 22;
        float scale = rd_f16(s);
        uint32_t qh = (uint32_t)s[2] | ((uint32_t)s[3] << 8) | ((uint32_t)s[4] << 16) | ((uint32_t)s[5] << 24);
        const float *ab = a + ib * 32;
        float sub = 0.0f;
        for (int q = 0; q < 16; q++) {
            int h0 = (qh >> q) & 1, h1 = (qh >> (q + 16)) & 1;
            int v0 = ((s[6 + q] & 0x0F) | (h0 << 4)) - 16, v1 = ((s[6 + q] >> 4) | (h1 << 4)) - 16;
            sub += (float)v0 * ab[q];
            sub += (float)v1 * ab[q + 16];
        }
        sumf += scale * sub;
    }
    return sumf;
}
/* lib.rs L315-328 dot_row_q8_0 (== mm_1d_q8_0 L648-670) */
static float row_q8_0(const float *a, const uint8_t *r, size_t k) {
    float sumf = 0.0f;
    for (size_t ib = 0; ib < k / 32; ib++) {
        const uint8_t *s = r + ib * 34;
        float scale = rd_f16(s);
        const float *ab = a + ib * 32;
        float sub = 0.0f;
        for (int q = 0; q < 32; q++) sub += (float)(int8_t)s[2 + q] * ab[q];
        sumf += scale * sub;
    }
    return sumf;
}
/* lib.rs L840-928 mm_1d_q3_k */
static float row_q3_k(const float *a, const uint8_t *r, size_t k) {
    float sumf = 0.0f;
    for (size_t ib = 0; ib < k / 256; ib++) {
        const uint8_t *s = r + ib * 110, *hmask = s, *qs = s + 32;
        float d_all = rd_f16(s + 108);
        int8_t scales[16];
        q3k_scales(s + 96, scales);
        const float *as = a + ib * 256;
        uint8_t m = 1; int is = 0, q_off = 0;
        for (int outer = 0; outer < 2; outer++) {
            int shift = 0;
            for (int jj = 0; jj < 4; jj++) {
                float dl1 = d_all * (float)(scales[is] - 32);
                float dl2 = d_all * (float)(scales[is + 1] - 32);
                const float *ab = as + outer * 128 + jj * 32;
                float s1 = 0.0f, s2 = 0.0f;
                for (int l = 0; l < 16; l++) {
                    int ql1 = (qs[q_off + l] >> shift) & 3, h1 = (hmask[l] & m) ? 0 : 4;
                    s1 += (float)(ql1 - h1) * ab[l];
                    int ql2 = (qs[q_off + l + 16] >> shift) & 3, h2 = (hmask[l + 16] & m) ? 0 : 4;
                    s2 += (float)(ql2 - h2) * ab[16 + l];
                }
                sumf += dl1 * s1 + dl2 * s2;
                is += 2; shift += 2; m = (uint8_t)(m << 1);
            }
            q_off += 32;
        }
    }
    return sumf;
}
/* lib.rs L354-385 dot_row_q4_k (== mm_1d_q4_k L730-781):
 * per group g: sumf += d1*va_lo - min1*a_lo + d2*va_hi - min2*a_hi,
 * evaluated left to right. */
static float row_q4_k(const float *a, const uint8_t *r, size_t k) {
    float sumf = 0.0f;
    for (size_t ib = 0; ib < k / 256; ib++) {
        const uint8_t *s = r + ib * 144;
        float d = rd_f16(s), dmin = rd_f16(s + 2);
        const uint8_t *scales = s + 4, *qs = s + 16;
        for (int g = 0; g < 4; g++) {
            int sc1, m1, sc2, m2;
            get_scale_min(scales, g * 2, &sc1, &m1);
            get_scale_min(scales, g * 2 + 1, &sc2, &m2);
            float d1 = d * (float)sc1, min1 = dmin * (float)m1;
            float d2 = d * (float)sc2, min2 = dmin * (float)m2;
            const float *ab = a + ib * 256 + g * 64;
            float va_lo = 0.0f, a_lo = 0.0f, va_hi = 0.0f, a_hi = 0.0f;
            for (int l = 0; l < 32; l++) {
                uint8_t byte = qs[g * 32 + l];
                float al = ab[l], ah = ab[32 + l];
                va_lo += (float)(byte & 0x0F) * al;
                a_lo += al;
                va_hi += (float)((byte >> 4) & 0x0F) * ah;
                a_hi += ah;
            }
            float t = d1 * va_lo;
            t = t - min1 * a_lo;
            t = t + d2 * va_hi;
            t = t - min2 * a_hi;
            sumf += t;
        }
    }
    return sumf;
}
/* lib.rs L388-422 dot_row_q5_k (== mm_1d_q5_k L783-838) */
static float row_q5_k(const float *a, const uint8_t *r, size_t k) {
    float sumf = 0.0f;
    for (size_t ib = 0; ib < k / 256; ib++) {
        const uint8_t *s = r + ib * 176;
        float d = rd_f16(s), dmin = rd_f16(s + 2);
        const uint8_t *scales = s + 4, *qh = s + 16, *qs = s + 48;
        for (int g = 0; g < 4; g++) {
            int sc1, m1, sc2, m2;
            get_scale_min(scales, g * 2, &sc1, &m1);
            get_scale_min(scales, g * 2 + 1, &sc2, &m2);
            float d1 = d * (float)sc1, min1 = dmin * (float)m1;
            float d2 = d * (float)sc2, min2 = dmin * (float)m2;
            const float *ab = a + ib * 256 + g * 64;
            float va_lo = 0.0f, a_lo = 0.0f, va_hi = 0.0f, a_hi = 0.0f;
            for (int l = 0; l < 32; l++) {
                uint8_t byte = qs[g * 32 + l];
                int h1 = ((qh[l] >> (2 * g)) & 1) << 4, h2 = ((qh[l] >> (2 * g + 1)) & 1) << 4;
                float al = ab[l], ah = ab[32 + l];
                va_lo += (float)((byte & 0x0F) | h1) * al;
                a_lo += al;
                va_hi += (float)(((byte >> 4) & 0x0F) | h2) * ah;
                a_hi += ah;
            }
            float t = d1 * va_lo;
            t = t - min1 * a_lo;
            t = t + d2 * va_hi;
            t = t - min2 * a_hi;
            sumf += t;
        }
    }
    return sumf;
}
/* lib.rs L425-454 dot_row_q6_k (== mm_1d_q6_k L1667-1705):
 * sumf += ((d*sc)*q)*a over positions l, l+32, l+64, l+96 of each half. */
static float row_q6_k(const float *a, const uint8_t *r, size_t k) {
    float sumf = 0.0f;
    for (size_t ib = 0; ib < k / 256; ib++) {
        const uint8_t *s = r + ib * 210, *ql = s, *qh = s + 128;
        const int8_t *sc = (const int8_t *)(s + 192);
        float d = rd_f16(s + 208);
        for (int o = 0; o < 2; o++) {
            const float *ab = a + ib * 256 + o * 128;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = ((ql[o * 64 + l] & 0x0F) | ((qh[o * 32 + l] & 3) << 4)) - 32;
                int q2 = ((ql[o * 64 + l + 32] & 0x0F) | (((qh[o * 32 + l] >> 2) & 3) << 4)) - 32;
                int q3 = ((ql[o * 64 + l] >> 4) | (((qh[o * 32 + l] >> 4) & 3) << 4)) - 32;
                int q4 = ((ql[o * 64 + l + 32] >> 4) | (((qh[o * 32 + l] >> 6) & 3) << 4)) - 32;
                float t;
                t = d * (float)sc[o * 8 + is]; t = t * (float)q1; t = t * ab[l]; sumf += t;
                t = d * (float)sc[o * 8 + is + 2]; t = t * (float)q2; t = t * ab[l + 32]; sumf += t;
                t = d * (float)sc[o * 8 + is + 4]; t = t * (float)q3; t = t * ab[l + 64]; sumf += t;
                t = d * (float)sc[o * 8 + is + 6]; t = t * (float)q4; t = t * ab[l + 96]; sumf += t;
            }
        }
    }
    return sumf;
}

/* lib.rs L1716-1760 mm_1d_q1_0: per block of 128, pos / neg over j
 * ascending (bit j set: pos += a, else neg += a); sumf += d * (pos - neg). */
static float row_q1_0(const float *a, const uint8_t *r, size_t k) {
    float sumf = 0.0f;
    for (size_t b = 0; b < k / 128; b++) {
        const uint8_t *s = r + b * 18;
        float d = rd_f16(s), pos = 0.0f, neg = 0.0f;
        for (int j = 0; j < 128; j++) {
            float av = a[b * 128 + j];
            if ((s[2 + j / 8] >> (j % 8)) & 1) pos += av; else neg += av;
        }
        sumf += d * (pos - neg);
    }
    return sumf;
}
/* lib.rs L1766-1815 mm_1d_q2_0: code 0 -> neg, 2 -> pos, 3 -> plus2, 1 ->
 * nothing; sumf += d * ((pos - neg) + 2 * plus2). */
static float row_q2_0(const float *a, const uint8_t *r, size_t k) {
    float sumf = 0.0f;
    for (size_t b = 0; b < k / 128; b++) {
        const uint8_t *s = r + b * 34;
        float d = rd_f16(s), pos = 0.0f, neg = 0.0f, plus2 = 0.0f;
        for (int j = 0; j < 128; j++) {
            int code = (s[2 + j / 4] >> ((j % 4) * 2)) & 3;
            float av = a[b * 128 + j];
            if (code == 0) neg += av; else if (code == 2) pos += av; else if (code == 3) plus2 += av;
        }
        float t = pos - neg;
        t = t + 2.0f * plus2;
        sumf += d * t;
    }
    return sumf;
}
/* lib.rs L1821-1875 mm_1d_stq1_0: lane value 2 -> pos, 0 -> neg; sumf +=
 * d * (pos - neg) per super-block of 256. */
static float row_stq1_0(const float *a, const uint8_t *r, size_t k) {
    float sumf = 0.0f;
    for (size_t b = 0; b < k / 256; b++) {
        const uint8_t *s = r + b * 42;
        float d = rd_f16(s + 40), pos = 0.0f, neg = 0.0f;
        for (int g = 0; g < 64; g++) {
            int code = (s[g / 2] >> (4 * (g & 1))) & 0xF, sg = (s[32 + g / 8] >> (g % 8)) & 1;
            uint8_t qp = STQ1_CB[(sg << 4) | code];
            for (int p = 0; p < 4; p++) {
                int q = (qp >> (2 * p)) & 3;
                float av = a[b * 256 + 4 * g + p];
                if (q == 2) pos += av; else if (q == 0) neg += av;
            }
        }
        sumf += d * (pos - neg);
    }
    return sumf;
}
/* lib.rs L1478-1537 mm_1d_i2_s: pos / neg over the whole row, byte gp of
 * each block of 128 in order, its codes for positions gp, 32 + gp, 64 + gp,
 * 96 + gp (bits 7:6, 5:4, 3:2, 1:0); code 2 -> pos, 0 -> neg; the row is
 * scale * (pos - neg) with the tensor's one f32 scale. */
static float row_i2_s(const float *a, const uint8_t *r, size_t k, float scale) {
    float pos = 0.0f, neg = 0.0f;
    for (size_t b = 0; b < k / 128; b++)
        for (int gp = 0; gp < 32; gp++) {
            uint8_t byte = r[b * 32 + gp];
            for (int c = 0; c < 4; c++) {
                int code = (byte >> (6 - 2 * c)) & 3;
                float av = a[b * 128 + (size_t)(32 * c + gp)];
                if (code == 2) pos += av; else if (code == 0) neg += av;
            }
        }
    return scale * (pos - neg);
}

typedef float (*row_fn)(const float *, const uint8_t *, size_t);

static row_fn pick_row(uint32_t t, uint32_t *qk, uint32_t *bb) {
    if (orc_block_geometry(t, qk, bb)) return 0;
    switch (t) {
    case T_F32: return row_f32;
    case T_F16: return row_f16;
    case T_BF16: return row_bf16;
    case T_Q4_0: return row_q4_0;
    case T_Q4_1: return row_q4_1;
    case T_Q5_0: return row_q5_0;
    case T_Q8_0: return row_q8_0;
    case T_Q3_K: return row_q3_k;
    case T_Q4_K: return row_q4_k;
    case T_Q5_K: return row_q5_k;
    case T_Q6_K: return row_q6_k;
    case T_Q1_0: return row_q1_0;
    case T_Q2_0: return row_q2_0;
    case T_STQ1_0: return row_stq1_0;
    default: return 0;
    }
}

/* lib.rs L216-270 `mm_1d` (and L943-1023 `mm_batched`, which is byte
 * identical to t_rows calls of mm_1d): out[t*n + j] = row_dot(a_t, W_j).
 * Rows are spread over `threads` OpenMP threads, one task per output row
 * as rayon's par_iter_mut does (L502); the arithmetic per row is serial,
 * so the result does not depend on the thread count.
 * Returns 0, -1 unsupported dtype, -2 n_cols not a block multiple. */
EXPORT int orc_mm_batched(const float *a, size_t t_rows, const uint8_t *w, uint32_t t,
                          size_t n_rows, size_t n_cols, float *out, int threads) {
    uint32_t qk, bb;
    if (threads < 1) threads = 1;
    if (t == T_I2_S) {
        if (n_cols % 128) return -2;
        float scale; memcpy(&scale, w + n_rows * (n_cols / 4), 4);
        for (size_t tr = 0; tr < t_rows; tr++) {
#pragma omp parallel for schedule(dynamic, 16) num_threads(threads)
            for (size_t j = 0; j < n_rows; j++)
                out[tr * n_rows + j] = row_i2_s(a + tr * n_cols, w + j * (n_cols / 4), n_cols, scale);
        }
        return 0;
    }
    row_fn f = pick_row(t, &qk, &bb);
    if (!f) return -1;
    if (n_cols % qk) return -2;
    size_t row_bytes = n_cols / qk * bb;
    for (size_t tr = 0; tr < t_rows; tr++) {
        const float *at = a + tr * n_cols;
        float *ot = out + tr * n_rows;
#pragma omp parallel for schedule(dynamic, 16) num_threads(threads)
        for (size_t j = 0; j < n_rows; j++) ot[j] = f(at, w + j * row_bytes, n_cols);
    }
    return 0;
}

EXPORT int orc_mm_1d(const float *a, const uint8_t *w, uint32_t t, size_t n_rows,
                     size_t n_cols, float *out, int threads) {
    return orc_mm_batched(a, 1, w, t, n_rows, n_cols, out, threads);
}

/* ------------------------------------------------------------------ */
/* Value-form products (independent restatement of the same order)     */
/* ------------------------------------------------------------------ */

/* rce-vm-backend-cpu/src/ml/nn.rs L477-518 `matmul_q`: x (m,k) f32,
 * q (n,k) i32 values, d (n,k/32) f32.  Q4_0 order 0,16,1,17,...,15,31. */
EXPORT void orc_matmul_q(const float *x, size_t m, size_t k, const int32_t *q, size_t n,
                         const float *d, int q4, float *out) {
    int order[32];
    for (int t = 0; t < 32; t++) order[t] = q4 ? ((t & 1) ? t / 2 + 16 : t / 2) : t;
    size_t nb = k / 32;
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) {
            const float *xr = x + i * k;
            const int32_t *qr = q + j * k;
            float sum = 0.0f;
            for (size_t b = 0; b < nb; b++) {
                float sub = 0.0f;
                for (int t = 0; t < 32; t++) {
                    size_t at = b * 32 + (size_t)order[t];
                    sub += (float)qr[at] * xr[at];
                }
                sum += d[j * nb + b] * sub;
            }
            out[i * n + j] = sum;
        }
}

/* kquant.rs L81-149 `matmul_k`: x (m,k); q (n,k) values; s, o (n, k/32)
 * (Q6_K: s (n, k/16), o unused). */
EXPORT void orc_matmul_k(const float *x, size_t m, size_t k, const int32_t *q, size_t n,
                         const float *s, const float *o, uint32_t fmt, float *out) {
    size_t sub = fmt == T_Q6_K ? 16 : 32, ns = k / sub;
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) {
            const float *xr = x + i * k, *sr = s + j * ns;
            const int32_t *qr = q + j * k;
            float y = 0.0f;
            if (fmt == T_Q6_K) {
                for (size_t sb = 0; sb < k / 256; sb++)
                    for (int half = 0; half < 2; half++) {
                        size_t base = sb * 256 + (size_t)half * 128;
                        for (int l = 0; l < 32; l++)
                            for (int c = 0; c < 4; c++) {
                                size_t p = base + (size_t)l + 32 * (size_t)c;
                                float t = sr[p / 16] * (float)qr[p];
                                t = t * xr[p];
                                y += t;
                            }
                    }
            } else {
                const float *orow = o + j * ns;
                for (size_t g = 0; g < k / 64; g++) {
                    size_t b1 = 2 * g, b2 = 2 * g + 1;
                    float u1 = 0.0f, a1 = 0.0f, u2 = 0.0f, a2 = 0.0f;
                    for (int t = 0; t < 32; t++) {
                        size_t p1 = b1 * 32 + (size_t)t, p2 = b2 * 32 + (size_t)t;
                        u1 += (float)qr[p1] * xr[p1];
                        a1 += xr[p1];
                        u2 += (float)qr[p2] * xr[p2];
                        a2 += xr[p2];
                    }
                    float t = sr[b1] * u1;
                    t = t - orow[b1] * a1;
                    t = t + sr[b2] * u2;
                    t = t - orow[b2] * a2;
                    y += t;
                }
            }
            out[i * n + j] = y;
        }
}

/* ------------------------------------------------------------------ */
/* Q8-activation path (defined by this build; no reference kernel)     */
/* ------------------------------------------------------------------ */
/*
 * The activation row is quantized per block of 32 with nn.rs
 * `quantize_block(x, false)` semantics: xq = round(x * (1/d)), d = amax/127,
 * stored scale dx = round_to_f16(d).  Each weight format's per-block
 * sub-sum (the reference's `sub`, `va`, `a` sums over a block of 32, or of
 * 16 for Q6_K) is replaced by dx * (exact integer dot of the block); the
 * rest of each row formula and its fold order are the reference's:
 *   Q8_0, Q4_0, Q5_0 : sub = dx * isum;      sumf += scale * sub
 *   Q4_1       : va = dx * isum, a = dx * xsum (isum over the raw
 *                nibbles 0..15); sumf += scale * va + min * a
 *   Q3_K       : per 32 values (outer, j) of lib.rs L840-928, the two
 *                halves of 16 get s1 = dx * isum1, s2 = dx * isum2;
 *                sumf += dl1 * s1 + dl2 * s2
 *   Q4_K, Q5_K : va = dx * isum, a = dx * xsum (xsum = sum of xq);
 *                sumf += d1*va_lo - min1*a_lo + d2*va_hi - min2*a_hi
 *                (Q5_K: the 5-bit values of lib.rs L388-422)
 *   Q6_K       : per super-block, ssb = sum over sub-blocks of 16 b ascending
 *                of (d*sc_b) * (dx * isum_b) from +0.0; sumf += ssb
 */
EXPORT void orc_quantize_act_q8(const float *x, size_t k, int8_t *xq, float *dx, int32_t *xsum) {
    for (size_t b = 0; b < k / 32; b++) {
        int32_t q[32]; float d; int32_t s = 0;
        orc_quantize_block(x + b * 32, 0, q, &d);
        for (int i = 0; i < 32; i++) { xq[b * 32 + i] = (int8_t)q[i]; s += q[i]; }
        dx[b] = d;
        if (xsum) xsum[b] = s;
    }
}

static float row_q8_path(uint32_t t, const int8_t *xq, const float *dx, const uint8_t *r, size_t k) {
    float sumf = 0.0f;
    if (t == T_Q8_0 || t == T_Q4_0 || t == T_Q5_0) {
        size_t bb = t == T_Q8_0 ? 34 : (t == T_Q4_0 ? 18 : 22);
        for (size_t ib = 0; ib < k / 32; ib++) {
            const uint8_t *s = r + ib * bb;
            const int8_t *xb = xq + ib * 32;
            int32_t isum = 0;
            if (t == T_Q8_0) {
                for (int q = 0; q < 32; q++) isum += (int32_t)(int8_t)s[2 + q] * xb[q];
            } else if (t == T_Q4_0) {
                for (int q = 0; q < 16; q++) {
                    isum += ((s[2 + q] & 0x0F) - 8) * xb[q];
                    isum += ((s[2 + q] >> 4) - 8) * xb[q + 16];
                }
            } else {  /* Q5_0: the 5-bit values of lib.rs L525-561 */
                uint32_t qh = (uint32_t)s[2] | ((uint32_t)s[3] << 8) | ((uint32_t)s[4] << 16) | ((uint32_t)s[5] << 24);
                for (int q = 0; q < 16; q++) {
                    isum += ((int)((s[6 + q] & 0x0F) | (((qh >> q) & 1) << 4)) - 16) * xb[q];
                    isum += ((int)((s[6 + q] >> 4) | (((qh >> (q + 16)) & 1) << 4)) - 16) * xb[q + 16];
                }
            }
            float sub = dx[ib] * (float)isum;
            sumf += rd_f16(s) * sub;
        }
    } else if (t == T_Q4_1) {
        for (size_t ib = 0; ib < k / 32; ib++) {
            const uint8_t *s = r + ib * 20;
            const int8_t *xb = xq + ib * 32;
            int32_t isum = 0, xs = 0;
            for (int q = 0; q < 16; q++) {
                isum += (s[4 + q] & 0x0F) * xb[q] + (s[4 + q] >> 4) * xb[q + 16];
                xs += xb[q] + xb[q + 16];
            }
            float va = dx[ib] * (float)isum, a = dx[ib] * (float)xs;
            float tt = rd_f16(s) * va;
            tt = tt + rd_f16(s + 2) * a;
            sumf += tt;
        }
    } else if (t == T_Q4_K || t == T_Q5_K) {
        const int q5 = t == T_Q5_K;
        const size_t bb = q5 ? 176 : 144, qs_off = q5 ? 48 : 16;
        for (size_t ib = 0; ib < k / 256; ib++) {
            const uint8_t *s = r + ib * bb;
            float d = rd_f16(s), dmin = rd_f16(s + 2);
            for (int g = 0; g < 4; g++) {
                int sc1, m1, sc2, m2;
                get_scale_min(s + 4, g * 2, &sc1, &m1);
                get_scale_min(s + 4, g * 2 + 1, &sc2, &m2);
                float d1 = d * (float)sc1, min1 = dmin * (float)m1;
                float d2 = d * (float)sc2, min2 = dmin * (float)m2;
                size_t b_lo = ib * 8 + (size_t)g * 2, b_hi = b_lo + 1;
                const int8_t *xl = xq + b_lo * 32, *xh = xq + b_hi * 32;
                int32_t il = 0, ih = 0, sl = 0, sh = 0;
                for (int l = 0; l < 32; l++) {
                    uint8_t byte = s[qs_off + g * 32 + l];
                    int h1 = 0, h2 = 0;
                    if (q5) {
                        h1 = ((s[16 + l] >> (2 * g)) & 1) << 4;
                        h2 = ((s[16 + l] >> (2 * g + 1)) & 1) << 4;
                    }
                    il += ((byte & 0x0F) | h1) * xl[l]; sl += xl[l];
                    ih += ((byte >> 4) | h2) * xh[l]; sh += xh[l];
                }
                float va_lo = dx[b_lo] * (float)il, a_lo = dx[b_lo] * (float)sl;
                float va_hi = dx[b_hi] * (float)ih, a_hi = dx[b_hi] * (float)sh;
                float tt = d1 * va_lo;
                tt = tt - min1 * a_lo;
                tt = tt + d2 * va_hi;
                tt = tt - min2 * a_hi;
                sumf += tt;
            }
        }
    } else if (t == T_Q3_K) {
        for (size_t ib = 0; ib < k / 256; ib++) {
            const uint8_t *s = r + ib * 110, *hmask = s, *qs = s + 32;
            float d_all = rd_f16(s + 108);
            int8_t scales[16];
            q3k_scales(s + 96, scales);
            for (int outer = 0; outer < 2; outer++)
                for (int jj = 0; jj < 4; jj++) {
                    const int is = 8 * outer + 2 * jj, shift = 2 * jj;
                    const uint8_t m = (uint8_t)(1u << (4 * outer + jj));
                    const size_t b = ib * 8 + (size_t)(4 * outer + jj);  /* the block of 32 */
                    const int8_t *xb = xq + b * 32;
                    int32_t i1 = 0, i2 = 0;
                    for (int l = 0; l < 16; l++) {
                        i1 += (((qs[32 * outer + l] >> shift) & 3) - ((hmask[l] & m) ? 0 : 4)) * xb[l];
                        i2 += (((qs[32 * outer + 16 + l] >> shift) & 3) - ((hmask[16 + l] & m) ? 0 : 4)) * xb[16 + l];
                    }
                    float dl1 = d_all * (float)(scales[is] - 32), dl2 = d_all * (float)(scales[is + 1] - 32);
                    float s1 = dx[b] * (float)i1, s2 = dx[b] * (float)i2;
                    float tt = dl1 * s1;
                    tt = tt + dl2 * s2;
                    sumf += tt;
                }
        }
    } else if (t == T_Q6_K) {
        for (size_t ib = 0; ib < k / 256; ib++) {
            const uint8_t *s = r + ib * 210;
            int32_t q[256], sc[16], mn[8]; float d, dmin;
            orc_unpack_k(s, T_Q6_K, q, sc, mn, &d, &dmin);
            float ssb = 0.0f;
            for (int b = 0; b < 16; b++) {
                int32_t isum = 0;
                const int8_t *xb = xq + ib * 256 + (size_t)b * 16;
                for (int i = 0; i < 16; i++) isum += q[b * 16 + i] * xb[i];
                float ds = d * (float)sc[b];
                float ab = dx[(ib * 256 + (size_t)b * 16) / 32] * (float)isum;
                ssb += ds * ab;
            }
            sumf += ssb;
        }
    }
    return sumf;
}

/* Q8-activation mm_batched: each activation row quantized, then the row
 * formulas above.  The whole-element formats (F32, F16, BF16) and the
 * multiply-free ternary ones (I2_S, Q1_0, Q2_0, STQ1_0) take no quantized
 * activations: their Q8 mode is the reference order.  Returns -1
 * for a dtype without a Q8 path. */
EXPORT int orc_mm_batched_q8(const float *a, size_t t_rows, const uint8_t *w, uint32_t t,
                             size_t n_rows, size_t n_cols, float *out, int threads) {
    uint32_t qk, bb;
    if (t == T_F32 || t == T_F16 || t == T_BF16 || t == T_I2_S || t == T_Q1_0 || t == T_Q2_0 || t == T_STQ1_0)
        return orc_mm_batched(a, t_rows, w, t, n_rows, n_cols, out, threads);
    if (t != T_Q8_0 && t != T_Q4_0 && t != T_Q5_0 && t != T_Q4_1 && t != T_Q3_K && t != T_Q4_K && t != T_Q5_K &&
        t != T_Q6_K)
        return -1;
    if (orc_block_geometry(t, &qk, &bb) || n_cols % qk) return -2;
    size_t row_bytes = n_cols / qk * bb;
    int8_t *xq = (int8_t *)malloc(n_cols);
    float *dx = (float *)malloc(n_cols / 32 * sizeof(float));
    if (threads < 1) threads = 1;
    for (size_t tr = 0; tr < t_rows; tr++) {
        orc_quantize_act_q8(a + tr * n_cols, n_cols, xq, dx, 0);
        float *ot = out + tr * n_rows;
#pragma omp parallel for schedule(dynamic, 16) num_threads(threads)
        for (size_t j = 0; j < n_rows; j++) ot[j] = row_q8_path(t, xq, dx, w + j * row_bytes, n_cols);
    }
    free(xq); free(dx);
    return 0;
}

/* Per-block integer dots of the Q8 path (for closed-form checks):
 * isum[j*nb + b] for Q8_0/Q4_0 blocks of 32. */
EXPORT int orc_block_isums(const int8_t *xq, const uint8_t *w, uint32_t t, size_t n_rows,
                           size_t n_cols, int32_t *isum) {
    if (t != T_Q8_0 && t != T_Q4_0) return -1;
    size_t nb = n_cols / 32, bb = t == T_Q8_0 ? 34 : 18;
    for (size_t j = 0; j < n_rows; j++)
        for (size_t ib = 0; ib < nb; ib++) {
            const uint8_t *s = w + (j * nb + ib) * bb;
            int32_t acc = 0;
            for (int q = 0; q < 32; q++) {
                int v = t == T_Q8_0 ? (int8_t)s[2 + q]
                                    : (q < 16 ? (s[2 + q] & 0x0F) - 8 : (s[2 + q - 16] >> 4) - 8);
                acc += v * xq[ib * 32 + q];
            }
            isum[j * nb + ib] = acc;
        }
    return 0;
}

/* ------------------------------------------------------------------ */
/* MoE (rce-op-moe, rce-qwen36-moe) and activations                    */
/* ------------------------------------------------------------------ */

/* rce-qwen36-moe/src/lib.rs L459-461 / rce-tinyllama L164-166 `silu`. */
EXPORT float orc_silu(float x) {
    if (x >= 0.0f) { float e = expf(-x); return x / (1.0f + e); }
    float e = expf(x);
    float t = x * e;
    return t / (1.0f + e);
}

/* rce-op-moe/src/lib.rs L35-73 `moe_router` from given logits (the
 * config supplies logits; the reference computes them with mm_1d first):
 * softmax over all experts (max-subtracted, f32 exp), sort descending,
 * keep top_k, optionally renormalize.  Ties keep the lower index first
 * (the reference's sort_unstable_by leaves tie order unspecified). */
EXPORT void orc_moe_router(const float *logits, size_t n_expert, size_t top_k, int normalize,
                           int32_t *idx_out, float *w_out) {
    float probs[1024];
    int idx[1024];
    float mx = -INFINITY;
    for (size_t e = 0; e < n_expert; e++) mx = fmaxf(mx, logits[e]);
    float sum = 0.0f;
    for (size_t e = 0; e < n_expert; e++) { probs[e] = expf(logits[e] - mx); }
    for (size_t e = 0; e < n_expert; e++) sum += probs[e];
    if (sum > 0.0f) for (size_t e = 0; e < n_expert; e++) probs[e] /= sum;
    for (size_t e = 0; e < n_expert; e++) idx[e] = (int)e;
    for (size_t i = 1; i < n_expert; i++) { /* stable insertion sort, descending */
        int v = idx[i]; size_t j = i;
        while (j > 0 && probs[idx[j - 1]] < probs[v]) { idx[j] = idx[j - 1]; j--; }
        idx[j] = v;
    }
    float s = 0.0f;
    for (size_t i = 0; i < top_k; i++) { idx_out[i] = idx[i]; w_out[i] = probs[idx[i]]; }
    if (normalize) {
        for (size_t i = 0; i < top_k; i++) s += w_out[i];
        if (s > 0.0f) for (size_t i = 0; i < top_k; i++) w_out[i] /= s;
    }
}

/* rce-op-moe/src/lib.rs L98-110 `moe_combine`: out = sum_j w_j * y_j in
 * decision order from +0.0.  ys is [top_k][d]. */
EXPORT void orc_moe_combine(const float *w, const float *ys, size_t top_k, size_t d, float *out) {
    for (size_t i = 0; i < d; i++) out[i] = 0.0f;
    for (size_t j = 0; j < top_k; j++)
        for (size_t i = 0; i < d; i++) { float t = w[j] * ys[j * d + i]; out[i] += t; }
}

/* The grouped-expert FFN of the MoE config, exact order: per token t and
 * decision j (rce-qwen36-moe L667-710 with the config's two matrices):
 * h = silu(mm_1d(x_t, w1[e])); y_j = mm_1d(h, w2[e]); out_t = moe_combine.
 * w1_bytes/w2_bytes: arrays of n_expert pointers to GGUF bytes. */
EXPORT float orc_silu_dev(float x);

/* how: 0 = the reference (mm_1d products, silu with the platform exp);
 * bit 0: silu with orc_exp_dev (the device's order, test instrumentation);
 * bit 1: the Q8-activation products (orc_mm_batched_q8) instead of mm_1d. */
EXPORT int orc_moe_ffn2(const float *x, size_t t_rows, size_t d_model, size_t d_ff,
                        const uint8_t *const *w1_bytes, const uint8_t *const *w2_bytes, uint32_t t, uint32_t t2,
                        const int32_t *ids, const float *gate_w, size_t top_k, float *out,
                        int threads, int how) {
    float *h = (float *)malloc(d_ff * sizeof(float));
    float *ys = (float *)malloc(top_k * d_model * sizeof(float));
    int rc = 0;
    const int q8 = (how & 2) != 0;
    for (size_t tr = 0; tr < t_rows && rc == 0; tr++) {
        for (size_t j = 0; j < top_k && rc == 0; j++) {
            int e = ids[tr * top_k + j];
            rc = q8 ? orc_mm_batched_q8(x + tr * d_model, 1, w1_bytes[e], t, d_ff, d_model, h, threads)
                    : orc_mm_1d(x + tr * d_model, w1_bytes[e], t, d_ff, d_model, h, threads);
            for (size_t i = 0; i < d_ff; i++) h[i] = (how & 1) ? orc_silu_dev(h[i]) : orc_silu(h[i]);
            if (!rc)
                rc = q8 ? orc_mm_batched_q8(h, 1, w2_bytes[e], t2, d_model, d_ff, ys + j * d_model, threads)
                        : orc_mm_1d(h, w2_bytes[e], t2, d_model, d_ff, ys + j * d_model, threads);
        }
        orc_moe_combine(gate_w + tr * top_k, ys, top_k, d_model, out + tr * d_model);
    }
    free(h); free(ys);
    return rc;
}

/* orc_moe_ffn2 with one dtype for both matrices. */
EXPORT int orc_moe_ffn(const float *x, size_t t_rows, size_t d_model, size_t d_ff,
                       const uint8_t *const *w1_bytes, const uint8_t *const *w2_bytes, uint32_t t,
                       const int32_t *ids, const float *gate_w, size_t top_k, float *out,
                       int threads, int how) {
    return orc_moe_ffn2(x, t_rows, d_model, d_ff, w1_bytes, w2_bytes, t, t, ids, gate_w, top_k, out, threads, how);
}

/* ------------------------------------------------------------------ */
/* Llama-2 decode step (rce-tinyllama, rce-op-attn)                     */
/* ------------------------------------------------------------------ */

/* rce-tinyllama/src/lib.rs L158-163 `rms_norm`: mean_sq = (sum of v*v,
 * one sequential fold from +0.0) / n; inv = 1 / sqrt(mean_sq + eps);
 * out = (v * inv) * w. */
EXPORT void orc_rms_norm(const float *x, const float *w, size_t n, float eps, float *out) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) { float t = x[i] * x[i]; ss += t; }
    float mean_sq = ss / (float)n;
    float inv = 1.0f / sqrtf(mean_sq + eps);
    for (size_t i = 0; i < n; i++) { float t = x[i] * inv; out[i] = t * w[i]; }
}

/* rce-op-attn/src/lib.rs L115-151 `rope_inplace_scaled` (no frequency
 * factors): log_base = ln(base); inv_freq_i = 1 / exp(log_base * (2i) /
 * rope_dim); theta = pos * inv_freq_i; pairs (x[i], x[i + half]) become
 * (a c - b s, a s + b c).  cos_sin (optional): the 2*half values
 * (c_0, s_0, c_1, s_1, ...) used, for checking a device table. */
EXPORT void orc_rope(float *x, size_t rope_dim, float base, size_t pos, float *cos_sin) {
    size_t half = rope_dim / 2;
    float log_base = logf(base);
    for (size_t i = 0; i < half; i++) {
        float e = log_base * (2.0f * (float)i);
        e = e / (float)rope_dim;
        float inv_freq = 1.0f / expf(e);
        float theta = (float)pos * inv_freq;
        float s = sinf(theta), c = cosf(theta);
        if (cos_sin) { cos_sin[2 * i] = c; cos_sin[2 * i + 1] = s; }
        float a = x[i], b = x[i + half];
        float ac = a * c, bs = b * s, as = a * s, bc = b * c;
        x[i] = ac - bs;
        x[i + half] = as + bc;
    }
}

/* rce-op-attn/src/lib.rs L185-251 `fused_attend_head_window` over
 * [0, seq_len): s_j = dot(q, k_j) * scale (dot = sequential sum of
 * products, L60-95 on x86); the first key sets out = 0 + 1 * v, l = 1,
 * m = s; every later key: m' = max(m, s), alpha = exp(m - m'),
 * beta = exp(s - m'), out = out * alpha + beta * v, l = l * alpha + beta;
 * finally out *= 1 / l. */
EXPORT void orc_attend_head(const float *q, const float *k_cache, const float *v_cache, size_t kv_head,
                            size_t seq_len, size_t kv_dim, size_t d_head, float scale, float *out) {
    size_t off = kv_head * d_head;
    float m = -INFINITY, l = 0.0f;
    for (size_t i = 0; i < d_head; i++) out[i] = 0.0f;
    for (size_t j = 0; j < seq_len; j++) {
        const float *k = k_cache + j * kv_dim + off, *v = v_cache + j * kv_dim + off;
        float dot = 0.0f;
        for (size_t i = 0; i < d_head; i++) { float t = q[i] * k[i]; dot += t; }
        float s = dot * scale;
        float m_new = fmaxf(m, s);
        if (isinf(m)) {
            for (size_t i = 0; i < d_head; i++) { float t = 1.0f * v[i]; out[i] += t; }
            l = 1.0f;
            m = s;
        } else {
            float alpha = expf(m - m_new), beta = expf(s - m_new);
            for (size_t i = 0; i < d_head; i++) out[i] *= alpha;
            for (size_t i = 0; i < d_head; i++) { float t = beta * v[i]; out[i] += t; }
            float la = l * alpha;
            l = la + beta;
            m = m_new;
        }
    }
    if (l != 0.0f) {
        float inv = 1.0f / l;
        for (size_t i = 0; i < d_head; i++) out[i] *= inv;
    }
}

/* ---- the GPU decode step's own orders (test instrumentation) -------------
 * Where the device's decode step documents an order of its own instead of
 * the reference's -- the sum of squares of rms_norm as a fixed tree, the
 * attention softmax as fixed-shape parallel reductions, exp as the
 * library's exp -- these functions restate that order, so the device can be
 * checked bit for bit against it (orc_llama_forward with dev_order).  The
 * reference-order functions above stay the parity definition against the
 * reference; these are judged by their own checks (tests/test_oracle_decoder.py:
 * orc_exp_dev's error bound over every float of its range, the trees and
 * the parallel attention against the reference order within rounding). */

/* exp as the device library computes it: x = n ln2 + r with n =
 * rint(x log2e) and r = (x - n ln2_hi) - n ln2_lo (Cody & Waite's split of
 * ln 2, W. J. Cody and W. Waite, Software Manual for the Elementary
 * Functions, 1980), exp(r) by its Taylor series to degree 7 in Horner form
 * with fused multiply-adds, then the two exact scalings by 2^(n/2) and
 * 2^(n - n/2).  0 below -104 (and for -inf), +inf above 88.75, NaN kept. */
EXPORT float orc_exp_dev(float x) {
    if (!(x > -104.0f)) return x != x ? x : 0.0f;
    if (x > 88.75f) return INFINITY;
    const float n = rintf(x * 0x1.715476p+0f);
    float r = fmaf(-n, 0x1.62e4p-1f, x);
    r = fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0x1p-1f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int ni = (int)n, e1 = ni / 2, e2 = ni - e1;
    union { uint32_t u; float f; } s1, s2;
    s1.u = (uint32_t)(e1 + 127) << 23;
    s2.u = (uint32_t)(e2 + 127) << 23;
    return (p * s1.f) * s2.f;
}

/* Largest error of orc_exp_dev in units in the last place of the correctly
 * rounded exp (exp in double, rounded to float) over every float whose bits
 * lie in [lo_bits, hi_bits] (as unsigned; one sign), and the input where it
 * occurs.  Results that are 0 or infinite on either side count as exact
 * when both agree. */
EXPORT double orc_exp_dev_max_ulp(uint32_t lo_bits, uint32_t hi_bits, uint32_t *worst_bits, int threads) {
    double worst = 0.0;
    uint32_t wb = lo_bits;
#ifdef _OPENMP
#pragma omp parallel num_threads(threads > 0 ? threads : omp_get_max_threads())
#endif
    {
        double lw = 0.0;
        uint32_t lb = lo_bits;
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t b = (int64_t)lo_bits; b <= (int64_t)hi_bits; b++) {
            union { uint32_t u; float f; } v;
            v.u = (uint32_t)b;
            const float got = orc_exp_dev(v.f);
            const float want = (float)exp((double)v.f);
            if (got == want) continue;
            double ulp;
            if (want == 0.0f || isinf(want) || isinf(got)) {
                ulp = 1e30;  /* one side 0 or infinite, the other not */
                if (want == 0.0f && !isinf(got)) ulp = (double)got / 0x1p-149;  /* subnormal steps */
            } else {
                int e;
                frexpf(want, &e);
                double u = ldexp(1.0, (e - 24 < -149 ? -149 : e - 24));
                ulp = fabs((double)got - (double)want) / u;
            }
            if (ulp > lw) { lw = ulp; lb = v.u; }
        }
#ifdef _OPENMP
#pragma omp critical
#endif
        {
            if (lw > worst) { worst = lw; wb = lb; }
        }
    }
    if (worst_bits) *worst_bits = wb;
    return worst;
}

/* silu (rce-tinyllama L164-166) with orc_exp_dev in place of exp. */
EXPORT float orc_silu_dev(float x) {
    if (x >= 0.0f) { float e = orc_exp_dev(-x); return x / (1.0f + e); }
    float e = orc_exp_dev(x);
    float t = x * e;
    return t / (1.0f + e);
}

/* The wave-wide sum of the device: the balanced pairwise tree over lane
 * order, as a butterfly in which lane i adds lane i ^ off for off = 1, 2,
 * 4, ..., 32 (adjacent lanes first; every lane ends with the same value). */
static float dev_wave_sum(float v[64]) {
    for (int off = 1; off <= 32; off <<= 1) {
        float t[64];
        for (int i = 0; i < 64; i++) t[i] = v[i] + v[i ^ off];
        memcpy(v, t, sizeof t);
    }
    return v[0];
}

/* rms_norm with the device's sum of squares.  nt > 0: the form fused into
 * the GEMV kernels -- thread t of nt holds tasks t and t + nt of 8
 * consecutive values (a sequential sum of squares each; a task past the end
 * adds 0), then the butterfly per wave of 64 threads, then the waves' sums
 * in wave order from 0.  nt < 0: the separate kernel of -nt threads --
 * thread t sums the squares of x[t], x[t - nt], ... in order, then the
 * same butterfly and wave order.  The rest is the reference's: mean_sq =
 * sum / n, inv = 1 / sqrt(mean_sq + eps), out = (x * inv) * w. */
EXPORT void orc_rms_norm_dev(const float *x, const float *w, size_t n, float eps, int nt, float *out) {
    const int threads = nt > 0 ? nt : -nt;
    float *ss = (float *)calloc((size_t)threads, sizeof(float));
    for (int t = 0; t < threads; t++) {
        float s = 0.0f;
        if (nt > 0) {
            for (int h = 0; h < 2; h++) {
                const size_t task = (size_t)t + (size_t)h * (size_t)threads;
                float q = 0.0f;
                if (task < n / 8)
                    for (int i = 0; i < 8; i++) { float sq = x[8 * task + i] * x[8 * task + i]; q = q + sq; }
                s = h == 0 ? q : s + q;
            }
        } else {
            for (size_t i = (size_t)t; i < n; i += (size_t)threads) { float sq = x[i] * x[i]; s = s + sq; }
        }
        ss[t] = s;
    }
    float tot = 0.0f;
    for (int wv = 0; wv < threads / 64; wv++) tot = tot + dev_wave_sum(ss + 64 * wv);
    free(ss);
    float mean_sq = tot / (float)n;
    float inv = 1.0f / sqrtf(mean_sq + eps);
    for (size_t i = 0; i < n; i++) { float t = x[i] * inv; out[i] = t * w[i]; }
}

/* One query head's attention as the device evaluates it (seq_len keys of
 * the caches, this position's row included): the keys form runs of ch =
 * 4096 / d_head from key 0, and wave w of four takes the runs w, w + 4,
 * w + 8, ... in that order; in a run, key j's
 * score is the sequential dot q . k_j times scale, m_new = max(m, the
 * run's scores), p_j = exp(s_j - m_new), l = l exp(m - m_new) + (butterfly
 * sum of the p_j over 64 lanes), and per dimension four partial sums a_k
 * over the run's keys j = k mod 4 in order, o = o exp(m - m_new) + ((a_0 +
 * a_1) + (a_2 + a_3)); then the waves with keys merge in wave order with
 * weights exp(m_w - M), M the largest m_w, and out = acc * (1 / l). */
EXPORT void orc_attend_head_dev(const float *q, const float *k_cache, const float *v_cache, size_t kv_head,
                                size_t seq_len, size_t kv_dim, size_t d_head, float scale, float *out) {
    enum { NW = 4 };
    const size_t off = kv_head * d_head, ch = 4096 / d_head;
    float wm[NW], wl[NW];
    float *wo = (float *)calloc(NW * d_head, sizeof(float));
    float *a = (float *)calloc(4 * d_head, sizeof(float));
    for (int wv = 0; wv < NW; wv++) {
        float m = -INFINITY, l = 0.0f;
        float *o = wo + wv * d_head;
        for (size_t c0 = (size_t)wv * ch; c0 < seq_len; c0 += NW * ch) {
            const size_t n = seq_len - c0 < ch ? seq_len - c0 : ch;
            float sc[64], p[64];
            float mx = -INFINITY;
            for (size_t j = 0; j < 64; j++) {
                sc[j] = -INFINITY;
                if (j < n) {
                    const float *k = k_cache + (c0 + j) * kv_dim + off;
                    float dot = 0.0f;
                    for (size_t i = 0; i < d_head; i++) { float t = q[i] * k[i]; dot = dot + t; }
                    sc[j] = dot * scale;
                }
                mx = fmaxf(mx, sc[j]);
            }
            const float m_new = fmaxf(m, mx);
            const float corr = orc_exp_dev(m - m_new);
            for (size_t j = 0; j < 64; j++) p[j] = j < n ? orc_exp_dev(sc[j] - m_new) : 0.0f;
            const float lc = l * corr;
            float pp[64];
            memcpy(pp, p, sizeof pp);
            l = lc + dev_wave_sum(pp);
            memset(a, 0, 4 * d_head * sizeof(float));
            for (size_t j = 0; j < n; j++) {
                const float *v = v_cache + (c0 + j) * kv_dim + off;
                float *ak = a + (j % 4) * d_head;
                for (size_t d = 0; d < d_head; d++) { float t = p[j] * v[d]; ak[d] = ak[d] + t; }
            }
            for (size_t d = 0; d < d_head; d++) {
                const float s01 = a[d] + a[d_head + d], s23 = a[2 * d_head + d] + a[3 * d_head + d];
                const float sv = s01 + s23, oc = o[d] * corr;
                o[d] = oc + sv;
            }
            m = m_new;
        }
        wm[wv] = m;
        wl[wv] = l;
    }
    float M = -INFINITY;
    for (int wv = 0; wv < NW; wv++) M = fmaxf(M, wm[wv]);
    float lacc = 0.0f;
    for (size_t d = 0; d < d_head; d++) out[d] = 0.0f;
    for (int wv = 0; wv < NW; wv++) {
        if (wm[wv] == -INFINITY) continue;
        const float wt = orc_exp_dev(wm[wv] - M);
        for (size_t d = 0; d < d_head; d++) { float t = wt * wo[wv * d_head + d]; out[d] = out[d] + t; }
        const float lw = wt * wl[wv];
        lacc = lacc + lw;
    }
    const float inv = 1.0f / lacc;
    for (size_t d = 0; d < d_head; d++) out[d] = out[d] * inv;
    free(wo);
    free(a);
}

/* One linear of the decoder: mm_1d (q8 = 0) or the Q8-activation path. */
static int dec_linear(const float *a, const uint8_t *w, uint32_t t, size_t n, size_t k, float *out, int q8,
                      int threads) {
    return q8 ? orc_mm_batched_q8(a, 1, w, t, n, k, out, threads) : orc_mm_1d(a, w, t, n, k, out, threads);
}

/* rce-tinyllama/src/lib.rs L303-330 `forward_embedding` with `attn_block`
 * (L252-287): one decode step at position `pos` from the input embedding.
 * dims: d_model, vocab, n_layers, n_q_heads, n_kv_heads, d_head,
 * rope_dim, d_ff, context_length.  lin: n_layers * 7 weights (GGUF bytes)
 * in the order wq, wk, wv, wo, ffn_gate, ffn_up, ffn_down, with their
 * dtypes in lin_dtype.  attn_norm / ffn_norm: [n_layers][d_model].
 * k_cache / v_cache: [n_layers][context_length][n_kv_heads * d_head]; the
 * step appends position pos.  logits: [vocab].  dev_order (may be NULL:
 * the reference's order): {nt_layers, nt_head}, the device's orders --
 * orc_rms_norm_dev with nt_layers for the layers' norms and nt_head for
 * the output norm, orc_attend_head_dev, orc_silu_dev.  x_trace (may be NULL):
 * [n_layers + 1][d_model], the residual stream entering each layer and,
 * last, leaving the final one (test instrumentation: it changes nothing
 * else).  Returns 0, or the failing linear's code, or -10 when pos >=
 * context_length. */
EXPORT int orc_llama_forward(const size_t *dims, float rope_base, float eps, int q8, const float *embedding,
                             const float *attn_norm, const float *ffn_norm, const uint8_t *const *lin,
                             const uint32_t *lin_dtype, const float *output_norm, const uint8_t *lm_head,
                             uint32_t lm_dtype, float *k_cache, float *v_cache, size_t pos, float *logits,
                             int threads, float *x_trace, const int *dev_order) {
    size_t dm = dims[0], vocab = dims[1], nl = dims[2], nq = dims[3], nkv = dims[4], dh = dims[5];
    size_t rope_dim = dims[6], dff = dims[7], ctx = dims[8];
    if (pos >= ctx) return -10;
    size_t qd = nq * dh, kvd = nkv * dh, qpk = nq / nkv;
    size_t big = dff > qd ? dff : qd;
    float *x = malloc(dm * 4), *xn = malloc(dm * 4), *q = malloc(qd * 4), *kk = malloc(kvd * 4);
    float *vv = malloc(kvd * 4), *att = malloc(qd * 4), *o = malloc(dm * 4);
    float *g = malloc(big * 4), *u = malloc(big * 4), *h = malloc(big * 4);
    int rc = 0;
    memcpy(x, embedding, dm * 4);
    float scale = 1.0f / sqrtf((float)dh);
    for (size_t il = 0; il < nl && rc == 0; il++) {
        const uint8_t *const *W = lin + il * 7;
        const uint32_t *T = lin_dtype + il * 7;
        float *kc = k_cache + il * ctx * kvd, *vc = v_cache + il * ctx * kvd;
        if (x_trace) memcpy(x_trace + il * dm, x, dm * 4);
        if (dev_order) orc_rms_norm_dev(x, attn_norm + il * dm, dm, eps, dev_order[0], xn);
        else orc_rms_norm(x, attn_norm + il * dm, dm, eps, xn);
        rc = dec_linear(xn, W[0], T[0], qd, dm, q, q8, threads);
        if (!rc) rc = dec_linear(xn, W[1], T[1], kvd, dm, kk, q8, threads);
        if (!rc) rc = dec_linear(xn, W[2], T[2], kvd, dm, vv, q8, threads);
        if (rc) break;
        for (size_t hh = 0; hh < nq; hh++) orc_rope(q + hh * dh, rope_dim, rope_base, pos, 0);
        for (size_t hh = 0; hh < nkv; hh++) orc_rope(kk + hh * dh, rope_dim, rope_base, pos, 0);
        memcpy(kc + pos * kvd, kk, kvd * 4);
        memcpy(vc + pos * kvd, vv, kvd * 4);
        for (size_t hh = 0; hh < nq; hh++) {
            if (dev_order) orc_attend_head_dev(q + hh * dh, kc, vc, hh / qpk, pos + 1, kvd, dh, scale, att + hh * dh);
            else orc_attend_head(q + hh * dh, kc, vc, hh / qpk, pos + 1, kvd, dh, scale, att + hh * dh);
        }
        rc = dec_linear(att, W[3], T[3], dm, qd, o, q8, threads);
        if (rc) break;
        for (size_t i = 0; i < dm; i++) x[i] += o[i];
        if (dev_order) orc_rms_norm_dev(x, ffn_norm + il * dm, dm, eps, dev_order[0], xn);
        else orc_rms_norm(x, ffn_norm + il * dm, dm, eps, xn);
        rc = dec_linear(xn, W[4], T[4], dff, dm, g, q8, threads);
        if (!rc) rc = dec_linear(xn, W[5], T[5], dff, dm, u, q8, threads);
        if (rc) break;
        for (size_t i = 0; i < dff; i++) h[i] = (dev_order ? orc_silu_dev(g[i]) : orc_silu(g[i])) * u[i];
        rc = dec_linear(h, W[6], T[6], dm, dff, o, q8, threads);
        if (rc) break;
        for (size_t i = 0; i < dm; i++) x[i] += o[i];
    }
    if (!rc) {
        if (x_trace) memcpy(x_trace + nl * dm, x, dm * 4);
        if (dev_order) orc_rms_norm_dev(x, output_norm, dm, eps, dev_order[1], xn);
        else orc_rms_norm(x, output_norm, dm, eps, xn);
        rc = dec_linear(xn, lm_head, lm_dtype, vocab, dm, logits, q8, threads);
    }
    free(x); free(xn); free(q); free(kk); free(vv); free(att); free(o); free(g); free(u); free(h);
    return rc;
}

/* rce-qwen36-moe/src/lib.rs L667-703, the routed part of moe_ffn_forward:
 * per token t and decision j, e = ids[t*top_k + j]: g = mm_1d(x_t, gate[e]),
 * u = mm_1d(x_t, up[e]), h[i] = silu(g[i]) * u[i] (swiglu_expert_serial),
 * y_j = mm_1d(h, down[e]); out_t = sum_j w_j * y_j from +0.0 in decision
 * order (L698-703, = moe_combine). */
EXPORT int orc_moe_swiglu_ffn(const float *x, size_t t_rows, size_t d_model, size_t d_ff,
                              const uint8_t *const *gate, const uint8_t *const *up, const uint8_t *const *down,
                              uint32_t t, const int32_t *ids, const float *gate_w, size_t top_k, float *out,
                              int threads) {
    float *g = (float *)malloc(d_ff * sizeof(float)), *u = (float *)malloc(d_ff * sizeof(float));
    float *ys = (float *)malloc(top_k * d_model * sizeof(float));
    int rc = 0;
    for (size_t tr = 0; tr < t_rows && rc == 0; tr++) {
        for (size_t j = 0; j < top_k && rc == 0; j++) {
            int e = ids[tr * top_k + j];
            rc = orc_mm_1d(x + tr * d_model, gate[e], t, d_ff, d_model, g, threads);
            if (!rc) rc = orc_mm_1d(x + tr * d_model, up[e], t, d_ff, d_model, u, threads);
            for (size_t i = 0; i < d_ff; i++) g[i] = orc_silu(g[i]) * u[i];
            if (!rc) rc = orc_mm_1d(g, down[e], t, d_model, d_ff, ys + j * d_model, threads);
        }
        orc_moe_combine(gate_w + tr * top_k, ys, top_k, d_model, out + tr * d_model);
    }
    free(g); free(u); free(ys);
    return rc;
}

EXPORT int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
