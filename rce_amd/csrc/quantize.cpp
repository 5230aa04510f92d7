// quantize.cpp -- GGUF block quantizers on the host (rce_qmm_quantize):
// the reference's encoders that produce Q8_0 / Q4_0 / Q4_K / Q6_K bytes from
// f32 weights, so a caller can build device weights without another tool.
//
//   Q8_0, Q4_0: quantize_block (rce-vm-backend-cpu/src/ml/nn.rs L541-563),
//     packed as spec/checker/tests/support/toy_gpt2.rs L46-58 does: f16
//     scale, then int8 values (Q8_0) or nibbles (lo = q[t] + 8, hi =
//     q[t + 16] + 8) (Q4_0).
//   Q4_K, Q5_K, Q6_K: quantize_k (rce-vm-backend-cpu/src/ml/kquant.rs L193-245)
//     and pack (L284-346).
// Scales are rounded with round_to_f16 (nn.rs L521-533): IEEE binary16
// round-to-nearest-even, overflow to infinity -- exactly the compiler's
// float -> _Float16 conversion -- and written with the reference's
// f16_bits (kquant.rs L267-281), which equals IEEE's encoding on every
// finite binary16 value.  Every + - * / is one binary32 rounding (built
// with -ffp-contract=off).  Blocks are independent, so the work is split
// over host threads by row ranges with no effect on the bytes.
//
// Non-finite inputs get the reference's bytes too: float -> int is Rust's
// saturating `as i32` (NaN -> 0), integer adds wrap as in a release build,
// narrowing keeps the low bits (`as u8`, `as i8`), and f16_bits of an
// infinity or NaN keeps its exponent's low bits (0x3C00 for +inf).  Such
// blocks arise from infinite or NaN weights and from blocks whose largest
// magnitude is so small that 1/d overflows to infinity.
#include "abi_internal.h"

#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>

using namespace rce_qmm_abi;

namespace {

// f16_bits (kquant.rs L267-281, spec/checker/tests/support/toy_gpt2.rs
// L30-42): the binary16 bits of x, a binary16 value (round_f16 made it one).
inline uint16_t f16_of(float x) {
    uint32_t b;
    std::memcpy(&b, &x, 4);
    const uint32_t s = (b >> 16) & 0x8000u, ab = b & 0x7FFFFFFFu;
    const float a = std::fabs(x);
    if (a == 0.0f) return (uint16_t)s;
    if (a < 0x1p-14f) return (uint16_t)(s | (uint32_t)(a / 0x1p-24f));  // subnormal: an exact integer
    const uint32_t e = (ab >> 23) - 127 + 15;  // 143 for an infinity or NaN: only its low bits stay
    return (uint16_t)(s | (e << 10) | ((ab >> 13) & 0x3FFu));
}
inline float round_f16(float x) { return (float)(_Float16)x; }
inline void put16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xFF);
    p[1] = (uint8_t)(v >> 8);
}
// Rust's `f as i32`: NaN -> 0, out of range -> the nearest bound (a C cast
// of those is undefined).
inline int32_t as_i32(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x <= -2147483648.0f) return INT32_MIN;
    return (int32_t)x;
}
inline int round_i(float x) { return as_i32(std::round(x)); }  // f32::round (half away from zero) as i32
inline int clamp_i(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// One block of 32 -> 34 bytes (Q8_0) or 18 bytes (Q4_0).
void encode_q32(const float *x, bool q4, uint8_t *out) {
    float amax = 0.0f, signed_max = 0.0f;  // first value of largest magnitude
    for (int i = 0; i < 32; i++) {
        const float a = std::fabs(x[i]);
        if (amax < a) {
            amax = a;
            signed_max = x[i];
        }
    }
    const float d = q4 ? signed_max / -8.0f : amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(out, f16_of(round_f16(d)));
    if (q4) {
        // the reference's q = min(15, floor(t)) - 8 is stored as (q + 8) as
        // u8, the adds wrapping: that is min(15, floor(t)) as u8
        uint8_t q[32];
        for (int i = 0; i < 32; i++) {
            float t = x[i] * id;
            t = t + 8.5f;
            const int32_t v = as_i32(std::floor(t));
            q[i] = (uint8_t)(v < 15 ? v : 15);
        }
        for (int t = 0; t < 16; t++) out[2 + t] = (uint8_t)(q[t] | (uint8_t)(q[t + 16] << 4));
    } else {
        for (int i = 0; i < 32; i++) {
            const float t = x[i] * id;
            out[2 + i] = (uint8_t)(int8_t)round_i(t);
        }
    }
}

// One super-block of 256 -> 144 bytes (Q4_K).
// Q4_K (nmax 15) and Q5_K (nmax 31, plus the qh plane of 5th bits).
void encode_q45_k(const float *x, uint8_t *out, bool q5) {
    const float nmax = q5 ? 31.0f : 15.0f;
    float w[8], v[8];
    for (int b = 0; b < 8; b++) {
        float lo = 0.0f, hi = -INFINITY;
        for (int i = 0; i < 32; i++) {
            const float t = x[32 * b + i];
            if (t < lo) lo = t;
            if (t > hi) hi = t;
        }
        const float span = hi - lo;
        w[b] = span / nmax;
        v[b] = -lo;
    }
    float bw = 0.0f, bv = 0.0f;
    for (int b = 0; b < 8; b++) {
        if (w[b] > bw) bw = w[b];
        if (v[b] > bv) bv = v[b];
    }
    const float d = round_f16(bw / 63.0f), dmin = round_f16(bv / 63.0f);
    int sc[8], mn[8];
    for (int b = 0; b < 8; b++) {
        sc[b] = d != 0.0f ? std::min(round_i(w[b] / d), 63) : 0;
        mn[b] = dmin != 0.0f ? std::min(round_i(v[b] / dmin), 63) : 0;
    }
    put16(out, f16_of(d));
    put16(out + 2, f16_of(dmin));
    uint8_t *s = out + 4;  // 6-bit scale / min packing (kquant.rs L284-292)
    for (int j = 0; j < 4; j++) {  // each value `as u8` first
        const uint8_t sj = (uint8_t)sc[j], sj4 = (uint8_t)sc[j + 4], mj = (uint8_t)mn[j], mj4 = (uint8_t)mn[j + 4];
        s[j] = (uint8_t)((sj & 63) | ((sj4 >> 4) << 6));
        s[j + 4] = (uint8_t)((mj & 63) | ((mj4 >> 4) << 6));
        s[j + 8] = (uint8_t)((sj4 & 15) | ((mj4 & 15) << 4));
    }
    int q[256];
    for (int p = 0; p < 256; p++) {
        const float sb = d * (float)sc[p / 32], ob = dmin * (float)mn[p / 32];
        const float num = x[p] + ob;
        q[p] = sb != 0.0f ? clamp_i(round_i(num / sb), 0, (int)nmax) : 0;
    }
    uint8_t *qs = out + 16;
    if (q5) {  // qh[l] bit 2g: position 64g + l, bit 2g+1: 64g + 32 + l (kquant.rs L310-318)
        uint8_t *qh = out + 16;
        for (int l = 0; l < 32; l++) qh[l] = 0;
        for (int g = 0; g < 4; g++)
            for (int l = 0; l < 32; l++) {
                qh[l] = (uint8_t)(qh[l] | (((q[64 * g + l] >> 4) & 1) << (2 * g)));
                qh[l] = (uint8_t)(qh[l] | (((q[64 * g + 32 + l] >> 4) & 1) << (2 * g + 1)));
            }
        qs = out + 48;
    }
    for (int g = 0; g < 4; g++)
        for (int l = 0; l < 32; l++)
            qs[32 * g + l] = (uint8_t)((q[64 * g + l] & 15) | ((q[64 * g + 32 + l] & 15) << 4));
}

// One super-block of 256 -> 210 bytes (Q6_K).
void encode_q6_k(const float *x, uint8_t *out) {
    float w[16];
    for (int b = 0; b < 16; b++) {
        float amax = 0.0f, m = 0.0f;
        for (int i = 0; i < 16; i++) {
            const float t = x[16 * b + i];
            if (amax < std::fabs(t)) {
                amax = std::fabs(t);
                m = t;
            }
        }
        w[b] = m / -32.0f;
    }
    float wmax = 0.0f;
    for (int b = 0; b < 16; b++)
        if (wmax < std::fabs(w[b])) wmax = std::fabs(w[b]);
    const float d = round_f16(wmax / 127.0f);
    int sc[16], q[256];
    for (int b = 0; b < 16; b++) sc[b] = d != 0.0f ? clamp_i(round_i(w[b] / d), -128, 127) : 0;
    for (int p = 0; p < 256; p++) {
        const float sb = d * (float)sc[p / 16];
        q[p] = sb != 0.0f ? clamp_i(round_i(x[p] / sb), -32, 31) : 0;
    }
    uint8_t *ql = out, *qh = out + 128;
    for (int h = 0; h < 2; h++)
        for (int l = 0; l < 32; l++) {
            const int q1 = q[128 * h + l] + 32, q2 = q[128 * h + l + 32] + 32;
            const int q3 = q[128 * h + l + 64] + 32, q4 = q[128 * h + l + 96] + 32;
            ql[64 * h + l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
            ql[64 * h + l + 32] = (uint8_t)((q2 & 15) | ((q4 & 15) << 4));
            qh[32 * h + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    for (int b = 0; b < 16; b++) out[192 + b] = (uint8_t)(int8_t)sc[b];
    put16(out + 208, f16_of(d));
}

}  // namespace

extern "C" rce_qmm_status rce_qmm_quantize(uint32_t dtype, const float *src, size_t n_rows, size_t n_cols,
                                           uint8_t *dst, size_t len) {
    if ((!src || !dst) && n_rows * n_cols) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    size_t qk, bb;
    switch (dtype) {
    case T_Q8_0: qk = 32; bb = 34; break;
    case T_Q4_0: qk = 32; bb = 18; break;
    case T_Q4_K: qk = 256; bb = 144; break;
    case T_Q5_K: qk = 256; bb = 176; break;
    case T_Q6_K: qk = 256; bb = 210; break;
    default: return fail(RCE_QMM_UNSUPPORTED_DTYPE, "no quantizer for dtype " + std::to_string(dtype));
    }
    if (n_cols % qk) return fail(RCE_QMM_BAD_SHAPE, "n_cols is not a multiple of the block size");
    const size_t nb = n_cols / qk;
    if (len != n_rows * nb * bb) return fail(RCE_QMM_BAD_SHAPE, "len != n_rows * row_bytes");
    auto rows = [&](size_t r0, size_t r1) {
        for (size_t r = r0; r < r1; r++)
            for (size_t b = 0; b < nb; b++) {
                const float *x = src + r * n_cols + b * qk;
                uint8_t *o = dst + (r * nb + b) * bb;
                switch (dtype) {
                case T_Q8_0: encode_q32(x, false, o); break;
                case T_Q4_0: encode_q32(x, true, o); break;
                case T_Q4_K: encode_q45_k(x, o, false); break;
                case T_Q5_K: encode_q45_k(x, o, true); break;
                default: encode_q6_k(x, o); break;
                }
            }
    };
    const size_t work = n_rows * n_cols;
    unsigned nt = std::thread::hardware_concurrency();
    nt = nt == 0 ? 1 : std::min(nt, 16u);  // one GPU's share of host cores
    if (work < (1u << 20) || n_rows < 2 * (size_t)nt) nt = 1;
    if (nt == 1) {
        rows(0, n_rows);
        return RCE_QMM_OK;
    }
    std::vector<std::thread> pool;
    const size_t per = (n_rows + nt - 1) / nt;
    try {
        for (unsigned t = 0; t < nt; t++) {
            const size_t r0 = t * per, r1 = std::min(n_rows, r0 + per);
            if (r0 < r1) pool.emplace_back(rows, r0, r1);
        }
    } catch (...) {
        for (auto &th : pool) th.join();
        return fail(RCE_QMM_INTERNAL, "could not start quantizer threads");
    }
    for (auto &th : pool) th.join();
    return RCE_QMM_OK;
}
