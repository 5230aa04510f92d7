// qmm_gemv.hip -- host side of the decode kernels: which shapes the GPU
// computes, the device layouts of the weights, the launch-shape choice and
// the dispatch to the per-format kernels (gemv_<format>.hip), plus the
// f16 widening and row dequantization kernels.
#include "qmm_gemv_kernels.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>

namespace rce_qmm {
namespace {

// ---------------------------------------------------------------------------
// f16 widening, row dequantization.
// ---------------------------------------------------------------------------

__global__ void k_f16_to_f32(const uint16_t *__restrict__ s, float *__restrict__ d, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) d[i] = h2f(s[i]);
}

// dequant.rs L360-382 (Q4_0), L385-433 (Q4_1, Q5_0), L438-454 (Q8_0),
// L468-543 (Q3_K), L546-589 (Q4_K), L606-655 (Q5_K), L658-701 (Q6_K): value
// i of row `row`.
__device__ float dequant_value(const DevWeight &w, size_t row, size_t i) {
    float v = 0.0f;
    if (w.dtype == T_Q4_0 || w.dtype == T_Q8_0) {
        const uint8_t *rp = w.base + row * w.row_stride;
        const size_t b = i / 32;
        const int p = (int)(i % 32);
        const float scale = h2f(*reinterpret_cast<const uint16_t *>(rp + 2 * b));
        if (w.dtype == T_Q4_0) {
            const uint8_t byte = rp[w.plane1 + 16 * b + (p & 15)];
            const int n = p < 16 ? (byte & 0x0F) - 8 : ((byte >> 4) & 0x0F) - 8;
            v = (float)n * scale;
        } else {
            const uint8_t byte = p < 16 ? rp[w.plane1 + 16 * b + p] : rp[w.plane2 + 16 * b + p - 16];
            v = (float)(int8_t)byte * scale;
        }
    } else if (w.dtype == T_Q5_0 || w.dtype == T_Q4_1) {  // dequant.rs L385-433
        const uint8_t *rp = w.base + row * w.row_stride;
        const size_t b = i / 32;
        const int p = (int)(i % 32);
        const uint8_t byte = rp[w.plane1 + 16 * b + (p & 15)];
        const int nib = p < 16 ? (byte & 0x0F) : (byte >> 4);
        if (w.dtype == T_Q5_0) {
            const float scale = h2f(*reinterpret_cast<const uint16_t *>(rp + 2 * b));
            const uint32_t qh = *reinterpret_cast<const uint32_t *>(rp + w.plane2 + 4 * b);
            v = (float)((nib | (int)(((qh >> p) & 1u) << 4)) - 16) * scale;
        } else {
            const uint32_t sm = *reinterpret_cast<const uint32_t *>(rp + 4 * b);
            const float t = (float)nib * h2f(sm & 0xFFFFu);
            v = t + h2f(sm >> 16);
        }
    } else if (w.dtype == T_Q1_0) {  // dequant.rs L272-299: bit set -> +d, else -d
        const uint8_t *rp = w.base + row * w.row_stride;
        const size_t b = i / 128;
        const int j = (int)(i % 128);
        const float d = h2f(*reinterpret_cast<const uint16_t *>(rp + 2 * b));
        v = ((rp[w.plane1 + 16 * b + j / 8] >> (j % 8)) & 1) ? d : -d;
    } else if (w.dtype == T_Q2_0) {  // dequant.rs L317-340: (q - 1) * d
        const uint8_t *rp = w.base + row * w.row_stride;
        const size_t b = i / 128;
        const int j = (int)(i % 128), byte = j / 4;
        const float d = h2f(*reinterpret_cast<const uint16_t *>(rp + 2 * b));
        const uint8_t x = byte < 16 ? rp[w.plane1 + 16 * b + byte] : rp[w.plane2 + 16 * b + byte - 16];
        v = (float)((int)((x >> (2 * (j % 4))) & 3) - 1) * d;
    } else if (w.dtype == T_STQ1_0) {  // dequant.rs L162-196, codes expanded at upload
        const uint8_t *rp = w.base + row * w.row_stride;
        const size_t b = i / 256;
        const int p = (int)(i % 256);
        const float d = h2f(*reinterpret_cast<const uint16_t *>(rp + 2 * b));
        v = (float)((int)((rp[w.plane1 + 64 * b + p / 4] >> (2 * (p % 4))) & 3) - 1) * d;
    } else if (w.dtype == T_I2_S) {  // dequant.rs L222-256: scale * map2bit[code]
        const size_t blk = i / 128;
        const int within = (int)(i % 128), slot = within / 32, gp = within % 32;
        const size_t j = 128 * blk + 4 * (size_t)gp + (size_t)slot;  // chain order
        const uint8_t *cp = w.base + (row >> 6) * w.group_stride + (j / 64) * 1024 + (row & 63) * 8 + (j % 64) / 8;
        const int bit = (int)(j % 8);
        const bool plus = (cp[0] >> bit) & 1, minus = (cp[512] >> bit) & 1;
        const float m = minus ? -1.0f : (plus ? 1.0f : 0.0f);
        v = *reinterpret_cast<const float *>(w.aux) * m;
    } else if (is_whole_element(w.dtype)) {  // dequant.rs L343-356: the value itself
        const size_t es = w.dtype == T_F32 ? 4 : 2, o = i * es;
        const uint8_t *p = w.base + (row >> 6) * w.group_stride + ((o / 16) * 64 + (row & 63)) * 16 + o % 16;
        if (w.dtype == T_F32) v = *reinterpret_cast<const float *>(p);
        else if (w.dtype == T_F16) v = h2f(*reinterpret_cast<const uint16_t *>(p));
        else v = __uint_as_float((uint32_t)*reinterpret_cast<const uint16_t *>(p) << 16);
    } else if (w.dtype == T_Q3_K) {  // dl * (float)q with q = low - (high ? 0 : 4)
        const uint8_t *rp = w.base + row * w.row_stride;
        const size_t u = i / 32;
        const int p = (int)(i % 32), h = p / 16, q = p % 16;
        const uint32_t lw = *reinterpret_cast<const uint32_t *>(rp + w.plane1 + 8 * u + 4 * h);
        const uint32_t hw = *reinterpret_cast<const uint32_t *>(rp + w.plane2 + 4 * u);
        const int8_t sc = *reinterpret_cast<const int8_t *>(rp + w.plane3 + 2 * u + h);
        const float d = h2f(*reinterpret_cast<const uint16_t *>(rp + 2 * (u / 8)));
        const int low = (int)((lw >> (8 * (q % 4) + 2 * (q / 4))) & 3u), high = (int)((hw >> p) & 1u);
        const float dl = d * (float)sc;
        v = dl * (float)(low - (high ? 0 : 4));
    } else if (w.dtype == T_Q4_K) {
        const uint8_t *rp = w.base + row * w.row_stride;
        const size_t sb = i / 256;
        const int p = (int)(i % 256), g = p / 64, l = p % 32, hi = (p % 64) >= 32;
        const uint4 h = *reinterpret_cast<const uint4 *>(rp + 16 * sb);
        int sc, m;
        k4_scale_min(h, 2 * g + hi, sc, m);
        const float d = h2f(h.x & 0xFFFFu), dmin = h2f(h.x >> 16);
        const float dd = d * (float)sc, mm = dmin * (float)m;
        const size_t u = 4 * sb + g;
        const uint8_t byte = l < 16 ? rp[w.plane1 + 16 * u + l] : rp[w.plane2 + 16 * u + l - 16];
        const int n = hi ? ((byte >> 4) & 0x0F) : (byte & 0x0F);
        v = dd * (float)n - mm;
    } else if (w.dtype == T_Q5_K) {  // dequant.rs L606-655
        const uint8_t *rp = w.base + row * w.row_stride;
        const size_t sb = i / 256;
        const int p = (int)(i % 256), g = p / 64, l = p % 32, hi = (p % 64) >= 32;
        const uint4 h = *reinterpret_cast<const uint4 *>(rp + 16 * sb);
        int sc, m;
        k4_scale_min(h, 2 * g + hi, sc, m);
        const float d = h2f(h.x & 0xFFFFu), dmin = h2f(h.x >> 16);
        const float dd = d * (float)sc, mm = dmin * (float)m;
        const size_t u = 4 * sb + g;
        const uint8_t byte = l < 16 ? rp[w.plane1 + 16 * u + l] : rp[w.plane2 + 16 * u + l - 16];
        const uint2 hb = *reinterpret_cast<const uint2 *>(rp + w.plane3 + 8 * u);
        const uint32_t h5 = ((hi ? hb.y : hb.x) >> l) & 1u;
        const int n = (int)((hi ? ((byte >> 4) & 0x0F) : (byte & 0x0F)) + 16 * h5);
        v = dd * (float)n - mm;
    } else if (w.dtype == T_Q6_K) {
        const uint8_t *sp = w.base + (row >> 6) * w.group_stride + (i / 256) * IL64_Q6K_SB;
        const size_t lane = row & 63;
        const int p = (int)(i % 256), o = p / 128, r = p % 128, m = r / 32, l = r % 32;
        // byte j (0..207) of the super-block's ql/qh/scales is in chunk j/16.
        auto byte_at = [&](int j) { return sp[((size_t)(j >> 4) * 64 + lane) * 16 + (j & 15)]; };
        const int qhb = byte_at(128 + 32 * o + l);
        int q;
        if (m == 0) q = ((byte_at(64 * o + l) & 0x0F) | ((qhb & 3) << 4)) - 32;
        else if (m == 1) q = ((byte_at(64 * o + l + 32) & 0x0F) | (((qhb >> 2) & 3) << 4)) - 32;
        else if (m == 2) q = ((byte_at(64 * o + l) >> 4) | (((qhb >> 4) & 3) << 4)) - 32;
        else q = ((byte_at(64 * o + l + 32) >> 4) | (((qhb >> 6) & 3) << 4)) - 32;
        const int sc = (int)(int8_t)byte_at(192 + 8 * o + l / 16 + 2 * m);
        const float d = h2f(*reinterpret_cast<const uint16_t *>(sp + IL64_Q6K_D + lane * 2));
        const float t = d * (float)sc;
        v = t * (float)q;
    }
    return v;
}

__global__ void k_dequant_row(DevWeight w, size_t row, float *__restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < w.n_cols) out[i] = dequant_value(w, row, i);
}

// The row index comes from device memory (a token id of the decode step);
// an id outside [0, n_rows) leaves x unchanged and marks the step skipped
// (the status words of launch_embed_row).
__global__ void k_embed_row(DevWeight w, const int32_t *__restrict__ row_dev, float *__restrict__ x,
                            int *__restrict__ status) {
    const int32_t id = row_dev[0];
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool bad = id < 0 || (size_t)id >= w.n_rows;
    if (i == 0) {
        if (bad) {
            if (status[0] == 0) status[0] = 1;
            status[1] = status[1] + 1;
        }
        status[2] = bad ? 1 : 0;
    }
    if (!bad && i < w.n_cols) x[i] = dequant_value(w, (size_t)id, i);
}

// The Q8 activations of `total` / (k / 8) tokens, quantized once into
// `ws` in the layout ActLds gives a block of that many tokens.
__global__ __launch_bounds__(64) void k_quantize_act(const float *__restrict__ A, size_t k, int total,
                                                     unsigned char *__restrict__ ws, int T) {
    const int task = blockIdx.x * 64 + threadIdx.x;
    QuantTask q;
    quant_task_load(A, (int)(k / 8), 0, total, task, q);
    ActLds L(ws, k, T);
    quant_task_finish<false>(q, k, total, task, L);
}

}  // namespace

// Column units per row must fit one block of up to 1024 threads.
bool gpu_supports(uint32_t dtype, size_t n_cols, int mode) {
    if (n_cols == 0 || (mode != 0 && mode != 1)) return false;
    // Q8 keeps one token's quantized row in LDS (1.375 B per value).
    if (mode == 1 && act_lds_bytes(n_cols, 1) > LDS_MAX) return false;
    switch (dtype) {
    case T_Q4_0:
    case T_Q8_0:
    case T_Q5_0:
    case T_Q4_1:
        return n_cols % 32 == 0 && n_cols / 32 <= 1024;
    case T_Q4_K:
    case T_Q5_K:
        return n_cols % 256 == 0 && n_cols / 64 <= 1024;
    case T_Q3_K:
        return n_cols % 256 == 0 && n_cols / 32 <= 1024;
    case T_F32:
    case T_F16:
    case T_BF16: {  // the row's values padded to whole stages must fit the LDS staging
        const size_t es = dtype == T_F32 ? 4 : 2, chunks = (n_cols * es + 15) / 16;
        return ((chunks + CHAIN_STAGE - 1) / CHAIN_STAGE) * CHAIN_STAGE * (16 / es) <= CHAIN_MAX_K;
    }
    case T_I2_S:
        return n_cols % 128 == 0 && n_cols <= CHAIN_MAX_K;
    case T_Q1_0:  // 128 activations per thread: blocks of 256 threads only
    case T_Q2_0:
        return n_cols % 128 == 0 && n_cols / 128 <= 256;
    case T_STQ1_0:
        return n_cols % 256 == 0 && n_cols / 256 <= 256;
    case T_Q6_K:
        return n_cols % 256 == 0 && n_cols / 256 <= 1024;
    default:
        return false;
    }
}

static size_t pad16(size_t x) { return (x + 15) & ~(size_t)15; }

size_t plan_layout(DevWeight &dw) {
    const size_t n = dw.n_rows, k = dw.n_cols;
    switch (dw.dtype) {
    case T_Q4_0:
        dw.layout = LAYOUT_SPLIT_Q4_0;
        dw.plane1 = pad16(2 * (k / 32));
        dw.plane2 = 0;
        dw.row_stride = dw.plane1 + 16 * (k / 32);
        return dw.row_stride * n;
    case T_Q8_0:
        dw.layout = LAYOUT_SPLIT_Q8_0;
        dw.plane1 = pad16(2 * (k / 32));
        dw.plane2 = dw.plane1 + 16 * (k / 32);
        dw.row_stride = dw.plane2 + 16 * (k / 32);
        return dw.row_stride * n;
    case T_Q4_K:  // the file's 144 B per super-block, then 32 B of scale pairs
        dw.layout = LAYOUT_SPLIT_Q4_K;
        dw.plane1 = 16 * (k / 256);
        dw.plane2 = dw.plane1 + 16 * (k / 64);
        dw.plane4 = 144 * (k / 256);
        dw.row_stride = 176 * (k / 256);
        return dw.row_stride * n;
    case T_Q5_K:  // 16 + 4 * (16 + 16 + 8) = 176 B per super-block, as in the file, then 32 B of scale pairs
        dw.layout = LAYOUT_SPLIT_Q5_K;
        dw.plane1 = 16 * (k / 256);
        dw.plane2 = dw.plane1 + 16 * (k / 64);
        dw.plane3 = dw.plane2 + 16 * (k / 64);
        dw.plane4 = 176 * (k / 256);
        dw.row_stride = 208 * (k / 256);
        return dw.row_stride * n;
    case T_Q5_0:
        dw.layout = LAYOUT_SPLIT_Q5_0;
        dw.plane1 = pad16(2 * (k / 32));
        dw.plane2 = dw.plane1 + 16 * (k / 32);
        dw.row_stride = pad16(dw.plane2 + 4 * (k / 32));
        return dw.row_stride * n;
    case T_Q4_1:
        dw.layout = LAYOUT_SPLIT_Q4_1;
        dw.plane1 = pad16(4 * (k / 32));
        dw.plane2 = 0;
        dw.row_stride = dw.plane1 + 16 * (k / 32);
        return dw.row_stride * n;
    case T_Q3_K:
        dw.layout = LAYOUT_SPLIT_Q3_K;
        dw.plane1 = pad16(2 * (k / 256));
        dw.plane2 = dw.plane1 + 8 * (k / 32);
        dw.plane3 = dw.plane2 + 4 * (k / 32);
        dw.row_stride = pad16(dw.plane3 + 2 * (k / 32));
        return dw.row_stride * n;
    case T_Q1_0:  // 2 + 16 bytes per block of 128: Q4_0's split layout
        dw.layout = LAYOUT_SPLIT_Q4_0;
        dw.plane1 = pad16(2 * (k / 128));
        dw.plane2 = 0;
        dw.row_stride = dw.plane1 + 16 * (k / 128);
        return dw.row_stride * n;
    case T_Q2_0:  // 2 + 32 bytes per block of 128: Q8_0's split layout
        dw.layout = LAYOUT_SPLIT_Q8_0;
        dw.plane1 = pad16(2 * (k / 128));
        dw.plane2 = dw.plane1 + 16 * (k / 128);
        dw.row_stride = dw.plane2 + 16 * (k / 128);
        return dw.row_stride * n;
    case T_STQ1_0:
        dw.layout = LAYOUT_SPLIT_STQ1_0;
        dw.plane1 = pad16(2 * (k / 256));
        dw.row_stride = dw.plane1 + 64 * (k / 256);
        return dw.row_stride * n;
    case T_I2_S:  // the codes as bit planes in the 64-row groups, then the tensor's f32 scale
        dw.layout = LAYOUT_I2S_PLANES;
        dw.group_stride = (k / 64) * 1024;
        dw.plane1 = dw.group_stride * ((n + 63) / 64);
        return dw.plane1 + 16;
    case T_F32:
    case T_F16:
    case T_BF16:
        dw.layout = LAYOUT_IL64_ROWS;
        dw.group_stride = (((k * (dw.dtype == T_F32 ? 4 : 2) + 15) / 16 + CHAIN_STAGE - 1) / CHAIN_STAGE) *
                          CHAIN_STAGE * 1024;
        return dw.group_stride * ((n + 63) / 64);
    case T_Q6_K:
        dw.layout = LAYOUT_IL64_Q6_K;
        dw.group_stride = (k / 256) * IL64_Q6K_SB;
        return dw.group_stride * ((n + 63) / 64);
    default:
        return 0;
    }
}

size_t layout_pad_bytes(const DevWeight &dw) {
    const int U = units_per_row(dw.dtype, dw.n_cols);
    const size_t rows = 16 * (size_t)(U > 0 && U < 1024 ? 1024 / U : 1);  // the most rows a tile can add
    if (dw.layout == LAYOUT_IL64_Q6_K || dw.layout == LAYOUT_IL64_ROWS || dw.layout == LAYOUT_I2S_PLANES)
        return ((rows + 63) / 64 + 1) * dw.group_stride;
    return rows * dw.row_stride;
}

// The matrix-core GEMM's scale pairs of one Q4_K / Q5_K super-block (its
// 12 scale bytes and f16 d, dmin): for sub-block j, get_scale_min's (sc, m)
// (rce-op-qmm/src/lib.rs L719-728), then binary16 {d * sc, -(dmin * m)},
// each product exact in f32 (11 x 6 bits) and rounded once.
static void kquant_scale_pairs(const uint8_t *hdr, uint8_t *out) {
    auto f16_to_f32 = [](const uint8_t *b) {
        _Float16 h;
        std::memcpy(&h, b, 2);
        return (float)h;
    };
    const float d = f16_to_f32(hdr), dmin = f16_to_f32(hdr + 2);
    const uint8_t *q = hdr + 4;
    for (int j = 0; j < 8; j++) {
        int sc, m;
        if (j < 4) {
            sc = q[j] & 63;
            m = q[j + 4] & 63;
        } else {
            sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
            m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
        }
        const _Float16 s = (_Float16)(d * (float)sc), b = (_Float16)(-(dmin * (float)m));
        std::memcpy(out + 4 * j, &s, 2);
        std::memcpy(out + 4 * j + 2, &b, 2);
    }
}

void relayout_host(const uint8_t *src, const DevWeight &dw, uint8_t *dst) {
    const size_t n = dw.n_rows, k = dw.n_cols;
    switch (dw.layout) {
    case LAYOUT_SPLIT_Q4_0:
    case LAYOUT_SPLIT_Q8_0: {  // also Q1_0 (as Q4_0) and Q2_0 (as Q8_0), blocks of 128
        const size_t qk = (dw.dtype == T_Q1_0 || dw.dtype == T_Q2_0) ? 128 : 32;
        const size_t nb = k / qk, bb = dw.layout == LAYOUT_SPLIT_Q8_0 ? 34 : 18;
        for (size_t r = 0; r < n; r++) {
            const uint8_t *s = src + r * nb * bb;
            uint8_t *d = dst + r * dw.row_stride;
            for (size_t b = 0; b < nb; b++) {
                const uint8_t *blk = s + b * bb;
                d[2 * b] = blk[0];
                d[2 * b + 1] = blk[1];
                for (int i = 0; i < 16; i++) d[dw.plane1 + 16 * b + i] = blk[2 + i];
                if (dw.layout == LAYOUT_SPLIT_Q8_0)
                    for (int i = 0; i < 16; i++) d[dw.plane2 + 16 * b + i] = blk[18 + i];
            }
        }
        break;
    }
    case LAYOUT_SPLIT_Q5_0:  // block: d, qh[4], qs[16]
    case LAYOUT_SPLIT_Q4_1: {  // block: d, m, qs[16]
        const bool q5 = dw.layout == LAYOUT_SPLIT_Q5_0;
        const size_t nb = k / 32, bb = q5 ? 22 : 20;
        for (size_t r = 0; r < n; r++) {
            const uint8_t *s = src + r * nb * bb;
            uint8_t *d = dst + r * dw.row_stride;
            for (size_t b = 0; b < nb; b++) {
                const uint8_t *blk = s + b * bb;
                if (q5) {
                    d[2 * b] = blk[0];
                    d[2 * b + 1] = blk[1];
                    for (int i = 0; i < 4; i++) d[dw.plane2 + 4 * b + i] = blk[2 + i];
                } else {
                    for (int i = 0; i < 4; i++) d[4 * b + i] = blk[i];
                }
                for (int i = 0; i < 16; i++) d[dw.plane1 + 16 * b + i] = blk[bb - 16 + i];
            }
        }
        break;
    }
    case LAYOUT_SPLIT_Q3_K: {  // block: hmask[32], qs[64], scales[12], d
        const size_t nsb = k / 256;
        for (size_t r = 0; r < n; r++) {
            const uint8_t *s = src + r * nsb * 110;
            uint8_t *d = dst + r * dw.row_stride;
            for (size_t sb = 0; sb < nsb; sb++) {
                const uint8_t *blk = s + sb * 110, *hmask = blk, *qs = blk + 32, *sp = blk + 96;
                d[2 * sb] = blk[108];
                d[2 * sb + 1] = blk[109];
                int sc[16];  // the 6-bit scales (dequant.rs L486-504)
                for (int g = 0; g < 16; g++)
                    sc[g] = ((g < 8 ? sp[g] & 0xF : sp[g - 8] >> 4) | (((sp[8 + g % 4] >> (2 * (g / 4))) & 3) << 4));
                for (int o = 0; o < 2; o++)
                    for (int j = 0; j < 4; j++) {
                        const size_t u = 8 * sb + 4 * o + j;
                        uint32_t lw[2] = {0, 0}, hw = 0;
                        for (int h = 0; h < 2; h++)
                            for (int q = 0; q < 16; q++) {
                                const uint32_t low = (qs[32 * o + 16 * h + q] >> (2 * j)) & 3u;
                                const uint32_t high = (hmask[16 * h + q] >> (4 * o + j)) & 1u;
                                lw[h] |= low << (8 * (q % 4) + 2 * (q / 4));
                                hw |= high << (16 * h + q);
                            }
                        for (int b = 0; b < 4; b++) {
                            d[dw.plane1 + 8 * u + b] = (uint8_t)(lw[0] >> (8 * b));
                            d[dw.plane1 + 8 * u + 4 + b] = (uint8_t)(lw[1] >> (8 * b));
                            d[dw.plane2 + 4 * u + b] = (uint8_t)(hw >> (8 * b));
                        }
                        d[dw.plane3 + 2 * u] = (uint8_t)(int8_t)(sc[2 * (4 * o + j)] - 32);
                        d[dw.plane3 + 2 * u + 1] = (uint8_t)(int8_t)(sc[2 * (4 * o + j) + 1] - 32);
                    }
            }
        }
        break;
    }
    case LAYOUT_SPLIT_Q4_K: {
        const size_t nsb = k / 256;
        for (size_t r = 0; r < n; r++) {
            const uint8_t *s = src + r * nsb * 144;
            uint8_t *d = dst + r * dw.row_stride;
            for (size_t sb = 0; sb < nsb; sb++) {
                const uint8_t *blk = s + sb * 144;
                for (int i = 0; i < 16; i++) d[16 * sb + i] = blk[i];
                kquant_scale_pairs(blk, d + dw.plane4 + 32 * sb);
                for (int g = 0; g < 4; g++) {
                    const size_t u = 4 * sb + g;
                    for (int l = 0; l < 16; l++) d[dw.plane1 + 16 * u + l] = blk[16 + 32 * g + l];
                    for (int l = 0; l < 16; l++) d[dw.plane2 + 16 * u + l] = blk[16 + 32 * g + 16 + l];
                }
            }
        }
        break;
    }
    case LAYOUT_SPLIT_Q5_K: {  // block: d, dmin, scales[12], qh[32], qs[128]
        const size_t nsb = k / 256;
        for (size_t r = 0; r < n; r++) {
            const uint8_t *s = src + r * nsb * 176;
            uint8_t *d = dst + r * dw.row_stride;
            for (size_t sb = 0; sb < nsb; sb++) {
                const uint8_t *blk = s + sb * 176, *qh = blk + 16, *qs = blk + 48;
                for (int i = 0; i < 16; i++) d[16 * sb + i] = blk[i];
                kquant_scale_pairs(blk, d + dw.plane4 + 32 * sb);
                for (int g = 0; g < 4; g++) {
                    const size_t u = 4 * sb + g;
                    for (int l = 0; l < 16; l++) d[dw.plane1 + 16 * u + l] = qs[32 * g + l];
                    for (int l = 0; l < 16; l++) d[dw.plane2 + 16 * u + l] = qs[32 * g + 16 + l];
                    uint64_t bits = 0;  // group g reads qh bits 2g (low half) and 2g+1 (high half)
                    for (int l = 0; l < 32; l++) {
                        bits |= (uint64_t)((qh[l] >> (2 * g)) & 1) << l;
                        bits |= (uint64_t)((qh[l] >> (2 * g + 1)) & 1) << (32 + l);
                    }
                    for (int b = 0; b < 8; b++) d[dw.plane3 + 8 * u + b] = (uint8_t)(bits >> (8 * b));
                }
            }
        }
        break;
    }
    case LAYOUT_SPLIT_STQ1_0: {  // block: qs[32], sign[8], d; codebook dequant.rs L141-148
        static const uint8_t CB[32] = {0xA9, 0x89, 0x29, 0x09, 0xA6, 0x86, 0x26, 0x06, 0x9A, 0x92, 0x1A,
                                       0x12, 0x6A, 0x62, 0x4A, 0x42, 0x01, 0x21, 0x81, 0xA1, 0x04, 0x24,
                                       0x84, 0xA4, 0x10, 0x18, 0x90, 0x98, 0x40, 0x48, 0x60, 0x68};
        const size_t nsb = k / 256;
        for (size_t r = 0; r < n; r++) {
            const uint8_t *s = src + r * nsb * 42;
            uint8_t *d = dst + r * dw.row_stride;
            for (size_t sb = 0; sb < nsb; sb++) {
                const uint8_t *blk = s + sb * 42;
                d[2 * sb] = blk[40];
                d[2 * sb + 1] = blk[41];
                for (int g = 0; g < 64; g++) {
                    const int code = (blk[g / 2] >> (4 * (g & 1))) & 0xF, sg = (blk[32 + g / 8] >> (g % 8)) & 1;
                    d[dw.plane1 + 64 * sb + g] = CB[(sg << 4) | code];  // group g = byte g: lanes 4g..4g+3
                }
            }
        }
        break;
    }
    case LAYOUT_I2S_PLANES: {  // lib.rs L1478-1537: code 2 (+1) and code 0 (-1) as bit planes
        const size_t rb = k / 4;
        std::memcpy(dst + dw.plane1, src + n * rb, 4);  // the tensor's scale
        for (size_t r = 0; r < n; r++) {
            const uint8_t *s = src + r * rb;
            uint8_t *g = dst + (r >> 6) * dw.group_stride + (r & 63) * 8;
            for (size_t j = 0; j < k; j++) {  // chain order: block b, byte gp, slot s
                const size_t b = j / 128, gp = (j % 128) / 4, slot = j % 4;
                const int code = (s[32 * b + gp] >> (6 - 2 * slot)) & 3;
                uint8_t *cp = g + (j / 64) * 1024 + (j % 64) / 8;
                if (code == 2) cp[0] |= (uint8_t)(1u << (j % 8));
                if (code == 0) cp[512] |= (uint8_t)(1u << (j % 8));
            }
        }
        break;
    }
    case LAYOUT_IL64_ROWS: {
        const size_t rb = k * (dw.dtype == T_F32 ? 4 : 2);
        for (size_t r = 0; r < n; r++) {
            uint8_t *g = dst + (r >> 6) * dw.group_stride + (r & 63) * 16;
            const uint8_t *s = src + r * rb;
            for (size_t c = 0; c * 16 < rb; c++)
                std::memcpy(g + c * 1024, s + c * 16, std::min<size_t>(16, rb - c * 16));
        }
        break;
    }
    case LAYOUT_IL64_Q6_K: {
        const size_t nsb = k / 256;
        for (size_t r = 0; r < n; r++) {
            const size_t lane = r & 63;
            uint8_t *g = dst + (r >> 6) * dw.group_stride;
            for (size_t sb = 0; sb < nsb; sb++) {
                const uint8_t *blk = src + (r * nsb + sb) * 210;
                uint8_t *d = g + sb * IL64_Q6K_SB;
                for (size_t j = 0; j < 13; j++)
                    for (int i = 0; i < 16; i++) d[(j * 64 + lane) * 16 + i] = blk[16 * j + i];
                d[IL64_Q6K_D + 2 * lane] = blk[208];
                d[IL64_Q6K_D + 2 * lane + 1] = blk[209];
                // the GEMM's pairs: s = f16(d sc) (the f32 product is exact: 11 x 8 bits), -32 s
                _Float16 dh;
                std::memcpy(&dh, blk + 208, 2);
                for (int jj = 0; jj < 16; jj++) {
                    const _Float16 sh = (_Float16)((float)dh * (float)(int8_t)blk[192 + jj]);
                    const _Float16 bh = (_Float16)(-32.0f * (float)sh);
                    std::memcpy(d + IL64_Q6K_P + (jj * 64 + lane) * 4, &sh, 2);
                    std::memcpy(d + IL64_Q6K_P + (jj * 64 + lane) * 4 + 2, &bh, 2);
                }
            }
        }
        break;
    }
    default:
        break;
    }
}

hipError_t launch_f16_to_f32(const uint16_t *src, float *dst, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_f16_to_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, dst, n);
    return hipGetLastError();
}

// HBM bytes of one column unit of one row (the algorithmic share).
static size_t unit_bytes(uint32_t dtype) {
    switch (dtype) {
    case T_Q4_0: return 18;
    case T_Q8_0: return 34;
    case T_Q5_0: return 22;
    case T_Q4_1: return 20;
    case T_Q3_K: return 14;  // 13.75: an eighth of the 110 B super-block
    case T_Q1_0: return 18;
    case T_Q2_0: return 34;
    case T_STQ1_0: return 42;
    case T_Q4_K: return 36;
    case T_Q5_K: return 44;
    case T_Q6_K: return 210;
    default: return 0;
    }
}

// Launch shape.  Measured on MI355X (the sweep over threads x rows per
// thread x tokens per block): the best single-token shapes stream about
// 36 KB of weight per 256-thread block with every load issued up front,
// and keep at least one block per CU; Q6_K (one 210-byte super-block per
// thread-row, heavy activation slice) is best at 4 rows per thread.  With
// several tokens, Q8 keeps up to 8 per block (the weight tile is read once
// per block) and EXACT 2, with 16 rows per lane where the grid keeps 256
// blocks (below).
GemvGeom pick_gemv_geom(const DevWeight &w, size_t t_rows, int mode) {
    GemvGeom g;
    const int U = units_per_row(w.dtype, w.n_cols);
    g.nt = nt_for(U);
    const bool q8 = mode == 1;
    const int P = g.nt / U;
    const bool k4 = w.dtype == T_Q4_K || w.dtype == T_Q5_K;  // 64-value units
    int tbmax = q8 ? (w.dtype == T_Q6_K ? 2 : (k4 ? 4 : 8)) : (k4 ? 2 : 4);
    if ((w.dtype == T_Q6_K && !q8) || is_ternary_block(w.dtype)) tbmax = 1;
    g.tb = 1;
    while (g.tb * 2 <= tbmax && (size_t)g.tb * 2 <= t_rows) g.tb *= 2;
    if (w.dtype == T_Q6_K) {
        g.rpl = 4;
    } else if (g.tb == 1 && !q8 && !is_ternary_block(w.dtype)) {
        // One token, EXACT (bound by its f32 arithmetic, so the work of the
        // busiest CU decides): the rows per lane that give the busiest of the 256 CUs
        // the least work, counted as blocks per CU x (rows per block + 8):
        // a block's own cost (activation loads, the fold, launch) is about
        // eight rows' worth.  On a tie, the fewest blocks.  This picks the
        // best of 2..16 rows per lane in a sweep of eight decode shapes
        // (Q4_0 11008x4096: 12, 8.4 us against 9.7 at 8; Q4_K 4096x4096:
        // 4; Q8_0 4096x4096: 8; Q4_0 4096x14336: 16).  Q8, lighter on
        // arithmetic and better with more waves, keeps the rule below (its
        // best in the same sweep).
        static const int opts[] = {2, 4, 8, 12, 16};
        size_t best_cost = ~(size_t)0, best_blocks = 0;
        for (int o : opts) {
            if (gemv_lds_bytes(U, g.nt, o, 1, q8, w.n_cols) > LDS_MAX) continue;
            const size_t rt = (size_t)P * o, blocks = (w.n_rows + rt - 1) / rt;
            const size_t cost = (blocks + 255) / 256 * (rt + 8);
            if (cost < best_cost || (cost == best_cost && blocks < best_blocks)) {
                best_cost = cost;
                best_blocks = blocks;
                g.rpl = o;
            }
        }
    } else {
        const double pass = (double)P * U * unit_bytes(w.dtype) * (256.0 / g.nt);
        const double want = 36864.0 / pass;
        static const int opts[] = {2, 4, 8, 12, 16};
        g.rpl = 2;
        for (int o : opts)
            if (std::abs(o - want) < std::abs(g.rpl - want)) g.rpl = o;
        // at least one block per CU
        while (g.rpl > 2 && (w.n_rows + (size_t)P * g.rpl - 1) / ((size_t)P * g.rpl) < 256) g.rpl = g.rpl == 16 ? 12 : (g.rpl == 12 ? 8 : g.rpl / 2);
        const bool heavy = (q8 && g.tb >= 4) || (!q8 && (g.tb >= 4 || (k4 && g.tb >= 2)));
        if (heavy && g.rpl > 4) g.rpl = 4;
        if (is_ternary_block(w.dtype) && g.rpl > 4) g.rpl = 4;  // 128 activations or 256-lane codes per row
        if (!q8 && g.tb >= 2 && !is_ternary_block(w.dtype)) {
            // Several tokens, EXACT: two tokens per block and the most rows
            // per lane that leave 256 blocks (a sweep over tokens per block x
            // rows per lane at 2-64 tokens, Q4_0 11008x4096, Q4_K and Q8_0
            // 4096x4096: 16 rows per lane against 4 takes Q4_0 at 8 tokens
            // from 51 to 40 us, Q8_0 from 23 to 15; more tokens per block
            // hold more activations per lane and fewer waves fit a SIMD).
            g.tb = 2;
            auto blocks = [&](int rpl) {
                return (w.n_rows + (size_t)P * rpl - 1) / ((size_t)P * rpl) * ((t_rows + 1) / 2);
            };
            g.rpl = 16;
            while (g.rpl > 2 && blocks(g.rpl) < 256) g.rpl = g.rpl == 16 ? 12 : (g.rpl == 12 ? 8 : g.rpl / 2);
        }
    }
    // shrink rows, then tokens, until the block's LDS fits
    while (gemv_lds_bytes(U, g.nt, g.rpl, g.tb, q8, w.n_cols) > LDS_MAX) {
        if (g.rpl > 2) g.rpl = g.rpl == 16 ? 12 : (g.rpl == 12 ? 8 : g.rpl / 2);
        else if (g.tb > 1) g.tb /= 2;
        else break;
    }
    return g;
}

hipError_t launch_gemv(const DevWeight &w, const float *a, size_t t_rows, float *out, int mode, hipStream_t s,
                       const GemvGeom *geom) {
    if (t_rows == 0 || w.n_rows == 0) return hipSuccess;
    if (mode != 0 && mode != 1) return hipErrorInvalidValue;
    if (is_row_chain(w.dtype)) return launch_gemv_chain(w, a, t_rows, out, s);
    const GemvGeom g = geom ? *geom : pick_gemv_geom(w, t_rows, is_ternary_block(w.dtype) ? 0 : mode);
    if (is_ternary_block(w.dtype)) return launch_gemv_ternary(w, g, a, t_rows, out, s);
    switch (w.dtype) {
    case T_Q4_0: return launch_gemv_q4_0(w, g, a, t_rows, out, mode, s);
    case T_Q8_0: return launch_gemv_q8_0(w, g, a, t_rows, out, mode, s);
    case T_Q4_K: return launch_gemv_q4_k(w, g, a, t_rows, out, mode, s);
    case T_Q5_K: return launch_gemv_q5_k(w, g, a, t_rows, out, mode, s);
    case T_Q6_K: return launch_gemv_q6_k(w, g, a, t_rows, out, mode, s);
    case T_Q5_0: return launch_gemv_q5_0(w, g, a, t_rows, out, mode, s);
    case T_Q4_1: return launch_gemv_q4_1(w, g, a, t_rows, out, mode, s);
    case T_Q3_K: return launch_gemv_q3_k(w, g, a, t_rows, out, mode, s);
    default: return hipErrorInvalidValue;
    }
}

bool gemv_fx_supports(uint32_t dtype, size_t n_cols, int mode, bool with_norm) {
    if (!gpu_supports(dtype, n_cols, mode)) return false;
    if (dtype == T_Q6_K && mode == 0) return false;  // EXACT Q6_K is not the activation-stationary kernel
    if (dtype != T_Q4_0 && dtype != T_Q8_0 && dtype != T_Q4_K && dtype != T_Q5_K && dtype != T_Q6_K &&
        dtype != T_Q5_0 && dtype != T_Q4_1 && dtype != T_Q3_K)
        return false;
    // the normalizing forms hold the row's sum-of-squares tasks (8 values
    // each) in two per thread
    return !with_norm || n_cols / 8 <= (size_t)(2 * nt_for(units_per_row(dtype, n_cols)));
}

hipError_t launch_gemv_fx(const FxLaunch &f, const float *a, int mode, hipStream_t s, const GemvGeom *geom) {
    const DevWeight &w = f.w[0];
    if (mode != 0 && mode != 1) return hipErrorInvalidValue;
    if (!gemv_fx_supports(w.dtype, w.n_cols, mode, (f.kind & FX_NORM) != 0)) return hipErrorInvalidValue;
    for (int i = 1; i < f.nw; i++)
        if (f.w[i].dtype != w.dtype || f.w[i].n_cols != w.n_cols) return hipErrorInvalidValue;
    GemvGeom g = pick_gemv_geom(w, 1, mode);
    if (g.rpl > 8) g.rpl = 8;  // the fused forms exist for 1, 2, 4 and 8 rows per lane
    // Rows per lane, measured on the decode step's shapes (2048-11264 rows):
    // the plain forms want at least one block per CU; the normalizing forms
    // repeat rms_norm's prologue in every block, so they take the most rows
    // per lane that still leave 128 blocks.  Gate/up pairs need an even count.
    size_t rows = 0;
    for (int i = 0; i < f.nw; i++) rows += f.w[i].n_rows;
    if ((f.kind & 7) == FX_SWIGLU) rows = w.n_rows;
    const int P = g.nt / units_per_row(w.dtype, w.n_cols);
    const int min_rpl = (f.kind & 7) == FX_SWIGLU ? 2 : 1;
    const size_t per_rpl = (f.kind & 7) == FX_SWIGLU ? (size_t)P / 2 : (size_t)P;  // output rows per block per rpl
    const size_t min_blocks = (f.kind & FX_NORM) ? 128 : 256;
    if (f.kind & FX_NORM) g.rpl = 8;
    while (g.rpl > min_rpl && (rows + per_rpl * g.rpl - 1) / (per_rpl * g.rpl) < min_blocks) g.rpl /= 2;
    if (geom) g = *geom;
    switch (w.dtype) {
    case T_Q4_0: return launch_gemv_fx_q4_0(f, g, a, mode, s);
    case T_Q8_0: return launch_gemv_fx_q8_0(f, g, a, mode, s);
    case T_Q4_K: return launch_gemv_fx_q4_k(f, g, a, mode, s);
    case T_Q5_K: return launch_gemv_fx_q5_k(f, g, a, mode, s);
    case T_Q6_K: return launch_gemv_fx_q6_k(f, g, a, mode, s);
    case T_Q5_0: return launch_gemv_fx_q5_0(f, g, a, mode, s);
    case T_Q4_1: return launch_gemv_fx_q4_1(f, g, a, mode, s);
    case T_Q3_K: return launch_gemv_fx_q3_k(f, g, a, mode, s);
    default: return hipErrorInvalidValue;
    }
}

// RCE_QMM_Q8_MFMA: 0 = never the matrix-core form, 2 = always where it
// applies (tests of both forms on the same shapes), unset = where faster.
// Read at every call, so a test can switch it.
static int q8_mfma_env() {
    const char *e = getenv("RCE_QMM_Q8_MFMA");
    return e ? atoi(e) : 1;
}
bool gemv_q8_mfma_enabled() { return q8_mfma_env() != 0; }
bool gemv_q8_mfma_forced() { return q8_mfma_env() == 2; }

bool gemv_q8_pre_supports(uint32_t dtype, size_t n_cols, size_t t_rows) {
    if (gemv_q8_mfma_supports(dtype, n_cols, t_rows)) return true;
    if (t_rows < 2 || t_rows > 65535 * 8 || !gpu_supports(dtype, n_cols, 1)) return false;
    if (dtype != T_Q4_0 && dtype != T_Q8_0 && dtype != T_Q4_K && dtype != T_Q5_K && dtype != T_Q6_K) return false;
    return nt_for(units_per_row(dtype, n_cols)) == 256;
}

hipError_t launch_gemv_q8_pre(const DevWeight &w, const float *a, size_t t_rows, float *out, void *ws,
                              hipStream_t s) {
    if (t_rows == 0 || w.n_rows == 0) return hipSuccess;
    if (gemv_q8_mfma_supports(w.dtype, w.n_cols, t_rows) && gemv_q8_mfma_enabled() &&
        (gemv_q8_mfma_preferred(w.n_cols, t_rows) || gemv_q8_mfma_forced())) {
        // Q4_0 / Q8_0: the int8 matrix-core form (gemv_q8_mfma.hip), every
        // token of a 16-token tile in one pass over the weight
        const size_t k = w.n_cols;
        const int total = (int)(t_rows * (k / 8));
        unsigned char *q = static_cast<unsigned char *>(ws);
        hipLaunchKernelGGL(k_quantize_act, dim3((unsigned)((total + 63) / 64)), dim3(64), 0, s, a, k, total, q,
                           (int)t_rows);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_gemv_q8_mfma(w, q, t_rows, out, s);
    }
    if (!gemv_q8_pre_supports(w.dtype, w.n_cols, t_rows)) return launch_gemv(w, a, t_rows, out, 1, s);
    GemvGeom g = pick_gemv_geom(w, t_rows, 1);
    if (g.nt != 256 || g.tb < 2) return launch_gemv(w, a, t_rows, out, 1, s);
    if (g.tb > 4) g.tb = 4;  // more token groups re-read the weight, mostly from the Infinity Cache
    // the blocks no longer hold the activations in LDS: more rows per lane,
    // as long as the fold's LDS fits
    const size_t k = w.n_cols;
    const int U = units_per_row(w.dtype, k);
    // (every block reads its tokens' slices of the workspace: fewer, taller
    // blocks read less of it)
    g.rpl = 16;
    while (g.rpl > 2 && (w.n_rows + (size_t)(256 / U) * g.rpl - 1) / ((size_t)(256 / U) * g.rpl) < 256) g.rpl /= 2;
    while (g.rpl > 2 && gemv_lds_bytes(U, 256, g.rpl, g.tb, false, k) > LDS_MAX) g.rpl /= 2;
    if (gemv_lds_bytes(U, 256, g.rpl, g.tb, false, k) > LDS_MAX) return launch_gemv(w, a, t_rows, out, 1, s);
    const int total = (int)(t_rows * (k / 8));
    unsigned char *q = static_cast<unsigned char *>(ws);
    hipLaunchKernelGGL(k_quantize_act, dim3((unsigned)((total + 63) / 64)), dim3(64), 0, s, a, k, total, q,
                       (int)t_rows);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    switch (w.dtype) {
    case T_Q4_0: return launch_as_preq_tb<Q4_0Q8, 8>(w, g, a, t_rows, out, q, s);
    case T_Q8_0: return launch_as_preq_tb<Q8_0Q8, 8>(w, g, a, t_rows, out, q, s);
    case T_Q4_K: return launch_as_preq_tb<Q4_KQ8, 4>(w, g, a, t_rows, out, q, s);
    case T_Q5_K: return launch_as_preq_tb<Q5_KQ8, 4>(w, g, a, t_rows, out, q, s);
    case T_Q6_K: return launch_as_preq_tb<Q6_KQ8, 2>(w, g, a, t_rows, out, q, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_embed_row(const DevWeight &w, const int32_t *row_dev, float *x, int *status, hipStream_t s) {
    hipLaunchKernelGGL(k_embed_row, dim3((unsigned)((w.n_cols + 255) / 256)), dim3(256), 0, s, w, row_dev, x, status);
    return hipGetLastError();
}

hipError_t launch_dequant_row(const DevWeight &w, size_t row, float *out, hipStream_t s) {
    hipLaunchKernelGGL(k_dequant_row, dim3((unsigned)((w.n_cols + 255) / 256)), dim3(256), 0, s, w, row, out);
    return hipGetLastError();
}

}  // namespace rce_qmm
