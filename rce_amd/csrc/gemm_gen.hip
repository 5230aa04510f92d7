// gemm_gen.hip -- the prefill GEMM of the GGUF quantized-matmul path for the
// formats without a nibble-specialised matrix-core kernel (Q8_0, Q5_K, Q6_K,
// Q5_0, Q4_1, F16; BF16 and F32 on the bf16 matrix cores, below):
// out[M, N] = A[M, K] . W[N, K]^T, A binary16, every weight dequantized once
// per output tile into a binary16 tile in LDS and contracted with
// v_mfma_f32_32x32x16_f16 (f32 accumulation); plain, or grouped over the
// MoE tile table (tiles, gather and the epilogues of gemm_f16.hip).  It replaces
// the reference's batched paths (rce-op-qmm/src/lib.rs L967-1023: the Q8_0
// tile path for M >= 16, the Q5_K weight-stationary loop L1025-1100, the
// per-row fallback of every other dtype) for the F16_MFMA mode.
//
// Tile 128 (M) x 64 (N), K in chunks of 64; 512 threads = 8 waves.
//   * Loads, per chunk and thread: 32 bytes of A (two 16-byte loads; one
//     load instruction of a wave covers 8 rows x 128 bytes) and the raw
//     bytes of 8 consecutive weights of one W row (tile row t / 8, weights
//     8 (t % 8) .. +7 of the chunk), issued DEPTH (six) chunks ahead into
//     registers, so HBM latency overlaps several chunks of matrix work
//     (gen_pipeline below).
//   * Stores: A as loaded; the 8 weights as binary16, each the reference's
//     f32 dequantized value (rce-ingest-gguf/src/dequant.rs) rounded once
//     to nearest-even.  Both tiles are double-buffered in LDS with 16-byte
//     slot g of row r at g ^ f(r), f(r) = (r & 7) ^ ((r >> 3) & 1), so the
//     fragment reads (32 rows, one slot) and the stores are conflict-free.
//   * MFMA: wave w = 4 kh + 2 ch + rh computes rows 64 rh .. +63 (two 32 x 32
//     blocks) of columns 32 ch .. +31 for k-steps 2 kh and 2 kh + 1 of every
//     chunk.  The two k-halves are added at the end through LDS, kh 0 plus
//     kh 1: each output's summation order is fixed (run-to-run identical).
// One barrier per CPB (two) chunks.  Values: f16 rounding of A and W (about 2^-12
// relative each) with f32 accumulation; weights whose dequantized magnitude
// exceeds 65504 become infinite.
#include "gemm_epilogue.h"
#include "qmm_internal.h"

#include <type_traits>

namespace rce_qmm {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int KC = 64, NT = 512;
#ifndef GEN_DEPTH
#define GEN_DEPTH 6
#endif
#ifndef GEN_CPB
#define GEN_CPB 2
#endif
constexpr int DEPTH = GEN_DEPTH;  // register sets of chunk loads in flight
constexpr int CPB = GEN_CPB;      // chunks per barrier
constexpr int NBUF = 2 * CPB;     // LDS chunk buffers
static_assert(DEPTH % CPB == 0 && DEPTH >= 2 * CPB, "load ring");
// Output tile 128 x 64.  This kernel is bound by its dequantization into
// LDS, done once per row tile and weight, so the tallest tile is the
// cheapest: a 64 x 128 tile (built and measured) dequantizes every weight
// once per 64 rows and took the configs[3] workload with Q6_K experts from
// 668 to 829 us.
constexpr int BM = 128, BN = 64;
constexpr int A_TILE = BM * KC * 2;               // 16 KB
constexpr int B_TILE = BN * KC * 2;               // 8 KB
constexpr int LDS_BYTES = NBUF * (A_TILE + B_TILE);  // NBUF chunk buffers
static_assert(4 * 2 * 4 * 64 * 16 <= LDS_BYTES, "the k-half partial sums reuse the tiles' LDS");

__host__ __device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

__host__ __device__ __forceinline__ float f16_bits(uint32_t bits) {
    _Float16 h;
    const uint16_t b = (uint16_t)bits;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// Byte i of w as a float (v_cvt_f32_ubyte*).
__host__ __device__ __forceinline__ float ub(uint32_t w, int i) { return (float)((w >> (8 * i)) & 0xFFu); }

template <class T>
__host__ __device__ __forceinline__ T ld(const uint8_t *p) {
    T v;
    __builtin_memcpy(&v, p, sizeof(T));
    return v;
}

__host__ __device__ __forceinline__ half8 to_half8(const float (&y)[8]) {
    half8 h;
#pragma unroll
    for (int i = 0; i < 8; i++) h[i] = (_Float16)y[i];
    return h;
}

// Four 4-bit fields (x & 0xF) moved to bit 4 of bytes 0..3.
__host__ __device__ __forceinline__ uint32_t bits_to_b4(uint32_t x) { return (((x & 0xFu) * 0x00204081u) & 0x01010101u) << 4; }

// q4_k_get_scale_min (rce-op-qmm/src/lib.rs L719-728) of sub-block j from
// the super-block header h = {d | dmin << 16, scale bytes 0..3, 4..7, 8..11}.
__host__ __device__ __forceinline__ void k_scale_min(const u32x4 &h, int j, uint32_t &sc, uint32_t &m) {
    const int sh = 8 * (j & 3);
    if (j < 4) {
        sc = (h.y >> sh) & 63;
        m = (h.z >> sh) & 63;
    } else {
        const uint32_t hw = h.w >> sh;
        sc = (hw & 0x0F) | (((h.y >> sh) >> 6 & 3) << 4);
        m = (hw >> 4 & 0x0F) | (((h.z >> sh) >> 6 & 3) << 4);
    }
}

// ---- formats: load(raw, w, row, c, o) fetches what weights 64 c + 8 o ..
// +7 of row `row` need; dequant(raw, c, o) forms them (the reference's f32
// value, rounded to binary16 once).  Each f32 value below is formed with the
// reference's roundings: its products d*q are exact in f32, so one fma
// equals the reference's multiply-then-add (a zero weight may carry the
// other sign, which no sum can show).

// Q8_0, LAYOUT_SPLIT_Q8_0: y = q * d (dequant.rs L438-454).
struct FQ8_0 {
    static constexpr bool IL64 = false;
    struct Raw {
        u32x2 q;
        uint32_t d;
    };
    __host__ __device__ static void load(Raw &r, const DevWeight &w, size_t row, int c, int o) {
        const uint8_t *rp = w.base + row * w.row_stride;
        const int b = 2 * c + (o >> 2), p = o & 3;
        r.q = ld<u32x2>(rp + (p < 2 ? w.plane1 + 16 * (size_t)b + 8 * p : w.plane2 + 16 * (size_t)b + 8 * (p - 2)));
        r.d = ld<uint16_t>(rp + 2 * (size_t)b);
    }
    __host__ __device__ static half8 dequant(const Raw &r, int, int) {
        const float d = f16_bits(r.d), b = -128.0f * d;
        const uint32_t q0 = r.q.x ^ 0x80808080u, q1 = r.q.y ^ 0x80808080u;  // q + 128
        float y[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            y[i] = __builtin_fmaf(ub(q0, i), d, b);
            y[4 + i] = __builtin_fmaf(ub(q1, i), d, b);
        }
        return to_half8(y);
    }
};

// Q4_K / Q5_K, LAYOUT_SPLIT_Q4_K / _Q5_K: chunk c is 64-group c; y = d1 * q
// - m1, d1 = d * sc, m1 = dmin * m, q = nibble (+ 16 * fifth bit)
// (dequant.rs L546-604, L606-656).
template <bool Q5>
struct FQK {
    static constexpr bool IL64 = false;
    struct Raw {
        u32x2 q;
        uint32_t hb;
        u32x4 h;
    };
    __host__ __device__ static void load(Raw &r, const DevWeight &w, size_t row, int c, int o) {
        const uint8_t *rp = w.base + row * w.row_stride;
        const int p = o & 3;
        r.q = ld<u32x2>(rp + (p < 2 ? w.plane1 + 16 * (size_t)c + 8 * p : w.plane2 + 16 * (size_t)c + 8 * (p - 2)));
        r.hb = Q5 ? (uint32_t)rp[w.plane3 + 8 * (size_t)c + o] : 0u;  // bit i: position 8 o + i
        r.h = ld<u32x4>(rp + 16 * (size_t)(c >> 2));
    }
    __host__ __device__ static half8 dequant(const Raw &r, int c, int o) {
        const int sh = o >= 4 ? 4 : 0;  // positions 32.. are the high nibbles
        uint32_t v0 = (r.q.x >> sh) & 0x0F0F0F0Fu, v1 = (r.q.y >> sh) & 0x0F0F0F0Fu;
        if (Q5) {
            v0 |= bits_to_b4(r.hb);
            v1 |= bits_to_b4(r.hb >> 4);
        }
        uint32_t sc, m;
        k_scale_min(r.h, 2 * (c & 3) + (o >> 2), sc, m);
        const float d1 = f16_bits(r.h.x) * (float)sc, m1 = f16_bits(r.h.x >> 16) * (float)m;
        float y[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            y[i] = __builtin_fmaf(d1, ub(v0, i), -m1);
            y[4 + i] = __builtin_fmaf(d1, ub(v1, i), -m1);
        }
        return to_half8(y);
    }
};

// Q6_K, LAYOUT_IL64_Q6_K: y = (d * sc) * (q - 32) (dequant.rs L658-700).
// Position p of super-block c / 4: half n = p / 128, quadrant qd = (p % 128)
// / 32, l = p % 32; ql byte 64 n + l + 32 (qd & 1) (high nibble for qd >= 2),
// qh byte 32 n + l (bits 2 qd, 2 qd + 1), scale 8 n + l / 16 + 2 qd.
struct FQ6_K {
    static constexpr bool IL64 = true;
    struct Raw {
        u32x2 ql, qh;
        uint32_t sc, d;
    };
    __host__ __device__ static void load(Raw &r, const DevWeight &w, size_t row, int c, int o) {
        const uint8_t *gb = w.base + (row >> 6) * w.group_stride + (size_t)(c >> 2) * IL64_Q6K_SB;
        const int ln = (int)(row & 63);
        const int p0 = 64 * (c & 3) + 8 * o, n = p0 >> 7, qd = (p0 >> 5) & 3, l = p0 & 31;
        const int qi = 64 * n + l + 32 * (qd & 1), hi = 32 * n + l, si = 8 * n + (l >> 4) + 2 * qd;
        r.ql = ld<u32x2>(gb + ((qi >> 4) * 64 + ln) * 16 + (qi & 15));
        r.qh = ld<u32x2>(gb + ((8 + (hi >> 4)) * 64 + ln) * 16 + (hi & 15));
        r.sc = (uint32_t)gb[(12 * 64 + ln) * 16 + si];
        r.d = ld<uint16_t>(gb + IL64_Q6K_D + 2 * ln);
    }
    __host__ __device__ static half8 dequant(const Raw &r, int c, int o) {
        const int qd = ((64 * (c & 3) + 8 * o) >> 5) & 3;
        const int sl = qd >= 2 ? 4 : 0, sh = 2 * qd;
        const uint32_t v0 = ((r.ql.x >> sl) & 0x0F0F0F0Fu) | (((r.qh.x >> sh) & 0x03030303u) << 4);
        const uint32_t v1 = ((r.ql.y >> sl) & 0x0F0F0F0Fu) | (((r.qh.y >> sh) & 0x03030303u) << 4);
        const float ds = f16_bits(r.d) * (float)(int8_t)r.sc, b = -32.0f * ds;
        float y[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            y[i] = __builtin_fmaf(ds, ub(v0, i), b);
            y[4 + i] = __builtin_fmaf(ds, ub(v1, i), b);
        }
        return to_half8(y);
    }
};

// Q4_0 / Q5_0 / Q4_1, LAYOUT_SPLIT_Q4_0 / _Q5_0 / _Q4_1: block b = 2 c + o / 4;
// its positions 0..15 are the low nibbles of its 16 bytes, 16..31 the high
// ones.  Q4_0 y = (q - 8) * d, Q5_0 y = (q + 16 * bit - 16) * d (qh bit =
// position), Q4_1 y = q * d + m (dequant.rs L360-436).
template <int KIND>  // 0 Q4_0, 1 Q5_0, 2 Q4_1
struct FQ32 {
    static constexpr bool IL64 = false;
    struct Raw {
        u32x2 q;
        uint32_t hb, dm;
    };
    __host__ __device__ static void load(Raw &r, const DevWeight &w, size_t row, int c, int o) {
        const uint8_t *rp = w.base + row * w.row_stride;
        const int b = 2 * c + (o >> 2), p = o & 3;
        r.q = ld<u32x2>(rp + w.plane1 + 16 * (size_t)b + 8 * (p & 1));
        r.hb = KIND == 1 ? (uint32_t)rp[w.plane2 + 4 * (size_t)b + p] : 0u;
        r.dm = KIND == 2 ? ld<uint32_t>(rp + 4 * (size_t)b) : (uint32_t)ld<uint16_t>(rp + 2 * (size_t)b);
    }
    __host__ __device__ static half8 dequant(const Raw &r, int, int o) {
        const int sh = (o & 2) ? 4 : 0;
        uint32_t v0 = (r.q.x >> sh) & 0x0F0F0F0Fu, v1 = (r.q.y >> sh) & 0x0F0F0F0Fu;
        if (KIND == 1) {
            v0 |= bits_to_b4(r.hb);
            v1 |= bits_to_b4(r.hb >> 4);
        }
        const float d = f16_bits(r.dm);
        const float b = KIND == 0 ? -8.0f * d : KIND == 1 ? -16.0f * d : f16_bits(r.dm >> 16);
        float y[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            y[i] = __builtin_fmaf(ub(v0, i), d, b);
            y[4 + i] = __builtin_fmaf(ub(v1, i), d, b);
        }
        return to_half8(y);
    }
};

// F16, LAYOUT_IL64_ROWS: weights 64 c + 8 o .. +7 are 16-byte chunk 8 c + o
// of the row, at (chunk * 64 + row % 64) * 16 in its 64-row group.
struct FF16 {
    static constexpr bool IL64 = true;
    struct Raw {
        u32x4 v;
    };
    __host__ __device__ static void load(Raw &r, const DevWeight &w, size_t row, int c, int o) {
        const uint8_t *gb = w.base + (row >> 6) * w.group_stride;
        r.v = ld<u32x4>(gb + ((size_t)(8 * c + o) * 64 + (row & 63)) * 16);
    }
    __host__ __device__ static half8 dequant(const Raw &r, int, int) {
        half8 h;
        __builtin_memcpy(&h, &r.v, 16);
        return h;
    }
};

// The chunk pipeline of k_gemm_gen, a host/device function so the test
// harness can replay its schedule (tests/gemm_gen_host.hip).  Operations:
// sync() a block barrier; load(slot, ch) chunk ch's global loads into
// register set `slot`; mma(ch, buf) the matrix work of chunk ch from LDS
// buffer buf; store(slot, ch, buf) register set `slot` (holding chunk ch)
// into LDS buffer buf.
//
// At the top of a trip, LDS buffers hold chunks c .. c + CPB - 1 (stored
// before the last barrier) and register set s holds chunk c + s
// (s < DEPTH).  Group u of a trip loads chunks c + u + DEPTH .. into the
// register sets chunks c + u .. used (already stored), multiplies chunks
// c + u .., and stores chunks c + u + CPB .. into the buffers read last in
// the previous group, which every wave has left at this barrier.
// The main loop runs whole trips of DEPTH chunks with no branch, so the
// compiler's wait for a register set's loads counts only the loads issued
// after it (a loop with conditional loads waits for all of them); loads
// past the last chunk reload it.  The tail takes the last 0 .. DEPTH + CPB
// - 1 chunks: those past c + DEPTH - 1 are loaded there, into the sets the
// tail's first group frees.
template <int DEPTH, int CPB, class Sync, class Load, class Mma, class Store>
__host__ __device__ __forceinline__ void gen_pipeline(const int nchunks, Sync &&sync, Load &&load, Mma &&mma,
                                                      Store &&store) {
    constexpr int NBUF = 2 * CPB;
    const int last = nchunks - 1;
#pragma unroll
    for (int u = 0; u < DEPTH; u++) load(u, u < last ? u : last);
#pragma unroll
    for (int v = 0; v < CPB; v++)
        if (v < nchunks) store(v, v, v);
    int c = 0;
    for (; c + DEPTH + CPB <= nchunks; c += DEPTH) {
#pragma unroll
        for (int u = 0; u < DEPTH; u += CPB) {
            sync();
#pragma unroll
            for (int v = 0; v < CPB; v++) load(u + v, c + u + v + DEPTH < last ? c + u + v + DEPTH : last);
#pragma unroll
            for (int v = 0; v < CPB; v++) mma(c + u + v, (c + u + v) % NBUF);
#pragma unroll
            for (int v = 0; v < CPB; v++) store((u + v + CPB) % DEPTH, c + u + v + CPB, (c + u + v + CPB) % NBUF);
        }
    }
#pragma unroll
    for (int u = 0; u < DEPTH + CPB; u += CPB) {
        if (c + u < nchunks) {
            sync();
#pragma unroll
            for (int v = 0; v < CPB; v++)
                if (u + v < DEPTH && c + u + v + DEPTH < nchunks) load(u + v, c + u + v + DEPTH);
#pragma unroll
            for (int v = 0; v < CPB; v++)
                if (c + u + v < nchunks) mma(c + u + v, (c + u + v) % NBUF);
#pragma unroll
            for (int v = 0; v < CPB; v++)
                if (c + u + v + CPB < nchunks) store((u + v + CPB) % DEPTH, c + u + v + CPB, (c + u + v + CPB) % NBUF);
        }
    }
}

// BF16 / F32, LAYOUT_IL64_ROWS (chunk c of a row: 16 bytes, at (c * 64 + row
// % 64) * 16 in its 64-row group; 8 BF16 or 4 F32 values).  These take the
// bf16 matrix cores: binary16 cannot hold every BF16 or F32 weight (their
// exponent range is binary32's).  dequant gives the weights as WT bf16
// terms: BF16 exactly (one term), F32 as hi = bf16(w) plus lo = bf16(w - hi)
// (16 significant bits; the rest is below 2^-16 of |w|).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
struct FBF16 {
    static constexpr bool IL64 = true, BF = true;
    static constexpr int WT = 1;
    struct Raw {
        u32x4 v;
    };
    __host__ __device__ static void load(Raw &r, const DevWeight &w, size_t row, int c, int o) {
        const uint8_t *gb = w.base + (row >> 6) * w.group_stride;
        r.v = ld<u32x4>(gb + ((size_t)(8 * c + o) * 64 + (row & 63)) * 16);
    }
    __host__ __device__ static void dequant(const Raw &r, int, int, bf16x8 (&t)[1]) { __builtin_memcpy(&t[0], &r.v, 16); }
};
struct FF32 {
    static constexpr bool IL64 = true, BF = true;
    static constexpr int WT = 2;
    struct Raw {
        u32x4 v0, v1;
    };
    __host__ __device__ static void load(Raw &r, const DevWeight &w, size_t row, int c, int o) {
        const uint8_t *gb = w.base + (row >> 6) * w.group_stride + (row & 63) * 16;
        const size_t ch = 16 * (size_t)c + 2 * o;  // weights 64 c + 8 o .. +7: chunks ch, ch + 1
        r.v0 = ld<u32x4>(gb + ch * 1024);
        r.v1 = ld<u32x4>(gb + (ch + 1) * 1024);
    }
    __host__ __device__ static void dequant(const Raw &r, int, int, bf16x8 (&t)[2]) {
        float v[8];
        __builtin_memcpy(v, &r.v0, 16);
        __builtin_memcpy(v + 4, &r.v1, 16);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const __bf16 hi = (__bf16)v[i];
            t[0][i] = hi;
            t[1][i] = (__bf16)(v[i] - (float)hi);
        }
    }
};

// BF and WT of a format (the binary16 formats define neither: false, 1).
template <class F, class = void>
struct IsBf : std::false_type {};
template <class F>
struct IsBf<F, std::void_t<decltype(F::BF)>> : std::bool_constant<F::BF> {};
template <class F, class = void>
struct WtOf : std::integral_constant<int, 1> {};
template <class F>
struct WtOf<F, std::void_t<decltype(F::WT)>> : std::integral_constant<int, F::WT> {};

// Eight binary16 values as bf16 hi = bf16(a) and lo = bf16(a - hi), both
// rounded to nearest even; a - hi has at most 4 significant bits, so lo is
// exact and hi + lo = a.
__device__ __forceinline__ void split_bf16(const u32x4 &a, bf16x8 &hi, bf16x8 &lo) {
    half8 h;
    __builtin_memcpy(&h, &a, 16);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float f = (float)h[i];
        hi[i] = (__bf16)f;
        lo[i] = (__bf16)(f - (float)hi[i]);
    }
}

template <class F>
struct Stage {
    u32x4 a0, a1;
    typename F::Raw w;
};

// Plain GEMM: tiles == nullptr, row tile mt covers rows mt * BM .. of M.
// Grouped (MoE): row tile mt is tiles[mt] (expert e, first row r0, rows <=
// BM), multiplied by wtab[e], its A rows gathered through `gather` (when not
// null); tiles at or past n_tiles[0] do nothing.  EPI (GemmEpilogue) is what
// the block stores for an output element o with f32 sum v: v (f32 out),
// binary16 silu(v), or binary16 silu(aux[o]) * v.
template <class F, int EPI>
__global__ __launch_bounds__(NT) void k_gemm_gen(DevWeight w_arg, const _Float16 *__restrict__ A, size_t M,
                                                 void *__restrict__ out_v, int m_tiles, const int *__restrict__ gather,
                                                 const MoeTile *__restrict__ tiles, const int *__restrict__ n_tiles,
                                                 const DevWeight *__restrict__ wtab, const float *__restrict__ aux) {
    __shared__ __align__(16) unsigned char lds[LDS_BYTES];
    int mt, nt;
    if (!tile_of_block<BN>(w_arg.n_rows, m_tiles, n_tiles, mt, nt)) return;  // before any barrier
    DevWeight w = w_arg;
    size_t m0 = (size_t)mt * BM;
    int rows = (int)(M - m0 < (size_t)BM ? M - m0 : BM);
    if (tiles) {
        const MoeTile tl = tiles[mt];
        w = wtab[tl.e];
        m0 = (size_t)tl.r0;
        rows = tl.rows;
    }
    const size_t N = w.n_rows, K = w.n_cols;
    const size_t n0 = (size_t)nt * BN;
    const int nchunks = (int)(K / KC);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // Loads: A rows ar and ar + 64 of the tile, 16-byte piece ap of the
    // chunk (rows past the tile's load its last row); W tile row wn, octet
    // wo (rows past N: the last row, or the 64-row group's padding for the
    // IL64 layouts).
    const int ar = tid >> 3, ap = tid & 7;
    const size_t r0a = m0 + (size_t)(ar < rows ? ar : rows - 1), r1a = m0 + (size_t)(ar + 64 < rows ? ar + 64 : rows - 1);
    const size_t am0 = gather ? (size_t)gather[r0a] : r0a, am1 = gather ? (size_t)gather[r1a] : r1a;
    const _Float16 *ag0 = A + am0 * K + 8 * ap, *ag1 = A + am1 * K + 8 * ap;
    const int wn = tid >> 3, wo = tid & 7;
    const size_t wrow = F::IL64 || n0 + wn < N ? n0 + wn : N - 1;
    // The bf16 formats (BF): A as two bf16 tiles, hi = bf16(a) then lo =
    // a - hi (exact: a binary16 value has 11 significant bits), and WT
    // weight tiles; one chunk per barrier (a chunk is 40 or 48 KB of LDS).
    constexpr bool BF = IsBf<F>::value;
    constexpr int WT = WtOf<F>::value;
    constexpr int KCPB = BF ? 1 : CPB, KNBUF = 2 * KCPB;
    constexpr int KA_TILE = BF ? 2 * A_TILE : A_TILE, KB_TILE = WT * B_TILE;
    static_assert(KNBUF * (KA_TILE + KB_TILE) <= LDS_BYTES, "LDS");
    const int a_st0 = ar * 128 + 16 * (ap ^ swz(ar)), a_st1 = a_st0 + 64 * 128;
    const int b_st = KNBUF * KA_TILE + wn * 128 + 16 * (wo ^ swz(wn));

    auto load = [&](Stage<F> &s, int c) {
        s.a0 = ld<u32x4>(reinterpret_cast<const uint8_t *>(ag0 + (size_t)c * KC));
        s.a1 = ld<u32x4>(reinterpret_cast<const uint8_t *>(ag1 + (size_t)c * KC));
        F::load(s.w, w, wrow, c, wo);
    };
    auto store = [&](const Stage<F> &s, int c, int buf) {
        if constexpr (BF) {
            bf16x8 hi0, lo0, hi1, lo1, t[WT];
            split_bf16(s.a0, hi0, lo0);
            split_bf16(s.a1, hi1, lo1);
            *reinterpret_cast<bf16x8 *>(lds + buf * KA_TILE + a_st0) = hi0;
            *reinterpret_cast<bf16x8 *>(lds + buf * KA_TILE + a_st1) = hi1;
            *reinterpret_cast<bf16x8 *>(lds + buf * KA_TILE + A_TILE + a_st0) = lo0;
            *reinterpret_cast<bf16x8 *>(lds + buf * KA_TILE + A_TILE + a_st1) = lo1;
            F::dequant(s.w, c, wo, t);
#pragma unroll
            for (int i = 0; i < WT; i++) *reinterpret_cast<bf16x8 *>(lds + buf * KB_TILE + i * B_TILE + b_st) = t[i];
        } else {
            *reinterpret_cast<u32x4 *>(lds + buf * A_TILE + a_st0) = s.a0;
            *reinterpret_cast<u32x4 *>(lds + buf * A_TILE + a_st1) = s.a1;
            *reinterpret_cast<half8 *>(lds + buf * B_TILE + b_st) = F::dequant(s.w, c, wo);
        }
    };

    // Fragment reads: A rows 64 rh + 32 b + l32, B rows 32 ch + l32, slot
    // 2 s + h for k-step s = 2 kh + j.
    const int rh = wave & 1, ch = (wave >> 1) & 1, kh = wave >> 2;
    const int l32 = lane & 31, h = lane >> 5;
    int a_rd[2][2], b_rd[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int g = 2 * (2 * kh + j) + h;
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int r = 64 * rh + 32 * b + l32;
            a_rd[b][j] = r * 128 + 16 * (g ^ swz(r));
        }
        const int r = 32 * ch + l32;
        b_rd[j] = KNBUF * KA_TILE + r * 128 + 16 * (g ^ swz(r));
    }
    f32x16 acc0 = {}, acc1 = {};
    auto mma = [&](int buf) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            if constexpr (BF) {
                // sum a.w as a_hi.w_hi + a_lo.w_hi (+ a_hi.w_lo for F32):
                // every product exact in f32, f32 accumulation
                const unsigned char *at = lds + buf * KA_TILE, *bt = lds + buf * KB_TILE;
                const bf16x8 a0h = *reinterpret_cast<const bf16x8 *>(at + a_rd[0][j]);
                const bf16x8 a0l = *reinterpret_cast<const bf16x8 *>(at + A_TILE + a_rd[0][j]);
                const bf16x8 a1h = *reinterpret_cast<const bf16x8 *>(at + a_rd[1][j]);
                const bf16x8 a1l = *reinterpret_cast<const bf16x8 *>(at + A_TILE + a_rd[1][j]);
                const bf16x8 bh = *reinterpret_cast<const bf16x8 *>(bt + b_rd[j]);
                acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0h, bh, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1h, bh, acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0l, bh, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1l, bh, acc1, 0, 0, 0);
                if constexpr (WT == 2) {
                    const bf16x8 bl = *reinterpret_cast<const bf16x8 *>(bt + B_TILE + b_rd[j]);
                    acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0h, bl, acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1h, bl, acc1, 0, 0, 0);
                }
            } else {
                const half8 a0 = *reinterpret_cast<const half8 *>(lds + buf * A_TILE + a_rd[0][j]);
                const half8 a1 = *reinterpret_cast<const half8 *>(lds + buf * A_TILE + a_rd[1][j]);
                const half8 bf = *reinterpret_cast<const half8 *>(lds + buf * B_TILE + b_rd[j]);
                acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, bf, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, bf, acc1, 0, 0, 0);
            }
        }
    };

    Stage<F> st[DEPTH];
    gen_pipeline<DEPTH, KCPB>(
        nchunks, [&] { __syncthreads(); }, [&](int slot, int ch) { load(st[slot], ch); },
        [&](int, int buf) { mma(buf); }, [&](int slot, int ch, int buf) { store(st[slot], ch, buf); });
    __syncthreads();  // every fragment read done: the partial sums reuse LDS

    // k-half 1 hands its sums to k-half 0 (element r of a block in lane l is
    // row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32 of the 32 x 32 block).
    f32x4 *red = reinterpret_cast<f32x4 *>(lds);
    const int pw = wave & 3;
    if (kh == 1) {
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            red[((pw * 2 + 0) * 4 + rq) * 64 + lane] = f32x4{acc0[4 * rq], acc0[4 * rq + 1], acc0[4 * rq + 2], acc0[4 * rq + 3]};
            red[((pw * 2 + 1) * 4 + rq) * 64 + lane] = f32x4{acc1[4 * rq], acc1[4 * rq + 1], acc1[4 * rq + 2], acc1[4 * rq + 3]};
        }
    }
    __syncthreads();
    if (kh == 1) return;
    const size_t col = n0 + 32 * ch + l32;
#pragma unroll
    for (int b = 0; b < 2; b++) {
        const f32x16 &acc = b ? acc1 : acc0;
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            const f32x4 other = red[((pw * 2 + b) * 4 + rq) * 64 + lane];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = 64 * rh + 32 * b + 8 * rq + 4 * h + e;
                if (m < rows && col < N) {
                    const size_t o = (m0 + m) * N + col;
                    const float v = acc[4 * rq + e] + other[e];
                    if constexpr (EPI == GEPI_F32) {
                        static_cast<float *>(out_v)[o] = v;
                    } else if constexpr (EPI == GEPI_SILU_F16) {  // rce-qwen36-moe/src/lib.rs L459-461
                        static_cast<_Float16 *>(out_v)[o] = (_Float16)silu_mfma(v);
                    } else {  // silu(g) * u, rce-qwen36-moe/src/lib.rs L667-676
                        static_cast<_Float16 *>(out_v)[o] = (_Float16)(silu_mfma(aux[o]) * v);
                    }
                }
            }
        }
    }
}

template <class F>
hipError_t launch(const DevWeight &w, const _Float16 *a, size_t M, float *out, hipStream_t s) {
    const size_t m_tiles = (M + BM - 1) / BM, n_tiles = (w.n_rows + BN - 1) / BN;
    if (m_tiles * n_tiles > 0x7fffffffu || m_tiles > 0x7fffffffu) return hipErrorInvalidValue;
    hipLaunchKernelGGL((k_gemm_gen<F, GEPI_F32>), dim3((unsigned)(m_tiles * n_tiles)), dim3(NT), 0, s, w, a, M,
                       (void *)out, (int)m_tiles, (const int *)nullptr, (const MoeTile *)nullptr, (const int *)nullptr,
                       (const DevWeight *)nullptr, (const float *)nullptr);
    return hipGetLastError();
}

template <class F>
hipError_t launch_grouped(int epi, const DevWeight &w, const DevWeight *wtab, const _Float16 *a, size_t a_rows,
                          const int *gather, const MoeTile *tiles, const int *n_tiles_dev, int max_tiles, void *out,
                          const float *aux, hipStream_t s) {
    const size_t n_tiles = (w.n_rows + BN - 1) / BN;
    if ((size_t)max_tiles * n_tiles > 0x7ffffff0u) return hipErrorInvalidValue;
    const dim3 grid((unsigned)grouped_grid(max_tiles, (int)n_tiles));
    switch (epi) {
    case GEPI_F32:
        hipLaunchKernelGGL((k_gemm_gen<F, GEPI_F32>), grid, dim3(NT), 0, s, w, a, a_rows, out, max_tiles, gather, tiles,
                           n_tiles_dev, wtab, aux);
        break;
    case GEPI_SILU_F16:
        hipLaunchKernelGGL((k_gemm_gen<F, GEPI_SILU_F16>), grid, dim3(NT), 0, s, w, a, a_rows, out, max_tiles, gather,
                           tiles, n_tiles_dev, wtab, aux);
        break;
    case GEPI_SWIGLU_F16:
        if (!aux) return hipErrorInvalidValue;
        hipLaunchKernelGGL((k_gemm_gen<F, GEPI_SWIGLU_F16>), grid, dim3(NT), 0, s, w, a, a_rows, out, max_tiles, gather,
                           tiles, n_tiles_dev, wtab, aux);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

bool gemm_gen_supports(uint32_t dtype, size_t n_cols) {
    if (n_cols == 0 || n_cols % KC) return false;
    switch (dtype) {
    case T_Q8_0:
    case T_Q5_0:
    case T_Q4_1:
    case T_F16:
    case T_BF16:
    case T_F32:
        return true;
    case T_Q5_K:
    case T_Q6_K:
        return n_cols % 256 == 0;
    default:
        return false;
    }
}

hipError_t launch_gemm_gen(const DevWeight &w, const void *a_f16, size_t M, float *out, hipStream_t s, bool nibble_forms) {
    if (M == 0 || w.n_rows == 0) return hipSuccess;
    const _Float16 *a = static_cast<const _Float16 *>(a_f16);
    const size_t k = w.n_cols;
    if (k == 0 || k % KC) return hipErrorInvalidValue;
    switch (w.dtype) {
    case T_Q8_0: return launch<FQ8_0>(w, a, M, out, s);
    case T_Q5_0: return launch<FQ32<1>>(w, a, M, out, s);
    case T_Q4_1: return launch<FQ32<2>>(w, a, M, out, s);
    case T_F16: return launch<FF16>(w, a, M, out, s);
    case T_BF16: return launch<FBF16>(w, a, M, out, s);
    case T_F32: return launch<FF32>(w, a, M, out, s);
    case T_Q5_K: return k % 256 ? hipErrorInvalidValue : launch<FQK<true>>(w, a, M, out, s);
    case T_Q6_K: return k % 256 ? hipErrorInvalidValue : launch<FQ6_K>(w, a, M, out, s);
    case T_Q4_0: return nibble_forms ? launch<FQ32<0>>(w, a, M, out, s) : hipErrorInvalidValue;
    case T_Q4_K: return nibble_forms && k % 256 == 0 ? launch<FQK<false>>(w, a, M, out, s) : hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm_gen_grouped(const DevWeight &w, const DevWeight *wtab, const void *a_f16, size_t a_rows,
                                   const int *gather, const MoeTile *tiles, const int *n_tiles_dev, int max_tiles,
                                   int epi, void *out, const float *aux, hipStream_t s) {
    if (max_tiles <= 0 || w.n_rows == 0 || a_rows == 0) return hipSuccess;
    if (!gemm_gen_supports(w.dtype, w.n_cols)) return hipErrorInvalidValue;
    const _Float16 *a = static_cast<const _Float16 *>(a_f16);
    switch (w.dtype) {
    case T_Q8_0: return launch_grouped<FQ8_0>(epi, w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles, out, aux, s);
    case T_Q5_0: return launch_grouped<FQ32<1>>(epi, w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles, out, aux, s);
    case T_Q4_1: return launch_grouped<FQ32<2>>(epi, w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles, out, aux, s);
    case T_BF16: return launch_grouped<FBF16>(epi, w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles, out, aux, s);
    case T_F32: return launch_grouped<FF32>(epi, w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles, out, aux, s);
    case T_F16: return launch_grouped<FF16>(epi, w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles, out, aux, s);
    case T_Q5_K: return launch_grouped<FQK<true>>(epi, w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles, out, aux, s);
    case T_Q6_K: return launch_grouped<FQ6_K>(epi, w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles, out, aux, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace rce_qmm
