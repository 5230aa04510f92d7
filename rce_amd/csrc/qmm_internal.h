// qmm_internal.h -- internal interface between the C ABI (qmm_abi.cpp) and
// the HIP kernels (qmm_gemv.hip, gemv_<format>.hip).  Not installed; callers use
// include/rce_qmm.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace rce_qmm {

// GGUF type tags (rce-ingest-gguf/src/parser.rs L306-341).
enum : uint32_t {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q8_0 = 8,
    T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30, T_I2_S = 36, T_Q1_0 = 41, T_Q2_0 = 42,
    // STQ1_0 shares the file tag 42 with Q2_0 (parser.rs L376-377): the ABI
    // names it tag 42 with bit 31 set (RCE_QMM_DTYPE_STQ1_0).
    T_STQ1_0 = 0x8000002Au
};

// How a weight's GGUF bytes are arranged in HBM.  Every layout holds the
// same bytes as the GGUF tensor plus at most 15 bytes of padding per row
// (Q6_K: rows padded to a multiple of 64); only their order differs.  Each is chosen so
// that one load instruction of a wave reads 1 KB of contiguous HBM.
enum Layout : int {
    // Row r at r*row_stride: [block scales, 2 B each, padded to 16]
    // [16 B of nibbles per block at plane1 + 16 b].
    LAYOUT_SPLIT_Q4_0 = 1,
    // Row r: [scales, padded to 16][bytes 0..15 of each block at
    // plane1 + 16 b][bytes 16..31 of each block at plane2 + 16 b].
    LAYOUT_SPLIT_Q8_0 = 2,
    // Row r: [16 B header (d, dmin, 12 scale bytes) per super-block]
    // [qs bytes l = 0..15 of 64-group u at plane1 + 16 u]
    // [qs bytes l = 16..31 of group u at plane2 + 16 u]
    // [at plane4 + 32 sb the super-block's eight binary16 pairs
    //  {f16(d sc_j), f16(-(dmin m_j))}, j = 0..7: the matrix-core GEMM's
    //  scales, formed once here instead of in every GEMM tile].
    LAYOUT_SPLIT_Q4_K = 3,
    // Rows in groups of 64; per group and super-block sb (IL64_Q6K_SB
    // bytes at sb * IL64_Q6K_SB) the 13 16-byte chunks of the super-block's
    // ql (0..7), qh (8..11) and scales (12) for the 64 rows, chunk j of row
    // r at (j * 64 + r % 64) * 16, then the rows' 2-byte d values, then at
    // IL64_Q6K_P the matrix-core GEMM's binary16 pairs {f16(d sc_j),
    // -32 f16(d sc_j)} of the 16 scales, pair j of row r at (j * 64 + r % 64) * 4.
    LAYOUT_IL64_Q6_K = 4,
    // Q5_K: LAYOUT_SPLIT_Q4_K's header and two qs planes, plus at plane3 +
    // 8 u one 8-byte word per 64-group u: bit l (l < 32) = the 5th bit of
    // position l, bit 32 + l = that of position 32 + l (the two qh bits of
    // the group, 2g and 2g + 1, of qh byte l); then Q4_K's scale pairs at
    // plane4.
    LAYOUT_SPLIT_Q5_K = 5,
    // Q5_0: LAYOUT_SPLIT_Q4_0's scales and nibble plane, plus the blocks'
    // 4-byte qh words at plane2 + 4 b; rows padded to 16 B.
    LAYOUT_SPLIT_Q5_0 = 6,
    // Q4_1: the blocks' (d, m) f16 pairs as 4-byte words, padded to 16,
    // then the 16 B of nibbles per block at plane1 + 16 b.
    LAYOUT_SPLIT_Q4_1 = 7,
    // Q3_K, per row: the super-blocks' f16 d, padded to 16; then per unit
    // u of 32 values (u = 8 sb + 4 o + j, the reference's (outer, j) loop)
    // at plane1 + 8 u two words of 2-bit low parts (word h holds positions
    // 16 h + q, q < 16, at bits 8 (q % 4) + 2 (q / 4)), at plane2 + 4 u the
    // 32 high bits (bit p = position p), at plane3 + 2 u the unit's two
    // 16-value scales as signed bytes (the 6-bit scale minus 32); rows
    // padded to 16 B.
    LAYOUT_SPLIT_Q3_K = 8,
    // F32 / F16 / BF16: rows in groups of 64, each row cut into 16-byte
    // chunks, zero-padded to a multiple of CHAIN_STAGE chunks; chunk c of
    // row r at (c * 64 + r % 64) * 16 within the group's group_stride bytes.
    LAYOUT_IL64_ROWS = 9,
    // STQ1_0: the super-blocks' f16 d, padded to 16, then per super-block
    // u the 256 lane codes its codebook gives (64 B at plane1 + 64 u:
    // position p at bits 2 (p % 4) of byte p / 4; 0 = -1, 1 = 0, 2 = +1).
    // Q1_0 uses LAYOUT_SPLIT_Q4_0 (2-byte d + 16 bytes per block of 128)
    // and Q2_0 LAYOUT_SPLIT_Q8_0 (2-byte d + 32 bytes).
    LAYOUT_SPLIT_STQ1_0 = 10,
    // I2_S: the codes as two bit planes in the reference's chain order
    // (element j of a row is position 128 b + 32 s + gp for j = 128 b +
    // 4 gp + s), rows in groups of 64: chunk c (elements 64 c .. 64 c + 63)
    // of a group is 1 KB at c * 1024, the plane P (code 2, +1) of its 64 rows
    // as 8 bytes each (bit e = element 64 c + e), then the plane N (code 0,
    // -1) likewise at + 512; the tensor's f32 scale at plane1 (aux).
    LAYOUT_I2S_PLANES = 11,
};

struct DevWeight {
    const uint8_t *base;  // device address of row 0 (IL64: of row group 0)
    uint32_t dtype;
    int layout;
    size_t n_rows, n_cols;
    size_t row_stride;    // SPLIT: bytes between rows
    size_t plane1;        // SPLIT: offset of the first 16-B plane in a row
    size_t plane2;        // SPLIT_Q8_0 / SPLIT_Q4_K / SPLIT_Q5_K / SPLIT_Q5_0: offset of the second plane
    size_t plane3;        // SPLIT_Q5_K: offset of the high-bit words; SPLIT_Q3_K: of the scales
    size_t plane4;        // SPLIT_Q4_K / SPLIT_Q5_K: offset of the f16 scale pairs
    size_t group_stride;  // IL64: bytes between 64-row groups
    const uint8_t *aux;   // I2_S: device address of the tensor's f32 scale
};

constexpr size_t IL64_Q6K_D = 13 * 64 * 16;          // 13312: the d values
constexpr size_t IL64_Q6K_P = IL64_Q6K_D + 64 * 2;   // 13440 = 64 * 210: the scale pairs
constexpr size_t IL64_Q6K_SB = IL64_Q6K_P + 64 * 64;  // 17536

// Launch shape of a decode kernel: threads per block, rows per lane, and
// activation rows (tokens) per block.
struct GemvGeom {
    int nt = 0, rpl = 0, tb = 0;
};

// The library's exp: x = n ln2 + r with n = rint(x log2e) and r = (x -
// n ln2_hi) - n ln2_lo (Cody & Waite's two-part ln 2, W. J. Cody and W.
// Waite, Software Manual for the Elementary Functions, 1980), exp(r) by its
// Taylor series to degree 7 in Horner form with fused multiply-adds, then
// two exact scalings by 2^(n/2) and 2^(n - n/2).  Within 1 ulp of the
// correctly rounded exp over every float in [-104, 88.75]; 0 below (and
// for -inf), +inf above, NaN kept.  A fixed sequence of IEEE operations,
// so a host restatement gives the same bits (the reference's f32::exp is
// the platform libm, which differs from any device exp in the last bit).
__device__ __forceinline__ float rce_exp(float x) {
    if (!(x > -104.0f)) return x != x ? x : 0.0f;
    if (x > 88.75f) return __builtin_inff();
    const float n = __builtin_rintf(x * 0x1.715476p+0f);
    float r = __builtin_fmaf(-n, 0x1.62e4p-1f, x);
    r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0x1p-1f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int ni = (int)n, e1 = ni / 2, e2 = ni - e1;
    const float s1 = __uint_as_float((uint32_t)(e1 + 127) << 23), s2 = __uint_as_float((uint32_t)(e2 + 127) << 23);
    return (p * s1) * s2;
}

// Reductions over the 64 lanes of a wave as the balanced pairwise tree in
// lane order (the tree a butterfly over lane xor 1, 2, 4, ..., 32 forms):
// levels 1-4 by DPP within rows of 16 lanes (quad permutes [1,0,3,2] and
// [2,3,0,1], then the half-row and row mirrors, each of which pairs a lane
// with one that holds the other half's partial), levels 5-6 from the four
// rows' partials read as scalars: (r0 + r1) + (r2 + r3).  Every lane gets
// the same value, with no trip through the LDS crossbar.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float rdlane_f32(float x, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}
__device__ __forceinline__ float wave_sum(float v) {
    v = v + dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
    v = v + dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
    v = v + dpp_f32<0x141>(v);  // row_half_mirror: the other quad of the 8
    v = v + dpp_f32<0x140>(v);  // row_mirror: the other 8 of the row
    const float r0 = rdlane_f32(v, 0), r1 = rdlane_f32(v, 16), r2 = rdlane_f32(v, 32), r3 = rdlane_f32(v, 48);
    const float s01 = r0 + r1, s23 = r2 + r3;
    return s01 + s23;
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x141>(v));
    v = fmaxf(v, dpp_f32<0x140>(v));
    const float r0 = rdlane_f32(v, 0), r1 = rdlane_f32(v, 16), r2 = rdlane_f32(v, 32), r3 = rdlane_f32(v, 48);
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// The reference's silu (rce-tinyllama/src/lib.rs L164-166, rce-qwen36-moe
// L459-461): x * sigmoid(x) with exp's argument kept non-positive, exp
// being rce_exp.
__device__ __forceinline__ float silu_ref(float x) {
    if (x >= 0.0f) {
        const float e = rce_exp(-x);
        return x / (1.0f + e);
    }
    const float e = rce_exp(x);
    const float t = x * e;
    return t / (1.0f + e);
}

// Fused forms of the single-token decode GEMV, used by the decode step
// (llama.cpp).  FX_SEG: the grid is split into up to three segments, each a
// weight of the same format and width with its own output (the q, k and v
// projections of one input in one launch; one segment = the plain GEMV).
// FX_RESIDUAL: out[j] = res[j] + row_sum_j, the residual add that follows
// the attention-output and down projections (res may alias out).
// FX_SWIGLU: every block computes the same rows of w[0] (gate) and w[1]
// (up) and writes silu(gate_j) * up_j.  FX_NORM (with FX_SEG or
// FX_SWIGLU): the input is the residual stream x and every block forms
// rms_norm(x, norm_w, eps) itself (rce-tinyllama L158-163) before the
// products: the sum of squares over tasks of 8 consecutive values (one
// sequential fold per task, tasks t and t + NT on thread t, then a fixed
// tree over the block), inv = 1 / sqrt(sum / n + eps), value (x * inv) * w.
enum : int { FX_SEG = 1, FX_RESIDUAL = 2, FX_SWIGLU = 3, FX_NORM = 8 };
// Plain launches only: the Q8 activations were quantized beforehand into
// GemvFx::preq (launch_gemv_q8_pre); blocks read their tokens' slices.
constexpr int FX_PREQ = 16;

struct GemvFx {
    DevWeight w2, w3;      // FX_SEG: segments 1 and 2; FX_SWIGLU: w2 = up
    float *out2, *out3;    // FX_SEG: their outputs
    unsigned blk2, blk3;   // FX_SEG: first block of segments 1 and 2
    const unsigned char *preq;  // FX_PREQ: the quantized activations of all preq_t tokens
    int preq_t;
    const float *res;      // FX_RESIDUAL
    const float *norm_w;   // FX_NORM
    float eps;             // FX_NORM
    int *pos;              // FX_SEG, non-null: ends a decode step (see FxLaunch)
    int *status;
    int ctx_len;
};

struct FxLaunch {
    int kind = FX_SEG;     // FX_SEG, FX_RESIDUAL, FX_SWIGLU, optionally | FX_NORM
    int nw = 1;            // weights used (FX_SEG 1..3, FX_SWIGLU 2, FX_RESIDUAL 1)
    DevWeight w[3]{};
    float *out[3]{};
    const float *res = nullptr;
    const float *norm_w = nullptr;
    float eps = 0.0f;
    // FX_SEG: when pos is given, one thread also ends a decode step, as
    // launch_rms_norm does with pos (unless status[2] marks the step
    // skipped: status[0] = 2 if pos[0] >= ctx_len, then pos[0] += 1); no
    // other kernel of the step may follow that reads pos.
    int *pos = nullptr;
    int *status = nullptr;
    int ctx_len = 0;
};

// Whether the fused forms exist for (dtype, n_cols, mode); with_norm: also
// with FX_NORM (the input row must be at most 16 values per thread).
bool gemv_fx_supports(uint32_t dtype, size_t n_cols, int mode, bool with_norm = false);
// One token; all weights of one launch share dtype and n_cols (and, for
// FX_SWIGLU, n_rows).
// `geom` overrides the launch shape (tuning only; nullptr = pick).
hipError_t launch_gemv_fx(const FxLaunch &f, const float *a, int mode, hipStream_t s,
                          const GemvGeom *geom = nullptr);
// Per-format launchers of the fused forms (gemv_<format>.hip).
hipError_t launch_gemv_fx_q4_0(const FxLaunch &f, const GemvGeom &g, const float *a, int mode, hipStream_t s);
hipError_t launch_gemv_fx_q8_0(const FxLaunch &f, const GemvGeom &g, const float *a, int mode, hipStream_t s);
hipError_t launch_gemv_fx_q4_k(const FxLaunch &f, const GemvGeom &g, const float *a, int mode, hipStream_t s);
hipError_t launch_gemv_fx_q5_k(const FxLaunch &f, const GemvGeom &g, const float *a, int mode, hipStream_t s);
hipError_t launch_gemv_fx_q6_k(const FxLaunch &f, const GemvGeom &g, const float *a, int mode, hipStream_t s);
hipError_t launch_gemv_fx_q5_0(const FxLaunch &f, const GemvGeom &g, const float *a, int mode, hipStream_t s);
hipError_t launch_gemv_fx_q4_1(const FxLaunch &f, const GemvGeom &g, const float *a, int mode, hipStream_t s);
hipError_t launch_gemv_fx_q3_k(const FxLaunch &f, const GemvGeom &g, const float *a, int mode, hipStream_t s);

// ---- decode step (decoder.hip) ----
// The decode step's status words: status[0] the first error code since the
// last check (1 a token id out of range, 2 a position past the cache),
// status[1] the number of steps skipped for a bad token id since then,
// status[2] 1 while the current step is such a skipped step (its cache row
// and position advance are left out), else 0.
// x = dequant_row(w, *row_dev) (QuantWeight::dequant_row), status[2] = 0;
// an id outside [0, n_rows) writes nothing to x, sets status[0] = 1 (if
// still 0) and status[2] = 1 and counts the step in status[1].
hipError_t launch_embed_row(const DevWeight &w, const int32_t *row_dev, float *x, int *status, hipStream_t s);
// out = rms_norm(x, w, eps) (rce-tinyllama L158-163) over n values.  When
// pos is given, one thread also ends a decode step unless status[2] marks
// it skipped: status[0] = 2 if pos[0] >= ctx_len, then pos[0] += 1 (no
// other kernel of the step may follow that reads pos).
hipError_t launch_rms_norm(const float *x, const float *w, size_t n, float eps, float *out, int *pos, int ctx_len,
                           int *status, hipStream_t s);
// RoPE of q (n_q heads) and k (n_kv heads) at position pos[0], append of k, v to
// the layer's caches, and per query head the reference's online-softmax
// attention over positions 0..pos (rce-op-attn L107-151, L185-251).
// qkv: [q (n_q * d_head) | k (n_kv * d_head) | v (n_kv * d_head)];
// rope_cs: [ctx_len][rope_dim / 2] (cos, sin) pairs; caches of
// ceil(ctx_len / 64) * 64 positions, values [position][n_kv * d_head], keys
// in 64-position tiles (decoder.hip); att: [n_q * d_head].  skip (may be
// null): when skip[0] != 0 the step is a skipped one and appends nothing to
// the caches.
hipError_t launch_attention(const float *qkv, const float *rope_cs, float *k_cache, float *v_cache,
                            const int *pos, int ctx_len, int n_q, int n_kv, int d_head, int rope_dim,
                            float scale, float *att, const int *skip, hipStream_t s);
// d_head 64 or 128, rope_dim even and <= d_head, and one layer's cache
// under 2 GiB (the kernel addresses it with 32-bit offsets).
bool attention_supports(int d_head, int rope_dim, size_t ctx_len, size_t n_kv);
// h = silu(g) * u, x = x + o: the unfused forms.
hipError_t launch_swiglu(const float *g, const float *u, float *h, size_t n, hipStream_t s);
hipError_t launch_add_inplace(float *x, const float *o, size_t n, hipStream_t s);

// Decode kernels available for (dtype, n_cols, mode 0 EXACT / 1 Q8).
bool gpu_supports(uint32_t dtype, size_t n_cols, int mode);

// Device layout of a weight: fills layout, row_stride, planes and
// group_stride of `dw` (dtype, n_rows, n_cols already set) and
// returns the device bytes it needs.
size_t plan_layout(DevWeight &dw);
// Zero bytes the allocation holds past the layout: a decode launch's last
// block reads whole tiles of rows, up to 16 x (1024 / units per row) rows
// (64-row groups for the interleaved layouts) past n_rows, instead of
// clamping each row; those rows' sums are never folded.  Sub-views end
// inside their parent, so the parent's padding covers them.
size_t layout_pad_bytes(const DevWeight &dw);
// GGUF bytes (row-major rows of blocks) -> the device layout of `dw`.
void relayout_host(const uint8_t *src, const DevWeight &dw, uint8_t *dst);

hipError_t launch_f16_to_f32(const uint16_t *src, float *dst, size_t n, hipStream_t s);
// mode 0: the reference's f32 order; mode 1: Q8 activations.  `geom`
// overrides the shape the library picks (tuning only; nullptr = pick).
hipError_t launch_gemv(const DevWeight &w, const float *a, size_t t_rows, float *out, int mode,
                       hipStream_t s, const GemvGeom *geom = nullptr);
// Q8 with several tokens: the activations are quantized once into `ws`
// (act_lds_bytes(n_cols, t_rows) bytes, 16-byte aligned) by one small
// kernel instead of by every block; the results are the same bits.  Falls
// back to launch_gemv where the pre-quantized form has no kernel.
hipError_t launch_gemv_q8_pre(const DevWeight &w, const float *a, size_t t_rows, float *out, void *ws,
                              hipStream_t s);
bool gemv_q8_pre_supports(uint32_t dtype, size_t n_cols, size_t t_rows);
// The int8 matrix-core form of the same (gemv_q8_mfma.hip): Q4_0 / Q8_0,
// n_cols a multiple of 256, 2 or more tokens; preq as k_quantize_act writes
// it (the ActLds layout of t_rows tokens).  Chosen where it is faster
// (gemv_q8_mfma_preferred); RCE_QMM_Q8_MFMA=0 turns it off, =2 forces it
// wherever it applies (same bits either way).
bool gemv_q8_mfma_supports(uint32_t dtype, size_t n_cols, size_t t_rows);
bool gemv_q8_mfma_preferred(size_t n_cols, size_t t_rows);
bool gemv_q8_mfma_enabled();
bool gemv_q8_mfma_forced();
hipError_t launch_gemv_q8_mfma(const DevWeight &w, const unsigned char *preq, size_t t_rows, float *out, hipStream_t s);
GemvGeom pick_gemv_geom(const DevWeight &w, size_t t_rows, int mode);
// Per-format launchers (gemv_<format>.hip), shape already chosen.
hipError_t launch_gemv_q4_0(const DevWeight &w, const GemvGeom &g, const float *a, size_t t_rows, float *out,
                            int mode, hipStream_t s);
hipError_t launch_gemv_q8_0(const DevWeight &w, const GemvGeom &g, const float *a, size_t t_rows, float *out,
                            int mode, hipStream_t s);
hipError_t launch_gemv_q4_k(const DevWeight &w, const GemvGeom &g, const float *a, size_t t_rows, float *out,
                            int mode, hipStream_t s);
hipError_t launch_gemv_q5_k(const DevWeight &w, const GemvGeom &g, const float *a, size_t t_rows, float *out,
                            int mode, hipStream_t s);
hipError_t launch_gemv_q6_k(const DevWeight &w, const GemvGeom &g, const float *a, size_t t_rows, float *out,
                            int mode, hipStream_t s);
hipError_t launch_gemv_q5_0(const DevWeight &w, const GemvGeom &g, const float *a, size_t t_rows, float *out,
                            int mode, hipStream_t s);
hipError_t launch_gemv_q4_1(const DevWeight &w, const GemvGeom &g, const float *a, size_t t_rows, float *out,
                            int mode, hipStream_t s);
hipError_t launch_gemv_q3_k(const DevWeight &w, const GemvGeom &g, const float *a, size_t t_rows, float *out,
                            int mode, hipStream_t s);
hipError_t launch_dequant_row(const DevWeight &w, size_t row, float *out, hipStream_t s);
// F32 / F16 / BF16 and I2_S (gemv_chain.hip): the reference's one chain
// (I2_S: two chains) per row, in both modes (there is no Q8 form of these
// weights).
hipError_t launch_gemv_chain(const DevWeight &w, const float *a, size_t t_rows, float *out, hipStream_t s);
constexpr size_t CHAIN_MAX_K = 16384;  // the row-chain kernels stage a token's activations in 64 KB of LDS
constexpr size_t CHAIN_STAGE = 12;     // F32 / F16 / BF16 rows are padded to whole stages of 12 zero chunks
__host__ __device__ inline bool is_whole_element(uint32_t dtype) { return dtype == T_F32 || dtype == T_F16 || dtype == T_BF16; }
__host__ __device__ inline bool is_row_chain(uint32_t dtype) { return is_whole_element(dtype) || dtype == T_I2_S; }
// Multiply-free block formats (gemv_ternary.hip): Q1_0, Q2_0, STQ1_0, one
// token per thread, the same kernel in both modes.
__host__ __device__ inline bool is_ternary_block(uint32_t dtype) {
    return dtype == T_Q1_0 || dtype == T_Q2_0 || dtype == T_STQ1_0;
}
hipError_t launch_gemv_ternary(const DevWeight &w, const GemvGeom &g, const float *a, size_t t_rows, float *out,
                               hipStream_t s);

// Prefill GEMM on the matrix cores (gemm_f16.hip): out[M, n_rows] =
// A[M, n_cols] . W^T, A binary16, W dequantized to binary16 tiles.
bool gemm_supports(uint32_t dtype, size_t n_cols);
// Q8_0 and Q6_K weights on the same kernel (plain GEMM, 128 x 64 tiles,
// K % 256 == 0).
bool gemm_q8_supports(uint32_t dtype, size_t n_cols);
bool gemm_shape_ok(size_t a_rows, const DevWeight &w);
// bm: output tile rows, 64 (tile 64 x 128), 96 (96 x 128) or 128 (128 x 64);
// 0 = by M.
hipError_t launch_gemm_f16(const DevWeight &w, const void *a_f16, size_t M, float *out, hipStream_t s, int bm = 0);
// The other formats' prefill GEMM (gemm_gen.hip): Q8_0, Q5_0, Q4_1, F16 (K
// a multiple of 64), Q5_K, Q6_K (K a multiple of 256); nibble_forms also
// admits Q4_0 and Q4_K (the same generic form, for cross-checks).  A must
// be 16-byte aligned.
bool gemm_gen_supports(uint32_t dtype, size_t n_cols);
hipError_t launch_gemm_gen(const DevWeight &w, const void *a_f16, size_t M, float *out, hipStream_t s,
                           bool nibble_forms = false);
// The tile rows the GEMM uses for M = rows_hint (plain) or for a mean of
// rows_hint rows per expert (grouped).
int gemm_tile_rows(size_t rows_hint, bool grouped);
// f32 activations -> binary16 (round to nearest even) for the GEMM.
hipError_t launch_f32_to_f16(const float *src, void *dst, size_t n, hipStream_t s);

// ---- grouped experts (moe.hip, gemm_f16.hip) ----
// A row tile of the grouped GEMM: expert e, slots r0 .. r0 + rows - 1.
struct MoeTile {
    int e, r0, rows, pad;
};

// Which output tile (row tile mt, column tile nt) block blockIdx.x of a
// prefill GEMM computes; false: none (the block returns before any barrier).
// Blocks are dispatched round-robin over the 8 XCDs (block L to XCD L % 8),
// each XCD with its own L2.
//   Plain (n_tiles_dev == nullptr; grid = m_tiles * column tiles): XCD x
//   takes a contiguous range of tiles in (nt, mt) order, so the m-tiles
//   sharing W rows run on one XCD.
//   Grouped (grid = grouped_grid(m_tiles, column tiles)): only the first
//   n_tiles_dev[0] row tiles exist; their V = n_tiles_dev[0] * column tiles
//   blocks are numbered in (mt, nt) order and XCD x takes the range
//   [x P, (x + 1) P), P = ceil(V / 8): each expert's tiles run on one or two
//   XCDs, whose L2 then holds that expert's activation rows (with the
//   (nt, mt) order every XCD read every expert's rows: 1.4x the HBM bytes
//   of the expert weights on configs[3], 1.1x with this one, at the same
//   speed), and blocks past V return at once.
__host__ __device__ inline int grouped_grid(int m_tiles, int col_tiles) { return (m_tiles * col_tiles + 7) / 8 * 8; }
#ifdef __HIPCC__
template <int BN>
__device__ __forceinline__ bool tile_of_block(size_t n_rows, int m_tiles, const int *n_tiles_dev, int &mt, int &nt) {
    const int G = gridDim.x, L = blockIdx.x;
    if (!n_tiles_dev) {
        const int logical = (G % 8 == 0) ? (L % 8) * (G / 8) + L / 8 : L;
        mt = logical % m_tiles;
        nt = logical / m_tiles;
        return true;
    }
    const int nn = (int)((n_rows + BN - 1) / BN), V = n_tiles_dev[0] * nn, P = (V + 7) / 8;
    const int v = (L % 8) * P + L / 8;
    if (L / 8 >= P || v >= V) return false;
    mt = v / nn;
    nt = v % nn;
    return true;
}
#endif
// Stable grouping of pairs p = token * top_k + j by expert ids[p]:
// offs[n_expert + 1], slot_of_pair[n_pairs] (-1: id out of range),
// tok_of_slot[n_pairs], tiles[n_pairs / bm + n_expert] (bm-row pieces of
// each expert's slots), n_tiles[1], status[1] (1: an id was out of range).
// With x16 non-null the same launch also writes x16[i] = binary16(x[i]),
// i < n_x.
hipError_t launch_moe_group(const int32_t *ids, size_t n_pairs, int top_k, int n_expert, int bm, int *offs,
                            int *slot_of_pair, int *tok_of_slot, MoeTile *tiles, int *n_tiles, int *status,
                            const float *x, void *x16, size_t n_x, hipStream_t s);
// xg[s, :] = x[tok_of_slot[s], :] for s < n_slots (device count)
hipError_t launch_gather_rows(const float *x, const int *tok_of_slot, const int *n_slots_dev, size_t max_slots,
                              size_t d, float *xg, hipStream_t s);
hipError_t launch_silu_inplace(float *h, const int *n_slots_dev, size_t max_slots, size_t d, hipStream_t s);
// SwiGLU experts: g = silu(g) * u over the first n_slots (device count) slots,
// in place.
hipError_t launch_swiglu_slots(float *g, const float *u, const int *n_slots_dev, size_t max_slots, size_t d,
                               hipStream_t s);
// out[t, :] = sum_j gate_w[t, j] * y[slot_of_pair[t * top_k + j], :], j in order, from +0.0
hipError_t launch_moe_combine(const float *y, const int *slot_of_pair, const float *gate_w, size_t t_rows, int top_k,
                              size_t d, float *out, hipStream_t s);
// What the grouped GEMM stores for output element o with f32 sum v:
// v (f32 out), binary16 silu(v), or binary16 silu(aux[o]) * v (aux: the
// f32 gate products of the same slots, SwiGLU).
enum GemmEpilogue { GEPI_F32 = 0, GEPI_SILU_F16 = 1, GEPI_SWIGLU_F16 = 2 };
// Grouped GEMM: for every tile (expert e, slots r0 ..): out[r0 + m, :] =
// epi(A[gather ? gather[r0 + m] : r0 + m, :] . wtab[e]^T).  `w` gives the
// dtype and shape shared by all experts; wtab is a device array of
// DevWeight; a_rows: rows of A (bounds the loads); max_tiles bounds
// n_tiles_dev[0].
hipError_t launch_gemm_f16_grouped(const DevWeight &w, const DevWeight *wtab, const void *a_f16, size_t a_rows,
                                   const int *gather, const MoeTile *tiles, const int *n_tiles_dev, int max_tiles,
                                   int bm, int epi, void *out, const float *aux, hipStream_t s);
// The same for the other formats (gemm_gen.hip: gemm_gen_supports' dtypes),
// 128 x 64 output tiles: any tile table whose tiles hold at most 128 rows.
hipError_t launch_gemm_gen_grouped(const DevWeight &w, const DevWeight *wtab, const void *a_f16, size_t a_rows,
                                   const int *gather, const MoeTile *tiles, const int *n_tiles_dev, int max_tiles,
                                   int epi, void *out, const float *aux, hipStream_t s);

}  // namespace rce_qmm
