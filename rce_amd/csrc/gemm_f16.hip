// gemm_f16.hip -- prefill-shaped GEMM of the GGUF quantized-matmul path on
// the CDNA4 matrix cores: out[M, N] = A[M, K] . W[N, K]^T with W in GGUF
// Q4_K, Q5_K, Q4_0, Q4_1, Q5_0, Q8_0 or Q6_K blocks (the last two in
// 128 x 64 tiles only), dequantized to binary16 MFMA
// fragments in registers and contracted with v_mfma_f32_32x32x16_f16 (f32
// accumulation).
//
// Tiling.  A block owns a BM x BN (M x N) output tile: 128 x 64 or 64 x 128
// (8192 outputs), so a 512 x 4096 product is 256 tiles, one per CU; or
// 96 x 128 for the grouped mode when experts get about 64 rows each (65-96
// rows in one tile instead of a 64-row tile and a mostly empty second one:
// the configs[3] MoE's W2 then needs one round of tiles over the CUs, not
// two).  The 64 x 128 tile moves a third less data into LDS per flop than
// 128 x 64 (8 KB of activations + 4.5 KB of weights per chunk instead of
// 16 + 2.25).  A block whose tile holds at most 64 (or 96) rows runs the
// 64-row (96-row) body over the same columns (k_gemm_f16 below).
// K runs in chunks of 64 (four MFMA k-steps of 16).  The block has ten waves:
//   * eight compute waves: wave w = 2*kq + t computes k-step kq of every
//     chunk for the BM x BN/2 sub-tile of columns BN/2 * t.. (RB x CB MFMA
//     blocks of 32 x 32, four in all): per chunk it reads RB A fragments
//     from LDS, dequantizes its CB W fragments itself from the raw GGUF
//     nibbles in LDS (each W nibble is dequantized by exactly one wave; no
//     B tile is written), and issues four MFMAs.  The four k-step partial
//     sums of each output are added at the end through LDS in a fixed order
//     (deterministic);
//   * two producer waves issue every global -> LDS load (the compute waves
//     read each chunk's {scale, bias} word from the weight group in LDS
//     themselves).  A load instruction can hold its wave up while the CU's
//     memory pipeline is busy (each 1 KB load occupies it ~20 cycles), so
//     the loads live in waves that do nothing else and the
//     MFMA/dequantization waves never stall on them.
// One barrier per chunk.  The producers wait (s_waitcnt vmcnt, one
// compile-time immediate per chunk position) for the data the compute
// waves read next before joining it.
//
// Global -> LDS traffic uses buffer_load_dwordx4 ... lds (16 bytes per lane,
// no registers; a uniform scalar offset per chunk).  Its throughput is set
// by the 64-byte segments an instruction touches, so every load covers
// whole segments:
//   * A: 8 rows x 128 bytes (one chunk of a row) per instruction, stored
//     XOR-swizzled (16-byte column g of row r at slot g ^ f(r),
//     f(r) = (r & 7) ^ ((r >> 3) & 1)) so the MFMA fragment reads (32 rows,
//     one column) are bank-conflict free whether 8 or 16 lanes are served
//     per LDS cycle; NS - 1 chunks ahead;
//   * W: per scale group (four chunks: one Q4_K super-block, eight Q4_0
//     blocks) each row's 2 x 64 bytes of nibbles (16-byte pieces rotated by
//     (row >> 2) & 3) and its scale words (Q4_0: the 16-byte header of f16
//     block scales; Q4_K: the 32 bytes of {d*sc, -dmin*m} pairs formed at
//     upload; the other formats below), loaded GA groups ahead.
// The compute waves read chunk c+1's A fragments and chunk c+2's nibbles
// while chunk c's MFMAs and chunk c+1's dequantization run.
//
// K order.  Any permutation of K inside a chunk is a valid contraction if A
// and W use the same one.  Lane half h (= lane / 32) of k-step kq holds the
// nibbles of the 8 bytes 8h..8h+7 of one 16-byte piece (low nibbles for
// even kq, high for odd); the A fragment is the matching 8 K positions:
//   Q4_K (64-group q of a super-block; positions 0..31 = low nibbles of qs
//   bytes 0..31, 32..63 = high; rce-op-qmm/src/lib.rs L354-385): kq 0, 1 =
//   low, high nibbles of bytes 0..15; kq 2, 3 = bytes 16..31;
//   Q4_0 (blocks 2q, 2q+1; block positions 0..15 = low nibbles of its 16
//   bytes, 16..31 = high; L496-522): kq 0, 1 = block 2q, kq 2, 3 = 2q+1.
//
// Dequantization (binary16: the "fp16-dequant MFMA" mode).  A nibble n
// becomes f16(1024 + n) by a byte permute with 0x64, minus 1024 (exact),
// then one packed f16 fma: Q4_K d1*n + (-min1) with d1 = f16(d*sc),
// min1 = f16(dmin*m) (the reference's scales, rounded to f16); Q4_0
// d*n + (-8d), which is d*(n - 8) exact before its single rounding.  The
// result differs from the reference's f32 order by the f16 rounding of the
// weights (normwise about 7e-4 at the Q4_K prefill shape; the stated budget
// is 2e-3) and is deterministic: each output's summation order is fixed.
#include "lds_limit.h"
#include "gemm_epilogue.h"
#include "qmm_internal.h"

#include <atomic>
#include <type_traits>

namespace rce_qmm {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// A lane's weight bytes of one k-step: l = 8 bytes (nibbles, or Q8_0's
// values, or Q6_K's ql); h = Q6_K's 8 qh bytes.
struct WRaw {
    u32x2 l, h;
};

constexpr int KC = 64;                           // K per chunk (four MFMA k-steps of 16)
constexpr int NC = 512;                          // compute threads (8 waves)
constexpr int NT = NC + 128;                     // + 2 producer waves
constexpr int NWBUF = 4, GA = 2;                 // W groups loaded GA groups ahead
// W buffer (g+GA) % NWBUF, refilled from iteration 4g, was last read for
// chunk 4(g+GA-NWBUF)+3 (iteration 4(g+GA-NWBUF)+1 < 4g).
static_assert(NWBUF >= GA + 1 && (NWBUF & (NWBUF - 1)) == 0, "W buffer ring");

// Output tile BM x BN: 128 x 64, 64 x 128, or 96 x 128 (grouped experts of
// 65-96 rows, in one row tile instead of a 64-row tile and a mostly empty
// second one).  Compute wave w = 2*kq + t holds RB x CB MFMA blocks of
// 32 x 32 (rows 32*rb, columns BN/2 * t + 32*cb).
// The weight format (below) sets the bytes of one scale group of the tile's
// columns in LDS (W_GROUP), the loads a producer issues for them at group
// position 0 (W_LOADS; at position 1 h_loads: the headers or scale pairs)
// and so the A stages that leave room for them (NS).  BN_ (0: the default
// above) sets the columns of the 64-row tile that a wider tile's block runs
// when it holds at most 64 rows (64 x 64 in a 128 x 64 launch).
template <int BM_, class Fmt, int BN_ = 0>
struct Tile {
    static constexpr int BM = BM_, BN = BN_ ? BN_ : (BM_ == 96 ? 128 : 8192 / BM_);
    // A stages (chunks), loaded NS - 1 ahead: six where the tile's LDS holds
    // them, else five
    static constexpr int pipe_lds(int ns) { return ns * BM * KC * 2 + NWBUF * Fmt::w_group(BN); }
    static constexpr int NS = pipe_lds(6) + BM * 4 <= 160 * 1024 ? 6 : 5;
    static constexpr int RB = BM / 32, CB = BN / 64;
    static constexpr int A_STAGE = BM * KC * 2;           // 16 KB / 8 KB
    static constexpr int A_LOADS = BM / 16;               // per producer per chunk (1 KB each)
    static constexpr int W_HALF = BN * 64;                // rows x 4 chunks x 16 B
    static constexpr int W_ROW_LOADS = BN / 16;           // loads of one 64-byte piece of every row
    static constexpr int W_LOADS = Fmt::w_loads(BN);      // per producer per group at position 0
    static constexpr int W_GROUP = Fmt::w_group(BN);
    static constexpr int OFF_W = NS * A_STAGE;
    static constexpr int PIPE_LDS = OFF_W + NWBUF * W_GROUP;
    static_assert(PIPE_LDS == pipe_lds(NS), "LDS layout");
    // the partial sums of every wave for one column block cb at a time
    static constexpr int RED_LDS = 8 * RB * 16 * 64 * 4;
    static constexpr int LDS = PIPE_LDS > RED_LDS ? PIPE_LDS : RED_LDS;
    static_assert(LDS + BM * 4 <= 160 * 1024, "LDS budget");
    // W group g must be complete at the barrier of chunk 4g-3 (the compute
    // waves read its bytes and scale words from chunk 4g-2 on): its last
    // load (iteration 4(g-GA)+1) precedes the loads of A chunk 4g-2
    // (iteration 4g-2-(NS-1)).
    static_assert(4 * GA >= NS + 2, "W groups loaded too late for the stage depth");
    static_assert(NS >= 3, "stage ring");
    static_assert(RB >= 2 && RB <= 4 && CB >= 1 && CB <= 2 && 2 * RB <= 8,
                  "2 to 4 row blocks (the dequantization is spread over the first two), 1 or 2 column blocks "
                  "per compute wave; a column block's 2 RB output blocks finished by as many waves");
    // Producer loads of iteration `it`, in order: the W loads of position
    // it % 4 (row halves at position 0, headers at 1), then the A loads of
    // chunk it + NS - 1.
    static constexpr int w_loads(int q) { return (q & 3) == 0 ? W_LOADS : (q & 3) == 1 ? Fmt::h_loads(BN) : 0; }
    // vmcnt immediate for a producer's barrier at chunk position q: the
    // loads it issued after chunk c+1's A loads (iterations c+3-NS .. c-1).
    static constexpr int vm_after(int q) {
        int n = 0;
        for (int d = 1; d <= NS - 3; d++) n += A_LOADS + w_loads(q - d);
        return n;
    }
};

__device__ __forceinline__ half2v as_h2(uint32_t u) {
    half2v h;
    __builtin_memcpy(&h, &u, 4);
    return h;
}

// One 16-byte load from global memory straight into LDS at
// lds_wave + 16 * lane (lds_wave must be the same for the whole wave).
__device__ __forceinline__ void load_lds16(const void *g, unsigned char *lds_wave) {
    __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1))) *)g,
                                     (void __attribute__((address_space(3))) *)lds_wave, 16, 0, 0);
}

// Buffer load of 16 bytes per lane straight into LDS at lds_wave + 16 * lane:
// byte voff (per lane) + soff (uniform) of the buffer described by r.
__device__ __forceinline__ void buf_load_lds16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                               unsigned char *lds_wave) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds_wave, 16, voff, soff, 0, 0);
}
// Raw byte buffer of n bytes (gfx9 descriptor word 3 for untyped access).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t byte_buffer(const void *base, uint32_t n) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)n, 0x00020000);
}

// LDS accesses of the pipelined loop are inline ds_read / ds_write: the
// compiler counts the global->LDS loads as writes to all of LDS and would
// wait for every load in flight before each LDS access (the whole
// pipeline).  Their completion is waited for explicitly instead
// (s_waitcnt lgkmcnt(0), then pin below).  OFF is the instruction's
// immediate byte offset.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
template <int OFF>
__device__ __forceinline__ half8 lds_read_frag(uint32_t a) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    half8 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(OFF) : "memory");
    return v;
}
template <int OFF>
__device__ __forceinline__ uint32_t lds_read_u8(uint32_t a) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    uint32_t v;
    asm volatile("ds_read_u8 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(OFF) : "memory");
    return v;
}
template <int OFF>
__device__ __forceinline__ uint32_t lds_read_u16(uint32_t a) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    uint32_t v;
    asm volatile("ds_read_u16 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(OFF) : "memory");
    return v;
}
template <int OFF>
__device__ __forceinline__ uint32_t lds_read4(uint32_t a) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(OFF) : "memory");
    return v;
}
template <int OFF>
__device__ __forceinline__ u32x2 lds_read8(uint32_t a) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    u32x2 v;
    asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(OFF) : "memory");
    return v;
}
// After s_waitcnt lgkmcnt(0): an empty asm that "redefines" a register
// the reads above filled, so no use of it can move ahead of the wait.
template <class T>
__device__ __forceinline__ void pin(T &r) {
    asm volatile("" : "+v"(r));
}
// pin the low word of a pair only (the high word never written)
__device__ __forceinline__ void pin_lo(u32x2 &r) {
    uint32_t x = r.x;
    asm volatile("" : "+v"(x));
    r.x = x;
}

// s_waitcnt vmcnt(N) (gfx9 encoding; expcnt and lgkmcnt not waited for),
// then a barrier without the memory fence __syncthreads would add (that
// fence waits for every load in flight, the whole pipeline).
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
    __builtin_amdgcn_s_barrier();
}

// Four bytes of x (nibbles masked to 0..15, or Q8_0's int8 values offset to
// 0..255) as two f16 pairs in byte order: value = s * (n - OFF + 1024) + b
// (packed f16 fma, one rounding), with sb = f16 {s, b}.  Eight VALU ops;
// two calls make one MFMA fragment.
template <int OFF = 1024>
__device__ __forceinline__ void dequant4(uint32_t x, uint32_t sb, half2v &lo, half2v &hi) {
    const uint32_t K64 = 0x64646464u;
    const half2v m1024 = {(_Float16)(-(float)OFF), (_Float16)(-(float)OFF)};
    const half2v p = as_h2(sb);
    const half2v sc = __builtin_shufflevector(p, p, 0, 0), bias = __builtin_shufflevector(p, p, 1, 1);
    // byte pairs (n, 0x64): f16 bits 0x64nn = 1024 + n
    const uint32_t p0 = __builtin_amdgcn_perm(x, K64, 0x00050004u);
    const uint32_t p1 = __builtin_amdgcn_perm(x, K64, 0x00070006u);
    lo = __builtin_elementwise_fma(as_h2(p0) + m1024, sc, bias);
    hi = __builtin_elementwise_fma(as_h2(p1) + m1024, sc, bias);
}

__device__ __forceinline__ half8 join8(half2v a, half2v b, half2v c, half2v d) {
    return half8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

// --- weight formats ----------------------------------------------------------
// A scale group is four chunks.  Per row it is NH 64-byte pieces of weight
// bytes and an HDR-byte header:
//   half_off(w, g, hf): byte offset inside a row of piece hf of group g;
//   hdr_off(w, g): byte offset of group g's header;
//   half_of(q, kq), piece_of(q, kq): the piece and its 16-byte part (0..3)
//     holding k-step kq of chunk q of the group;
//   acol(kq): the 16-byte A column (0..7 within the chunk) of lane half 0;
//   sidx(kq): which of a column's two scale sets k-step kq uses;
//   the compute waves read chunk q's {scale, bias} word straight from the
//     group's header in LDS (at hoff(BN) + column * CST + sbyte(q, kq)),
//     SBW bytes zero-extended: an f16 d read as {d, +0}, or a pair the
//     upload formed (the device layouts of Q4_K, Q5_K, Q6_K), so no wave
//     spends a step forming scales.

// Q4_K: halves = qs bytes 0..15 (plane 1) and 16..31 (plane 2) of the
// super-block's four 64-groups; header = the super-block's eight f16
// {d sc_j, -(dmin m_j)} pairs (plane 4, formed at upload from d, dmin and
// the 12 scale bytes); scale set 0 / 1 = the low / high nibble sub-block
// of each 64-group, so chunk q set si is pair 2q + si.
struct Q4K {
    static constexpr int NH = 2, OFF = 1024, HDR = 32, SBW = 4, CST = HDR;
    static constexpr bool IL64 = false, HB = false;
    static constexpr int w_group(int bn) { return NH * bn * 64 + bn * HDR; }
    static constexpr int w_loads(int bn) { return bn / 16 * NH / 2; }
    static constexpr int h_loads(int bn) { return bn / 64; }  // 32 rows x 32 bytes per load
    static constexpr int hoff(int bn) { return NH * bn * 64; }
    __device__ static uint32_t vals(uint32_t x, int nsh) { return (x >> nsh) & 0x0F0F0F0Fu; }
    __device__ static size_t half_off(const DevWeight &w, int g, int hf) {
        return (hf ? w.plane2 : w.plane1) + 64 * (size_t)g;
    }
    __device__ static size_t hdr_off(const DevWeight &w, int g) { return w.plane4 + 32 * (size_t)g; }
    __device__ static int half_of(int, int kq) { return kq >> 1; }
    __device__ static int piece_of(int q, int) { return q; }
    __device__ static int acol(int kq) { return (kq & 1) * 4 + (kq >> 1) * 2; }
    __device__ static int sidx(int kq) { return kq & 1; }
    __device__ static int sbyte(int q, int kq) { return 4 * (2 * q + sidx(kq)); }
};

// Q5_K (LAYOUT_SPLIT_Q5_K): Q4_K's halves, header and scales, plus per row
// and group the 32 bytes of fifth bits of its four 64-groups (plane 3: one
// 8-byte word per 64-group, bit l / 32 + l = the fifth bit of position l /
// 32 + l), loaded with the halves.  A lane's eight weights of k-step kq of
// chunk q are positions 32(kq & 1) + 16(kq / 2) + 8h .. +7 of 64-group q:
// their fifth bits are byte 4(kq & 1) + 2(kq / 2) + h of that word.
// u = nibble | bit << 4 in 0..31, value d1 u - min1 as for Q4_K.
struct Q5K : Q4K {
    static constexpr bool HB = true;
    static constexpr int w_group(int bn) { return NH * bn * 64 + bn * HDR + bn * 32; }
    static constexpr int w_loads(int bn) { return bn / 16 * NH / 2 + bn / 64; }
    // the row's 32 fifth-bit bytes of group g, and the byte (of lane half 0)
    // of chunk q, k-step kq
    __device__ static size_t hb_src(const DevWeight &w, int g) { return w.plane3 + 32 * (size_t)g; }
    __device__ static int hb_off(int q, int kq) { return 8 * q + 4 * (kq & 1) + 2 * (kq >> 1); }
};

// Q4_0: halves = the 16-byte nibble runs of blocks 8g..8g+3 and 8g+4..8g+7;
// header = their eight f16 scales; scale set 0 / 1 = block 2q / 2q+1.
// f16(1024 + n) - 1032 = n - 8 exactly, then (n - 8) d + 0 rounds once
// (the chunk's {scale, bias} word is the header's f16 d read
// zero-extended, {d, +0}).
struct Q40 {
    static constexpr int NH = 2, OFF = 1032, HDR = 16, SBW = 2, CST = HDR;
    static constexpr bool IL64 = false, HB = false;
    static constexpr int w_group(int bn) { return NH * bn * 64 + bn * HDR; }
    static constexpr int w_loads(int bn) { return bn / 16 * NH / 2; }
    static constexpr int h_loads(int) { return 1; }  // BN / 2 lanes of 16 bytes
    static constexpr int hoff(int bn) { return NH * bn * 64; }
    __device__ static uint32_t vals(uint32_t x, int nsh) { return (x >> nsh) & 0x0F0F0F0Fu; }
    __device__ static size_t half_off(const DevWeight &w, int g, int hf) {
        return w.plane1 + 128 * (size_t)g + 64 * hf;
    }
    __device__ static size_t hdr_off(const DevWeight &, int g) { return 16 * (size_t)g; }
    __device__ static int half_of(int q, int) { return q >> 1; }
    __device__ static int piece_of(int q, int kq) { return 2 * (q & 1) + (kq >> 1); }
    __device__ static int acol(int kq) { return 2 * kq; }
    __device__ static int sidx(int kq) { return kq >> 1; }
    // header byte of the f16 d of chunk q's block 2q + sidx(kq)
    __device__ static int sbyte(int q, int kq) { return 4 * q + 2 * sidx(kq); }
};


// Q4_1 (LAYOUT_SPLIT_Q4_1): Q4_0's nibble halves; header = the eight
// blocks' 4-byte {d, m} words (rce-op-qmm/src/lib.rs L615-645: value
// d q + m), which are the {scale, bias} words as they stand: the weight is
// d n + m rounded once to binary16.
struct Q41 : Q40 {
    static constexpr int OFF = 1024, HDR = 32, SBW = 4, CST = HDR;
    static constexpr int w_group(int bn) { return NH * bn * 64 + bn * HDR; }
    static constexpr int h_loads(int bn) { return bn / 64; }  // 32 rows x 32 bytes per load
    __device__ static size_t hdr_off(const DevWeight &, int g) { return 32 * (size_t)g; }
    __device__ static int sbyte(int q, int kq) { return 4 * (2 * q + sidx(kq)); }
};

// Q5_0 (LAYOUT_SPLIT_Q5_0): Q4_0's scales and nibble halves, plus the
// eight blocks' 4-byte qh words of a group (plane 2), 32 bytes per row,
// loaded with the halves: bit p of a block's word is the fifth bit of its
// position p (rce-op-qmm/src/lib.rs L525-561).  A lane's eight weights of
// k-step kq of chunk q are positions 16(kq & 1) + 8h .. +7 of block
// 2q + kq / 2, so their fifth bits are byte 2(kq & 1) + h of that word.
// u = nibble | bit << 4 in 0..31, f16(1024 + u) - 1040 = u - 16 exactly,
// then (u - 16) d + 0 rounds once.
struct Q50 : Q40 {
    static constexpr int OFF = 1040;
    static constexpr bool HB = true;
    static constexpr int w_group(int bn) { return NH * bn * 64 + bn * HDR + bn * 32; }
    static constexpr int w_loads(int bn) { return bn / 16 * NH / 2 + bn / 64; }
    __device__ static size_t hb_src(const DevWeight &w, int g) { return w.plane2 + 32 * (size_t)g; }
    __device__ static int hb_off(int q, int kq) { return 4 * (2 * q + (kq >> 1)) + 2 * (kq & 1); }
};

// Q8_0: four 64-byte pieces per row and group: bytes 0..15 (plane 1) and
// 16..31 (plane 2) of blocks 8g..8g+3 and 8g+4..8g+7 (piece 2 plane +
// half); header = the eight blocks' f16 scales, set 0 / 1 = block 2q /
// 2q+1.  K-step kq of chunk q is plane kq & 1 of block 2q + kq / 2.  A
// value q (int8) is read as u = q + 128 (the byte xor 0x80), f16(1024 + u)
// - 1152 = q exactly, and d * q + 0 rounds once: the reference's f32 value
// d * q rounded to binary16.
struct Q80 {
    static constexpr int NH = 4, OFF = 1152, HDR = 16, SBW = 2, CST = HDR;  // {d, +0} read from the header, as Q40
    static constexpr bool IL64 = false, HB = false;
    static constexpr int w_group(int bn) { return NH * bn * 64 + bn * HDR; }
    static constexpr int w_loads(int bn) { return bn / 16 * NH / 2; }
    static constexpr int h_loads(int) { return 1; }
    static constexpr int hoff(int bn) { return NH * bn * 64; }
    __device__ static size_t half_off(const DevWeight &w, int g, int hf) {
        return ((hf >> 1) ? w.plane2 : w.plane1) + 128 * (size_t)g + 64 * (hf & 1);
    }
    __device__ static size_t hdr_off(const DevWeight &, int g) { return 16 * (size_t)g; }
    __device__ static int half_of(int q, int kq) { return 2 * (kq & 1) + (q >> 1); }
    __device__ static int piece_of(int q, int kq) { return 2 * (q & 1) + (kq >> 1); }
    __device__ static int acol(int kq) { return (kq >> 1) * 4 + (kq & 1) * 2; }
    __device__ static int sidx(int kq) { return kq >> 1; }
    __device__ static int sbyte(int q, int kq) { return 4 * q + 2 * sidx(kq); }
    __device__ static uint32_t vals(uint32_t x, int) { return x ^ 0x80808080u; }
};

// Q6_K (LAYOUT_IL64_Q6_K, 64-row groups, so only the 64-column tile): a
// scale group is one super-block, whose 16-byte ql (0..7) and qh (8..11)
// chunks of the tile's 64 rows lie as 12 contiguous KB, then (after the
// scales chunk and the d values, which the GEMM does not read) the rows'
// 16 f16 {s, -32 s} pairs as [pair][row], 4 KB (rce-op-qmm/src/lib.rs
// L425-454, dequant.rs L658-701); the group buffer holds the 12 KB and the
// pairs.
// Chunk q of the super-block is positions 64q .. 64q+63: 128-half n = q/2,
// quarters 2(q&1) and 2(q&1)+1; k-step kq takes quarter 2(q&1) + kq/2,
// positions l = 16(kq&1) .. +15 of it, lane half h l + 8h .. +7: ql bytes
// 64n + 32(kq/2) + 16(kq&1) + 8h (chunk 4n + 2(kq/2) + (kq&1)), nibble
// 4(q&1); qh bytes 32n + 16(kq&1) + 8h (chunk 8 + 2n + (kq&1)), bits
// 2(2(q&1) + kq/2); scale 4q + kq (set kq).  u = ql | qh << 4 is q + 32 in
// 0..63, and s u - 32 s with s = f16(d sc) rounds once to f16(s (u - 32))
// (the reference's f32 d sc q rounded to binary16, but for the rounding of
// d sc to binary16, as Q4_K's d sc).
struct Q6K {
    static constexpr bool IL64 = true, HB = false;
    static constexpr int NH = 0, OFF = 1024, HDR = 0, SBW = 4, CST = 4;
    static constexpr int w_group(int) { return 16 * 1024; }
    static constexpr int w_loads(int) { return 6; }  // chunks 6 pw .. 6 pw + 5
    static constexpr int h_loads(int) { return 2; }  // pair KB 2 pw, 2 pw + 1
    static constexpr int hoff(int) { return 12 * 1024; }
    __device__ static int acol(int kq) { return (kq >> 1) * 4 + (kq & 1) * 2; }
    __device__ static int sidx(int kq) { return kq; }
    __device__ static int sbyte(int q, int kq) { return (4 * q + kq) * 256; }  // pair 4q + kq
    __device__ static int ql_chunk(int q, int kq) { return 4 * (q >> 1) + 2 * (kq >> 1) + (kq & 1); }
    __device__ static int qh_chunk(int q, int kq) { return 8 + 2 * (q >> 1) + (kq & 1); }
};

template <int U>
using ic = std::integral_constant<int, U>;

// One block's output tile in the T shape: rows m0 .. m0 + rows - 1 (arow:
// the activation row of each, padded to T::BM), columns n0 .. n0 + BN - 1
// of w.  EPI (GemmEpilogue) is what the block stores for an output element
// o with f32 sum v: v (f32 out); binary16 silu(v); binary16 silu(aux[o]) * v.
template <class T, class Fmt, int EPI>
__device__ __forceinline__ void gemm_tile(const DevWeight &w, const _Float16 *__restrict__ A, uint32_t a_bytes,
                                          void *__restrict__ out_v, const float *__restrict__ aux, size_t m0,
                                          int rows, size_t n0, const int *arow, unsigned char *lds) {
    constexpr int BM = T::BM, BN = T::BN, RB = T::RB, CB = T::CB, NS = T::NS, NH = Fmt::NH;
    constexpr int A_STAGE = T::A_STAGE, W_HALF = T::W_HALF, W_GROUP = T::W_GROUP;
    constexpr int OFF_W = T::OFF_W;
    const size_t N = w.n_rows, K = w.n_cols;
    const int nchunks = (int)(K / KC), ngroups = nchunks / 4;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool producer = wave >= NC / 64;
    const int l32 = lane & 31, h = lane >> 5;
    const uint32_t lds0 = lds_addr(lds);

    if (producer) {
        // ===== producer waves: every global -> LDS load, and the scales.
        // Loads are a uniform base (kernel argument + per-chunk offset)
        // plus this lane's loop-invariant 32-bit offset (the host checks
        // the ranges); issuing them may stall on the memory pipeline, which
        // holds up only these two waves.
        const int pw = wave - NC / 64;  // 0, 1
        //   A: rows BM/2*pw .. +BM/2-1; instruction i covers rows
        //      BM/2*pw + 8i .. +7, 8 lanes per row; lane slot p holds
        //      column p ^ f(row).  Lanes of rows past the tile's own (a
        //      grouped tile's expert has fewer) read past the buffer's end,
        //      which moves no data and lands zeros; their sums are not
        //      stored.  (Where that offset plus the chunk offsets could wrap
        //      32 bits, they read the tile's last row instead.)
        const bool pad_oob = (uint64_t)a_bytes + 2 * (uint64_t)K < ((uint64_t)1 << 32);
        uint32_t a_lane[T::A_LOADS];
#pragma unroll
        for (int i = 0; i < T::A_LOADS; i++) {
            const int ar = BM / 2 * pw + 8 * i + (lane >> 3);
            const int aswz = (ar & 7) ^ ((ar >> 3) & 1);
            a_lane[i] = ar >= rows && pad_oob ? a_bytes
                                              : (uint32_t)arow[ar] * (uint32_t)(2 * K) + 16u * (uint32_t)((lane & 7) ^ aswz);
        }
        const __amdgpu_buffer_rsrc_t abuf = byte_buffer(A, a_bytes);
        //   W: half pw of the group; instruction i covers rows 16i .. +15,
        //      4 lanes per row, slot p holding piece p ^ ((row >> 2) & 3);
        //      headers: rows BN/2*pw + lane for lanes 0..BN/2-1
        //      The buffer starts at the tile's first row, so its offsets
        //      span the tile's rows only.
        const size_t wtile = N - n0 < (size_t)BN ? N - n0 : (size_t)BN;  // rows of this tile
        uint32_t w_lane[T::W_ROW_LOADS];
#pragma unroll
        for (int i = 0; i < T::W_ROW_LOADS; i++) {
            const int wr = 16 * i + (lane >> 2);
            const size_t wrow = (size_t)wr < wtile ? (size_t)wr : wtile - 1;  // rows past the end load the last row
            w_lane[i] = (uint32_t)(wrow * w.row_stride) + 16u * (uint32_t)((lane & 3) ^ ((wr >> 2) & 3));
        }
        // HB (Q5_K): the fifth-bit bytes, 32 per row; instruction i of this
        // producer covers rows 32 (BN/64 pw + i) .. +31, 2 lanes per row
        constexpr int HB_LOADS = Fmt::HB ? BN / 64 : 0;
        uint32_t hb_lane[HB_LOADS > 0 ? HB_LOADS : 1];
#pragma unroll
        for (int i = 0; i < HB_LOADS; i++) {
            const int hr = 32 * (HB_LOADS * pw + i) + (lane >> 1);
            const size_t hbrow = (size_t)hr < wtile ? (size_t)hr : wtile - 1;
            hb_lane[i] = (uint32_t)(hbrow * w.row_stride) + 16u * (uint32_t)(lane & 1);
        }
        // headers of rows BN/2 pw ..: 16-byte headers one lane per row
        // (lanes 0..BN/2-1); 32-byte ones two lanes per row, instruction i
        // covering rows BN/2 pw + 32 i .. +31
        constexpr int H_LOADS = Fmt::IL64 ? 1 : Fmt::h_loads(BN);
        uint32_t h_lane[H_LOADS];
#pragma unroll
        for (int i = 0; i < H_LOADS; i++) {
            size_t hrow = Fmt::HDR == 16 ? (size_t)(BN / 2 * pw + (lane & (BN / 2 - 1)))
                                         : (size_t)(BN / 2 * pw + 32 * i + (lane >> 1));
            hrow = hrow < wtile ? hrow : wtile - 1;
            h_lane[i] = (uint32_t)(hrow * w.row_stride) + (Fmt::HDR == 16 ? 0u : 16u * (uint32_t)(lane & 1));
        }
        // IL64 (Q6_K): the tile's 64 columns are one 64-row group, and every
        // load is one 1 KB chunk of it (lane l: bytes 16 l ..)
        const __amdgpu_buffer_rsrc_t wbuf =
            Fmt::IL64 ? byte_buffer(w.base + (n0 >> 6) * w.group_stride, (uint32_t)w.group_stride)
                      : byte_buffer(w.base + n0 * w.row_stride, (uint32_t)(wtile * w.row_stride));
        const uint32_t a_soff_max = (uint32_t)(nchunks - 1) * (KC * 2);
        // W position q of group gs into the group buffer dst: at 0 the
        // weight bytes (split formats: the 64-byte pieces pw, pw + 2, ... of
        // every row; IL64: chunks 6 pw .. 6 pw + 5), at 1 the headers of
        // rows BN/2 pw .. (IL64: the scales chunk, or the d values).
        auto load_w = [&](int q, int gs, unsigned char *dst) {
            if constexpr (Fmt::IL64) {
                const uint32_t sb = (uint32_t)gs * (uint32_t)IL64_Q6K_SB, lo = 16u * (uint32_t)lane;
                if (q == 0) {
#pragma unroll
                    for (int j = 0; j < 6; j++)
                        buf_load_lds16(wbuf, lo, sb + (uint32_t)(6 * pw + j) * 1024u, dst + (6 * pw + j) * 1024);
                } else {
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        buf_load_lds16(wbuf, lo, sb + (uint32_t)IL64_Q6K_P + (uint32_t)(2 * pw + j) * 1024u,
                                       dst + (12 + 2 * pw + j) * 1024);
                }
            } else if (q == 0) {
#pragma unroll
                for (int hf = 0; hf < NH; hf += 2) {  // pieces pw, pw + 2, ...
                    const uint32_t soff = (uint32_t)Fmt::half_off(w, gs, hf + pw);
#pragma unroll
                    for (int i = 0; i < T::W_ROW_LOADS; i++)
                        buf_load_lds16(wbuf, w_lane[i], soff, dst + (hf + pw) * W_HALF + i * 1024);
                }
                if constexpr (Fmt::HB) {
#pragma unroll
                    for (int i = 0; i < HB_LOADS; i++)
                        buf_load_lds16(wbuf, hb_lane[i], (uint32_t)Fmt::hb_src(w, gs),
                                       dst + NH * W_HALF + BN * Fmt::HDR + (HB_LOADS * pw + i) * 1024);
                }
            } else if constexpr (Fmt::HDR == 16) {
                if (lane < BN / 2)
                    buf_load_lds16(wbuf, h_lane[0], (uint32_t)Fmt::hdr_off(w, gs), dst + NH * W_HALF + pw * (BN / 2) * 16);
            } else {
#pragma unroll
                for (int i = 0; i < H_LOADS; i++)
                    buf_load_lds16(wbuf, h_lane[i], (uint32_t)Fmt::hdr_off(w, gs),
                                   dst + NH * W_HALF + (BN / 2 * pw + 32 * i) * Fmt::HDR);
            }
        };
        // Loads of (virtual) iteration it: W position it % 4 of group
        // it/4 + GA, then A chunk it + NS - 1 into stage it % NS.  Past the
        // end both repeat the last group / chunk: those loads only keep the
        // in-order counts of the waits uniform, and data the block has just
        // read is still in its L2, so the drain before the epilogue is short.
        auto issue = [&](int it) {
            const int q = it & 3;
            if (q < 2) {
                const int g = (it >> 2) + GA, gs = g < ngroups ? g : ngroups - 1;
                load_w(q, gs, lds + OFF_W + (g & (NWBUF - 1)) * W_GROUP);
            }
            const uint32_t soff = __builtin_elementwise_min((uint32_t)(it + NS - 1) * (KC * 2), a_soff_max);
            unsigned char *dst = lds + ((it + NS - 1) % NS) * A_STAGE + pw * (A_STAGE / 2);
#pragma unroll
            for (int i = 0; i < T::A_LOADS; i++) buf_load_lds16(abuf, a_lane[i], soff, dst + i * 1024);
        };
        // prologue: virtual iterations -4GA .. -1
#pragma unroll
        for (int it = -4 * GA; it < 0; it++) {
            if ((it & 3) < 2) {
                const int q = it & 3, g = (it >> 2) + GA, gs = g < ngroups ? g : ngroups - 1;
                load_w(q, gs, lds + OFF_W + (g & (NWBUF - 1)) * W_GROUP);
            }
            if (it + NS - 1 >= 0) {
                const uint32_t soff = __builtin_elementwise_min((uint32_t)(it + NS - 1) * (KC * 2), a_soff_max);
                unsigned char *dst = lds + ((it + NS - 1) % NS) * A_STAGE + pw * (A_STAGE / 2);
#pragma unroll
                for (int i = 0; i < T::A_LOADS; i++) buf_load_lds16(abuf, a_lane[i], soff, dst + i * 1024);
            }
        }
        wait_vm_barrier<T::vm_after(3)>();  // barrier P1: A chunks 0, 1 and W groups 0, 1 done
        for (int g = 0; g < ngroups; g++) {
            auto step = [&](auto uc) {
                constexpr int u = decltype(uc)::value;
                wait_vm_barrier<T::vm_after(u)>();
                issue(4 * g + u);
            };
            step(ic<0>{});
            step(ic<1>{});
            step(ic<2>{});
            step(ic<3>{});
        }
        __builtin_amdgcn_s_waitcnt(0);  // drain the padding loads before LDS is reused
        __syncthreads();                 // barrier E1
#pragma unroll
        for (int cb = 0; cb < CB; cb++) {  // the compute waves' epilogue barriers, one by one
            if (cb > 0) __syncthreads();
            __syncthreads();  // barrier E2
        }
        return;
    }

    // ===== compute waves: wave w = 2*kq + t
    const int t = wave & 1, kq = wave >> 1;
    // LDS read addresses of this lane; A row block rb is +32 rows (+4096
    // bytes), W column block cb +32 rows of nibbles (+2048 bytes) and +32
    // columns of scales (+128 bytes): immediates.
    const int g0 = Fmt::acol(kq) + h;
    const uint32_t a_rd = lds0 + (uint32_t)(l32 * 128 + 16 * (g0 ^ ((l32 & 7) ^ ((l32 >> 3) & 1))));
    const int ncol = BN / 2 * t + l32;  // tile column of this lane in column block 0
    uint32_t w_rd[4], wh_rd[4];         // weight bytes of chunk position q, lane half h (group buffer 0)
#pragma unroll
    for (int q = 0; q < 4; q++) {
        if constexpr (Fmt::IL64) {  // ql and qh chunks: column c at c * 16
            w_rd[q] = lds0 + OFF_W + (uint32_t)(Fmt::ql_chunk(q, kq) * 1024 + ncol * 16 + 8 * h);
            wh_rd[q] = lds0 + OFF_W + (uint32_t)(Fmt::qh_chunk(q, kq) * 1024 + ncol * 16 + 8 * h);
        } else {
            w_rd[q] = lds0 + OFF_W + (uint32_t)(Fmt::half_of(q, kq) * W_HALF + ncol * 64 +
                                                16 * (Fmt::piece_of(q, kq) ^ ((ncol >> 2) & 3)) + 8 * h);
            if constexpr (Fmt::HB)  // the fifth-bit byte of the lane's eight weights
                wh_rd[q] = lds0 + OFF_W + (uint32_t)(NH * W_HALF + BN * Fmt::HDR + ncol * 32 + Fmt::hb_off(q, kq) + h);
            else
                wh_rd[q] = w_rd[q];
        }
    }
    // {scale, bias} word of chunk position q of group g: the column's header
    // (or, Q6_K, its pair in the [pair][column] block) in the group buffer
    const uint32_t hd_rd = lds0 + OFF_W + (uint32_t)(Fmt::hoff(BN) + ncol * Fmt::CST);
    auto sb_addr = [&](int g, int q) -> uint32_t {
        return hd_rd + (uint32_t)((g & (NWBUF - 1)) * W_GROUP + Fmt::sbyte(q, kq));
    };

    f32x16 acc[RB * CB];
#pragma unroll
    for (int i = 0; i < RB * CB; i++) acc[i] = f32x16{};
    const int nsh = 4 * (kq & 1);  // low or high nibbles
    // the four byte values of word i (0, 1) of a lane's eight weights of
    // chunk position q
    auto nib = [&](const WRaw &r, int i, int q) -> uint32_t {
        const uint32_t x = i ? r.l.y : r.l.x;
        if constexpr (Fmt::IL64) {  // ql nibble | qh 2 bits << 4
            const uint32_t y = i ? r.h.y : r.h.x;
            return ((x >> (4 * (q & 1))) & 0x0F0F0F0Fu) | (((y >> (2 * (2 * (q & 1) + (kq >> 1)))) & 0x03030303u) << 4);
        } else if constexpr (Fmt::HB) {  // nibble | fifth bit << 4: bit e of the byte's half to byte e
            const uint32_t b4 = i ? (r.h.x >> 4) & 15u : r.h.x & 15u;
            return Fmt::vals(x, nsh) | (((b4 * 0x00204081u) & 0x01010101u) << 4);
        } else {
            return Fmt::vals(x, nsh);
        }
    };
    auto read_a = [&](half8 *a, uint32_t addr) {
        a[0] = lds_read_frag<0>(addr);
        if constexpr (RB > 1) a[1] = lds_read_frag<4096>(addr);
        if constexpr (RB > 2) a[2] = lds_read_frag<8192>(addr);
        if constexpr (RB > 3) a[3] = lds_read_frag<12288>(addr);
    };
    // column block cb: +32 rows of 64-byte pieces (split formats) or +32
    // columns of 16 bytes (IL64)
    constexpr int CBW = Fmt::IL64 ? 512 : 2048;
    auto read_w = [&](WRaw *r, uint32_t addr, uint32_t addr_h) {
        r[0].l = lds_read8<0>(addr);
        if constexpr (CB > 1) r[1].l = lds_read8<CBW>(addr);
        if constexpr (Fmt::IL64) {
            r[0].h = lds_read8<0>(addr_h);
            if constexpr (CB > 1) r[1].h = lds_read8<CBW>(addr_h);
        } else if constexpr (Fmt::HB) {
            r[0].h.x = lds_read_u8<0>(addr_h);
            if constexpr (CB > 1) r[1].h.x = lds_read_u8<1024>(addr_h);  // +32 rows of 32 bytes
        }
    };
    // one chunk's {scale, bias} per column block (a register each, not the
    // group's four: the 96-row tile's accumulators need the room)
    auto read_sb = [&](uint32_t *v, uint32_t addr) {
        if constexpr (Fmt::SBW == 2) {  // f16 d zero-extended: {d, +0}
            v[0] = lds_read_u16<0>(addr);
            if constexpr (CB > 1) v[1] = lds_read_u16<32 * Fmt::CST>(addr);  // +32 columns
        } else {  // a pair formed at upload
            v[0] = lds_read4<0>(addr);
            if constexpr (CB > 1) v[1] = lds_read4<32 * Fmt::CST>(addr);
        }
    };
    auto wait_reads = [&](half8 *a, WRaw *r, uint32_t *v) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int i = 0; i < RB; i++) pin(a[i]);
#pragma unroll
        for (int i = 0; i < CB; i++) {
            pin(r[i].l);
            if constexpr (Fmt::IL64) pin(r[i].h);
            if constexpr (Fmt::HB) pin_lo(r[i].h);  // one byte: only the low word is live
            pin(v[i]);
        }
    };

    __builtin_amdgcn_s_barrier();  // barrier P1
    half8 a_cur[RB], b_cur[CB];
    WRaw raw_nxt[CB];
    uint32_t sb_nxt[CB];  // {scale, bias} of chunk c+1
    {
        WRaw raw0[CB];
        uint32_t sb0[CB];
        read_a(a_cur, a_rd);
        read_w(raw0, w_rd[0], wh_rd[0]);
        read_w(raw_nxt, w_rd[1], wh_rd[1]);
        read_sb(sb0, sb_addr(0, 0));
        read_sb(sb_nxt, sb_addr(0, 1));
        wait_reads(a_cur, raw0, sb0);
#pragma unroll
        for (int cb = 0; cb < CB; cb++) {
            pin(raw_nxt[cb].l);
            if constexpr (Fmt::IL64) pin(raw_nxt[cb].h);
            if constexpr (Fmt::HB) pin_lo(raw_nxt[cb].h);
            pin(sb_nxt[cb]);
        }
#pragma unroll
        for (int cb = 0; cb < CB; cb++) {
            half2v h0, h1, h2, h3;
            dequant4<Fmt::OFF>(nib(raw0[cb], 0, 0), sb0[cb], h0, h1);
            dequant4<Fmt::OFF>(nib(raw0[cb], 1, 0), sb0[cb], h2, h3);
            b_cur[cb] = join8(h0, h1, h2, h3);
        }
    }

    // ---- main loop: one scale group (four chunks) per trip; chunk c's A is
    // in stage c % NS.
    int st1 = 1;  // stage of chunk c+1
    for (int g = 0; g < ngroups; g++) {
        // nibble reads of chunk c+2 (steps 0, 1: this group; 2, 3: the next)
        const uint32_t wb_cur = (uint32_t)((g & (NWBUF - 1)) * W_GROUP);
        const uint32_t wb_nxt = (uint32_t)(((g + 1) & (NWBUF - 1)) * W_GROUP);
        auto step = [&](auto uc) {
            constexpr int u = decltype(uc)::value;
            // chunk c+1's A and W are in LDS (the producers waited for them);
            // every wave is done with the reads of chunk c
            __builtin_amdgcn_s_barrier();
            // LDS reads: A fragments of chunk c+1, nibbles and {scale,
            // bias} of chunk c+2 (from u = 2 on: the next group's, whose
            // scales the producers wrote at u = 1)
            const uint32_t sa = a_rd + (uint32_t)(st1 * A_STAGE);
            st1 = st1 == NS - 1 ? 0 : st1 + 1;
            half8 a_nxt[RB];
            WRaw raw_nn[CB];
            uint32_t sb_nn[CB];
            read_a(a_nxt, sa);
            read_w(raw_nn, w_rd[(u + 2) & 3] + (u >= 2 ? wb_nxt : wb_cur), wh_rd[(u + 2) & 3] + (u >= 2 ? wb_nxt : wb_cur));
            read_sb(sb_nn, sb_addr(u >= 2 ? g + 1 : g, (u + 2) & 3));
            __builtin_amdgcn_sched_barrier(0);
            // Chunk c's MFMAs and chunk c+1's dequantization (the next
            // group's first chunk for u = 3), independent of each other.
            half2v hq[CB][4];
#pragma unroll
            for (int cb = 0; cb < CB; cb++) {
                const uint32_t sb = sb_nxt[cb];
#pragma unroll
                for (int rb = 0; rb < RB; rb++) {
                    acc[rb * CB + cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_cur[rb], b_cur[cb], acc[rb * CB + cb], 0, 0, 0);
                    if (rb == 0) dequant4<Fmt::OFF>(nib(raw_nxt[cb], 0, (u + 1) & 3), sb, hq[cb][0], hq[cb][1]);
                    if (rb == 1) dequant4<Fmt::OFF>(nib(raw_nxt[cb], 1, (u + 1) & 3), sb, hq[cb][2], hq[cb][3]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            wait_reads(a_nxt, raw_nn, sb_nn);
#pragma unroll
            for (int i = 0; i < RB; i++) a_cur[i] = a_nxt[i];
#pragma unroll
            for (int cb = 0; cb < CB; cb++) {
                b_cur[cb] = join8(hq[cb][0], hq[cb][1], hq[cb][2], hq[cb][3]);
                raw_nxt[cb] = raw_nn[cb];
                sb_nxt[cb] = sb_nn[cb];
            }
        };
        step(ic<0>{});
        step(ic<1>{});
        step(ic<2>{});
        step(ic<3>{});
    }
    __syncthreads();  // barrier E1: the producers have drained their loads

    // Partial sums to LDS, one column block cb at a time: element r of
    // acc[rb * CB + cb] in lane l is row 8(r/4) + 4(l/32) + r%4, column l%32
    // of that 32 x 32 block.  Layout [wave][rb][r/4][lane][r%4]
    // (conflict-free 16-byte accesses).  Wave w < 2 RB then finishes output
    // block (row block w / 2, column half w % 2) of column block cb: the
    // partials of the waves 2*kq + ot, k-steps 0, 1, 2, 3 added in order.
    f32x4 *red = reinterpret_cast<f32x4 *>(lds);
#pragma unroll
    for (int cb = 0; cb < CB; cb++) {
        if (cb > 0) __syncthreads();  // the previous column block's partials are read
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
            for (int rq = 0; rq < 4; rq++) {
                const f32x16 &a = acc[rb * CB + cb];
                const f32x4 v = {a[4 * rq], a[4 * rq + 1], a[4 * rq + 2], a[4 * rq + 3]};
                red[((wave * RB + rb) * 4 + rq) * 64 + lane] = v;
            }
        __syncthreads();  // barrier E2
        if (wave < 2 * RB) {
            const int orb = wave >> 1, ot = wave & 1;
            const size_t col = n0 + (size_t)(BN / 2 * ot + 32 * cb + l32);
#pragma unroll
            for (int rq = 0; rq < 4; rq++) {
                f32x4 sum = red[((ot * RB + orb) * 4 + rq) * 64 + lane];
#pragma unroll
                for (int k2 = 1; k2 < 4; k2++) sum += red[(((2 * k2 + ot) * RB + orb) * 4 + rq) * 64 + lane];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int m = 32 * orb + 8 * rq + 4 * h + e;
                    if (m < rows && col < N) {
                        const size_t o = (m0 + m) * N + col;
                        if constexpr (EPI == GEPI_F32) {
                            static_cast<float *>(out_v)[o] = sum[e];
                        } else if constexpr (EPI == GEPI_SILU_F16) {  // rce-qwen36-moe/src/lib.rs L459-461
                            static_cast<_Float16 *>(out_v)[o] = (_Float16)silu_mfma(sum[e]);
                        } else {  // silu(g) * u, rce-qwen36-moe/src/lib.rs L667-676
                            const float hv = silu_mfma(aux[o]) * sum[e];
                            static_cast<_Float16 *>(out_v)[o] = (_Float16)hv;
                        }
                    }
                }
            }
        }
    }
}

// Plain GEMM: tiles == nullptr, row tile mt covers rows mt*BM .. of M.
// Grouped (MoE): row tile mt is tiles[mt] (expert e, first row r0, rows),
// multiplied by wtab[e]; tiles at or past n_tiles[0] do nothing.
template <class Fmt, int BM_, int EPI, int BN_ = 0>
__global__ __launch_bounds__(NT) void k_gemm_f16(DevWeight w_arg, const _Float16 *__restrict__ A,
                                                 const int *__restrict__ gather, size_t M, uint32_t a_bytes,
                                                 void *__restrict__ out_v, const float *__restrict__ aux, int m_tiles,
                                                 const MoeTile *__restrict__ tiles, const int *__restrict__ n_tiles,
                                                 const DevWeight *__restrict__ wtab) {
    using T = Tile<BM_, Fmt, BN_>;
    constexpr int BM = T::BM;
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ int arow[BM];
    // Which tile: plain launches as tile_of_block places them (the m-tiles
    // sharing W rows on one XCD); grouped launches take the tiles in
    // (row tile, column tile) order, block L tile L, so consecutive column
    // tiles of an expert go to consecutive XCDs and every XCD gets an equal
    // share of every expert's tiles.  The tiles differ in cost (below: a
    // row tile of at most 64 rows runs the 64-row body), and placing whole
    // experts on XCDs, as tile_of_block does, left the XCD of the largest
    // expert to finish last (configs[3] 234 -> 221 us with both changes; the
    // placement alone measured the same as expert-major).  Blocks past the
    // tile count return before any barrier.
    int mt, nt;
    if (n_tiles) {
        const int nn = (int)((w_arg.n_rows + T::BN - 1) / T::BN), L = blockIdx.x;
        if (L >= n_tiles[0] * nn) return;
        mt = L / nn;
        nt = L % nn;
    } else if (!tile_of_block<T::BN>(w_arg.n_rows, m_tiles, n_tiles, mt, nt)) {
        return;
    }
    DevWeight w = w_arg;
    size_t m0 = (size_t)mt * BM;
    int rows = (int)(M - m0 < (size_t)BM ? M - m0 : BM);
    if (tiles) {
        const MoeTile tl = tiles[mt];
        w = wtab[tl.e];
        m0 = (size_t)tl.r0;
        rows = tl.rows;
    }
    const int tid = threadIdx.x;
    if (tid < BM) {
        const size_t m = m0 + (tid < rows ? tid : rows - 1);  // rows past the tile load its last row
        arow[tid] = gather ? gather[m] : (int)m;
    }
    __syncthreads();
    const size_t n0 = (size_t)nt * T::BN;
    // A 96- or 128-row tile that holds at most 64 rows (a grouped tile whose
    // expert has that few, a plain GEMM's last row tile) runs the 64-row
    // tile's body over the same columns: a third or half fewer activation
    // copies and MFMAs, and each output's sum formed the same way (a wave's
    // k-step partial over the tile's chunks in order, the four partials
    // added in order).
    if constexpr (BM_ > 64) {
        using T64 = Tile<64, Fmt, T::BN>;
        static_assert(T64::BN == T::BN && T64::LDS <= T::LDS, "the 64-row body in the wider tile's launch");
        if (rows <= 64) {
            gemm_tile<T64, Fmt, EPI>(w, A, a_bytes, out_v, aux, m0, rows, n0, arow, lds);
            return;
        }
    }
    // likewise a 128-row tile holding at most 96 rows runs the 96 x BN body
    if constexpr (BM_ > 96) {
        using T96 = Tile<96, Fmt, T::BN>;
        static_assert(T96::BN == T::BN && T96::LDS <= T::LDS, "the 96-row body in the wider tile's launch");
        if (rows <= 96) {
            gemm_tile<T96, Fmt, EPI>(w, A, a_bytes, out_v, aux, m0, rows, n0, arow, lds);
            return;
        }
    }
    gemm_tile<T, Fmt, EPI>(w, A, a_bytes, out_v, aux, m0, rows, n0, arow, lds);
}

__global__ void k_f32_to_f16(const float *__restrict__ s, _Float16 *__restrict__ d, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) d[i] = (_Float16)s[i];
}

template <class Fmt, int BM, int EPI, int BN_ = 0>
hipError_t set_lds_attr() {
    return ensure_lds_limit((const void *)k_gemm_f16<Fmt, BM, EPI, BN_>, Tile<BM, Fmt, BN_>::LDS);
}

template <class Fmt, int BM, int BN_ = 0>
hipError_t launch_fmt(const DevWeight &w, const _Float16 *a, size_t M, float *out, hipStream_t s) {
    using T = Tile<BM, Fmt, BN_>;
    const int m_tiles = (int)((M + T::BM - 1) / T::BM), n_tiles = (int)((w.n_rows + T::BN - 1) / T::BN);
    hipError_t e = set_lds_attr<Fmt, BM, GEPI_F32, BN_>();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_gemm_f16<Fmt, BM, GEPI_F32, BN_>), dim3(m_tiles * n_tiles), dim3(NT), T::LDS, s, w, a,
                       (const int *)nullptr, M, (uint32_t)(M * w.n_cols * 2), (void *)out, (const float *)nullptr,
                       m_tiles, (const MoeTile *)nullptr, (const int *)nullptr, (const DevWeight *)nullptr);
    return hipGetLastError();
}

template <class Fmt, int BM, int EPI>
hipError_t launch_fmt_grouped(const DevWeight &w, const DevWeight *wtab, const _Float16 *a, size_t a_rows,
                              const int *gather, const MoeTile *tiles, const int *n_tiles_dev, int max_tiles, void *out,
                              const float *aux, hipStream_t s) {
    using T = Tile<BM, Fmt>;
    const int n_tiles = (int)((w.n_rows + T::BN - 1) / T::BN);
    hipError_t e = set_lds_attr<Fmt, BM, EPI>();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_gemm_f16<Fmt, BM, EPI>), dim3(grouped_grid(max_tiles, n_tiles)), dim3(NT), T::LDS, s, w, a,
                       gather, a_rows, (uint32_t)(a_rows * w.n_cols * 2), out, aux, max_tiles, tiles, n_tiles_dev, wtab);
    return hipGetLastError();
}

template <class Fmt, int BM>
hipError_t launch_grouped_epi(int epi, const DevWeight &w, const DevWeight *wtab, const _Float16 *a, size_t a_rows,
                              const int *gather, const MoeTile *tiles, const int *n_tiles_dev, int max_tiles, void *out,
                              const float *aux, hipStream_t s) {
    switch (epi) {
    case GEPI_F32:
        return launch_fmt_grouped<Fmt, BM, GEPI_F32>(w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles, out, aux, s);
    case GEPI_SILU_F16:
        return launch_fmt_grouped<Fmt, BM, GEPI_SILU_F16>(w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles, out,
                                                          aux, s);
    case GEPI_SWIGLU_F16:
        if (!aux) return hipErrorInvalidValue;
        return launch_fmt_grouped<Fmt, BM, GEPI_SWIGLU_F16>(w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles,
                                                            out, aux, s);
    default:
        return hipErrorInvalidValue;
    }
}

}  // namespace

// The kernel's per-lane load offsets are 32-bit: the activations (all of
// them: a grouped tile gathers rows from anywhere) below 2^32 bytes, and a
// tile's 128 weight rows; the tile counts are ints.
bool gemm_shape_ok(size_t a_rows, const DevWeight &w) {
    return a_rows * w.n_cols * 2 < ((size_t)1 << 32) && 128 * w.row_stride < ((size_t)1 << 32) &&
           w.n_rows < ((size_t)1 << 31);
}

hipError_t gemm_prepare_lds() {
    hipError_t e = hipSuccess;
    auto all_epi = [&](auto fmt, auto bm) {
        using F = decltype(fmt);
        constexpr int BM = decltype(bm)::value;
        if (e == hipSuccess) e = set_lds_attr<F, BM, GEPI_F32>();
        if (e == hipSuccess) e = set_lds_attr<F, BM, GEPI_SILU_F16>();
        if (e == hipSuccess) e = set_lds_attr<F, BM, GEPI_SWIGLU_F16>();
    };
    auto all_bm = [&](auto fmt) {
        using F = decltype(fmt);
        all_epi(fmt, ic<64>{});
        all_epi(fmt, ic<96>{});
        all_epi(fmt, ic<128>{});
        // the plain GEMM's 64 x 64 tile (short M)
        if (e == hipSuccess) e = set_lds_attr<F, 64, GEPI_F32, 64>();
    };
    all_bm(Q4K{});
    all_bm(Q5K{});
    all_bm(Q40{});
    all_bm(Q41{});
    all_bm(Q50{});
    all_epi(Q80{}, ic<128>{});
    all_epi(Q6K{}, ic<128>{});
    if (e == hipSuccess) e = set_lds_attr<Q80, 64, GEPI_F32, 64>();
    if (e == hipSuccess) e = set_lds_attr<Q6K, 64, GEPI_F32, 64>();
    return e;
}

bool gemm_q8_supports(uint32_t dtype, size_t n_cols) {
    return (dtype == T_Q8_0 || dtype == T_Q6_K) && n_cols % 256 == 0 && n_cols < ((size_t)1 << 31);
}

bool gemm_supports(uint32_t dtype, size_t n_cols) {
    if (n_cols >= (size_t)1 << 31 || n_cols == 0) return false;
    if (dtype == T_Q4_K || dtype == T_Q5_K) return n_cols % 256 == 0;
    if (dtype == T_Q4_0 || dtype == T_Q4_1 || dtype == T_Q5_0) return n_cols % 256 == 0;  // whole groups of 8 blocks
    return false;
}

hipError_t launch_f32_to_f16(const float *src, void *dst, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_f32_to_f16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src,
                       static_cast<_Float16 *>(dst), n);
    return hipGetLastError();
}

int gemm_tile_rows(size_t rows_hint, bool grouped) {
    // plain: the fewest rows that hold M (96 for 65..96);
    // grouped: experts' rows scatter around the mean (about +-8 for 64), so
    // a mean of 49..80 takes 96-row tiles: one tile per expert, not a
    // 64-row tile and a mostly empty second one
    if (grouped) return rows_hint <= 48 ? 64 : (rows_hint <= 80 ? 96 : 128);
    return rows_hint <= 64 ? 64 : (rows_hint <= 96 ? 96 : 128);
}

// Call f with the format tag of a nibble-kernel weight type (false when the
// type has no format here).
template <class F>
static bool with_fmt(uint32_t dtype, F &&f) {
    switch (dtype) {
    case T_Q4_K: f(Q4K{}); return true;
    case T_Q5_K: f(Q5K{}); return true;
    case T_Q4_0: f(Q40{}); return true;
    case T_Q4_1: f(Q41{}); return true;
    case T_Q5_0: f(Q50{}); return true;
    default: return false;
    }
}

hipError_t launch_gemm_f16_grouped(const DevWeight &w, const DevWeight *wtab, const void *a_f16, size_t a_rows,
                                   const int *gather, const MoeTile *tiles, const int *n_tiles_dev, int max_tiles,
                                   int bm, int epi, void *out, const float *aux, hipStream_t s) {
    if (max_tiles <= 0 || w.n_rows == 0 || a_rows == 0) return hipSuccess;
    if (!gemm_shape_ok(a_rows, w)) return hipErrorInvalidValue;
    const _Float16 *a = static_cast<const _Float16 *>(a_f16);
    // Q8_0 and Q6_K: the 128 x 64 tile only
    if (gemm_q8_supports(w.dtype, w.n_cols)) {
        if (bm != 128) return hipErrorInvalidValue;
        return w.dtype == T_Q8_0
                   ? launch_grouped_epi<Q80, 128>(epi, w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles, out, aux, s)
                   : launch_grouped_epi<Q6K, 128>(epi, w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles, out, aux, s);
    }
    hipError_t e = hipErrorInvalidValue;
    with_fmt(w.dtype, [&](auto fmt) {
        using F = decltype(fmt);
        if (bm == 64) e = launch_grouped_epi<F, 64>(epi, w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles, out, aux, s);
        if (bm == 96) e = launch_grouped_epi<F, 96>(epi, w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles, out, aux, s);
        if (bm == 128)
            e = launch_grouped_epi<F, 128>(epi, w, wtab, a, a_rows, gather, tiles, n_tiles_dev, max_tiles, out, aux, s);
    });
    return e;
}

// Compute units of the current device (0 if unknown), read once per device.
static int cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int c = cache[dev].load(std::memory_order_relaxed);
    if (c == 0 && hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && c > 0)
        cache[dev].store(c, std::memory_order_relaxed);
    return c > 0 ? c : 0;
}

hipError_t launch_gemm_f16(const DevWeight &w, const void *a_f16, size_t M, float *out, hipStream_t s, int bm) {
    if (M == 0 || w.n_rows == 0) return hipSuccess;
    if (!gemm_shape_ok(M, w)) return hipErrorInvalidValue;
    const _Float16 *a = static_cast<const _Float16 *>(a_f16);
    const size_t n64 = (w.n_rows + 63) / 64, m64 = (M + 63) / 64, cus = cu_count() ? (size_t)cu_count() : 256;
    // Q8_0 / Q6_K: 64-column tiles only, 128 rows, or 64 where that makes
    // more blocks in one round (below)
    if (gemm_q8_supports(w.dtype, w.n_cols)) {
        const bool q64 = bm == 0 && ((M + 127) / 128) * n64 < cus && m64 * n64 <= cus;
        if (w.dtype == T_Q8_0) return q64 ? launch_fmt<Q80, 64, 64>(w, a, M, out, s) : launch_fmt<Q80, 128>(w, a, M, out, s);
        return q64 ? launch_fmt<Q6K, 64, 64>(w, a, M, out, s) : launch_fmt<Q6K, 128>(w, a, M, out, s);
    }
    bool sq64 = false;  // the 64 x 64 tile
    if (bm == 0) {
        bm = gemm_tile_rows(M, false);
        // Past one row tile of 128, 96 x 128 tiles where they take fewer
        // rounds over the CUs than 128 x 64 ones at less total tile work
        // (tile work ~ rows x columns: a round of 96 x 128 tiles costs about
        // 1.5 rounds of 128 x 64): M 640 and 768 at N 4096 are 320 and 384
        // tiles of 128 x 64 (two rounds, the second part empty), 224 and 256
        // of 96 x 128 (one).
        if (bm == 128) {
            const size_t t128 = ((M + 127) / 128) * ((w.n_rows + 63) / 64), t96 = ((M + 95) / 96) * ((w.n_rows + 127) / 128);
            if (((t96 + cus - 1) / cus) * 3 < ((t128 + cus - 1) / cus) * 2) bm = 96;
        }
        // Where the default tile leaves less than one tile per CU (short M),
        // 64 x 64 tiles, as long as they still take one round: more blocks,
        // each with less of the work.  Each output's sum is formed the same
        // way in every tile shape (a wave's k-step partial over the chunks in
        // order, the four partials added in order), so the bits do not
        // depend on the choice.
        const size_t bn = bm == 128 ? 64 : 128;
        sq64 = ((M + bm - 1) / bm) * ((w.n_rows + bn - 1) / bn) < cus && m64 * n64 <= cus;
    }
    hipError_t e = hipErrorInvalidValue;
    with_fmt(w.dtype, [&](auto fmt) {
        using F = decltype(fmt);
        if (sq64)
            e = launch_fmt<F, 64, 64>(w, a, M, out, s);
        else if (bm == 64)
            e = launch_fmt<F, 64>(w, a, M, out, s);
        else if (bm == 96)
            e = launch_fmt<F, 96>(w, a, M, out, s);
        else if (bm == 128)
            e = launch_fmt<F, 128>(w, a, M, out, s);
    });
    return e;
}

}  // namespace rce_qmm
