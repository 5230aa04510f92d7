// qmm_internal.h -- internal interface between the C ABI (qmm_abi.cpp) and
// the HIP kernels (qmm_gemv.hip, qmm_mfma.hip).  Not installed; callers use
// include/rce_qmm.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace rce_qmm {

// GGUF type tags (rce-ingest-gguf/src/parser.rs L306-341).
enum : uint32_t {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q8_0 = 8,
    T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30
};

// How a weight's GGUF bytes are arranged in HBM.  Every layout holds the
// same bytes as the GGUF tensor (plus alignment padding); only their order
// differs, chosen so that a wave's loads are contiguous 128-bit reads.
enum Layout : int {
    // Row-major rows; inside each row the 2-byte block scales of all blocks
    // first (padded to 16 bytes), then the blocks' quant bytes.  Q4_0, Q8_0.
    LAYOUT_SPLIT = 1,
    // Row-major rows of untouched GGUF blocks.  Q4_K (its 144-byte
    // super-block is already 16-byte aligned: 16 B of d/dmin/scales + 128 B).
    LAYOUT_NATIVE = 2,
    // Groups of 64 rows; per group and super-block the 64 rows' bytes are
    // interleaved in 16-byte chunks so lane r of a wave reads row r of the
    // group with contiguous wave-wide loads.  Q6_K (read one row per lane).
    LAYOUT_IL64 = 3,
};

// Bytes of one Q6_K super-block for a 64-row group in LAYOUT_IL64:
// ql 8 chunks x 64 rows x 16 B, qh 4 x 64 x 16, scales 64 x 16, d 64 x 2.
constexpr size_t IL64_Q6K_QL = 0;
constexpr size_t IL64_Q6K_QH = 8 * 64 * 16;             // 8192
constexpr size_t IL64_Q6K_SC = IL64_Q6K_QH + 4 * 64 * 16; // 12288
constexpr size_t IL64_Q6K_D = IL64_Q6K_SC + 64 * 16;      // 13312
constexpr size_t IL64_Q6K_SB = 64 * 210;                  // 13440

struct DevWeight {
    const uint8_t *base;  // device address of row 0 (LAYOUT_IL64: of group 0)
    uint32_t dtype;
    int layout;
    size_t n_rows, n_cols;
    size_t row_stride;    // SPLIT / NATIVE: bytes between rows
    size_t qs_off;        // SPLIT: offset of the quant bytes inside a row
    size_t group_stride;  // IL64: bytes between 64-row groups
};

// Kernels available for (dtype, n_cols, mode); mirrors rce_qmm_supports.
bool gpu_supports(uint32_t dtype, size_t n_cols, int mode);

hipError_t launch_f16_to_f32(const uint16_t *src, float *dst, size_t n, hipStream_t s);
hipError_t launch_gemv_exact(const DevWeight &w, const float *a, size_t t_rows, float *out,
                             hipStream_t s);
// Q8-activation path: quantizes the f32 activation rows inside the kernel.
hipError_t launch_gemv_q8(const DevWeight &w, const float *a, size_t t_rows, float *out,
                          hipStream_t s);
hipError_t launch_dequant_row(const DevWeight &w, size_t row, float *out, hipStream_t s);

}  // namespace rce_qmm
