/*
 * rce_qmm.h -- C ABI of the MI355X (gfx950) GGUF block-quantized matmul
 * library (librce_qmm.so).
 *
 * Drop-in replacement for the quantized-matmul operator of the reference's
 * compute substrate (openIE-dev/rce, compute/crates/rce-op-qmm).  Plain
 * pointers and sizes only; no exceptions cross this boundary.  Every entry
 * point returns an rce_qmm_status; the text of the last failure on the
 * calling thread is available from rce_qmm_last_error(), the convention of
 * compute/crates/rce-c/include/rce.h (RceStatus + rce_last_error).
 *
 * Numerics.  Three modes:
 *   RCE_QMM_MODE_EXACT     f32 activations, the reference's own operation
 *                          order (one binary32 rounding per op, no fused
 *                          multiply-add in the reference's arithmetic).
 *                          Bit-identical to rce_op_qmm::mm_1d / mm_batched
 *                          for activations of magnitude below 2^123 (the
 *                          forms (q - c) * a of Q4_0 / Q5_0 / Q3_K are one
 *                          fma of q, a and -c * a, which overflows before
 *                          the reference's product does); larger or
 *                          non-finite activations can give another
 *                          overflow or NaN pattern.
 *   RCE_QMM_MODE_Q8        activations quantized once per row to Q8 blocks
 *                          of 32 (nn.rs quantize_block semantics), exact
 *                          int32 block dot products, then the reference's
 *                          per-block formula and fold order.  Deterministic;
 *                          differs from EXACT by the activation rounding.
 *   RCE_QMM_MODE_F16_MFMA  (matmul / grouped experts) weights dequantized to
 *                          binary16 tiles (BF16 / F32 weights: bf16 terms,
 *                          activations split into two bf16 terms) and
 *                          contracted on the matrix cores with f32
 *                          accumulation in a fixed order; within 2e-3
 *                          normwise of mm_batched (grouped experts: 3e-3).
 * Every mode is run-to-run bit-identical: no floating-point atomics, fixed
 * reduction trees.
 *
 * Threading.  A context owns one HIP stream on one device.  Calls on one
 * context are serialized by the caller (like the reference's per-thread
 * adapter, rce-tinyllama/src/lib.rs L196-239); use one context per thread.
 * Host-pointer entry points are synchronous on return.  The *_dev entry
 * points are asynchronous on the stream they are given (NULL = the
 * context's stream).
 */
#ifndef RCE_QMM_H
#define RCE_QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2: GGUF files (rce_qmm_gguf_*, rce_qmm_weight_from_gguf) and the
 * NOT_FOUND / PARSE_ERROR / IO_ERROR statuses, added to version 1. */
#define RCE_QMM_ABI_VERSION 2u

typedef enum rce_qmm_status {
    RCE_QMM_OK = 0,
    RCE_QMM_NULL_ARGUMENT = 1,
    RCE_QMM_BAD_SHAPE = 2,
    RCE_QMM_UNSUPPORTED_DTYPE = 3,
    RCE_QMM_NO_DEVICE = 4,
    RCE_QMM_HIP_ERROR = 5,
    RCE_QMM_OUT_OF_MEMORY = 6,
    RCE_QMM_INTERNAL = 7,
    RCE_QMM_NOT_FOUND = 8,    /* a tensor or metadata key the file does not hold */
    RCE_QMM_PARSE_ERROR = 9,  /* not a GGUF v2/v3 file, or a malformed one */
    RCE_QMM_IO_ERROR = 10     /* the file could not be opened or mapped */
} rce_qmm_status;

/* GGUF type tags, as GgufDtype::to_u32 (rce-ingest-gguf/src/parser.rs
 * L343-378).  The library accepts any u32; rce_qmm_supports() says which
 * it computes on the GPU. */
enum {
    RCE_QMM_F32 = 0,
    RCE_QMM_F16 = 1,
    RCE_QMM_Q4_0 = 2,
    RCE_QMM_Q4_1 = 3,
    RCE_QMM_Q5_0 = 6,
    RCE_QMM_Q8_0 = 8,
    RCE_QMM_Q3_K = 11,
    RCE_QMM_Q4_K = 12,
    RCE_QMM_Q5_K = 13,
    RCE_QMM_Q6_K = 14,
    RCE_QMM_BF16 = 30
};

typedef enum rce_qmm_mode {
    RCE_QMM_MODE_EXACT = 0,
    RCE_QMM_MODE_Q8 = 1,
    RCE_QMM_MODE_F16_MFMA = 2
} rce_qmm_mode;

/* Opaque handles. */
typedef struct rce_qmm_context rce_qmm_context;
typedef struct rce_qmm_weight rce_qmm_weight;

/* ---- errors / version ------------------------------------------------ */

/* Text of the last failure on this thread ("" if none).  Mirrors
 * rce_last_error (compute/crates/rce-c/include/rce.h). */
const char *rce_qmm_last_error(void);
const char *rce_qmm_status_str(rce_qmm_status s);
uint32_t rce_qmm_abi_version(void);

/* ---- context ----------------------------------------------------------- */

/* Bind to HIP device `device`, create the context's stream and scratch.
 * Replaces MetalQmmContext::new (rce-op-qmm-metal/src/lib.rs L46-52):
 * no GPU -> RCE_QMM_NO_DEVICE (the caller then stays on the CPU path). */
rce_qmm_status rce_qmm_context_create(int device, rce_qmm_context **out);
/* Releases the caller's hold on the context.  Decoders made on it
 * (rce_qmm_llama_create) hold it too: it is freed when the last of them is
 * destroyed, so destroying the context first is safe. */
void rce_qmm_context_destroy(rce_qmm_context *ctx);
/* The hipStream_t the context launches on, as void*. */
rce_qmm_status rce_qmm_context_stream(rce_qmm_context *ctx, void **stream);
/* Wait for all work on the context's stream. */
rce_qmm_status rce_qmm_synchronize(rce_qmm_context *ctx);

/* 1 if the GPU computes (dtype, n_cols) in `mode`, else 0.  Same role as
 * MetalQmmContext::supports (rce-op-qmm-metal/src/lib.rs L127-139) and the
 * cost()=INFINITY decline of format-specific backends
 * (rce-placement-adapter/src/lib.rs L253-266). */
int rce_qmm_supports(uint32_t dtype, size_t n_cols, rce_qmm_mode mode);

/* ---- weights ------------------------------------------------------------ */

/* dtype arguments are GGUF type tags (parser.rs L306-378), except that
 * STQ1_0, which shares tag 42 with Q2_0 in files (hunyuan-dense files read
 * it as STQ1_0, parser.rs L529-541), is named RCE_QMM_DTYPE_STQ1_0 here.
 * I2_S weights are the ceil(n_rows * n_cols / 4) code bytes followed by the
 * tensor's one f32 scale. */
#define RCE_QMM_DTYPE_STQ1_0 0x8000002Au

/* A device-resident QuantWeight made from GGUF bytes: the weight
 * [n_rows = N_out, n_cols = K_in], row-major, each row k/QK blocks
 * (rce-op-qmm/src/lib.rs L60-91 QuantWeight, L123-138 from_owned_bytes).
 * The bytes are copied to HBM once, in a device layout of about the same
 * byte count (Q4_K / Q5_K / Q6_K add their matrix-core GEMM scales, 32 or
 * 64 bytes per super-block); the caller keeps its buffer.
 * len must equal n_rows * row_bytes(dtype, n_cols) (I2_S: plus its 4-byte scale). */
rce_qmm_status rce_qmm_weight_from_bytes(rce_qmm_context *ctx, uint32_t dtype, size_t n_rows,
                                         size_t n_cols, const uint8_t *bytes, size_t len,
                                         rce_qmm_weight **out);

/* QuantWeight::sub_view (rce-op-qmm/src/lib.rs L99-118) (not for I2_S: its
 * scale belongs to the whole tensor): a view of
 * byte_len bytes at byte_offset of `w`'s GGUF bytes, read as
 * [n_rows, n_cols].  Shares the device copy (no HBM copy).  The view must
 * start on a row boundary of `w` and keep n_cols (the stacked-expert case
 * of rce-qwen36-moe/src/lib.rs L216-223 split_experts); Q6_K views must
 * also start on a multiple of 64 rows.  Other views: RCE_QMM_BAD_SHAPE. */
rce_qmm_status rce_qmm_weight_sub_view(const rce_qmm_weight *w, size_t byte_offset,
                                       size_t byte_len, size_t n_rows, size_t n_cols,
                                       rce_qmm_weight **out);

/* Release a weight or view (the device copy is freed with the last one). */
void rce_qmm_weight_destroy(rce_qmm_weight *w);

/* dtype, shape and GGUF byte length of a weight (QuantWeight fields). */
rce_qmm_status rce_qmm_weight_info(const rce_qmm_weight *w, uint32_t *dtype, size_t *n_rows,
                                   size_t *n_cols, size_t *len);

/* ---- drop-in host-pointer entry points (synchronous, EXACT mode) --------- */

/* rce_op_qmm::mm_1d (rce-op-qmm/src/lib.rs L216-270): out[j] = sum_i a[i]
 * W[j,i] for a[n_cols] f32, out[n_rows] f32, bit-identical to the
 * reference's scalar kernels.  Unsupported dtype -> RCE_QMM_UNSUPPORTED_DTYPE
 * (the reference panics, L268; callers fall back to the CPU path). */
rce_qmm_status rce_qmm_mm_1d(rce_qmm_context *ctx, const float *a, const rce_qmm_weight *w,
                             float *out);

/* rce_op_qmm::mm_1d_serial (rce-op-qmm/src/lib.rs L281-304): the same
 * result as mm_1d (the reference differs only in host threading). */
rce_qmm_status rce_qmm_mm_1d_serial(rce_qmm_context *ctx, const float *a,
                                    const rce_qmm_weight *w, float *out);

/* rce_op_qmm::mm_batched (rce-op-qmm/src/lib.rs L967-1023): a [t_rows,
 * n_cols] -> out [t_rows, n_rows], byte-identical to t_rows calls of mm_1d. */
rce_qmm_status rce_qmm_mm_batched(rce_qmm_context *ctx, const float *a, size_t t_rows,
                                  const rce_qmm_weight *w, float *out);

/* QuantWeight::dequant_row (rce-op-qmm/src/lib.rs L150-167 ->
 * rce-ingest-gguf dequant.rs L115-134): row `row` as n_cols f32 values,
 * bit-identical to dequantize_to_f32. */
rce_qmm_status rce_qmm_dequant_row(rce_qmm_context *ctx, const rce_qmm_weight *w, size_t row,
                                   float *out);

/* GGUF bytes of f32 weights [n_rows, n_cols] (row-major) by the reference's
 * quantizers: Q8_0 / Q4_0 by quantize_block (rce-vm-backend-cpu/src/ml/nn.rs
 * L541-563, packed as spec/checker/tests/support/toy_gpt2.rs L46-58), Q4_K /
 * Q5_K / Q6_K by quantize_k + pack (kquant.rs L193-346).  len must equal n_rows *
 * row_bytes(dtype, n_cols).  Host only (no device needed); bit-identical for
 * any thread count.  Every input value is accepted: infinities, NaNs and
 * blocks whose 1/d overflows get the bytes of the reference's release build
 * (saturating float -> i32, wrapping adds, low bits kept by `as u8` / `as i8`
 * and by f16_bits, which writes an infinite scale as 0x3C00). */
rce_qmm_status rce_qmm_quantize(uint32_t dtype, const float *src, size_t n_rows, size_t n_cols, uint8_t *dst,
                                size_t len);

/* ---- device-resident entry points (asynchronous on `stream`) ------------ */

/* mm_batched on device buffers: a_dev [t_rows, n_cols] of a_dtype
 * (RCE_QMM_F32, or RCE_QMM_F16 whose values are widened exactly to f32 as
 * the reference's callers do), out_dev [t_rows, n_rows] f32.  No host
 * synchronization; the library's scratch is owned by the context, so calls
 * on one context must not overlap on different streams (one context per
 * stream).  RCE_QMM_MODE_F16_MFMA (the prefill form) takes Q4_K / Q4_0 /
 * Q5_K / Q6_K with n_cols a multiple of 256 and Q8_0 / Q5_0 / Q4_1 / F16 /
 * BF16 / F32 with n_cols a multiple of 64 (rce_qmm_supports); its F16
 * activations must be 16-byte aligned. */
rce_qmm_status rce_qmm_mm_batched_dev(rce_qmm_context *ctx, const void *a_dev, uint32_t a_dtype,
                                      size_t t_rows, const rce_qmm_weight *w, float *out_dev,
                                      rce_qmm_mode mode, void *stream);

/* No counterpart in the reference.  rce_qmm_mm_batched_dev for callers that
 * cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc): the same arguments,
 * kernels and bits, and no hipMalloc / hipFree / allocating library call.
 * The scratch the call needs -- 4 t_rows n_cols bytes to widen F16
 * activations (EXACT, Q8), 1.375 t_rows n_cols bytes for several tokens'
 * Q8 activations (Q8, t_rows >= 2), 2 t_rows n_cols bytes to round F32
 * activations to f16 (F16_MFMA), each rounded up to 256 -- comes from a
 * fixed device array of RCE_QMM_NOALLOC_SCRATCH_BYTES that each GPU the
 * library runs on holds until the process ends; a call that needs more
 * returns RCE_QMM_BAD_SHAPE.  All calls on one GPU share that array:
 * calls that overlap on one GPU (other streams, other contexts) race. */
#define RCE_QMM_NOALLOC_SCRATCH_BYTES (16u << 20)
rce_qmm_status rce_qmm_mm_batched_dev_noalloc(rce_qmm_context *ctx, const void *a_dev, uint32_t a_dtype,
                                              size_t t_rows, const rce_qmm_weight *w, float *out_dev,
                                              rce_qmm_mode mode, void *stream);

/* ---- grouped experts (MoE) ----------------------------------------------- */

/* rce_op_moe::moe_router (rce-op-moe/src/lib.rs L35-73) from given router
 * logits [n_tokens, n_expert] (host): softmax over all experts (max
 * subtracted, f32 exp), descending sort (ties: lower index first), top_k,
 * renormalized when `normalize`.  Writes ids/weights [n_tokens, top_k]. */
rce_qmm_status rce_qmm_moe_router(const float *logits, size_t n_tokens, size_t n_expert,
                                  size_t top_k, int normalize, int32_t *ids, float *weights);

/* Grouped-expert FFN on device buffers: for every token t and decision j,
 * e = ids[t, j]: h = silu(W1[e] x_t), y_j = W2[e] h, and
 * out_t = sum_j weights[t, j] * y_j in decision order from +0.0
 * (rce-qwen36-moe/src/lib.rs L667-710 with the router of rce-op-moe;
 * moe_combine L98-110).  w1[e]: [d_ff, d_model], w2[e]: [d_model, d_ff];
 * the w1 of one dtype, the w2 of one dtype (the two may differ, as a
 * Q4_K_M file's Q4_K gate with its Q6_K down).  x_dev [t_rows, d_model] f32, ids_dev [t_rows, top_k]
 * i32, weights_dev [t_rows, top_k] f32, out_dev [t_rows, d_model] f32.
 * Tokens are grouped per expert on the device (stable by expert, then
 * token, then decision). */
rce_qmm_status rce_qmm_moe_ffn_dev(rce_qmm_context *ctx, const rce_qmm_weight *const *w1,
                                   const rce_qmm_weight *const *w2, size_t n_expert,
                                   const float *x_dev, size_t t_rows, const int32_t *ids_dev,
                                   const float *weights_dev, size_t top_k, float *out_dev,
                                   rce_qmm_mode mode, void *stream);

/* The SwiGLU experts of rce-qwen36-moe (moe_ffn_forward's routed part,
 * src/lib.rs L667-703): for every token t and decision j, e = ids[t, j]:
 * g = gate[e] x_t, u = up[e] x_t, h = silu(g) * u, y_j = down[e] h
 * (swiglu_expert_serial, L667-676), out_t = sum_j weights[t, j] * y_j in
 * decision order from +0.0 (L698-703).  gate[e], up[e]: [d_ff, d_model],
 * down[e]: [d_model, d_ff]; gate and up of one dtype, down of one dtype
 * (it may differ from theirs); buffers and grouping as
 * rce_qmm_moe_ffn_dev.  The shared expert and its sigmoid gate (L704-709)
 * stay with the caller (for instance one more call with n_expert = 1 and
 * the per-token gate as the weight). */
rce_qmm_status rce_qmm_moe_swiglu_dev(rce_qmm_context *ctx, const rce_qmm_weight *const *gate,
                                      const rce_qmm_weight *const *up, const rce_qmm_weight *const *down,
                                      size_t n_expert, const float *x_dev, size_t t_rows,
                                      const int32_t *ids_dev, const float *weights_dev, size_t top_k,
                                      float *out_dev, rce_qmm_mode mode, void *stream);

/* ---- Llama-2 decode step (the TinyLlama caller) -------------------------- */

/* TinyLlamaConfig (rce-tinyllama/src/lib.rs L28-41); d_head = d_model /
 * n_q_heads there, given explicitly here. */
typedef struct rce_qmm_llama_config {
    size_t d_model, vocab, n_layers, n_q_heads, n_kv_heads, d_head, rope_dim, d_ff, context_length;
    float rope_freq_base, eps;
} rce_qmm_llama_config;

/* TinyLlamaBlock (rce-tinyllama/src/lib.rs L94-99): host f32 norm weights
 * [d_model] (copied at creation) and weight handles wq [n_q*d_head,
 * d_model], wk / wv [n_kv*d_head, d_model], wo [d_model, n_q*d_head],
 * ffn_gate / ffn_up [d_ff, d_model], ffn_down [d_model, d_ff]. */
typedef struct rce_qmm_llama_block {
    const float *attn_norm, *ffn_norm;
    const rce_qmm_weight *wq, *wk, *wv, *wo, *ffn_gate, *ffn_up, *ffn_down;
} rce_qmm_llama_block;

/* A device-resident decoder: weights (shared with the handles given, which
 * may be destroyed afterwards), KV caches of context_length positions and the
 * decode-step state (TinyLlamaState, L144-155).  Every linear runs on the
 * decode GEMV kernels in `mode` (EXACT or Q8) -- the qmm_1d calls of
 * forward_embedding (L303-330) and attn_block (L252-287) -- and the steps
 * between them (rms_norm, RoPE, attention, silu, residual adds) run on the
 * device; one step is replayed from a HIP graph.
 * Numerics: EXACT linears are the reference's bit for bit given their
 * inputs; rms_norm's sum of squares is a fixed tree instead of a sequential
 * fold and exp / silu use the device expf, so logits match the reference
 * to a tolerance, not bitwise.  Run-to-run bit-identical. */
typedef struct rce_qmm_llama rce_qmm_llama;

rce_qmm_status rce_qmm_llama_create(rce_qmm_context *ctx, const rce_qmm_llama_config *cfg,
                                    const rce_qmm_weight *token_embd, const float *output_norm,
                                    const rce_qmm_weight *lm_head, const rce_qmm_llama_block *blocks,
                                    rce_qmm_mode mode, rce_qmm_llama **out);
void rce_qmm_llama_destroy(rce_qmm_llama *m);

/* TinyLlamaRuntime::new_state (L355): position 0, empty caches. */
rce_qmm_status rce_qmm_llama_reset(rce_qmm_llama *m);
/* TinyLlamaState::pos: positions decoded since the last reset (a step
 * queued by rce_qmm_llama_forward_token_dev counts until
 * rce_qmm_llama_check reports it skipped). */
rce_qmm_status rce_qmm_llama_pos(const rce_qmm_llama *m, size_t *pos);

/* forward_logits / forward_token (L356, L289-294): logits [vocab] (host)
 * of token_id at the current position, which then advances.  Synchronous.
 * token_id outside [0, token_embd rows) or a full cache: RCE_QMM_BAD_SHAPE
 * (the reference panics), state unchanged. */
rce_qmm_status rce_qmm_llama_forward_token(rce_qmm_llama *m, int32_t token_id, float *logits);
/* forward_logits_embed / forward_embedding (L362, L303-330): the same
 * from a [d_model] input embedding (host).  Synchronous. */
rce_qmm_status rce_qmm_llama_forward_embedding(rce_qmm_llama *m, const float *embedding, float *logits);
/* forward_token on device memory, asynchronous on `stream` (NULL = the
 * context's stream): token id read from token_dev, logits written to
 * logits_dev [vocab].  A full cache is RCE_QMM_BAD_SHAPE at the call.  A
 * token id out of range, found on the device, skips that step: no cache
 * row is written and the position does not advance, so later steps decode
 * as if it had not been given; its logits are undefined, and
 * rce_qmm_llama_check reports it. */
rce_qmm_status rce_qmm_llama_forward_token_dev(rce_qmm_llama *m, const int32_t *token_dev, float *logits_dev,
                                               void *stream);
/* Wait for the decoder's work -- on the context's stream and on the stream
 * of the last rce_qmm_llama_forward_token_dev call -- and report (then
 * clear) an error found on the device since the last check:
 * RCE_QMM_BAD_SHAPE for token ids out of range (the position then counts
 * only the steps that ran). */
rce_qmm_status rce_qmm_llama_check(rce_qmm_llama *m);

/* ---- the "hip:op-qmm" priced backend (rce-placement-adapter) ------------- */

/* The adapter's qmm dtype ids (QMM_DTYPE_*, rce-placement-adapter/src/lib.rs
 * L80-90: 1 Q8_0, 2 Q4_K, 3 Q5_K, 4 Q6_K, 5 Q4_0, 6 Q5_0, 7 Q4_1, 8 Q1_0,
 * 9 Q2_0, 10 Q3_K) as GGUF tags; 0 for QMM_DTYPE_UNKNOWN (0) and any other id. */
uint32_t rce_qmm_dtype_for_qmm_id(size_t qmm_dtype_id);

/* The library's analytical prior (basis est) for the ("qmm", "hip:op-qmm")
 * cost cell, in the units of LinearCoeffs (rce-placement L231-242): pJ per
 * FLOP, pJ per byte, pJ per call.  Replaces nothing in the reference; it is
 * the cell default_qmm_cost_table (adapter L163-182) inserts for MetalQmm. */
void rce_qmm_hip_cost_prior(double *a_pj_per_flop, double *b_pj_per_byte, double *c_pj_overhead);

/* HipQmm::cost (the PricedBackend::cost of CpuQmm / MetalQmm, adapter
 * L214-266) for op "qmm": a_shape = [k], w_shape = [n_rows, n_cols,
 * weight_bytes, dtype_id].  *picojoules = +inf when the GPU declines (short
 * shapes, an id without a tag, no kernel for (tag, n_cols)): pick_priced
 * then routes the call to CpuQmm.  Else a * flops + b * bytes + c with
 * qmm_1d_flops_bytes (L141-145): flops = 2 n k, bytes = weight_bytes + 4 k
 * + 4 n.  The coefficients are the cell's (the caller's CostTable may have
 * calibrated them). */
rce_qmm_status rce_qmm_hip_cost(const size_t *a_shape, size_t a_len, const size_t *w_shape, size_t w_len,
                                double a_pj_per_flop, double b_pj_per_byte, double c_pj_overhead,
                                double *picojoules);

/* The GPU's accumulated energy in microjoules (ROCm SMI's energy counter,
 * opened at first use), and the reading's timestamp in ns: what an
 * EnergyMeter (adapter L48-74) for HIP dispatches brackets a call with, as
 * SubstrateEnergyMeter does with RAPL (substrate_meter.rs L104-130); its
 * basis is `reported`.  `device` is ROCm SMI's index (the HIP index on a
 * one-GPU node).  On MI355X the counter advances once a second (15.3 uJ
 * units): a window shorter than that reads 0, as the reference's meter
 * expects of tiny dispatches; calibrate over windows of seconds.
 * RCE_QMM_NOT_FOUND where no counter can be read. */
rce_qmm_status rce_qmm_energy_read(int device, uint64_t *microjoules, uint64_t *timestamp_ns);

/* ---- GGUF files (rce-ingest-gguf) ---------------------------------------- */

/* A parsed GGUF v2/v3 file: header, metadata and tensor infos
 * (GgufFile, parser.rs L431-446).  Strings and value bytes handed out
 * below stay valid until rce_qmm_gguf_close. */
typedef struct rce_qmm_gguf rce_qmm_gguf;

/* GgufFile::parse (parser.rs L446-551) over the caller's bytes, which must
 * outlive the handle.  Never reads tensor data.  RCE_QMM_PARSE_ERROR with
 * the reference's error text for a bad magic, a version outside 2..=3, a
 * truncated file, invalid UTF-8, an unknown value type or more than 8
 * dimensions. */
rce_qmm_status rce_qmm_gguf_parse(const uint8_t *bytes, size_t len, rce_qmm_gguf **out);
/* mmap_load_sequential + GgufFile::parse (mmap.rs, parser.rs L446): the
 * file is mapped read-only for the handle's lifetime; RCE_QMM_IO_ERROR
 * when it cannot be opened or mapped. */
rce_qmm_status rce_qmm_gguf_open(const char *path, rce_qmm_gguf **out);
void rce_qmm_gguf_close(rce_qmm_gguf *g);
/* version, tensor and metadata counts, data_offset (absolute start of the
 * tensor data: the end of the infos padded to alignment) and alignment
 * (general.alignment if U32/U64, else 32) (GgufFile fields, L431-445). */
rce_qmm_status rce_qmm_gguf_header(const rce_qmm_gguf *g, uint32_t *version, size_t *n_tensors, size_t *n_metadata,
                                   uint64_t *data_offset, uint64_t *alignment);
/* Metadata entry i (GgufMetadata): key, value type tag (GGUF_TYPE_*,
 * parser.rs L187-199) and the value's bytes as encoded in the file (little
 * endian; strings and arrays with their length prefixes). */
rce_qmm_status rce_qmm_gguf_metadata(const rce_qmm_gguf *g, size_t i, const char **key, uint32_t *type,
                                     const uint8_t **value, size_t *value_len);
/* The first metadata entry with this key (get_metadata, L553);
 * RCE_QMM_NOT_FOUND if none. */
rce_qmm_status rce_qmm_gguf_find_metadata(const rce_qmm_gguf *g, const char *key, size_t *index);
/* Tensor info i (GgufTensorInfo, L404-418): name, dims (ne0 first; dims
 * must hold 8), GGUF dtype tag, offset relative to data_offset, and its
 * size in the file (tensor_byte_size, dequant.rs L18-60; 0 for dtypes
 * with no size rule; tag 42 sized as STQ1_0 in hunyuan-dense files). */
rce_qmm_status rce_qmm_gguf_tensor(const rce_qmm_gguf *g, size_t i, const char **name, uint32_t *ndim, uint64_t *dims,
                                   uint32_t *dtype, uint64_t *offset, uint64_t *nbytes);
rce_qmm_status rce_qmm_gguf_find_tensor(const rce_qmm_gguf *g, const char *name, size_t *index);
/* QuantWeight::from_gguf (rce-op-qmm/src/lib.rs L173-209): the tensor
 * `name` as a device-resident weight of the declared [n_rows, n_cols]
 * (n_rows * n_cols must equal the tensor's element count, and its bytes
 * must lie inside the file), then as rce_qmm_weight_from_bytes.  The
 * handle can be closed afterwards: the weight holds its own device copy. */
rce_qmm_status rce_qmm_weight_from_gguf(rce_qmm_context *ctx, const rce_qmm_gguf *g, const char *name, size_t n_rows,
                                        size_t n_cols, rce_qmm_weight **out);
/* read_tensor_f32 (dequant.rs L85-112) for F32, F16 and BF16 tensors (norm
 * weights): n must equal the element count. */
rce_qmm_status rce_qmm_gguf_read_f32(const rce_qmm_gguf *g, const char *name, float *out, size_t n);

/* ---- measurement ---------------------------------------------------------- */

/* No counterpart in the reference: one launch on `stream` that reads
 * `bytes` (a multiple of 16, 16-byte aligned) of buf_dev once and does
 * nothing else, the HBM read rate a single decode-GEMV launch of that byte
 * count could reach (launch cost and ramp included).  sink_dev: 4 writable
 * bytes (written only if the buffer's XOR-fold hits one fixed word).  variant 0..8 picks a launch
 * shape (one pass of 256 threads x 4 / 8 / 16 loads, 1024 x 8, 256 x 8
 * non-temporal, grid-stride 1024 or 2048 blocks of 256 x 8, 512 blocks of
 * 512 x 8, one pass of 512 x 4); 9 launches one empty block. */
rce_qmm_status rce_qmm_read_ceiling_dev(rce_qmm_context *ctx, const void *buf_dev, size_t bytes, void *sink_dev,
                                        int variant, void *stream);

/* ---- device memory helpers (for callers without a HIP runtime) ---------- */

rce_qmm_status rce_qmm_dev_alloc(rce_qmm_context *ctx, size_t bytes, void **out);
rce_qmm_status rce_qmm_dev_free(rce_qmm_context *ctx, void *p);
rce_qmm_status rce_qmm_memcpy_h2d(rce_qmm_context *ctx, void *dst, const void *src, size_t bytes);
rce_qmm_status rce_qmm_memcpy_d2h(rce_qmm_context *ctx, void *dst, const void *src, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* RCE_QMM_H */
