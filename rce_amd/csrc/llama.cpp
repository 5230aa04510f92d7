// llama.cpp -- the device-resident Llama-2 decode step behind the
// rce_qmm_llama_* entry points (include/rce_qmm.h): the TinyLlama runtime's
// forward_embedding / attn_block (rce-tinyllama/src/lib.rs L252-330) with
// every qmm_1d on the decode GEMV kernels and the steps between them on the
// device (decoder.hip), one step recorded once into a HIP graph.
//
// Kernels of one step (L layers):
//   [embed row]            outside the graph, token input only
//   per layer:
//     q | k | v = W{q,k,v} rms_norm(x)  one FX_SEG | FX_NORM launch when the
//                                       three weights share format and width
//     attention                         RoPE, cache append, softmax . V
//     x = x + Wo att                    FX_RESIDUAL
//     h = silu(Wg n) * (Wu n),          FX_SWIGLU | FX_NORM when gate and up
//         n = rms_norm(x)               share format
//     x = x + Wd h                      FX_RESIDUAL
//   logits = lm_head rms_norm(x, output_norm)   one FX_SEG | FX_NORM launch
//                                       that also advances the position (or
//                                       a separate rms_norm that does)
// Every kernel of a step reads the position from pos (device memory), so
// the recorded graph replays for any position.  Linears whose format has no
// fused form run as a separate rms_norm and plain GEMVs followed by the
// unfused add / swiglu kernels.
#include "abi_internal.h"

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>

using namespace rce_qmm;
using namespace rce_qmm_abi;

struct rce_qmm_llama {
    rce_qmm_context *ctx = nullptr;
    rce_qmm_llama_config cfg{};
    int mode = 0;
    std::vector<std::shared_ptr<DevAlloc>> keep;  // the weights' device memory
    DevWeight embd{}, head{};
    struct Layer {
        DevWeight wq, wk, wv, wo, gate, up, down;
        bool qkv_seg = false, wo_res = false, ffn_swiglu = false, down_res = false;
        bool qkv_norm = false, ffn_norm = false;  // the fused forms also form rms_norm
    };
    bool head_norm = false;  // the head GEMV forms the output rms_norm and advances the position
    std::vector<Layer> layers;
    // device memory (one allocation)
    void *mem = nullptr;
    float *x = nullptr, *xn = nullptr, *qkv = nullptr, *att = nullptr, *h = nullptr, *g = nullptr, *u = nullptr,
          *o = nullptr, *logits = nullptr, *norms = nullptr, *rope_cs = nullptr, *kc = nullptr, *vc = nullptr;
    int *pos_dev = nullptr, *status = nullptr, *token = nullptr;  // status: the three words of launch_embed_row
    // pinned host staging
    int32_t *h_token = nullptr;
    int *h_status = nullptr;
    float *h_logits = nullptr;
    size_t pos = 0;  // host mirror of pos_dev (plus the skipped steps not yet checked)
    hipEvent_t last_dev = nullptr;  // after the last forward_token_dev step, on the caller's stream
    bool last_dev_pending = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    float *graph_logits = nullptr;  // where the captured graph writes logits
    bool eager = false;  // RCE_QMM_LLAMA_GRAPH=0: launch the step's kernels one by one (tools that
                         // cannot follow graph replays)

    size_t qd() const { return cfg.n_q_heads * cfg.d_head; }
    size_t kvd() const { return cfg.n_kv_heads * cfg.d_head; }
    float *attn_norm(size_t il) const { return norms + (2 * il) * cfg.d_model; }
    float *ffn_norm(size_t il) const { return norms + (2 * il + 1) * cfg.d_model; }
    float *out_norm() const { return norms + 2 * cfg.n_layers * cfg.d_model; }
    // positions rounded up to whole 64-position key tiles (decoder.hip)
    size_t cache_layer() const { return ((cfg.context_length + 63) / 64 * 64) * kvd(); }
};

namespace {

void drop_graph(rce_qmm_llama *m) {
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    m->exec = nullptr;
    m->graph = nullptr;
    m->graph_logits = nullptr;
}

rce_qmm_status check_linear(const char *name, size_t il, const rce_qmm_weight *w, size_t rows, size_t cols, int mode,
                            int device) {
    const std::string where = std::string(name) + (il == (size_t)-1 ? "" : " of layer " + std::to_string(il));
    if (!w) return fail(RCE_QMM_NULL_ARGUMENT, "null weight: " + where);
    if (w->device != device) return fail(RCE_QMM_BAD_SHAPE, where + " lives on another device");
    if (w->dw.n_rows != rows || w->dw.n_cols != cols)
        return fail(RCE_QMM_BAD_SHAPE, where + " is [" + std::to_string(w->dw.n_rows) + ", " +
                                           std::to_string(w->dw.n_cols) + "], expected [" + std::to_string(rows) + ", " +
                                           std::to_string(cols) + "]");
    if (!gpu_supports(w->dw.dtype, w->dw.n_cols, mode))
        return fail(RCE_QMM_UNSUPPORTED_DTYPE, where + ": dtype " + std::to_string(w->dw.dtype) + " with n_cols " +
                                                   std::to_string(cols) + " has no decode kernel in this mode");
    return RCE_QMM_OK;
}

bool fx_ok(const DevWeight &w, int mode) { return gemv_fx_supports(w.dtype, w.n_cols, mode); }

// Unwritten KV-cache rows hold quiet NaNs (at creation and after a reset),
// so a kernel that lets a row past the position into a result shows it
// as NaN instead of depending on what the memory held.
hipError_t poison_caches(rce_qmm_llama *m, hipStream_t s) {
    const size_t n = m->cfg.n_layers * m->cache_layer();
    hipError_t e = hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(m->kc), 0x7fc00000, n, s);
    if (e == hipSuccess) e = hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(m->vc), 0x7fc00000, n, s);
    return e;
}

// The step's kernels after the input embedding is in x.
rce_qmm_status enqueue_body(rce_qmm_llama *m, float *logits, hipStream_t s) {
    const rce_qmm_llama_config &c = m->cfg;
    const size_t dm = c.d_model, qd = m->qd(), kvd = m->kvd();
    const int ctx_len = (int)c.context_length;
    const float scale = 1.0f / std::sqrt((float)c.d_head);  // rce-tinyllama L269
    auto norm = [&](const float *w, int *pos) {
        return launch_rms_norm(m->x, w, dm, c.eps, m->xn, pos, ctx_len, m->status, s);
    };
    for (size_t il = 0; il < c.n_layers; il++) {
        const rce_qmm_llama::Layer &L = m->layers[il];
        float *kc = m->kc + il * m->cache_layer(), *vc = m->vc + il * m->cache_layer();
        if (!L.qkv_norm) HIP_TRY(norm(m->attn_norm(il), nullptr));
        if (L.qkv_seg) {
            FxLaunch f;
            f.kind = L.qkv_norm ? (FX_SEG | FX_NORM) : FX_SEG;
            f.nw = 3;
            f.w[0] = L.wq; f.w[1] = L.wk; f.w[2] = L.wv;
            f.out[0] = m->qkv; f.out[1] = m->qkv + qd; f.out[2] = m->qkv + qd + kvd;
            f.norm_w = m->attn_norm(il);
            f.eps = c.eps;
            HIP_TRY(launch_gemv_fx(f, L.qkv_norm ? m->x : m->xn, m->mode, s));
        } else {
            HIP_TRY(launch_gemv(L.wq, m->xn, 1, m->qkv, m->mode, s));
            HIP_TRY(launch_gemv(L.wk, m->xn, 1, m->qkv + qd, m->mode, s));
            HIP_TRY(launch_gemv(L.wv, m->xn, 1, m->qkv + qd + kvd, m->mode, s));
        }
        HIP_TRY(launch_attention(m->qkv, m->rope_cs, kc, vc, m->pos_dev, ctx_len, (int)c.n_q_heads, (int)c.n_kv_heads,
                                 (int)c.d_head, (int)c.rope_dim, scale, m->att, m->status + 2, s));
        if (L.wo_res) {
            FxLaunch f;
            f.kind = FX_RESIDUAL;
            f.w[0] = L.wo;
            f.out[0] = m->x;
            f.res = m->x;
            HIP_TRY(launch_gemv_fx(f, m->att, m->mode, s));
        } else {
            HIP_TRY(launch_gemv(L.wo, m->att, 1, m->o, m->mode, s));
            HIP_TRY(launch_add_inplace(m->x, m->o, dm, s));
        }
        if (!L.ffn_norm) HIP_TRY(norm(m->ffn_norm(il), nullptr));
        if (L.ffn_swiglu) {
            FxLaunch f;
            f.kind = L.ffn_norm ? (FX_SWIGLU | FX_NORM) : FX_SWIGLU;
            f.nw = 2;
            f.w[0] = L.gate; f.w[1] = L.up;
            f.out[0] = m->h;
            f.norm_w = m->ffn_norm(il);
            f.eps = c.eps;
            HIP_TRY(launch_gemv_fx(f, L.ffn_norm ? m->x : m->xn, m->mode, s));
        } else {
            HIP_TRY(launch_gemv(L.gate, m->xn, 1, m->g, m->mode, s));
            HIP_TRY(launch_gemv(L.up, m->xn, 1, m->u, m->mode, s));
            HIP_TRY(launch_swiglu(m->g, m->u, m->h, c.d_ff, s));
        }
        if (L.down_res) {
            FxLaunch f;
            f.kind = FX_RESIDUAL;
            f.w[0] = L.down;
            f.out[0] = m->x;
            f.res = m->x;
            HIP_TRY(launch_gemv_fx(f, m->h, m->mode, s));
        } else {
            HIP_TRY(launch_gemv(L.down, m->h, 1, m->o, m->mode, s));
            HIP_TRY(launch_add_inplace(m->x, m->o, dm, s));
        }
    }
    if (m->head_norm) {  // the step's last kernel advances the position
        FxLaunch f;
        f.kind = FX_SEG | FX_NORM;
        f.w[0] = m->head;
        f.out[0] = logits;
        f.norm_w = m->out_norm();
        f.eps = c.eps;
        f.pos = m->pos_dev;
        f.status = m->status;
        f.ctx_len = ctx_len;
        HIP_TRY(launch_gemv_fx(f, m->x, m->mode, s));
    } else {
        HIP_TRY(norm(m->out_norm(), m->pos_dev));  // the step's last reader of pos advances it
        HIP_TRY(launch_gemv(m->head, m->xn, 1, logits, m->mode, s));
    }
    return RCE_QMM_OK;
}

// The graph of one step writing `logits`, recorded on first use (and again
// when the caller's logits buffer changes).
rce_qmm_status graph_for(rce_qmm_llama *m, float *logits, hipStream_t s) {
    if (m->exec && m->graph_logits == logits) return RCE_QMM_OK;
    drop_graph(m);
    HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    rce_qmm_status st = enqueue_body(m, logits, s);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(s, &g);
    if (st) {
        if (g) (void)hipGraphDestroy(g);
        return st;
    }
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
    e = hipGraphInstantiate(&m->exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        m->exec = nullptr;
        return hip_fail(e, "hipGraphInstantiate");
    }
    m->graph = g;
    m->graph_logits = logits;
    return RCE_QMM_OK;
}

rce_qmm_status run_step(rce_qmm_llama *m, float *logits, hipStream_t s) {
    if (m->pos >= m->cfg.context_length)
        return fail(RCE_QMM_BAD_SHAPE, "the KV cache is full (context_length " + std::to_string(m->cfg.context_length) + ")");
    if (m->eager) {
        rce_qmm_status st = enqueue_body(m, logits, s);
        if (st) return st;
    } else {
        rce_qmm_status st = graph_for(m, logits, s);
        if (st) return st;
        HIP_TRY(hipGraphLaunch(m->exec, s));
    }
    m->pos++;
    return RCE_QMM_OK;
}

// Wait for the decoder's work on `s` and on the stream of the last
// forward_token_dev step, read the device status and clear it.  Steps
// skipped for a bad token id did not advance the device position: the host
// mirror gives them back.
rce_qmm_status take_status(rce_qmm_llama *m, hipStream_t s) {
    if (m->last_dev_pending) {
        HIP_TRY(hipEventSynchronize(m->last_dev));
        m->last_dev_pending = false;
    }
    HIP_TRY(hipMemcpyAsync(m->h_status, m->status, 2 * sizeof(int), hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    const int code = m->h_status[0], skipped = m->h_status[1];
    if (code == 0) return RCE_QMM_OK;
    HIP_TRY(hipMemsetAsync(m->status, 0, 2 * sizeof(int), s));
    HIP_TRY(hipStreamSynchronize(s));
    m->pos -= std::min<size_t>(m->pos, (size_t)std::max(skipped, 0));
    if (code == 1)
        return fail(RCE_QMM_BAD_SHAPE, "token id out of range of token_embd (" + std::to_string(skipped) +
                                           " step(s) skipped: no cache row, no position advance)");
    return fail(RCE_QMM_BAD_SHAPE, "decode position past the KV cache");
}

rce_qmm_status finish_host(rce_qmm_llama *m, float *logits, hipStream_t s) {
    const size_t vb = m->cfg.vocab * sizeof(float);
    HIP_TRY(hipMemcpyAsync(m->h_logits, m->logits, vb, hipMemcpyDeviceToHost, s));
    rce_qmm_status st = take_status(m, s);
    if (st) return st;
    std::memcpy(logits, m->h_logits, vb);
    return RCE_QMM_OK;
}

}  // namespace

extern "C" {

rce_qmm_status rce_qmm_llama_create(rce_qmm_context *ctx, const rce_qmm_llama_config *cfg,
                                    const rce_qmm_weight *token_embd, const float *output_norm,
                                    const rce_qmm_weight *lm_head, const rce_qmm_llama_block *blocks,
                                    rce_qmm_mode mode, rce_qmm_llama **out) {
    if (!ctx || !cfg || !token_embd || !output_norm || !lm_head || !out || (cfg->n_layers && !blocks))
        return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    *out = nullptr;
    if (mode != RCE_QMM_MODE_EXACT && mode != RCE_QMM_MODE_Q8)
        return fail(RCE_QMM_UNSUPPORTED_DTYPE, "the decoder runs its linears in EXACT or Q8 mode");
    const rce_qmm_llama_config c = *cfg;
    const int md = (int)mode;
    if (c.d_model == 0 || c.vocab == 0 || c.n_q_heads == 0 || c.n_kv_heads == 0 || c.context_length == 0 ||
        c.n_q_heads % c.n_kv_heads)
        return fail(RCE_QMM_BAD_SHAPE, "config: zero size or n_q_heads not a multiple of n_kv_heads");
    if (c.context_length > (size_t)1 << 30) return fail(RCE_QMM_BAD_SHAPE, "config: context_length too large");
    if (!attention_supports((int)c.d_head, (int)c.rope_dim, c.context_length, c.n_kv_heads))
        return fail(RCE_QMM_BAD_SHAPE, "config: d_head must be 64 or 128, rope_dim even and <= d_head, and one "
                                       "layer's KV cache under 2 GiB");
    const size_t dm = c.d_model, qd = c.n_q_heads * c.d_head, kvd = c.n_kv_heads * c.d_head;
    rce_qmm_status st;
    if (token_embd->device != ctx->device) return fail(RCE_QMM_BAD_SHAPE, "token_embd lives on another device");
    if (token_embd->dw.n_cols != dm) return fail(RCE_QMM_BAD_SHAPE, "token_embd must have d_model columns");
    if ((st = check_linear("lm_head", (size_t)-1, lm_head, c.vocab, dm, md, ctx->device))) return st;
    for (size_t il = 0; il < c.n_layers; il++) {
        const rce_qmm_llama_block &b = blocks[il];
        if (!b.attn_norm || !b.ffn_norm) return fail(RCE_QMM_NULL_ARGUMENT, "null norm weight of layer " + std::to_string(il));
        if ((st = check_linear("wq", il, b.wq, qd, dm, md, ctx->device))) return st;
        if ((st = check_linear("wk", il, b.wk, kvd, dm, md, ctx->device))) return st;
        if ((st = check_linear("wv", il, b.wv, kvd, dm, md, ctx->device))) return st;
        if ((st = check_linear("wo", il, b.wo, dm, qd, md, ctx->device))) return st;
        if ((st = check_linear("ffn_gate", il, b.ffn_gate, c.d_ff, dm, md, ctx->device))) return st;
        if ((st = check_linear("ffn_up", il, b.ffn_up, c.d_ff, dm, md, ctx->device))) return st;
        if ((st = check_linear("ffn_down", il, b.ffn_down, dm, c.d_ff, md, ctx->device))) return st;
    }
    if ((st = set_device(ctx->device))) return st;

    rce_qmm_llama *m = new (std::nothrow) rce_qmm_llama();
    if (!m) return fail(RCE_QMM_OUT_OF_MEMORY, "decoder object");
    m->ctx = ctx;
    ctx->refs.fetch_add(1);  // released by rce_qmm_llama_destroy
    m->cfg = c;
    m->mode = md;
    if (const char *g = std::getenv("RCE_QMM_LLAMA_GRAPH")) m->eager = g[0] == '0';
    auto keep = [&](const rce_qmm_weight *w) { m->keep.push_back(w->alloc); return w->dw; };
    m->embd = keep(token_embd);
    m->head = keep(lm_head);
    m->head_norm = gemv_fx_supports(m->head.dtype, m->head.n_cols, md, true) &&
                   std::getenv("RCE_QMM_LLAMA_NORM_KERNEL") == nullptr;
    for (size_t il = 0; il < c.n_layers; il++) {
        const rce_qmm_llama_block &b = blocks[il];
        rce_qmm_llama::Layer L;
        L.wq = keep(b.wq); L.wk = keep(b.wk); L.wv = keep(b.wv); L.wo = keep(b.wo);
        L.gate = keep(b.ffn_gate); L.up = keep(b.ffn_up); L.down = keep(b.ffn_down);
        L.qkv_seg = fx_ok(L.wq, md) && L.wk.dtype == L.wq.dtype && L.wv.dtype == L.wq.dtype;
        L.qkv_norm = L.qkv_seg && gemv_fx_supports(L.wq.dtype, L.wq.n_cols, md, true) &&
                     std::getenv("RCE_QMM_LLAMA_NORM_KERNEL") == nullptr;
        L.wo_res = fx_ok(L.wo, md);
        L.ffn_swiglu = fx_ok(L.gate, md) && L.up.dtype == L.gate.dtype;
        L.ffn_norm = L.ffn_swiglu && gemv_fx_supports(L.gate.dtype, L.gate.n_cols, md, true) &&
                     std::getenv("RCE_QMM_LLAMA_NORM_KERNEL") == nullptr;
        L.down_res = fx_ok(L.down, md);
        m->layers.push_back(L);
    }

    // device memory: activations, norms, RoPE table, KV caches, counters
    const size_t half = c.rope_dim / 2;
    const size_t big = std::max(c.d_ff, qd);
    const size_t n_f[] = {dm, dm, qd + 2 * kvd, qd, c.d_ff, c.d_ff, c.d_ff, std::max(dm, big), c.vocab,
                          (2 * c.n_layers + 1) * dm, c.context_length * std::max<size_t>(half, 1) * 2,
                          c.n_layers * m->cache_layer(), c.n_layers * m->cache_layer()};
    constexpr int NF = sizeof(n_f) / sizeof(n_f[0]);
    size_t off[NF + 1], total = 0;
    for (int i = 0; i < NF; i++) {
        off[i] = total;
        total = align_up(total + n_f[i] * sizeof(float), 256);
    }
    off[NF] = total;
    const size_t int_bytes = 256;  // pos, status, token
    total += int_bytes;
    hipError_t e = hipMalloc(&m->mem, total);
    if (e != hipSuccess) {
        m->mem = nullptr;
        delete m;
        return fail(RCE_QMM_OUT_OF_MEMORY, std::string("decoder hipMalloc: ") + hipGetErrorString(e));
    }
    char *base = static_cast<char *>(m->mem);
    float **fp[] = {&m->x, &m->xn, &m->qkv, &m->att, &m->h, &m->g, &m->u, &m->o, &m->logits,
                    &m->norms, &m->rope_cs, &m->kc, &m->vc};
    static_assert(sizeof(fp) / sizeof(fp[0]) == NF, "one pointer per buffer");
    for (int i = 0; i < NF; i++) *fp[i] = reinterpret_cast<float *>(base + off[i]);
    int *ints = reinterpret_cast<int *>(base + off[NF]);
    m->pos_dev = ints;
    m->token = ints + 1;
    m->status = ints + 4;
    auto cleanup = [&](rce_qmm_status s2) {
        rce_qmm_llama_destroy(m);
        return s2;
    };
    if (hipHostMalloc(reinterpret_cast<void **>(&m->h_token), 64, hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void **>(&m->h_status), 64, hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void **>(&m->h_logits), c.vocab * sizeof(float), hipHostMallocDefault) !=
            hipSuccess)
        return cleanup(fail(RCE_QMM_OUT_OF_MEMORY, "decoder pinned staging"));
    if ((e = hipEventCreateWithFlags(&m->last_dev, hipEventDisableTiming)) != hipSuccess)
        return cleanup(hip_fail(e, "decoder event"));

    // norm weights [attn_norm, ffn_norm] per layer, then output_norm
    std::vector<float> norms((2 * c.n_layers + 1) * dm);
    for (size_t il = 0; il < c.n_layers; il++) {
        std::memcpy(&norms[(2 * il) * dm], blocks[il].attn_norm, dm * sizeof(float));
        std::memcpy(&norms[(2 * il + 1) * dm], blocks[il].ffn_norm, dm * sizeof(float));
    }
    std::memcpy(&norms[2 * c.n_layers * dm], output_norm, dm * sizeof(float));
    // rope_inplace_scaled (rce-op-attn/src/lib.rs L115-151), per position
    // and pair i: inv_freq = 1 / exp(ln(base) * (2i) / rope_dim), theta =
    // pos * inv_freq, with the C library's logf / expf / sinf / cosf.
    std::vector<float> cs(c.context_length * std::max<size_t>(half, 1) * 2, 0.0f);
    const float log_base = logf(c.rope_freq_base);
    std::vector<float> inv_freq(half);
    for (size_t i = 0; i < half; i++) {
        float ex = log_base * (2.0f * (float)i);
        ex = ex / (float)c.rope_dim;
        inv_freq[i] = 1.0f / expf(ex);
    }
    for (size_t p = 0; p < c.context_length; p++)
        for (size_t i = 0; i < half; i++) {
            const float theta = (float)p * inv_freq[i];
            cs[(p * half + i) * 2] = cosf(theta);
            cs[(p * half + i) * 2 + 1] = sinf(theta);
        }
    hipStream_t s = ctx->stream;
    if ((e = hipMemcpyAsync(m->norms, norms.data(), norms.size() * sizeof(float), hipMemcpyHostToDevice, s)) ||
        (e = hipMemcpyAsync(m->rope_cs, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice, s)) ||
        (e = poison_caches(m, s)) || (e = hipMemsetAsync(ints, 0, int_bytes, s)) || (e = hipStreamSynchronize(s)))
        return cleanup(hip_fail(e, "decoder upload"));
    *out = m;
    return RCE_QMM_OK;
}

void rce_qmm_llama_destroy(rce_qmm_llama *m) {
    if (!m) return;
    (void)hipSetDevice(m->ctx->device);
    (void)hipStreamSynchronize(m->ctx->stream);
    drop_graph(m);
    if (m->mem) (void)hipFree(m->mem);
    if (m->h_token) (void)hipHostFree(m->h_token);
    if (m->h_status) (void)hipHostFree(m->h_status);
    if (m->h_logits) (void)hipHostFree(m->h_logits);
    if (m->last_dev) (void)hipEventDestroy(m->last_dev);
    rce_qmm_context *ctx = m->ctx;
    delete m;
    context_release(ctx);
}

rce_qmm_status rce_qmm_llama_reset(rce_qmm_llama *m) {
    if (!m) return fail(RCE_QMM_NULL_ARGUMENT, "null decoder");
    rce_qmm_status st = set_device(m->ctx->device);
    if (st) return st;
    hipStream_t s = m->ctx->stream;
    if (m->last_dev_pending) {
        HIP_TRY(hipEventSynchronize(m->last_dev));
        m->last_dev_pending = false;
    }
    HIP_TRY(poison_caches(m, s));
    HIP_TRY(hipMemsetAsync(m->pos_dev, 0, 256, s));  // pos, token, status words
    HIP_TRY(hipStreamSynchronize(s));
    m->pos = 0;
    return RCE_QMM_OK;
}

rce_qmm_status rce_qmm_llama_pos(const rce_qmm_llama *m, size_t *pos) {
    if (!m || !pos) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    *pos = m->pos;
    return RCE_QMM_OK;
}

rce_qmm_status rce_qmm_llama_forward_token(rce_qmm_llama *m, int32_t token_id, float *logits) {
    if (!m || !logits) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    if (token_id < 0 || (size_t)token_id >= m->embd.n_rows)
        return fail(RCE_QMM_BAD_SHAPE, "token id " + std::to_string(token_id) + " out of range of token_embd (" +
                                           std::to_string(m->embd.n_rows) + " rows)");
    rce_qmm_status st = set_device(m->ctx->device);
    if (st) return st;
    hipStream_t s = m->ctx->stream;
    if (m->pos >= m->cfg.context_length) return fail(RCE_QMM_BAD_SHAPE, "the KV cache is full");
    *m->h_token = token_id;
    HIP_TRY(hipMemcpyAsync(m->token, m->h_token, sizeof(int32_t), hipMemcpyHostToDevice, s));
    HIP_TRY(launch_embed_row(m->embd, m->token, m->x, m->status, s));
    if ((st = run_step(m, m->logits, s))) return st;
    return finish_host(m, logits, s);
}

rce_qmm_status rce_qmm_llama_forward_embedding(rce_qmm_llama *m, const float *embedding, float *logits) {
    if (!m || !embedding || !logits) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    rce_qmm_status st = set_device(m->ctx->device);
    if (st) return st;
    hipStream_t s = m->ctx->stream;
    if (m->pos >= m->cfg.context_length) return fail(RCE_QMM_BAD_SHAPE, "the KV cache is full");
    HIP_TRY(hipMemcpyAsync(m->x, embedding, m->cfg.d_model * sizeof(float), hipMemcpyHostToDevice, s));
    HIP_TRY(hipMemsetAsync(m->status + 2, 0, sizeof(int), s));  // not a skipped step (outside the graph)
    if ((st = run_step(m, m->logits, s))) return st;
    return finish_host(m, logits, s);
}

rce_qmm_status rce_qmm_llama_forward_token_dev(rce_qmm_llama *m, const int32_t *token_dev, float *logits_dev,
                                               void *stream) {
    if (!m || !token_dev || !logits_dev) return fail(RCE_QMM_NULL_ARGUMENT, "null argument");
    rce_qmm_status st = set_device(m->ctx->device);
    if (st) return st;
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : m->ctx->stream;
    if (m->pos >= m->cfg.context_length) return fail(RCE_QMM_BAD_SHAPE, "the KV cache is full");
    HIP_TRY(launch_embed_row(m->embd, token_dev, m->x, m->status, s));
    if ((st = run_step(m, logits_dev, s))) return st;
    HIP_TRY(hipEventRecord(m->last_dev, s));  // rce_qmm_llama_check waits for it
    m->last_dev_pending = true;
    return RCE_QMM_OK;
}

rce_qmm_status rce_qmm_llama_check(rce_qmm_llama *m) {
    if (!m) return fail(RCE_QMM_NULL_ARGUMENT, "null decoder");
    rce_qmm_status st = set_device(m->ctx->device);
    if (st) return st;
    return take_status(m, m->ctx->stream);
}

}  // extern "C"
