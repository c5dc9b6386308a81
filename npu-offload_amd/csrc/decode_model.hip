// decode_model.hip — one greedy decode step of a whole MoE decoder on the GPU (include/moe_gpu.h, moe_model_*).
//
// Replaces the reference engine's host step (track2_opt/solar_engine/src/main.rs:372-387 `step`, with `layer`
// :106-126 and `moe_host` :128-141 per layer): the embedding row of the token, then per layer
//   h  = rmsnorm(x, input_layernorm)                       folded into the q|k|v GEMV (moe_qkv_rope_append_dev)
//   q, k, v = round_bf(gemv(q|k|v_proj, h))                one [QD + 2 KVD, H] table, one launch, whose epilogue
//   rope(q), rope(k), kc[pos] = k, vc[pos] = v             ropes q and k and appends k and v to the caches
//   a  = attention(q, kc[0..pos], vc[0..pos])              moe_attn_decode_oproj_dev (one launch for both when
//   o  = round_bf(gemv(o_proj, a))                         QD = 4096; else moe_attn_decode_dev + moe_gemv_dev)
//   x  = bf16(x + o); h2 = rmsnorm(x, post_attention_layernorm); x = bf16(x + bf16(bf16(moe) + bf16(shared)))
//                                                          one fused MoE launch (moe_gpu_block_dev)
// and after the last layer the final RMSNorm, the LM-head GEMV and the greedy argmax (moe_head_argmax_dev).  Every
// launch goes to the model's stream in order; a step allocates nothing and needs no host synchronisation (the token
// comes from and goes to device memory), so steps chain back to back.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdio.h>

#include <string>
#include <vector>

#include "moe_gpu.h"

namespace {

__global__ void embed_kernel(const uint16_t* __restrict__ emb, const int32_t* __restrict__ token, int V, int H,
                             uint16_t* __restrict__ x, int* __restrict__ bad) {
    const int t = *token;
    if (t < 0 || t >= V) {  // an id outside the vocabulary: flagged, the row is left as it was
        if (threadIdx.x == 0 && blockIdx.x == 0) *bad = 1;
        return;
    }
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < H / 8; i += gridDim.x * blockDim.x)
        reinterpret_cast<uint4*>(x)[i] = reinterpret_cast<const uint4*>(emb + (size_t)t * H)[i];
}

std::string g_model_create_err = "no error";

}  // namespace

struct moe_model {
    int device = 0;
    moe_model_config c{};
    int QD = 0, KVD = 0;
    hipStream_t own_stream = nullptr, stream = nullptr;
    moe_gpu* experts = nullptr;
    moe_head* head = nullptr;
    std::vector<uint16_t*> qkv_w, o_w, in_norm, post_norm;  // per layer
    std::vector<uint16_t*> kc, vc;                          // per layer [max_ctx, NKV, D]
    std::vector<unsigned char> loaded;
    uint16_t* emb = nullptr;   // [V, H]
    uint16_t* cos = nullptr;   // [max_ctx, D]
    uint16_t* sin = nullptr;
    uint16_t* x = nullptr;     // residual stream, two buffers
    uint16_t* x2 = nullptr;
    uint16_t* qkv = nullptr;   // [QD + 2 KVD]
    uint16_t* attn = nullptr;  // [QD]
    uint16_t* o = nullptr;     // [H]
    void* attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    int32_t* d_tok = nullptr;  // [2]: host-path token in, next token out
    float* d_best = nullptr;
    int* d_bad = nullptr;
    int32_t* h_tok = nullptr;  // pinned host staging of the host path
    bool has_emb = false, has_rope = false;
    int active_layers = 0;     // layers a step runs (the first ones), then the head
    uint16_t* last_x = nullptr;  // residual after the last layer of the last step
    std::string err = "no error";
};

namespace {

int mfail(moe_model* m, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (m) m->err = buf; else g_model_create_err = buf;
    return code;
}

#define MCHK(m, expr)                                                                                          \
    do {                                                                                                       \
        hipError_t e_ = (expr);                                                                                \
        if (e_ != hipSuccess)                                                                                  \
            return mfail((m), e_ == hipErrorNoBinaryForGpu ? MOE_GPU_ENOKERNEL : MOE_GPU_EHIP, "%s: %s (%s:%d)", \
                         #expr, hipGetErrorString(e_), __FILE__, __LINE__);                                    \
    } while (0)

// a sub-call's failure, with the sub-context's message
#define SUB(m, expr, what)                                                                                     \
    do {                                                                                                       \
        int rc_ = (expr);                                                                                      \
        if (rc_ != MOE_GPU_OK) return mfail((m), rc_, "%s: %s", (what), sub_msg(m));                           \
    } while (0)

const char* sub_msg(moe_model* m) {
    static thread_local std::string s;
    s = std::string("experts: ") + moe_gpu_last_error(m->experts) + "; head: " + moe_head_last_error(m->head) +
        "; attention: " + moe_attn_last_error();
    return s.c_str();
}

int alloc(moe_model* m, void** p, size_t bytes, const char* what) {
    if (hipMalloc(p, bytes) != hipSuccess) {
        *p = nullptr;
        (void)hipGetLastError();
        return mfail(m, MOE_GPU_ENOMEM, "hipMalloc(%zu) for %s failed", bytes, what);
    }
    return MOE_GPU_OK;
}

int enter(moe_model* m) {
    if (!m) return MOE_GPU_EINVAL;
    MCHK(m, hipSetDevice(m->device));
    return MOE_GPU_OK;
}

int put(moe_model* m, void* dst, const void* src, size_t bytes) {  // host or device source
    MCHK(m, hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, m->stream));
    return MOE_GPU_OK;
}

// The step's kernels on the model's stream; token / next / best are device pointers.
int run_step(moe_model* m, const int32_t* token, int pos, int32_t* next, float* best) {
    const moe_model_config& c = m->c;
    if (pos < 0 || pos >= c.max_ctx) return mfail(m, MOE_GPU_EINVAL, "pos %d outside [0, max_ctx=%d)", pos, c.max_ctx);
    if (!m->has_emb || !m->has_rope) return mfail(m, MOE_GPU_ESTATE, "embedding or rope tables not loaded");
    for (int l = 0; l < c.n_layers; l++)
        if (!m->loaded[l]) return mfail(m, MOE_GPU_ESTATE, "layer %d: attention weights not loaded", l);
    hipLaunchKernelGGL(embed_kernel, dim3(2), dim3(256), 0, m->stream, m->emb, token, c.vocab, c.H, m->x, m->d_bad);
    MCHK(m, hipGetLastError());
    const uint16_t* cs = m->cos + (size_t)pos * c.head_dim;
    const uint16_t* sn = m->sin + (size_t)pos * c.head_dim;
    const float scale = 1.0f / sqrtf((float)c.head_dim);
    uint16_t *x = m->x, *xn = m->x2;
    for (int l = 0; l < m->active_layers; l++) {
        SUB(m, moe_qkv_rope_append_dev(c.H, c.n_q_heads, c.n_kv_heads, c.head_dim, m->qkv_w[l], x, m->in_norm[l], c.eps,
                                       cs, sn, m->qkv, m->kc[l], m->vc[l], pos, m->stream),
            "q|k|v projection, rope, kv append");
        if (m->QD == 4096) {  // attention and the o projection in one launch (its weights stream during the exchanges)
            SUB(m, moe_attn_decode_oproj_dev(c.n_q_heads, c.n_kv_heads, c.head_dim, pos + 1, scale, m->qkv, m->kc[l],
                                             m->vc[l], m->attn, m->o_w[l], c.H, m->o, m->attn_ws, m->attn_ws_bytes,
                                             m->stream),
                "attention + o projection");
        } else {
            SUB(m, moe_attn_decode_dev(c.n_q_heads, c.n_kv_heads, c.head_dim, pos + 1, scale, m->qkv, m->kc[l],
                                       m->vc[l], m->attn, m->attn_ws, m->attn_ws_bytes, m->stream),
                "attention");
            SUB(m, moe_gemv_dev(c.H, m->QD, m->o_w[l], m->attn, m->o, m->stream), "o projection");
        }
        SUB(m, moe_gpu_block_dev(m->experts, l, 1, x, m->o, m->post_norm[l], c.eps, 0, 0, xn, nullptr, nullptr,
                                 nullptr),
            "moe block");
        uint16_t* t = x;
        x = xn;
        xn = t;
    }
    m->last_x = x;
    SUB(m, moe_head_argmax_dev(m->head, 1, x, c.argmax_rule, next, best, nullptr), "lm head");
    return MOE_GPU_OK;
}

}  // namespace

extern "C" {

int moe_model_create(int device, const moe_model_config* cfg, moe_model** out) {
    if (!out || !cfg) return mfail(nullptr, MOE_GPU_EINVAL, "NULL cfg/out");
    *out = nullptr;
    const moe_model_config& c = *cfg;
    if (c.n_layers < 1 || c.vocab < 1 || c.max_ctx < 1 || c.n_q_heads < 1 || c.n_kv_heads < 1 || c.head_dim != 128 ||
        c.n_q_heads % c.n_kv_heads != 0 || !(c.eps >= 0.f))
        return mfail(nullptr, MOE_GPU_EINVAL, "bad model config (head_dim must be 128, n_q_heads a multiple of n_kv_heads)");
    if ((c.n_q_heads * c.head_dim) % 1024 != 0 || c.H % 4096 != 0)
        return mfail(nullptr, MOE_GPU_EINVAL, "H must be a multiple of 4096 and n_q_heads * head_dim of 1024");
    if (c.route_rule != MOE_GPU_ROUTE_SOFTMAX && c.route_rule != MOE_GPU_ROUTE_SIGMOID)
        return mfail(nullptr, MOE_GPU_EINVAL, "route_rule must be MOE_GPU_ROUTE_SOFTMAX or _SIGMOID");
    if (c.argmax_rule != MOE_HEAD_ARGMAX_FP32 && c.argmax_rule != MOE_HEAD_ARGMAX_BF16)
        return mfail(nullptr, MOE_GPU_EINVAL, "argmax_rule must be MOE_HEAD_ARGMAX_FP32 or _BF16");
    if (hipSetDevice(device) != hipSuccess) return mfail(nullptr, MOE_GPU_EHIP, "hipSetDevice(%d) failed", device);
    moe_model* m = new moe_model();
    m->device = device;
    m->c = c;
    m->QD = c.n_q_heads * c.head_dim;
    m->active_layers = c.n_layers;
    m->KVD = c.n_kv_heads * c.head_dim;
    auto bail = [&](int code) {
        g_model_create_err = m->err;
        moe_model_destroy(m);
        return code;
    };
    if (hipStreamCreateWithFlags(&m->own_stream, hipStreamNonBlocking) != hipSuccess)
        return bail(mfail(m, MOE_GPU_EHIP, "hipStreamCreate failed"));
    m->stream = m->own_stream;
    int rc = moe_gpu_create(device, c.H, c.F, c.E, c.topk, c.n_shared, c.n_layers, 1, &m->experts);
    if (rc) return bail(mfail(m, rc, "experts: %s", moe_gpu_last_error(nullptr)));
    if ((rc = moe_gpu_set_option(m->experts, MOE_GPU_OPT_ROUTE_RULE, c.route_rule)))
        return bail(mfail(m, rc, "experts: %s", moe_gpu_last_error(m->experts)));
    if ((rc = moe_gpu_set_stream(m->experts, m->stream))) return bail(mfail(m, rc, "experts stream"));
    rc = moe_head_create(device, c.H, c.vocab, c.eps, &m->head);
    if (rc) return bail(mfail(m, rc, "head: %s", moe_head_last_error(nullptr)));
    if ((rc = moe_head_set_stream(m->head, m->stream))) return bail(mfail(m, rc, "head stream"));
    const int L = c.n_layers;
    m->qkv_w.assign(L, nullptr); m->o_w.assign(L, nullptr); m->in_norm.assign(L, nullptr);
    m->post_norm.assign(L, nullptr); m->kc.assign(L, nullptr); m->vc.assign(L, nullptr); m->loaded.assign(L, 0);
    const size_t kvb = (size_t)c.max_ctx * m->KVD * 2;
    for (int l = 0; l < L; l++) {
        if ((rc = alloc(m, (void**)&m->qkv_w[l], (size_t)(m->QD + 2 * m->KVD) * c.H * 2, "q|k|v weights")) ||
            (rc = alloc(m, (void**)&m->o_w[l], (size_t)c.H * m->QD * 2, "o weights")) ||
            (rc = alloc(m, (void**)&m->in_norm[l], (size_t)c.H * 2, "input norm")) ||
            (rc = alloc(m, (void**)&m->post_norm[l], (size_t)c.H * 2, "post norm")) ||
            (rc = alloc(m, (void**)&m->kc[l], kvb, "key cache")) || (rc = alloc(m, (void**)&m->vc[l], kvb, "value cache")))
            return bail(rc);
        if (hipMemsetAsync(m->kc[l], 0, kvb, m->stream) != hipSuccess ||
            hipMemsetAsync(m->vc[l], 0, kvb, m->stream) != hipSuccess)
            return bail(mfail(m, MOE_GPU_EHIP, "clearing the kv cache failed"));
    }
    if ((rc = alloc(m, (void**)&m->emb, (size_t)c.vocab * c.H * 2, "embedding")) ||
        (rc = alloc(m, (void**)&m->cos, (size_t)c.max_ctx * c.head_dim * 2, "rope cos")) ||
        (rc = alloc(m, (void**)&m->sin, (size_t)c.max_ctx * c.head_dim * 2, "rope sin")) ||
        (rc = alloc(m, (void**)&m->x, (size_t)c.H * 2, "residual")) ||
        (rc = alloc(m, (void**)&m->x2, (size_t)c.H * 2, "residual")) ||
        (rc = alloc(m, (void**)&m->qkv, (size_t)(m->QD + 2 * m->KVD) * 2, "q|k|v")) ||
        (rc = alloc(m, (void**)&m->attn, (size_t)m->QD * 2, "attention output")) ||
        (rc = alloc(m, (void**)&m->o, (size_t)c.H * 2, "o")) || (rc = alloc(m, (void**)&m->d_tok, 8, "token")) ||
        (rc = alloc(m, (void**)&m->d_best, 4, "best")) || (rc = alloc(m, (void**)&m->d_bad, 4, "flag")))
        return bail(rc);
    m->attn_ws_bytes = moe_attn_workspace_bytes(c.n_q_heads, c.head_dim, c.max_ctx);
    if ((rc = alloc(m, &m->attn_ws, m->attn_ws_bytes, "attention workspace"))) return bail(rc);
    if (hipMemset(m->attn_ws, 0, m->attn_ws_bytes) != hipSuccess)  // the attention workspace starts zero-filled
        return bail(mfail(m, MOE_GPU_EHIP, "hipMemset of the attention workspace failed"));
    if (hipHostMalloc((void**)&m->h_tok, 8, hipHostMallocDefault) != hipSuccess)
        return bail(mfail(m, MOE_GPU_ENOMEM, "hipHostMalloc failed"));
    if (hipMemsetAsync(m->d_bad, 0, 4, m->stream) != hipSuccess || hipStreamSynchronize(m->stream) != hipSuccess)
        return bail(mfail(m, MOE_GPU_EHIP, "initialisation failed"));
    *out = m;
    return MOE_GPU_OK;
}

void moe_model_destroy(moe_model* m) {
    if (!m) return;
    (void)hipSetDevice(m->device);
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    if (m->experts) moe_gpu_destroy(m->experts);
    if (m->head) moe_head_destroy(m->head);
    for (auto* v : {&m->qkv_w, &m->o_w, &m->in_norm, &m->post_norm, &m->kc, &m->vc})
        for (uint16_t* p : *v)
            if (p) (void)hipFree(p);
    void* ps[] = {m->emb, m->cos, m->sin, m->x, m->x2, m->qkv, m->attn, m->o, m->attn_ws, m->d_tok, m->d_best, m->d_bad};
    for (void* p : ps)
        if (p) (void)hipFree(p);
    if (m->h_tok) (void)hipHostFree(m->h_tok);
    if (m->own_stream) (void)hipStreamDestroy(m->own_stream);
    delete m;
}

const char* moe_model_last_error(const moe_model* m) { return m ? m->err.c_str() : g_model_create_err.c_str(); }

moe_gpu* moe_model_experts(moe_model* m) { return m ? m->experts : nullptr; }
moe_head* moe_model_head(moe_model* m) { return m ? m->head : nullptr; }

int moe_model_set_stream(moe_model* m, void* stream) {
    int rc = enter(m);
    if (rc) return rc;
    m->stream = stream ? (hipStream_t)stream : m->own_stream;
    SUB(m, moe_gpu_set_stream(m->experts, m->stream), "experts stream");
    SUB(m, moe_head_set_stream(m->head, m->stream), "head stream");
    return MOE_GPU_OK;
}

int moe_model_synchronize(moe_model* m) {
    int rc = enter(m);
    if (rc) return rc;
    MCHK(m, hipStreamSynchronize(m->stream));
    int bad = 0;
    MCHK(m, hipMemcpy(&bad, m->d_bad, 4, hipMemcpyDeviceToHost));
    if (bad) {
        MCHK(m, hipMemset(m->d_bad, 0, 4));
        return mfail(m, MOE_GPU_EINVAL, "a step's token id was outside [0, vocab)");
    }
    SUB(m, moe_gpu_synchronize(m->experts), "experts");
    return MOE_GPU_OK;
}

int moe_model_load_layer(moe_model* m, int layer, const uint16_t* in_norm, const uint16_t* wq, const uint16_t* wk,
                         const uint16_t* wv, const uint16_t* wo, const uint16_t* post_norm) {
    int rc = enter(m);
    if (rc) return rc;
    if (layer < 0 || layer >= m->c.n_layers) return mfail(m, MOE_GPU_EINVAL, "layer %d outside [0, %d)", layer, m->c.n_layers);
    if (!in_norm || !wq || !wk || !wv || !wo || !post_norm) return mfail(m, MOE_GPU_EINVAL, "NULL weight pointer");
    const size_t H = m->c.H;
    if ((rc = put(m, m->qkv_w[layer], wq, (size_t)m->QD * H * 2)) ||
        (rc = put(m, m->qkv_w[layer] + (size_t)m->QD * H, wk, (size_t)m->KVD * H * 2)) ||
        (rc = put(m, m->qkv_w[layer] + (size_t)(m->QD + m->KVD) * H, wv, (size_t)m->KVD * H * 2)) ||
        (rc = put(m, m->o_w[layer], wo, H * m->QD * 2)) || (rc = put(m, m->in_norm[layer], in_norm, H * 2)) ||
        (rc = put(m, m->post_norm[layer], post_norm, H * 2)))
        return rc;
    MCHK(m, hipStreamSynchronize(m->stream));  // a host source may be reused by the caller after the call
    m->loaded[layer] = 1;
    return MOE_GPU_OK;
}

int moe_model_get_config(moe_model* m, moe_model_config* cfg) {
    int rc = enter(m);
    if (rc) return rc;
    if (!cfg) return mfail(m, MOE_GPU_EINVAL, "NULL config");
    *cfg = m->c;
    return MOE_GPU_OK;
}

int moe_model_load_embedding(moe_model* m, const uint16_t* emb) {
    int rc = enter(m);
    if (rc) return rc;
    if (!emb) return mfail(m, MOE_GPU_EINVAL, "NULL embedding");
    if ((rc = put(m, m->emb, emb, (size_t)m->c.vocab * m->c.H * 2))) return rc;
    MCHK(m, hipStreamSynchronize(m->stream));
    m->has_emb = true;
    return MOE_GPU_OK;
}

int moe_model_load_rope(moe_model* m, const uint16_t* cos_tab, const uint16_t* sin_tab) {
    int rc = enter(m);
    if (rc) return rc;
    if (!cos_tab || !sin_tab) return mfail(m, MOE_GPU_EINVAL, "NULL rope table");
    const size_t n = (size_t)m->c.max_ctx * m->c.head_dim * 2;
    if ((rc = put(m, m->cos, cos_tab, n)) || (rc = put(m, m->sin, sin_tab, n))) return rc;
    MCHK(m, hipStreamSynchronize(m->stream));
    m->has_rope = true;
    return MOE_GPU_OK;
}

int moe_model_set_layers(moe_model* m, int n) {
    int rc = enter(m);
    if (rc) return rc;
    if (n < 1 || n > m->c.n_layers) return mfail(m, MOE_GPU_EINVAL, "layers %d outside [1, %d]", n, m->c.n_layers);
    m->active_layers = n;
    return MOE_GPU_OK;
}

int moe_model_kv_cache(moe_model* m, int layer, uint16_t** k_cache, uint16_t** v_cache) {
    int rc = enter(m);
    if (rc) return rc;
    if (layer < 0 || layer >= m->c.n_layers || !k_cache || !v_cache) return mfail(m, MOE_GPU_EINVAL, "bad layer / NULL");
    *k_cache = m->kc[layer];
    *v_cache = m->vc[layer];
    return MOE_GPU_OK;
}

int moe_model_step_dev(moe_model* m, const int32_t* token, int pos, int32_t* next, float* best) {
    int rc = enter(m);
    if (rc) return rc;
    if (!token || !next) return mfail(m, MOE_GPU_EINVAL, "NULL token/next");
    return run_step(m, token, pos, next, best ? best : m->d_best);
}

int moe_model_step(moe_model* m, int token, int pos, int32_t* next, float* best) {
    int rc = enter(m);
    if (rc) return rc;
    if (!next) return mfail(m, MOE_GPU_EINVAL, "NULL next");
    if (token < 0 || token >= m->c.vocab) return mfail(m, MOE_GPU_EINVAL, "token %d outside [0, %d)", token, m->c.vocab);
    m->h_tok[0] = token;
    MCHK(m, hipMemcpyAsync(m->d_tok, m->h_tok, 4, hipMemcpyHostToDevice, m->stream));
    if ((rc = run_step(m, m->d_tok, pos, m->d_tok + 1, m->d_best))) return rc;
    MCHK(m, hipMemcpyAsync(m->h_tok + 1, m->d_tok + 1, 4, hipMemcpyDeviceToHost, m->stream));
    float b = 0.f;
    MCHK(m, hipMemcpyAsync(&b, m->d_best, 4, hipMemcpyDeviceToHost, m->stream));
    if ((rc = moe_model_synchronize(m))) return rc;
    *next = m->h_tok[1];
    if (best) *best = b;
    return MOE_GPU_OK;
}

int moe_model_residual(moe_model* m, uint16_t* x) {
    int rc = enter(m);
    if (rc) return rc;
    if (!x) return mfail(m, MOE_GPU_EINVAL, "NULL x");
    if (!m->last_x) return mfail(m, MOE_GPU_ESTATE, "no step has run");
    MCHK(m, hipMemcpyAsync(x, m->last_x, (size_t)m->c.H * 2, hipMemcpyDefault, m->stream));
    MCHK(m, hipStreamSynchronize(m->stream));
    return MOE_GPU_OK;
}

}  // extern "C"
