// moe_gpu_api.hip — the extern "C" boundary (include/moe_gpu.h): context, HBM expert tables, weight loads and the
// orchestration of the routed-MoE kernels on one HIP stream.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "moe_gpu.h"
#include "moe_kernels.h"

using moe::Dims;
using moe::ExpertArgs;
using moe::FusedArgs;
using moe::LayerPtrs;
using moe::Slots;
using moe::Sync;

namespace {

struct Layer {
    uint16_t* wr = nullptr;
    float* bias = nullptr;
    uint16_t* gu = nullptr;   // E tiled gate|up tables
    uint16_t* dn = nullptr;   // E tiled down tables
    uint16_t* sgu = nullptr;  // n_shared tiled gate|up tables
    uint16_t* sdn = nullptr;
    int8_t* gu_q8 = nullptr;
    int8_t* dn_q8 = nullptr;
    float* sc_q8 = nullptr;
    std::vector<unsigned char> loaded, loaded_q8, shared_loaded;
    bool router = false;
    int n_loaded = 0, n_loaded_q8 = 0, n_shared_loaded = 0;
};

std::string g_create_err = "no error";

}  // namespace

struct moe_gpu {
    int device = 0;
    Dims d{};
    int n_layers = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    std::string err = "no error";
    std::vector<Layer> layers;
    uint16_t* d_x = nullptr;
    float* d_out = nullptr;
    float* d_logits = nullptr;      // plain router logits (route() readback)
    uint64_t* d_logits_tag = nullptr;  // tagged router logits read by the routing units
    int32_t* d_ids = nullptr;
    float* d_gates = nullptr;
    Slots* d_slots = nullptr;
    Sync* d_sync = nullptr;
    uint64_t* d_act = nullptr;      // tagged SiLU(g)*u pairs
    uint64_t* d_ypart = nullptr;    // tagged down outputs
    uint16_t* d_stage = nullptr;  // max(3F, E) * H bf16 staging for host loads (an expert, or the router table)
    int8_t* d_stage_q8 = nullptr;
    float* d_stage_sc = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    bool timing = false;
    bool timed = false;
    uint64_t* d_trace = nullptr;  // fused-kernel unit trace (allocated when tracing is switched on)
    int trace_units = 0;
    bool fused = true;     // one persistent kernel per layer call (MOE_GPU_OPT_FUSED)
    int wg_per_cu = 1;     // fused grid: workgroups per CU, 0 = as many as fit (MOE_GPU_OPT_WG_PER_CU)
    int last_grid = 0;
    int ksplit = 0;        // K parts per routed gate|up tile, 0 = automatic (MOE_GPU_OPT_KSPLIT)
    int ksplit_shared = 0; // K parts per shared gate|up tile, 0 = automatic (MOE_GPU_OPT_KSPLIT_SHARED)
    int lag = 0;           // fused queue lag of down blocks, 0 = automatic (MOE_GPU_OPT_LAG)
    int shared_waits = 0;  // MOE_GPU_OPT_SHARED_WAITS
    int grid_req = 0;      // fused grid override, 0 = automatic (MOE_GPU_OPT_GRID)
    int router_poll = 1024;  // MOE_GPU_OPT_ROUTER_POLL
    int route_rule = moe::kRouteSoftmax;  // MOE_GPU_OPT_ROUTE_RULE
    uint64_t* d_gpart = nullptr;    // tagged split gate|up partial sums
    unsigned epoch = 0;             // tag of the last call (tags are never 0)
    unsigned fused_launches = 0;    // selects the fused kernel's work-queue head
    size_t act_bytes = 0, ypart_bytes = 0, gpart_bytes = 0, logits_tag_bytes = 0;
    // per-kernel profiling: event pairs recorded around each launch, resolved on read
    bool profiling = false;
    std::vector<hipEvent_t> prof_pool;
    std::vector<int> prof_kid;  // kernel slot of each recorded pair
    size_t prof_used = 0;       // events in use (2 per launch)
    double prof_ms[8] = {0};
    int prof_n[8] = {0};
};

namespace {

int fail(moe_gpu* c, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (c) c->err = buf; else g_create_err = buf;
    return code;
}

#define HIPCHK(c, expr)                                                                                        \
    do {                                                                                                       \
        hipError_t e_ = (expr);                                                                                \
        if (e_ != hipSuccess) return fail((c), MOE_GPU_EHIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_), \
                                          __FILE__, __LINE__);                                                 \
    } while (0)

int dev_alloc(moe_gpu* c, void** p, size_t bytes, const char* what) {
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        *p = nullptr;
        (void)hipGetLastError();
        return fail(c, MOE_GPU_ENOMEM, "hipMalloc(%zu bytes) for %s failed: %s", bytes, what, hipGetErrorString(e));
    }
    return MOE_GPU_OK;
}

int enter(moe_gpu* c) {
    if (!c) return MOE_GPU_EINVAL;
    HIPCHK(c, hipSetDevice(c->device));
    return MOE_GPU_OK;
}

int check_layer(moe_gpu* c, int layer) {
    if (layer < 0 || layer >= c->n_layers) return fail(c, MOE_GPU_EINVAL, "layer %d outside [0, %d)", layer, c->n_layers);
    return MOE_GPU_OK;
}

// Per-layer tables are allocated (and zeroed) on first use, each kind on its own: a layer whose routed experts are
// only ever loaded as int8 holds no bf16 routed tables.
void ensure_meta(moe_gpu* c, Layer& L) {
    if (L.loaded.empty()) {
        L.loaded.assign(c->d.E, 0);
        L.loaded_q8.assign(c->d.E, 0);
        L.shared_loaded.assign(c->d.n_shared, 0);
    }
}

int ensure_router(moe_gpu* c, int layer) {
    Layer& L = c->layers[layer];
    ensure_meta(c, L);
    if (L.wr) return MOE_GPU_OK;
    const Dims& d = c->d;
    int rc;
    if ((rc = dev_alloc(c, (void**)&L.wr, (size_t)d.E * d.H * 2, "router weight"))) return rc;
    if ((rc = dev_alloc(c, (void**)&L.bias, (size_t)d.E * 4, "router bias"))) return rc;
    HIPCHK(c, hipMemsetAsync(L.wr, 0, (size_t)d.E * d.H * 2, c->stream));
    HIPCHK(c, hipMemsetAsync(L.bias, 0, (size_t)d.E * 4, c->stream));
    return MOE_GPU_OK;
}

int ensure_bf16(moe_gpu* c, int layer) {
    Layer& L = c->layers[layer];
    ensure_meta(c, L);
    if (L.gu) return MOE_GPU_OK;
    const Dims& d = c->d;
    const size_t gub = d.gu_stride() * 2, dnb = d.dn_stride() * 2;
    int rc;
    if ((rc = dev_alloc(c, (void**)&L.gu, (size_t)d.E * gub, "gate|up tables"))) return rc;
    if ((rc = dev_alloc(c, (void**)&L.dn, (size_t)d.E * dnb, "down tables"))) return rc;
    HIPCHK(c, hipMemsetAsync(L.gu, 0, (size_t)d.E * gub, c->stream));
    HIPCHK(c, hipMemsetAsync(L.dn, 0, (size_t)d.E * dnb, c->stream));
    return MOE_GPU_OK;
}

int ensure_shared(moe_gpu* c, int layer) {
    Layer& L = c->layers[layer];
    ensure_meta(c, L);
    if (L.sgu || c->d.n_shared == 0) return MOE_GPU_OK;
    const Dims& d = c->d;
    const size_t gub = d.gu_stride() * 2, dnb = d.dn_stride() * 2;
    int rc;
    if ((rc = dev_alloc(c, (void**)&L.sgu, (size_t)d.n_shared * gub, "shared gate|up"))) return rc;
    if ((rc = dev_alloc(c, (void**)&L.sdn, (size_t)d.n_shared * dnb, "shared down"))) return rc;
    HIPCHK(c, hipMemsetAsync(L.sgu, 0, (size_t)d.n_shared * gub, c->stream));
    HIPCHK(c, hipMemsetAsync(L.sdn, 0, (size_t)d.n_shared * dnb, c->stream));
    return MOE_GPU_OK;
}

int ensure_q8(moe_gpu* c, int layer) {
    Layer& L = c->layers[layer];
    ensure_meta(c, L);
    if (L.gu_q8) return MOE_GPU_OK;
    const Dims& d = c->d;
    int rc;
    if ((rc = dev_alloc(c, (void**)&L.gu_q8, (size_t)d.E * d.gu_stride(), "int8 gate|up tables"))) return rc;
    if ((rc = dev_alloc(c, (void**)&L.dn_q8, (size_t)d.E * d.dn_stride(), "int8 down tables"))) return rc;
    if ((rc = dev_alloc(c, (void**)&L.sc_q8, (size_t)d.E * (2 * d.F + d.H) * 4, "int8 scales"))) return rc;
    HIPCHK(c, hipMemsetAsync(L.gu_q8, 0, (size_t)d.E * d.gu_stride(), c->stream));
    HIPCHK(c, hipMemsetAsync(L.dn_q8, 0, (size_t)d.E * d.dn_stride(), c->stream));
    HIPCHK(c, hipMemsetAsync(L.sc_q8, 0, (size_t)d.E * (2 * d.F + d.H) * 4, c->stream));
    return MOE_GPU_OK;
}

LayerPtrs ptrs(const moe_gpu* c, int layer) {
    const Layer& L = c->layers[layer];
    LayerPtrs p;
    p.wr = L.wr; p.bias = L.bias; p.gu = L.gu; p.dn = L.dn; p.sgu = L.sgu; p.sdn = L.sdn;
    p.gu_q8 = L.gu_q8; p.dn_q8 = L.dn_q8; p.sc_q8 = L.sc_q8;
    return p;
}

int check_T(moe_gpu* c, int T) {
    if (T < 1 || T > c->d.max_t) return fail(c, MOE_GPU_EINVAL, "T=%d outside [1, max_tokens=%d]", T, c->d.max_t);
    return MOE_GPU_OK;
}

int norm_keep(moe_gpu* c, int keep) { return (keep <= 0 || keep > c->d.k) ? c->d.k : keep; }

// load one expert's bf16 g,u,d (device pointers) into table slots dst_gu / dst_dn
int relayout_expert(moe_gpu* c, const uint16_t* g, const uint16_t* u, const uint16_t* dd, uint16_t* dst_gu,
                    uint16_t* dst_dn) {
    HIPCHK(c, moe::launch_relayout_gu(g, u, c->d.H, c->d.F, dst_gu, c->stream));
    HIPCHK(c, moe::launch_relayout_dn(dd, c->d.H, c->d.F, dst_dn, c->stream));
    return MOE_GPU_OK;
}

int stage_host_expert(moe_gpu* c, const uint16_t* g, const uint16_t* u, const uint16_t* dd) {
    const size_t n = (size_t)c->d.F * c->d.H;
    HIPCHK(c, hipMemcpyAsync(c->d_stage, g, n * 2, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(c->d_stage + n, u, n * 2, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(c->d_stage + 2 * n, dd, n * 2, hipMemcpyHostToDevice, c->stream));
    return MOE_GPU_OK;
}

int sync_and_check(moe_gpu* c) {
    HIPCHK(c, hipStreamSynchronize(c->stream));
    int err = 0;
    unsigned serr = 0;
    HIPCHK(c, hipMemcpy(&err, &c->d_slots->err, sizeof(int), hipMemcpyDeviceToHost));
    HIPCHK(c, hipMemcpy(&serr, &c->d_sync->err, sizeof(unsigned), hipMemcpyDeviceToHost));
    if (serr) {  // a bounded wait of the fused kernel gave up: results of that call are invalid; start clean
        HIPCHK(c, hipMemset(c->d_sync, 0, sizeof(Sync)));
        return fail(c, MOE_GPU_EHIP, "fused kernel dependency wait timed out; counters reset");
    }
    if (err == 1) return fail(c, MOE_GPU_EINVAL, "expert id outside [-1, E) in ids");
    if (err == 2) return fail(c, MOE_GPU_EINVAL, "an expert id repeats within one token's ids");
    return MOE_GPU_OK;
}

int begin_timing(moe_gpu* c) {
    if (c->timing) HIPCHK(c, hipEventRecord(c->ev0, c->stream));
    return MOE_GPU_OK;
}
int end_timing(moe_gpu* c) {
    if (c->timing) {
        HIPCHK(c, hipEventRecord(c->ev1, c->stream));
        c->timed = true;
    }
    return MOE_GPU_OK;
}

enum { K_ROUTER = 0, K_TOPK = 1, K_GATEUP = 2, K_DOWN = 3, K_FUSED = 4, K_SLOTS = 5 };
const char* const kKernelNames[K_SLOTS] = {"router_kernel", "topk_group_kernel", "gateup_kernel", "down_kernel",
                                           "fused_layer_kernel"};

int prof_mark(moe_gpu* c, int kid) {  // called before and after each launch
    if (!c->profiling) return MOE_GPU_OK;
    if (c->prof_used == c->prof_pool.size()) {
        hipEvent_t e;
        HIPCHK(c, hipEventCreate(&e));
        c->prof_pool.push_back(e);
    }
    if (c->prof_used % 2 == 0) c->prof_kid.push_back(kid);
    HIPCHK(c, hipEventRecord(c->prof_pool[c->prof_used++], c->stream));
    return MOE_GPU_OK;
}

int prof_resolve(moe_gpu* c) {
    if (c->prof_used == 0) return MOE_GPU_OK;
    HIPCHK(c, hipEventSynchronize(c->prof_pool[c->prof_used - 1]));
    for (size_t i = 0; i + 1 < c->prof_used; i += 2) {
        float ms = 0.f;
        HIPCHK(c, hipEventElapsedTime(&ms, c->prof_pool[i], c->prof_pool[i + 1]));
        const int k = c->prof_kid[i / 2];
        c->prof_ms[k] += ms;
        c->prof_n[k] += 1;
    }
    c->prof_used = 0;
    c->prof_kid.clear();
    return MOE_GPU_OK;
}

#define LAUNCH(c, kid, expr)                   \
    do {                                       \
        int rc_ = prof_mark((c), (kid));       \
        if (rc_) return rc_;                   \
        HIPCHK((c), (expr));                   \
        if ((rc_ = prof_mark((c), (kid)))) return rc_; \
    } while (0)

// Zero every tagged buffer (tag 0 is never a call's epoch).
int clear_tags(moe_gpu* c) {  // a fill kernel, not hipMemsetAsync: safe inside a caller's graph capture
    HIPCHK(c, moe::launch_zero(c->d_logits_tag, c->logits_tag_bytes / 8, c->stream));
    HIPCHK(c, moe::launch_zero(c->d_act, c->act_bytes / 8, c->stream));
    HIPCHK(c, moe::launch_zero(c->d_ypart, c->ypart_bytes / 8, c->stream));
    HIPCHK(c, moe::launch_zero(c->d_gpart, c->gpart_bytes / 8, c->stream));
    return MOE_GPU_OK;
}

// A fresh tag for the next call.  After 2^32 - 1 calls the tags wrap: the buffers are cleared so that no word of an
// old call can carry the new tag.
int next_epoch(moe_gpu* c, unsigned* ep) {
    if (++c->epoch == 0) {
        int rc = clear_tags(c);
        if (rc) return rc;
        c->epoch = 1;
    }
    *ep = c->epoch;
    return MOE_GPU_OK;
}

// K parts per gate|up tile: the option, else (Solar, H = 4096, measured on the fused schedule, us per call):
//  - routed tiles: whole (kp 1) in bf16 calls at every batch: kp 2 -> 1 measured batch 1 59.6 -> 59.4, batch 2
//    92.6 -> 92.4, batch 4 147.4 -> 137.7, batch 8 268 -> 240; in int8 calls about 128 K weights per part (kp 2 at
//    H = 4096: 39.0 -> 37.0 at batch 1 against whole tiles).  The rule depends on the precision only, so a token's
//    result does not depend on the batch it is in (the K split sets the summation order);
//  - shared tiles (bf16 in every call): about 64 K weights per part in bf16 calls (kps 2 -> 4: 61.2 -> 60.2 at batch 1),
//    so that the routing-independent work spreads over more workgroups while the routing is computed; 128 K in int8
//    calls, whose routed work is smaller (kps 4 -> 2: 38.6 -> 37.3).
static int kparts_auto(int H, size_t per_part) {
    const size_t weights = (size_t)64 * H;
    int kp = 1;
    while (kp < moe::kMaxKp && weights / (kp * 2) >= per_part) kp *= 2;
    return kp;
}
static int kparts(const moe_gpu* c, bool int8) {
    if (c->ksplit > 0) return c->ksplit;
    return int8 ? kparts_auto(c->d.H, (size_t)128 << 10) : 1;
}
static int kparts_shared(const moe_gpu* c, bool int8) {
    if (c->ksplit_shared > 0) return c->ksplit_shared;
    return kparts_auto(c->d.H, (size_t)(int8 ? 128 : 64) << 10);
}

// The expert pipeline of one call.  do_topk: route on the device from the layer's router (ids/gates are outputs);
// otherwise ids/gates are the caller's routing.  Fused: one persistent kernel; unfused: one kernel per phase.
int run_layer(moe_gpu* c, int layer, int T, const moe::StageSrc& in, int32_t* ids, float* gates, bool do_topk,
              int keep, int n_shared, unsigned flags, float* out, uint16_t* x_next = nullptr) {
    int rc;
    // A call's epoch, queue head and cross-workgroup words are per launch: a captured launch replayed would read the
    // previous replay's words as its own, so these calls refuse capture.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    HIPCHK(c, hipStreamIsCapturing(c->stream, &cap));
    if (cap != hipStreamCaptureStatusNone)
        return fail(c, MOE_GPU_ESTATE, "layer / moe calls cannot be captured into a graph (per-launch epochs and queue)");
    ExpertArgs a;
    a.L = ptrs(c, layer);
    a.d = c->d;
    a.T = T; a.keep = keep; a.n_shared = n_shared;
    a.int8 = (flags & MOE_GPU_INT8) ? 1 : 0;
    a.accumulate = (flags & MOE_GPU_ACCUMULATE) ? 1 : 0;
    a.in = in; a.out = out; a.x_next = x_next; a.ids = ids; a.gates = gates;
    a.slots = c->d_slots; a.act = c->d_act; a.ypart = c->d_ypart;
    a.maxs = c->d.n_shared + T * keep;
    a.kp = kparts(c, a.int8 != 0);
    a.kps = kparts_shared(c, a.int8 != 0);
    a.gpart = c->d_gpart;
    if ((rc = next_epoch(c, &a.epoch))) return rc;
    a.err = &c->d_sync->err;
    // Up to 7 tokens: the fused kernel.  8 or more (the batch >= 8 grouped case): the unfused kernels, whose cores for
    // units of more than 4 tokens use MFMA (measured at Solar batch 8: 205 us against the fused kernel's 211 us, whose
    // registers have no room for the MFMA cores).
    if (c->fused && T < 8) {
        FusedArgs f;
        f.e = a;
        f.logits = c->d_logits_tag;
        f.sync = c->d_sync;
        f.nR = do_topk ? moe::router_units(c->d.E, T) : 0;
        f.do_topk = do_topk ? 1 : 0;
        f.rule = c->route_rule;
        f.router_poll = c->router_poll;
        f.trace = c->d_trace;
        f.lag = c->lag > 0 ? c->lag : 8;
        f.phase = (int)(c->fused_launches++ & 1u);
        f.shared_waits = c->shared_waits;
        c->trace_units = moe::fused_units(f.nR, a.maxs, c->d.n_shared, c->d.F, c->d.H, a.kp, a.kps);
        LAUNCH(c, K_FUSED, moe::launch_fused(f, c->wg_per_cu, c->grid_req, c->stream, &c->last_grid));
        return MOE_GPU_OK;
    }
    if (do_topk)
        LAUNCH(c, K_ROUTER, moe::launch_router(a.L, c->d, T, a.in, c->d_logits_tag, nullptr, a.epoch, c->stream));
    // slots 0 .. d.n_shared-1 are always the shared experts' (summed only when this call includes them)
    LAUNCH(c, K_TOPK, moe::launch_topk_group(a.L, c->d, T, keep, c->d.n_shared, do_topk, c->route_rule,
                                             c->d_logits_tag, a.epoch, a.err, ids, gates, c->d_slots, c->stream));
    LAUNCH(c, K_GATEUP, moe::launch_gateup(a, c->d_sync, c->stream));
    LAUNCH(c, K_DOWN, moe::launch_down(a, c->stream));
    return MOE_GPU_OK;
}

moe::StageSrc plain_src(const uint16_t* x) { return moe::StageSrc{x, nullptr, nullptr, nullptr, 0.f}; }

int need_router(moe_gpu* c, int layer) {
    const Layer& L = c->layers[layer];
    if (!L.router) return fail(c, MOE_GPU_ESTATE, "layer %d: router weights not loaded", layer);
    return MOE_GPU_OK;
}

// all_routed: the call may reach any routed expert (device-side ids), so every one must be loaded in the precision
// the call uses (a bf16 reload leaves an expert's int8 copy stale, and it then counts as not loaded)
int need_experts(moe_gpu* c, int layer, unsigned flags, int with_shared, bool all_routed) {
    const Layer& L = c->layers[layer];
    const bool q8 = (flags & MOE_GPU_INT8) != 0;
    if (q8 ? !L.gu_q8 : !L.gu)
        return fail(c, MOE_GPU_ESTATE, "layer %d: no %s routed experts loaded", layer, q8 ? "int8" : "bf16");
    const int n = q8 ? L.n_loaded_q8 : L.n_loaded;
    if (all_routed && n < c->d.E)
        return fail(c, MOE_GPU_ESTATE, "layer %d: %d of %d routed experts loaded%s", layer, n, c->d.E,
                    q8 ? " with a current int8 copy" : " in bf16");
    if (with_shared && L.n_shared_loaded < c->d.n_shared)
        return fail(c, MOE_GPU_ESTATE, "layer %d: %d of %d shared experts loaded", layer, L.n_shared_loaded,
                    c->d.n_shared);
    return MOE_GPU_OK;
}

}  // namespace

// ======================================================================================================== C ABI
extern "C" {

int moe_gpu_create(int device, int H, int F, int E, int topk, int n_shared, int n_layers, int max_tokens,
                   moe_gpu** out) {
    if (!out) return fail(nullptr, MOE_GPU_EINVAL, "out is NULL");
    *out = nullptr;
    if (H <= 0 || H % 512) return fail(nullptr, MOE_GPU_EINVAL, "H=%d must be a positive multiple of 512", H);
    if (F <= 0 || F % 256) return fail(nullptr, MOE_GPU_EINVAL, "F=%d must be a positive multiple of 256", F);
    if (E < 1 || E > moe::kMaxExperts) return fail(nullptr, MOE_GPU_EINVAL, "E=%d outside [1, %d]", E, moe::kMaxExperts);
    if (topk < 1 || topk > moe::kMaxTopk || topk > E)
        return fail(nullptr, MOE_GPU_EINVAL, "topk=%d outside [1, min(E, %d)]", topk, moe::kMaxTopk);
    if (n_shared < 0 || n_shared > moe::kMaxShared)
        return fail(nullptr, MOE_GPU_EINVAL, "n_shared=%d outside [0, %d]", n_shared, moe::kMaxShared);
    if (n_layers < 1) return fail(nullptr, MOE_GPU_EINVAL, "n_layers=%d < 1", n_layers);
    if (H > 64 * moe::kMaxHTiles) return fail(nullptr, MOE_GPU_EINVAL, "H=%d above %d", H, 64 * moe::kMaxHTiles);
    if (max_tokens * topk > moe::kMaxTokens * moe::kMaxTopk || (size_t)max_tokens * H * 2 > 96 * 1024)
        return fail(nullptr, MOE_GPU_EINVAL, "max_tokens=%d too large for H=%d (activations staged in 96 KB of LDS)",
                    max_tokens, H);
    if (max_tokens < 1 || max_tokens > moe::kMaxTokens)
        return fail(nullptr, MOE_GPU_EINVAL, "max_tokens=%d outside [1, %d]", max_tokens, moe::kMaxTokens);
    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess || ndev == 0)
        return fail(nullptr, MOE_GPU_EHIP, "no HIP device (%s)", e != hipSuccess ? hipGetErrorString(e) : "count 0");
    if (device < 0 || device >= ndev) return fail(nullptr, MOE_GPU_EINVAL, "device %d outside [0, %d)", device, ndev);
    e = hipSetDevice(device);
    if (e != hipSuccess) return fail(nullptr, MOE_GPU_EHIP, "hipSetDevice(%d): %s", device, hipGetErrorString(e));
    if (!moe::kernels_available()) {
        hipDeviceProp_t prop;
        (void)hipGetDeviceProperties(&prop, device);
        return fail(nullptr, MOE_GPU_ENOKERNEL, "libmoe_gpu has no code object for device %d (%s); built for gfx950",
                    device, prop.gcnArchName);
    }
    moe_gpu* c = new moe_gpu();
    c->device = device;
    c->d.H = H; c->d.F = F; c->d.E = E; c->d.k = topk; c->d.n_shared = n_shared; c->d.max_t = max_tokens;
    c->n_layers = n_layers;
    c->layers.resize(n_layers);
    int rc = MOE_GPU_OK;
    auto bail = [&](int code) {
        g_create_err = c->err;
        moe_gpu_destroy(c);
        return code;
    };
    if (hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking) != hipSuccess)
        return bail(fail(c, MOE_GPU_EHIP, "hipStreamCreate failed"));
    c->stream = c->own_stream;
    const int maxs = n_shared + max_tokens * topk;
    const size_t kq = (size_t)n_shared + topk;
    if ((rc = dev_alloc(c, (void**)&c->d_x, (size_t)max_tokens * H * 2, "x"))) return bail(rc);
    if ((rc = dev_alloc(c, (void**)&c->d_out, (size_t)max_tokens * H * 4, "out"))) return bail(rc);
    if ((rc = dev_alloc(c, (void**)&c->d_logits, (size_t)max_tokens * E * 4, "logits"))) return bail(rc);
    c->logits_tag_bytes = (size_t)max_tokens * E * 8;
    if ((rc = dev_alloc(c, (void**)&c->d_logits_tag, c->logits_tag_bytes, "tagged logits"))) return bail(rc);
    if ((rc = dev_alloc(c, (void**)&c->d_ids, (size_t)max_tokens * topk * 4, "ids"))) return bail(rc);
    if ((rc = dev_alloc(c, (void**)&c->d_gates, (size_t)max_tokens * topk * 4, "gates"))) return bail(rc);
    if ((rc = dev_alloc(c, (void**)&c->d_slots, sizeof(Slots), "slots"))) return bail(rc);
    if ((rc = dev_alloc(c, (void**)&c->d_sync, sizeof(Sync), "sync counters"))) return bail(rc);
    c->act_bytes = (size_t)maxs * max_tokens * (F / 2) * 8;
    c->ypart_bytes = (size_t)max_tokens * kq * H * 8;
    if ((rc = dev_alloc(c, (void**)&c->d_act, c->act_bytes, "act"))) return bail(rc);
    if ((rc = dev_alloc(c, (void**)&c->d_ypart, c->ypart_bytes, "ypart"))) return bail(rc);
    // split gate|up partials: at most max_tokens * (n_shared + topk) (slot, token) pairs, 4 parts per tile
    c->gpart_bytes = (size_t)max_tokens * kq * (F / 32) * moe::kMaxKp * 64 * 8;
    if ((rc = dev_alloc(c, (void**)&c->d_gpart, c->gpart_bytes, "gate|up partials"))) return bail(rc);
    if ((rc = dev_alloc(c, (void**)&c->d_stage, (size_t)std::max(3 * F, E) * H * 2, "staging"))) return bail(rc);
    if ((rc = dev_alloc(c, (void**)&c->d_stage_q8, (size_t)3 * F * H, "int8 staging"))) return bail(rc);
    if ((rc = dev_alloc(c, (void**)&c->d_stage_sc, (size_t)(2 * F + H) * 4, "scale staging"))) return bail(rc);
    if (hipMemset(c->d_slots, 0, sizeof(Slots)) != hipSuccess || hipMemset(c->d_sync, 0, sizeof(Sync)) != hipSuccess ||
        clear_tags(c) != MOE_GPU_OK || hipStreamSynchronize(c->stream) != hipSuccess)
        return bail(fail(c, MOE_GPU_EHIP, "hipMemset of the workspace failed"));
    if (const char* v = getenv("MOE_GPU_FUSED")) c->fused = atoi(v) != 0;
    if (const char* v = getenv("MOE_GPU_WG_PER_CU")) c->wg_per_cu = atoi(v);
    if (hipEventCreate(&c->ev0) != hipSuccess || hipEventCreate(&c->ev1) != hipSuccess)
        return bail(fail(c, MOE_GPU_EHIP, "hipEventCreate failed"));
    *out = c;
    return MOE_GPU_OK;
}

void moe_gpu_destroy(moe_gpu* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (Layer& L : c->layers) {
        void* ps[] = {L.wr, L.bias, L.gu, L.dn, L.sgu, L.sdn, L.gu_q8, L.dn_q8, L.sc_q8};
        for (void* p : ps)
            if (p) (void)hipFree(p);
    }
    void* ws[] = {c->d_x, c->d_out, c->d_logits, c->d_logits_tag, c->d_ids, c->d_gates, c->d_slots, c->d_sync,
                  c->d_act, c->d_ypart, c->d_gpart, c->d_stage, c->d_stage_q8, c->d_stage_sc};
    for (void* p : ws)
        if (p) (void)hipFree(p);
    for (hipEvent_t e : c->prof_pool) (void)hipEventDestroy(e);
    if (c->d_trace) (void)hipFree(c->d_trace);
    if (c->ev0) (void)hipEventDestroy(c->ev0);
    if (c->ev1) (void)hipEventDestroy(c->ev1);
    if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
    delete c;
}

const char* moe_gpu_last_error(const moe_gpu* c) { return c ? c->err.c_str() : g_create_err.c_str(); }

int moe_gpu_set_stream(moe_gpu* c, void* stream) {
    int rc = enter(c);
    if (rc) return rc;
    c->stream = stream ? (hipStream_t)stream : c->own_stream;
    return MOE_GPU_OK;
}

int moe_gpu_synchronize(moe_gpu* c) {
    int rc = enter(c);
    if (rc) return rc;
    return sync_and_check(c);
}

// ------------------------------------------------------------------------------------------------------ weights
static int load_expert_common(moe_gpu* c, int layer, int e, const uint16_t* g, const uint16_t* u, const uint16_t* d,
                              bool shared, bool host) {
    int rc = enter(c);
    if (rc) return rc;
    if ((rc = check_layer(c, layer))) return rc;
    const int lim = shared ? c->d.n_shared : c->d.E;
    if (e < 0 || e >= lim) return fail(c, MOE_GPU_EINVAL, "%s expert %d outside [0, %d)", shared ? "shared" : "routed", e, lim);
    if (!g || !u || !d) return fail(c, MOE_GPU_EINVAL, "NULL weight pointer");
    if ((rc = shared ? ensure_shared(c, layer) : ensure_bf16(c, layer))) return rc;
    Layer& L = c->layers[layer];
    const size_t n = (size_t)c->d.F * c->d.H;
    if (host) {
        if ((rc = stage_host_expert(c, g, u, d))) return rc;
        g = c->d_stage; u = c->d_stage + n; d = c->d_stage + 2 * n;
    }
    uint16_t* dgu = (shared ? L.sgu : L.gu) + (size_t)e * c->d.gu_stride();
    uint16_t* ddn = (shared ? L.sdn : L.dn) + (size_t)e * c->d.dn_stride();
    if ((rc = relayout_expert(c, g, u, d, dgu, ddn))) return rc;
    if (host) HIPCHK(c, hipStreamSynchronize(c->stream));  // staging buffer is reused by the next load
    if (shared) {
        if (!L.shared_loaded[e]) { L.shared_loaded[e] = 1; L.n_shared_loaded++; }
    } else {
        if (!L.loaded[e]) { L.loaded[e] = 1; L.n_loaded++; }
        if (L.loaded_q8[e]) { L.loaded_q8[e] = 0; L.n_loaded_q8--; }  // int8 copy is stale now
    }
    return MOE_GPU_OK;
}

int moe_gpu_load_expert(moe_gpu* c, int layer, int e, const uint16_t* g, const uint16_t* u, const uint16_t* d) {
    return load_expert_common(c, layer, e, g, u, d, false, true);
}
int moe_gpu_load_shared(moe_gpu* c, int layer, int s, const uint16_t* g, const uint16_t* u, const uint16_t* d) {
    return load_expert_common(c, layer, s, g, u, d, true, true);
}
int moe_gpu_load_expert_dev(moe_gpu* c, int layer, int e, const uint16_t* g, const uint16_t* u, const uint16_t* d) {
    return load_expert_common(c, layer, e, g, u, d, false, false);
}
int moe_gpu_load_shared_dev(moe_gpu* c, int layer, int s, const uint16_t* g, const uint16_t* u, const uint16_t* d) {
    return load_expert_common(c, layer, s, g, u, d, true, false);
}

int moe_gpu_load_router(moe_gpu* c, int layer, const uint16_t* wr, const float* bias) {
    int rc = enter(c);
    if (rc) return rc;
    if ((rc = check_layer(c, layer))) return rc;
    if (!wr) return fail(c, MOE_GPU_EINVAL, "NULL router weight");
    if ((rc = ensure_router(c, layer))) return rc;
    Layer& L = c->layers[layer];
    HIPCHK(c, hipMemcpyAsync(c->d_stage, wr, (size_t)c->d.E * c->d.H * 2, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, moe::launch_relayout_router(c->d_stage, c->d.E, c->d.H, L.wr, c->stream));
    if (bias) HIPCHK(c, hipMemcpyAsync(L.bias, bias, (size_t)c->d.E * 4, hipMemcpyHostToDevice, c->stream));
    else HIPCHK(c, hipMemsetAsync(L.bias, 0, (size_t)c->d.E * 4, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    L.router = true;
    return MOE_GPU_OK;
}

int moe_gpu_load_expert_q8(moe_gpu* c, int layer, int e, const int8_t* q, const float* sc) {
    int rc = enter(c);
    if (rc) return rc;
    if ((rc = check_layer(c, layer))) return rc;
    if (e < 0 || e >= c->d.E) return fail(c, MOE_GPU_EINVAL, "routed expert %d outside [0, %d)", e, c->d.E);
    if (!q || !sc) return fail(c, MOE_GPU_EINVAL, "NULL int8 pointer");
    if ((rc = ensure_q8(c, layer))) return rc;
    Layer& L = c->layers[layer];
    const Dims& d = c->d;
    HIPCHK(c, hipMemcpyAsync(c->d_stage_q8, q, (size_t)3 * d.F * d.H, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(c->d_stage_sc, sc, (size_t)(2 * d.F + d.H) * 4, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, moe::launch_relayout_q8(c->d_stage_q8, c->d_stage_sc, d.H, d.F, L.gu_q8 + (size_t)e * d.gu_stride(),
                                      L.dn_q8 + (size_t)e * d.dn_stride(), L.sc_q8 + (size_t)e * (2 * d.F + d.H),
                                      c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (!L.loaded_q8[e]) { L.loaded_q8[e] = 1; L.n_loaded_q8++; }
    return MOE_GPU_OK;
}

int moe_gpu_quantize_experts(moe_gpu* c, int layer, int e0, int e1) {
    int rc = enter(c);
    if (rc) return rc;
    if ((rc = check_layer(c, layer))) return rc;
    if (e0 < 0 || e1 > c->d.E || e0 >= e1) return fail(c, MOE_GPU_EINVAL, "expert range [%d, %d) invalid", e0, e1);
    Layer& L = c->layers[layer];
    if (!L.gu) return fail(c, MOE_GPU_ESTATE, "layer %d: no bf16 experts to quantise", layer);
    ensure_meta(c, L);
    for (int e = e0; e < e1; e++)
        if (!L.loaded[e]) return fail(c, MOE_GPU_ESTATE, "layer %d: expert %d has no bf16 weights", layer, e);
    if ((rc = ensure_q8(c, layer))) return rc;
    const Dims& d = c->d;
    HIPCHK(c, moe::launch_quantize(L.gu + (size_t)e0 * d.gu_stride(), L.dn + (size_t)e0 * d.dn_stride(), d.H, d.F,
                                   e1 - e0, d.gu_stride(), d.dn_stride(), L.gu_q8 + (size_t)e0 * d.gu_stride(),
                                   L.dn_q8 + (size_t)e0 * d.dn_stride(), L.sc_q8 + (size_t)e0 * (2 * d.F + d.H),
                                   c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    for (int e = e0; e < e1; e++)
        if (!L.loaded_q8[e]) { L.loaded_q8[e] = 1; L.n_loaded_q8++; }
    return MOE_GPU_OK;
}

int moe_gpu_get_expert_q8(moe_gpu* c, int layer, int e, int8_t* q, float* sc) {
    int rc = enter(c);
    if (rc) return rc;
    if ((rc = check_layer(c, layer))) return rc;
    if (e < 0 || e >= c->d.E) return fail(c, MOE_GPU_EINVAL, "routed expert %d outside [0, %d)", e, c->d.E);
    Layer& L = c->layers[layer];
    if (!L.gu_q8 || L.loaded_q8.empty() || !L.loaded_q8[e])
        return fail(c, MOE_GPU_ESTATE, "layer %d expert %d: no int8 copy", layer, e);
    const Dims& d = c->d;
    HIPCHK(c, moe::launch_unlayout_q8(L.gu_q8 + (size_t)e * d.gu_stride(), L.dn_q8 + (size_t)e * d.dn_stride(),
                                      L.sc_q8 + (size_t)e * (2 * d.F + d.H), d.H, d.F, c->d_stage_q8, c->d_stage_sc,
                                      c->stream));
    HIPCHK(c, hipMemcpyAsync(q, c->d_stage_q8, (size_t)3 * d.F * d.H, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipMemcpyAsync(sc, c->d_stage_sc, (size_t)(2 * d.F + d.H) * 4, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return MOE_GPU_OK;
}

// ------------------------------------------------------------------------------------------------------ compute (device)
int moe_gpu_route_dev(moe_gpu* c, int layer, int T, const uint16_t* x, int keep, int32_t* ids, float* gates,
                      float* logits) {
    int rc = enter(c);
    if (rc) return rc;
    if ((rc = check_layer(c, layer)) || (rc = check_T(c, T)) || (rc = need_router(c, layer))) return rc;
    if (!x || !ids || !gates) return fail(c, MOE_GPU_EINVAL, "NULL x/ids/gates");
    keep = norm_keep(c, keep);
    const LayerPtrs L = ptrs(c, layer);
    unsigned ep = 0;
    if ((rc = next_epoch(c, &ep))) return rc;
    if ((rc = begin_timing(c))) return rc;
    LAUNCH(c, K_ROUTER, moe::launch_router(L, c->d, T, plain_src(x), c->d_logits_tag, logits, ep, c->stream));
    LAUNCH(c, K_TOPK, moe::launch_topk_group(L, c->d, T, keep, c->d.n_shared, true, c->route_rule, c->d_logits_tag,
                                             ep, &c->d_sync->err, ids, gates, c->d_slots, c->stream));
    return end_timing(c);
}

}  // extern "C"

// all_routed: the ids are on the device and unchecked, so every routed expert must be loaded in the call's precision;
// the host entry point checks each id instead
static int moe_dev_impl(moe_gpu* c, int layer, int T, const uint16_t* x, const int32_t* ids, const float* gates,
                        int keep, int with_shared, unsigned flags, float* out, bool all_routed) {
    int rc = enter(c);
    if (rc) return rc;
    if ((rc = check_layer(c, layer)) || (rc = check_T(c, T)) ||
        (rc = need_experts(c, layer, flags, with_shared, all_routed)))
        return rc;
    if (!x || !ids || !gates || !out) return fail(c, MOE_GPU_EINVAL, "NULL x/ids/gates/out");
    keep = norm_keep(c, keep);
    if ((rc = begin_timing(c))) return rc;
    if ((rc = run_layer(c, layer, T, plain_src(x), const_cast<int32_t*>(ids), const_cast<float*>(gates), false, keep,
                        with_shared ? c->d.n_shared : 0, flags, out)))
        return rc;
    return end_timing(c);
}

extern "C" {

int moe_gpu_moe_dev(moe_gpu* c, int layer, int T, const uint16_t* x, const int32_t* ids, const float* gates, int keep,
                    int with_shared, unsigned flags, float* out) {
    return moe_dev_impl(c, layer, T, x, ids, gates, keep, with_shared, flags, out, true);
}

int moe_gpu_layer_dev(moe_gpu* c, int layer, int T, const uint16_t* x, int keep, unsigned flags, float* out,
                      int32_t* ids, float* gates) {
    int rc = enter(c);
    if (rc) return rc;
    if ((rc = check_layer(c, layer)) || (rc = check_T(c, T)) || (rc = need_router(c, layer)) ||
        (rc = need_experts(c, layer, flags, 1, true)))
        return rc;
    if (!x || !out) return fail(c, MOE_GPU_EINVAL, "NULL x/out");
    keep = norm_keep(c, keep);
    int32_t* di = ids ? ids : c->d_ids;
    float* dg = gates ? gates : c->d_gates;
    if ((rc = begin_timing(c))) return rc;
    if ((rc = run_layer(c, layer, T, plain_src(x), di, dg, true, keep, c->d.n_shared, flags, out))) return rc;
    return end_timing(c);
}

int moe_gpu_block_dev(moe_gpu* c, int layer, int T, const uint16_t* resid, const uint16_t* attn_o,
                      const uint16_t* norm_w, float eps, int keep, unsigned flags, uint16_t* x_next, float* out,
                      int32_t* ids, float* gates) {
    int rc = enter(c);
    if (rc) return rc;
    if ((rc = check_layer(c, layer)) || (rc = check_T(c, T)) || (rc = need_router(c, layer)) ||
        (rc = need_experts(c, layer, flags, 1, true)))
        return rc;
    if (!resid || !attn_o || !norm_w || !x_next) return fail(c, MOE_GPU_EINVAL, "NULL resid/attn_o/norm_w/x_next");
    if (flags & MOE_GPU_ACCUMULATE) return fail(c, MOE_GPU_EINVAL, "block calls write x_next; MOE_GPU_ACCUMULATE unsupported");
    if (!(eps >= 0.f)) return fail(c, MOE_GPU_EINVAL, "eps must be >= 0");
    keep = norm_keep(c, keep);
    moe::StageSrc in{nullptr, resid, attn_o, norm_w, eps};
    if ((rc = begin_timing(c))) return rc;
    if ((rc = run_layer(c, layer, T, in, ids ? ids : c->d_ids, gates ? gates : c->d_gates, true, keep, c->d.n_shared,
                        flags, out, x_next)))
        return rc;
    return end_timing(c);
}

// ------------------------------------------------------------------------------------------------------ compute (host)
int moe_gpu_route(moe_gpu* c, int layer, int T, const uint16_t* x, int keep, int32_t* ids, float* gates,
                  float* logits) {
    int rc = enter(c);
    if (rc) return rc;
    if ((rc = check_T(c, T))) return rc;
    if (!x || !ids || !gates) return fail(c, MOE_GPU_EINVAL, "NULL x/ids/gates");
    HIPCHK(c, hipMemcpyAsync(c->d_x, x, (size_t)T * c->d.H * 2, hipMemcpyHostToDevice, c->stream));
    if ((rc = moe_gpu_route_dev(c, layer, T, c->d_x, keep, c->d_ids, c->d_gates, c->d_logits))) return rc;
    HIPCHK(c, hipMemcpyAsync(ids, c->d_ids, (size_t)T * c->d.k * 4, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipMemcpyAsync(gates, c->d_gates, (size_t)T * c->d.k * 4, hipMemcpyDeviceToHost, c->stream));
    if (logits)
        HIPCHK(c, hipMemcpyAsync(logits, c->d_logits, (size_t)T * c->d.E * 4, hipMemcpyDeviceToHost, c->stream));
    return sync_and_check(c);
}

int moe_gpu_moe(moe_gpu* c, int layer, int T, const uint16_t* x, const int32_t* ids, const float* gates, int keep,
                int with_shared, unsigned flags, float* out) {
    int rc = enter(c);
    if (rc) return rc;
    if ((rc = check_layer(c, layer)) || (rc = check_T(c, T))) return rc;
    if (!x || !ids || !gates || !out) return fail(c, MOE_GPU_EINVAL, "NULL x/ids/gates/out");
    const int k = c->d.k, kp = norm_keep(c, keep);
    const Layer& L = c->layers[layer];
    for (int t = 0; t < T; t++)
        for (int r = 0; r < kp; r++) {
            const int e = ids[t * k + r];
            if (e == -1) continue;  // empty rank
            if (e < 0 || e >= c->d.E)
                return fail(c, MOE_GPU_EINVAL, "ids[%d][%d]=%d outside [-1, %d)", t, r, e, c->d.E);
            for (int r2 = 0; r2 < r; r2++)
                if (ids[t * k + r2] == e) return fail(c, MOE_GPU_EINVAL, "token %d selects expert %d twice", t, e);
            if (L.loaded.empty() || !((flags & MOE_GPU_INT8) ? L.loaded_q8[e] : L.loaded[e]))
                return fail(c, MOE_GPU_ESTATE, "layer %d: expert %d not loaded%s", layer, e,
                            (flags & MOE_GPU_INT8) ? " (int8)" : "");
        }
    HIPCHK(c, hipMemcpyAsync(c->d_x, x, (size_t)T * c->d.H * 2, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(c->d_ids, ids, (size_t)T * k * 4, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(c->d_gates, gates, (size_t)T * k * 4, hipMemcpyHostToDevice, c->stream));
    if (flags & MOE_GPU_ACCUMULATE)
        HIPCHK(c, hipMemcpyAsync(c->d_out, out, (size_t)T * c->d.H * 4, hipMemcpyHostToDevice, c->stream));
    if ((rc = moe_dev_impl(c, layer, T, c->d_x, c->d_ids, c->d_gates, keep, with_shared, flags, c->d_out, false)))
        return rc;
    HIPCHK(c, hipMemcpyAsync(out, c->d_out, (size_t)T * c->d.H * 4, hipMemcpyDeviceToHost, c->stream));
    return sync_and_check(c);
}

int moe_gpu_layer(moe_gpu* c, int layer, int T, const uint16_t* x, int keep, unsigned flags, float* out, int32_t* ids,
                  float* gates) {
    int rc = enter(c);
    if (rc) return rc;
    if ((rc = check_T(c, T))) return rc;
    if (!x || !out) return fail(c, MOE_GPU_EINVAL, "NULL x/out");
    HIPCHK(c, hipMemcpyAsync(c->d_x, x, (size_t)T * c->d.H * 2, hipMemcpyHostToDevice, c->stream));
    if (flags & MOE_GPU_ACCUMULATE)
        HIPCHK(c, hipMemcpyAsync(c->d_out, out, (size_t)T * c->d.H * 4, hipMemcpyHostToDevice, c->stream));
    if ((rc = moe_gpu_layer_dev(c, layer, T, c->d_x, keep, flags, c->d_out, c->d_ids, c->d_gates))) return rc;
    HIPCHK(c, hipMemcpyAsync(out, c->d_out, (size_t)T * c->d.H * 4, hipMemcpyDeviceToHost, c->stream));
    if (ids) HIPCHK(c, hipMemcpyAsync(ids, c->d_ids, (size_t)T * c->d.k * 4, hipMemcpyDeviceToHost, c->stream));
    if (gates) HIPCHK(c, hipMemcpyAsync(gates, c->d_gates, (size_t)T * c->d.k * 4, hipMemcpyDeviceToHost, c->stream));
    return sync_and_check(c);
}

// ------------------------------------------------------------------------------------------------------ bench/test
uint64_t moe_gpu_synth_key(uint64_t seed, uint64_t tensor_id) { return moe::synth_key(seed, tensor_id); }

int moe_gpu_synth_fill(moe_gpu* c, uint16_t* dst, uint64_t n, uint64_t key, uint64_t start, float cc) {
    int rc = enter(c);
    if (rc) return rc;
    if (!dst || n % 8) return fail(c, MOE_GPU_EINVAL, "synth_fill: NULL dst or n %% 8 != 0");
    HIPCHK(c, moe::launch_synth_fill(dst, n, key, start, cc, c->stream));
    return MOE_GPU_OK;
}

int moe_gpu_synth_layer(moe_gpu* c, int layer, uint64_t seed, float cw, const float* bias) {
    int rc = enter(c);
    if (rc) return rc;
    if ((rc = check_layer(c, layer)) || (rc = ensure_router(c, layer)) || (rc = ensure_bf16(c, layer)) ||
        (rc = ensure_shared(c, layer)))
        return rc;
    Layer& L = c->layers[layer];
    const Dims& d = c->d;
    auto tid = [&](int e, int m) { return ((uint64_t)layer * 4096 + (uint64_t)e) * 4 + (uint64_t)m; };
    HIPCHK(c, moe::launch_synth_fill(c->d_stage, (uint64_t)d.E * d.H, moe::synth_key(seed, tid(4095, 0)), 0, cw,
                                     c->stream));
    HIPCHK(c, moe::launch_relayout_router(c->d_stage, d.E, d.H, L.wr, c->stream));
    if (bias) HIPCHK(c, hipMemcpyAsync(L.bias, bias, (size_t)d.E * 4, hipMemcpyHostToDevice, c->stream));
    else HIPCHK(c, hipMemsetAsync(L.bias, 0, (size_t)d.E * 4, c->stream));
    for (int e = 0; e < d.E; e++)
        HIPCHK(c, moe::launch_synth_tiled(moe::synth_key(seed, tid(e, 0)), moe::synth_key(seed, tid(e, 1)),
                                          moe::synth_key(seed, tid(e, 2)), cw, d.H, d.F, L.gu + (size_t)e * d.gu_stride(),
                                          L.dn + (size_t)e * d.dn_stride(), c->stream));
    for (int s = 0; s < d.n_shared; s++)
        HIPCHK(c, moe::launch_synth_tiled(moe::synth_key(seed, tid(4000 + s, 0)), moe::synth_key(seed, tid(4000 + s, 1)),
                                          moe::synth_key(seed, tid(4000 + s, 2)), cw, d.H, d.F,
                                          L.sgu + (size_t)s * d.gu_stride(), L.sdn + (size_t)s * d.dn_stride(),
                                          c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    L.router = true;
    for (int e = 0; e < d.E; e++) {
        if (!L.loaded[e]) { L.loaded[e] = 1; L.n_loaded++; }
        if (L.loaded_q8[e]) { L.loaded_q8[e] = 0; L.n_loaded_q8--; }
    }
    for (int s = 0; s < d.n_shared; s++)
        if (!L.shared_loaded[s]) { L.shared_loaded[s] = 1; L.n_shared_loaded++; }
    return MOE_GPU_OK;
}

int moe_gpu_enable_timing(moe_gpu* c, int on) {
    int rc = enter(c);
    if (rc) return rc;
    c->timing = on != 0;
    c->timed = false;
    return MOE_GPU_OK;
}

int moe_gpu_set_option(moe_gpu* c, int opt, int value) {
    int rc = enter(c);
    if (rc) return rc;
    switch (opt) {
        case MOE_GPU_OPT_FUSED: c->fused = value != 0; return MOE_GPU_OK;
        case MOE_GPU_OPT_WG_PER_CU:
            if (value < 0) return fail(c, MOE_GPU_EINVAL, "workgroups per CU %d < 0", value);
            c->wg_per_cu = value;
            return MOE_GPU_OK;
        case MOE_GPU_OPT_KSPLIT:
            if (value != 0 && value != 1 && value != 2 && value != 4)
                return fail(c, MOE_GPU_EINVAL, "K split %d not in {0, 1, 2, 4}", value);
            c->ksplit = value;
            return MOE_GPU_OK;
        case MOE_GPU_OPT_KSPLIT_SHARED:
            if (value != 0 && value != 1 && value != 2 && value != 4)
                return fail(c, MOE_GPU_EINVAL, "shared K split %d not in {0, 1, 2, 4}", value);
            c->ksplit_shared = value;
            return MOE_GPU_OK;
        case MOE_GPU_OPT_LAG:
            if (value < 0) return fail(c, MOE_GPU_EINVAL, "lag %d < 0", value);
            c->lag = value;
            return MOE_GPU_OK;
        case MOE_GPU_OPT_SHARED_WAITS: c->shared_waits = value != 0; return MOE_GPU_OK;
        case MOE_GPU_OPT_GRID:
            if (value < 0) return fail(c, MOE_GPU_EINVAL, "grid %d < 0", value);
            c->grid_req = value;
            return MOE_GPU_OK;
        case MOE_GPU_OPT_ROUTER_POLL:
            if (value < 0) return fail(c, MOE_GPU_EINVAL, "router poll %d < 0", value);
            c->router_poll = value;
            return MOE_GPU_OK;
        case MOE_GPU_OPT_ROUTE_RULE:
            if (value != MOE_GPU_ROUTE_SOFTMAX && value != MOE_GPU_ROUTE_SIGMOID)
                return fail(c, MOE_GPU_EINVAL, "route rule %d not MOE_GPU_ROUTE_SOFTMAX / _SIGMOID", value);
            c->route_rule = value == MOE_GPU_ROUTE_SIGMOID ? moe::kRouteSigmoid : moe::kRouteSoftmax;
            return MOE_GPU_OK;
        default: return fail(c, MOE_GPU_EINVAL, "unknown option %d", opt);
    }
}

int moe_gpu_trace_units(moe_gpu* c, int on) {
    int rc = enter(c);
    if (rc) return rc;
    if (on && !c->d_trace) {
        const size_t units = (size_t)moe::fused_units(moe::router_units(c->d.E, c->d.max_t),
                                                      c->d.n_shared + c->d.max_t * c->d.k, c->d.n_shared, c->d.F,
                                                      c->d.H, moe::kMaxKp, moe::kMaxKp);
        const size_t bytes = units * moe::kTraceFields * sizeof(uint64_t);
        if ((rc = dev_alloc(c, (void**)&c->d_trace, bytes, "unit trace"))) return rc;
        HIPCHK(c, hipMemset(c->d_trace, 0, bytes));
    } else if (!on && c->d_trace) {
        HIPCHK(c, hipStreamSynchronize(c->stream));
        HIPCHK(c, hipFree(c->d_trace));
        c->d_trace = nullptr;
    }
    return MOE_GPU_OK;
}

int moe_gpu_read_trace(moe_gpu* c, uint64_t* buf, int max_units, int* units) {
    int rc = enter(c);
    if (rc) return rc;
    if (!c->d_trace) return fail(c, MOE_GPU_ESTATE, "unit tracing is off");
    if (!buf || !units) return fail(c, MOE_GPU_EINVAL, "NULL buffer");
    const int n = c->trace_units < max_units ? c->trace_units : max_units;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    HIPCHK(c, hipMemcpy(buf, c->d_trace, (size_t)n * moe::kTraceFields * sizeof(uint64_t), hipMemcpyDeviceToHost));
    *units = n;
    return MOE_GPU_OK;
}

int moe_gpu_get_shape(moe_gpu* c, int* H, int* F, int* E, int* topk, int* n_shared, int* n_layers) {
    int rc = enter(c);
    if (rc) return rc;
    if (H) *H = c->d.H;
    if (F) *F = c->d.F;
    if (E) *E = c->d.E;
    if (topk) *topk = c->d.k;
    if (n_shared) *n_shared = c->d.n_shared;
    if (n_layers) *n_layers = c->n_layers;
    return MOE_GPU_OK;
}

int moe_gpu_get_option(moe_gpu* c, int opt, int* value) {
    int rc = enter(c);
    if (rc) return rc;
    if (!value) return fail(c, MOE_GPU_EINVAL, "NULL value");
    switch (opt) {
        case MOE_GPU_OPT_FUSED: *value = c->fused ? 1 : 0; return MOE_GPU_OK;
        case MOE_GPU_OPT_WG_PER_CU: *value = c->wg_per_cu; return MOE_GPU_OK;
        case MOE_GPU_OPT_LAST_GRID: *value = c->last_grid; return MOE_GPU_OK;
        case MOE_GPU_OPT_KSPLIT: *value = c->ksplit; return MOE_GPU_OK;
        case MOE_GPU_OPT_LAG: *value = c->lag; return MOE_GPU_OK;
        case MOE_GPU_OPT_SHARED_WAITS: *value = c->shared_waits; return MOE_GPU_OK;
        case MOE_GPU_OPT_KSPLIT_SHARED: *value = c->ksplit_shared; return MOE_GPU_OK;
        case MOE_GPU_OPT_GRID: *value = c->grid_req; return MOE_GPU_OK;
        case MOE_GPU_OPT_ROUTER_POLL: *value = c->router_poll; return MOE_GPU_OK;
        case MOE_GPU_OPT_ROUTE_RULE:
            *value = c->route_rule == moe::kRouteSigmoid ? MOE_GPU_ROUTE_SIGMOID : MOE_GPU_ROUTE_SOFTMAX;
            return MOE_GPU_OK;
        default: return fail(c, MOE_GPU_EINVAL, "unknown option %d", opt);
    }
}

int moe_gpu_profile_kernels(moe_gpu* c, int on) {
    int rc = enter(c);
    if (rc) return rc;
    if (!on && (rc = prof_resolve(c))) return rc;
    c->profiling = on != 0;
    return MOE_GPU_OK;
}

int moe_gpu_profile_slots(void) { return K_SLOTS; }

int moe_gpu_profile_read(moe_gpu* c, int kernel, double* total_ms, int* launches, const char** name) {
    int rc = enter(c);
    if (rc) return rc;
    if (kernel < 0 || kernel >= K_SLOTS) return fail(c, MOE_GPU_EINVAL, "kernel slot %d outside [0, %d)", kernel, K_SLOTS);
    if ((rc = prof_resolve(c))) return rc;
    if (total_ms) *total_ms = c->prof_ms[kernel];
    if (launches) *launches = c->prof_n[kernel];
    if (name) *name = kKernelNames[kernel];
    return MOE_GPU_OK;
}

int moe_gpu_profile_reset(moe_gpu* c) {
    int rc = enter(c);
    if (rc) return rc;
    if ((rc = prof_resolve(c))) return rc;
    for (int k = 0; k < 8; k++) { c->prof_ms[k] = 0; c->prof_n[k] = 0; }
    return MOE_GPU_OK;
}

int moe_gpu_last_time_ms(moe_gpu* c, float* ms) {
    int rc = enter(c);
    if (rc) return rc;
    if (!ms) return fail(c, MOE_GPU_EINVAL, "NULL ms");
    if (!c->timed) return fail(c, MOE_GPU_ESTATE, "no timed call since timing was enabled");
    HIPCHK(c, hipEventSynchronize(c->ev1));
    HIPCHK(c, hipEventElapsedTime(ms, c->ev0, c->ev1));
    return MOE_GPU_OK;
}

}  // extern "C"
