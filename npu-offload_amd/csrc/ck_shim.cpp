// ck_shim.cpp — libck_gpu.so: the reference engine's CPU-kernel boundary, served by the GPU tier.
//
// track2_opt/solar_engine links the `extern "C"` block of src/host.rs:18-37 against csrc/cpu_kern.c (built by its
// build.rs).  This library exports the same symbols with the same signatures, so the engine links it instead (its
// build.rs links `ck_gpu` in place of compiling cpu_kern.c) and its host paths run on one MI355X:
//   ck_gemv                    fp32 GEMV in ck_gemv's own summation order (moe_gemv_f32_dev): bit-identical y
//   ck_place_expert            the reference's copy into the caller's buffer, plus an upload of the expert to the
//                              GPU tier, keyed by that buffer's address
//   ck_moe3                    experts given by placed base pointers: the grouped GPU expert call (moe_gpu_moe),
//                              out += sum_e w[e] * expert_e(x) in list order
//   ck_moe1 / ck_moe2          the same for experts given as (g, u, d) pointers (uploaded on first use)
//   ck_place_expert_q8         the int8 copy in the caller's buffers (q, sc, rs: quantised on the GPU with quant_row's
//                              rule, bit-identical) and in the GPU tier, keyed by q
//   ck_moe_q8w                 the int8 weight-only experts (MOE_GPU_INT8)
//   ck_moe_q8 / ck_moe_q8x     served by the same weight-only path: the GPU keeps the activations in bf16, so the
//                              reference's int8-activation approximation (q8) does not apply; q8x is weight-only in
//                              the reference as well
//   ck_set_threads, ck_touch_experts, ck_read_bw, ck_mmio_*   host-side helpers kept for linking (no GPU work)
// The tier holds experts in "pool layers" of kPoolE slots each (a moe_gpu context with n_layers = pool layers); a
// call's experts are grouped into runs of consecutive list entries in the same pool layer, of at most topk = 8, each
// run one accumulate call, so the sum keeps the list order.  Calls are synchronous, like the reference's.  void
// functions cannot return errors: a failure is recorded for ck_gpu_last_error() and printed once to stderr.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <chrono>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "moe_gpu.h"

namespace {

constexpr int kPoolE = 128;       // expert slots per pool layer
constexpr int kPoolLayers = 96;   // 12288 experts
constexpr int kTopk = 8;          // experts per tier call

struct Slot {
    int layer, e;
};

struct Shim {
    std::mutex mu;
    moe_gpu* tier = nullptr;
    int H = 0, F = 0, next_slot = 0;
    std::unordered_map<const void*, Slot> bf16, q8;  // host pointer -> tier slot
    std::string err = "no error";
    bool reported = false;
    // ck_gemv: device copies of the weight tables, keyed by host pointer, checked by size and by a copy of their first
    // and last 128 bytes (a freed host buffer's address can come back holding another table)
    struct Table {
        uint16_t* d = nullptr;
        size_t n = 0;
        unsigned char head[128], tail[128];
    };
    std::unordered_map<const void*, Table> tables;
    uint16_t* d_x = nullptr;
    float* d_y = nullptr;
    size_t cap_x = 0, cap_y = 0;
};

Shim& shim() {
    static Shim s;
    return s;
}

void record(Shim& s, const std::string& msg) {
    s.err = msg;
    if (!s.reported) {
        fprintf(stderr, "libck_gpu: %s\n", msg.c_str());
        s.reported = true;
    }
}

bool ensure_tier(Shim& s, int H, int F) {
    if (s.tier) {
        if (H != s.H || F != s.F) {
            record(s, "H/F differ from the first call's (one expert shape per process)");
            return false;
        }
        return true;
    }
    const int rc = moe_gpu_create(0, H, F, kPoolE, kTopk, 0, kPoolLayers, 1, &s.tier);
    if (rc != MOE_GPU_OK) {
        record(s, std::string("moe_gpu_create: ") + moe_gpu_last_error(nullptr));
        s.tier = nullptr;
        return false;
    }
    s.H = H;
    s.F = F;
    return true;
}

bool tier_ok(Shim& s, int rc, const char* what) {
    if (rc == MOE_GPU_OK) return true;
    record(s, std::string(what) + ": " + moe_gpu_last_error(s.tier));
    return false;
}

bool new_slot(Shim& s, Slot* out) {
    if (s.next_slot >= kPoolE * kPoolLayers) {
        record(s, "expert pool full");
        return false;
    }
    *out = Slot{s.next_slot / kPoolE, s.next_slot % kPoolE};
    s.next_slot++;
    return true;
}

// out[H] += sum_i w[i] * expert(slot[i])(x), in list order: runs of consecutive entries of one pool layer, <= kTopk
void run_experts(Shim& s, int E, const Slot* slots, const float* w, const uint16_t* x, float* out, unsigned flags) {
    int i = 0;
    while (i < E) {
        int j = i + 1;
        while (j < E && j - i < kTopk && slots[j].layer == slots[i].layer) j++;
        int32_t ids[kTopk];
        float g[kTopk];
        for (int r = 0; r < kTopk; r++) {
            ids[r] = r < j - i ? slots[i + r].e : -1;
            g[r] = r < j - i ? w[i + r] : 0.f;
        }
        if (!tier_ok(s, moe_gpu_moe(s.tier, slots[i].layer, 1, x, ids, g, j - i, 0, flags | MOE_GPU_ACCUMULATE, out),
                     "moe_gpu_moe"))
            return;
        i = j;
    }
}

// Slot of an expert given by (g, u, d) pointers, uploaded on first use only (the engine's mmap'd safetensors weights
// are immutable and keep their addresses).
bool slot_of_gud(Shim& s, const uint16_t* g, const uint16_t* u, const uint16_t* d, Slot* out) {
    auto it = s.bf16.find(g);
    if (it != s.bf16.end()) {
        *out = it->second;
        return true;
    }
    Slot sl;
    if (!new_slot(s, &sl)) return false;
    if (!tier_ok(s, moe_gpu_load_expert(s.tier, sl.layer, sl.e, g, u, d), "moe_gpu_load_expert")) return false;
    s.bf16[g] = sl;
    *out = sl;
    return true;
}

}  // namespace

extern "C" {

const char* ck_gpu_last_error(void) { return shim().err.c_str(); }

void ck_set_threads(int n) { (void)n; }  // the GPU tier has no host thread team

void ck_gemv(const uint16_t* W, const uint16_t* x, float* y, int M, int K) {
    Shim& s = shim();
    std::lock_guard<std::mutex> lock(s.mu);
    if (M <= 0) return;
    const size_t n = (size_t)M * K;
    Shim::Table& t = s.tables[W];
    const size_t edge = n * 2 < 128 ? n * 2 : 128;
    const unsigned char* wb = reinterpret_cast<const unsigned char*>(W);
    if (t.n != n || memcmp(t.head, wb, edge) != 0 || memcmp(t.tail, wb + n * 2 - edge, edge) != 0) {
        if (t.d) (void)hipFree(t.d);
        t.d = nullptr;
        if (hipMalloc((void**)&t.d, n * 2) != hipSuccess || hipMemcpy(t.d, W, n * 2, hipMemcpyHostToDevice) != hipSuccess) {
            record(s, "ck_gemv: table upload failed");
            t.n = 0;
            return;
        }
        t.n = n;
        memcpy(t.head, wb, edge);
        memcpy(t.tail, wb + n * 2 - edge, edge);
    }
    if ((size_t)K > s.cap_x) {
        if (s.d_x) (void)hipFree(s.d_x);
        if (hipMalloc((void**)&s.d_x, (size_t)K * 2) != hipSuccess) { record(s, "ck_gemv: x alloc failed"); s.cap_x = 0; return; }
        s.cap_x = K;
    }
    if ((size_t)M > s.cap_y) {
        if (s.d_y) (void)hipFree(s.d_y);
        if (hipMalloc((void**)&s.d_y, (size_t)M * 4) != hipSuccess) { record(s, "ck_gemv: y alloc failed"); s.cap_y = 0; return; }
        s.cap_y = M;
    }
    if (hipMemcpy(s.d_x, x, (size_t)K * 2, hipMemcpyHostToDevice) != hipSuccess) { record(s, "ck_gemv: x upload"); return; }
    const int rc = moe_gemv_f32_dev(M, K, t.d, s.d_x, s.d_y, nullptr);
    if (rc != MOE_GPU_OK) { record(s, "ck_gemv: moe_gemv_f32_dev failed (K % 512 == 0 required)"); return; }
    if (hipMemcpy(y, s.d_y, (size_t)M * 4, hipMemcpyDeviceToHost) != hipSuccess) record(s, "ck_gemv: y download");
}

void ck_place_expert(const uint16_t* g, const uint16_t* u, const uint16_t* d, uint16_t* dst, int H, int F) {
    Shim& s = shim();
    std::lock_guard<std::mutex> lock(s.mu);
    const size_t n = (size_t)F * H;
    memcpy(dst, g, n * 2);  // the reference's layout [g | u | d] in the caller's buffer (cpu_kern.c:124-138)
    memcpy(dst + n, u, n * 2);
    memcpy(dst + 2 * n, d, n * 2);
    if (!ensure_tier(s, H, F)) return;
    Slot sl;
    auto it = s.bf16.find(dst);  // a reused buffer address keeps its slot and gets the new weights
    if (it != s.bf16.end()) sl = it->second;
    else if (!new_slot(s, &sl)) return;
    if (!tier_ok(s, moe_gpu_load_expert(s.tier, sl.layer, sl.e, g, u, d), "moe_gpu_load_expert")) return;
    s.bf16[dst] = sl;
}

void ck_moe3(int E, const uint16_t* const* base, const float* w, const uint16_t* x, float* out, int H, int F) {
    Shim& s = shim();
    std::lock_guard<std::mutex> lock(s.mu);
    if (E <= 0 || !ensure_tier(s, H, F)) return;
    std::vector<Slot> sl(E);
    for (int i = 0; i < E; i++) {
        auto it = s.bf16.find(base[i]);
        if (it == s.bf16.end()) {  // not placed through this library: upload from the [g | u | d] layout
            const size_t n = (size_t)F * H;
            if (!slot_of_gud(s, base[i], base[i] + n, base[i] + 2 * n, &sl[i])) return;
            s.bf16[base[i]] = sl[i];
        } else {
            sl[i] = it->second;
        }
    }
    run_experts(s, E, sl.data(), w, x, out, 0);
}

static void moe_gud(int E, const uint16_t* const* g, const uint16_t* const* u, const uint16_t* const* d,
                    const float* w, const uint16_t* x, float* out, int H, int F) {
    Shim& s = shim();
    std::lock_guard<std::mutex> lock(s.mu);
    if (E <= 0 || !ensure_tier(s, H, F)) return;
    std::vector<Slot> sl(E);
    for (int i = 0; i < E; i++)
        if (!slot_of_gud(s, g[i], u[i], d[i], &sl[i])) return;
    run_experts(s, E, sl.data(), w, x, out, 0);
}

void ck_moe1(int E, const uint16_t* const* g, const uint16_t* const* u, const uint16_t* const* d, const float* w,
             const uint16_t* x, float* out, int H, int F) {
    moe_gud(E, g, u, d, w, x, out, H, F);
}

void ck_moe2(int E, const uint16_t* const* g, const uint16_t* const* u, const uint16_t* const* d, const float* w,
             const uint16_t* x, float* out, int H, int F) {
    moe_gud(E, g, u, d, w, x, out, H, F);
}

void ck_place_expert_q8(const uint16_t* g, const uint16_t* u, const uint16_t* d, int8_t* qbuf, float* sc, int32_t* rs,
                        int H, int F) {
    Shim& s = shim();
    std::lock_guard<std::mutex> lock(s.mu);
    if (!ensure_tier(s, H, F)) return;
    // quantise on the GPU (quant_row's rule, bit-identical): the bf16 expert goes to the slot of the caller's q
    // buffer (placing into the same buffer again reuses it; any other buffer gets a slot of its own, so that freed and
    // reused host addresses of g / u / d never make two placed experts share a slot), and its int8 copy is read back
    // into the caller's buffers
    Slot sl;
    auto it = s.q8.find(qbuf);
    if (it != s.q8.end()) sl = it->second;
    else if (!new_slot(s, &sl)) return;
    if (!tier_ok(s, moe_gpu_load_expert(s.tier, sl.layer, sl.e, g, u, d), "moe_gpu_load_expert")) return;
    if (!tier_ok(s, moe_gpu_quantize_experts(s.tier, sl.layer, sl.e, sl.e + 1), "moe_gpu_quantize_experts")) return;
    if (!tier_ok(s, moe_gpu_get_expert_q8(s.tier, sl.layer, sl.e, qbuf, sc), "moe_gpu_get_expert_q8")) return;
    const int rows = 2 * F + H;
    for (int r = 0; r < rows; r++) {  // per-row sums of q (the reference's rs, used by its int8-activation variant)
        const int n = r < 2 * F ? H : F;
        const int8_t* q = qbuf + (r < 2 * F ? (size_t)r * H : (size_t)2 * F * H + (size_t)(r - 2 * F) * F);
        int32_t acc = 0;
        for (int i = 0; i < n; i++) acc += q[i];
        rs[r] = acc;
    }
    s.q8[qbuf] = sl;
}

static void moe_q8_any(int E, int8_t* const* q, const float* w, const uint16_t* x, float* out, int H, int F) {
    Shim& s = shim();
    std::lock_guard<std::mutex> lock(s.mu);
    if (E <= 0 || !ensure_tier(s, H, F)) return;
    std::vector<Slot> sl(E);
    for (int i = 0; i < E; i++) {
        auto it = s.q8.find(q[i]);
        if (it == s.q8.end()) {
            record(s, "ck_moe_q8*: an expert was not placed with ck_place_expert_q8 through this library");
            return;
        }
        sl[i] = it->second;
    }
    run_experts(s, E, sl.data(), w, x, out, MOE_GPU_INT8);
}

void ck_moe_q8w(int E, int8_t* const* q, float* const* sc, const float* w, const uint16_t* x, float* out, int H, int F) {
    (void)sc;
    moe_q8_any(E, q, w, x, out, H, F);
}

void ck_moe_q8(int E, int8_t* const* q, float* const* sc, int32_t* const* rs, const float* w, const uint16_t* x,
               float* out, int H, int F) {
    (void)sc;
    (void)rs;
    moe_q8_any(E, q, w, x, out, H, F);
}

void ck_moe_q8x(int E, int8_t* const* q, float* const* sc, int32_t* const* rs, const float* w, const uint16_t* x,
                float* out, int H, int F) {
    (void)sc;
    (void)rs;
    moe_q8_any(E, q, w, x, out, H, F);
}

// Host-side helpers of the reference (no GPU work): a cache warm-up of placed experts (nothing to warm: the experts
// are in HBM), a host read-bandwidth probe, and the NPU's MMIO copy.
float ck_touch_experts(int E, const uint16_t* const* base, int H, int F) {
    (void)E; (void)base; (void)H; (void)F;
    return 0.f;
}

double ck_read_bw(size_t n_per_thread, int iters) {
    std::vector<uint64_t> buf(n_per_thread / 8 + 1, 1);
    double best = 0;
    for (int it = 0; it < iters; it++) {
        const auto t0 = std::chrono::steady_clock::now();
        uint64_t acc = 0;
        for (uint64_t v : buf) acc += v;
        const double dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        volatile uint64_t sink = acc;
        (void)sink;
        if (dt > 0 && n_per_thread / dt / 1e9 > best) best = n_per_thread / dt / 1e9;
    }
    return best;
}

void ck_mmio_set_threads(int n) { (void)n; }
void ck_mmio_read(const uint8_t* src, uint8_t* dst, size_t len) { memcpy(dst, src, len); }

}  // extern "C"
