// lm_head.hip — the last stage of a decode step on one GPU: final RMSNorm, LM-head GEMV over the vocabulary and the
// greedy argmax (include/moe_gpu.h, moe_head_*).  Replaces the host step's tail (track2_opt/solar_engine/src/
// main.rs:381-386: rmsnorm(x, model.norm.weight), gemv(lm_head.weight), first maximum) and the chip path's
// lm_head_am + best_key (src/dense/lm_head.rs:174-181, src/chip.rs:183-194: bf16 logits, ties -> lowest row).
//
// One launch streams the [V, H] bf16 table once for up to kHeadMaxT tokens.  HBM-bound: V*H*2 bytes per launch
// (1.61 GB at V = 196608, H = 4096), about 1 FLOP per byte per token.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdio.h>

#include <string>

#include "launch_util.h"
#include "moe_gpu.h"

namespace {

constexpr int kHeadMaxT = 4;  // tokens per launch; more tokens take several launches
constexpr int kWaves = 4;     // 256 threads
// A wave step covers RB rows, loaded CG 16-byte chunks per lane at a time (a row of H bf16 is H / 512 chunks per
// lane): <8, 2> for any H % 1024 == 0, <HEAD_RB, HEAD_CG> when H % (512 * HEAD_CG) == 0.  At V = 196608, H = 4096
// (one token, pipelined loads): 4 whole rows per step 244.8 us, 2 / 3 / 5 rows 251.3 / 249.9 / 248.8 us, 8 rows of
// 2 KiB slices 279.5 us, 8 rows of 4 KiB 286.5 us.
constexpr int kRB = 8, kCG = 2;
#ifndef HEAD_RB
#define HEAD_RB 4
#endif
#ifndef HEAD_CG
#define HEAD_CG 8
#endif
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }
// round to nearest even, as host.rs:41-46 (NaN is not special-cased there either)
__device__ __forceinline__ uint32_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}
// 64-bit key whose unsigned order is (value, then lower row): the float's bits made order-preserving in the high
// word, the complemented row in the low word.  The reference's first-maximum loop (main.rs:384-385, `lg[i] > lg[best]`
// from best = 0) treats -0 and +0 as equal, so -0 is keyed as +0; it never moves to a NaN and never leaves a NaN at row
// 0, so a NaN ranks with -inf except at row 0, where it ranks above all (the pick is then row 0).  The chip's rule
// (chip.rs:183-194, `val > best || (val == best && row < best_row)`) never picks a NaN: row0_nan_wins = false.
__device__ __forceinline__ unsigned long long key_of(float v, int row, bool row0_nan_wins) {
    if (v != v)
        return row == 0 && row0_nan_wins ? ~0ull : ((unsigned long long)0x007FFFFFu << 32) | (uint32_t)(~(uint32_t)row);
    if (v == 0.f) v = 0.f;
    const uint32_t b = __float_as_uint(v);
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)o << 32) | (uint32_t)(~(uint32_t)row);
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

struct HeadArgs {
    const uint16_t* x;         // [T, H] bf16 residual stream
    const uint16_t* wf;        // [H] bf16 final-norm weight
    const uint16_t* w;         // [V, H] bf16 LM-head table, row-major
    float* logits;             // [T, V] fp32, or null
    unsigned long long* keys;  // [kHeadMaxT] running maxima
    int32_t* ids;              // [T] result rows
    float* best;               // [T] result values
    int T, H, V, rule;
    float eps;
};

// Decodes the running maxima into ids / best and clears them for the next launch (they start at zero from the
// context's creation).
__global__ void head_finish(HeadArgs a) {
    const int t = threadIdx.x;
    if (t >= a.T) return;
    const unsigned long long k = a.keys[t];
    a.keys[t] = 0ull;
    const uint32_t o = (uint32_t)(k >> 32);
    const uint32_t b = (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
    a.ids[t] = (int32_t)(~(uint32_t)k);
    a.best[t] = __uint_as_float(b);
}

// Workgroup: 4 waves.  Each workgroup first normalises the T tokens into LDS (every workgroup repeats this 2*T*H
// byte read, served by L2), then its waves take steps of kRB consecutive rows, grid-strided over the table.  Lane l
// reads 16-byte chunks l, l + 64, ... of each row (one wave load = 1 KiB of a row), multiplies them with the same
// chunks of the normalised tokens from LDS and keeps fp32 partial sums; a butterfly sums the 64 lanes.
template <int NT, int RB, int CG>
__global__ __launch_bounds__(256) void head_kernel(HeadArgs a) {
    extern __shared__ __align__(16) uint16_t hn[];  // [NT][H] bf16
    __shared__ float red[NT][kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int H = a.H, V = a.V, T = a.T;

    // RMSNorm (host.rs:71-76): ms = sum(x^2) / H in fp32, r = 1 / sqrt(ms + eps), hn = bf16(bf16(x * r) * w).
    // Token columns t >= T normalise token 0 and are never read back.
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const uint16_t* xt = a.x + (size_t)(t < T ? t : 0) * H;
        float s = 0.f;
        for (int i = tid; i < H; i += 256) {
            const float v = bf2f(xt[i]);
            s = fmaf(v, v, s);
        }
        s = wave_sum(s);
        if (lane == 0) red[t][wv] = s;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float ms = (red[t][0] + red[t][1] + red[t][2] + red[t][3]) / (float)H;
        const float r = 1.0f / sqrtf(ms + a.eps);
        const uint16_t* xt = a.x + (size_t)(t < T ? t : 0) * H;
        for (int i = tid; i < H; i += 256)
            hn[t * H + i] = (uint16_t)f2bf(bf2f(f2bf(bf2f(xt[i]) * r)) * bf2f(a.wf[i]));
    }
    __syncthreads();

    const int nch = H / 512;  // chunks per lane per row
    const int gw = blockIdx.x * kWaves + wv, nw = gridDim.x * kWaves;
    unsigned long long best[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) best[t] = 0ull;

    // The wave walks its load groups in order (c0 over a row step's chunks, then its next row step); the next
    // group's loads are issued as soon as the current group's products are done, so they are in flight during the
    // step's butterfly and argmax.
    u32x4 wq[RB][CG];
    float acc[NT][RB];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < RB; ++r) acc[t][r] = 0.f;
    auto load_group = [&](int r0_, int c0_) {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int row = r0_ + r < V ? r0_ + r : V - 1;  // rows past V re-read the last row; discarded below
            const u32x4* wr = reinterpret_cast<const u32x4*>(a.w + (size_t)row * H);
#pragma unroll
            for (int c = 0; c < CG; ++c) wq[r][c] = __builtin_nontemporal_load(&wr[(c0_ + c) * 64 + lane]);
        }
    };
    int r0 = gw * RB, c0 = 0;
    if (r0 < V) load_group(r0, 0);
    while (r0 < V) {
#pragma unroll
        for (int c = 0; c < CG; ++c) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const u32x4 h4 = *reinterpret_cast<const u32x4*>(&hn[t * H + ((c0 + c) * 64 + lane) * 8]);
                const uint32_t hw[4] = {h4.x, h4.y, h4.z, h4.w};
#pragma unroll
                for (int r = 0; r < RB; ++r) {
                    const uint32_t ww[4] = {wq[r][c].x, wq[r][c].y, wq[r][c].z, wq[r][c].w};
                    float s = acc[t][r];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        s = fmaf(__uint_as_float(ww[j] << 16), __uint_as_float(hw[j] << 16), s);
                        s = fmaf(__uint_as_float(ww[j] & 0xFFFF0000u), __uint_as_float(hw[j] & 0xFFFF0000u), s);
                    }
                    acc[t][r] = s;
                }
            }
        }
        int nr0 = r0, nc0 = c0 + CG;
        if (nc0 >= nch) {
            nc0 = 0;
            nr0 = r0 + nw * RB;
        }
        if (nr0 < V) load_group(nr0, nc0);
        if (nc0 == 0) {  // row step r0 complete
#pragma unroll
            for (int t = 0; t < NT; ++t) {
#pragma unroll
                for (int r = 0; r < RB; ++r) {
                    const float tot = wave_sum(acc[t][r]);
                    acc[t][r] = 0.f;
                    const int row = r0 + r;
                    if (row < V && t < T) {
                        if (a.logits && lane == r) a.logits[(size_t)t * V + row] = tot;
                        const float v = a.rule ? bf2f(f2bf(tot)) : tot;
                        const unsigned long long k = key_of(v, row, a.rule == 0);
                        best[t] = k > best[t] ? k : best[t];
                    }
                }
            }
        }
        r0 = nr0;
        c0 = nc0;
    }
    if (lane == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
            if (t < T && best[t]) atomicMax(&a.keys[t], best[t]);
    }
}

// One workgroup per token row: the per-layer RMSNorm of host.rs:71-76 (input_layernorm / post_attention_layernorm),
// the same arithmetic as the head's prologue.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* x, const uint16_t* w, uint16_t* out, int H,
                                                      float eps) {
    __shared__ float red[kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint16_t* xt = x + (size_t)blockIdx.x * H;
    float s = 0.f;
    for (int i = tid; i < H; i += 256) {
        const float v = bf2f(xt[i]);
        s = fmaf(v, v, s);
    }
    s = wave_sum(s);
    if (lane == 0) red[wv] = s;
    __syncthreads();
    const float ms = (red[0] + red[1] + red[2] + red[3]) / (float)H;
    const float r = 1.0f / sqrtf(ms + eps);
    for (int i = tid; i < H; i += 256)
        out[(size_t)blockIdx.x * H + i] = (uint16_t)f2bf(bf2f(f2bf(bf2f(xt[i]) * r)) * bf2f(w[i]));
}

}  // namespace

struct moe_head {
    int device = 0;
    int H = 0, V = 0;
    float eps = 1e-5f;
    hipStream_t own_stream = nullptr, stream = nullptr;
    uint16_t* w = nullptr;
    uint16_t* wf = nullptr;
    unsigned long long* keys = nullptr;
    int32_t* d_ids = nullptr;
    float* d_best = nullptr;
    uint16_t* d_x = nullptr;  // host path staging, [kHeadMaxT, H]
    float* d_logits = nullptr;  // host path logits staging, [kHeadMaxT, V], allocated on first request
    bool loaded = false;
    int grid[kHeadMaxT + 1] = {};
    std::string err = "no error";
};

namespace {

std::string g_head_create_err = "no error";

int hfail(moe_head* h, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (h) h->err = buf;
    else g_head_create_err = buf;
    return code;
}

#define HCHK(h, expr)                                                                                           \
    do {                                                                                                        \
        hipError_t e_ = (expr);                                                                                 \
        if (e_ != hipSuccess)                                                                                   \
            return hfail((h), e_ == hipErrorNoBinaryForGpu ? MOE_GPU_ENOKERNEL : MOE_GPU_EHIP, "%s: %s (%s:%d)", \
                         #expr, hipGetErrorString(e_), __FILE__, __LINE__);                                     \
    } while (0)

template <int NT, int RB, int CG>
int head_grid(moe_head* h, size_t lds, int* grid) {
    const void* fn = reinterpret_cast<const void*>(&head_kernel<NT, RB, CG>);
    // the limit is process-wide (another context's smaller table must not lower it): raised only, every launch
    HCHK(h, moe::raise_lds_limit(fn, lds));
    if (h->grid[NT] == 0) {
        int ncu = 0, per_cu = 0;
        HCHK(h, hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, h->device));
        HCHK(h, hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, lds));
        if (per_cu < 1) return hfail(h, MOE_GPU_EINVAL, "head kernel does not fit a CU with %zu bytes of LDS", lds);
        h->grid[NT] = ncu * per_cu;
    }
    const int steps = (h->V + RB - 1) / RB;
    const int need = (steps + kWaves - 1) / kWaves;
    *grid = h->grid[NT] < need ? h->grid[NT] : need;
    return MOE_GPU_OK;
}

template <int NT, int RB, int CG>
int head_launch_rc(moe_head* h, HeadArgs a) {
    const size_t lds = (size_t)NT * h->H * sizeof(uint16_t);
    int grid = 0, rc;
    if ((rc = head_grid<NT, RB, CG>(h, lds, &grid)) != MOE_GPU_OK) return rc;
    hipLaunchKernelGGL((head_kernel<NT, RB, CG>), dim3(grid), dim3(256), lds, h->stream, a);
    HCHK(h, hipGetLastError());
    return MOE_GPU_OK;
}

template <int NT>
int head_launch(moe_head* h, HeadArgs a) {
    return h->H % (512 * HEAD_CG) == 0 ? head_launch_rc<NT, HEAD_RB, HEAD_CG>(h, a) : head_launch_rc<NT, kRB, kCG>(h, a);
}

// Launch sequence for tokens [0, T) of device buffers, kHeadMaxT tokens per table pass.
int head_run(moe_head* h, int T, const uint16_t* x, int rule, int32_t* ids, float* best, float* logits) {
    for (int t0 = 0; t0 < T; t0 += kHeadMaxT) {
        const int n = T - t0 < kHeadMaxT ? T - t0 : kHeadMaxT;
        HeadArgs a{x + (size_t)t0 * h->H, h->wf, h->w, logits ? logits + (size_t)t0 * h->V : nullptr, h->keys,
                   ids + t0, best + t0, n, h->H, h->V, rule, h->eps};
        int rc = n == 1 ? head_launch<1>(h, a) : n == 2 ? head_launch<2>(h, a) : head_launch<4>(h, a);
        if (rc != MOE_GPU_OK) return rc;
        hipLaunchKernelGGL(head_finish, dim3(1), dim3(64), 0, h->stream, a);
        HCHK(h, hipGetLastError());
    }
    return MOE_GPU_OK;
}

int head_check(moe_head* h, int T, int rule, const void* x, const void* ids, const void* best) {
    if (!h) return MOE_GPU_EINVAL;
    if (!h->loaded) return hfail(h, MOE_GPU_ESTATE, "LM-head weights not loaded");
    if (T < 1 || T > 64) return hfail(h, MOE_GPU_EINVAL, "T=%d outside [1, 64]", T);
    if (rule != MOE_HEAD_ARGMAX_FP32 && rule != MOE_HEAD_ARGMAX_BF16)
        return hfail(h, MOE_GPU_EINVAL, "unknown argmax rule %d", rule);
    if (!x || !ids || !best) return hfail(h, MOE_GPU_EINVAL, "null x / ids / best");
    return MOE_GPU_OK;
}

}  // namespace

extern "C" {

int moe_head_create(int device, int H, int V, float eps, moe_head** out) {
    if (!out) return hfail(nullptr, MOE_GPU_EINVAL, "null out");
    *out = nullptr;
    if (H < 512 || H % (512 * kCG) != 0 || H > 16384)
        return hfail(nullptr, MOE_GPU_EINVAL, "H=%d: need H %% %d == 0 and 512 <= H <= 16384", H, 512 * kCG);
    if (V < 1) return hfail(nullptr, MOE_GPU_EINVAL, "V=%d < 1", V);
    if (!(eps >= 0.f)) return hfail(nullptr, MOE_GPU_EINVAL, "eps must be >= 0");
    moe_head* h = new moe_head;
    h->device = device;
    h->H = H;
    h->V = V;
    h->eps = eps;
    auto fail_create = [&](int code) {
        g_head_create_err = h->err;
        moe_head_destroy(h);
        return code;
    };
#define HCREATE(expr)                                                                                            \
    do {                                                                                                         \
        hipError_t e_ = (expr);                                                                                  \
        if (e_ != hipSuccess) {                                                                                  \
            hfail(h, e_ == hipErrorOutOfMemory ? MOE_GPU_ENOMEM : MOE_GPU_EHIP, "%s: %s", #expr, hipGetErrorString(e_)); \
            return fail_create(e_ == hipErrorOutOfMemory ? MOE_GPU_ENOMEM : MOE_GPU_EHIP);                       \
        }                                                                                                        \
    } while (0)
    HCREATE(hipSetDevice(device));
    HCREATE(hipStreamCreateWithFlags(&h->own_stream, hipStreamNonBlocking));
    h->stream = h->own_stream;
    HCREATE(hipMalloc(&h->w, (size_t)V * H * sizeof(uint16_t)));
    HCREATE(hipMalloc(&h->wf, (size_t)H * sizeof(uint16_t)));
    HCREATE(hipMalloc(&h->keys, kHeadMaxT * sizeof(unsigned long long)));
    HCREATE(hipMemset(h->keys, 0, kHeadMaxT * sizeof(unsigned long long)));
    HCREATE(hipMalloc(&h->d_ids, 64 * sizeof(int32_t)));
    HCREATE(hipMalloc(&h->d_best, 64 * sizeof(float)));
    HCREATE(hipMalloc(&h->d_x, (size_t)64 * H * sizeof(uint16_t)));
#undef HCREATE
    *out = h;
    return MOE_GPU_OK;
}

void moe_head_destroy(moe_head* h) {
    if (!h) return;
    (void)hipSetDevice(h->device);
    if (h->own_stream) (void)hipStreamSynchronize(h->own_stream);
    (void)hipFree(h->w);
    (void)hipFree(h->wf);
    (void)hipFree(h->keys);
    (void)hipFree(h->d_ids);
    (void)hipFree(h->d_best);
    (void)hipFree(h->d_x);
    (void)hipFree(h->d_logits);
    if (h->own_stream) (void)hipStreamDestroy(h->own_stream);
    delete h;
}

const char* moe_head_last_error(const moe_head* h) { return h ? h->err.c_str() : g_head_create_err.c_str(); }

int moe_head_set_stream(moe_head* h, void* stream) {
    if (!h) return MOE_GPU_EINVAL;
    h->stream = stream ? (hipStream_t)stream : h->own_stream;
    return MOE_GPU_OK;
}

int moe_head_synchronize(moe_head* h) {
    if (!h) return MOE_GPU_EINVAL;
    HCHK(h, hipSetDevice(h->device));
    HCHK(h, hipStreamSynchronize(h->stream));
    return MOE_GPU_OK;
}

int moe_head_load(moe_head* h, const uint16_t* w_lm, const uint16_t* w_final) {
    if (!h) return MOE_GPU_EINVAL;
    if (!w_lm || !w_final) return hfail(h, MOE_GPU_EINVAL, "null weights");
    HCHK(h, hipSetDevice(h->device));
    HCHK(h, hipMemcpyAsync(h->w, w_lm, (size_t)h->V * h->H * 2, hipMemcpyHostToDevice, h->stream));
    HCHK(h, hipMemcpyAsync(h->wf, w_final, (size_t)h->H * 2, hipMemcpyHostToDevice, h->stream));
    HCHK(h, hipStreamSynchronize(h->stream));
    h->loaded = true;
    return MOE_GPU_OK;
}

int moe_head_load_dev(moe_head* h, const uint16_t* w_lm, const uint16_t* w_final) {
    if (!h) return MOE_GPU_EINVAL;
    if (!w_lm || !w_final) return hfail(h, MOE_GPU_EINVAL, "null weights");
    HCHK(h, hipSetDevice(h->device));
    HCHK(h, hipMemcpyAsync(h->w, w_lm, (size_t)h->V * h->H * 2, hipMemcpyDeviceToDevice, h->stream));
    HCHK(h, hipMemcpyAsync(h->wf, w_final, (size_t)h->H * 2, hipMemcpyDeviceToDevice, h->stream));
    HCHK(h, hipStreamSynchronize(h->stream));
    h->loaded = true;
    return MOE_GPU_OK;
}

int moe_head_argmax(moe_head* h, int T, const uint16_t* x, int rule, int32_t* ids, float* best, float* logits) {
    int rc = head_check(h, T, rule, x, ids, best);
    if (rc != MOE_GPU_OK) return rc;
    HCHK(h, hipSetDevice(h->device));
    if (logits && !h->d_logits) {
        const size_t bytes = (size_t)64 * h->V * sizeof(float);
        hipError_t e = hipMalloc(&h->d_logits, bytes);
        if (e != hipSuccess) {
            h->d_logits = nullptr;
            return hfail(h, MOE_GPU_ENOMEM, "hipMalloc(%zu bytes) for logits failed: %s", bytes, hipGetErrorString(e));
        }
    }
    HCHK(h, hipMemcpyAsync(h->d_x, x, (size_t)T * h->H * 2, hipMemcpyHostToDevice, h->stream));
    if ((rc = head_run(h, T, h->d_x, rule, h->d_ids, h->d_best, logits ? h->d_logits : nullptr)) != MOE_GPU_OK)
        return rc;
    HCHK(h, hipMemcpyAsync(ids, h->d_ids, (size_t)T * sizeof(int32_t), hipMemcpyDeviceToHost, h->stream));
    HCHK(h, hipMemcpyAsync(best, h->d_best, (size_t)T * sizeof(float), hipMemcpyDeviceToHost, h->stream));
    if (logits)
        HCHK(h, hipMemcpyAsync(logits, h->d_logits, (size_t)T * h->V * sizeof(float), hipMemcpyDeviceToHost,
                               h->stream));
    HCHK(h, hipStreamSynchronize(h->stream));
    return MOE_GPU_OK;
}

int moe_rmsnorm_dev(int T, int H, const uint16_t* x, const uint16_t* w, float eps, uint16_t* out, void* stream) {
    if (T < 1 || H < 1 || H > (1 << 20) || !x || !w || !out || !(eps >= 0.f)) return MOE_GPU_EINVAL;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(256), 0, static_cast<hipStream_t>(stream), x, w, out, H, eps);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e == hipErrorNoBinaryForGpu ? MOE_GPU_ENOKERNEL : MOE_GPU_EHIP;
    return MOE_GPU_OK;
}

int moe_head_argmax_dev(moe_head* h, int T, const uint16_t* x, int rule, int32_t* ids, float* best, float* logits) {
    int rc = head_check(h, T, rule, x, ids, best);
    if (rc != MOE_GPU_OK) return rc;
    HCHK(h, hipSetDevice(h->device));
    return head_run(h, T, x, rule, ids, best, logits);
}

}  // extern "C"
