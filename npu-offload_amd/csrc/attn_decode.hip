// attn_decode.hip — GQA decode attention of one token over a layer's KV cache (include/moe_gpu.h, moe_attn_*).
// Replaces the host step's attention core (track2_opt/solar_engine/src/main.rs:86-104): for q head h, kv head
// h / (NQ / NKV), positions t < S:
//   sc[t] = bf16(bf16(q_h . k_t) * scale)   (the dot summed left to right in fp32)
//   p[t]  = bf16(exp(sc[t] - max sc) / sum exp(sc - max sc))
//   out_h = bf16(sum_t p[t] * v_t)
// Three kernels: scores (one lane per position and kv head, the dot in the reference's order, so the scores are
// bit-identical), softmax + partial P.V per 128-position chunk, and the sum of the chunk partials.  HBM-bound on the
// cache read: 2 * S * NKV * D * 2 bytes per call (16.8 MB at S = 4096, NKV = 8, D = 128).
#include <hip/hip_runtime.h>

#include <stddef.h>

#include <mutex>

#include "moe_gpu.h"

namespace {

constexpr int kD = 128;      // head dim
#ifndef ATTN_CHUNK
#define ATTN_CHUNK 128
#endif
#ifndef ATTN_ST
#define ATTN_ST 64
#endif
constexpr int kChunk = ATTN_CHUNK;  // positions per P.V workgroup
constexpr int kST = ATTN_ST;        // threads (positions) per score workgroup
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ uint32_t f2bf(float f) {  // round to nearest even (host.rs:41-46)
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

struct AttnArgs {
    const uint16_t* q;  // [NQ, D] bf16
    const uint16_t* k;  // [S, NKV, D] bf16
    const uint16_t* v;  // [S, NKV, D] bf16
    uint16_t* out;      // [NQ, D] bf16
    float* scores;      // [NQ, S]
    float* part;        // [NQ, nchunk, D]
    int NQ, NKV, G, S, nchunk;
    float scale;
};

// grid (ceil(S / kST), NKV): thread = one position of kv head blockIdx.y, all G q heads of that kv head.
template <int G>
__global__ __launch_bounds__(kST) void attn_scores(AttnArgs a) {
    const int g = blockIdx.y, tid = threadIdx.x;
    // q is the same for every lane: read with wave-uniform indices it comes in through scalar loads and feeds the
    // fma as a scalar operand (20.4 us per call at S = 4096 against 22.3 us with q staged in LDS)
    const uint32_t* qg = reinterpret_cast<const uint32_t*>(a.q + (size_t)g * G * kD);
    const int t = blockIdx.x * kST + tid;
    if (t >= a.S) return;
    const u32x4* kr = reinterpret_cast<const u32x4*>(a.k + ((size_t)t * a.NKV + g) * kD);
    u32x4 kk[kD / 8];
#pragma unroll
    for (int c = 0; c < kD / 8; ++c) kk[c] = __builtin_nontemporal_load(&kr[c]);
    float dot[G];  // products of bf16 values are exact in fp32, so fma = multiply-then-add here
#pragma unroll
    for (int h = 0; h < G; ++h) dot[h] = 0.f;
#pragma unroll
    for (int c = 0; c < kD / 8; ++c) {
        const uint32_t w4[4] = {kk[c].x, kk[c].y, kk[c].z, kk[c].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float k0 = __uint_as_float(w4[j] << 16), k1 = __uint_as_float(w4[j] & 0xFFFF0000u);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const uint32_t qq = qg[(h * kD + c * 8 + 2 * j) / 2];
                dot[h] = fmaf(__uint_as_float(qq << 16), k0, dot[h]);
                dot[h] = fmaf(__uint_as_float(qq & 0xFFFF0000u), k1, dot[h]);
            }
        }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) a.scores[(size_t)(g * G + h) * a.S + t] = bf2f(f2bf(bf2f(f2bf(dot[h])) * a.scale));
}

// grid (nchunk, NKV): the softmax statistics of the G heads over all S scores, then p for this chunk's positions
// and the chunk's partial sum of p * v (wave w takes positions 64w .. 64w + 63 of the chunk; lane l dims 2l, 2l + 1).
// Every loop issues its loads together before using them (indices clamped into range, so no load is
// conditional): the statistics cost two L2 round trips per 4096 positions, p one, and the V rows one.
constexpr int kSB = 16;  // scores per thread per head per statistics block (a block = 4096 positions)
template <int G>
__global__ __launch_bounds__(256) void attn_pv(AttnArgs a) {
    __shared__ float red[4][G];
    __shared__ float stat_m[G], stat_t[G];
    __shared__ float ps[G][kChunk];
    __shared__ float accs[4][G][kD];
    const int g = blockIdx.y, S = a.S, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int t0 = blockIdx.x * kChunk, n = min(kChunk, S - t0);
    const float* sc0 = a.scores + (size_t)g * G * S;
    float m[G], sum[G];
#pragma unroll
    for (int h = 0; h < G; ++h) m[h] = -INFINITY, sum[h] = 0.f;
    // the first block of scores stays in registers for the second pass (S <= 4096 reads the scores once)
    float v0[G][kSB];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int u = 0; u < kSB; ++u) {
            const int t = u * 256 + tid;
            const float x = sc0[(size_t)h * S + min(t, S - 1)];
            v0[h][u] = t < S ? x : -INFINITY;
            m[h] = fmaxf(m[h], v0[h][u]);
        }
    for (int b0 = 256 * kSB; b0 < S; b0 += 256 * kSB) {
        float v[G][kSB];
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int u = 0; u < kSB; ++u) {
                const int t = b0 + u * 256 + tid;
                const float x = sc0[(size_t)h * S + min(t, S - 1)];
                v[h][u] = t < S ? x : -INFINITY;
            }
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int u = 0; u < kSB; ++u) m[h] = fmaxf(m[h], v[h][u]);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
        for (int k = 32; k >= 1; k >>= 1) m[h] = fmaxf(m[h], __shfl_xor(m[h], k, 64));
        if (lane == 0) red[wv][h] = m[h];
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) m[h] = fmaxf(fmaxf(red[0][h], red[1][h]), fmaxf(red[2][h], red[3][h]));
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int u = 0; u < kSB; ++u)
            if (u * 256 + tid < S) sum[h] += expf(v0[h][u] - m[h]);
    for (int b0 = 256 * kSB; b0 < S; b0 += 256 * kSB) {
        float v[G][kSB];
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int u = 0; u < kSB; ++u) {
                const int t = b0 + u * 256 + tid;
                const float x = sc0[(size_t)h * S + min(t, S - 1)];
                v[h][u] = t < S ? x : -INFINITY;
            }
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int u = 0; u < kSB; ++u)
                if (b0 + u * 256 + tid < S) sum[h] += expf(v[h][u] - m[h]);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
        for (int k = 32; k >= 1; k >>= 1) sum[h] += __shfl_xor(sum[h], k, 64);
        if (lane == 0) red[wv][h] = sum[h];
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) {
        if (tid == h) {
            stat_m[h] = m[h];
            stat_t[h] = (red[0][h] + red[1][h]) + (red[2][h] + red[3][h]);
        }
    }
    __syncthreads();
    static_assert(kChunk % 64 == 0 && kChunk <= 256, "one p per thread of the first kChunk threads");
    if (tid < kChunk) {  // whole waves
        float sv[G];
#pragma unroll
        for (int h = 0; h < G; ++h) sv[h] = sc0[(size_t)h * S + t0 + min(tid, n - 1)];
#pragma unroll
        for (int h = 0; h < G; ++h)
            ps[h][tid] = tid < n ? bf2f(f2bf(expf(sv[h] - stat_m[h]) / stat_t[h])) : 0.f;
    }
    __syncthreads();
    constexpr int kPW = kChunk / 4;  // positions per wave
    uint32_t vv[kPW];
#pragma unroll
    for (int u = 0; u < kPW; ++u) {
        const int j = wv * kPW + u;
        vv[u] = *reinterpret_cast<const uint32_t*>(a.v + ((size_t)(t0 + min(j, n - 1)) * a.NKV + g) * kD + 2 * lane);
    }
    float acc[G][2];
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h][0] = acc[h][1] = 0.f;
#pragma unroll
    for (int u = 0; u < kPW; ++u) {
        const int j = wv * kPW + u;  // ps[h][j] = 0 for j >= n
        const float v0 = __uint_as_float(vv[u] << 16), v1 = __uint_as_float(vv[u] & 0xFFFF0000u);
#pragma unroll
        for (int h = 0; h < G; ++h) {
            acc[h][0] = fmaf(ps[h][j], v0, acc[h][0]);
            acc[h][1] = fmaf(ps[h][j], v1, acc[h][1]);
        }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
        accs[wv][h][2 * lane] = acc[h][0];
        accs[wv][h][2 * lane + 1] = acc[h][1];
    }
    __syncthreads();
    for (int i = tid; i < G * kD; i += 256) {
        const int h = i / kD, d = i % kD;
        const float s = (accs[0][h][d] + accs[1][h][d]) + (accs[2][h][d] + accs[3][h][d]);
        a.part[((size_t)(g * G + h) * a.nchunk + blockIdx.x) * kD + d] = s;
    }
}

// one thread per (q head, dim): the chunk partials summed in chunk order, rounded to bf16
__global__ __launch_bounds__(256) void attn_out(AttnArgs a) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.NQ * kD) return;
    const int h = i / kD, d = i % kD;
    float s = 0.f;
    const float* ph = a.part + (size_t)h * a.nchunk * kD + d;
    int c = 0;
    for (; c + 16 <= a.nchunk; c += 16) {  // 16 loads in flight, summed in chunk order
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = ph[(size_t)(c + u) * kD];
#pragma unroll
        for (int u = 0; u < 16; ++u) s += v[u];
    }
    for (; c < a.nchunk; ++c) s += ph[(size_t)c * kD];
    a.out[i] = (uint16_t)f2bf(s);
}

thread_local const char* t_err = "no error";

int afail(int code, const char* msg) {
    t_err = msg;
    return code;
}

}  // namespace

extern "C" {

size_t moe_attn_workspace_bytes(int n_q_heads, int head_dim, int S) {
    if (n_q_heads < 1 || head_dim != kD || S < 1) return 0;
    const size_t nchunk = (size_t)(S + kChunk - 1) / kChunk;
    return (size_t)n_q_heads * S * sizeof(float) + (size_t)n_q_heads * nchunk * kD * sizeof(float);
}

const char* moe_attn_last_error(void) { return t_err; }

}  // extern "C"

namespace {

// Checks the arguments and enqueues the three kernels with `workspace` (>= moe_attn_workspace_bytes bytes, device
// memory) as the scores / partials buffer.
int attn_launch(int n_q_heads, int n_kv_heads, int head_dim, int S, float scale, const uint16_t* q,
                const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out, void* workspace, size_t workspace_bytes,
                void* stream) {
    if (head_dim != kD) return afail(MOE_GPU_EINVAL, "head_dim must be 128");
    const int G = n_kv_heads >= 1 && n_q_heads % n_kv_heads == 0 ? n_q_heads / n_kv_heads : 0;
    if (G != 1 && G != 2 && G != 4 && G != 8)
        return afail(MOE_GPU_EINVAL, "need n_q_heads = G * n_kv_heads with G in {1, 2, 4, 8}");
    if (S < 1 || S > (1 << 24)) return afail(MOE_GPU_EINVAL, "S outside [1, 2^24]");
    if (!q || !k_cache || !v_cache || !out || !workspace) return afail(MOE_GPU_EINVAL, "null pointer");
    if (workspace_bytes < moe_attn_workspace_bytes(n_q_heads, head_dim, S))
        return afail(MOE_GPU_EINVAL, "workspace smaller than moe_attn_workspace_bytes()");
    if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 15)
        return afail(MOE_GPU_EINVAL, "k_cache / v_cache must be 16-byte aligned");
    const int nchunk = (S + kChunk - 1) / kChunk;
    float* scores = static_cast<float*>(workspace);
    AttnArgs a{q, k_cache, v_cache, out, scores, scores + (size_t)n_q_heads * S, n_q_heads, n_kv_heads,
               n_q_heads / n_kv_heads, S, nchunk, scale};
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 gs((S + kST - 1) / kST, n_kv_heads), gp(nchunk, n_kv_heads);
    switch (a.G) {
        case 1: hipLaunchKernelGGL(attn_scores<1>, gs, dim3(kST), 0, st, a); hipLaunchKernelGGL(attn_pv<1>, gp, dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL(attn_scores<2>, gs, dim3(kST), 0, st, a); hipLaunchKernelGGL(attn_pv<2>, gp, dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL(attn_scores<4>, gs, dim3(kST), 0, st, a); hipLaunchKernelGGL(attn_pv<4>, gp, dim3(256), 0, st, a); break;
        default: hipLaunchKernelGGL(attn_scores<8>, gs, dim3(kST), 0, st, a); hipLaunchKernelGGL(attn_pv<8>, gp, dim3(256), 0, st, a); break;
    }
    hipLaunchKernelGGL(attn_out, dim3((n_q_heads * kD + 255) / 256), dim3(256), 0, st, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return afail(e == hipErrorNoBinaryForGpu ? MOE_GPU_ENOKERNEL : MOE_GPU_EHIP, hipGetErrorString(e));
    return MOE_GPU_OK;
}

// The allocation-free entry point's scratch: the scores and partials of one call, for up to kScratchMaxNQ query
// heads and kScratchMaxS positions (4 MiB per GPU, held until the process ends).  Host code never uses the array's
// name as an address: the device address is looked up once per device (hipGetSymbolAddress, with that device
// current) and kept in g_scratch.
constexpr int kScratchMaxNQ = 64, kScratchMaxS = 8192;
constexpr size_t kScratchBytes =
    (size_t)kScratchMaxNQ * kScratchMaxS * sizeof(float) +
    (size_t)kScratchMaxNQ * ((kScratchMaxS + kChunk - 1) / kChunk) * kD * sizeof(float);
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];
constexpr int kMaxDevices = 64;
void* g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

int scratch_of_current_device(void** ptr) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return afail(MOE_GPU_EHIP, "hipGetDevice failed");
    if (dev < 0 || dev >= kMaxDevices) return afail(MOE_GPU_EINVAL, "device index beyond the scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return afail(e == hipErrorNoBinaryForGpu ? MOE_GPU_ENOKERNEL : MOE_GPU_EHIP,
                         "hipGetSymbolAddress(scratch) failed");
        g_scratch[dev] = p;
    }
    *ptr = g_scratch[dev];
    return MOE_GPU_OK;
}

}  // namespace

extern "C" {

int moe_attn_decode_dev(int n_q_heads, int n_kv_heads, int head_dim, int S, float scale, const uint16_t* q,
                        const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out, void* workspace,
                        size_t workspace_bytes, void* stream) {
    return attn_launch(n_q_heads, n_kv_heads, head_dim, S, scale, q, k_cache, v_cache, out, workspace, workspace_bytes,
                       stream);
}

size_t moe_attn_noalloc_max_bytes(void) { return kScratchBytes; }

int moe_attn_decode_noalloc_dev(int n_q_heads, int n_kv_heads, int head_dim, int S, float scale, const uint16_t* q,
                                const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out, void* stream) {
    const size_t need = moe_attn_workspace_bytes(n_q_heads, head_dim, S);
    if (need == 0) return afail(MOE_GPU_EINVAL, "bad n_q_heads / head_dim / S");
    if (need > kScratchBytes)
        return afail(MOE_GPU_EINVAL, "n_q_heads * S beyond the allocation-free scratch (moe_attn_noalloc_max_bytes)");
    void* ws = nullptr;
    const int rc = scratch_of_current_device(&ws);
    if (rc != MOE_GPU_OK) return rc;
    return attn_launch(n_q_heads, n_kv_heads, head_dim, S, scale, q, k_cache, v_cache, out, ws, kScratchBytes, stream);
}

}  // extern "C"
