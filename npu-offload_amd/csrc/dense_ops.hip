// dense_ops.hip — the attention block's dense steps of a decode step (include/moe_gpu.h, moe_gemv_dev /
// moe_rope_dev), replacing the host layer's projections and rotary embedding (track2_opt/solar_engine/src/
// main.rs:109-113 and :119: gemv(q/k/v/o_proj) followed by round_bf; main.rs:65-77: rope).
#include <hip/hip_runtime.h>

#include "ck_dot.h"
#include "launch_util.h"
#include "moe_gpu.h"

namespace {

constexpr int kWaves = 4;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ uint32_t f2bf(float f) {  // round to nearest even (host.rs:41-46)
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// y[m] = bf16(sum_k W[m, k] x[k]) for one token: x staged in LDS; waves take steps of RB whole rows, CG 16-byte
// chunks per lane per load group, the next group's loads issued before the step's butterfly (the LM head's scheme).
// The first group's weight loads are issued before x is staged, so the staging round trip overlaps them.
// norm_w != null: x is the residual stream and the GEMV reads rmsnorm(x, norm_w) (host.rs:71-76: ms = sum(x^2) / K in
// fp32, r = 1 / sqrt(ms + eps), h = bf16(bf16(x * r) * w)), which every workgroup computes into LDS (each thread's
// 16-byte chunks of x and of the weight loaded at once; the squares summed per thread over its chunks in order, then a
// 64-lane butterfly, then the 4 wavefronts in order): the layer's input norm folded into its q|k|v projection.
constexpr int kXC = 4;  // 16-byte chunks of x per thread per staging pass (one pass for K <= 8192)

// ROPE (the q|k|v projection with RoPE and the KV append in its epilogue, main.rs:109-118): y = qkv rows of 128-wide
// heads [q (NQ) | k (NKV) | v (NKV)]; wave step s takes rows (h = s / 32, p = s % 32) 128 h + 2p, + 1, + 64, + 65, i.e.
// two element pairs that RoPE rotates into each other, so the step's four sums give four roped outputs: q heads go to
// y, k heads to the key cache row of pos, v heads (not rotated) to the value cache row.  The sums, the roundings and
// RoPE's arithmetic are those of the plain GEMV followed by rope_append_kernel, so the bits are the same.
struct RopeArgs {
    const uint16_t* cs;  // cos row of pos [128]
    const uint16_t* sn;  // sin row of pos [128]
    uint16_t* kc;        // key cache row of pos [NKV, 128]
    uint16_t* vc;        // value cache row of pos [NKV, 128]
    int NQ, NKV;
};
template <bool ROPE, int RB>
__device__ __forceinline__ int step_row(int s, int r) {  // row r of wave step s
    if (!ROPE) return s * RB + r;
    return (s >> 5) * 128 + 2 * (s & 31) + (r & 1) + ((r >> 1) << 6);
}

template <int RB, int CG, bool ROPE = false>
__global__ __launch_bounds__(256) void gemv_kernel(const uint16_t* __restrict__ W, const uint16_t* __restrict__ x,
                                                   uint16_t* __restrict__ y, int M, int K,
                                                   const uint16_t* __restrict__ norm_w, float eps, RopeArgs ra) {
    static_assert(!ROPE || RB == 4, "RoPE steps take 4 rows");
    extern __shared__ __align__(16) uint16_t xs[];
    __shared__ float red[kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nch = K / 512;
    const int gw = blockIdx.x * kWaves + wv, nw = gridDim.x * kWaves;
    u32x4 wq[RB][CG];
    float acc[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) acc[r] = 0.f;
    const int nsteps = (M + RB - 1) / RB;
    auto load_group = [&](int s_, int c0_) {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            int row = step_row<ROPE, RB>(s_, r);
            row = row < M ? row : M - 1;  // rows past M re-read the last row; discarded below
            const u32x4* wr = reinterpret_cast<const u32x4*>(W + (size_t)row * K);
#pragma unroll
            for (int c = 0; c < CG; ++c) wq[r][c] = __builtin_nontemporal_load(&wr[(c0_ + c) * 64 + lane]);
        }
    };
    int st = gw, c0 = 0;  // wave step, chunk group
    if (st < nsteps) load_group(st, 0);
    // stage x (normalised when norm_w): thread tid holds 16-byte chunks tid + 256 j
    const int nc = K / 8;
    const u32x4* x4 = reinterpret_cast<const u32x4*>(x);
    const u32x4* w4 = reinterpret_cast<const u32x4*>(norm_w);
    float rs = 1.f;
    if (norm_w) {
        float s = 0.f;
        for (int j0 = 0; j0 < nc; j0 += 256 * kXC) {
            u32x4 xv[kXC];
#pragma unroll
            for (int j = 0; j < kXC; ++j)
                if (j0 + 256 * j + tid < nc) xv[j] = x4[j0 + 256 * j + tid];
#pragma unroll
            for (int j = 0; j < kXC; ++j) {
                if (j0 + 256 * j + tid < nc) {
                    const uint32_t e4[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float lo = bf2f(e4[i] & 0xFFFFu), hi = bf2f(e4[i] >> 16);
                        s = fmaf(lo, lo, s);
                        s = fmaf(hi, hi, s);
                    }
                }
            }
        }
        s = wave_sum(s);
        if (lane == 0) red[wv] = s;
        __syncthreads();
        const float ms = (((red[0] + red[1]) + red[2]) + red[3]) / (float)K;
        rs = 1.0f / sqrtf(ms + eps);
    }
    for (int j0 = 0; j0 < nc; j0 += 256 * kXC) {
        u32x4 xv[kXC], nv[kXC];
#pragma unroll
        for (int j = 0; j < kXC; ++j) {
            if (j0 + 256 * j + tid < nc) {
                xv[j] = x4[j0 + 256 * j + tid];
                if (norm_w) nv[j] = w4[j0 + 256 * j + tid];
            }
        }
#pragma unroll
        for (int j = 0; j < kXC; ++j) {
            const int c = j0 + 256 * j + tid;
            if (c < nc) {
                u32x4 o = xv[j];
                if (norm_w) {
                    const uint32_t e4[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
                    const uint32_t n4[4] = {nv[j].x, nv[j].y, nv[j].z, nv[j].w};
                    uint32_t r4[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t lo = f2bf(bf2f(f2bf(bf2f(e4[i] & 0xFFFFu) * rs)) * bf2f(n4[i] & 0xFFFFu));
                        const uint32_t hi = f2bf(bf2f(f2bf(bf2f(e4[i] >> 16) * rs)) * bf2f(n4[i] >> 16));
                        r4[i] = lo | (hi << 16);
                    }
                    o = u32x4{r4[0], r4[1], r4[2], r4[3]};
                }
                *reinterpret_cast<u32x4*>(&xs[8 * c]) = o;
            }
        }
    }
    __syncthreads();
    while (st < nsteps) {
#pragma unroll
        for (int c = 0; c < CG; ++c) {
            const u32x4 h4 = *reinterpret_cast<const u32x4*>(&xs[((c0 + c) * 64 + lane) * 8]);
            const uint32_t hw[4] = {h4.x, h4.y, h4.z, h4.w};
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const uint32_t ww[4] = {wq[r][c].x, wq[r][c].y, wq[r][c].z, wq[r][c].w};
                float s = acc[r];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    s = fmaf(__uint_as_float(ww[j] << 16), __uint_as_float(hw[j] << 16), s);
                    s = fmaf(__uint_as_float(ww[j] & 0xFFFF0000u), __uint_as_float(hw[j] & 0xFFFF0000u), s);
                }
                acc[r] = s;
            }
        }
        int nst = st, nc0 = c0 + CG;
        if (nc0 >= nch) {
            nc0 = 0;
            nst = st + nw;
        }
        if (nst < nsteps) load_group(nst, nc0);
        if (nc0 == 0) {
            if constexpr (!ROPE) {
#pragma unroll
                for (int r = 0; r < RB; ++r) {
                    const float tot = wave_sum(acc[r]);
                    acc[r] = 0.f;
                    if (lane == r && st * RB + r < M) y[st * RB + r] = (uint16_t)f2bf(tot);
                }
            } else {
                float xb[4];  // the four rows' bf16 results: rows i, i + 1 (first half) and i + 64, i + 65
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    xb[r] = bf2f(f2bf(wave_sum(acc[r])));
                    acc[r] = 0.f;
                }
                const int h = st >> 5, i = 2 * (st & 31);
                if (lane < 4) {
                    const int r = lane, e = i + (r & 1) + ((r >> 1) << 6);  // this lane's element of the head
                    const float own = xb[r];
                    uint16_t out;
                    if (h < ra.NQ + ra.NKV) {  // q or k: rot = -x[e + 64] for e < 64, x[e - 64] above
                        const float rot = r < 2 ? -xb[r + 2] : xb[r - 2];
                        const float av = bf2f(f2bf(own * bf2f(ra.cs[e])));
                        const float bv = bf2f(f2bf(rot * bf2f(ra.sn[e])));
                        out = (uint16_t)f2bf(av + bv);
                    } else {
                        out = (uint16_t)f2bf(own);
                    }
                    if (h < ra.NQ) y[(size_t)h * 128 + e] = out;
                    else if (h < ra.NQ + ra.NKV) ra.kc[(size_t)(h - ra.NQ) * 128 + e] = out;
                    else ra.vc[(size_t)(h - ra.NQ - ra.NKV) * 128 + e] = out;
                }
            }
        }
        st = nst;
        c0 = nc0;
    }
}

// fp32 GEMV in the reference's ck_gemv order (ck_row_dot): y[m] = W[m] . x, bit-identical to ck_gemv (cpu_kern.c:31-35)
// whenever no product or partial sum is a denormal.  Each wave takes one row per step, grid-strided; x is staged into
// shared memory once per workgroup, after the first rows' loads are in flight.  LDS: K * 2 bytes of x, then the four
// waves' 1 KiB segment buffers.
__global__ __launch_bounds__(256) void gemv_ck_kernel(const uint16_t* __restrict__ W, const uint16_t* __restrict__ x,
                                                      float* __restrict__ y, int M, int K) {
    extern __shared__ __align__(16) uint16_t xs[];
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    moe::ckdot::lds_v4u* seg = (moe::ckdot::lds_v4u*)(xs + K) + wv * 64;
    bool first = true;
    for (int r0 = blockIdx.x * kWaves; r0 < M; r0 += gridDim.x * kWaves) {  // the same trip count in every wave
        const int row = r0 + wv < M ? r0 + wv : M - 1;
        float acc[1];
        moe::ck_row_dot<1>(reinterpret_cast<const moe::ckdot::v4u*>(W + (size_t)row * K), K, 1, seg,
                           (const moe::ckdot::lds_u32*)xs, acc, [&]() __attribute__((always_inline)) {
                               if (first) {
                                   for (int i = tid * 8; i < K; i += 256 * 8)
                                       *reinterpret_cast<u32x4*>(&xs[i]) = *reinterpret_cast<const u32x4*>(&x[i]);
                                   __syncthreads();
                               }
                           });
        first = false;
        if (lane == 0 && r0 + wv < M) y[r0 + wv] = acc[0];
    }
}

// One workgroup per head, in place (main.rs:65-77): rot[i] = -x[i + D/2] for i < D/2, x[i - D/2] otherwise;
// x[i] = bf16(bf16(x[i] * cos[i]) + bf16(rot[i] * sin[i])).  The head is staged in LDS first.
__device__ __forceinline__ void rope_head(const uint16_t* src, uint16_t* dst, const uint16_t* cs, const uint16_t* sn,
                                          int D, float* old) {
    for (int i = threadIdx.x; i < D; i += blockDim.x) old[i] = bf2f(src[i]);
    __syncthreads();
    const int half = D / 2;
    for (int i = threadIdx.x; i < D; i += blockDim.x) {
        const float rot = i < half ? -old[i + half] : old[i - half];
        const float a = bf2f(f2bf(old[i] * bf2f(cs[i])));
        const float b = bf2f(f2bf(rot * bf2f(sn[i])));
        dst[i] = (uint16_t)f2bf(a + b);
    }
}

__global__ __launch_bounds__(256) void rope_kernel(uint16_t* x, const uint16_t* cs, const uint16_t* sn, int D) {
    __shared__ float old[1024];
    uint16_t* xh = x + (size_t)blockIdx.x * D;
    rope_head(xh, xh, cs, sn, D, old);
}

// The attention block's step between the q|k|v projection and attention (main.rs:112-118), one launch: workgroup h <
// NQ ropes q head h in place; NQ <= h < NQ + NKV ropes k head h - NQ into the key cache row of position pos;
// the last NKV workgroups copy the v heads into the value cache row.  qkv = [q (NQ*D) | k (NKV*D) | v (NKV*D)].
__global__ __launch_bounds__(256) void rope_append_kernel(uint16_t* qkv, const uint16_t* cs, const uint16_t* sn,
                                                          uint16_t* kc, uint16_t* vc, int NQ, int NKV, int D, int pos) {
    __shared__ float old[1024];
    const int h = blockIdx.x;
    const size_t row = (size_t)pos * NKV * D;
    if (h < NQ) {
        uint16_t* xh = qkv + (size_t)h * D;
        rope_head(xh, xh, cs, sn, D, old);
    } else if (h < NQ + NKV) {
        const int g = h - NQ;
        rope_head(qkv + (size_t)(NQ + g) * D, kc + row + (size_t)g * D, cs, sn, D, old);
    } else {
        const int g = h - NQ - NKV;
        const uint16_t* src = qkv + (size_t)(NQ + NKV + g) * D;
        for (int i = threadIdx.x; i < D; i += blockDim.x) vc[row + (size_t)g * D + i] = src[i];
    }
}

// Resident workgroups per (device, kernel, LDS size), queried once per thread: a launch stays one host call.
int gemv_grid(const void* fn, size_t lds, int M, int RB, int* grid) {
    struct Entry {
        int dev;
        const void* fn;
        size_t lds;
        int wgs;
    };
    static thread_local Entry cache[8];
    static thread_local int n_cache = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return MOE_GPU_EHIP;
    // every launch checks the process-wide LDS limit (raised only, never lowered), independent of the occupancy cache
    if (moe::raise_lds_limit(fn, lds) != hipSuccess) return MOE_GPU_EHIP;
    int wgs = 0;
    for (int i = 0; i < n_cache; ++i)
        if (cache[i].dev == dev && cache[i].fn == fn && cache[i].lds == lds) wgs = cache[i].wgs;
    if (wgs == 0) {
        int ncu = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return MOE_GPU_EHIP;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, lds) != hipSuccess) return MOE_GPU_EHIP;
        if (per_cu < 1) return MOE_GPU_EINVAL;
        wgs = ncu * per_cu;
        cache[n_cache < 8 ? n_cache++ : 7] = Entry{dev, fn, lds, wgs};
    }
    const int need = ((M + RB - 1) / RB + kWaves - 1) / kWaves;
    *grid = wgs < need ? wgs : need;
    return MOE_GPU_OK;
}

template <int RB, int CG, bool ROPE = false>
int gemv_launch(const uint16_t* W, const uint16_t* x, uint16_t* y, int M, int K, const uint16_t* norm_w, float eps,
                hipStream_t st, RopeArgs ra = RopeArgs{}) {
    const void* fn = reinterpret_cast<const void*>(&gemv_kernel<RB, CG, ROPE>);
    const size_t lds = (size_t)K * sizeof(uint16_t);
    int grid = 0, rc = gemv_grid(fn, lds, M, RB, &grid);
    if (rc != MOE_GPU_OK) return rc;
    hipLaunchKernelGGL((gemv_kernel<RB, CG, ROPE>), dim3(grid), dim3(256), lds, st, W, x, y, M, K, norm_w, eps, ra);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? MOE_GPU_OK : e == hipErrorNoBinaryForGpu ? MOE_GPU_ENOKERNEL : MOE_GPU_EHIP;
}

}  // namespace

extern "C" {

static int gemv_any(int M, int K, const uint16_t* W, const uint16_t* x, uint16_t* y, const uint16_t* norm_w, float eps,
                    void* stream) {
    if (M < 1 || K < 1024 || K % 1024 != 0 || K > 65536 || !W || !x || !y) return MOE_GPU_EINVAL;
    if ((reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(x)) & 15) return MOE_GPU_EINVAL;
    hipStream_t st = static_cast<hipStream_t>(stream);
    // whole 4096-column rows when K allows; 4 rows per wave step for tall W, 1 row for short W (1024 rows x 4 is a
    // quarter of the waves the chip holds)
    if (K % 4096 == 0)
        return M >= 4096 ? gemv_launch<4, 8>(W, x, y, M, K, norm_w, eps, st) : gemv_launch<1, 8>(W, x, y, M, K, norm_w, eps, st);
    return gemv_launch<8, 2>(W, x, y, M, K, norm_w, eps, st);
}

int moe_gemv_dev(int M, int K, const uint16_t* W, const uint16_t* x, uint16_t* y, void* stream) {
    return gemv_any(M, K, W, x, y, nullptr, 0.f, stream);
}

int moe_gemv_f32_dev(int M, int K, const uint16_t* W, const uint16_t* x, float* y, void* stream) {
    if (M < 1 || K < 512 || K % 512 != 0 || K > 65536 || !W || !x || !y) return MOE_GPU_EINVAL;
    if ((reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(x)) & 15) return MOE_GPU_EINVAL;
    const void* fn = reinterpret_cast<const void*>(&gemv_ck_kernel);
    const size_t lds = (size_t)K * 2 + (size_t)kWaves * 1024;
    int grid = 0, rc = gemv_grid(fn, lds, M, 1, &grid);
    if (rc != MOE_GPU_OK) return rc;
    hipLaunchKernelGGL(gemv_ck_kernel, dim3(grid), dim3(256), lds, static_cast<hipStream_t>(stream), W, x, y, M, K);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? MOE_GPU_OK : e == hipErrorNoBinaryForGpu ? MOE_GPU_ENOKERNEL : MOE_GPU_EHIP;
}

int moe_gemv_norm_dev(int M, int K, const uint16_t* W, const uint16_t* x, const uint16_t* norm_w, float eps,
                      uint16_t* y, void* stream) {
    if (!norm_w || !(eps >= 0.f)) return MOE_GPU_EINVAL;
    return gemv_any(M, K, W, x, y, norm_w, eps, stream);
}

int moe_rope_append_dev(int n_q_heads, int n_kv_heads, int head_dim, uint16_t* qkv, const uint16_t* cos_row,
                        const uint16_t* sin_row, uint16_t* k_cache, uint16_t* v_cache, int pos, void* stream) {
    if (n_q_heads < 1 || n_kv_heads < 1 || head_dim < 2 || head_dim % 2 != 0 || head_dim > 1024 || pos < 0 || !qkv ||
        !cos_row || !sin_row || !k_cache || !v_cache)
        return MOE_GPU_EINVAL;
    hipLaunchKernelGGL(rope_append_kernel, dim3(n_q_heads + 2 * n_kv_heads), dim3(head_dim < 256 ? head_dim : 256), 0,
                       static_cast<hipStream_t>(stream), qkv, cos_row, sin_row, k_cache, v_cache, n_q_heads,
                       n_kv_heads, head_dim, pos);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? MOE_GPU_OK : e == hipErrorNoBinaryForGpu ? MOE_GPU_ENOKERNEL : MOE_GPU_EHIP;
}

int moe_qkv_rope_append_dev(int H, int n_q_heads, int n_kv_heads, int head_dim, const uint16_t* W, const uint16_t* x,
                            const uint16_t* norm_w, float eps, const uint16_t* cos_row, const uint16_t* sin_row,
                            uint16_t* q, uint16_t* k_cache, uint16_t* v_cache, int pos, void* stream) {
    if (H < 4096 || H % 4096 != 0 || H > 65536 || n_q_heads < 1 || n_kv_heads < 1 || head_dim != 128 || pos < 0 ||
        !W || !x || !cos_row || !sin_row || !q || !k_cache || !v_cache || (norm_w && !(eps >= 0.f)))
        return MOE_GPU_EINVAL;
    if ((reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(x)) & 15) return MOE_GPU_EINVAL;
    const size_t row = (size_t)pos * n_kv_heads * 128;
    const RopeArgs ra{cos_row, sin_row, k_cache + row, v_cache + row, n_q_heads, n_kv_heads};
    // half-row load groups (4 rows x 4 KiB per wave, the next group issued before the sums): at Solar's q|k|v
    // (6144 x 4096, one wave step per wave) 12.1 us against 14.5 us with whole rows, whose 32 KiB per wave in flight
    // at once slow the HBM down (the same summation order, so the same bits)
    return gemv_launch<4, 4, true>(W, x, q, (n_q_heads + 2 * n_kv_heads) * 128, H, norm_w, eps,
                                   static_cast<hipStream_t>(stream), ra);
}

int moe_rope_dev(int n_heads, int head_dim, uint16_t* x, const uint16_t* cos_row, const uint16_t* sin_row,
                 void* stream) {
    if (n_heads < 1 || head_dim < 2 || head_dim % 2 != 0 || head_dim > 1024 || !x || !cos_row || !sin_row)
        return MOE_GPU_EINVAL;
    hipLaunchKernelGGL(rope_kernel, dim3(n_heads), dim3(head_dim < 256 ? head_dim : 256), 0,
                       static_cast<hipStream_t>(stream), x, cos_row, sin_row, head_dim);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? MOE_GPU_OK : e == hipErrorNoBinaryForGpu ? MOE_GPU_ENOKERNEL : MOE_GPU_EHIP;
}

}  // extern "C"
