// dense_ops.hip — the attention block's dense steps of a decode step (include/moe_gpu.h, moe_gemv_dev /
// moe_rope_dev), replacing the host layer's projections and rotary embedding (track2_opt/solar_engine/src/
// main.rs:109-113 and :119: gemv(q/k/v/o_proj) followed by round_bf; main.rs:65-77: rope).
#include <hip/hip_runtime.h>

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
template <int RB, int CG>
__global__ __launch_bounds__(256) void gemv_kernel(const uint16_t* __restrict__ W, const uint16_t* __restrict__ x,
                                                   uint16_t* __restrict__ y, int M, int K) {
    extern __shared__ __align__(16) uint16_t xs[];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    for (int i = tid * 8; i < K; i += 256 * 8)
        *reinterpret_cast<u32x4*>(&xs[i]) = *reinterpret_cast<const u32x4*>(&x[i]);
    __syncthreads();
    const int nch = K / 512;
    const int gw = blockIdx.x * kWaves + wv, nw = gridDim.x * kWaves;
    u32x4 wq[RB][CG];
    float acc[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) acc[r] = 0.f;
    auto load_group = [&](int r0_, int c0_) {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int row = r0_ + r < M ? r0_ + r : M - 1;  // rows past M re-read the last row; discarded below
            const u32x4* wr = reinterpret_cast<const u32x4*>(W + (size_t)row * K);
#pragma unroll
            for (int c = 0; c < CG; ++c) wq[r][c] = __builtin_nontemporal_load(&wr[(c0_ + c) * 64 + lane]);
        }
    };
    int r0 = gw * RB, c0 = 0;
    if (r0 < M) load_group(r0, 0);
    while (r0 < M) {
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
        int nr0 = r0, nc0 = c0 + CG;
        if (nc0 >= nch) {
            nc0 = 0;
            nr0 = r0 + nw * RB;
        }
        if (nr0 < M) load_group(nr0, nc0);
        if (nc0 == 0) {
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const float tot = wave_sum(acc[r]);
                acc[r] = 0.f;
                if (lane == r && r0 + r < M) y[r0 + r] = (uint16_t)f2bf(tot);
            }
        }
        r0 = nr0;
        c0 = nc0;
    }
}

// One workgroup per head, in place (main.rs:65-77): rot[i] = -x[i + D/2] for i < D/2, x[i - D/2] otherwise;
// x[i] = bf16(bf16(x[i] * cos[i]) + bf16(rot[i] * sin[i])).  The head is staged in LDS first.
__global__ __launch_bounds__(256) void rope_kernel(uint16_t* x, const uint16_t* cs, const uint16_t* sn, int D) {
    __shared__ float old[1024];
    uint16_t* xh = x + (size_t)blockIdx.x * D;
    for (int i = threadIdx.x; i < D; i += blockDim.x) old[i] = bf2f(xh[i]);
    __syncthreads();
    const int half = D / 2;
    for (int i = threadIdx.x; i < D; i += blockDim.x) {
        const float rot = i < half ? -old[i + half] : old[i - half];
        const float a = bf2f(f2bf(old[i] * bf2f(cs[i])));
        const float b = bf2f(f2bf(rot * bf2f(sn[i])));
        xh[i] = (uint16_t)f2bf(a + b);
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
    int wgs = 0;
    for (int i = 0; i < n_cache; ++i)
        if (cache[i].dev == dev && cache[i].fn == fn && cache[i].lds == lds) wgs = cache[i].wgs;
    if (wgs == 0) {
        int ncu = 0, per_cu = 0;
        if (lds > 64 * 1024 && hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
            return MOE_GPU_EHIP;
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

template <int RB, int CG>
int gemv_launch(const uint16_t* W, const uint16_t* x, uint16_t* y, int M, int K, hipStream_t st) {
    const void* fn = reinterpret_cast<const void*>(&gemv_kernel<RB, CG>);
    const size_t lds = (size_t)K * sizeof(uint16_t);
    int grid = 0, rc = gemv_grid(fn, lds, M, RB, &grid);
    if (rc != MOE_GPU_OK) return rc;
    hipLaunchKernelGGL((gemv_kernel<RB, CG>), dim3(grid), dim3(256), lds, st, W, x, y, M, K);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? MOE_GPU_OK : e == hipErrorNoBinaryForGpu ? MOE_GPU_ENOKERNEL : MOE_GPU_EHIP;
}

}  // namespace

extern "C" {

int moe_gemv_dev(int M, int K, const uint16_t* W, const uint16_t* x, uint16_t* y, void* stream) {
    if (M < 1 || K < 1024 || K % 1024 != 0 || K > 65536 || !W || !x || !y) return MOE_GPU_EINVAL;
    if ((reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(x)) & 15) return MOE_GPU_EINVAL;
    hipStream_t st = static_cast<hipStream_t>(stream);
    // whole 4096-column rows when K allows; 4 rows per wave step for tall W, 1 row for short W (1024 rows x 4 is a
    // quarter of the waves the chip holds)
    if (K % 4096 == 0) return M >= 4096 ? gemv_launch<4, 8>(W, x, y, M, K, st) : gemv_launch<1, 8>(W, x, y, M, K, st);
    return gemv_launch<8, 2>(W, x, y, M, K, st);
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
