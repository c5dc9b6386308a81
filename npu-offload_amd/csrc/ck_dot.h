// ck_dot.h — one wavefront's dot product of a bf16 weight row with staged bf16 tokens in the reference's ck_gemv
// order (track2_opt/solar_engine/csrc/cpu_kern.c:9-19, :31-35): the router unit of the fused layer kernel and the fp32
// GEMV (moe_gemv_f32_dev) both use it, so their results are bit-identical to the reference's ck_gemv.
//
// ck_gemv's dot product runs 32 fp32 lanes (two 16-lane vdpbf16ps accumulators over 64-element steps).  Chain c
// (c < 16: the first accumulator's lane c, else the second's lane c - 16) owns dword c of every 64-element step, i.e.
// elements (2c, 2c + 1) of each step, and adds their products one after the other, the odd element first, over the
// steps in order (a bf16 x bf16 product is exact in fp32, so each fused multiply-add equals the reference's add of the
// product).  The 32 chains then meet in an xor butterfly over 16, 8, 4, 2, 1: the pair sums acc0 + acc1 and then GCC's
// _mm512_reduce_add_ps tree (256-bit halves, 128-bit halves, (2,3,0,1), last pair) in that order.  The reference's
// vdpbf16ps flushes denormal inputs and results; this code does not, so the bits agree whenever no product or partial
// sum is a denormal fp32 number.
//
// The row is loaded 16 bytes per lane (lane l holds chunks l + 64 j: one wave load reads 1 KiB of the row), every load
// of a 4096-element batch in flight at once; each 1 KiB segment (8 steps) then passes through the wave's own 1 KiB of
// shared memory, from which lane c (and c + 32, a duplicate) reads its chain's dwords.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

namespace ckdot {
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4u lds_v4u;
typedef __attribute__((address_space(3))) unsigned lds_u32;
__device__ __forceinline__ float lo(unsigned v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float hi(unsigned v) { return __uint_as_float(v & 0xFFFF0000u); }
}  // namespace ckdot

// acc[t] (t < NT) = row . x_t in ck_gemv's order, for the wave's row `row` (H elements, H % 512 == 0), tokens staged in
// shared memory as dwords (token t's element pair (2k, 2k+1) at xd[t * H/2 + k]; columns t >= T read token 0).  seg:
// the wave's 1 KiB shared-memory segment buffer.  after_issue() runs once the first batch's loads are in flight (a
// caller stages the tokens there).  Every lane returns the result.
template <int NT, typename AfterIssue>
__device__ __forceinline__ void ck_row_dot(const ckdot::v4u* __restrict__ row, int H, int T, ckdot::lds_v4u* seg,
                                           const ckdot::lds_u32* xd, float* acc, AfterIssue after_issue) {
    using namespace ckdot;
    const int lane = threadIdx.x & 63, c = lane & 31;
    const int nj = H / 512, hd = H / 2;  // 1 KiB segments; dwords per token row
    const lds_u32* segd = (const lds_u32*)seg + c;
    const lds_u32* xc = xd + c;
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.f;
    v4u w[8];
#pragma unroll
    for (int j = 0; j < 8; j++)
        if (j < nj) w[j] = row[lane + 64 * j];
    after_issue();
#pragma unroll 1
    for (int j0 = 0; j0 < nj; j0 += 8) {
        if (j0 > 0) {
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (j0 + j < nj) w[j] = row[lane + 64 * (j0 + j)];
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (j0 + j < nj) {
                seg[lane] = w[j];  // segment j0 + j: 64-element steps 8 (j0 + j) .. 8 (j0 + j) + 7
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int bb = 0; bb < 8; bb++) {
                    const unsigned wv = segd[32 * bb];
                    const float w0 = lo(wv), w1 = hi(wv);
                    const int b = 8 * (j0 + j) + bb;
#pragma unroll
                    for (int t = 0; t < NT; t++) {  // no per-token branch: the reads of a step stay in flight together
                        const unsigned xv = xc[(t < T ? t : 0) * hd + 32 * b];
                        acc[t] = fmaf(w1, hi(xv), acc[t]);
                        acc[t] = fmaf(w0, lo(xv), acc[t]);
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
        }
    }
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) {
#pragma unroll
        for (int t = 0; t < NT; t++) acc[t] = acc[t] + __shfl_xor(acc[t], m, 64);
    }
}

}  // namespace moe
