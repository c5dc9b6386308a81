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

#include <type_traits>

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

// The router table in chain order: row e's dword k = 32 s + c (step s, chain c) sits at dword
// 4 (32 (s / 4) + c) + s % 4 of the row, so that chain c's dwords of four consecutive steps form one 16-byte chunk and
// a lane loads exactly its chain's operands, in step order.  H % 512 == 0.
__host__ __device__ __forceinline__ size_t ck_chain_dword(int H, int e, int k) {
    const int s = k >> 5, c = k & 31;
    return (size_t)e * (H / 2) + 4 * (32 * (s >> 2) + c) + (s & 3);
}

// Two rows per wavefront from the chain-ordered table: lanes 0-31 run row `row0`'s 32 chains, lanes 32-63 row
// `row1`'s (each a row base in u32x4 units), with the tokens read from shared memory as dwords (xd as in ck_row_dot).
// The same order as ck_row_dot, without passing the weights through shared memory: chain c's 16-byte chunk q holds
// its dwords of steps 4q .. 4q + 3.  Lanes 0 and 32 return their row's results.
namespace ckdot {
typedef __attribute__((address_space(3))) float lds_f32;
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2f lds_v2f;

// One token in fp32 (xf: element 2k + j of the token at xf[2k + j]): chunks q0 .. q0 + N - 1 of a lane's chain, the
// element pairs of 8 chunks read together (one 8-byte read per step), no conversions of the token.
template <int N>
__device__ __forceinline__ void chain_consume_f32(const v4u* w, int q0, const lds_v2f* xfc, float& acc) {
    constexpr int G = 8 < N ? 8 : N;
    static_assert(N % G == 0, "chunk groups");
#pragma unroll
    for (int g = 0; g < N; g += G) {
        v2f xv[G * 4];
#pragma unroll
        for (int u = 0; u < G; u++)
#pragma unroll
            for (int i = 0; i < 4; i++) xv[4 * u + i] = xfc[32 * (4 * (q0 + g + u) + i)];
#pragma unroll
        for (int u = 0; u < G; u++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const unsigned wv = w[g + u][i];
                acc = fmaf(hi(wv), xv[4 * u + i].y, acc);
                acc = fmaf(lo(wv), xv[4 * u + i].x, acc);
            }
        }
    }
}

// Chunks q0 .. q0 + N - 1 of a lane's chain (N a compile-time count, no branches): the token dwords of XG chunks
// (4 XG steps x NT tokens, at most 32) are read from shared memory together, then consumed in step order.
template <int NT, int N>
__device__ __forceinline__ void chain_consume(const v4u* w, int q0, int T, int hd, const lds_u32* xc, float* acc) {
    constexpr int XG = NT >= 8 ? 1 : NT >= 4 ? 2 : NT >= 2 ? 4 : 8;
    constexpr int G = XG < N ? XG : N;
    static_assert(N % G == 0, "chunk groups");
#pragma unroll
    for (int g = 0; g < N; g += G) {
        unsigned xv[G * 4][NT];
#pragma unroll
        for (int u = 0; u < G; u++)
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int t = 0; t < NT; t++) xv[4 * u + i][t] = xc[(t < T ? t : 0) * hd + 32 * (4 * (q0 + g + u) + i)];
#pragma unroll
        for (int u = 0; u < G; u++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const unsigned wv = w[g + u][i];
                const float w0 = lo(wv), w1 = hi(wv);
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    acc[t] = fmaf(w1, hi(xv[4 * u + i][t]), acc[t]);
                    acc[t] = fmaf(w0, lo(xv[4 * u + i][t]), acc[t]);
                }
            }
        }
    }
}
}  // namespace ckdot

// H = 256 * QN (QN = 8 or 16): every load of the row issued at once, the rest without branches.  Other H (a multiple
// of 512): two chunks per round trip.  xf (NT = 1 only, may be null): the token also staged in fp32, which saves the
// token's conversions (the products and sums are the same).
template <int NT, typename AfterIssue>
__device__ __forceinline__ void ck_rows_dot_chain(const ckdot::v4u* __restrict__ row0, const ckdot::v4u* __restrict__ row1,
                                                  int H, int T, const ckdot::lds_u32* xd, const ckdot::lds_f32* xf,
                                                  float* acc, AfterIssue after_issue) {
    using namespace ckdot;
    const int lane = threadIdx.x & 63, c = lane & 31;
    const int nq = H / 256, hd = H / 2;
    const v4u* p = (lane < 32 ? row0 : row1) + c;
    const lds_u32* xc = xd + c;
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.f;
    auto fixed = [&](auto qn) __attribute__((always_inline)) {
        constexpr int QN = decltype(qn)::value;
        v4u w[QN];
#pragma unroll
        for (int q = 0; q < QN; q++) w[q] = __builtin_nontemporal_load(p + 32 * q);
        after_issue();
        if (NT == 1 && xf) chain_consume_f32<QN>(w, 0, (const lds_v2f*)xf + c, acc[0]);
        else chain_consume<NT, QN>(w, 0, T, hd, xc, acc);
    };
    if (nq == 16) {
        fixed(std::integral_constant<int, 16>());
    } else if (nq == 8) {
        fixed(std::integral_constant<int, 8>());
    } else {
        v4u w[2];
#pragma unroll 1
        for (int q0 = 0; q0 < nq; q0 += 2) {
            w[0] = __builtin_nontemporal_load(p + 32 * q0);
            w[1] = __builtin_nontemporal_load(p + 32 * (q0 + 1));
            if (q0 == 0) after_issue();
            chain_consume<NT, 2>(w, q0, T, hd, xc, acc);
        }
    }
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) {
#pragma unroll
        for (int t = 0; t < NT; t++) acc[t] = acc[t] + __shfl_xor(acc[t], m, 64);
    }
}

}  // namespace moe
