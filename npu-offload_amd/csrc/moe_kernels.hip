// moe_kernels.hip — gfx950 kernels of the routed-MoE data plane: router GEMV, softmax top-k + expert grouping,
// grouped SwiGLU experts (gate|up + SiLU*mul, down), fixed-order combine; one-time relayout / quantise / synthetic
// fill kernels.
//
// Decode-time expert GEMVs are HBM-bound (1 flop per weight byte at batch 1), so everything is organised around
// streaming weights.  Each weight matrix lives in a 64-row tiled layout in which one 16-byte chunk of each of 64
// consecutive rows is contiguous: a wavefront load instruction reads 1 KB of contiguous HBM and lane l owns row l.
// Each wavefront keeps 8-16 such loads in flight (a rolling software pipeline), activations are staged once per
// workgroup in LDS and read as broadcasts, and the K range of a tile is split over the 4 wavefronts of a workgroup
// and reduced through LDS in a fixed order.
//
// The work of one layer call is a list of units — router rows, the top-k/grouping unit, gate|up tiles, down tiles —
// executed either by one kernel per phase (the unfused path) or by one persistent cooperative kernel that walks the
// list with dependency counters (the fused path).  Both paths run the same unit functions, so they agree bit for bit.
#include "moe_kernels.h"

#include <math.h>

namespace moe {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
// LDS pointers carry their address space so that reads compile to ds_read (LGKM counter), never to flat loads that
// would share the vector-memory counter with the in-flight weight stream.
#define LDS_AS __attribute__((address_space(3)))
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef LDS_AS u32x4 lds_u32x4;
typedef LDS_AS float lds_float;

constexpr unsigned kSpinLimit = 1u << 20;  // bounded dependency waits (~1 s): a wait never hangs the GPU

__device__ __forceinline__ float bf_lo(unsigned v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(unsigned v) { return __uint_as_float(v & 0xFFFF0000u); }

__device__ __forceinline__ uint16_t f2bf_dev(float f) {  // RNE by the bias trick (same bits as the host f2bf)
    unsigned u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ void unpack8(const u32x4 v, float* f) {
    f[0] = bf_lo(v.x); f[1] = bf_hi(v.x); f[2] = bf_lo(v.y); f[3] = bf_hi(v.y);
    f[4] = bf_lo(v.z); f[5] = bf_hi(v.z); f[6] = bf_lo(v.w); f[7] = bf_hi(v.w);
}

__device__ __forceinline__ void unpack16_i8(const u32x4 v, float* f) {
    const unsigned d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; q++) {
#pragma unroll
        for (int b = 0; b < 4; b++) f[4 * q + b] = (float)(int)(signed char)(d[q] >> (8 * b));
    }
}

__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.f + expf(-g))) * u; }

__device__ __forceinline__ u32x4 ld_stream(const u32x4* p) { return __builtin_nontemporal_load(p); }

// Data that crosses workgroups inside one launch (logits, the slot table, ids/gates, act, partial outputs) is written
// and read with agent-scope relaxed atomics: on gfx950 these are plain global loads/stores carrying the sc1 bit, which
// keeps them coherent across the XCDs' L2s without any cache writeback or invalidate.  A producer orders its data
// before the counter it bumps by waiting for its own stores to complete (vmcnt(0)) before the workgroup barrier; a
// consumer reads the data only after it has observed the counter.  Agent-scope fences (an L2 writeback/invalidate per
// wavefront, microseconds each under load) are never needed on the hot path.
template <typename V>
__device__ __forceinline__ V ld_sync(const V* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
template <typename V>
__device__ __forceinline__ void st_sync(V* p, V v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void wait_own_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0), others untouched

// wavefront index within the workgroup as a wave-uniform (scalar) value, so loop bounds derived from it stay scalar
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// --------------------------------------------------------------------------------------------------------------------
// Chunk dot products of the expert GEMVs: v_dot2_f32_bf16 on packed bf16 pairs (no unpacking), per lane and token one
// chain over chunks ascending and pairs ascending.  xs: LDS activation chunks; token j's chunk c at xs[xoff[j] + c].
// N tokens are always computed (the unit picks N >= its token count; extra columns read token 0 and are discarded),
// so the streamed loop has no data-dependent branches and the load pipeline keeps its depth.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(unsigned a, unsigned b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

template <int N>
__device__ __forceinline__ void dot_chunk_bf16(const u32x4 w, const lds_u32x4* xs, const int* xoff, int c, float* acc) {
#pragma unroll
    for (int j = 0; j < N; j++) {
        const u32x4 x = xs[xoff[j] + c];
        float a = acc[j];
        a = dot2(w.x, x.x, a);
        a = dot2(w.y, x.y, a);
        a = dot2(w.z, x.z, a);
        a = dot2(w.w, x.w, a);
        acc[j] = a;
    }
}

// four int8 weights -> two packed bf16 pairs (exact: |q| <= 127 has at most 7 significant bits)
__device__ __forceinline__ void i8x4_to_bf16(unsigned v, unsigned& p01, unsigned& p23) {
    const float f0 = (float)(int)(signed char)v, f1 = (float)(int)(signed char)(v >> 8);
    const float f2 = (float)(int)(signed char)(v >> 16), f3 = (float)((int)v >> 24);
    p01 = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xFFFF0000u);
    p23 = (__float_as_uint(f2) >> 16) | (__float_as_uint(f3) & 0xFFFF0000u);
}

// int8 chunk c (16 weights) meets bf16 activation chunks 2c and 2c+1
template <int N>
__device__ __forceinline__ void dot_chunk_q8(const u32x4 w, const lds_u32x4* xs, const int* xoff, int c, float* acc) {
    unsigned p[8];
    i8x4_to_bf16(w.x, p[0], p[1]);
    i8x4_to_bf16(w.y, p[2], p[3]);
    i8x4_to_bf16(w.z, p[4], p[5]);
    i8x4_to_bf16(w.w, p[6], p[7]);
#pragma unroll
    for (int j = 0; j < N; j++) {
        const u32x4 x0 = xs[xoff[j] + 2 * c], x1 = xs[xoff[j] + 2 * c + 1];
        float a = acc[j];
        a = dot2(p[0], x0.x, a);
        a = dot2(p[1], x0.y, a);
        a = dot2(p[2], x0.z, a);
        a = dot2(p[3], x0.w, a);
        a = dot2(p[4], x1.x, a);
        a = dot2(p[5], x1.y, a);
        a = dot2(p[6], x1.z, a);
        a = dot2(p[7], x1.w, a);
        acc[j] = a;
    }
}

// Stream chunks [c0, c1) of a 64-row tile (lane = row), consuming in ascending order.  Two register banks of D
// loads alternate (load B, consume A, reload A, consume B), so D to 2D loads are always in flight and a reload only
// ever targets a bank that has been consumed; the steady-state loop has no branches.
template <int N, bool Q8>
__device__ __forceinline__ void tile_stream(const u32x4* __restrict__ tile, int c0, int c1, const lds_u32x4* xs,
                                            const int* xoff, float* acc) {
    constexpr int D = N >= 8 ? 4 : 8;  // wide token counts hold N activation chunks per weight chunk in registers
    const u32x4* p = tile + (threadIdx.x & 63);
    u32x4 A[D], B[D];
    auto load = [&](u32x4* bank, int c) {
#pragma unroll
        for (int u = 0; u < D; u++) bank[u] = ld_stream(p + (size_t)(c + u) * 64);
    };
    auto consume = [&](const u32x4* bank, int c) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            if (Q8) dot_chunk_q8<N>(bank[u], xs, xoff, c + u, acc);
            else dot_chunk_bf16<N>(bank[u], xs, xoff, c + u, acc);
        }
    };
    const int nb = (c1 - c0) / D;
    int b = 0;
    if (nb > 0) load(A, c0);
    for (; b + 2 < nb; b += 2) {
        load(B, c0 + (b + 1) * D);
        consume(A, c0 + b * D);
        load(A, c0 + (b + 2) * D);
        consume(B, c0 + (b + 1) * D);
    }
    if (nb - b == 2) {
        load(B, c0 + (b + 1) * D);
        consume(A, c0 + b * D);
        consume(B, c0 + (b + 1) * D);
    } else if (nb - b == 1) {
        consume(A, c0 + b * D);
    }
    for (int c = c0 + nb * D; c < c1; c++) {  // fewer than D leftover chunks
        const u32x4 w = ld_stream(p + (size_t)c * 64);
        if (Q8) dot_chunk_q8<N>(w, xs, xoff, c, acc);
        else dot_chunk_bf16<N>(w, xs, xoff, c, acc);
    }
}

// Sum the 4 wavefronts' partials in wave order; result for (token j, row lane) in red[j * 64 + lane].
template <int NT>
__device__ __forceinline__ void reduce_waves(lds_float* red, const float* acc, int ntok) {
    const int wave = wave_id(), lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < NT; j++)
        if (j < ntok) red[(wave * NT + j) * 64 + lane] = acc[j];
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int j = 0; j < NT; j++)
            if (j < ntok)
                red[j * 64 + lane] = ((red[j * 64 + lane] + red[(NT + j) * 64 + lane]) + red[(2 * NT + j) * 64 + lane]) +
                                     red[(3 * NT + j) * 64 + lane];
    }
    __syncthreads();
}

// --------------------------------------------------------------------------------------------------------------------
// Dynamic shared-memory plan of a workgroup (16-byte aligned pieces):
//   xs    [T][H/8] u32x4      all tokens' activations, staged once per workgroup
//   as    [NT][F/8] u32x4     one slot's act rows (down units)
//   red   [4][NT][64] float   cross-wave reduction
// (the route unit's scratch is static __shared__ memory inside route_unit)
struct Lds {
    lds_u32x4* xs;
    lds_u32x4* as;
    lds_float* red;
};

// `as` doubles as the route unit's score table: NT tokens x E (rounded up to 4) biased scores + NT x topk ranks.
__host__ __device__ inline size_t as_bytes(int NT, int F, int E) {
    const size_t act = (size_t)NT * (F / 8) * 16, route = (size_t)NT * (((E + 3) & ~3) + kMaxTopk) * 4;
    return ((act > route ? act : route) + 15) & ~(size_t)15;
}

size_t lds_bytes(int T, int NT, int H, int F, int E) {
    return (size_t)T * (H / 8) * 16 + as_bytes(NT, F, E) + (size_t)4 * NT * 64 * 4;
}

__device__ inline Lds lds_carve(unsigned char* base_generic, int T, int NT, int H, int F, int E) {
    LDS_AS unsigned char* base = (LDS_AS unsigned char*)base_generic;
    Lds s;
    s.xs = (lds_u32x4*)base;
    base += (size_t)T * (H / 8) * 16;
    s.as = (lds_u32x4*)base;
    base += as_bytes(NT, F, E);
    s.red = (lds_float*)base;
    return s;
}

__device__ inline void stage_x(const Lds& s, const uint16_t* __restrict__ x, int T, int H) {
    const int n = T * (H / 8);
    const u32x4* src = reinterpret_cast<const u32x4*>(x);
    for (int i = threadIdx.x; i < n; i += blockDim.x) s.xs[i] = src[i];
    __syncthreads();
}

// --------------------------------------------------------------------------------------------------------------------
// Unit: router rows.  Wave w computes logits[t, e] for e = e0 + w and all T tokens.  Reduction order (mirrored bit
// for bit by the host oracle): lane l owns chunks c = l + 64 j; per token a fused multiply-add chain over j
// ascending and elements 0..7 ascending; then a 64-lane xor butterfly (32, 16, 8, 4, 2, 1).
template <int NT>
__device__ __forceinline__ void router_unit(const Lds& s, const uint16_t* __restrict__ wr, int e0, int E, int H, int T,
                            float* __restrict__ logits) {
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int e = e0 + wave;
    if (e >= E) return;
    const u32x4* row = reinterpret_cast<const u32x4*>(wr + (size_t)e * H);
    const int nc = H / 8, nj = H / 512;
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.f;
    for (int j0 = 0; j0 < nj; j0 += 8) {
        u32x4 w[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (j0 + j < nj) w[j] = row[lane + 64 * (j0 + j)];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (j0 + j < nj) {
                float wf[8];
                unpack8(w[j], wf);
                const int c = lane + 64 * (j0 + j);
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    if (t < T) {
                        float xf[8];
                        unpack8(s.xs[t * nc + c], xf);
#pragma unroll
                        for (int i = 0; i < 8; i++) acc[t] = fmaf(wf[i], xf[i], acc[t]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        if (t < T) {
            float v = acc[t];
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m, 64);
            if (lane == 0) st_sync(&logits[(size_t)t * E + e], v);
        }
    }
}

// --------------------------------------------------------------------------------------------------------------------
// Unit: softmax top-k (one wavefront per token, tokens strided over the 4 waves) and expert grouping (workgroup).
// Selection compares biased logits, ties to the lower expert index; gates = softmax restricted to the kept ranks.
// Grouping: routed slots in first-seen order scanning tokens then ranks; shared slots first.
// Maximum over the 64 lanes of a wavefront: DPP exchanges within rows of 16 lanes, then the four row results.
__device__ __forceinline__ float dpp_max_step(float v, int ctrl_id) {
    int o;
    switch (ctrl_id) {  // dpp_ctrl must be a compile-time constant
        case 0: o = __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0xB1, 0xF, 0xF, false); break;   // quad_perm [1,0,3,2]
        case 1: o = __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x4E, 0xF, 0xF, false); break;   // quad_perm [2,3,0,1]
        case 2: o = __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x141, 0xF, 0xF, false); break;  // row_half_mirror
        default: o = __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x140, 0xF, 0xF, false); break; // row_mirror
    }
    return fmaxf(v, __int_as_float(o));
}
__device__ __forceinline__ float wave_max(float v) {
    v = dpp_max_step(v, 0);
    v = dpp_max_step(v, 1);
    v = dpp_max_step(v, 2);
    v = dpp_max_step(v, 3);  // every lane of a 16-lane row now holds the row maximum
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

__device__ __forceinline__ void route_unit(const Lds& s, const float* __restrict__ logits, const float* __restrict__ bias,
                                           int T, int E, int k, int keep, int n_shared, int do_topk,
                                           int32_t* __restrict__ ids, float* __restrict__ gates,
                                           Slots* __restrict__ slots) {
    __shared__ int ent_e[kMaxTokens * kMaxTopk];       // expert of entry (t, r), r < keep; -1 = empty rank
    __shared__ int first_pos[kMaxExperts];
    __shared__ int slot_of[kMaxExperts];
    __shared__ int ent_flag[kMaxTokens * kMaxTopk];
    const int tid = threadIdx.x;
    const int n = T * keep;
    if (tid == 0) st_sync(&slots->err, 0);
    __syncthreads();
    if (do_topk) {
        // One wavefront per token (tokens strided over the workgroup's wavefronts).  Lane l holds the biased scores
        // of experts l + 64 i.  Each of the k rounds takes the maximum remaining score with a DPP reduction (no
        // shared-memory round trips) and the lowest expert index holding it with ballots, i.e. the order is
        // (score descending, index ascending); NaN scores rank last.
        const int wave = wave_id(), lane = tid & 63;
        const int nI = (E + 63) / 64;
        for (int t0 = 0; t0 < T; t0 += kWaves) {
            const int t = t0 + wave;
            if (t < T) {
                float sc[kMaxExperts / 64];
#pragma unroll
                for (int i = 0; i < kMaxExperts / 64; i++)  // every load issued before any use: one round trip
                    sc[i] = ld_sync(&logits[(size_t)t * E + min(lane + 64 * i, E - 1)]);
#pragma unroll
                for (int i = 0; i < kMaxExperts / 64; i++) {
                    const int e = lane + 64 * i;
                    float v = sc[i] + (bias ? bias[min(e, E - 1)] : 0.f);
                    if (!(v == v)) v = -INFINITY;
                    sc[i] = e < E ? v : -INFINITY;
                }
                unsigned live = 0;  // bit i: element i of this lane is a real, not yet selected expert
#pragma unroll
                for (int i = 0; i < kMaxExperts / 64; i++)
                    if (lane + 64 * i < E) live |= 1u << i;
                float my_sc = 0.f;
                int my_id = 0;
                for (int r = 0; r < k; r++) {
                    float lm = -INFINITY;
#pragma unroll
                    for (int i = 0; i < kMaxExperts / 64; i++)
                        if ((live >> i) & 1u) lm = fmaxf(lm, sc[i]);
                    const float m = wave_max(lm);
                    int id = -1;
                    for (int i = 0; i < nI && id < 0; i++) {
                        const unsigned long long hit = __ballot(((live >> i) & 1u) && sc[i] == m);
                        if (hit) id = 64 * i + (__ffsll(hit) - 1);
                    }
                    if (id < 0) id = 0;  // unreachable: k <= E and every live score is comparable
                    if ((id & 63) == lane) live &= ~(1u << (id >> 6));
                    if (lane == r) { my_sc = m; my_id = id; }
                }
                // gates: softmax restricted to the kept ranks; lane r holds rank r, rank 0 the maximum
                const float top = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_sc), 0));
                const float ex = expf(my_sc - top);
                float tot = 0.f;
                for (int q = 0; q < keep; q++) tot += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), q));
                if (lane < k) {
                    st_sync(&ids[t * k + lane], (int32_t)my_id);
                    st_sync(&gates[t * k + lane], lane < keep ? ex / tot : 0.f);
                    if (lane < keep) ent_e[t * keep + lane] = my_id;
                }
            }
        }
    } else {
        for (int p = tid; p < n; p += blockDim.x) {
            int e = ld_sync(&ids[(p / keep) * k + p % keep]);
            if (e < -1 || e >= E) {  // out of range: flag and drop the entry
                st_sync(&slots->err, 1);
                e = -1;
            }
            ent_e[p] = e;
        }
    }
    __syncthreads();
    // 4. grouping: routed slots in first-seen order scanning tokens then ranks (runtime.py:344-347), after the
    //    n_shared shared slots.  Up to 64 entries (every decode batch of T * keep <= 64) are grouped in wave 0's
    //    registers: lane i holds entry i, readlane/ballot replace shared-memory round trips.
    if (n <= 64) {
        if (tid < 64) {
            const int lane = tid;
            const int my_e = lane < n ? ent_e[lane] : -1;
            int cnt = 0, pos = 0, firstj = 64;
            for (int j = 0; j < n; j++) {
                const int ej = __builtin_amdgcn_readlane(my_e, j);
                const bool m = my_e >= 0 && ej == my_e;
                cnt += m;
                pos += m && j < lane;
                if (m && j < firstj) firstj = j;
            }
            const bool flag = my_e >= 0 && firstj == lane;
            const unsigned long long mask = __ballot(flag);
            const int slot = n_shared + (int)__popcll(mask & ((1ull << firstj) - 1ull));  // slot of my first occurrence
            if (flag) {
                st_sync(&slots->expert[slot], my_e);
                st_sync(&slots->ntok[slot], cnt < T ? cnt : T);
            }
            if (my_e >= 0) {
                if (pos < T) {
                    st_sync(&slots->tok[slot][pos], lane / keep);
                    st_sync(&slots->rank[slot][pos], lane % keep);
                } else {
                    st_sync(&slots->err, 2);  // an expert repeated within one token's ids
                }
            }
            if (lane == 0) st_sync(&slots->nslot, n_shared + (int)__popcll(mask));
        }
    } else {
        for (int e = tid; e < E; e += blockDim.x) first_pos[e] = 0x7FFFFFFF;
        __syncthreads();
        const int my_e = tid < n ? ent_e[tid] : -1;
        if (my_e >= 0) atomicMin(&first_pos[my_e], tid);
        __syncthreads();
        if (tid < n) ent_flag[tid] = my_e >= 0 && first_pos[my_e] == tid;
        __syncthreads();
        if (tid < n && ent_flag[tid]) {
            int before = 0;
            for (int j = 0; j < tid; j++) before += ent_flag[j];
            const int sl = n_shared + before;
            slot_of[my_e] = sl;
            int cnt = 0;
            for (int j = 0; j < n; j++) cnt += ent_e[j] == my_e;
            st_sync(&slots->expert[sl], my_e);
            st_sync(&slots->ntok[sl], cnt < T ? cnt : T);
        }
        __syncthreads();
        if (my_e >= 0) {
            const int sl = slot_of[my_e];
            int pos = 0;
            for (int j = 0; j < tid; j++) pos += ent_e[j] == my_e;
            if (pos < T) {
                st_sync(&slots->tok[sl][pos], tid / keep);
                st_sync(&slots->rank[sl][pos], tid % keep);
            } else {
                st_sync(&slots->err, 2);
            }
        }
        if (tid == 0) {
            int nf = 0;
            for (int j = 0; j < n; j++) nf += ent_flag[j];
            st_sync(&slots->nslot, n_shared + nf);
        }
    }
    if (tid < n_shared) {
        st_sync(&slots->expert[tid], -1 - tid);
        st_sync(&slots->ntok[tid], T);
        for (int j = 0; j < T; j++) { st_sync(&slots->tok[tid][j], j); st_sync(&slots->rank[tid][j], -1); }
    }
    __syncthreads();
}

// --------------------------------------------------------------------------------------------------------------------
// Unit: gate|up tile.  Slot s, 32 f values = one 64-row tile (32 gate rows + their 32 up rows) over K = H, the 4
// wavefronts splitting K; act[s][j][f] = bf16(silu(g) * u) for the slot's tokens.
template <int N>
__device__ __forceinline__ void gateup_core(const Lds& s, const ExpertArgs& a, int sl, int tile, int e, int ntok, const int* tok) {
    const int H = a.d.H, F = a.d.F;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int nc = H / 8;
    int xoff[N];
#pragma unroll
    for (int j = 0; j < N; j++) xoff[j] = j < ntok ? tok[j] * nc : 0;
    float acc[N];
#pragma unroll
    for (int j = 0; j < N; j++) acc[j] = 0.f;
    const bool q8 = a.int8 && e >= 0;
    if (!q8) {
        const uint16_t* base =
            e >= 0 ? a.L.gu + (size_t)e * a.d.gu_stride() : a.L.sgu + (size_t)(-1 - e) * a.d.gu_stride();
        const u32x4* t = reinterpret_cast<const u32x4*>(base) + (size_t)tile * nc * 64;
        const int cpw = nc / kWaves;
        tile_stream<N, false>(t, wave * cpw, (wave + 1) * cpw, s.xs, xoff, acc);
    } else {
        const int ncq = H / 16;
        const u32x4* t = reinterpret_cast<const u32x4*>(a.L.gu_q8 + (size_t)e * a.d.gu_stride()) + (size_t)tile * ncq * 64;
        const int cpw = ncq / kWaves;
        tile_stream<N, true>(t, wave * cpw, (wave + 1) * cpw, s.xs, xoff, acc);
    }
    reduce_waves<N>(s.red, acc, N);
    if (wave == 0) {
        const float scale = q8 ? a.L.sc_q8[(size_t)e * (2 * F + H) + tile * 64 + lane] : 1.f;
#pragma unroll
        for (int j = 0; j < N; j++) {
            float v = s.red[j * 64 + lane];
            if (q8) v = v * scale;
            const float up = __shfl_down(v, 8, 64);  // gate row lane (bit 3 clear) meets its up row (lane + 8)
            const unsigned h = f2bf_dev(silu_mul(v, up));
            const unsigned h_next = __shfl_down(h, 1, 64);  // f + 1 lives in the next lane
            if (j < ntok && !gu_row_up(lane) && !(lane & 1))
                st_sync(reinterpret_cast<unsigned*>(a.act + ((size_t)sl * a.d.max_t + j) * F + gu_row_f(tile, lane)),
                        h | (h_next << 16));
        }
    }
    __syncthreads();  // s.red is reused by the next unit
}

template <int NT>
__device__ __forceinline__ void gateup_unit(const Lds& s, const ExpertArgs& a, int sl, int tile, int e, int ntok, const int* tok) {
    if (ntok <= 1 || NT == 1) gateup_core<1>(s, a, sl, tile, e, ntok, tok);
    else if (ntok <= 2 || NT == 2) gateup_core<(NT < 2 ? NT : 2)>(s, a, sl, tile, e, ntok, tok);
    else if (ntok <= 4 || NT == 4) gateup_core<(NT < 4 ? NT : 4)>(s, a, sl, tile, e, ntok, tok);
    else if (ntok <= 8 || NT == 8) gateup_core<(NT < 8 ? NT : 8)>(s, a, sl, tile, e, ntok, tok);
    else gateup_core<NT>(s, a, sl, tile, e, ntok, tok);
}

// Unit: down tile.  Slot s, 64 output rows over K = F; y written unweighted to ypart[t][q][h] with q = s for a shared
// slot and n_shared + rank for a routed one.
template <int N>
__device__ __forceinline__ void down_core(const Lds& s, const ExpertArgs& a, int sl, int ht, int e, int ntok, const int* tok,
                          const int* rank) {
    const int H = a.d.H, F = a.d.F;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int nc = F / 8;
    const unsigned* src = reinterpret_cast<const unsigned*>(a.act + (size_t)sl * a.d.max_t * F);
    LDS_AS unsigned* dst = (LDS_AS unsigned*)s.as;
    for (int i = threadIdx.x; i < ntok * (F / 2); i += blockDim.x) dst[i] = ld_sync(src + i);
    __syncthreads();
    int xoff[N];
#pragma unroll
    for (int j = 0; j < N; j++) xoff[j] = j < ntok ? j * nc : 0;
    float acc[N];
#pragma unroll
    for (int j = 0; j < N; j++) acc[j] = 0.f;
    const bool q8 = a.int8 && e >= 0;
    if (!q8) {
        const uint16_t* base =
            e >= 0 ? a.L.dn + (size_t)e * a.d.dn_stride() : a.L.sdn + (size_t)(-1 - e) * a.d.dn_stride();
        const u32x4* t = reinterpret_cast<const u32x4*>(base) + (size_t)ht * nc * 64;
        const int cpw = nc / kWaves;
        tile_stream<N, false>(t, wave * cpw, (wave + 1) * cpw, s.as, xoff, acc);
    } else {
        const int ncq = F / 16;
        const u32x4* t = reinterpret_cast<const u32x4*>(a.L.dn_q8 + (size_t)e * a.d.dn_stride()) + (size_t)ht * ncq * 64;
        const int cpw = ncq / kWaves;
        tile_stream<N, true>(t, wave * cpw, (wave + 1) * cpw, s.as, xoff, acc);
    }
    reduce_waves<N>(s.red, acc, N);
    if (wave == 0) {
        const int h = ht * 64 + lane;
        const float scale = q8 ? a.L.sc_q8[(size_t)e * (2 * F + H) + 2 * F + h] : 1.f;
        const int kq = a.d.n_shared + a.d.k;
#pragma unroll
        for (int j = 0; j < N; j++) {
            if (j < ntok) {
                const int q = e < 0 ? sl : a.d.n_shared + rank[j];
                float y = s.red[j * 64 + lane];
                if (q8) y = y * scale;
                st_sync(&a.ypart[((size_t)tok[j] * kq + q) * H + h], y);
            }
        }
    }
    __syncthreads();  // s.as / s.red are reused by the next unit
}

template <int NT>
__device__ __forceinline__ void down_unit(const Lds& s, const ExpertArgs& a, int sl, int ht, int e, int ntok, const int* tok,
                          const int* rank) {
    if (ntok <= 1 || NT == 1) down_core<1>(s, a, sl, ht, e, ntok, tok, rank);
    else if (ntok <= 2 || NT == 2) down_core<(NT < 2 ? NT : 2)>(s, a, sl, ht, e, ntok, tok, rank);
    else if (ntok <= 4 || NT == 4) down_core<(NT < 4 ? NT : 4)>(s, a, sl, ht, e, ntok, tok, rank);
    else if (ntok <= 8 || NT == 8) down_core<(NT < 8 ? NT : 8)>(s, a, sl, ht, e, ntok, tok, rank);
    else down_core<NT>(s, a, sl, ht, e, ntok, tok, rank);
}

// Combine one output element: (out or 0) + shared terms + gate * routed terms, fixed order.
__device__ __forceinline__ void combine_elem(const ExpertArgs& a, int t, int h) {
    const int H = a.d.H, k = a.d.k, kq = a.d.n_shared + a.d.k;
    const size_t o = (size_t)t * H + h;
    float acc = a.accumulate ? a.out[o] : 0.f;
    for (int q = 0; q < a.n_shared; q++) acc = acc + ld_sync(&a.ypart[((size_t)t * kq + q) * H + h]);
    for (int r = 0; r < a.keep; r++)
        if (ld_sync(&a.ids[t * k + r]) >= 0)
            acc = fmaf(ld_sync(&a.gates[t * k + r]), ld_sync(&a.ypart[((size_t)t * kq + a.d.n_shared + r) * H + h]), acc);
    a.out[o] = acc;
}

// Coherent snapshot of one slot of the table the route unit published.
template <int NT>
struct SlotView {
    int expert, ntok;
    int tok[NT], rank[NT];
    __device__ __forceinline__ void load(const Slots* sp, int sl) {  // independent loads: one round trip
        expert = ld_sync(&sp->expert[sl]);
        ntok = ld_sync(&sp->ntok[sl]);
#pragma unroll
        for (int j = 0; j < NT; j++) {
            tok[j] = ld_sync(&sp->tok[sl][j]);
            rank[j] = ld_sync(&sp->rank[sl][j]);
        }
#pragma unroll
        for (int j = 0; j < NT; j++)
            if (j >= ntok) tok[j] = rank[j] = 0;  // entries past ntok are stale: keep indices in range
    }
};

// Publish this workgroup's coherent stores, then count the unit as done.
__device__ __forceinline__ void signal_add(unsigned* p, unsigned v) {
    wait_own_stores();
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Poll with relaxed agent-scope loads; after the barrier the workgroup reads the producers' data with ld_sync.
__device__ __forceinline__ void wait_ge(unsigned* p, unsigned target, unsigned* err, uint64_t* stamp = nullptr) {
    if (threadIdx.x == 0) {
        unsigned n = 0;
        while (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            __builtin_amdgcn_s_sleep(2);
            ++n;
            // give up after kSpinLimit polls, or at once when another wait of this launch already gave up
            if (n > kSpinLimit || ((n & 255) == 0 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
                __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
        if (stamp) *stamp = __builtin_amdgcn_s_memrealtime();
    }
    __syncthreads();
}



// After a down unit of tile ht (live or skipped), count it; the last of the tile's maxs units combines the tile.
__device__ __forceinline__ void down_done_combine(const ExpertArgs& a, Sync* sy, int ht) {
    __shared__ int s_last;
    wait_own_stores();
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(&sy->d_done[ht * kSyncPad], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (unsigned)(a.maxs - 1);
    __syncthreads();
    if (s_last)  // every down unit of this tile has published its partial outputs
        for (int i = threadIdx.x; i < a.T * 64; i += blockDim.x) combine_elem(a, i / 64, ht * 64 + i % 64);
    __syncthreads();
}

// At kernel exit the last workgroup clears the counters for the next launch on this context.
__device__ __forceinline__ void exit_and_reset(Sync* sy) {
    __shared__ int s_last;
    wait_own_stores();
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(&sy->exit_count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 gridDim.x - 1;
    __syncthreads();
    if (s_last) {
        for (int i = threadIdx.x; i < kMaxSlots; i += blockDim.x) st_sync(&sy->gu_done[i * kSyncPad], 0u);
        for (int i = threadIdx.x; i < kMaxHTiles; i += blockDim.x) st_sync(&sy->d_done[i * kSyncPad], 0u);
        if (threadIdx.x == 0) {
            st_sync(&sy->router_done, 0u);
            st_sync(&sy->route_ready, 0u);
            st_sync(&sy->next_unit, 0u);
            st_sync(&sy->exit_count, 0u);
        }
    }
}

// ====================================================================================================================
// Unfused path: one kernel per phase (stream order provides the dependencies).
__global__ __launch_bounds__(256) void router_kernel(LayerPtrs L, Dims d, int T, const uint16_t* __restrict__ x,
                                                     float* __restrict__ logits) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    const Lds s = lds_carve(lds_raw, T, 1, d.H, d.F, d.E);
    stage_x(s, x, T, d.H);
    if (T <= 1) router_unit<1>(s, L.wr, blockIdx.x * kWaves, d.E, d.H, T, logits);
    else if (T <= 4) router_unit<4>(s, L.wr, blockIdx.x * kWaves, d.E, d.H, T, logits);
    else router_unit<kMaxTokens>(s, L.wr, blockIdx.x * kWaves, d.E, d.H, T, logits);
}

__global__ __launch_bounds__(256) void topk_group_kernel(LayerPtrs L, Dims d, int T, int keep, int n_shared,
                                                         int do_topk, const float* __restrict__ logits,
                                                         int32_t* __restrict__ ids, float* __restrict__ gates,
                                                         Slots* __restrict__ slots) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    const Lds s = lds_carve(lds_raw, 0, T, d.H, d.F, d.E);
    route_unit(s, logits, L.bias, T, d.E, d.k, keep, n_shared, do_topk, ids, gates, slots);
}

template <int NT>
__global__ __launch_bounds__(256) void gateup_kernel(ExpertArgs a) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    const Lds s = lds_carve(lds_raw, a.T, NT, a.d.H, a.d.F, a.d.E);
    const int ntile = a.d.F / 32;
    const int sl = blockIdx.x / ntile, tile = blockIdx.x % ntile;
    if (sl >= ld_sync(&a.slots->nslot) || (sl < a.d.n_shared && sl >= a.n_shared)) return;  // unused / left out
    SlotView<NT> v;
    v.load(a.slots, sl);
    stage_x(s, a.x, a.T, a.d.H);
    gateup_unit<NT>(s, a, sl, tile, v.expert, v.ntok, v.tok);
}

template <int NT>
__global__ __launch_bounds__(256) void down_kernel(ExpertArgs a, Sync* sy) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    const Lds s = lds_carve(lds_raw, 0, NT, a.d.H, a.d.F, a.d.E);
    const int nht = a.d.H / 64;
    const int sl = blockIdx.x / nht, ht = blockIdx.x % nht;
    if (sl < ld_sync(&a.slots->nslot) && (sl >= a.d.n_shared || sl < a.n_shared)) {  // else unused / left out
        SlotView<NT> v;
        v.load(a.slots, sl);
        down_unit<NT>(s, a, sl, ht, v.expert, v.ntok, v.tok, v.rank);
    }
    down_done_combine(a, sy, ht);
    exit_and_reset(sy);
}


// ====================================================================================================================
// Fused path: one persistent kernel walks the unit list
//   [router units][route unit][shared gate|up][routed gate|up][down, slot-major]
// through a work queue: a global counter hands out unit indices in ascending order, and each workgroup fetches its
// next index while it works on the current one.  A unit waits only on units of smaller index; the smallest
// unfinished unit is therefore always some running workgroup's current unit and can proceed, so the grid needs no
// co-residency guarantee (a plain launch).  Every wait is also bounded by kSpinLimit.  The last down unit of each
// 64-row tile combines that tile; the last workgroup to finish clears the counters for the next launch.
template <int NT>
__global__ __launch_bounds__(256) void fused_layer_kernel(FusedArgs f) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    const ExpertArgs& a = f.e;
    const Lds s = lds_carve(lds_raw, a.T, NT, a.d.H, a.d.F, a.d.E);
    Sync* sy = f.sync;
    const int H = a.d.H, F = a.d.F;
    const int ntile = F / 32, nht = H / 64;
    const int maxs = a.maxs;
    const int uR = f.nR, uRoute = uR + 1, uGUs = uRoute + a.d.n_shared * ntile, uGU = uRoute + maxs * ntile;
    const int uEnd = uGU + maxs * nht;
    __shared__ int s_unit;
    if (threadIdx.x == 0) s_unit = (int)__hip_atomic_fetch_add(&sy->next_unit, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    stage_x(s, a.x, a.T, H);  // ends with a barrier: s_unit is visible
    uint64_t t_start = 0;
    for (int u = s_unit; u < uEnd;) {
        int next = 0;
        if (threadIdx.x == 0) {  // fetch the next unit now; its latency hides behind this unit's work
            next = (int)__hip_atomic_fetch_add(&sy->next_unit, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (f.trace) {
                t_start = __builtin_amdgcn_s_memrealtime();
                f.trace[(size_t)u * 4 + 1] = 0;
            }
        }
        if (u < uR) {
            router_unit<NT>(s, a.L.wr, u * kWaves, a.d.E, H, a.T, f.logits);
            signal_add(&sy->router_done, 1);
        } else if (u < uRoute) {
            if (uR) wait_ge(&sy->router_done, (unsigned)uR, &sy->err, f.trace ? f.trace + (size_t)u * 4 + 1 : nullptr);
            route_unit(s, f.logits, a.L.bias, a.T, a.d.E, a.d.k, a.keep, a.d.n_shared, f.do_topk, a.ids, a.gates,
                       a.slots);
            signal_add(&sy->route_ready, 1);
        } else if (u < uGU) {
            const int sl = (u - uRoute) / ntile, tile = (u - uRoute) % ntile;
            if (u < uGUs) {  // shared slot: all tokens in order, no routing dependency
                if (sl < a.n_shared) {
                    int tok[NT];
#pragma unroll
                    for (int j = 0; j < NT; j++) tok[j] = j;
                    gateup_unit<NT>(s, a, sl, tile, -1 - sl, a.T, tok);
                }
            } else {
                wait_ge(&sy->route_ready, 1, &sy->err, f.trace ? f.trace + (size_t)u * 4 + 1 : nullptr);
                if (sl < ld_sync(&a.slots->nslot)) {
                    SlotView<NT> v;
                    v.load(a.slots, sl);
                    gateup_unit<NT>(s, a, sl, tile, v.expert, v.ntok, v.tok);
                }
            }
            signal_add(&sy->gu_done[sl * kSyncPad], 1);
        } else {
            const int sl = (u - uGU) / nht, ht = (u - uGU) % nht;
            wait_ge(&sy->route_ready, 1, &sy->err);
            const bool live = sl < ld_sync(&a.slots->nslot) && (sl >= a.d.n_shared || sl < a.n_shared);
            if (live) {
                SlotView<NT> v;
                v.load(a.slots, sl);
                wait_ge(&sy->gu_done[sl * kSyncPad], (unsigned)ntile, &sy->err, f.trace ? f.trace + (size_t)u * 4 + 1 : nullptr);
                down_unit<NT>(s, a, sl, ht, v.expert, v.ntok, v.tok, v.rank);
            }
            down_done_combine(a, sy, ht);
        }
        if (f.trace && threadIdx.x == 0) {
            f.trace[(size_t)u * 4 + 0] = t_start;
            f.trace[(size_t)u * 4 + 2] = __builtin_amdgcn_s_memrealtime();
            f.trace[(size_t)u * 4 + 3] = blockIdx.x;
        }
        __syncthreads();  // the whole workgroup is done with unit u before s_unit changes
        if (threadIdx.x == 0) s_unit = next;
        __syncthreads();
        u = s_unit;
    }
    exit_and_reset(sy);
}

// --------------------------------------------------------------------------------------------------------------------
// One-time layout kernels (one thread per 16-byte destination chunk).
__global__ void relayout_gu_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u, int H, int F,
                                   u32x4* __restrict__ dst) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t nc = H / 8, total = (size_t)(F / 32) * nc * 64;
    if (q >= total) return;
    const int i = q % 64;
    const size_t c = (q / 64) % nc;
    const int tile = (int)(q / (64 * nc));
    const int f = gu_row_f(tile, i);
    const uint16_t* src = gu_row_up(i) ? u : g;
    dst[q] = reinterpret_cast<const u32x4*>(src + (size_t)f * H)[c];
}

__global__ void relayout_dn_kernel(const uint16_t* __restrict__ d, int H, int F, u32x4* __restrict__ dst) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t nc = F / 8, total = (size_t)(H / 64) * nc * 64;
    if (q >= total) return;
    const int i = q % 64;
    const size_t c = (q / 64) % nc;
    const int tile = (int)(q / (64 * nc));
    dst[q] = reinterpret_cast<const u32x4*>(d + (size_t)(tile * 64 + i) * F)[c];
}

// q in ck_place_expert_q8 layout ([2F rows of H][H rows of F]) <-> tiled int8 + tile-ordered scales (dir 1 = back).
__global__ void relayout_q8_kernel(int8_t* __restrict__ q, float* __restrict__ sc, int H, int F,
                                   int8_t* __restrict__ gu_t, int8_t* __restrict__ dn_t, float* __restrict__ sc_t,
                                   int dir) {
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t ncg = H / 16, ncd = F / 16;
    const size_t ng = (size_t)(F / 32) * ncg * 64, nd = (size_t)(H / 64) * ncd * 64;
    if (id < ng) {
        const int i = id % 64;
        const size_t c = (id / 64) % ncg;
        const int tile = (int)(id / (64 * ncg));
        const int f = gu_row_f(tile, i);
        const int r = gu_row_up(i) ? F + f : f;
        u32x4* tiled = reinterpret_cast<u32x4*>(gu_t) + id;
        u32x4* lin = reinterpret_cast<u32x4*>(q + (size_t)r * H) + c;
        if (dir == 0) *tiled = *lin; else *lin = *tiled;
        if (c == 0) {
            if (dir == 0) sc_t[tile * 64 + i] = sc[r]; else sc[r] = sc_t[tile * 64 + i];
        }
    } else if (id < ng + nd) {
        const size_t id2 = id - ng;
        const int i = id2 % 64;
        const size_t c = (id2 / 64) % ncd;
        const int tile = (int)(id2 / (64 * ncd));
        const int h = tile * 64 + i;
        u32x4* tiled = reinterpret_cast<u32x4*>(dn_t) + id2;
        u32x4* lin = reinterpret_cast<u32x4*>(q + (size_t)2 * F * H + (size_t)h * F) + c;
        if (dir == 0) *tiled = *lin; else *lin = *tiled;
        if (c == 0) {
            if (dir == 0) sc_t[2 * F + h] = sc[2 * F + h]; else sc[2 * F + h] = sc_t[2 * F + h];
        }
    }
}

// quant_row on the device (track2_opt/solar_engine/csrc/cpu_kern.c:218-224): one wavefront per weight row, reading the
// bf16 tiled table and writing the int8 tiled table and the row scale.  max|w| is order-independent and the scale,
// reciprocal, product and round-to-nearest-even are single IEEE operations, so the result equals the host's bits.
__global__ __launch_bounds__(256) void quantize_kernel(const uint16_t* __restrict__ src, size_t src_stride,
                                                       int8_t* __restrict__ dst, size_t dst_stride,
                                                       float* __restrict__ sc, size_t sc_stride, int sc_off, int K,
                                                       int rows_per_exp, size_t total_rows) {
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const size_t row = (size_t)blockIdx.x * 4 + wave;
    if (row >= total_rows) return;
    const int ex = (int)(row / rows_per_exp);
    const int rr = (int)(row % rows_per_exp);
    const int tile = rr / 64, i = rr % 64;
    const int ncb = K / 8, ncq = K / 16;
    const uint16_t* s = src + (size_t)ex * src_stride;
    int8_t* dq = dst + (size_t)ex * dst_stride;
    float m = 0.f;
    for (int c = lane; c < ncb; c += 64) {
        float f[8];
        unpack8(reinterpret_cast<const u32x4*>(s)[((size_t)tile * ncb + c) * 64 + i], f);
#pragma unroll
        for (int k2 = 0; k2 < 8; k2++) m = fmaxf(m, fabsf(f[k2]));
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    const float scl = m > 0.f ? m / 127.f : 1.f, inv = 1.f / scl;
    for (int c = lane; c < ncb; c += 64) {
        float f[8];
        unpack8(reinterpret_cast<const u32x4*>(s)[((size_t)tile * ncb + c) * 64 + i], f);
        unsigned lo = 0, hi = 0;
#pragma unroll
        for (int k2 = 0; k2 < 8; k2++) {
            float qv = rintf(f[k2] * inv);
            qv = fminf(fmaxf(qv, -127.f), 127.f);
            const unsigned b = (unsigned)(int)qv & 0xFFu;
            if (k2 < 4) lo |= b << (8 * k2); else hi |= b << (8 * (k2 - 4));
        }
        u32x2 v;
        v.x = lo; v.y = hi;
        *reinterpret_cast<u32x2*>(dq + (((size_t)tile * ncq + c / 2) * 64 + i) * 16 + (c & 1) * 8) = v;
    }
    if (lane == 0) sc[(size_t)ex * sc_stride + sc_off + rr] = scl;
}

// --------------------------------------------------------------------------------------------------------------------
// Synthetic generator (bench/test support).  Same integer hash and single fp32 multiply as the host generator.
__host__ __device__ inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ int ih8(uint64_t key, uint64_t i) {
    const uint64_t G = 0x9E3779B97F4A7C15ull;
    const uint64_t a = mix64(key + (2 * i + 1) * G), b = mix64(key + (2 * i + 2) * G);
    int s = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) s += (int)((a >> (16 * k)) & 0xFFFF) + (int)((b >> (16 * k)) & 0xFFFF);
    return s - 262140;
}
__device__ __forceinline__ u32x4 synth_chunk(uint64_t key, uint64_t i0, float c) {
    unsigned w[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const unsigned lo = f2bf_dev((float)ih8(key, i0 + 2 * k) * c);
        const unsigned hi = f2bf_dev((float)ih8(key, i0 + 2 * k + 1) * c);
        w[k] = lo | (hi << 16);
    }
    u32x4 v;
    v.x = w[0]; v.y = w[1]; v.z = w[2]; v.w = w[3];
    return v;
}

__global__ void synth_tiled_kernel(uint64_t key_g, uint64_t key_u, uint64_t key_d, float cw, int H, int F,
                                   u32x4* __restrict__ gu, u32x4* __restrict__ dn) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t ncg = H / 8, ncd = F / 8;
    const size_t ng = (size_t)(F / 32) * ncg * 64, nd = (size_t)(H / 64) * ncd * 64;
    if (q < ng) {
        const int i = q % 64;
        const size_t c = (q / 64) % ncg;
        const int tile = (int)(q / (64 * ncg));
        const int f = gu_row_f(tile, i);
        gu[q] = synth_chunk(gu_row_up(i) ? key_u : key_g, (size_t)f * H + c * 8, cw);
    } else if (q < ng + nd) {
        const size_t q2 = q - ng;
        const int i = q2 % 64;
        const size_t c = (q2 / 64) % ncd;
        const int tile = (int)(q2 / (64 * ncd));
        dn[q2] = synth_chunk(key_d, (size_t)(tile * 64 + i) * F + c * 8, cw);
    }
}

__global__ void synth_fill_kernel(u32x4* __restrict__ dst, uint64_t nchunk, uint64_t key, uint64_t start, float c) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q < nchunk) dst[q] = synth_chunk(key, start + q * 8, c);
}

// ==================================================================================================================
// launch helpers
static inline unsigned nblk(size_t n, int b) { return (unsigned)((n + b - 1) / b); }

static hipError_t set_lds(const void* fn, size_t lds) {
    if (lds <= 48 * 1024) return hipSuccess;
    return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

static int nt_bucket(int T) { return T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : T <= 8 ? 8 : 16; }

hipError_t launch_router(const LayerPtrs& L, const Dims& d, int T, const uint16_t* x, float* logits, hipStream_t st) {
    const size_t lds = lds_bytes(T, 1, d.H, d.F, d.E);
    hipError_t e = set_lds(reinterpret_cast<const void*>(&router_kernel), lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(router_kernel, dim3(nblk(d.E, kWaves)), dim3(256), lds, st, L, d, T, x, logits);
    return hipGetLastError();
}

hipError_t launch_topk_group(const LayerPtrs& L, const Dims& d, int T, int keep, int n_shared, bool do_topk,
                             const float* logits, int32_t* ids, float* gates, Slots* slots, hipStream_t st) {
    const size_t lds = lds_bytes(0, T, d.H, d.F, d.E);
    hipError_t e = set_lds(reinterpret_cast<const void*>(&topk_group_kernel), lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(topk_group_kernel, dim3(1), dim3(256), lds, st, L, d, T, keep, n_shared, do_topk ? 1 : 0, logits,
                       ids, gates, slots);
    return hipGetLastError();
}

template <int NT>
static hipError_t gateup_nt(const ExpertArgs& ea, hipStream_t st) {
    const int maxs = ea.maxs;
    const size_t lds = lds_bytes(ea.T, NT, ea.d.H, ea.d.F, ea.d.E);
    hipError_t e = set_lds(reinterpret_cast<const void*>(&gateup_kernel<NT>), lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(gateup_kernel<NT>, dim3(maxs * (ea.d.F / 32)), dim3(256), lds, st, ea);
    return hipGetLastError();
}

template <int NT>
static hipError_t down_nt(const ExpertArgs& ea, Sync* sy, hipStream_t st) {
    const size_t lds = lds_bytes(0, NT, ea.d.H, ea.d.F, ea.d.E);
    hipError_t e = set_lds(reinterpret_cast<const void*>(&down_kernel<NT>), lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(down_kernel<NT>, dim3(ea.maxs * (ea.d.H / 64)), dim3(256), lds, st, ea, sy);
    return hipGetLastError();
}

hipError_t launch_gateup(const ExpertArgs& ea, hipStream_t st) {
    switch (nt_bucket(ea.T)) {
        case 1: return gateup_nt<1>(ea, st);
        case 2: return gateup_nt<2>(ea, st);
        case 4: return gateup_nt<4>(ea, st);
        case 8: return gateup_nt<8>(ea, st);
        default: return gateup_nt<16>(ea, st);
    }
}

hipError_t launch_down(const ExpertArgs& ea, Sync* sy, hipStream_t st) {
    switch (nt_bucket(ea.T)) {
        case 1: return down_nt<1>(ea, sy, st);
        case 2: return down_nt<2>(ea, sy, st);
        case 4: return down_nt<4>(ea, sy, st);
        case 8: return down_nt<8>(ea, sy, st);
        default: return down_nt<16>(ea, sy, st);
    }
}


template <int NT>
static hipError_t fused_nt(FusedArgs f, int wg_per_cu, hipStream_t st, int* grid_out) {
    const void* fn = reinterpret_cast<const void*>(&fused_layer_kernel<NT>);
    const size_t lds = lds_bytes(f.e.T, NT, f.e.d.H, f.e.d.F, f.e.d.E);
    // occupancy per (device, LDS size), computed once: the launch itself stays a single host call
    static thread_local int c_dev = -1, c_ncu = 0, c_per_cu = 0;
    static thread_local size_t c_lds = 0;
    hipError_t e;
    int dev = 0;
    if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
    if (dev != c_dev || lds != c_lds) {
        if ((e = set_lds(fn, lds)) != hipSuccess) return e;
        if ((e = hipDeviceGetAttribute(&c_ncu, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
        if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&c_per_cu, fn, 256, lds)) != hipSuccess) return e;
        c_dev = dev;
        c_lds = lds;
    }
    int per_cu = c_per_cu, ncu = c_ncu;
    if (wg_per_cu > 0 && wg_per_cu < per_cu) per_cu = wg_per_cu;
    if (per_cu < 1) return hipErrorInvalidConfiguration;
    const int units = f.nR + 1 + f.e.maxs * (f.e.d.F / 32) + f.e.maxs * (f.e.d.H / 64);
    int grid = ncu * per_cu;
    if (grid > units) grid = units;
    if (grid_out) *grid_out = grid;
    hipLaunchKernelGGL(fused_layer_kernel<NT>, dim3(grid), dim3(256), lds, st, f);
    return hipGetLastError();
}

hipError_t launch_fused(const FusedArgs& f, int wg_per_cu, hipStream_t st, int* grid_out) {
    switch (nt_bucket(f.e.T)) {
        case 1: return fused_nt<1>(f, wg_per_cu, st, grid_out);
        case 2: return fused_nt<2>(f, wg_per_cu, st, grid_out);
        case 4: return fused_nt<4>(f, wg_per_cu, st, grid_out);
        case 8: return fused_nt<8>(f, wg_per_cu, st, grid_out);
        default: return fused_nt<16>(f, wg_per_cu, st, grid_out);
    }
}

hipError_t launch_relayout_gu(const uint16_t* g, const uint16_t* u, int H, int F, uint16_t* dst, hipStream_t st) {
    const size_t n = (size_t)(F / 32) * (H / 8) * 64;
    hipLaunchKernelGGL(relayout_gu_kernel, dim3(nblk(n, 256)), dim3(256), 0, st, g, u, H, F,
                       reinterpret_cast<u32x4*>(dst));
    return hipGetLastError();
}

hipError_t launch_relayout_dn(const uint16_t* dsrc, int H, int F, uint16_t* dst, hipStream_t st) {
    const size_t n = (size_t)(H / 64) * (F / 8) * 64;
    hipLaunchKernelGGL(relayout_dn_kernel, dim3(nblk(n, 256)), dim3(256), 0, st, dsrc, H, F,
                       reinterpret_cast<u32x4*>(dst));
    return hipGetLastError();
}

hipError_t launch_relayout_q8(const int8_t* q, const float* sc, int H, int F, int8_t* gu_dst, int8_t* dn_dst,
                              float* sc_dst, hipStream_t st) {
    const size_t n = (size_t)(F / 32) * (H / 16) * 64 + (size_t)(H / 64) * (F / 16) * 64;
    hipLaunchKernelGGL(relayout_q8_kernel, dim3(nblk(n, 256)), dim3(256), 0, st, const_cast<int8_t*>(q),
                       const_cast<float*>(sc), H, F, gu_dst, dn_dst, sc_dst, 0);
    return hipGetLastError();
}

hipError_t launch_unlayout_q8(const int8_t* gu_src, const int8_t* dn_src, const float* sc_src, int H, int F, int8_t* q,
                              float* sc, hipStream_t st) {
    const size_t n = (size_t)(F / 32) * (H / 16) * 64 + (size_t)(H / 64) * (F / 16) * 64;
    hipLaunchKernelGGL(relayout_q8_kernel, dim3(nblk(n, 256)), dim3(256), 0, st, q, sc, H, F,
                       const_cast<int8_t*>(gu_src), const_cast<int8_t*>(dn_src), const_cast<float*>(sc_src), 1);
    return hipGetLastError();
}

hipError_t launch_quantize(const uint16_t* gu, const uint16_t* dn, int H, int F, int n_exp, size_t gu_stride,
                           size_t dn_stride, int8_t* gu_q8, int8_t* dn_q8, float* sc, hipStream_t st) {
    const size_t sc_stride = (size_t)2 * F + H;
    const size_t rows_gu = (size_t)n_exp * 2 * F, rows_dn = (size_t)n_exp * H;
    hipLaunchKernelGGL(quantize_kernel, dim3(nblk(rows_gu, 4)), dim3(256), 0, st, gu, gu_stride, gu_q8, gu_stride, sc,
                       sc_stride, 0, H, 2 * F, rows_gu);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(quantize_kernel, dim3(nblk(rows_dn, 4)), dim3(256), 0, st, dn, dn_stride, dn_q8, dn_stride, sc,
                       sc_stride, 2 * F, F, H, rows_dn);
    return hipGetLastError();
}

hipError_t launch_synth_tiled(uint64_t key_g, uint64_t key_u, uint64_t key_d, float c, int H, int F, uint16_t* gu,
                              uint16_t* dn, hipStream_t st) {
    const size_t n = (size_t)(F / 32) * (H / 8) * 64 + (size_t)(H / 64) * (F / 8) * 64;
    hipLaunchKernelGGL(synth_tiled_kernel, dim3(nblk(n, 256)), dim3(256), 0, st, key_g, key_u, key_d, c, H, F,
                       reinterpret_cast<u32x4*>(gu), reinterpret_cast<u32x4*>(dn));
    return hipGetLastError();
}

hipError_t launch_synth_fill(uint16_t* dst, uint64_t n, uint64_t key, uint64_t start, float c, hipStream_t st) {
    const uint64_t nchunk = n / 8;
    hipLaunchKernelGGL(synth_fill_kernel, dim3(nblk(nchunk, 256)), dim3(256), 0, st, reinterpret_cast<u32x4*>(dst),
                       nchunk, key, start, c);
    return hipGetLastError();
}

uint64_t synth_key(uint64_t seed, uint64_t tensor_id) { return mix64(seed * 0xD1B54A32D192ED03ull + tensor_id); }

bool kernels_available() {
    hipFuncAttributes attr;
    return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&router_kernel)) == hipSuccess;
}

}  // namespace moe
