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
// The work of one layer call is a list of units — router rows, the top-k/grouping unit, gate|up tile parts, down
// tiles — executed either by one kernel per phase (the unfused path) or by one persistent kernel that walks the list
// through a work queue (the fused path).  Cross-workgroup values are epoch-tagged words that consumers poll directly.
// Both paths run the same unit functions, so they agree bit for bit.
#include "moe_kernels.h"

#include <math.h>

#include "ck_dot.h"
#include "launch_util.h"

namespace moe {

// Build partitioning.  Compiled as one translation unit (MOE_PART undefined), or as parts compiled in parallel:
// MOE_PART=0 holds everything except the token-bucket kernels, MOE_PART=N (1, 2, 4, 8, 16) only bucket N's kernels
// and launchers (explicitly instantiated there, declared extern in part 0).
#if !defined(MOE_PART)
#define MOE_COMMON 1
#elif MOE_PART == 0
#define MOE_COMMON 1
#define MOE_EXTERN_BUCKETS 1
#else
#define MOE_COMMON 0
#endif

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
// LDS pointers carry their address space so that reads compile to ds_read (LGKM counter), never to flat loads that
// would share the vector-memory counter with the in-flight weight stream.
#define LDS_AS __attribute__((address_space(3)))
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef LDS_AS u32x4 lds_u32x4;
typedef LDS_AS float lds_float;

constexpr unsigned kSpinLimit = 1u << 20;  // bounded dependency waits (~1 s): a wait never hangs the GPU
// Shared-memory scratch of route_local (carved from the act-row region, unused while a unit computes its routing).
constexpr int kRouteKeys = 1024;  // sort keys of one pass (tokens x experts)
#ifndef MOE_TOPK_THREADS
#define MOE_TOPK_THREADS 512
#endif
constexpr int kTopkThreads = MOE_TOPK_THREADS;  // the standalone routing kernel's workgroup
constexpr size_t kRouteScratchBytes = (size_t)kRouteKeys * 8 + (size_t)kRouteKeys * 4;

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

// Data that crosses workgroups inside one launch is written and read with agent-scope relaxed atomics: on gfx950 these
// are plain global loads/stores carrying the sc1 bit, coherent across the XCDs' L2s without any cache writeback or
// invalidate.  Every such value is a 64-bit word (epoch << 32) | payload, stored with one store and read with one load
// (single-copy atomic): the host gives each call a fresh epoch, so a consumer that reads a word carrying the call's
// epoch holds a value of this call.  Consumers poll the data itself (bounded); producers never wait for their stores
// to complete, and there are no dependency counters, so each dependency costs one memory round trip.
template <typename V>
__device__ __forceinline__ V ld_sync(const V* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
template <typename V>
__device__ __forceinline__ void st_sync(V* p, V v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

__device__ __forceinline__ void st_tag(uint64_t* p, unsigned epoch, unsigned v) {
    st_sync(p, ((uint64_t)epoch << 32) | v);
}
__device__ __forceinline__ bool tag_ok(uint64_t w, unsigned epoch) { return (unsigned)(w >> 32) == epoch; }

// Words w[m] (m < M, loaded earlier from ptr(m), needed where need(m)) that do not carry the epoch yet are re-loaded
// together, one round trip per pass, until all do.  Gives up after kSpinLimit passes, or early once another wait of
// the launch gave up (err set), so no wait can hang the GPU; the host then reports the call as failed.
template <int M, typename Ptr, typename Need>
__device__ __forceinline__ bool pending_words(const uint64_t (&w)[M], Need need, unsigned epoch) {
    bool p = false;
#pragma unroll
    for (int m = 0; m < M; m++) p = p || (need(m) && !tag_ok(w[m], epoch));
    return p;
}
template <int M, typename Ptr, typename Need>
__device__ __forceinline__ void settle(uint64_t (&w)[M], Ptr ptr, Need need, unsigned epoch, unsigned* err) {
    unsigned n = 0;
    while (pending_words<M, Ptr>(w, need, epoch)) {
        ++n;
        if (n > kSpinLimit || ((n & 255) == 0 && ld_sync(err))) {
            st_sync(err, 1u);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int m = 0; m < M; m++)
            if (need(m) && !tag_ok(w[m], epoch)) w[m] = ld_sync(ptr(m));
    }
}
// The same wait bounded by `limit` passes, without flagging an error: returns false when words are still missing.
template <int M, typename Ptr, typename Need>
__device__ __forceinline__ bool settle_for(uint64_t (&w)[M], Ptr ptr, Need need, unsigned epoch, int limit) {
    for (int n = 0; pending_words<M, Ptr>(w, need, epoch); ++n) {
        if (n >= limit) return false;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int m = 0; m < M; m++)
            if (need(m) && !tag_ok(w[m], epoch)) w[m] = ld_sync(ptr(m));
    }
    return true;
}

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
// ever targets a bank that has been consumed; the steady-state loop has no branches.  begin() issues the first bank,
// so a caller can start the stream before it waits for the activations (run() consumes them).
// Loads per register bank (1 KB each per wavefront) of the gate|up and down streams.  On the Solar layer 8 measured
// best for both: depths 4 to 20 were all slower, and so was interleaving the 4 wavefronts chunk by chunk (each
// wavefront streams a contiguous quarter of its part).
#ifndef MOE_GU_DEPTH
#define MOE_GU_DEPTH 8
#endif
#ifndef MOE_DN_DEPTH
#define MOE_DN_DEPTH 8
#endif
template <int N, bool Q8, int DEPTH>
struct TileStream {
    // wide token counts hold N activation chunks per weight chunk in registers: at most 4 loads per bank
    static constexpr int D = N >= 8 ? (DEPTH < 4 ? DEPTH : 4) : DEPTH;
    const u32x4* p;
    int c0, c1;
    u32x4 A[D];
    __device__ __forceinline__ void load(u32x4* bank, int c) {
#pragma unroll
        for (int u = 0; u < D; u++) bank[u] = ld_stream(p + (size_t)(c + u) * 64);
    }
    __device__ __forceinline__ void consume(const u32x4* bank, int c, const lds_u32x4* xs, const int* xoff, float* acc) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            if (Q8) dot_chunk_q8<N>(bank[u], xs, xoff, c + u, acc);
            else dot_chunk_bf16<N>(bank[u], xs, xoff, c + u, acc);
        }
    }
    __device__ __forceinline__ void begin(const u32x4* __restrict__ tile, int c0_, int c1_) {
        p = tile + (threadIdx.x & 63);
        c0 = c0_;
        c1 = c1_;
        if ((c1 - c0) / D > 0) load(A, c0);
    }
    __device__ __forceinline__ void run(const lds_u32x4* xs, const int* xoff, float* acc) {
        u32x4 B[D];
        const int nb = (c1 - c0) / D;
        int b = 0;
        for (; b + 2 < nb; b += 2) {
            load(B, c0 + (b + 1) * D);
            consume(A, c0 + b * D, xs, xoff, acc);
            load(A, c0 + (b + 2) * D);
            consume(B, c0 + (b + 1) * D, xs, xoff, acc);
        }
        if (nb - b == 2) {
            load(B, c0 + (b + 1) * D);
            consume(A, c0 + b * D, xs, xoff, acc);
            consume(B, c0 + (b + 1) * D, xs, xoff, acc);
        } else if (nb - b == 1) {
            consume(A, c0 + b * D, xs, xoff, acc);
        }
        const int cl = c0 + nb * D;  // fewer than D leftover chunks: all their loads issued, then consumed in order
        if (cl < c1) {
#pragma unroll
            for (int u = 0; u < D; u++)
                if (cl + u < c1) B[u] = ld_stream(p + (size_t)(cl + u) * 64);
#pragma unroll
            for (int u = 0; u < D; u++) {
                if (cl + u < c1) {
                    if (Q8) dot_chunk_q8<N>(B[u], xs, xoff, cl + u, acc);
                    else dot_chunk_bf16<N>(B[u], xs, xoff, cl + u, acc);
                }
            }
        }
    }
};

template <int N, bool Q8>
__device__ __forceinline__ void tile_stream(const u32x4* __restrict__ tile, int c0, int c1, const lds_u32x4* xs,
                                            const int* xoff, float* acc) {
    TileStream<N, Q8, MOE_GU_DEPTH> ts;
    ts.begin(tile, c0, c1);
    ts.run(xs, xoff, acc);
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
// MFMA path of the batch >= 8 grouped case (a call of 8 or more tokens, units with more than 4 tokens): the tile's
// 64 rows x up to 8 tokens as 4 row blocks of v_mfma_f32_16x16x32_bf16 (16 rows x 16 token columns x 32 k; columns
// of tokens past the unit's count are computed from token 0's activations and dropped).  Operand layout (checked on
// the device): lane l holds A row l % 16 and B column l % 16 over k = 8 (l / 16) .. 8 (l / 16) + 7; D rows
// 4 (l / 16) .. 4 (l / 16) + 3 of column l % 16.  The tile layout [chunk][64 rows] of 16-byte chunks gives each lane
// its A operand in one 16-byte load (row 16 b + l % 16 of chunk c + l / 16); its B operand is one LDS read of the
// token's activation chunk.  The sums run in the MFMA's order, not the dot2 chains', so this path matches the
// others within the layer bars rather than bit for bit.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma_bf16(u32x4 a, u32x4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
}

// Chunks [c0, c1) of a 64-row tile in groups of 4 (bf16: 8 k per chunk, one MFMA per row block; int8: 16 k per chunk,
// two MFMAs per row block, the weights widened to bf16 exactly).  Two banks of MF_DEPTH groups alternate as in
// TileStream; lanes whose chunk lies past c1 (the last group) load zeros.
#ifndef MOE_MF_DEPTH
#define MOE_MF_DEPTH 2
#endif
template <bool Q8>
struct MfmaStream {
    static constexpr int D = MOE_MF_DEPTH;
    const u32x4* p;  // tile + (lane / 16) * 64 + lane % 16
    int c0, c1;
    u32x4 A[D][4];
    __device__ __forceinline__ void load(u32x4 (&bank)[D][4], int c) {
        const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
        for (int u = 0; u < D; u++) {
            const bool ok = c + 4 * u + g < c1;
#pragma unroll
            for (int b = 0; b < 4; b++)
                bank[u][b] = ok ? ld_stream(p + (size_t)(c + 4 * u) * 64 + 16 * b) : u32x4{0u, 0u, 0u, 0u};
        }
    }
    __device__ __forceinline__ void consume(const u32x4 (&bank)[D][4], int c, const lds_u32x4* xs, int xo,
                                            f32x4_t (&d)[4]) {
        const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
        for (int u = 0; u < D; u++) {
            const int cc = min(c + 4 * u + g, c1 - 1);  // past c1: a valid chunk, its A operand is zero
            if (!Q8) {
                const u32x4 x = xs[xo + cc];
#pragma unroll
                for (int b = 0; b < 4; b++) d[b] = mfma_bf16(bank[u][b], x, d[b]);
            } else {
                const u32x4 x0 = xs[xo + 2 * cc], x1 = xs[xo + 2 * cc + 1];
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    unsigned w[8];
                    i8x4_to_bf16(bank[u][b].x, w[0], w[1]);
                    i8x4_to_bf16(bank[u][b].y, w[2], w[3]);
                    i8x4_to_bf16(bank[u][b].z, w[4], w[5]);
                    i8x4_to_bf16(bank[u][b].w, w[6], w[7]);
                    d[b] = mfma_bf16(u32x4{w[0], w[1], w[2], w[3]}, x0, d[b]);
                    d[b] = mfma_bf16(u32x4{w[4], w[5], w[6], w[7]}, x1, d[b]);
                }
            }
        }
    }
    __device__ __forceinline__ void begin(const u32x4* __restrict__ tile, int c0_, int c1_) {
        const int lane = threadIdx.x & 63;
        p = tile + (lane >> 4) * 64 + (lane & 15);
        c0 = c0_;
        c1 = c1_;
        if (c1 > c0) load(A, c0);
    }
    __device__ __forceinline__ void run(const lds_u32x4* xs, int xo, f32x4_t (&d)[4]) {
        u32x4 B[D][4];
        const int step = 4 * D, nb = (c1 - c0 + step - 1) / step;
        int b = 0;
        for (; b + 2 < nb; b += 2) {
            load(B, c0 + (b + 1) * step);
            consume(A, c0 + b * step, xs, xo, d);
            load(A, c0 + (b + 2) * step);
            consume(B, c0 + (b + 1) * step, xs, xo, d);
        }
        if (nb - b == 2) {
            load(B, c0 + (b + 1) * step);
            consume(A, c0 + b * step, xs, xo, d);
            consume(B, c0 + (b + 1) * step, xs, xo, d);
        } else if (nb - b == 1) {
            consume(A, c0 + b * step, xs, xo, d);
        }
    }
};

// This lane's token column l % 16 as an activation chunk offset: slot token (l % 16) if it exists, else token 0's.
// (masks and ors, not selects: a select chain over the array compiled to a scratch-memory table lookup)
template <int NT>
__device__ __forceinline__ int mfma_xoff(const int* xoff, int ntok) {
    const int j = threadIdx.x & 15, jj = j < ntok ? j : 0;
    int xo = 0;
#pragma unroll
    for (int i = 0; i < NT; i++) xo |= xoff[i] & -(int)(jj == i);
    return xo;
}

// The MFMA partials of the 4 wavefronts into red[(wave * NT + j) * 64 + row], then summed as reduce_waves does.
template <int NT>
__device__ __forceinline__ void reduce_waves_mfma(lds_float* red, const f32x4_t (&d)[4], int ntok) {
    const int wave = wave_id(), lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
    if (j < NT && j < ntok) {
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[(wave * NT + j) * 64 + 16 * b + 4 * g + r] = d[b][r];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int jj = 0; jj < NT; jj++)
            if (jj < ntok)
                red[jj * 64 + lane] = ((red[jj * 64 + lane] + red[(NT + jj) * 64 + lane]) + red[(2 * NT + jj) * 64 + lane]) +
                                      red[(3 * NT + jj) * 64 + lane];
    }
    __syncthreads();
}

// --------------------------------------------------------------------------------------------------------------------
// Dynamic shared-memory plan of a workgroup (16-byte aligned pieces):
//   xs    [T][H/8] u32x4      all tokens' activations, staged once per workgroup
//   as    [NT][F/8] u32x4     one slot's act rows (down units)
//   red   [4][NT][64] float   cross-wave reduction
//   xf    [H] float           T = 1 only: the token in fp32, for the router units' dot products
// (the routing table is static __shared__ memory: RouteTab)
struct Lds {
    lds_u32x4* xs;
    lds_u32x4* as;
    lds_float* red;
    lds_float* xf;  // T = 1 only, else null
};

// `as` also serves as route_local's scratch
__host__ __device__ inline size_t as_bytes(int NT, int F, int E) {
    (void)E;
    const size_t act = (size_t)NT * (F / 8) * 16;
    return act > kRouteScratchBytes ? act : kRouteScratchBytes;
}

#if MOE_COMMON
size_t lds_bytes(int T, int NT, int H, int F, int E) {
    return (size_t)T * (H / 8) * 16 + as_bytes(NT, F, E) + (size_t)4 * NT * 64 * 4 + (T == 1 ? (size_t)H * 4 : 0);
}
#endif  // MOE_COMMON

__device__ inline Lds lds_carve(unsigned char* base_generic, int T, int NT, int H, int F, int E) {
    LDS_AS unsigned char* base = (LDS_AS unsigned char*)base_generic;
    Lds s;
    s.xs = (lds_u32x4*)base;
    base += (size_t)T * (H / 8) * 16;
    s.as = (lds_u32x4*)base;
    base += as_bytes(NT, F, E);
    s.red = (lds_float*)base;
    base += (size_t)4 * NT * 64 * 4;
    s.xf = T == 1 ? (lds_float*)base : nullptr;
    return s;
}

__device__ __forceinline__ float round_bf(float v) { return bf_lo(f2bf_dev(v)); }

__device__ __forceinline__ u32x4 pack_bf16x8(const float* v) {
    u32x4 r;
    r.x = f2bf_dev(v[0]) | ((unsigned)f2bf_dev(v[1]) << 16);
    r.y = f2bf_dev(v[2]) | ((unsigned)f2bf_dev(v[3]) << 16);
    r.z = f2bf_dev(v[4]) | ((unsigned)f2bf_dev(v[5]) << 16);
    r.w = f2bf_dev(v[6]) | ((unsigned)f2bf_dev(v[7]) << 16);
    return r;
}

// Stage the T tokens' activations into s.xs, and at T = 1 also into s.xf as fp32 (every thread returns after the
// closing barrier).
//   plain: a copy of in.x;
//   block mode: r = bf16(resid + attn_o) (main.rs:122), then RMSNorm (host.rs:71-76): ms = sum(r^2) / H,
//   rs = 1 / sqrt(ms + eps), h = bf16(bf16(r * rs) * w).  The squares are summed in a fixed order (per thread over
//   its chunks in order, then a 64-lane xor butterfly, then the 4 wavefronts in order), so every workgroup stages
//   the same bits.  Each thread handles 16-byte chunks c = tid + j * kThreads, two per pass (H = 4096: one pass, one
//   round trip for resid, attn_o and the norm weight together), with few registers: the router unit stages while
//   its weight loads are held in registers.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef LDS_AS f32x4 lds_f32x4;
__device__ __forceinline__ void store_f32x8(lds_float* dst, const float* f) {
    reinterpret_cast<lds_f32x4*>(dst)[0] = f32x4{f[0], f[1], f[2], f[3]};
    reinterpret_cast<lds_f32x4*>(dst)[1] = f32x4{f[4], f[5], f[6], f[7]};
}

__device__ __forceinline__ void stage_in(const Lds& s, const StageSrc& in, int T, int H) {
    const int n = T * (H / 8);
    if (!in.resid) {
        const u32x4* src = reinterpret_cast<const u32x4*>(in.x);
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            const u32x4 v = src[i];
            s.xs[i] = v;
            if (s.xf) {
                float f[8];
                unpack8(v, f);
                store_f32x8(s.xf + 8 * i, f);
            }
        }
        __syncthreads();
        return;
    }
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id(), nc = H / 8;
    const u32x4* xr = reinterpret_cast<const u32x4*>(in.resid);
    const u32x4* xo = reinterpret_cast<const u32x4*>(in.attn_o);
    const u32x4* wn = reinterpret_cast<const u32x4*>(in.norm_w);
    const bool w_held = nc <= 2 * kThreads;  // the norm weights of this thread's chunks stay in registers
    u32x4 w0 = {0u, 0u, 0u, 0u}, w1 = {0u, 0u, 0u, 0u};
    if (w_held) {
        if (tid < nc) w0 = wn[tid];
        if (tid + kThreads < nc) w1 = wn[tid + kThreads];
    }
    for (int t = 0; t < T; t++) {
        float sq = 0.f;
        for (int c0 = tid; c0 < nc; c0 += 2 * kThreads) {
            const int c1 = c0 + kThreads;
            const u32x4 a0 = xr[(size_t)t * nc + c0], b0 = xo[(size_t)t * nc + c0];
            u32x4 a1 = a0, b1 = b0;
            if (c1 < nc) {
                a1 = xr[(size_t)t * nc + c1];
                b1 = xo[(size_t)t * nc + c1];
            }
#pragma unroll
            for (int h = 0; h < 2; h++) {
                if (h == 1 && c1 >= nc) break;
                float fa[8], fb[8], r[8];
                unpack8(h ? a1 : a0, fa);
                unpack8(h ? b1 : b0, fb);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    r[i] = round_bf(fa[i] + fb[i]);  // main.rs:122
                    sq = fmaf(r[i], r[i], sq);
                }
                s.xs[t * nc + (h ? c1 : c0)] = pack_bf16x8(r);
            }
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) sq = sq + __shfl_xor(sq, m, 64);
        if (lane == 0) s.red[t * kWaves + wave] = sq;
    }
    __syncthreads();
    for (int t = 0; t < T; t++) {
        const float ms = (((s.red[t * kWaves] + s.red[t * kWaves + 1]) + s.red[t * kWaves + 2]) + s.red[t * kWaves + 3]) /
                         (float)H;
        const float rs = 1.0f / sqrtf(ms + in.eps);
        for (int c = tid; c < nc; c += kThreads) {
            const u32x4 wv = w_held ? (c == tid ? w0 : w1) : wn[c];
            float fr[8], fw[8], h[8];
            unpack8(s.xs[t * nc + c], fr);
            unpack8(wv, fw);
#pragma unroll
            for (int i = 0; i < 8; i++) h[i] = round_bf(round_bf(fr[i] * rs) * fw[i]);
            s.xs[t * nc + c] = pack_bf16x8(h);
            if (s.xf) store_f32x8(s.xf + 8 * c, h);
        }
    }
    __syncthreads();
}

// Outputs of one combined element o = t * H + h: out (fp32, when given) and, in block mode, the next residual
// x = bf16(r + bf16(bf16(routed) + bf16(shared))) with r = bf16(resid + attn_o), as the host layer's moe_host
// (main.rs:133-141: the shared and the routed sums each rounded to bf16, their sum rounded, added to the residual).
__device__ __forceinline__ void combine_store(const ExpertArgs& a, size_t o, float acc, float acc_s, float acc_r) {
    if (a.out) a.out[o] = acc;
    if (a.x_next) {
        const float r = round_bf(bf_lo(a.in.resid[o]) + bf_lo(a.in.attn_o[o]));
        a.x_next[o] = f2bf_dev(r + round_bf(round_bf(acc_r) + round_bf(acc_s)));
    }
}

// --------------------------------------------------------------------------------------------------------------------
// Unit: router rows, in the reference's own order (ck_rows_dot_chain, ck_dot.h): the logits are bit-identical to
// ck_gemv's (track2_opt/solar_engine/csrc/cpu_kern.c:9-19, :31-35).  The table is in chain order (ck_chain_dword);
// wave w < kRouterRows / 2 computes rows e0 + 2w (lanes 0-31) and e0 + 2w + 1 (lanes 32-63) for all T tokens.
// stage: the activations (from src) are staged once the weight loads are in flight.  src travels by value: an
// address of a kernel argument would make the compiler copy the arguments to scratch memory.
// Several tokens: a unit takes kRouterTG of them (tokens t0 ..), so that T tokens spread over more workgroups.
template <int NT>
__device__ __forceinline__ void router_unit(const Lds& s, const uint16_t* __restrict__ wr, int e0, int E, int H, int T,
                                            uint64_t* __restrict__ logits, float* __restrict__ logits_out,
                                            unsigned epoch, bool stage, const StageSrc src, bool stamp,
                                            uint64_t& t_in, uint64_t& t_dot, int t0 = 0) {
    static_assert(kRouterRows == 2 || kRouterRows == 4 || kRouterRows == 8, "two router rows per wavefront");
    const int wave = wave_id(), lane = threadIdx.x & 63;
    if (2 * wave >= kRouterRows) {  // a wavefront without rows only takes part in the staging
        if (stage) stage_in(s, src, T, H);
        return;
    }
    const int ea = e0 + 2 * wave, e = ea + (lane >> 5);
    float acc[NT];
    const u32x4* w = reinterpret_cast<const u32x4*>(wr);
    const size_t rs = (size_t)H / 8;  // u32x4 per row
    ck_rows_dot_chain<NT>(w + (size_t)min(ea, E - 1) * rs, w + (size_t)min(ea + 1, E - 1) * rs, H, T - t0,
                          (const LDS_AS unsigned*)s.xs + (size_t)t0 * (H / 2), NT == 1 ? s.xf : nullptr, acc,
                          [&]() __attribute__((always_inline)) {
                              if (stage) stage_in(s, src, T, H);
                              if (stamp) t_in = __builtin_amdgcn_s_memrealtime();
                          });
    if (stamp) t_dot = __builtin_amdgcn_s_memrealtime();
    if ((lane & 31) == 0 && e < E) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (t0 + t < T) {
                st_tag(&logits[(size_t)(t0 + t) * E + e], epoch, __float_as_uint(acc[t]));
                if (logits_out) logits_out[(size_t)(t0 + t) * E + e] = acc[t];
            }
        }
    }
}

// --------------------------------------------------------------------------------------------------------------------
// Routing.
// Per-workgroup routing table in shared memory.  Every workgroup of the fused kernel that needs the routing computes
// it itself from the logits (the computation is deterministic, so all copies agree bit for bit) instead of waiting
// for one workgroup to publish it: this removes a publish / poll / reload hop from the critical path.
struct RouteTab {
    int nslot;
    int err;                                          // 1: an id outside [-1, E); 2: an expert repeated in a token
    int id[kMaxTokens * kMaxTopk];                    // [t][k] expert of rank r; -1: empty rank or dropped id
    float gate[kMaxTokens * kMaxTopk];                // [t][k] gate of rank r (0 for ranks >= keep)
    short slot_e[kMaxSlots];                          // expert of a slot (shared slot s: -1 - s)
    unsigned char slot_n[kMaxSlots];                  // tokens of a slot
    unsigned char slot_p[kMaxSlots][kMaxTokens];      // routed slot: entry p = t * keep + r; shared slot: token
    short slot_pair[kMaxSlots];                       // first (slot, token) pair: shared s -> s * T, then routed
};
typedef LDS_AS RouteTab lds_RouteTab;

// Total order of the selection as one unsigned 64-bit key: biased score (NaN ranks as -inf) through the
// order-preserving float -> uint map in the high word, the complemented expert index in the low word, so that a
// larger key means (higher score, or equal score and lower index).
__device__ __forceinline__ uint64_t route_key(float v, int e) {
    const unsigned u = __float_as_uint(v);
    const unsigned o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)o << 32) | (unsigned)~e;
}
__device__ __forceinline__ float route_key_score(uint64_t key) {
    const unsigned o = (unsigned)(key >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

// sigmoid of a logit as the reference's route() computes it in fp32 (host.rs:119-121: 1 / (1 + exp(-v))).  exp is
// evaluated in double and rounded once to fp32, which is the correctly rounded fp32 exp except when the value lies
// within a double rounding error of an fp32 rounding boundary; the add and the divide are single IEEE operations.
__device__ __forceinline__ float sigmoid_ref(float v) {
    const float ex = (float)exp(-(double)v);
    return 1.f / (1.f + ex);
}

// The largest of each 16-lane row's 64-bit keys, in every lane of the row (DPP moves within the row, each step
// combining equal halves).  All 64 lanes must be active.
__device__ __forceinline__ uint64_t row_max_u64(uint64_t v) {
#define MOE_DPP_MAX_STEP(CTRL)                                                                             \
    {                                                                                                      \
        const unsigned lo_ = (unsigned)__builtin_amdgcn_mov_dpp((int)(unsigned)v, CTRL, 0xF, 0xF, false);  \
        const unsigned hi_ = (unsigned)__builtin_amdgcn_mov_dpp((int)(unsigned)(v >> 32), CTRL, 0xF, 0xF, false); \
        const uint64_t o_ = ((uint64_t)hi_ << 32) | lo_;                                                   \
        v = o_ > v ? o_ : v;                                                                               \
    }
    MOE_DPP_MAX_STEP(0xB1)   // quad [1,0,3,2]
    MOE_DPP_MAX_STEP(0x4E)   // quad [2,3,0,1]
    MOE_DPP_MAX_STEP(0x141)  // row half mirror
    MOE_DPP_MAX_STEP(0x140)  // row mirror
#undef MOE_DPP_MAX_STEP
    return v;
}

// Several tokens' selection: token tl of the pass (t0 + tl overall) on row tl of the workgroup's 16-lane rows, KQ keys
// per lane (experts l, l + 16, .. of the token's E), k rounds of the row maximum.  Called by the whole workgroup.
template <int KQ>
__device__ __forceinline__ void select_rows(lds_RouteTab* rt, const LDS_AS uint64_t* keys, const LDS_AS float* sgv,
                                            int t0, int nt, int E, int k, int rule) {
    const int g = threadIdx.x >> 4, l16 = threadIdx.x & 15, ng = blockDim.x >> 4;
    for (int base = 0; base < nt; base += ng) {  // uniform: every lane runs the DPP steps
        const int tl = base + g;
        const bool live = tl < nt;
        uint64_t kk[KQ];
#pragma unroll
        for (int q = 0; q < KQ; q++) kk[q] = live && l16 + 16 * q < E ? keys[tl * E + l16 + 16 * q] : 0ull;
        for (int r = 0; r < k; r++) {
            uint64_t m[KQ];
#pragma unroll
            for (int q = 0; q < KQ; q++) m[q] = kk[q];
#pragma unroll
            for (int w = KQ / 2; w >= 1; w >>= 1)
#pragma unroll
                for (int q = 0; q < w; q++) m[q] = m[q + w] > m[q] ? m[q + w] : m[q];
            const uint64_t top = row_max_u64(m[0]);
#pragma unroll
            for (int q = 0; q < KQ; q++)
                if (kk[q] == top) kk[q] = 0ull;
            if (live && l16 == 0) {
                const int t = t0 + tl, e = (int)~(unsigned)top;
                rt->id[t * k + r] = e;
                rt->gate[t * k + r] = rule == kRouteSigmoid ? sgv[tl * E + e] : route_key_score(top);
            }
        }
    }
}

// Top-k and expert grouping into rt.  Selection: the k largest keys (score descending, index ascending); each thread
// counts, for one (token, expert) and a slice of the experts, how many keys beat it (its rank), reading the keys as
// shared-memory broadcasts, so the whole workgroup works on it.  Scores and gates by rule:
//   softmax (npu-kernels/npu_kernels/rngd/layer_template/src/host.rs.tpl:247-267): score = logit + bias; gates = the
//     softmax restricted to the kept ranks, exp(s_r - s_0) / sum_{q < keep} exp(s_q - s_0), summed in rank order;
//   sigmoid (track2_opt/solar_engine/src/host.rs:119-128): s = sigmoid(logit), score = s + bias (the bias only
//     selects); gates = s_r / (sum_{q < keep} s_q + 1e-20), summed in rank order.
// Grouping: routed slots in first-seen order scanning tokens then ranks (solar_hybrid/runtime.py:344-347), after the
// n_shared shared slots.  do_topk == 0: the caller's ids / gates are taken as given (ids outside [-1, E) dropped).
// scr: kRouteScratchBytes of LDS.  poll >= 0 bounds the wait for the tagged logits to that many passes: the call then
// returns 1, uniformly, when logits are still missing (their router units have not run), and the caller computes
// them itself and calls again; poll < 0 waits up to the launch-wide limit.  Returns 0 once rt is complete.
// MULTI false: the caller only ever has one token (the several-token selection is left out of its code).
template <bool MULTI = true>
__device__ __forceinline__ int route_local(lds_RouteTab* rt, LDS_AS unsigned char* scr,
                                           const uint64_t* __restrict__ logits, unsigned epoch, unsigned* err,
                                           const float* __restrict__ bias, const int32_t* ids_in,
                                           const float* gates_in, int T, int E, int k, int keep, int n_shared,
                                           int do_topk, int rule, int poll) {
    const int tid = threadIdx.x, nthr = blockDim.x;
    LDS_AS uint64_t* keys = (LDS_AS uint64_t*)scr;
    LDS_AS int* cnt = (LDS_AS int*)(scr + (size_t)kRouteKeys * 8);
    int bad = 0;
    if (do_topk) {
        const int tc = min(T, max(1, kRouteKeys / E));  // tokens per pass
        for (int t0 = 0; t0 < T; t0 += tc) {
            const int nt = min(tc, T - t0), items = nt * E;
            // 1. keys: every tagged logit load of the pass issued before any use (4 per thread at most)
            constexpr int M = kRouteKeys / kThreads;
            uint64_t w[M];
            float b[M];
            auto lptr = [&](int m) {
                const int i = min(tid + m * nthr, items - 1);
                return logits + (size_t)(t0 + i / E) * E + i % E;
            };
            auto lneed = [&](int m) { return tid + m * nthr < items; };
#pragma unroll
            for (int m = 0; m < M; m++) {
                if (lneed(m)) {
                    w[m] = ld_sync(lptr(m));
                    b[m] = bias ? bias[(tid + m * nthr) % E] : 0.f;
                }
            }
            if (poll < 0) {
                settle(w, lptr, lneed, epoch, err);
            } else if (__syncthreads_or(!settle_for(w, lptr, lneed, epoch, poll))) {
                return 1;
            }
            float sg[M];  // sigmoid rule: the unbiased scores (the gates' numerators)
#pragma unroll
            for (int m = 0; m < M; m++) {
                if (lneed(m)) {
                    const int i = tid + m * nthr;
                    const float lg = __uint_as_float((unsigned)w[m]);
                    sg[m] = rule == kRouteSigmoid ? sigmoid_ref(lg) : 0.f;
                    float v = (rule == kRouteSigmoid ? sg[m] : lg) + b[m];
                    if (!(v == v)) v = -INFINITY;
                    if (v == 0.f) v = 0.f;  // -0 and +0 compare equal: one key
                    keys[i] = route_key(v, i % E);
                    if (MULTI && T > 1) ((LDS_AS float*)cnt)[i] = sg[m];
                }
            }
            __syncthreads();
            if (MULTI && T > 1 && E <= 16 * 16) {
                // 2'. several tokens: one 16-lane row per token takes the k largest keys one by one (a key's expert
                //     index makes every key distinct, so this is the same selection as counting ranks below), lane l of
                //     the row holding the keys of experts l, l + 16, ...; the row's maximum takes four DPP moves and no
                //     cross-row step, and the taken key is zeroed (every real key is nonzero)
                if (E <= 8 * 16) select_rows<8>(rt, keys, (const LDS_AS float*)cnt, t0, nt, E, k, rule);
                else select_rows<16>(rt, keys, (const LDS_AS float*)cnt, t0, nt, E, k, rule);
                __syncthreads();
            } else {
            // 2. ranks: work item (part p, item i) counts the keys of experts [p E / parts, (p + 1) E / parts) above
            //    key i; parts spread a small pass over the whole workgroup
            int parts = 1;  // a power of two dividing E
            while (parts < 8 && items * parts * 2 <= nthr && E % (parts * 2) == 0) parts *= 2;
            const int span = E / parts;  // keys compared per work item: the same count in every lane
            for (int wi = tid; wi < items * parts; wi += nthr) {
                const int p = wi / items, i = wi - p * items;
                const int tl = i / E;
                const uint64_t ki = keys[i];
                const LDS_AS uint64_t* kr = keys + tl * E + p * span;
                int c = 0, j = 0;
                for (; j + 8 <= span; j += 8) {  // 8 shared-memory reads in flight, then 8 compares
                    uint64_t kv[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) kv[u] = kr[j + u];
#pragma unroll
                    for (int u = 0; u < 8; u++) c += kv[u] > ki;
                }
                for (; j < span; j++) c += kr[j] > ki;
                cnt[wi] = c;
            }
            __syncthreads();
            // 3. the k best of each token, in rank order (the gate slot holds the score until step 4: the biased
            //    score for softmax, the unbiased sigmoid for sigmoid)
#pragma unroll
            for (int m = 0; m < M; m++) {
                const int i = tid + m * nthr;
                if (i < items) {
                    int r = 0;
                    for (int p = 0; p < parts; p++) r += cnt[p * items + i];
                    if (r < k) {
                        const int t = t0 + i / E;
                        rt->id[t * k + r] = i % E;
                        rt->gate[t * k + r] = rule == kRouteSigmoid ? sg[m] : route_key_score(keys[i]);
                    }
                }
            }
            __syncthreads();
            }
            // 4. gates, one wavefront per token, lane r holding rank r
            const int wave = wave_id(), lane = tid & 63;
            for (int tl = wave; tl < nt; tl += nthr / 64) {
                const int t = t0 + tl;
                const float sc = lane < k ? rt->gate[t * k + lane] : 0.f;
                if (rule == kRouteSigmoid) {
                    float tot = 0.f;
                    for (int q = 0; q < keep; q++) tot += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc), q));
                    tot = tot + 1e-20f;
                    if (lane < k) rt->gate[t * k + lane] = lane < keep ? sc / tot : 0.f;
                } else {
                    const float top = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc), 0));
                    const float ex = expf(sc - top);
                    float tot = 0.f;
                    for (int q = 0; q < keep; q++) tot += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), q));
                    if (lane < k) rt->gate[t * k + lane] = lane < keep ? ex / tot : 0.f;
                }
                if (T == 1) {  // one token's k distinct experts: slot n_shared + r holds rank r (closed-form grouping)
                    if (lane < keep) {
                        const int sl = n_shared + lane;
                        rt->slot_e[sl] = (short)rt->id[lane];
                        rt->slot_n[sl] = 1;
                        rt->slot_p[sl][0] = (unsigned char)lane;
                        rt->slot_pair[sl] = (short)sl;
                    }
                    if (lane < n_shared) {
                        rt->slot_e[lane] = (short)(-1 - lane);
                        rt->slot_n[lane] = 1;
                        rt->slot_p[lane][0] = 0;
                        rt->slot_pair[lane] = (short)lane;
                    }
                    if (lane == 0) {
                        rt->nslot = n_shared + keep;
                        rt->err = 0;
                    }
                }
            }
            __syncthreads();  // keys / cnt are reused by the next pass
        }
    } else {
        for (int p = tid; p < T * k; p += nthr) {  // the caller's routing, written before this launch
            int e = ids_in[p];
            if (e < -1 || e >= E) {  // out of range: flag and drop the entry
                bad = 1;
                e = -1;
            }
            rt->id[p] = e;
            rt->gate[p] = gates_in[p];
        }
    }
    if (do_topk && T == 1) {  // grouped above
        __syncthreads();
        return 0;
    }
    bad = __syncthreads_or(bad);
    // Grouping: entry p = t * keep + r (n = T * keep <= 128).  A slot's number counts the first occurrences before its
    // own first occurrence.
    const int n = T * keep;
    if (MULTI && do_topk) {
        // The selection's entries: distinct experts within a token, every id in [0, E).  Per expert, the tokens that
        // hold it (a bit mask) and its first entry, by shared-memory atomics; first occurrences are counted from two
        // wave ballots.
        LDS_AS unsigned* tmask = (LDS_AS unsigned*)scr;
        LDS_AS unsigned* firstp = tmask + kMaxExperts;
        LDS_AS uint64_t* fmask = (LDS_AS uint64_t*)(firstp + kMaxExperts);
        for (int e = tid; e < E; e += nthr) {
            tmask[e] = 0u;
            firstp[e] = ~0u;
        }
        __syncthreads();
        int e = 0, t = 0;
        if (tid < n) {
            t = tid / keep;
            e = rt->id[t * k + tid - t * keep];
            __hip_atomic_fetch_or(&tmask[e], 1u << t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            __hip_atomic_fetch_min(&firstp[e], (unsigned)tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        __syncthreads();
        const bool isfirst = tid < n && firstp[e] == (unsigned)tid;
        const uint64_t bm = __ballot(isfirst);
        if ((tid & 63) == 0 && tid < 128) fmask[tid >> 6] = bm;
        __syncthreads();
        const uint64_t m0 = fmask[0], m1 = fmask[1];
        if (tid < n) {
            const unsigned f = firstp[e], tm = tmask[e];
            const int before =
                f < 64 ? __popcll(m0 & ((1ull << f) - 1)) : __popcll(m0) + __popcll(m1 & ((1ull << (f - 64)) - 1));
            const int slot = n_shared + before;
            if (isfirst) {
                rt->slot_e[slot] = (short)e;
                rt->slot_n[slot] = (unsigned char)__popc(tm);
            }
            rt->slot_p[slot][__popc(tm & ((1u << t) - 1))] = (unsigned char)tid;
        }
        if (tid == 0) {
            rt->nslot = n_shared + __popcll(m0) + __popcll(m1);
            rt->err = bad;
        }
    } else {
        // The caller's entries (ids may repeat within a token): compared through shared-memory broadcasts.
        LDS_AS int* ent = (LDS_AS int*)scr;  // entry -> expert, padded with -2 to a multiple of 4
        LDS_AS int* fst = ent + 128;         // 1 where an entry is its expert's first occurrence
        const int n4 = (n + 3) & ~3;
        int my_e = -1, first = 0, pos = 0, c = 0;
        if (tid < n4) {
            my_e = tid < n ? rt->id[(tid / keep) * k + tid % keep] : -2;
            ent[tid] = my_e;
        }
        __syncthreads();
        if (tid < n && my_e >= 0) {
            first = tid;
            for (int j = 0; j < n4; j += 4) {
                const i32x4 q = *(const LDS_AS i32x4*)(ent + j);
                const int v[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const bool hit = v[u] == my_e;
                    c += hit;
                    pos += hit && j + u < tid;
                    if (hit && j + u < first) first = j + u;
                }
            }
        }
        if (tid < n4) fst[tid] = tid < n && my_e >= 0 && first == tid;
        __syncthreads();
        int rep = 0;
        int before = 0;  // first occurrences before mine: a uniform loop over all entries
        for (int j = 0; j < n4; j += 4) {
            const i32x4 q = *(const LDS_AS i32x4*)(fst + j);
            before += (j < first ? q.x : 0) + (j + 1 < first ? q.y : 0) + (j + 2 < first ? q.z : 0) +
                      (j + 3 < first ? q.w : 0);
        }
        if (tid < n && my_e >= 0) {
            const int slot = n_shared + before;
            if (first == tid) {
                rt->slot_e[slot] = (short)my_e;
                rt->slot_n[slot] = (unsigned char)(c < T ? c : T);
            }
            if (pos < T) {
                rt->slot_p[slot][pos] = (unsigned char)tid;
            } else {  // an expert repeated within one token's ids: the extra entry is dropped
                rt->id[(tid / keep) * k + tid % keep] = -1;
                rep = 1;
            }
        }
        const int nfirst = __syncthreads_count(tid < n && my_e >= 0 && first == tid);
        rep = __syncthreads_or(rep);
        if (tid == 0) {
            rt->nslot = n_shared + nfirst;
            rt->err = rep ? 2 : bad;
        }
    }
    if (tid < n_shared) {
        rt->slot_e[tid] = (short)(-1 - tid);
        rt->slot_n[tid] = (unsigned char)T;
        rt->slot_pair[tid] = (short)(tid * T);
        for (int j = 0; j < T; j++) rt->slot_p[tid][j] = (unsigned char)j;
    }
    __syncthreads();
    // pair offsets of the routed slots: exclusive prefix sum of their token counts (lane i: slots i and 64 + i)
    if (tid < 64) {
        const int lane = tid;
        const int nr = rt->nslot - n_shared;
        const int c0 = lane < nr ? rt->slot_n[n_shared + lane] : 0, c1 = 64 + lane < nr ? rt->slot_n[n_shared + 64 + lane] : 0;
        int i0 = c0, i1 = c1;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int u0 = __shfl_up(i0, d, 64), u1 = __shfl_up(i1, d, 64);
            if (lane >= d) {
                i0 += u0;
                i1 += u1;
            }
        }
        const int tot0 = __shfl(i0, 63, 64);
        if (lane < nr) rt->slot_pair[n_shared + lane] = (short)(n_shared * T + i0 - c0);
        if (64 + lane < nr) rt->slot_pair[n_shared + 64 + lane] = (short)(n_shared * T + tot0 + i1 - c1);
    }
    __syncthreads();
    return 0;
}

// Write the routing outputs (ids / gates when computed here) and the global slot table used by the unfused kernels.
__device__ __forceinline__ void route_publish(const lds_RouteTab* rt, int T, int k, int keep, int n_shared, int do_topk,
                                              int32_t* __restrict__ ids, float* __restrict__ gates,
                                              Slots* __restrict__ slots) {
    const int tid = threadIdx.x;
    for (int p = tid; p < T * k; p += blockDim.x) {
        if (do_topk) {
            st_sync(&ids[p], (int32_t)rt->id[p]);
            st_sync(&gates[p], rt->gate[p]);
        }
        st_sync(&slots->vid[p], (int)rt->id[p]);
        st_sync(&slots->vgate[p], rt->gate[p]);
    }
    const int ns = rt->nslot;
    for (int i = tid; i < ns * kMaxTokens; i += blockDim.x) {
        const int s = i / kMaxTokens, j = i % kMaxTokens;
        if (j == 0) {
            st_sync(&slots->expert[s], (int)rt->slot_e[s]);
            st_sync(&slots->ntok[s], (int)rt->slot_n[s]);
            st_sync(&slots->pair[s], (int)rt->slot_pair[s]);
        }
        if (j < rt->slot_n[s]) {
            const int p = rt->slot_p[s][j];
            st_sync(&slots->tok[s][j], s < n_shared ? p : p / keep);
            st_sync(&slots->rank[s][j], s < n_shared ? -1 : p % keep);
        }
    }
    if (tid == 0) {
        st_sync(&slots->nslot, ns);
        st_sync(&slots->err, rt->err);
    }
}

// --------------------------------------------------------------------------------------------------------------------
// Unit: gate|up tile part.  Slot s, 32 f values = one 64-row tile (32 gate rows + their 32 up rows), K part kpi of
// kp (a.kps for a shared slot, a.kp for a routed one; chunks [kpi, kpi + 1) * H/8/kp), the 4 wavefronts splitting the
// part; act[s][j][f] = bf16(silu(g) * u) for
// the slot's tokens.  Sums: wavefronts in order within a part, then parts in order.  Parts below kp - 1 publish their
// partial sums to gpart; part kp - 1 (the tile's last unit in queue order) reads them back, finishes the tile and
// publishes act.  pair0: the slot's first (slot, token) pair, indexing gpart.
template <int N, bool Q8OK, bool MF = false>
__device__ __forceinline__ void gateup_core(const Lds& s, const ExpertArgs& a, int sl, int tile, int kpi, int e, int ntok,
                                            const int* tok, int pair0, uint64_t& stamp) {
    const int H = a.d.H, F = a.d.F, kp = e < 0 ? a.kps : a.kp, ntile = F / 32;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int nc = H / 8;
    int xoff[N];
#pragma unroll
    for (int j = 0; j < N; j++) xoff[j] = j < ntok ? tok[j] * nc : 0;
    const bool q8 = Q8OK && a.int8 && e >= 0;  // Q8OK false: no int8 code in this instantiation
    if constexpr (MF) {
        f32x4_t d[4] = {};
        const int xo = mfma_xoff<N>(xoff, ntok);
        if (!q8) {
            const uint16_t* base =
                e >= 0 ? a.L.gu + (size_t)e * a.d.gu_stride() : a.L.sgu + (size_t)(-1 - e) * a.d.gu_stride();
            const u32x4* t = reinterpret_cast<const u32x4*>(base) + (size_t)tile * nc * 64;
            const int cpw = nc / (kWaves * kp), c0 = (kpi * kWaves + wave) * cpw;
            MfmaStream<false> ms;
            ms.begin(t, c0, c0 + cpw);
            ms.run(s.xs, xo, d);
        } else {
            const int ncq = H / 16;
            const u32x4* t =
                reinterpret_cast<const u32x4*>(a.L.gu_q8 + (size_t)e * a.d.gu_stride()) + (size_t)tile * ncq * 64;
            const int cpw = ncq / (kWaves * kp), c0 = (kpi * kWaves + wave) * cpw;
            MfmaStream<true> ms;
            ms.begin(t, c0, c0 + cpw);
            ms.run(s.xs, xo, d);
        }
        reduce_waves_mfma<N>(s.red, d, ntok);
    } else {
        float acc[N];
#pragma unroll
        for (int j = 0; j < N; j++) acc[j] = 0.f;
        if (!q8) {
            const uint16_t* base =
                e >= 0 ? a.L.gu + (size_t)e * a.d.gu_stride() : a.L.sgu + (size_t)(-1 - e) * a.d.gu_stride();
            const u32x4* t = reinterpret_cast<const u32x4*>(base) + (size_t)tile * nc * 64;
            const int cpw = nc / (kWaves * kp), c0 = (kpi * kWaves + wave) * cpw;
            tile_stream<N, false>(t, c0, c0 + cpw, s.xs, xoff, acc);
        } else {
            const int ncq = H / 16;
            const u32x4* t =
                reinterpret_cast<const u32x4*>(a.L.gu_q8 + (size_t)e * a.d.gu_stride()) + (size_t)tile * ncq * 64;
            const int cpw = ncq / (kWaves * kp), c0 = (kpi * kWaves + wave) * cpw;
            tile_stream<N, true>(t, c0, c0 + cpw, s.xs, xoff, acc);
        }
        reduce_waves<N>(s.red, acc, N);
    }
    if (wave == 0) {
        uint64_t* gp0 = a.gpart + (((size_t)pair0 * ntile + tile) * kMaxKp) * 64 + lane;  // + (j*ntile*kMaxKp + q)*64
        if (kpi < kp - 1) {
#pragma unroll
            for (int j = 0; j < N; j++)
                if (j < ntok)
                    st_tag(gp0 + ((size_t)j * ntile * kMaxKp + kpi) * 64, a.epoch, __float_as_uint(s.red[j * 64 + lane]));
        } else {
            const float scale = q8 ? a.L.sc_q8[(size_t)e * (2 * F + H) + tile * 64 + lane] : 1.f;
            uint64_t w[N][kMaxKp - 1];  // the other parts' partials: all loads issued before any use
            auto gptr = [&](int j, int q) { return gp0 + ((size_t)(j < ntok ? j : 0) * ntile * kMaxKp + q) * 64; };
#pragma unroll
            for (int j = 0; j < N; j++)
#pragma unroll
                for (int q = 0; q < kMaxKp - 1; q++)
                    if (q < kp - 1) w[j][q] = ld_sync(gptr(j, q));
#pragma unroll
            for (int j = 0; j < N; j++) {
                settle(w[j], [&](int q) { return gptr(j, q); }, [&](int q) { return q < kp - 1; }, a.epoch, a.err);
                if (j == 0) stamp = __builtin_amdgcn_s_memrealtime();
                float v = 0.f;
#pragma unroll
                for (int q = 0; q < kMaxKp - 1; q++) {
                    if (q < kp - 1) {
                        const float pv = __uint_as_float((unsigned)w[j][q]);
                        v = q == 0 ? pv : v + pv;
                    }
                }
                v = kp > 1 ? v + s.red[j * 64 + lane] : s.red[j * 64 + lane];
                if (q8) v = v * scale;
                const float up = __shfl_down(v, 8, 64);  // gate row lane (bit 3 clear) meets its up row (lane + 8)
                const unsigned h = f2bf_dev(silu_mul(v, up));
                const unsigned h_next = __shfl_down(h, 1, 64);  // f + 1 lives in the next lane
                if (j < ntok && !gu_row_up(lane) && !(lane & 1))
                    st_tag(a.act + ((size_t)sl * a.d.max_t + j) * (F / 2) + gu_row_f(tile, lane) / 2, a.epoch,
                           h | (h_next << 16));
            }
        }
    }
    __syncthreads();  // s.red is reused by the next unit
}

// MFOK: the MFMA cores may be used (the unfused kernels; the fused kernel's register budget has no room for them).
template <int NT, bool Q8OK = true, bool MFOK = false>
__device__ __forceinline__ void gateup_unit(const Lds& s, const ExpertArgs& a, int sl, int tile, int kpi, int e, int ntok,
                                            const int* tok, int pair0, uint64_t& stamp) {
    if (ntok <= 1 || NT == 1) gateup_core<1, Q8OK>(s, a, sl, tile, kpi, e, ntok, tok, pair0, stamp);
    else if (ntok <= 2 || NT == 2) gateup_core<(NT < 2 ? NT : 2), Q8OK>(s, a, sl, tile, kpi, e, ntok, tok, pair0, stamp);
    else if (ntok <= 4 || NT == 4) gateup_core<(NT < 4 ? NT : 4), Q8OK>(s, a, sl, tile, kpi, e, ntok, tok, pair0, stamp);
    else if (ntok <= 8 || NT == 8) {
        if (MFOK && NT >= 8 && a.T >= 8)  // the batch >= 8 grouped case: MFMA
            gateup_core<(NT < 8 ? NT : 8), Q8OK, (MFOK && NT >= 8)>(s, a, sl, tile, kpi, e, ntok, tok, pair0, stamp);
        else
            gateup_core<(NT < 8 ? NT : 8), Q8OK>(s, a, sl, tile, kpi, e, ntok, tok, pair0, stamp);
    } else {
        gateup_core<NT, Q8OK, (MFOK && NT > 8)>(s, a, sl, tile, kpi, e, ntok, tok, pair0, stamp);  // > 8 tokens
    }
}

// Unit: down tile.  Slot s, 64 output rows over K = F; y written unweighted to ypart[t][q][h] with q = s for a shared
// slot and n_shared + rank for a routed one.
// The fused kernel's combiner of a tile (the last slot's down unit) folds the combine into its own unit when every
// (term, token, row) word of the tile fits kCombW words per thread: it loads the other units' outputs right after
// its stream, before its own stores, and takes its own terms from shared memory, so no store round trip sits on the
// kernel's last path.
constexpr int kCombW = 3;
// Trace stamps of a down unit (taken when `on`): act rows staged, weight stream done, a combining unit's other
// terms in.
struct DownStamps {
    bool on = false;
    uint64_t aux = 0, run = 0, ready = 0;
};
__device__ __forceinline__ bool combine_in_unit(const ExpertArgs& a) {
    return a.T * 64 * (a.d.n_shared + a.d.k) <= kCombW * kThreads;
}

template <int N, bool Q8OK, bool MF = false>
__device__ __forceinline__ void down_core(const Lds& s, const ExpertArgs& a, int sl, int ht, int e, int ntok, const int* tok,
                          const int* rank, DownStamps& st, bool comb, const lds_RouteTab* crt) {
    const int H = a.d.H, F = a.d.F;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int nc = F / 8;
    // the weight stream starts first: its first bank is in flight while the act rows are polled (a second bank
    // here, or the act loads ahead of the bank, measured slower)
    const bool q8 = Q8OK && a.int8 && e >= 0;  // Q8OK false: no int8 code in this instantiation
    // (MF: the MFMA streams; otherwise the dot2 streams)
    TileStream<MF ? 1 : N, false, MF ? 1 : MOE_DN_DEPTH> tb;
    TileStream<MF ? 1 : N, true, MF ? 1 : MOE_DN_DEPTH> tq;
    MfmaStream<false> mb;
    MfmaStream<true> mq;
    if (!q8) {
        const uint16_t* base =
            e >= 0 ? a.L.dn + (size_t)e * a.d.dn_stride() : a.L.sdn + (size_t)(-1 - e) * a.d.dn_stride();
        const u32x4* t = reinterpret_cast<const u32x4*>(base) + (size_t)ht * nc * 64;
        const int cpw = nc / kWaves;
        if constexpr (MF) mb.begin(t, wave * cpw, (wave + 1) * cpw);
        else tb.begin(t, wave * cpw, (wave + 1) * cpw);
    } else {
        const int ncq = F / 16;
        const u32x4* t = reinterpret_cast<const u32x4*>(a.L.dn_q8 + (size_t)e * a.d.dn_stride()) + (size_t)ht * ncq * 64;
        const int cpw = ncq / kWaves;
        if constexpr (MF) mq.begin(t, wave * cpw, (wave + 1) * cpw);
        else tq.begin(t, wave * cpw, (wave + 1) * cpw);
    }
    // the slot's act rows, published by the gate|up tiles' last parts: 8 loads per thread in flight, then polled
    const uint64_t* src = a.act + (size_t)sl * a.d.max_t * (F / 2);
    LDS_AS unsigned* dst = (LDS_AS unsigned*)s.as;
    const int na = ntok * (F / 2);
    for (int i0 = 0; i0 < na; i0 += 8 * (int)blockDim.x) {
        uint64_t w[8];
        auto aptr = [&](int m) { return src + i0 + m * (int)blockDim.x + (int)threadIdx.x; };
        auto aneed = [&](int m) { return i0 + m * (int)blockDim.x + (int)threadIdx.x < na; };
#pragma unroll
        for (int m = 0; m < 8; m++)
            if (aneed(m)) w[m] = ld_sync(aptr(m));
        settle(w, aptr, aneed, a.epoch, a.err);
#pragma unroll
        for (int m = 0; m < 8; m++)
            if (aneed(m)) dst[i0 + m * (int)blockDim.x + (int)threadIdx.x] = (unsigned)w[m];
    }
    __syncthreads();
    if (st.on) st.aux = __builtin_amdgcn_s_memrealtime();
    int xoff[N];
#pragma unroll
    for (int j = 0; j < N; j++) xoff[j] = j < ntok ? j * nc : 0;
    float acc[N];
#pragma unroll
    for (int j = 0; j < N; j++) acc[j] = 0.f;
    f32x4_t d[4] = {};
    if constexpr (MF) {
        const int xo = mfma_xoff<N>(xoff, ntok);
        if (!q8) mb.run(s.as, xo, d);
        else mq.run(s.as, xo, d);
    } else {
        if (!q8) tb.run(s.as, xoff, acc);
        else tq.run(s.as, xoff, acc);
    }
    if (st.on) st.run = __builtin_amdgcn_s_memrealtime();
    const int S = a.d.n_shared, k = a.d.k, kq = S + k, ne = a.T * 64;
    // combiner (comb; crt is its routing table): word w = q * ne + t * 64 + row of the tile; this unit's own terms
    // come from its reduction.  (An LDS pointer can sit at address 0: never test one against null.)
    auto own = [&](int q, int t) {
        bool o = false;
#pragma unroll
        for (int j = 0; j < N; j++) o = o || (j < ntok && tok[j] == t && (e < 0 ? sl : S + rank[j]) == q);
        return o;
    };
    auto cneed = [&](int m) {
        const int w = (int)threadIdx.x + m * (int)blockDim.x;
        if (w >= kq * ne) return false;
        const int q = w / ne, t = (w % ne) / 64;
        const bool live = q < S ? q < a.n_shared : (q - S < a.keep && crt->id[t * k + q - S] >= 0);
        return live && !own(q, t);
    };
    auto cptr = [&](int m) {
        const int w = (int)threadIdx.x + m * (int)blockDim.x;
        const int q = w / ne, i = w % ne;
        return a.ypart + ((size_t)(i / 64) * kq + q) * H + ht * 64 + i % 64;
    };
    uint64_t cw[kCombW];
    if (comb) {
#pragma unroll
        for (int m = 0; m < kCombW; m++)
            if (cneed(m)) cw[m] = ld_sync(cptr(m));
    }
    if constexpr (MF) reduce_waves_mfma<N>(s.red, d, ntok);
    else reduce_waves<N>(s.red, acc, N);
    const float scale = q8 ? a.L.sc_q8[(size_t)e * (2 * F + H) + 2 * F + ht * 64 + lane] : 1.f;
    if (wave == 0 && !comb) {  // a combiner's own outputs are read by no other unit
        const int h = ht * 64 + lane;
#pragma unroll
        for (int j = 0; j < N; j++) {
            if (j < ntok) {
                const int q = e < 0 ? sl : S + rank[j];
                float y = s.red[j * 64 + lane];
                if (q8) y = y * scale;
                st_tag(&a.ypart[((size_t)tok[j] * kq + q) * H + h], a.epoch, __float_as_uint(y));
            }
        }
    }
    if (comb) {
        lds_float* cv = (lds_float*)s.as;  // [kq][T][64] terms of the tile
        settle(cw, cptr, cneed, a.epoch, a.err);
        if (st.on) st.ready = __builtin_amdgcn_s_memrealtime();
#pragma unroll
        for (int m = 0; m < kCombW; m++) {
            const int w = (int)threadIdx.x + m * (int)blockDim.x;
            if (cneed(m)) cv[w] = __uint_as_float((unsigned)cw[m]);
        }
        if (wave == 0) {
#pragma unroll
            for (int j = 0; j < N; j++) {
                if (j < ntok) {
                    float y = s.red[j * 64 + lane];
                    if (q8) y = y * scale;
                    cv[(e < 0 ? sl : S + rank[j]) * ne + tok[j] * 64 + lane] = y;
                }
            }
        }
        __syncthreads();
        for (int i = threadIdx.x; i < ne; i += blockDim.x) {  // fixed order: shared terms, then ranks
            const int t = i / 64;
            const size_t o = (size_t)t * H + ht * 64 + i % 64;
            float acc2 = a.accumulate ? a.out[o] : 0.f, acc_s = 0.f, acc_r = 0.f;
            for (int q = 0; q < kq; q++) {
                if (q < S) {
                    if (q < a.n_shared) {
                        acc2 = acc2 + cv[q * ne + i];
                        acc_s = acc_s + cv[q * ne + i];
                    }
                } else if (q - S < a.keep && crt->id[t * k + q - S] >= 0) {
                    acc2 = fmaf(crt->gate[t * k + q - S], cv[q * ne + i], acc2);
                    acc_r = fmaf(crt->gate[t * k + q - S], cv[q * ne + i], acc_r);
                }
            }
            combine_store(a, o, acc2, acc_s, acc_r);
        }
    }
    __syncthreads();  // s.as / s.red are reused by the next unit
}

template <int NT, bool Q8OK = true, bool MFOK = false>
__device__ __forceinline__ void down_unit(const Lds& s, const ExpertArgs& a, int sl, int ht, int e, int ntok, const int* tok,
                          const int* rank, DownStamps& st, bool comb = false, const lds_RouteTab* crt = nullptr) {
    if (ntok <= 1 || NT == 1) down_core<1, Q8OK>(s, a, sl, ht, e, ntok, tok, rank, st, comb, crt);
    else if (ntok <= 2 || NT == 2) down_core<(NT < 2 ? NT : 2), Q8OK>(s, a, sl, ht, e, ntok, tok, rank, st, comb, crt);
    else if (ntok <= 4 || NT == 4) down_core<(NT < 4 ? NT : 4), Q8OK>(s, a, sl, ht, e, ntok, tok, rank, st, comb, crt);
    else if (ntok <= 8 || NT == 8) {
        if (MFOK && NT >= 8 && a.T >= 8)  // the batch >= 8 grouped case: MFMA
            down_core<(NT < 8 ? NT : 8), Q8OK, (MFOK && NT >= 8)>(s, a, sl, ht, e, ntok, tok, rank, st, comb, crt);
        else
            down_core<(NT < 8 ? NT : 8), Q8OK>(s, a, sl, ht, e, ntok, tok, rank, st, comb, crt);
    } else {
        down_core<NT, Q8OK, (MFOK && NT > 8)>(s, a, sl, ht, e, ntok, tok, rank, st, comb, crt);  // > 8 tokens
    }
}

// Combine 64-row output tile ht of every token from the routing table rt: (out or 0) + shared terms in order + gate *
// routed terms in rank order (ranks with id -1 produced no output).  The down outputs are polled (tagged words).
__device__ __forceinline__ void combine_tile(const ExpertArgs& a, const lds_RouteTab* rt, int ht) {
    const int H = a.d.H, k = a.d.k, S = a.d.n_shared, kq = S + k;
    for (int i = threadIdx.x; i < a.T * 64; i += blockDim.x) {
        const int t = i / 64, h = ht * 64 + i % 64;
        const uint64_t* yp = a.ypart + (size_t)t * kq * H + h;  // + q * H
        uint64_t w[kMaxShared + kMaxTopk];
        auto yptr = [&](int q) { return yp + (size_t)q * H; };
        auto ylive = [&](int q) {
            return q < kq && (q < S ? q < a.n_shared : (q - S < a.keep && rt->id[t * k + q - S] >= 0));
        };
#pragma unroll
        for (int q = 0; q < kMaxShared + kMaxTopk; q++)  // every live term's load issued before any use
            if (ylive(q)) w[q] = ld_sync(yptr(q));
        settle(w, yptr, ylive, a.epoch, a.err);
        const size_t o = (size_t)t * H + h;
        float acc = a.accumulate ? a.out[o] : 0.f, acc_s = 0.f, acc_r = 0.f;
#pragma unroll
        for (int q = 0; q < kMaxShared + kMaxTopk; q++) {  // q < S: shared expert q; else rank q - S
            if (q >= kq) continue;
            const float y = __uint_as_float((unsigned)w[q]);
            if (q < S) {
                if (q < a.n_shared) {
                    acc = acc + y;
                    acc_s = acc_s + y;
                }
            } else if (q - S < a.keep && rt->id[t * k + q - S] >= 0) {
                acc = fmaf(rt->gate[t * k + q - S], y, acc);
                acc_r = fmaf(rt->gate[t * k + q - S], y, acc_r);
            }
        }
        combine_store(a, o, acc, acc_s, acc_r);
    }
}

// One slot of this workgroup's routing table.
template <int NT>
struct SlotRt {
    int expert, ntok, pair0;
    int tok[NT], rank[NT];
    __device__ __forceinline__ void load(const lds_RouteTab* rt, int sl, int n_shared, int keep) {
        expert = rt->slot_e[sl];
        ntok = rt->slot_n[sl];
        pair0 = rt->slot_pair[sl];
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int p = j < ntok ? rt->slot_p[sl][j] : 0;  // entries past ntok: keep indices in range
            tok[j] = sl < n_shared ? p : p / keep;
            rank[j] = sl < n_shared ? -1 : p % keep;
        }
    }
};

// Coherent snapshot of one slot of the table the route unit published.
template <int NT>
struct SlotView {
    int expert, ntok, pair0;
    int tok[NT], rank[NT];
    __device__ __forceinline__ void load(const Slots* sp, int sl) {  // independent loads: one round trip
        expert = ld_sync(&sp->expert[sl]);
        ntok = ld_sync(&sp->ntok[sl]);
        pair0 = ld_sync(&sp->pair[sl]);
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

// ====================================================================================================================
// Unfused path: one kernel per phase (stream order provides the dependencies; the tagged reads succeed at once).
#if MOE_COMMON
__global__ __launch_bounds__(256) void router_kernel(LayerPtrs L, Dims d, int T, StageSrc in,
                                                     uint64_t* __restrict__ logits, float* __restrict__ logits_out,
                                                     unsigned epoch) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    const Lds s = lds_carve(lds_raw, T, 1, d.H, d.F, d.E);
    const int e0 = blockIdx.x * kRouterRows, t0 = blockIdx.y * kRouterTG;
    uint64_t u0 = 0, u1 = 0;  // stamps (unused)
    if (T <= 1) router_unit<1>(s, L.wr, e0, d.E, d.H, T, logits, logits_out, epoch, true, in, false, u0, u1);
    else router_unit<kRouterTG>(s, L.wr, e0, d.E, d.H, T, logits, logits_out, epoch, true, in, false, u0, u1, t0);
}

__global__ __launch_bounds__(kTopkThreads) void topk_group_kernel(LayerPtrs L, Dims d, int T, int keep, int n_shared,
                                                         int do_topk, int rule, const uint64_t* __restrict__ logits,
                                                         unsigned epoch, unsigned* err, int32_t* __restrict__ ids,
                                                         float* __restrict__ gates, Slots* __restrict__ slots) {
    __shared__ RouteTab rt_mem;
    __shared__ __align__(16) unsigned char scr_mem[kRouteScratchBytes];
    lds_RouteTab* rt = (lds_RouteTab*)&rt_mem;
    route_local(rt, (LDS_AS unsigned char*)scr_mem, logits, epoch, err, L.bias, ids, gates, T, d.E, d.k, keep, n_shared,
                do_topk, rule, -1);
    route_publish(rt, T, d.k, keep, n_shared, do_topk, ids, gates, slots);
}

#endif  // MOE_COMMON

// The unfused gate|up kernel's shared memory: the staged tokens and the cross-wave reduction only (its units read no
// act rows), so that two workgroups fit on a CU at batch 8 (2 x 72 KiB).
__host__ __device__ inline size_t gu_lds_bytes(int T, int NT, int H) {
    return (size_t)T * (H / 8) * 16 + (size_t)4 * NT * 64 * 4;
}

template <int NT>
__global__ __launch_bounds__(256) void gateup_kernel(ExpertArgs a, Sync* sy) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    Lds s;
    s.xs = (lds_u32x4*)(LDS_AS unsigned char*)lds_raw;
    s.as = nullptr;
    s.red = (lds_float*)((LDS_AS unsigned char*)lds_raw + (size_t)a.T * (a.d.H / 8) * 16);
    s.xf = nullptr;
    if (blockIdx.x == 0 && threadIdx.x < 2) st_sync(&sy->next_unit[threadIdx.x * kSyncPad], 0u);  // fused queue heads
    const int ntile = a.d.F / 32, S = a.d.n_shared, gs = ntile * a.kps, g = ntile * a.kp;
    const int b = (int)blockIdx.x, shared = b < S * gs;  // shared slots' parts first
    const int kp = shared ? a.kps : a.kp, ub = shared ? b : b - S * gs;
    const int sl = shared ? b / gs : S + ub / g, tile = (ub % (shared ? gs : g)) / kp, kpi = ub % kp;
    if (sl >= a.slots->nslot || (sl < a.d.n_shared && sl >= a.n_shared)) return;  // unused / left out
    SlotView<NT> v;
    v.load(a.slots, sl);
    stage_in(s, a.in, a.T, a.d.H);
    uint64_t stamp = 0;
    gateup_unit<NT, true, true>(s, a, sl, tile, kpi, v.expert, v.ntok, v.tok, v.pair0, stamp);
}

// Routing table of the combine, from the published slot table.
__device__ __forceinline__ void load_combine_table(lds_RouteTab* rt, const Slots* sp, int T, int k) {
    for (int p = threadIdx.x; p < T * k; p += blockDim.x) {
        rt->id[p] = sp->vid[p];
        rt->gate[p] = sp->vgate[p];
    }
    __syncthreads();
}

// The 8-token bucket (the batch >= 8 grouped case) is held to two waves per SIMD: at one (312 registers) each
// workgroup's act round trip left its CU idle; with two (256 registers, 256 bytes of scratch) Solar batch 8 went from
// 204-208 to 192.6 us per call, the same bits.
template <int NT>
__global__ __launch_bounds__(256, NT == 8 ? 2 : 1) void down_kernel(ExpertArgs a) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    __shared__ RouteTab rt_mem;
    lds_RouteTab* rt = (lds_RouteTab*)&rt_mem;
    const Lds s = lds_carve(lds_raw, 0, NT, a.d.H, a.d.F, a.d.E);
    const int nht = a.d.H / 64;
    const int sl = blockIdx.x / nht, ht = blockIdx.x % nht;
    if (sl < a.slots->nslot && (sl >= a.d.n_shared || sl < a.n_shared)) {  // else unused / left out
        SlotView<NT> v;
        v.load(a.slots, sl);
        DownStamps stamp;
        down_unit<NT, true, true>(s, a, sl, ht, v.expert, v.ntok, v.tok, v.rank, stamp);
    }
    if (sl == a.maxs - 1) {  // the last slot's unit of each tile combines it
        load_combine_table(rt, a.slots, a.T, a.d.k);
        combine_tile(a, rt, ht);
    }
}

// ====================================================================================================================
// Fused path: one persistent kernel walks the unit list
//   [router units][route publisher][shared slots' gate|up parts][the first routed gate|up blocks]
//   [shared slots' downs][more routed gate|up blocks, then gate|up and down blocks][remaining routed downs]
// A slot's gate|up block holds its F/32 tiles x kp K parts (parts of a tile adjacent, the finishing part last); its
// down block holds its H/64 down tiles.  Routed slot s's gate|up block is followed by routed slot (s - lag)'s down
// block, so a down unit is handed out about lag blocks after the gate|up units it reads.  Workgroup b runs units b and grid + b
// first; further units come from a work queue (a counter handed out in ascending order, fetched while the current
// unit runs).  A unit only ever waits for data produced by units of smaller index, and the smallest unfinished unit
// always has a running workgroup on it, so the grid needs no co-residency guarantee (a plain launch); every wait is
// also bounded.  Each
// workgroup that needs the routing computes it into its own shared-memory table from the tagged logits; the
// publisher unit only writes ids / gates / the slot table for the caller.  The last slot's down unit of each 64-row
// tile combines that tile.
struct UnitRef {
    int kind;  // 0 router, 1 publisher, 2 gate|up part, 3 down tile
    int sl, idx;
};
__device__ __forceinline__ UnitRef decode_unit(int u, int uR, int S, int M, int gs, int g, int nht, int lag, int grid) {
    if (u < uR) return {0, 0, u};
    u -= uR;
    if (u < 1) return {1, 0, 0};
    u -= 1;
    if (u < S * gs) return {2, u / gs, u % gs};  // shared slots' gate|up parts (gs per slot)
    u -= S * gs;
    const int Mr = M - S;               // routed slots S .. M - 1, numbered r = slot - S below
    const int n0 = min(lag, Mr);        // gate|up-only blocks: r = 0 .. n0 - 1
    // The shared slots' downs come after the first nx routed gate|up blocks, about 1.25 grids of units: queued
    // right after the shared gate|up parts, their workgroups sat waiting for the shared act rows while routed parts
    // waited for workgroups (0.7 us slower at Solar batch 1, 2 us for int8); after 4 of Solar's 8 blocks measured
    // 0.35 us faster than after all 8, after 2 or 6 slower.
    const int nx = min(n0, max(1, (5 * grid / 4 + g - 1) / g));
    if (u < nx * g) return {2, S + u / g, u % g};
    u -= nx * g;
    if (u < S * nht) return {3, u / nht, u % nht};
    u -= S * nht;
    if (u < (n0 - nx) * g) return {2, S + nx + u / g, u % g};
    u -= (n0 - nx) * g;
    const int n1 = max(0, Mr - lag);    // paired steps i: gate|up of r = lag + i, then down of r = i
    if (u < n1 * (g + nht)) {
        const int i = u / (g + nht), w = u % (g + nht);
        return w < g ? UnitRef{2, S + lag + i, w} : UnitRef{3, S + i, w - g};
    }
    u -= n1 * (g + nht);
    return {3, S + n1 + u / nht, u % nht};  // downs of the last routed slots
}

template <int NT, bool Q8OK>
__global__ __launch_bounds__(256) void fused_layer_kernel(FusedArgs f) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    __shared__ RouteTab rt_mem;
    __shared__ int s_unit, s_routed, s_staged;
    lds_RouteTab* rt = (lds_RouteTab*)&rt_mem;
    const ExpertArgs& a = f.e;
    const Lds s = lds_carve(lds_raw, a.T, NT, a.d.H, a.d.F, a.d.E);
    Sync* sy = f.sync;
    const int H = a.d.H, F = a.d.F, S = a.d.n_shared;
    const int nRG = (a.d.E + kRouterRows - 1) / kRouterRows;  // router row groups (router unit u: u % nRG, u / nRG)
    const int ntile = F / 32, nht = H / 64, g = ntile * a.kp, gs = ntile * a.kps;
    const int maxs = a.maxs;
    // The list is laid out for maxs slots; with 2 to 8 tokens, once the routing is known every workgroup trims
    // it to the live slots (rt->nslot: tokens sharing experts leave many of the S + T * keep slots empty), the same
    // bits in every workgroup, so the units past the live slots are never handed out (Solar batch 8: 268 -> 208 us
    // per call).  Units past the routing-independent prefix (router units, publisher, shared gate|up parts) are then
    // decoded only once the routing is known.
    const int prefix = f.nR + 1 + S * gs;
    int M = maxs, uEnd = fused_units(f.nR, maxs, S, F, H, a.kp, a.kps);
    const int ph = f.phase & 1;
    unsigned* queue = &sy->next_unit[ph * kSyncPad];
    if (threadIdx.x == 0) {
        s_routed = 0;
        s_staged = 0;
        if (blockIdx.x == 0) st_sync(&sy->next_unit[(ph ^ 1) * kSyncPad], 0u);  // the next launch's head
    }
    __syncthreads();
    auto ensure_staged = [&]() __attribute__((always_inline)) {
        if (!s_staged) {
            stage_in(s, a.in, a.T, H);
            if (threadIdx.x == 0) s_staged = 1;
            __syncthreads();
        }
    };
    auto ensure_routed = [&]() __attribute__((always_inline)) {
        if (!s_routed) {
            if (route_local<(NT > 1)>(rt, (LDS_AS unsigned char*)s.as, f.logits, a.epoch, a.err, a.L.bias, a.ids, a.gates, a.T,
                            a.d.E, a.d.k, a.keep, S, f.do_topk, f.rule, f.do_topk ? f.router_poll : -1)) {
                // Router logits still missing after the bounded wait: a router unit's workgroup is not running (the
                // grid is not all resident).  Compute every router row here (the same bits: rewriting a logit that
                // its unit also writes is harmless), then wait for them without a limit.
                ensure_staged();
                uint64_t u0 = 0, u1 = 0;  // stamps (unused)
                for (int r = 0; r < f.nR; r++) {
                    if (NT == 1)
                        router_unit<1>(s, a.L.wr, r * kRouterRows, a.d.E, H, a.T, f.logits, nullptr, a.epoch, false,
                                       a.in, false, u0, u1);
                    else
                        router_unit<kRouterTG>(s, a.L.wr, (r % nRG) * kRouterRows, a.d.E, H, a.T, f.logits, nullptr,
                                               a.epoch, false, a.in, false, u0, u1, (r / nRG) * kRouterTG);
                }
                __syncthreads();
                route_local<(NT > 1)>(rt, (LDS_AS unsigned char*)s.as, f.logits, a.epoch, a.err, a.L.bias, a.ids, a.gates, a.T,
                            a.d.E, a.d.k, a.keep, S, f.do_topk, f.rule, -1);
            }
            if (threadIdx.x == 0) s_routed = 1;
            __syncthreads();
        }
    };
    uint64_t t_start = 0;
    int next = 0;  // thread 0: the unit after the current one
    // Every unit is handed out by the queue in ascending order, each to a workgroup that is running, except router
    // unit b, which workgroup b (b < nS) runs first: a unit only waits for units of smaller index, and the smallest
    // unfinished queue unit always has a running workgroup, so the grid needs no co-residency; a missing router unit
    // is covered by ensure_routed.  The index after the current unit is fetched while the current one runs.
    const int grid = (int)gridDim.x, nS = min(grid, f.nR);
    auto claim = [&]() __attribute__((always_inline)) {
        return nS + (int)__hip_atomic_fetch_add(queue, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    if ((int)blockIdx.x >= nS) {
        if (threadIdx.x == 0) s_unit = claim();
        __syncthreads();
    }
    for (int u = (int)blockIdx.x < nS ? (int)blockIdx.x : __builtin_amdgcn_readfirstlane(s_unit); u < uEnd;) {
        if (threadIdx.x == 0) {
            next = claim();
            if (f.trace) t_start = __builtin_amdgcn_s_memrealtime();
        }
        if (NT > 1 && u >= prefix) {  // one token: its keep experts are distinct, every slot is live
            ensure_routed();
            M = max(rt->nslot, 1);
            uEnd = fused_units(f.nR, M, S, F, H, a.kp, a.kps);
            if (u >= uEnd) break;  // the claimed units are past the live slots: nothing is left for this workgroup
        }
        const UnitRef ur = decode_unit(u, f.nR, S, M, gs, g, nht, f.lag, grid);
        uint64_t t_ready = 0, t_aux = 0, t_aux2 = 0;
        uint64_t& aux = t_aux;
        if (ur.kind == 0) {
            const bool stage = !s_staged;
            if (NT == 1)
                router_unit<1>(s, a.L.wr, ur.idx * kRouterRows, a.d.E, H, a.T, f.logits, nullptr, a.epoch, stage, a.in,
                               f.trace != nullptr, t_aux, t_aux2);
            else
                router_unit<kRouterTG>(s, a.L.wr, (ur.idx % nRG) * kRouterRows, a.d.E, H, a.T, f.logits, nullptr,
                                       a.epoch, stage, a.in, f.trace != nullptr, t_aux, t_aux2,
                                       (ur.idx / nRG) * kRouterTG);
            if (stage && threadIdx.x == 0) s_staged = 1;
        } else if (ur.kind == 1) {
            ensure_routed();
            if (f.trace) t_ready = __builtin_amdgcn_s_memrealtime();
            route_publish(rt, a.T, a.d.k, a.keep, S, f.do_topk, a.ids, a.gates, a.slots);
        } else if (ur.kind == 2) {
            const int sl = ur.sl, kp = sl < S ? a.kps : a.kp, tile = ur.idx / kp, kpi = ur.idx % kp;
            ensure_staged();  // x first: its load overlaps the wait for the routing
            if (sl < S) {  // shared slot: all tokens in order, no routing dependency
                if (f.shared_waits) ensure_routed();  // optional: keep the memory system quiet while routing
                if (sl < a.n_shared) {
                    int tok[NT];
#pragma unroll
                    for (int j = 0; j < NT; j++) tok[j] = j;
                    gateup_unit<NT, Q8OK>(s, a, sl, tile, kpi, -1 - sl, a.T, tok, sl * a.T, aux);
                }
            } else {
                ensure_routed();
                if (f.trace) t_ready = __builtin_amdgcn_s_memrealtime();
                if (sl < rt->nslot) {
                    SlotRt<NT> v;
                    v.load(rt, sl, S, a.keep);
                    gateup_unit<NT, Q8OK>(s, a, sl, tile, kpi, v.expert, v.ntok, v.tok, v.pair0, aux);
                }
            }
        } else {
            const int sl = ur.sl, ht = ur.idx;
            bool combined = false;
            DownStamps ds;
            ds.on = f.trace != nullptr;
            if (sl < S) {  // shared slot: all tokens in order, no routing dependency
                if (sl < a.n_shared) {
                    int tok[NT], rank[NT];
#pragma unroll
                    for (int j = 0; j < NT; j++) {
                        tok[j] = j;
                        rank[j] = -1;
                    }
                    down_unit<NT, Q8OK>(s, a, sl, ht, -1 - sl, a.T, tok, rank, ds);
                }
            } else {
                ensure_routed();
                if (sl < rt->nslot) {
                    SlotRt<NT> v;
                    v.load(rt, sl, S, a.keep);
                    const bool fold = sl == M - 1 && combine_in_unit(a);
                    down_unit<NT, Q8OK>(s, a, sl, ht, v.expert, v.ntok, v.tok, v.rank, ds, fold, rt);
                    combined = fold;
                }
            }
            t_aux = ds.aux;
            t_aux2 = ds.run;
            t_ready = ds.ready;
            if (sl == M - 1 && !combined) {  // the last slot's unit of each tile combines it
                ensure_routed();
                combine_tile(a, rt, ht);
            }
        }
        if (f.trace && threadIdx.x == 0) {
            uint64_t* tr = f.trace + (size_t)u * kTraceFields;
            tr[0] = t_start;
            tr[1] = t_ready;
            tr[2] = __builtin_amdgcn_s_memrealtime();
            tr[3] = blockIdx.x;
            tr[4] = t_aux;
            tr[5] = t_aux2;
        }
        __syncthreads();  // the whole workgroup is done with unit u before s_unit changes
        if (threadIdx.x == 0) s_unit = next;
        __syncthreads();
        u = __builtin_amdgcn_readfirstlane(s_unit);  // uniform: unit decoding stays in scalar registers
    }
}

#if MOE_COMMON
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

// Router table [E][H] bf16 -> chain order (ck_chain_dword): one thread per destination 16-byte chunk.
__global__ void relayout_router_kernel(const unsigned* __restrict__ src, int E, int H, u32x4* __restrict__ dst) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t per_row = H / 8;
    if (q >= (size_t)E * per_row) return;
    const int e = (int)(q / per_row), r = (int)(q % per_row), qq = r / 32, c = r % 32;
    const unsigned* row = src + (size_t)e * (H / 2);
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = row[32 * (4 * qq + i) + c];
    dst[q] = v;
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

__global__ void zero_kernel(uint64_t* __restrict__ dst, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) dst[i] = 0;
}

__global__ void synth_fill_kernel(u32x4* __restrict__ dst, uint64_t nchunk, uint64_t key, uint64_t start, float c) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q < nchunk) dst[q] = synth_chunk(key, start + q * 8, c);
}

// ==================================================================================================================
// launch helpers
#endif  // MOE_COMMON

static inline unsigned nblk(size_t n, int b) { return (unsigned)((n + b - 1) / b); }

static hipError_t set_lds(const void* fn, size_t lds) { return raise_lds_limit(fn, lds); }

static int nt_bucket(int T) { return T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : T <= 8 ? 8 : 16; }

#if MOE_COMMON
hipError_t launch_router(const LayerPtrs& L, const Dims& d, int T, const StageSrc& in, uint64_t* logits,
                         float* logits_out, unsigned epoch, hipStream_t st) {
    const size_t lds = lds_bytes(T, 1, d.H, d.F, d.E);
    hipError_t e = set_lds(reinterpret_cast<const void*>(&router_kernel), lds);
    if (e != hipSuccess) return e;
    const dim3 grid(nblk(d.E, kRouterRows), T > 1 ? nblk(T, kRouterTG) : 1);  // (row groups, token groups)
    hipLaunchKernelGGL(router_kernel, grid, dim3(256), lds, st, L, d, T, in, logits, logits_out, epoch);
    return hipGetLastError();
}

hipError_t launch_topk_group(const LayerPtrs& L, const Dims& d, int T, int keep, int n_shared, bool do_topk, int rule,
                             const uint64_t* logits, unsigned epoch, unsigned* err, int32_t* ids, float* gates,
                             Slots* slots, hipStream_t st) {
    hipLaunchKernelGGL(topk_group_kernel, dim3(1), dim3(kTopkThreads), 0, st, L, d, T, keep, n_shared, do_topk ? 1 : 0, rule,
                       logits, epoch, err, ids, gates, slots);
    return hipGetLastError();
}

#endif  // MOE_COMMON

template <int NT>
hipError_t gateup_nt(const ExpertArgs& ea, Sync* sy, hipStream_t st) {
    const int maxs = ea.maxs;
    const size_t lds = gu_lds_bytes(ea.T, NT, ea.d.H);
    hipError_t e = set_lds(reinterpret_cast<const void*>(&gateup_kernel<NT>), lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(gateup_kernel<NT>, dim3(gateup_units(maxs, ea.d.n_shared, ea.d.F, ea.kp, ea.kps)), dim3(256), lds, st, ea, sy);
    return hipGetLastError();
}

template <int NT>
hipError_t down_nt(const ExpertArgs& ea, hipStream_t st) {
    const size_t lds = lds_bytes(0, NT, ea.d.H, ea.d.F, ea.d.E);
    hipError_t e = set_lds(reinterpret_cast<const void*>(&down_kernel<NT>), lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(down_kernel<NT>, dim3(ea.maxs * (ea.d.H / 64)), dim3(256), lds, st, ea);
    return hipGetLastError();
}

template <int NT>
hipError_t fused_nt(FusedArgs f, int wg_per_cu, int grid_req, hipStream_t st, int* grid_out);
#if defined(MOE_EXTERN_BUCKETS)
#define MOE_BUCKET_DECL(N)                                                                         \
    extern template hipError_t gateup_nt<N>(const ExpertArgs&, Sync*, hipStream_t);                \
    extern template hipError_t down_nt<N>(const ExpertArgs&, hipStream_t);                         \
    extern template hipError_t fused_nt<N>(FusedArgs, int, int, hipStream_t, int*);
MOE_BUCKET_DECL(1)
MOE_BUCKET_DECL(2)
MOE_BUCKET_DECL(4)
MOE_BUCKET_DECL(8)
MOE_BUCKET_DECL(16)
#endif
#if defined(MOE_PART) && MOE_PART > 0
template hipError_t gateup_nt<MOE_PART>(const ExpertArgs&, Sync*, hipStream_t);
template hipError_t down_nt<MOE_PART>(const ExpertArgs&, hipStream_t);
#endif

#if MOE_COMMON
hipError_t launch_gateup(const ExpertArgs& ea, Sync* sy, hipStream_t st) {
    switch (nt_bucket(ea.T)) {
        case 1: return gateup_nt<1>(ea, sy, st);
        case 2: return gateup_nt<2>(ea, sy, st);
        case 4: return gateup_nt<4>(ea, sy, st);
        case 8: return gateup_nt<8>(ea, sy, st);
        default: return gateup_nt<16>(ea, sy, st);
    }
}

hipError_t launch_down(const ExpertArgs& ea, hipStream_t st) {
    switch (nt_bucket(ea.T)) {
        case 1: return down_nt<1>(ea, st);
        case 2: return down_nt<2>(ea, st);
        case 4: return down_nt<4>(ea, st);
        case 8: return down_nt<8>(ea, st);
        default: return down_nt<16>(ea, st);
    }
}

#endif  // MOE_COMMON

template <int NT>
hipError_t fused_nt(FusedArgs f, int wg_per_cu, int grid_req, hipStream_t st, int* grid_out) {
    // int8 routed experts get their own instantiation: the bf16 kernel carries no int8 code
    auto kern = f.e.int8 ? &fused_layer_kernel<NT, true> : &fused_layer_kernel<NT, false>;
    const void* fn = reinterpret_cast<const void*>(kern);
    const size_t lds = lds_bytes(f.e.T, NT, f.e.d.H, f.e.d.F, f.e.d.E);
    // occupancy per (device, LDS size), computed once: the launch itself stays a single host call
    static thread_local int c_dev = -1, c_ncu = 0, c_per_cu = 0;
    static thread_local size_t c_lds = 0;
    static thread_local const void* c_fn = nullptr;
    hipError_t e;
    int dev = 0;
    if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
    if ((e = set_lds(fn, lds)) != hipSuccess) return e;
    if (dev != c_dev || lds != c_lds || fn != c_fn) {
        if ((e = hipDeviceGetAttribute(&c_ncu, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
        if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&c_per_cu, fn, 256, lds)) != hipSuccess) return e;
        c_dev = dev;
        c_lds = lds;
        c_fn = fn;
    }
    int per_cu = c_per_cu, ncu = c_ncu;
    if (wg_per_cu > 0 && wg_per_cu < per_cu) per_cu = wg_per_cu;
    if (per_cu < 1) return hipErrorInvalidConfiguration;
    const int units = fused_units(f.nR, f.e.maxs, f.e.d.n_shared, f.e.d.F, f.e.d.H, f.e.kp, f.e.kps);
    int grid = grid_req > 0 ? grid_req : ncu * per_cu;  // a requested grid may exceed what fits at once
    if (grid > units) grid = units;
    if (grid_out) *grid_out = grid;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), lds, st, f);
    return hipGetLastError();
}

// The fused kernel exists for up to 8 tokens: its 16-token bucket spilled several hundred bytes of registers, so
// calls of 9 to 16 tokens (possible for H <= 3072) run the unfused kernels, whose arithmetic is the same.
#if defined(MOE_PART) && MOE_PART > 0 && MOE_PART <= 8
template hipError_t fused_nt<MOE_PART>(FusedArgs, int, int, hipStream_t, int*);
#endif

#if MOE_COMMON
hipError_t launch_fused(const FusedArgs& f, int wg_per_cu, int grid, hipStream_t st, int* grid_out) {
    switch (nt_bucket(f.e.T)) {
        case 1: return fused_nt<1>(f, wg_per_cu, grid, st, grid_out);
        case 2: return fused_nt<2>(f, wg_per_cu, grid, st, grid_out);
        case 4: return fused_nt<4>(f, wg_per_cu, grid, st, grid_out);
        case 8: return fused_nt<8>(f, wg_per_cu, grid, st, grid_out);
        default: return hipErrorInvalidValue;  // T > 8: the unfused path
    }
}

hipError_t launch_relayout_gu(const uint16_t* g, const uint16_t* u, int H, int F, uint16_t* dst, hipStream_t st) {
    const size_t n = (size_t)(F / 32) * (H / 8) * 64;
    hipLaunchKernelGGL(relayout_gu_kernel, dim3(nblk(n, 256)), dim3(256), 0, st, g, u, H, F,
                       reinterpret_cast<u32x4*>(dst));
    return hipGetLastError();
}

hipError_t launch_relayout_router(const uint16_t* src, int E, int H, uint16_t* dst, hipStream_t st) {
    const size_t n = (size_t)E * (H / 8);
    hipLaunchKernelGGL(relayout_router_kernel, dim3(nblk(n, 256)), dim3(256), 0, st,
                       reinterpret_cast<const unsigned*>(src), E, H, reinterpret_cast<u32x4*>(dst));
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

hipError_t launch_zero(uint64_t* dst, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(zero_kernel, dim3((unsigned)blocks), dim3(256), 0, st, dst, n);
    return hipGetLastError();
}

#endif  // MOE_COMMON

}  // namespace moe
