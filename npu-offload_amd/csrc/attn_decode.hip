// attn_decode.hip — GQA decode attention of one token over a layer's KV cache (include/moe_gpu.h, moe_attn_*).
// Replaces the host step's attention core (track2_opt/solar_engine/src/main.rs:86-104): for q head h, kv head
// h / (NQ / NKV), positions t < S:
//   sc[t] = bf16(bf16(q_h . k_t) * scale)   (the dot summed left to right in fp32)
//   p[t]  = bf16(exp(sc[t] - max sc) / sum exp(sc - max sc))
//   out_h = bf16(sum_t p[t] * v_t)
// One launch (attn_fused_kernel): a workgroup per (128-position chunk, kv head) computes its chunk's scores (one lane
// per position, the dot in the reference's order, so the scores are bit-identical), publishes the chunk's softmax
// statistics, combines every chunk's into the group's max and total, publishes its chunk's partial P.V and sums its
// share of the outputs over the chunks.  HBM-bound on the cache read: 2 * S * NKV * D * 2 bytes per call (16.8 MB at
// S = 4096, NKV = 8, D = 128).
#include <hip/hip_runtime.h>

#include <stddef.h>
#include <stdlib.h>

#include <algorithm>
#include <mutex>
#include <unordered_map>

#include "launch_util.h"
#include "moe_gpu.h"

namespace {

constexpr int kD = 128;  // head dim
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(4))) uint32_t cu32;  // constant address space: loads may go through scalar loads

__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ uint32_t f2bf(float f) {  // round to nearest even (host.rs:41-46)
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

// ==================================================================================================================
// One launch: workgroup (w, g) of kT = 512 threads owns chunks [w R, w R + R) of kv head g (a chunk: 128 consecutive
// positions; R = 1 unless the grid would not fit on the chip at once) for all G q heads of the group:
//  1. per own chunk: its K rows (staged in LDS; thread (head slot hq = tid / 128, position tid % 128) takes G / 4 heads,
//     or one for G < 4), the scores in the reference's dot order (to LDS and to the workspace), the chunk statistics
//     per head m_c = max sc and s_c = sum exp(sc - m_c), published as tagged words;
//  2. once every chunk's statistics of the group are in: M = max_c m_c, tot = sum_c s_c exp(m_c - M) (the same
//     operations in every workgroup of the group, so every one gets the same bits);
//  3. per own chunk: p = bf16(exp(sc - M) / tot) and the chunk's partial P.V (wave w: positions 16 w .. 16 w + 15 in
//     order; the 8 waves summed as a fixed tree), published as tagged words;
//  4. it sums its share of the group's G * 128 outputs over the chunks in order and writes them as bf16.
// Tagged words are (epoch << 32) | payload.  The epoch is counted in the workspace's header, on the device, so that a
// call replayed from a HIP graph gets a new one too: every workgroup reads the previous epoch at its start and counts
// itself in `started`; the last to start stores this call's epoch for the next call.  Epochs skip values whose low 16
// bits are zero: a score is a bf16 value widened to fp32 (low 16 bits zero), so the upper half of a word over the
// scores of an earlier call with a larger S never equals an epoch either.  The call whose epoch reaches kEpochWrap is
// also counted out in `done`: the last workgroup to finish clears the tag area and restarts the epochs.  A wait that
// stays unmet for `poll` passes (a producer workgroup not resident) computes the missing chunk itself through the
// same functions, so the launch needs no co-residency and the bits do not depend on which workgroup computed what.
constexpr int kP = 128;          // positions per chunk
constexpr int kT = 512;          // threads per workgroup: 8 waves, 2 per SIMD
constexpr int kWv = kT / 64;     // waves per workgroup
constexpr int kVP = kP / kWv;    // positions per wave in the P.V product
constexpr int kMaxC = 512;       // chunks per kv head (S <= 65536)

constexpr unsigned kEpochWrap = 0xFFFF0000u;
constexpr int kOK = 4096;             // o projection: columns (NQ * kD), one 8-chunk load group per lane per row
constexpr int kOC = kOK / 512;        // 16-byte chunks per lane per row
constexpr int kORows = 2 * (kT / 64); // o rows per workgroup: two per wave
constexpr size_t kHdrBytes = 256;  // workspace header: [0] last epoch, [1] started, [2] done

struct FusedAttn {
    uint64_t* hdr;     // the workspace's header
    uint64_t* end;     // the end of the workspace (the tag area is [stats, end))
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    uint16_t* out;
    float* scores;     // [NQ, S] the scores of this call (left for the caller)
    uint64_t* stats;   // [NQ][C][2] tagged (m, s)
    uint64_t* part;    // [NQ][C][kD] tagged partial P.V
    int NQ, NKV, S, C, R, W;  // chunks, chunks per workgroup, workgroups per kv head
    int poll;                 // passes of a wait before the fallback
    float scale;
    // the o projection folded in (moe_attn_decode_oproj_dev; wo null otherwise): o_out = bf16(wo . out), wo [Mo, NQ*kD]
    const uint16_t* wo;
    uint16_t* o_out;
    uint64_t* aout;  // [NQ * kD] tagged attention outputs (bf16 bits), read by every workgroup's o rows
    int Mo, Wa;      // o rows; attention workgroups (W * NKV, the first Wa of the grid)
};

__device__ __forceinline__ unsigned next_epoch(unsigned e) {
    ++e;
    return (e & 0xFFFFu) ? e : e + 1;
}

__device__ __forceinline__ uint64_t tagw(unsigned epoch, float v) { return ((uint64_t)epoch << 32) | __float_as_uint(v); }
__device__ __forceinline__ void st_word(uint64_t* p, uint64_t w) {
    __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_word(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int kKS = kD * 2 + 16;  // bytes per staged K row: 256 + 16 of padding, so that 16 lanes reading 16 consecutive
                                  // rows at one offset hit 16 distinct 16-byte bank groups

template <int G>
struct AttnLds {
    union {  // never live at the same time (each use ends at a barrier before the next begins)
        __attribute__((aligned(16))) unsigned char kst[kP * kKS];  // a chunk's K rows
        float acc[kWv][G][kD];                                     // per-wave partial P.V
        float tab[G * kD + kMaxC];  // this workgroup's share of the outputs: [chunk][output] partials
    };
    __attribute__((aligned(16))) float sc[G][kP];  // scores, then p
    float part[G][kD];                             // a chunk's partial P.V
    float m[G], s[G], M[G], tot[G];
    float mt[G][kMaxC], st[G][kMaxC];  // every chunk's statistics of the group
    unsigned char missing[kMaxC];
    int nmiss, anymiss;
    unsigned ep;  // the header's last epoch, as thread 0 read it
    __attribute__((aligned(16))) uint16_t ox[kOK];  // the o projection's input: every attention output (bf16)
};

// Scores of chunk c into L.sc (positions past S: -inf), and to the workspace when write_ws, from the chunk's K rows in
// L.kst: thread (hq, t) takes position t for heads hq * GH .. hq * GH + GH - 1.
template <int G>
__device__ __forceinline__ void chunk_scores(const FusedAttn& a, AttnLds<G>& L, int g, int c, bool write_ws) {
    const int t = threadIdx.x & (kP - 1);
    const int hq = __builtin_amdgcn_readfirstlane(threadIdx.x / kP);  // uniform per wave
    constexpr int GH = G >= 4 ? G / 4 : 1;  // heads per thread
    const int h0 = hq * GH;
    const int pos = c * kP + t;
    if (h0 < G) {
        // q is the same for every lane of a wave and is not written by the call: read through the constant address
        // space with wave-uniform indices it comes in through scalar loads and feeds the fma as a scalar operand.
        // Products of bf16 values are exact in fp32, so fma = multiply-then-add.
        const cu32* qg = (const cu32*)(a.q + (size_t)(g * G + h0) * kD);
        const u32x4* kr = reinterpret_cast<const u32x4*>(L.kst + t * kKS);
        float dot[GH];
#pragma unroll
        for (int h = 0; h < GH; ++h) dot[h] = 0.f;
#pragma unroll
        for (int cc = 0; cc < kD / 8; ++cc) {
            const u32x4 k4 = kr[cc];
            const uint32_t w4[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float k0 = __uint_as_float(w4[j] << 16), k1 = __uint_as_float(w4[j] & 0xFFFF0000u);
#pragma unroll
                for (int h = 0; h < GH; ++h) {
                    const uint32_t qq = qg[(h * kD + cc * 8 + 2 * j) / 2];
                    dot[h] = fmaf(__uint_as_float(qq << 16), k0, dot[h]);
                    dot[h] = fmaf(__uint_as_float(qq & 0xFFFF0000u), k1, dot[h]);
                }
            }
        }
#pragma unroll
        for (int h = 0; h < GH; ++h) {
            const float v = bf2f(f2bf(bf2f(f2bf(dot[h])) * a.scale));
            L.sc[h0 + h][t] = pos < a.S ? v : -INFINITY;
            if (write_ws && pos < a.S) a.scores[(size_t)(g * G + h0 + h) * a.S + pos] = v;
        }
    }
    __syncthreads();
}

// A value reduced over the 64 lanes of a wave in a fixed order, every lane getting the same bits: xor 1 and xor 2 within
// quads, then mirrors within 8 and within 16 lanes (DPP moves, each step combining two equal partial results), then
// the four rows of 16 as (r0 op r1) op (r2 op r3).  All 64 lanes must be active.
template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
    v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false)));   // quad [1,0,3,2]
    v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false)));   // quad [2,3,0,1]
    v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false)));  // row half mirror
    v = op(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false)));  // row mirror
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return op(op(r0, r1), op(r2, r3));
}
struct MaxOp {
    __device__ float operator()(float x, float y) const { return fmaxf(x, y); }
};
struct AddOp {
    __device__ float operator()(float x, float y) const { return x + y; }
};

// Chunk c's scores back from the workspace (written by this workgroup) into L.sc.
template <int G>
__device__ __forceinline__ void load_scores(const FusedAttn& a, AttnLds<G>& L, int g, int c) {
    for (int i = threadIdx.x; i < G * kP; i += kT) {
        const int h = i / kP, pos = c * kP + i % kP;
        L.sc[h][i % kP] = pos < a.S ? a.scores[(size_t)(g * G + h) * a.S + pos] : -INFINITY;
    }
    __syncthreads();
}

// K rows of chunk c, coalesced: load j of thread i takes 16 bytes (i % 16) of row (i + kT j) / 16 (rows clamped into
// range; unused rows are discarded by the score mask).
constexpr int kKL = kP * kD * 2 / 16 / kT;  // 16-byte loads per thread
__device__ __forceinline__ void load_k(const FusedAttn& a, int g, int c, u32x4 (&kr)[kKL]) {
#pragma unroll
    for (int j = 0; j < kKL; ++j) {
        const int i = threadIdx.x + kT * j, r = i / 16;
        const int pos = min(c * kP + r, a.S - 1);
        kr[j] = reinterpret_cast<const u32x4*>(a.k + ((size_t)pos * a.NKV + g) * kD)[i % 16];
    }
}
template <int G>
__device__ __forceinline__ void store_k(AttnLds<G>& L, const u32x4 (&kr)[kKL]) {
#pragma unroll
    for (int j = 0; j < kKL; ++j) {
        const int i = threadIdx.x + kT * j;
        *reinterpret_cast<u32x4*>(L.kst + (i / 16) * kKS + (i % 16) * 16) = kr[j];
    }
    __syncthreads();
}

// V rows of chunk c for wave w's kVP positions, lane l's dims 2l, 2l + 1.
__device__ __forceinline__ void load_v(const FusedAttn& a, int g, int c, uint32_t (&vv)[kVP]) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int u = 0; u < kVP; ++u) {
        const int pos = min(c * kP + w * kVP + u, a.S - 1);
        vv[u] = *reinterpret_cast<const uint32_t*>(a.v + ((size_t)pos * a.NKV + g) * kD + 2 * lane);
    }
}

// The chunk's statistics per head from L.sc into L.m / L.s: wave w handles heads w, w + kWv (positions t and t + 64 per
// lane, then wave reductions).
template <int G>
__device__ __forceinline__ void chunk_stats(AttnLds<G>& L) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (int h = w; h < G; h += kWv) {
        const float x0 = L.sc[h][lane], x1 = L.sc[h][lane + 64];
        const float m = wave_reduce(fmaxf(x0, x1), MaxOp());
        const float e =
            wave_reduce((x0 == -INFINITY ? 0.f : expf(x0 - m)) + (x1 == -INFINITY ? 0.f : expf(x1 - m)), AddOp());
        if (lane == 0) {
            L.m[h] = m;
            L.s[h] = e;
        }
    }
    __syncthreads();
}

// p = bf16(exp(sc - M) / tot) in place, then the chunk's partial P.V into L.part (vv: this thread's V values).
template <int G>
__device__ __forceinline__ void chunk_pv(AttnLds<G>& L, const uint32_t (&vv)[kVP]) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    for (int i = tid; i < G * kP; i += kT) {
        const int h = i / kP, t = i % kP;
        const float x = L.sc[h][t];
        L.sc[h][t] = x == -INFINITY ? 0.f : bf2f(f2bf(expf(x - L.M[h]) / L.tot[h]));
    }
    __syncthreads();
    float acc[G][2];
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h][0] = acc[h][1] = 0.f;
#pragma unroll
    for (int u4 = 0; u4 < kVP; u4 += 4) {
        f32x4 p4[G];  // p of 4 positions per head (one broadcast read each)
#pragma unroll
        for (int h = 0; h < G; ++h) p4[h] = *reinterpret_cast<const f32x4*>(&L.sc[h][w * kVP + u4]);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t vw = vv[u4 + u];
            const float v0 = __uint_as_float(vw << 16), v1 = __uint_as_float(vw & 0xFFFF0000u);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                acc[h][0] = fmaf(p4[h][u], v0, acc[h][0]);
                acc[h][1] = fmaf(p4[h][u], v1, acc[h][1]);
            }
        }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
        L.acc[w][h][2 * lane] = acc[h][0];
        L.acc[w][h][2 * lane + 1] = acc[h][1];
    }
    __syncthreads();
    for (int i = tid; i < G * kD; i += kT) {
        const int h = i / kD, d = i % kD;
        L.part[h][d] = ((L.acc[0][h][d] + L.acc[1][h][d]) + (L.acc[2][h][d] + L.acc[3][h][d])) +
                       ((L.acc[4][h][d] + L.acc[5][h][d]) + (L.acc[6][h][d] + L.acc[7][h][d]));
    }
    __syncthreads();
}

// M and tot per head from every chunk's statistics in L.mt / L.st (wave w: heads w, w + kWv): M = the max over the
// chunks; tot = sum_c s_c exp(m_c - M), lane l adding chunks l, l + 64, ... in order, then a wave reduction (the same
// operations in every workgroup of the group).  The caller has synchronised since L.mt / L.st were written; L.M /
// L.tot are read after a later barrier.
template <int G>
__device__ __forceinline__ void group_totals(AttnLds<G>& L, int C) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (int h = w; h < G; h += kWv) {
        float m = -INFINITY;
        for (int cc = lane; cc < C; cc += 64) m = fmaxf(m, L.mt[h][cc]);
        m = wave_reduce(m, MaxOp());
        float tot = 0.f;
        for (int cc = lane; cc < C; cc += 64) tot = fmaf(L.st[h][cc], expf(L.mt[h][cc] - m), tot);
        tot = wave_reduce(tot, AddOp());
        if (lane == 0) {
            L.M[h] = m;
            L.tot[h] = tot;
        }
    }
}

// Tagged words polled in groups of kGW per thread, every load of a group in flight together: the words whose bit is set
// in `need` are loaded until they carry `epoch`; true when all did within `poll` passes.
constexpr int kGW = 8;
template <typename Ptr>
__device__ __forceinline__ bool poll_words(uint64_t (&w)[kGW], unsigned need, Ptr ptr, unsigned epoch, int poll) {
#pragma unroll
    for (int j = 0; j < kGW; ++j)
        if (need >> j & 1) w[j] = ld_word(ptr(j));
    for (int n = 0;; ++n) {
        bool all = true;
#pragma unroll
        for (int j = 0; j < kGW; ++j) all = all && (!(need >> j & 1) || (unsigned)(w[j] >> 32) == epoch);
        if (all) return true;
        if (n >= poll) return false;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int j = 0; j < kGW; ++j)
            if ((need >> j & 1) && (unsigned)(w[j] >> 32) != epoch) w[j] = ld_word(ptr(j));
    }
}

// A share whose partials did not all arrive: every chunk's partial is recomputed here in chunk order (the producer's
// functions) and the whole share summed as the gather does (outputs already written get the same bits).
template <int G, typename Put>
__device__ void share_fallback(const FusedAttn& a, AttnLds<G>& L, int g, int o0, int nout, uint32_t (&vv)[kVP], Put put) {
    const int tid = threadIdx.x, C = a.C;
    constexpr int kJ = (G * kD + kT - 1) / kT;
    float sums[kJ];
#pragma unroll
    for (int j = 0; j < kJ; ++j) sums[j] = 0.f;
    for (int cc = 0; cc < C; ++cc) {
        u32x4 kr[kKL];
        load_k(a, g, cc, kr);
        load_v(a, g, cc, vv);
        store_k<G>(L, kr);
        chunk_scores<G>(a, L, g, cc, false);
        chunk_pv<G>(L, vv);
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
            const int i = tid + kT * j;
            if (i < nout) {
                const float v = L.part[(o0 + i) / kD][(o0 + i) % kD];
                sums[j] = cc == 0 ? v : sums[j] + v;
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
        const int i = tid + kT * j;
        if (i < nout) put((g * G + (o0 + i) / kD) * kD + (o0 + i) % kD, f2bf(sums[j]));
    }
}

// Every output of kv head g computed here from the cache (the statistics of every chunk, the totals, every chunk's
// partial), with the producers' functions, so the bits are theirs: the o projection's fallback for outputs that never
// arrived.  put(output index, bf16 bits).
template <int G, typename Put>
__device__ void group_fallback(const FusedAttn& a, AttnLds<G>& L, int g, uint32_t (&vv)[kVP], Put put) {
    const int tid = threadIdx.x;
    for (int cc = 0; cc < a.C; ++cc) {
        u32x4 kr[kKL];
        load_k(a, g, cc, kr);
        store_k<G>(L, kr);
        chunk_scores<G>(a, L, g, cc, false);
        chunk_stats<G>(L);
        if (tid < G) {
            L.mt[tid][cc] = L.m[tid];
            L.st[tid][cc] = L.s[tid];
        }
        __syncthreads();
    }
    group_totals<G>(L, a.C);
    __syncthreads();
    share_fallback<G>(a, L, g, 0, G * kD, vv, put);
}

// Sum over a wave by xor butterflies 32 .. 1 (the order of the dense GEMV's, whose bits the o projection keeps).
__device__ __forceinline__ float wave_sum_xor(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// OPROJ: the o projection folded in.  Workgroup b also owns o rows kORows b .. kORows b + kORows - 1 (wave w: two rows,
// lane l: 16-byte chunks 64 c + l of each), whose weights it loads once it has published its chunk statistics (so they
// stream while the exchanges wait); the grid is max(W * NKV, Mo / kORows) workgroups, those past W * NKV only
// computing o rows.  5. Every attention output arrives as a tagged word (published by step 4); each row is then summed
// in the dense GEMV's order (lane chunks in order, then a xor butterfly), so o is bit-identical to moe_gemv_dev's.
template <int G, bool OPROJ>
__global__ __launch_bounds__(kT) void attn_fused_kernel(FusedAttn a) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    AttnLds<G>& L = *reinterpret_cast<AttnLds<G>*>(lds_raw);
    const int b = (int)blockIdx.x;
    const bool attn_wg = !OPROJ || b < a.Wa;
    const int g = attn_wg ? b / a.W : 0, wg = attn_wg ? b % a.W : 0, C = a.C, tid = threadIdx.x;
    const int c0 = attn_wg ? wg * a.R : 0, c1 = attn_wg ? min(c0 + a.R, C) : 0;  // own chunks
    const int poll = a.poll;
    const unsigned long long total = gridDim.x;
    const int olane = tid & 63, owv = tid >> 6;
    const bool has_o = OPROJ && b * kORows < a.Mo;
    u32x4 wo_r[2][kOC];
    auto load_wo = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int row = min(b * kORows + 2 * owv + r, a.Mo - 1);  // rows past Mo re-read the last; discarded
            const u32x4* wr = reinterpret_cast<const u32x4*>(a.wo + (size_t)row * kOK);
#pragma unroll
            for (int c = 0; c < kOC; ++c) wo_r[r][c] = __builtin_nontemporal_load(&wr[c * 64 + olane]);
        }
    };
    if (has_o && !attn_wg) load_wo();
    if (tid == 0) {
        L.ep = (unsigned)ld_word(a.hdr);  // read once, by the thread that counts the workgroup as started
        L.anymiss = 0;
    }
    // 1. own chunks: scores and statistics, published (the first chunk's V rows loaded with its K rows)
    uint32_t vv[kVP];
    unsigned epoch = 0;
    bool wrap = false;
    for (int i = tid; i < C; i += kT) L.missing[i] = 0;
    if (!attn_wg) {  // (uniform) an o-only workgroup takes the call's epoch here
        __syncthreads();
        epoch = next_epoch(L.ep);
        wrap = epoch >= kEpochWrap;
    }
    for (int c = c0; c < c1; ++c) {
        u32x4 kr[kKL];
        load_k(a, g, c, kr);
        uint32_t warm = 0;
        if (c == c0) {
            load_v(a, g, c, vv);
            // the group's q lines (G * 256 bytes) into the scalar cache while the K rows load: the score loop's
            // scalar loads then hit instead of each waiting for L2
            const cu32* qw = (const cu32*)(a.q + (size_t)g * G * kD);
#pragma unroll
            for (int l = 0; l < G * kD * 2 / 64; ++l) warm ^= qw[l * 16];
        }
        store_k<G>(L, kr);
        if (warm == 0x7FC00001u && a.S < 0) L.nmiss = 1;  // never true (S >= 1): keeps the loads above
        chunk_scores<G>(a, L, g, c, true);
        chunk_stats<G>(L);
        epoch = next_epoch(L.ep);  // the same in every workgroup of the call
        wrap = epoch >= kEpochWrap;
        if (tid < G) {
            uint64_t* sp = a.stats + ((size_t)(g * G + tid) * C + c) * 2;
            st_word(sp, tagw(epoch, L.m[tid]));
            st_word(sp + 1, tagw(epoch, L.s[tid]));
            L.mt[tid][c] = L.m[tid];
            L.st[tid][c] = L.s[tid];
        }
    }
    if (has_o && attn_wg) load_wo();
    // counted as started (thread 0 read the epoch before); the return is needed only after the waits below
    unsigned long long started = 0;
    if (tid == 0) started = __hip_atomic_fetch_add(a.hdr + 1, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // an attention output: bf16 to `out`, and (OPROJ) a tagged word for every workgroup's o rows
    auto put_out = [&](int o, uint32_t bits) __attribute__((always_inline)) {
        a.out[o] = (uint16_t)bits;
        if (OPROJ) st_word(a.aout + o, ((uint64_t)epoch << 32) | bits);
    };
    if (attn_wg) {  // (uniform) steps 2 to 4
    // 2. the other chunks' statistics of the group; item i = (head i / C, chunk i % C), two words each
    for (int i0 = 0; i0 < G * C; i0 += kT * (kGW / 2)) {
        uint64_t w[kGW];
        auto item = [&](int j) { return i0 + tid + kT * (j >> 1); };
        auto other = [&](int it) { return it < G * C && (it % C < c0 || it % C >= c1); };
        unsigned need = 0;
#pragma unroll
        for (int j = 0; j < kGW; ++j)
            if (other(item(j))) need |= 1u << j;
        auto ptr = [&](int j) {
            const int it = item(j);
            return a.stats + ((size_t)(g * G + it / C) * C + it % C) * 2 + (j & 1);
        };
        poll_words(w, need, ptr, epoch, poll);
#pragma unroll
        for (int j = 0; j < kGW; j += 2) {
            const int it = item(j);
            if (other(it)) {
                const bool ok = (unsigned)(w[j] >> 32) == epoch && (unsigned)(w[j + 1] >> 32) == epoch;
                L.mt[it / C][it % C] = __uint_as_float((unsigned)w[j]);
                L.st[it / C][it % C] = __uint_as_float((unsigned)w[j + 1]);
                if (!ok) {
                    L.missing[it % C] = 1;
                    L.anymiss = 1;
                }
            }
        }
    }
    __syncthreads();
    const bool refill = L.anymiss;  // (uniform) L.sc no longer holds the last own chunk's scores
    if (refill) {
        for (int cc = 0; cc < C; ++cc) {  // fallback: a missing chunk's statistics by the producer's own computation
            if (!L.missing[cc]) continue;   // (uniform: every thread reads the same flag)
            u32x4 kr[kKL];
            load_k(a, g, cc, kr);
            store_k<G>(L, kr);
            chunk_scores<G>(a, L, g, cc, false);
            chunk_stats<G>(L);
            if (tid < G) {
                L.mt[tid][cc] = L.m[tid];
                L.st[tid][cc] = L.s[tid];
            }
            __syncthreads();
        }
    }
    group_totals<G>(L, C);
    // 3. p and each own chunk's partial P.V, published (the scores back from the workspace unless L.sc holds them)
    for (int c = c0; c < c1; ++c) {
        if (c != c0) load_v(a, g, c, vv);
        if (c1 - c0 == 1 && !refill)
            __syncthreads();  // L.M, L.tot written
        else
            load_scores<G>(a, L, g, c);
        chunk_pv<G>(L, vv);
        for (int i = tid; i < G * kD; i += kT) {
            const int h = i / kD, d = i % kD;
            st_word(a.part + ((size_t)(g * G + h) * C + c) * kD + d, tagw(epoch, L.part[h][d]));
        }
    }
    // 4. this workgroup's share of the group's G * kD outputs, each the chunk partials summed in chunk order.  In
    //    passes of n outputs: word i = (chunk i / n, output ob + i % n) gathered into L.tab, then summed.
    const int per = (G * kD + a.W - 1) / a.W, o0 = min(wg * per, G * kD), o1 = min(o0 + per, G * kD);
    const int nout = o1 - o0, nb = (G * kD + kMaxC) / C;
    bool fallback = false;
    for (int ob = o0; ob < o1; ob += nb) {
        const int n = min(nb, o1 - ob);
        if (tid == 0) L.nmiss = 0;
        __syncthreads();
        for (int i0 = 0; i0 < n * C; i0 += kT * kGW) {
            uint64_t w[kGW];
            unsigned need = 0;
#pragma unroll
            for (int j = 0; j < kGW; ++j)
                if (i0 + tid + kT * j < n * C) need |= 1u << j;
            auto ptr = [&](int j) {
                const int i = i0 + tid + kT * j, o = ob + i % n;
                return a.part + ((size_t)(g * G + o / kD) * C + i / n) * kD + o % kD;
            };
            if (!poll_words(w, need, ptr, epoch, poll)) L.nmiss = 1;
#pragma unroll
            for (int j = 0; j < kGW; ++j)
                if (need >> j & 1) L.tab[i0 + tid + kT * j] = __uint_as_float((unsigned)w[j]);
        }
        __syncthreads();
        if (L.nmiss) {  // uniform
            fallback = true;
            break;
        }
        for (int i = tid; i < n; i += kT) {
            float sum = L.tab[i];
            int cc = 1;
            for (; cc + 8 <= C; cc += 8) {  // 8 reads in flight, then the adds in chunk order
                float t8[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) t8[k] = L.tab[(cc + k) * n + i];
#pragma unroll
                for (int k = 0; k < 8; ++k) sum = sum + t8[k];
            }
            for (; cc < C; ++cc) sum = sum + L.tab[cc * n + i];
            const int o = ob + i;
            put_out((g * G + o / kD) * kD + o % kD, f2bf(sum));
        }
        __syncthreads();  // L.tab is refilled by the next pass
    }
    if (fallback) share_fallback<G>(a, L, g, o0, nout, vv, put_out);
    }  // steps 2 to 4
    if (has_o) {  // (uniform) 5. the o rows, from every attention output
        const int nO = a.NQ * kD;  // == kOK
        uint64_t w[kGW];
        unsigned need = 0;
#pragma unroll
        for (int j = 0; j < kGW; ++j)
            if (tid + kT * j < nO) need |= 1u << j;
        if (tid == 0) L.nmiss = 0;
        __syncthreads();
        if (!poll_words(w, need, [&](int j) { return a.aout + tid + kT * j; }, epoch, poll)) L.nmiss = 1;
#pragma unroll
        for (int j = 0; j < kGW; ++j)
            if (need >> j & 1) L.ox[tid + kT * j] = (uint16_t)w[j];
        __syncthreads();
        if (L.nmiss) {  // (uniform) an output never arrived (its producer not running): every output computed here
            for (int gg = 0; gg < a.NKV; ++gg)
                group_fallback<G>(a, L, gg, vv, [&](int o, uint32_t bits) { L.ox[o] = (uint16_t)bits; });
            __syncthreads();
        }
        float acc[2] = {0.f, 0.f};
#pragma unroll
        for (int c = 0; c < kOC; ++c) {
            const u32x4 h4 = *reinterpret_cast<const u32x4*>(&L.ox[(c * 64 + olane) * 8]);
            const uint32_t hw[4] = {h4.x, h4.y, h4.z, h4.w};
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const uint32_t ww[4] = {wo_r[r][c].x, wo_r[r][c].y, wo_r[r][c].z, wo_r[r][c].w};
                float sr = acc[r];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    sr = fmaf(__uint_as_float(ww[j] << 16), __uint_as_float(hw[j] << 16), sr);
                    sr = fmaf(__uint_as_float(ww[j] & 0xFFFF0000u), __uint_as_float(hw[j] & 0xFFFF0000u), sr);
                }
                acc[r] = sr;
            }
        }
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const float tot = wave_sum_xor(acc[r]);
            const int row = b * kORows + 2 * owv + r;
            if (olane == r && row < a.Mo) a.o_out[row] = (uint16_t)f2bf(tot);
        }
    }
    // the last workgroup to start stores this call's epoch for the next call (every workgroup has read the header by
    // then); the count's return is read only here, long after it was issued, as the counts of all workgroups go to one
    // word and come back one after another
    if (tid == 0 && started == total - 1) {
        if (!wrap) st_word(a.hdr, epoch);
        st_word(a.hdr + 1, 0);
    }
    if (wrap) {  // (uniform) the last workgroup to finish clears the tag area and restarts the epochs
        __syncthreads();
        if (tid == 0)
            L.nmiss = __hip_atomic_fetch_add(a.hdr + 2, 1ull, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == total - 1;
        __syncthreads();
        if (L.nmiss) {
            for (uint64_t* p = a.stats + tid; p < a.end; p += kT) st_word(p, 0);
            __syncthreads();
            if (tid == 0) {
                st_word(a.hdr, 0);
                st_word(a.hdr + 2, 0);
            }
        }
    }
}


thread_local const char* t_err = "no error";

int afail(int code, const char* msg) {
    t_err = msg;
    return code;
}

}  // namespace

extern "C" {

size_t moe_attn_workspace_bytes(int n_q_heads, int head_dim, int S) {
    if (n_q_heads < 1 || head_dim != kD || S < 1 || S > kP * kMaxC) return 0;
    const size_t C = (size_t)(S + kP - 1) / kP;
    const size_t scores = ((size_t)n_q_heads * S * sizeof(float) + 255) / 256 * 256;
    // header, scores, tagged statistics, tagged partials, tagged outputs (read by the folded o projection)
    return kHdrBytes + scores + (size_t)n_q_heads * C * 2 * 8 + (size_t)n_q_heads * C * kD * 8 + (size_t)n_q_heads * kD * 8;
}

const char* moe_attn_last_error(void) { return t_err; }

}  // extern "C"

namespace {

// Clears the allocation-free scratch before its first call on a device (a fill kernel, no memset node).
std::mutex g_clear_mu;
__global__ void attn_zero_kernel(uint64_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
}

// Passes of a wait before the fallback computes the missing chunk: 256 (about 100 us), or MOE_ATTN_POLL (0..2^20) as
// read at each call; 0 makes every wait for another workgroup's words end at once (the fallback paths are then taken
// wherever a word is not in yet, which the tests use to check that they give the same bits).
int poll_limit() {
    const char* e = getenv("MOE_ATTN_POLL");
    if (!e || !*e) return 256;
    const long v = strtol(e, nullptr, 10);
    return v < 0 ? 0 : v > (1 << 20) ? (1 << 20) : (int)v;
}

// Per device and G: the LDS limit raised once, and the workgroups of attn_fused_kernel<G> resident at once.
struct KernelInfo {
    bool ready;
    hipError_t err;
    int resident;
};
std::mutex g_info_mu;
std::unordered_map<int, KernelInfo> g_info;

template <int G, bool OPROJ>
hipError_t attn_go(FusedAttn& a, hipStream_t st) {
    const void* fn = reinterpret_cast<const void*>(&attn_fused_kernel<G, OPROJ>);
    const size_t lds = sizeof(AttnLds<G>);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    KernelInfo info;
    {
        std::lock_guard<std::mutex> lock(g_info_mu);
        KernelInfo& ki = g_info[dev * 32 + 2 * G + (OPROJ ? 1 : 0)];
        if (!ki.ready) {
            ki.err = moe::raise_lds_limit(fn, lds);
            int per_cu = 0, cus = 0;
            if (ki.err == hipSuccess) ki.err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kT, lds);
            if (ki.err == hipSuccess) ki.err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
            ki.resident = per_cu * cus;
            ki.ready = true;
        }
        info = ki;
    }
    if (info.err != hipSuccess) return info.err;
    // R chunks per workgroup: the smallest that lets the whole grid be resident (the waits then end without the
    // fallback); the results do not depend on R.
    a.R = 1;
    if (info.resident > 0)
        while ((size_t)((a.C + a.R - 1) / a.R) * a.NKV > (size_t)info.resident && a.R < a.C) ++a.R;
    a.W = (a.C + a.R - 1) / a.R;
    a.Wa = a.W * a.NKV;  // workgroup b < Wa: kv head b / W, chunk group b % W
    int grid = a.Wa;
    if (OPROJ) grid = std::max(grid, (a.Mo + kORows - 1) / kORows);
    hipLaunchKernelGGL((attn_fused_kernel<G, OPROJ>), dim3(grid), dim3(kT), lds, st, a);
    return hipGetLastError();
}

// Checks the arguments and enqueues the kernel with `workspace` (>= moe_attn_workspace_bytes bytes of device memory,
// zero-filled before its first call and written only by these calls) holding the header, the scores, the tagged chunk
// statistics and the tagged partials.  `cleared` (the allocation-free scratch only): false until the scratch has been
// cleared on this device, which this call then does first.
int attn_launch(int n_q_heads, int n_kv_heads, int head_dim, int S, float scale, const uint16_t* q,
                const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out, void* workspace, size_t workspace_bytes,
                void* stream, bool* cleared, const uint16_t* wo = nullptr, int o_rows = 0, uint16_t* o_out = nullptr) {
    if (head_dim != kD) return afail(MOE_GPU_EINVAL, "head_dim must be 128");
    const int G = n_kv_heads >= 1 && n_q_heads % n_kv_heads == 0 ? n_q_heads / n_kv_heads : 0;
    if (G != 1 && G != 2 && G != 4 && G != 8)
        return afail(MOE_GPU_EINVAL, "need n_q_heads = G * n_kv_heads with G in {1, 2, 4, 8}");
    if (S < 1 || S > kP * kMaxC) return afail(MOE_GPU_EINVAL, "S outside [1, 65536]");
    if (!q || !k_cache || !v_cache || !out || !workspace) return afail(MOE_GPU_EINVAL, "null pointer");
    if (wo) {
        if (n_q_heads * head_dim != kOK) return afail(MOE_GPU_EINVAL, "the folded o projection needs n_q_heads * 128 = 4096");
        if (o_rows < 1 || !o_out) return afail(MOE_GPU_EINVAL, "o projection: o_rows < 1 or null o_out");
        if (reinterpret_cast<uintptr_t>(wo) & 15) return afail(MOE_GPU_EINVAL, "w_o must be 16-byte aligned");
    }
    if (workspace_bytes < moe_attn_workspace_bytes(n_q_heads, head_dim, S))
        return afail(MOE_GPU_EINVAL, "workspace smaller than moe_attn_workspace_bytes()");
    if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache) |
         reinterpret_cast<uintptr_t>(workspace)) & 15)
        return afail(MOE_GPU_EINVAL, "k_cache / v_cache / workspace must be 16-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int C = (S + kP - 1) / kP;
    const size_t scores_bytes = ((size_t)n_q_heads * S * sizeof(float) + 255) / 256 * 256;
    unsigned char* ws = static_cast<unsigned char*>(workspace);
    FusedAttn a;
    a.hdr = reinterpret_cast<uint64_t*>(ws);
    a.end = reinterpret_cast<uint64_t*>(ws + workspace_bytes / 8 * 8);
    a.q = q;
    a.k = k_cache;
    a.v = v_cache;
    a.out = out;
    a.scores = reinterpret_cast<float*>(ws + kHdrBytes);
    a.stats = reinterpret_cast<uint64_t*>(ws + kHdrBytes + scores_bytes);
    a.part = a.stats + (size_t)n_q_heads * C * 2;
    a.aout = a.part + (size_t)n_q_heads * C * kD;
    a.wo = wo;
    a.o_out = o_out;
    a.Mo = o_rows;
    a.NQ = n_q_heads;
    a.NKV = n_kv_heads;
    a.S = S;
    a.C = C;
    a.scale = scale;
    a.poll = poll_limit();
    if (cleared) {
        std::lock_guard<std::mutex> lock(g_clear_mu);
        if (!*cleared) {
            hipLaunchKernelGGL(attn_zero_kernel, dim3(1024), dim3(256), 0, st, a.hdr, workspace_bytes / 8);
            const hipError_t ez = hipGetLastError();
            if (ez != hipSuccess) return afail(MOE_GPU_EHIP, hipGetErrorString(ez));
            *cleared = true;
        }
    }
    hipError_t e = hipSuccess;
    if (wo) {
        switch (G) {
            case 1: e = attn_go<1, true>(a, st); break;
            case 2: e = attn_go<2, true>(a, st); break;
            case 4: e = attn_go<4, true>(a, st); break;
            default: e = attn_go<8, true>(a, st); break;
        }
    } else {
        switch (G) {
            case 1: e = attn_go<1, false>(a, st); break;
            case 2: e = attn_go<2, false>(a, st); break;
            case 4: e = attn_go<4, false>(a, st); break;
            default: e = attn_go<8, false>(a, st); break;
        }
    }
    if (e != hipSuccess) return afail(e == hipErrorNoBinaryForGpu ? MOE_GPU_ENOKERNEL : MOE_GPU_EHIP, hipGetErrorString(e));
    return MOE_GPU_OK;
}

// The allocation-free entry point's scratch: the scores, statistics and partials of one call, for up to kScratchMaxNQ
// query heads and kScratchMaxS positions (6.3 MB per GPU, held until the process ends).  Host code never uses the
// array's name as an address: the device address is looked up once per device (hipGetSymbolAddress, with that device
// current) and kept in g_scratch; g_scratch_clear records that the first call on the device cleared it.
constexpr int kScratchMaxNQ = 64, kScratchMaxS = 8192;
constexpr size_t kScratchBytes = kHdrBytes + (size_t)kScratchMaxNQ * kScratchMaxS * sizeof(float) +
                                 (size_t)kScratchMaxNQ * (kScratchMaxS / kP) * (2 + kD) * 8 + (size_t)kScratchMaxNQ * kD * 8;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];
constexpr int kMaxDevices = 64;
void* g_scratch[kMaxDevices];
bool g_scratch_clear[kMaxDevices];
std::mutex g_scratch_mu;

int scratch_of_current_device(void** ptr, bool** cleared) {
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
    *cleared = &g_scratch_clear[dev];
    return MOE_GPU_OK;
}

}  // namespace

extern "C" {

int moe_attn_decode_dev(int n_q_heads, int n_kv_heads, int head_dim, int S, float scale, const uint16_t* q,
                        const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out, void* workspace,
                        size_t workspace_bytes, void* stream) {
    return attn_launch(n_q_heads, n_kv_heads, head_dim, S, scale, q, k_cache, v_cache, out, workspace, workspace_bytes,
                       stream, nullptr);
}

int moe_attn_decode_oproj_dev(int n_q_heads, int n_kv_heads, int head_dim, int S, float scale, const uint16_t* q,
                              const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out, const uint16_t* w_o,
                              int o_rows, uint16_t* o_out, void* workspace, size_t workspace_bytes, void* stream) {
    if (!w_o) return afail(MOE_GPU_EINVAL, "null w_o");
    return attn_launch(n_q_heads, n_kv_heads, head_dim, S, scale, q, k_cache, v_cache, out, workspace, workspace_bytes,
                       stream, nullptr, w_o, o_rows, o_out);
}

size_t moe_attn_noalloc_max_bytes(void) { return kScratchBytes; }

int moe_attn_decode_noalloc_dev(int n_q_heads, int n_kv_heads, int head_dim, int S, float scale, const uint16_t* q,
                                const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out, void* stream) {
    const size_t need = moe_attn_workspace_bytes(n_q_heads, head_dim, S);
    if (need == 0) return afail(MOE_GPU_EINVAL, "bad n_q_heads / head_dim / S");
    if (need > kScratchBytes)
        return afail(MOE_GPU_EINVAL, "n_q_heads * S beyond the allocation-free scratch (moe_attn_noalloc_max_bytes)");
    void* ws = nullptr;
    bool* cleared = nullptr;
    const int rc = scratch_of_current_device(&ws, &cleared);
    if (rc != MOE_GPU_OK) return rc;
    return attn_launch(n_q_heads, n_kv_heads, head_dim, S, scale, q, k_cache, v_cache, out, ws, kScratchBytes, stream,
                       cleared);
}

}  // extern "C"
