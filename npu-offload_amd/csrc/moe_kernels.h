// moe_kernels.h — device data layout and launch helpers shared by the HIP kernels and the C ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace moe {

constexpr int kTileRows = 64;      // rows per weight tile: one row per lane of a wavefront
constexpr int kChunk = 8;          // bf16 elements per 16-byte chunk
constexpr int kChunkQ8 = 16;       // int8 elements per 16-byte chunk
constexpr int kWaves = 4;          // wavefronts per workgroup in the GEMV kernels
constexpr int kThreads = kWaves * 64;
constexpr int kMaxTokens = 16;     // tokens per call (T * topk <= 128 entries for the grouping unit)
constexpr int kMaxTopk = 8;
constexpr int kMaxShared = 4;
constexpr int kMaxExperts = 512;
constexpr int kMaxSlots = kMaxShared + kMaxTokens * kMaxTopk;
#ifndef MOE_ROUTER_ROWS
#define MOE_ROUTER_ROWS 8
#endif
constexpr int kRouterRows = MOE_ROUTER_ROWS;  // router rows per router unit (2, 4 or 8): two per wavefront
constexpr int kRouterTG = 2;                  // tokens per router unit when a call has several
// Router units of a call: row groups of kRouterRows, times token groups of kRouterTG when T > 1 (unit u: row group
// u % row groups, token group u / row groups).
inline int router_units(int E, int T) {
    const int nrg = (E + kRouterRows - 1) / kRouterRows;
    return T > 1 ? nrg * ((T + kRouterTG - 1) / kRouterTG) : nrg;
}

// Routing rules of the compute calls (the flag bits MOE_GPU_ROUTE_* of the C ABI select them).
enum RouteRule { kRouteSoftmax = 0, kRouteSigmoid = 1 };

// Per-call expert grouping, built on the device: slot s < n_shared is shared expert s (expert = -1 - s) over all
// tokens; routed slots follow in first-seen order scanning tokens then ranks (solar_hybrid/runtime.py:344-347).
struct Slots {
    int nslot;
    int err;  // 1: an id outside [-1, E); 2: an expert repeated within one token (device-side validation)
    int pad_[2];
    int expert[kMaxSlots];
    int ntok[kMaxSlots];
    int tok[kMaxSlots][kMaxTokens];
    int rank[kMaxSlots][kMaxTokens];  // routed: rank of this expert in token tok's top-k; shared: -1
    int pair[kMaxSlots];              // first (slot, token) pair of the slot: shared s -> s * T, routed slots follow
    int vid[kMaxTokens * kMaxTopk];   // [t][k] expert whose down output the combine reads; -1: none (empty/dropped)
    float vgate[kMaxTokens * kMaxTopk];  // [t][k] gate used by the combine
};

// Where a layer's weights live.  Routed expert e's bf16 gate|up table starts at gu + e * gu_stride (elements), its down
// table at dn + e * dn_stride; shared expert s at sgu + s * gu_stride, sdn + s * dn_stride.  int8 copies: gu_q8 + e *
// q8_gu_stride (bytes), dn_q8 + e * q8_dn_stride, scales sc_q8 + e * (2F + H) (gate|up rows in tile order, then down).
struct LayerPtrs {
    const uint16_t* wr;
    const float* bias;
    const uint16_t* gu;
    const uint16_t* dn;
    const uint16_t* sgu;
    const uint16_t* sdn;
    const int8_t* gu_q8;
    const int8_t* dn_q8;
    const float* sc_q8;
};

struct Dims {
    int H, F, E, k, n_shared, max_t;
    __host__ __device__ size_t gu_stride() const { return (size_t)2 * F * H; }
    __host__ __device__ size_t dn_stride() const { return (size_t)H * F; }
};

// Tiled layouts (element offsets):
//   gate|up bf16: [F/32 tiles][H/8 chunks][64 rows][8];   tile row i -> f = 32*tile + 8*(i/16) + i%8, up = (i/8)%2
//   down bf16:    [H/64 tiles][F/8 chunks][64 rows][8];   tile row i -> h = 64*tile + i
//   int8 twins use 16-element chunks: [F/32][H/16][64][16] and [H/64][F/16][64][16].
__host__ __device__ inline int gu_row_f(int tile, int i) { return 32 * tile + 8 * (i >> 4) + (i & 7); }
__host__ __device__ inline int gu_row_up(int i) { return (i >> 3) & 1; }

constexpr int kMaxHTiles = 256;  // H <= 16384 (64-row down tiles)
constexpr int kMaxKp = 4;        // K parts of a gate|up tile

// Where a call's token activations come from.  x: the MoE input [T][H] bf16 as given.  Block mode (resid != null,
// a decode layer's second half, track2_opt/solar_engine/src/main.rs:120-124): the input is
// rmsnorm(bf16(resid + attn_o), norm_w) (host.rs:71-76), computed by every workgroup that stages it.
struct StageSrc {
    const uint16_t* x;       // [T][H] bf16, or null in block mode
    const uint16_t* resid;   // [T][H] bf16 residual stream before the attention output is added
    const uint16_t* attn_o;  // [T][H] bf16 attention block output (o_proj, rounded)
    const uint16_t* norm_w;  // [H] bf16 post-attention RMSNorm weight
    float eps;
};

// Everything one expert pipeline call needs (device pointers).
struct ExpertArgs {
    LayerPtrs L;
    Dims d;
    int T, keep, n_shared, int8, accumulate;  // n_shared: shared experts summed in this call (0 or d.n_shared)
    int maxs;                                 // slots this call can use: d.n_shared + T * keep
    StageSrc in;                              // the tokens' activations
    float* out;                               // [T][H] fp32, or null in block mode
    uint16_t* x_next;                         // block mode: the next residual [T][H] bf16, else null
    int32_t* ids;                             // [T][k]
    float* gates;                             // [T][k]
    Slots* slots;
    // cross-workgroup intermediates, tagged words (epoch << 32) | payload
    uint64_t* act;                            // [maxs][max_t][F/2] pairs of bf16 SiLU(g)*u
    uint64_t* ypart;                          // [T][n_shared + k][H] fp32 down outputs
    uint64_t* gpart;                          // [pairs][F/32][kMaxKp][64] fp32 partial sums of split gate|up tiles
    int kp;                                   // K parts of a routed slot's gate|up tile (1, 2 or 4): one unit each
    int kps;                                  // K parts of a shared slot's gate|up tile (1, 2 or 4)
    unsigned epoch;                           // this call's tag (never 0)
    unsigned* err;                            // set when a bounded wait gave up (sticky until the host clears it)
};

// Work-queue heads of the fused kernel.  Fused launch n (the host counts them) hands out units from
// next_unit[n & 1] and clears next_unit[(n + 1) & 1] for the next launch; the unfused path clears both.  Each head
// sits in its own 128-byte line.  Workgroup b < min(grid, router units) runs router unit b first; every other unit
// is handed out by the queue, in ascending order, to a running workgroup.
constexpr int kSyncPad = 32;  // unsigneds per line
struct Sync {
    unsigned err;  // set when a bounded wait gave up (sticky until the host clears it)
    unsigned pad0_[kSyncPad - 1];
    unsigned next_unit[2 * kSyncPad];
};

// Unit trace record (fused kernel, optional): start, inputs ready, end (100 MHz s_memrealtime ticks), workgroup,
// aux, aux2.  Inputs ready: routed gate|up part: routing known; combining down unit: the other terms in; else 0.
// aux: gate|up finishing part: sibling partials in; down unit: act rows staged; router unit: its operands in (weights
// loaded, tokens staged); else 0.  aux2: down unit: weight stream done; router unit: dot products done; else 0.
constexpr int kTraceFields = 6;

struct FusedArgs {
    ExpertArgs e;
    uint64_t* logits;  // [T][E] tagged router logits
    Sync* sync;
    uint64_t* trace;  // optional: per unit {start, dependencies met, end, workgroup} in 100 MHz realtime ticks
    int nR;         // router units (0 when the caller gives ids)
    int do_topk;
    int rule;       // RouteRule
    int phase;      // work-queue head of this launch (fused launch count & 1)
    int lag;        // queue order: routed slot s's down block follows routed slot (s + lag)'s gate|up block (lag >= 1)
    int shared_waits;  // 1: shared gate|up parts start only once the routing is known
    // passes of the bounded wait for the router logits before a workgroup computes the missing router rows itself
    // (a router unit whose workgroup is not resident never blocks the routing); 0: compute them as soon as one is
    // missing at the first look
    int router_poll;
};

// Fused-kernel unit count: router units, the route publisher, then every slot's gate|up and down units (S shared
// slots of kps parts per gate|up tile, maxs - S routed slots of kp parts).
__host__ __device__ inline int fused_units(int nR, int maxs, int S, int F, int H, int kp, int kps) {
    return nR + 1 + (S * kps + (maxs - S) * kp) * (F / 32) + maxs * (H / 64);
}
// Gate|up units of the unfused kernel: one per (slot, tile, K part), shared slots first.
__host__ __device__ inline int gateup_units(int maxs, int S, int F, int kp, int kps) {
    return (S * kps + (maxs - S) * kp) * (F / 32);
}

size_t lds_bytes(int T, int NT, int H, int F, int E);

// ---- launch helpers (moe_kernels.hip) ---------------------------------------------------------------------------
// logits: tagged [T][E] (always written); logits_out: optional plain fp32 copy
hipError_t launch_router(const LayerPtrs& L, const Dims& d, int T, const StageSrc& in, uint64_t* logits,
                         float* logits_out, unsigned epoch, hipStream_t st);
hipError_t launch_topk_group(const LayerPtrs& L, const Dims& d, int T, int keep, int n_shared, bool do_topk, int rule,
                             const uint64_t* logits, unsigned epoch, unsigned* err, int32_t* ids, float* gates,
                             Slots* slots, hipStream_t st);
// gate|up parts; also clears the fused work-queue heads (the unfused path does not use them)
hipError_t launch_gateup(const ExpertArgs& a, Sync* sync, hipStream_t st);
// down projection + the gated combine (the down unit of the last slot combines each 64-row tile)
hipError_t launch_down(const ExpertArgs& a, hipStream_t st);
// wg_per_cu <= 0: as many workgroups per CU as fit (a plain launch: the work queue needs no co-residency);
// grid > 0 overrides the grid size (it may exceed what fits at once); grid_out receives the grid size
hipError_t launch_fused(const FusedArgs& f, int wg_per_cu, int grid, hipStream_t st, int* grid_out);

hipError_t launch_relayout_gu(const uint16_t* g, const uint16_t* u, int H, int F, uint16_t* dst, hipStream_t st);
// router table [E][H] bf16 (row-major, src) -> the chain order the router units read (dst, same size)
hipError_t launch_relayout_router(const uint16_t* src, int E, int H, uint16_t* dst, hipStream_t st);
hipError_t launch_relayout_dn(const uint16_t* d, int H, int F, uint16_t* dst, hipStream_t st);
hipError_t launch_relayout_q8(const int8_t* q, const float* sc, int H, int F, int8_t* gu_dst, int8_t* dn_dst,
                              float* sc_dst, hipStream_t st);
hipError_t launch_unlayout_q8(const int8_t* gu_src, const int8_t* dn_src, const float* sc_src, int H, int F, int8_t* q,
                              float* sc, hipStream_t st);
hipError_t launch_quantize(const uint16_t* gu, const uint16_t* dn, int H, int F, int n_exp, size_t gu_stride,
                           size_t dn_stride, int8_t* gu_q8, int8_t* dn_q8, float* sc, hipStream_t st);
hipError_t launch_synth_tiled(uint64_t key_g, uint64_t key_u, uint64_t key_d, float c, int H, int F, uint16_t* gu,
                              uint16_t* dn, hipStream_t st);
hipError_t launch_synth_fill(uint16_t* dst, uint64_t n, uint64_t key, uint64_t start, float c, hipStream_t st);
hipError_t launch_zero(uint64_t* dst, size_t n, hipStream_t st);

uint64_t synth_key(uint64_t seed, uint64_t tensor_id);
// Returns true when the code object holds kernels for the current device.
bool kernels_available();

}  // namespace moe
