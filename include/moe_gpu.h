/*
 * moe_gpu.h — C ABI of the MI355X (gfx950) routed-MoE expert tier.
 *
 * The library replaces, for one GPU holding every expert of every layer in HBM, the expert tiers of
 * npu-offload's Rust engine (track2_opt/solar_engine): the NPU expert kernels driven through chip.rs and the host
 * CPU cold-expert path bound by the extern "C" block of track2_opt/solar_engine/src/host.rs:18-37 (compiled from
 * track2_opt/solar_engine/csrc/cpu_kern.c).  Conventions follow that block:
 *   - bf16 travels as raw uint16_t bits; int8 weights as int8_t; gates and outputs as fp32; dimensions are int.
 *   - The caller owns every buffer it passes.  The library owns its HBM tables and per-call workspace.
 *   - Unlike the void ck_* functions, every entry point returns MOE_GPU_OK (0) or a negative MOE_GPU_E* code and
 *     keeps a message for moe_gpu_last_error() (the engine's chip replies are eyre::Result, chip.rs:59).
 *   - A context is thread-affine: one host thread drives one context (the chip-thread pattern, chip.rs:96-143).
 *
 * Shapes: H hidden, F expert intermediate, E routed experts, k = topk, S = n_shared always-on experts, T tokens.
 * Constraints: H % 512 == 0, H <= 16384, F % 256 == 0, E <= 512, 1 <= k <= 8, 0 <= S <= 4, 1 <= T <= max_tokens <= 16,
 * max_tokens * H * 2 <= 96 KB (the tokens' activations are staged in LDS).
 *
 * Expert math (solar_hybrid/cpu_moe.cpp:38-96 semantics): for expert e and token t,
 *   g = Wg_e x_t, u = Wu_e x_t (fp32 accumulation of bf16 products), act = bf16(silu(g) * u),
 *   y_e[t] = Wd_e act (fp32).
 * Router logits: logits[t, e] = W_r[e] . x[t] in the reference's own summation order (ck_gemv, cpu_kern.c:9-19,
 * :31-35): bit-identical to it whenever no product or partial sum is a denormal fp32 number.
 * Routing, by the context's MOE_GPU_OPT_ROUTE_RULE (ties in the selection always go to the lower expert index):
 *   MOE_GPU_ROUTE_SOFTMAX (default; npu-kernels/.../layer_template/src/host.rs.tpl:247-267): score = logits + bias;
 *     the k largest scores are selected; gates over the first `keep` ranks are the softmax restricted to them
 *     (renormalised); ranks >= keep are dropped (their gate is 0).
 *   MOE_GPU_ROUTE_SIGMOID (Solar's route(), track2_opt/solar_engine/src/host.rs:119-128): s = 1 / (1 + exp(-logit)),
 *     selection by s + bias (the bias only selects), gates s_r / (sum_{q < keep} s_q + 1e-20).
 * Combine, per token, in this fixed order: out[t] (= 0, or the caller's value with MOE_GPU_ACCUMULATE)
 *   += y_shared_s[t] for s = 0..S-1, then += gate[t,r] * y_{id[t,r]}[t] for r = 0..keep-1 (one fused multiply-add
 *   per term).  A token's result does not depend on which other tokens share the call.
 */
#ifndef MOE_GPU_H
#define MOE_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct moe_gpu moe_gpu;

enum {
    MOE_GPU_OK = 0,
    MOE_GPU_EINVAL = -1,   /* bad argument, shape or layer/expert index */
    MOE_GPU_EHIP = -2,     /* HIP runtime error (message has hipGetErrorString) */
    MOE_GPU_ENOMEM = -3,   /* HBM allocation failed */
    MOE_GPU_ESTATE = -4,   /* weights not loaded for the requested layer / path */
    MOE_GPU_ENOKERNEL = -5 /* the HIP code object for this GPU is missing (wrong arch) */
};

/* flags for the compute calls */
#define MOE_GPU_ACCUMULATE 1u /* out += result (ck_* semantics, cpu_kern.c:141 `out[h] += ...`) instead of out = result */
#define MOE_GPU_INT8 2u       /* routed experts use their int8 weight-only copy (ck_moe_q8w, cpu_kern.c:306-333) */

/* ----------------------------------------------------------------------------------------------- context
 * Replaces Chip::spawn (track2_opt/solar_engine/src/chip.rs:96-111) for a HIP device: creates the stream and the
 * per-call workspace.  Layer tables are allocated on first load, each kind on its own (router, bf16 routed experts,
 * shared experts, int8 routed experts): a layer whose routed experts are only loaded as int8 holds no bf16 routed
 * tables.  n_layers bounds the layer index.
 * The layer / moe calls refuse a stream that is capturing a graph (MOE_GPU_ESTATE): their epochs and work queue are
 * per launch, so a replayed launch would read the previous replay's words. */
int moe_gpu_create(int device, int H, int F, int E, int topk, int n_shared, int n_layers, int max_tokens,
                   moe_gpu** out);
void moe_gpu_destroy(moe_gpu* ctx);
/* Message of the last failing call on this context (never NULL).  With ctx == NULL: the last create() failure. */
const char* moe_gpu_last_error(const moe_gpu* ctx);
/* Run subsequent work on `stream` (a hipStream_t, e.g. the caller's current stream); NULL restores the
 * context's own stream. */
int moe_gpu_set_stream(moe_gpu* ctx, void* stream);
int moe_gpu_synchronize(moe_gpu* ctx);

/* ----------------------------------------------------------------------------------------------- weights
 * Host row-major bf16 -> HBM in the GPU layout.  Replaces the expert-table upload of chip.rs:208-233 and the
 * NUMA placement ck_place_expert (cpu_kern.c:124-138, host.rs:144-153).  g, u: [F,H]; d: [H,F]. */
int moe_gpu_load_expert(moe_gpu* ctx, int layer, int e, const uint16_t* g, const uint16_t* u, const uint16_t* d);
/* Always-on shared expert s (gate 1.0): host's moe_cpu(&[sh], &[1.0]) at main.rs:131-135. */
int moe_gpu_load_shared(moe_gpu* ctx, int layer, int s, const uint16_t* g, const uint16_t* u, const uint16_t* d);
/* Router weight wr [E,H] bf16 (mlp.gate.weight, main.rs:129) and optional per-expert score bias [E] (NULL = 0). */
int moe_gpu_load_router(moe_gpu* ctx, int layer, const uint16_t* wr, const float* bias);
/* Device-pointer twins of the three loads (source already in HBM, e.g. a safetensors slab copied once). */
int moe_gpu_load_expert_dev(moe_gpu* ctx, int layer, int e, const uint16_t* g, const uint16_t* u, const uint16_t* d);
int moe_gpu_load_shared_dev(moe_gpu* ctx, int layer, int s, const uint16_t* g, const uint16_t* u, const uint16_t* d);
/* int8 weight-only copy of routed expert e in ck_place_expert_q8's layout (cpu_kern.c:226-241):
 * q = [(2F + H) rows] (gate rows, up rows: length H; then down rows: length F), sc = [2F + H] fp32 row scales. */
int moe_gpu_load_expert_q8(moe_gpu* ctx, int layer, int e, const int8_t* q, const float* sc);
/* Quantise the resident bf16 routed experts [e0, e1) of a layer on the device with quant_row's rule
 * (cpu_kern.c:218-224: s = max|w|/127 or 1, q = rint(w * (1/s)) clamped to +-127); bit-identical to the host
 * quantiser.  Replaces ck_place_expert_q8 at engine init (main.rs:509-516). */
int moe_gpu_quantize_experts(moe_gpu* ctx, int layer, int e0, int e1);
/* Read back the int8 copy of expert e in ck_place_expert_q8's layout (for checks). */
int moe_gpu_get_expert_q8(moe_gpu* ctx, int layer, int e, int8_t* q, float* sc);

/* ----------------------------------------------------------------------------------------------- compute (host buffers)
 * Synchronous; x [T,H] bf16, out [T,H] fp32, ids/gates [T,k].  */

/* Router GEMV + top-k on the device (the context's routing rule, MOE_GPU_OPT_ROUTE_RULE: softmax by default, or
 * Solar's sigmoid rule): replaces ck_gemv(mlp.gate.weight) (cpu_kern.c:31-35, main.rs:129; the logits are its bits) or
 * the NPU shared_router logits (dense/shared.rs:191-210) followed by the host route() (host.rs:119-128).  keep <= 0
 * means keep = k.  logits [T,E] may be NULL. */
int moe_gpu_route(moe_gpu* ctx, int layer, int T, const uint16_t* x, int keep, int32_t* ids, float* gates,
                  float* logits);
/* Grouped routed experts + shared experts + combine for caller-chosen ids/gates [T,k]: replaces ck_moe3
 * (cpu_kern.c:141-172, via moe_cpu_placed host.rs:156-159), ck_moe_q8w (with MOE_GPU_INT8), the batched cpu_moe
 * (cpu_moe.cpp:38-96) and the NPU ffn_k8/experts_b + combine kernels dispatched by moe_phase (main.rs:149-209).
 * Ranks >= keep are skipped (keep <= 0: all k), and so is any rank whose id is -1 (a token may carry fewer experts
 * than keep, as the variable-E ck_* calls do).  Gates are used as given (no renormalisation).
 * with_shared = 0 leaves the shared experts out (the routed-only sum of ck_moe3). */
int moe_gpu_moe(moe_gpu* ctx, int layer, int T, const uint16_t* x, const int32_t* ids, const float* gates, int keep,
                int with_shared, unsigned flags, float* out);
/* route + moe in one call, ids never leave the device (LayerA2 + ExpertsB of chip.rs combined).
 * ids/gates may be NULL; when given they receive the routing decision. */
int moe_gpu_layer(moe_gpu* ctx, int layer, int T, const uint16_t* x, int keep, unsigned flags, float* out,
                  int32_t* ids, float* gates);

/* ----------------------------------------------------------------------------------------------- compute (device buffers)
 * Same operations on device pointers, enqueued on the context's stream without synchronising. */
int moe_gpu_route_dev(moe_gpu* ctx, int layer, int T, const uint16_t* x, int keep, int32_t* ids, float* gates,
                      float* logits);
/* moe_dev cannot check device-side ids, so it requires every routed expert of the layer to be loaded in the call's
 * precision (with MOE_GPU_INT8: a current int8 copy of each; a bf16 reload makes an expert's int8 copy stale). */
int moe_gpu_moe_dev(moe_gpu* ctx, int layer, int T, const uint16_t* x, const int32_t* ids, const float* gates,
                    int keep, int with_shared, unsigned flags, float* out);
int moe_gpu_layer_dev(moe_gpu* ctx, int layer, int T, const uint16_t* x, int keep, unsigned flags, float* out,
                      int32_t* ids, float* gates);
/* A decode layer's second half as one call (track2_opt/solar_engine/src/main.rs:120-141, the residual add, the
 * post-attention RMSNorm and moe_host): with r = bf16(resid + attn_o) and h2 = rmsnorm(r, norm_w) (host.rs:71-76;
 * the sum of squares in the GPU's fixed order), the layer call on h2 (routing by the context's rule), then
 *   x_next = bf16(r + bf16(bf16(routed) + bf16(shared)))   (the routed and shared sums as moe_host rounds them).
 * resid, attn_o, x_next [T, H] bf16, norm_w [H] bf16; out [T, H] fp32 (the layer output, optional), ids / gates
 * optional.  MOE_GPU_ACCUMULATE is not accepted.  Device pointers, enqueued, not synchronised. */
int moe_gpu_block_dev(moe_gpu* ctx, int layer, int T, const uint16_t* resid, const uint16_t* attn_o,
                      const uint16_t* norm_w, float eps, int keep, unsigned flags, uint16_t* x_next, float* out,
                      int32_t* ids, float* gates);

/* ----------------------------------------------------------------------------------------------- bench/test support
 * No reference counterpart.  Deterministic synthetic weights generated in HBM (no host upload), bit-identical to the
 * host generator of the test suite: element i of tensor `tid` = bf16((float)(IrwinHall8(mix64 stream of key) - mean)
 * * c), key = synth_key(seed, tid); tid = (layer * 4096 + e) * 4 + m, m = 0 gate, 1 up, 2 down (shared s: e = 4000+s;
 * router: e = 4095, m = 0); i = row-major index in the logical matrix.  c = sigma / 53509.9... */
int moe_gpu_synth_layer(moe_gpu* ctx, int layer, uint64_t seed, float c_weight, const float* bias);
int moe_gpu_synth_fill(moe_gpu* ctx, uint16_t* dst_dev, uint64_t n, uint64_t key, uint64_t start, float c);
uint64_t moe_gpu_synth_key(uint64_t seed, uint64_t tensor_id);
/* Duration in ms of the last compute call's kernels when timing is enabled (hipEvents on the context stream). */
int moe_gpu_enable_timing(moe_gpu* ctx, int on);
int moe_gpu_last_time_ms(moe_gpu* ctx, float* ms);
/* Execution options.  MOE_GPU_OPT_FUSED (default 1): each layer/moe call of up to 8 tokens (calls of 9 to 16 tokens,
 * possible for H <= 3072, always take the unfused kernels) is one persistent kernel that walks router
 * rows, top-k/grouping, gate|up tile parts and down tiles (a work queue; cross-workgroup values are epoch-tagged words
 * that their consumers poll); 0 runs
 * one kernel per phase (same arithmetic, bit-identical results).  MOE_GPU_OPT_WG_PER_CU: fused grid size in
 * workgroups per CU (default 1; 0 = as many as fit).  MOE_GPU_OPT_LAST_GRID (read only): grid of the last fused
 * launch.  MOE_GPU_OPT_KSPLIT: K parts per routed gate|up tile, 1, 2 or 4 (0 = automatic: whole tiles in bf16 calls,
 * about 128 K weights per part in MOE_GPU_INT8 calls); it changes the summation order, identically in both paths.
 * MOE_GPU_OPT_KSPLIT_SHARED: the same for the shared experts' tiles (0 = automatic: about 64 K weights per part, 128 K
 * in MOE_GPU_INT8 calls).
 * MOE_GPU_OPT_LAG: fused queue order, a routed slot's down tiles are queued after the gate|up parts of the routed
 * slot `lag` places later (0 = automatic: 8).  MOE_GPU_OPT_SHARED_WAITS: 1
 * holds the shared experts' gate|up parts until the routing is known (0 = stream them while routing).
 * MOE_GPU_OPT_GRID: fused grid size in workgroups (0 = automatic: what fits at once); a larger grid is allowed (units
 * are handed out by a queue to running workgroups only, so a grid that is not all resident still completes).
 * MOE_GPU_OPT_ROUTER_POLL: passes of the bounded wait for the router logits (default 1024) after which a workgroup
 * computes the missing router rows itself (a router unit whose workgroup is not resident then cannot hold the call
 * up); 0 computes them at the first miss (a test of that path; the bits are the same).  MOE_GPU_OPT_ROUTE_RULE:
 * MOE_GPU_ROUTE_SOFTMAX (default) or MOE_GPU_ROUTE_SIGMOID, see the routing rules above. */
#define MOE_GPU_OPT_FUSED 1
#define MOE_GPU_OPT_WG_PER_CU 2
#define MOE_GPU_OPT_LAST_GRID 3
#define MOE_GPU_OPT_KSPLIT 4
#define MOE_GPU_OPT_LAG 5
#define MOE_GPU_OPT_SHARED_WAITS 6
#define MOE_GPU_OPT_KSPLIT_SHARED 7
#define MOE_GPU_OPT_GRID 8
#define MOE_GPU_OPT_ROUTER_POLL 9
#define MOE_GPU_OPT_ROUTE_RULE 10
#define MOE_GPU_ROUTE_SOFTMAX 0
#define MOE_GPU_ROUTE_SIGMOID 1
int moe_gpu_set_option(moe_gpu* ctx, int opt, int value);
int moe_gpu_get_option(moe_gpu* ctx, int opt, int* value);
/* The context's shape as created (any pointer may be NULL). */
int moe_gpu_get_shape(moe_gpu* ctx, int* H, int* F, int* E, int* topk, int* n_shared, int* n_layers);
/* Unit trace of the fused kernel: with on != 0, each fused launch records for every unit of its work list
 * {start, inputs ready, end, workgroup, aux, aux2} in the 100 MHz s_memrealtime clock.  Inputs ready: a routed gate|up
 * part's routing known, a combining down unit's other terms in, else 0; aux: a gate|up tile's finishing part has its
 * sibling parts' sums, a down unit its act rows, a router unit its operands, else 0; aux2: a down unit's weight stream
 * done, a router unit's dot products done, else 0.  read_trace
 * copies the last launch's records (6 uint64 per unit, in the fused kernel's unit order). */
int moe_gpu_trace_units(moe_gpu* ctx, int on);
int moe_gpu_read_trace(moe_gpu* ctx, uint64_t* buf, int max_units, int* units);
/* Per-kernel profiling: with on != 0 every kernel launched by the compute calls is bracketed by a hipEvent pair on the
 * stream it runs on.  profile_read synchronises and returns, for kernel slot `kernel` (0 .. moe_gpu_profile_slots()-1),
 * the summed duration and the launch count since the last reset, and its kernel symbol name. */
int moe_gpu_profile_kernels(moe_gpu* ctx, int on);
int moe_gpu_profile_slots(void);
int moe_gpu_profile_read(moe_gpu* ctx, int kernel, double* total_ms, int* launches, const char** name);
int moe_gpu_profile_reset(moe_gpu* ctx);

/* ----------------------------------------------------------------------------------------------- LM head
 * The step's tail after the last layer: final RMSNorm, LM-head GEMV over the vocabulary, greedy argmax.  Replaces the
 * host step's `rmsnorm(x, model.norm.weight)`, `gemv(lm_head.weight)` and first-maximum loop
 * (track2_opt/solar_engine/src/main.rs:381-386, host.rs:71-76) and the chip's lm_head_am + best_key
 * (src/dense/lm_head.rs:174-181, src/chip.rs:183-194).  Its own context: the table is [V, H] bf16 (1.61 GB for
 * V = 196608, H = 4096) and is streamed once per call for up to 4 tokens.
 *   hn[t] = bf16(bf16(x[t] * r) * w_final), r = 1 / sqrt(sum(x[t]^2) / H + eps)   (fp32; sum order is the GPU's)
 *   logit[t, v] = sum_h W[v, h] * hn[t, h]   (fp32 accumulation of bf16 products)
 *   ids[t] = the row of the largest logit, exact ties -> lowest row; best[t] its value.  MOE_HEAD_ARGMAX_FP32 compares
 *   the fp32 logits (main.rs:384-385), MOE_HEAD_ARGMAX_BF16 the logits rounded to bf16 (chip.rs:183-194).
 * Constraints: H % 1024 == 0, 1024 <= H <= 16384, V >= 1, 1 <= T <= 64. */
typedef struct moe_head moe_head;
#define MOE_HEAD_ARGMAX_FP32 0
#define MOE_HEAD_ARGMAX_BF16 1
int moe_head_create(int device, int H, int V, float eps, moe_head** out);
void moe_head_destroy(moe_head* h);
const char* moe_head_last_error(const moe_head* h); /* h == NULL: the last failed create */
int moe_head_set_stream(moe_head* h, void* stream);
int moe_head_synchronize(moe_head* h);
/* w_lm [V, H] bf16 row-major (lm_head.weight), w_final [H] bf16 (model.norm.weight); host or device pointers */
int moe_head_load(moe_head* h, const uint16_t* w_lm, const uint16_t* w_final);
int moe_head_load_dev(moe_head* h, const uint16_t* w_lm, const uint16_t* w_final);
/* x [T, H] bf16 residual stream; ids [T]; best [T]; logits [T, V] fp32 or NULL.  Host pointers, synchronous. */
int moe_head_argmax(moe_head* h, int T, const uint16_t* x, int rule, int32_t* ids, float* best, float* logits);
/* The same on device pointers, enqueued on the head's stream and not synchronised. */
int moe_head_argmax_dev(moe_head* h, int T, const uint16_t* x, int rule, int32_t* ids, float* best, float* logits);

/* Per-layer RMSNorm (input_layernorm / post_attention_layernorm; host.rs:71-76, as the head's final norm above):
 * out[t] = bf16(bf16(x[t] * r) * w), r = 1 / sqrt(sum(x[t]^2) / H + eps).  x, out [T, H] bf16, w [H] bf16; device
 * pointers, enqueued on `stream` (NULL: the null stream).  Returns MOE_GPU_EINVAL / MOE_GPU_EHIP without a message. */
int moe_rmsnorm_dev(int T, int H, const uint16_t* x, const uint16_t* w, float eps, uint16_t* out, void* stream);

/* Projection GEMV of one token with the host's rounding (main.rs:109-111, :119: gemv then round_bf): y[m] = bf16(sum_k
 * W[m,k] x[k]) (fp32 accumulation in the GPU's order).  W [M, K] bf16 row-major, x [K], y [M]; K % 1024 == 0,
 * K <= 65536, W and x 16-byte aligned.  Device pointers, enqueued on `stream`. */
int moe_gemv_dev(int M, int K, const uint16_t* W, const uint16_t* x, uint16_t* y, void* stream);
/* fp32 GEMV in the reference's own order: y[m] = W[m] . x summed exactly as ck_gemv does (cpu_kern.c:9-19, :31-35: two
 * 16-lane vdpbf16ps accumulators over 64-element steps, then GCC's reduce tree), so y is bit-identical to ck_gemv's
 * whenever no product or partial sum is a denormal fp32 number.  K % 512 == 0, K <= 65536, W and x 16-byte aligned.
 * Device pointers, enqueued on `stream`. */
int moe_gemv_f32_dev(int M, int K, const uint16_t* W, const uint16_t* x, float* y, void* stream);
/* The same GEMV on rmsnorm(x, norm_w) (host.rs:71-76), which each workgroup computes from the residual x [K] itself:
 * a layer's input norm folded into its q|k|v projection (main.rs:108-111).  The sum of squares runs in the GPU's fixed
 * order (per thread over strided elements, a 64-lane butterfly, then the 4 wavefronts in order). */
int moe_gemv_norm_dev(int M, int K, const uint16_t* W, const uint16_t* x, const uint16_t* norm_w, float eps,
                      uint16_t* y, void* stream);
/* Rotary embedding in place (main.rs:65-77, HF rotate_half in bf16): for each of n_heads rows of head_dim,
 * x[i] = bf16(bf16(x[i] * cos[i]) + bf16(rot[i] * sin[i])), rot = (-x[D/2..D), x[0..D/2)).  cos_row / sin_row: the
 * bf16 [head_dim] rows of the position (rope_cos.bin / rope_sin.bin).  head_dim even, <= 1024. */
int moe_rope_dev(int n_heads, int head_dim, uint16_t* x, const uint16_t* cos_row, const uint16_t* sin_row,
                 void* stream);
/* The step between the projection and attention in one launch (main.rs:112-118): qkv = [q (NQ*D) | k (NKV*D) |
 * v (NKV*D)] bf16; q is roped in place, k is roped into k_cache[pos] and v copied into v_cache[pos] (caches
 * [max_ctx, NKV, D]).  Device pointers, enqueued on `stream`. */
int moe_rope_append_dev(int n_q_heads, int n_kv_heads, int head_dim, uint16_t* qkv, const uint16_t* cos_row,
                        const uint16_t* sin_row, uint16_t* k_cache, uint16_t* v_cache, int pos, void* stream);
/* The q|k|v projection and the step above in one launch (main.rs:109-118: rmsnorm when norm_w, gemv(q|k|v_proj),
 * round_bf, rope(q), rope(k), the cache append): W [(NQ + 2 NKV) * 128, H] bf16 (the q, k and v tables stacked), x [H]
 * bf16; q [NQ * 128] receives roped q, k_cache / v_cache row pos the roped k and the v.  head_dim 128, H % 4096 == 0.
 * Bit-identical to moe_gemv_norm_dev (or moe_gemv_dev) followed by moe_rope_append_dev. */
int moe_qkv_rope_append_dev(int H, int n_q_heads, int n_kv_heads, int head_dim, const uint16_t* W, const uint16_t* x,
                            const uint16_t* norm_w, float eps, const uint16_t* cos_row, const uint16_t* sin_row,
                            uint16_t* q, uint16_t* k_cache, uint16_t* v_cache, int pos, void* stream);

/* ----------------------------------------------------------------------------------------------- decode attention
 * GQA attention of one token over a layer's KV cache, replacing the host step's core (track2_opt/solar_engine/src/
 * main.rs:86-104): for q head h and kv head h / (NQ / NKV), positions t < S,
 *   sc[t] = bf16(bf16(q_h . k_t) * scale)  (dot summed left to right in fp32: bit-identical scores),
 *   p[t] = bf16(exp(sc[t] - max sc) / sum exp(sc - max sc)),  out_h = bf16(sum_t p[t] v_t)  (fp32 sums in the GPU's order).
 * q [NQ, D] bf16 (after RoPE), k_cache / v_cache [S, NKV, D] bf16 (16-byte aligned), out [NQ, D] bf16; D = 128,
 * NQ = G * NKV with G in {1, 2, 4, 8}, 1 <= S <= 65536.  Device pointers; enqueued on `stream` (NULL: the null
 * stream), not synchronised; one kernel launch, which may be captured in a HIP graph and replayed.  The caller
 * passes a device workspace of moe_attn_workspace_bytes() bytes (0 for arguments out of range) dedicated to these
 * calls, zero-filled before its first call: a 256-byte header (the call counter), the call's scores ([NQ, S] fp32
 * from byte 256, left there for the caller), then tagged per-chunk statistics, partials and outputs.  Between calls nothing
 * else may write it (zeroing all of it again is allowed).  Pass the same workspace_bytes on every call on a
 * workspace.  Calls that share a workspace and overlap in time (two streams) race. */
size_t moe_attn_workspace_bytes(int n_q_heads, int head_dim, int S);
int moe_attn_decode_dev(int n_q_heads, int n_kv_heads, int head_dim, int S, float scale, const uint16_t* q,
                        const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out, void* workspace,
                        size_t workspace_bytes, void* stream);
const char* moe_attn_last_error(void); /* message of this thread's last failed moe_attn_decode_dev */
/* moe_attn_decode_dev with the layer's o projection folded into the same launch, replacing main.rs:86-104 and :119
 * (attention, then round_bf(gemv(o_proj, attention output))): out as moe_attn_decode_dev, and o_out [o_rows] bf16 =
 * bf16(w_o . out) with w_o [o_rows, NQ * D] bf16 row-major (16-byte aligned), bit-identical to moe_gemv_dev(o_rows,
 * NQ * D, w_o, out, o_out).  Needs NQ * D = 4096; same workspace and rules as moe_attn_decode_dev. */
int moe_attn_decode_oproj_dev(int n_q_heads, int n_kv_heads, int head_dim, int S, float scale, const uint16_t* q,
                              const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out, const uint16_t* w_o,
                              int o_rows, uint16_t* o_out, void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free variant of moe_attn_decode_dev.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * workspace lives in a file-scope device array of moe_attn_noalloc_max_bytes() bytes (6.4 MB: 64 query heads x 8192
 * positions), one per GPU, held until the process ends; its address is looked up once per device.  The call
 * allocates nothing (its first call on a device also enqueues the clearing of the array: make that call outside a
 * graph capture); it returns MOE_GPU_EINVAL, enqueueing nothing, when moe_attn_workspace_bytes(n_q_heads,
 * head_dim, S) exceeds that size.  Outputs are bit-identical to moe_attn_decode_dev's.  All calls on one GPU share
 * its array: calls that overlap on one GPU (two streams, two threads) race; serialise them on one stream. */
size_t moe_attn_noalloc_max_bytes(void);
int moe_attn_decode_noalloc_dev(int n_q_heads, int n_kv_heads, int head_dim, int S, float scale, const uint16_t* q,
                                const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out, void* stream);

/* ----------------------------------------------------------------------------------------------- decode step
 * One greedy decode step of a whole MoE decoder, replacing the engine's host step (track2_opt/solar_engine/src/
 * main.rs:372-387 `step`, with `layer` :106-126 and `moe_host` :128-141): x = embedding[token]; per layer the
 * input RMSNorm + q|k|v GEMV, RoPE + KV append at pos, GQA attention over positions 0..pos, o GEMV, then
 * moe_gpu_block_dev (residual add, post-attention RMSNorm, routed + shared experts, residual add); then the final
 * RMSNorm, the LM head and the greedy argmax.  The model owns a moe_gpu context (its experts and routers: load them
 * through moe_model_experts()) and a moe_head (moe_model_head()); all run on the model's stream.  Batch 1. */
typedef struct moe_model moe_model;
typedef struct moe_model_config {
    int H, n_q_heads, n_kv_heads, head_dim;  /* head_dim 128; H % 4096 == 0 */
    int F, E, topk, n_shared;                /* the MoE block (moe_gpu_create) */
    int n_layers, vocab, max_ctx;            /* max_ctx: KV cache and rope table length */
    float eps;                               /* RMSNorm epsilon (host.rs:15: 1e-5) */
    int route_rule;                          /* MOE_GPU_ROUTE_SIGMOID for Solar's route(), or _SOFTMAX */
    int argmax_rule;                         /* MOE_HEAD_ARGMAX_FP32 (main.rs:384-385) or _BF16 (chip.rs:183-194) */
} moe_model_config;
int moe_model_create(int device, const moe_model_config* cfg, moe_model** out);
void moe_model_destroy(moe_model* m);
const char* moe_model_last_error(const moe_model* m); /* m == NULL: the last failed create */
moe_gpu* moe_model_experts(moe_model* m);
moe_head* moe_model_head(moe_model* m);
int moe_model_set_stream(moe_model* m, void* stream);
/* Waits for the model's stream; reports a step whose token id was outside the vocabulary. */
int moe_model_synchronize(moe_model* m);
/* Attention-block weights of one layer, host or device pointers, row-major bf16 (model.layers.{l}.*): in_norm [H]
 * (input_layernorm), wq [NQ*D, H], wk / wv [NKV*D, H], wo [H, NQ*D], post_norm [H] (post_attention_layernorm). */
int moe_model_load_layer(moe_model* m, int layer, const uint16_t* in_norm, const uint16_t* wq, const uint16_t* wk,
                         const uint16_t* wv, const uint16_t* wo, const uint16_t* post_norm);
int moe_model_load_embedding(moe_model* m, const uint16_t* emb);                   /* [vocab, H] bf16 */
int moe_model_get_config(moe_model* m, moe_model_config* cfg);                     /* the configuration as created */
int moe_model_load_rope(moe_model* m, const uint16_t* cos_tab, const uint16_t* sin_tab); /* [max_ctx, D] bf16 */
/* Steps run the first n layers (default all), then the head: a stage of a model split over several devices, or a
 * layer-by-layer check. */
int moe_model_set_layers(moe_model* m, int n);
/* Device pointers of a layer's KV cache [max_ctx, NKV, D] bf16 (zeroed at create; a caller may fill positions). */
int moe_model_kv_cache(moe_model* m, int layer, uint16_t** k_cache, uint16_t** v_cache);
/* token, next: device int32; best (device fp32, optional) receives the picked logit.  Writes the KV caches at pos and
 * attends over positions 0..pos.  Enqueued, not synchronised. */
int moe_model_step_dev(moe_model* m, const int32_t* token, int pos, int32_t* next, float* best);
/* The same from / to host values, synchronous. */
int moe_model_step(moe_model* m, int token, int pos, int32_t* next, float* best);
/* The residual stream after the last layer of the last step (before the final norm), [H] bf16 to host or device. */
int moe_model_residual(moe_model* m, uint16_t* x);

/* ----------------------------------------------------------------------------------------------- weights on disk
 * The model directory of safetensors files, replacing the engine's Weights (track2_opt/solar_engine/src/host.rs:78-117):
 * every *.safetensors file of `dir`, in name order, memory-mapped read-only; tensors found by their HF names (a name in
 * a later file replaces an earlier one).  The mapping stays until moe_st_close; pointers from moe_st_tensor are into
 * it.  Headers are validated (offsets inside the file and matching dtype x shape), so a malformed file is an error,
 * never a read outside the mapping. */
typedef struct moe_st moe_st;
#define MOE_ST_BF16 0
#define MOE_ST_F32 1
#define MOE_ST_F16 2
#define MOE_ST_I8 3
#define MOE_ST_I32 4
#define MOE_ST_I64 5
#define MOE_ST_U8 6
int moe_st_open(const char* dir, moe_st** out);
void moe_st_close(moe_st* st);
const char* moe_st_last_error(const moe_st* st); /* st == NULL: the last failed open or placement read */
int moe_st_count(const moe_st* st);              /* number of tensors */
/* Tensor by name: data pointer into the mapping, byte size, MOE_ST_* dtype, shape; *ndim is the capacity of `shape` on
 * entry, the tensor's rank on return.  Any output may be NULL.  MOE_GPU_EINVAL when absent. */
int moe_st_tensor(const moe_st* st, const char* name, const void** data, size_t* nbytes, int* dtype, int64_t* shape,
                  int* ndim);
/* MoE half of model layer `model_layer` into the context's layer `tier_layer` (the engine's names: main.rs:466-468,
 * :519; host.rs:111-116): router mlp.gate.weight [E, H] and mlp.gate.e_score_correction_bias [E] (fp32 or bf16; zero
 * when absent), shared experts mlp.shared_experts.{gate,up,down}_proj.weight (n_shared > 1: mlp.shared_experts.{s}.*),
 * and routed experts mlp.experts.{e}.{gate,up,down}_proj.weight for e in experts[0..n) (n < 0: every e < E).  Shapes
 * are checked against the context. */
int moe_st_load_moe_layer(const moe_st* st, moe_gpu* ctx, int model_layer, int tier_layer, const int32_t* experts,
                          int n);
/* A whole decode model: per layer the attention block (input_layernorm, self_attn.{q,k,v,o}_proj,
 * post_attention_layernorm) and the MoE half (every expert), then model.embed_tokens.weight, lm_head.weight and
 * model.norm.weight.  Shapes are checked against the model's configuration. */
int moe_st_load_model(const moe_st* st, moe_model* m);
/* The engine's placement.json (main.rs:455; moe_offload/placement.py:3): [layer][tier] -> expert ids in slot order.
 * *n receives the count of (layer, tier)'s ids, written to ids when it fits `cap` (ids may be NULL to ask the count). */
int moe_placement_read(const char* path, int layer, int tier, int32_t* ids, int cap, int* n);

#ifdef __cplusplus
}
#endif
#endif /* MOE_GPU_H */
