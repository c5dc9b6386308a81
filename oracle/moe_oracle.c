/*
 * moe_oracle.c — CPU restatement of npu-offload's routed-MoE data plane.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle: only tests/, the smoke check and the CPU-baseline leg of
 * the benchmark load it.  The GPU product path never calls into it (libmoe_gpu.so does not link it and fails loudly
 * when its own HIP kernels are missing).
 *
 * What it restates (reference files, path:line relative to the reference repository root):
 *   - bf16 helpers f2bf / bf2f ........ solar_hybrid/cpu_moe.cpp:30-34, track2_opt/solar_engine/src/host.rs:41-50
 *   - dot_bf16 (vdpbf16ps, 2 accs) .... solar_hybrid/cpu_moe.cpp:17-28, track2_opt/solar_engine/csrc/cpu_kern.c:9-19
 *   - cpu_moe (batched experts) ....... solar_hybrid/cpu_moe.cpp:38-96
 *   - ck_moe3 (batch-1, placed) ....... track2_opt/solar_engine/csrc/cpu_kern.c:140-172 (+ ck_place_expert :124-138)
 *   - ck_gemv (router GEMV) ........... track2_opt/solar_engine/csrc/cpu_kern.c:31-35
 *   - quant_row ....................... track2_opt/solar_engine/csrc/cpu_kern.c:218-224
 *   - ck_moe_q8w (int8 weight-only) ... track2_opt/solar_engine/csrc/cpu_kern.c:291-333
 *   - softmax route() ................. npu-kernels/npu_kernels/rngd/layer_template/src/host.rs.tpl:247-267
 *   - sigmoid route() (Solar) ......... track2_opt/solar_engine/src/host.rs:119-128
 *   - expert grouping (first seen) .... solar_hybrid/runtime.py:344-354
 *
 * The scalar dot products emulate the exact arithmetic of the reference's AVX-512 code: 16 fp32 lanes, each lane
 * accumulating the odd then the even bf16 product of its dword pair with one rounding each (vdpbf16ps: DAZ inputs,
 * FTZ output, RNE), two accumulators over 64-element steps, then GCC's _mm512_reduce_add_ps tree.  They therefore
 * reproduce the reference's fp32 bits, which the tests check against the reference's own compiled cpu_kern.c.
 *
 * The HIP router kernel computes its logits in ck_gemv's own order, so or_gemv() is also the GPU logits' mirror.
 *
 * The AVX-512 CPU-baseline port of cpu_moe lives in cpu_moe_port.c (its own library, AVX-512 flags).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define OR_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------ bf16 helpers (cpu_moe.cpp:30-34) */
static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

OR_API uint16_t or_f2bf(float f) { /* round-to-nearest-even by the bias trick, no NaN special case */
    uint32_t u = f_bits(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
OR_API float or_bf2f(uint16_t b) { return bits_f((uint32_t)b << 16); }

/* ------------------------------------------------------------------ vdpbf16ps lane emulation */
static inline float daz(float v) { return (f_bits(v) & 0x7F800000u) == 0 ? bits_f(f_bits(v) & 0x80000000u) : v; }
static inline float ftz(float v) { return daz(v); }

/* one vdpbf16ps step on one fp32 lane: acc += a[1]*b[1]; acc += a[0]*b[0] (odd element first) */
static inline float dp_lane(float acc, float a0, float a1, float b0, float b1) {
    acc = ftz(daz(acc) + daz(a1) * daz(b1));
    acc = ftz(daz(acc) + daz(a0) * daz(b0));
    return acc;
}

/* GCC's _mm512_reduce_add_ps: 256-bit halves, 128-bit halves, (2,3,0,1) shuffle, last pair */
static inline float reduce16(const float* v) {
    float t3[8], t6[4];
    for (int i = 0; i < 8; i++) t3[i] = v[8 + i] + v[i];
    for (int i = 0; i < 4; i++) t6[i] = t3[4 + i] + t3[i];
    float t80 = t6[0] + t6[2], t81 = t6[1] + t6[3];
    return t80 + t81;
}

/* accumulate one 32-element bf16 block (512-bit register) into a 16-lane accumulator */
static inline void dp_block_bf16(float* acc, const uint16_t* a, const uint16_t* b) {
    for (int j = 0; j < 16; j++)
        acc[j] = dp_lane(acc[j], or_bf2f(a[2 * j]), or_bf2f(a[2 * j + 1]), or_bf2f(b[2 * j]), or_bf2f(b[2 * j + 1]));
}

/* dot_bf16 (cpu_moe.cpp:18-28, cpu_kern.c:9-19): n % 32 == 0.  dot2_bf16 (cpu_kern.c:68-79) has the same
 * per-row arithmetic when n % 64 == 0. */
OR_API float or_dot_bf16(const uint16_t* a, const uint16_t* b, int n) {
    float acc0[16] = {0}, acc1[16] = {0}, s[16];
    int i = 0;
    for (; i + 64 <= n; i += 64) {
        dp_block_bf16(acc0, a + i, b + i);
        dp_block_bf16(acc1, a + i + 32, b + i + 32);
    }
    for (; i < n; i += 32) dp_block_bf16(acc0, a + i, b + i);
    for (int j = 0; j < 16; j++) s[j] = acc0[j] + acc1[j];
    return reduce16(s);
}

/* dot_bf16_i8 (cpu_kern.c:298-305): x bf16, w int8 widened exactly to bf16; n % 64 == 0 */
OR_API float or_dot_bf16_i8(const uint16_t* x, const int8_t* w, int n) {
    float acc0[16] = {0}, acc1[16] = {0}, s[16];
    for (int i = 0; i < n; i += 64) {
        for (int j = 0; j < 16; j++) {
            const int k0 = i + 2 * j, k1 = i + 32 + 2 * j;
            acc0[j] = dp_lane(acc0[j], or_bf2f(x[k0]), or_bf2f(x[k0 + 1]), (float)w[k0], (float)w[k0 + 1]);
            acc1[j] = dp_lane(acc1[j], or_bf2f(x[k1]), or_bf2f(x[k1 + 1]), (float)w[k1], (float)w[k1 + 1]);
        }
    }
    for (int j = 0; j < 16; j++) s[j] = acc0[j] + acc1[j];
    return reduce16(s);
}

static inline float silu_mul(float g, float u) { return (g / (1.f + expf(-g))) * u; } /* cpu_moe.cpp:75 */

/* ------------------------------------------------------------------ ck_gemv (cpu_kern.c:31-35) */
OR_API void or_gemv(const uint16_t* W, const uint16_t* x, float* y, int M, int K) {
    for (int m = 0; m < M; m++) y[m] = or_dot_bf16(W + (size_t)m * K, x, K);
}

/* ------------------------------------------------------------------ cpu_moe (cpu_moe.cpp:38-96)
 * x [T,H] bf16; gus[e] = [Wg_e; Wu_e] : [2F,H] bf16 row-major; ds[e] : [H,F] bf16 row-major;
 * toks[e] : ntok[e] token rows (int64); ws[e] : ntok[e] fp32 gates.  out [T,H] fp32 is written (zeroed first).
 * Per (expert, token): g,u fp32 dots; act = bf16(silu(g)*u); out[t,h] += w * dot(d_row, act), experts in list order.
 * The reference's `+= w*dot` compiles to one fused multiply-add (checked against the reference build). */
OR_API void or_cpu_moe(int T, int H, int F, int E, const uint16_t* x, const uint16_t* const* gus,
                       const uint16_t* const* ds, const int64_t* const* toks, const int* ntok,
                       const float* const* ws, float* out) {
    memset(out, 0, sizeof(float) * (size_t)T * H);
    if (E <= 0) return;
    float* g = (float*)malloc(sizeof(float) * 2 * (size_t)F);
    uint16_t* act = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)F);
    for (int e = 0; e < E; e++) {
        for (int j = 0; j < ntok[e]; j++) {
            const int64_t t = toks[e][j];
            const uint16_t* xt = x + (size_t)t * H;
            for (int r = 0; r < 2 * F; r++) g[r] = or_dot_bf16(gus[e] + (size_t)r * H, xt, H);
            for (int f = 0; f < F; f++) act[f] = or_f2bf(silu_mul(g[f], g[F + f]));
            for (int h = 0; h < H; h++) {
                float* o = out + (size_t)t * H + h;
                *o = fmaf(ws[e][j], or_dot_bf16(ds[e] + (size_t)h * F, act, F), *o);
            }
        }
    }
    /* note: the reference sums experts per output row in list order (phase 2 loops e inside hb); visiting experts
     * in the outer loop here gives the same per-element sequence of fused multiply-adds. */
    free(g); free(act);
}

/* ------------------------------------------------------------------ ck_moe3 (cpu_kern.c:140-172), one token
 * base[e] = ck_place_expert layout: [g F*H][u F*H][d H*F] bf16.  out [H] fp32 is accumulated (+=). */
OR_API void or_ck_moe3(int E, const uint16_t* const* base, const float* w, const uint16_t* x, float* out, int H, int F) {
    if (E <= 0) return;
    float* g = (float*)malloc(sizeof(float) * 2 * (size_t)F * E);
    uint16_t* act = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)F * E);
    for (int e = 0; e < E; e++)
        for (int r = 0; r < 2 * F; r++) g[(size_t)e * 2 * F + r] = or_dot_bf16(base[e] + (size_t)r * H, x, H);
    for (int e = 0; e < E; e++)
        for (int f = 0; f < F; f++)
            act[(size_t)e * F + f] = or_f2bf(silu_mul(g[(size_t)e * 2 * F + f], g[(size_t)e * 2 * F + F + f]));
    for (int e = 0; e < E; e++) {
        const uint16_t* D = base[e] + (size_t)2 * F * H;
        for (int h = 0; h < H; h++) out[h] = fmaf(w[e], or_dot_bf16(D + (size_t)h * F, act + (size_t)e * F, F), out[h]);
    }
    free(g); free(act);
}

/* ------------------------------------------------------------------ int8 weight-only (cpu_kern.c:218-241, :291-333) */
/* quant_row: s = max|w|/127 (1 if the row is all zero), q = lrintf(w * (1/s)) clamped to [-127,127], rs = sum q */
OR_API void or_quant_row(const uint16_t* src, int n, int8_t* dst, float* sc, int32_t* rs) {
    float m = 0.f;
    for (int i = 0; i < n; i++) { float v = fabsf(or_bf2f(src[i])); if (v > m) m = v; }
    const float s = m > 0 ? m / 127.f : 1.f, inv = 1.f / s;
    int32_t sum = 0;
    for (int i = 0; i < n; i++) {
        int q = (int)lrintf(or_bf2f(src[i]) * inv);
        q = q > 127 ? 127 : (q < -127 ? -127 : q);
        dst[i] = (int8_t)q; sum += q;
    }
    *sc = s; if (rs) *rs = sum;
}

/* ck_place_expert_q8 layout: q [(2F+H) rows] (gate rows, up rows, then down rows of length F), sc/rs [2F+H] */
OR_API void or_quant_expert(const uint16_t* g, const uint16_t* u, const uint16_t* d, int8_t* q, float* sc, int32_t* rs,
                            int H, int F) {
    for (int r = 0; r < 2 * F; r++) {
        const uint16_t* src = r < F ? g + (size_t)r * H : u + (size_t)(r - F) * H;
        or_quant_row(src, H, q + (size_t)r * H, &sc[r], rs ? &rs[r] : 0);
    }
    int8_t* qd = q + (size_t)2 * F * H;
    for (int h = 0; h < H; h++) or_quant_row(d + (size_t)h * F, F, qd + (size_t)h * F, &sc[2 * F + h], rs ? &rs[2 * F + h] : 0);
}

/* ck_moe_q8w: g = dot_i8(x, q_row) * sc; act = bf16(silu(g)*u); out[h] += w * dot_i8(act, qd_row) * sc  (+=) */
OR_API void or_moe_q8w(int E, const int8_t* const* q, const float* const* sc, const float* w, const uint16_t* x, float* out,
                       int H, int F) {
    if (E <= 0) return;
    float* g = (float*)malloc(sizeof(float) * 2 * (size_t)F);
    uint16_t* act = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)F);
    for (int e = 0; e < E; e++) {
        for (int r = 0; r < 2 * F; r++) g[r] = or_dot_bf16_i8(x, q[e] + (size_t)r * H, H) * sc[e][r];
        for (int f = 0; f < F; f++) act[f] = or_f2bf(silu_mul(g[f], g[F + f]));
        const int8_t* qd = q[e] + (size_t)2 * F * H;
        for (int h = 0; h < H; h++) {
            const float p = w[e] * or_dot_bf16_i8(act, qd + (size_t)h * F, F);
            out[h] = fmaf(p, sc[e][2 * F + h], out[h]);
        }
    }
    free(g); free(act);
}

/* ------------------------------------------------------------------ softmax route (host.rs.tpl:247-267)
 * Per token: score = logits (+ bias, added to the logits: the bias is a routing prior on the logit scale);
 * s = softmax(score) over all E; select the k largest scores, stable with ties to the lower index;
 * gates over the first `keep` ranks: w_i = s_i / sum_{j<keep} s_j (sequential sum, rank order).
 * Selection compares the scores themselves (softmax is monotone, so this is the reference's order; exact ties
 * go to the lower index as torch.topk / the reference's stable sort do). */
OR_API void or_route_softmax(int T, int E, int k, int keep, const float* logits, const float* bias, int32_t* ids,
                             float* gates) {
    float* sc = (float*)malloc(sizeof(float) * E);
    float* s = (float*)malloc(sizeof(float) * E);
    int* idx = (int*)malloc(sizeof(int) * E);
    if (keep <= 0 || keep > k) keep = k;
    for (int t = 0; t < T; t++) {
        const float* lg = logits + (size_t)t * E;
        float m = -INFINITY;
        for (int e = 0; e < E; e++) { sc[e] = bias ? lg[e] + bias[e] : lg[e]; if (sc[e] > m) m = sc[e]; }
        float z = 0.f;
        for (int e = 0; e < E; e++) { s[e] = expf(sc[e] - m); z += s[e]; }
        for (int e = 0; e < E; e++) s[e] = s[e] / z;
        /* insertion-sort the index list by (score desc, index asc): stable */
        for (int e = 0; e < E; e++) {
            int p = e;
            while (p > 0 && sc[idx[p - 1]] < sc[e]) { idx[p] = idx[p - 1]; p--; }
            idx[p] = e;
        }
        float tot = 0.f;
        for (int j = 0; j < keep; j++) tot += s[idx[j]];
        for (int j = 0; j < k; j++) {
            ids[(size_t)t * k + j] = idx[j];
            gates[(size_t)t * k + j] = j < keep ? s[idx[j]] / tot : 0.f;
        }
    }
    free(sc); free(s); free(idx);
}

/* ------------------------------------------------------------------ sigmoid route (host.rs:119-128)
 * Solar's route(): s = 1 / (1 + exp(-logit)) in fp32 (exp is the C library's expf, the function Rust's f32::exp
 * calls); the k largest s + bias are selected by a stable descending sort (ties keep the lower index); the gates are
 * the unbiased s of the selected ranks over (their sequential sum + 1e-20).  keep < k (this build's rank drop) sums
 * and keeps only the first keep ranks. */
OR_API void or_route_sigmoid(int T, int E, int k, int keep, const float* logits, const float* bias, int32_t* ids,
                             float* gates) {
    float* s = (float*)malloc(sizeof(float) * E);
    float* key = (float*)malloc(sizeof(float) * E);
    int* idx = (int*)malloc(sizeof(int) * E);
    if (keep <= 0 || keep > k) keep = k;
    for (int t = 0; t < T; t++) {
        const float* lg = logits + (size_t)t * E;
        for (int e = 0; e < E; e++) {
            s[e] = 1.0f / (1.0f + expf(-lg[e]));
            key[e] = bias ? s[e] + bias[e] : s[e];
        }
        for (int e = 0; e < E; e++) {
            int p = e;
            while (p > 0 && key[idx[p - 1]] < key[e]) { idx[p] = idx[p - 1]; p--; }
            idx[p] = e;
        }
        float tot = 0.f;
        for (int j = 0; j < keep; j++) tot += s[idx[j]];
        tot += 1e-20f;
        for (int j = 0; j < k; j++) {
            ids[(size_t)t * k + j] = idx[j];
            gates[(size_t)t * k + j] = j < keep ? s[idx[j]] / tot : 0.f;
        }
    }
    free(s); free(key); free(idx);
}

/* ------------------------------------------------------------------ layer combine (fixed order)
 * out[t,h] = (accumulate ? out : 0) + sum_{s<nsh} ysh[t,s,h] + sum_{r<keep, ids[t,r] >= 0} gates[t,r] * yr[t,r,h],
 * one rounding per term (fused multiply-add for the gated terms), shared experts first, then ranks ascending.
 * This is the combine order libmoe_gpu documents; each term is cpu_moe's `O += w * dot` (cpu_moe.cpp:91). */
OR_API void or_combine(int T, int H, int nsh, int k, int keep, const float* ysh, const float* yr, const int32_t* ids,
                       const float* gates, float* out, int accumulate) {
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++) {
            float acc = accumulate ? out[(size_t)t * H + h] : 0.f;
            for (int s = 0; s < nsh; s++) acc = acc + ysh[((size_t)t * nsh + s) * H + h];
            for (int r = 0; r < keep; r++)
                if (ids[t * k + r] >= 0) acc = fmaf(gates[t * k + r], yr[((size_t)t * k + r) * H + h], acc);
            out[(size_t)t * H + h] = acc;
        }
}

/* ------------------------------------------------------------------ deterministic synthetic generator
 * Shared definition with the device generator of libmoe_gpu (same integer hash, same single fp32 multiply, same
 * bf16 rounding), so full-size GPU tensors can be regenerated on the host bit-for-bit.
 * value(key, i) = bf16( (float)(S - 262140) * c ),  S = sum of the eight 16-bit fields of
 * mix64(key + (2i+1)*G) and mix64(key + (2i+2)*G),  G = 0x9E3779B97F4A7C15, mix64 = splitmix64 finaliser.
 * S is Irwin-Hall(8) over [0, 65535]: mean 262140, sd 53509.9...; c = sigma / sd, passed in as an fp32. */
static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static inline int ih8(uint64_t key, uint64_t i) {
    const uint64_t G = 0x9E3779B97F4A7C15ull;
    uint64_t a = mix64(key + (2 * i + 1) * G), b = mix64(key + (2 * i + 2) * G);
    int s = 0;
    for (int k = 0; k < 4; k++) s += (int)((a >> (16 * k)) & 0xFFFF) + (int)((b >> (16 * k)) & 0xFFFF);
    return s - 262140;
}
OR_API uint64_t or_synth_key(uint64_t seed, uint64_t tensor_id) { return mix64(seed * 0xD1B54A32D192ED03ull + tensor_id); }
OR_API void or_synth_bf16(uint64_t key, uint64_t start, uint64_t n, float c, uint16_t* out) {
    for (uint64_t i = 0; i < n; i++) out[i] = or_f2bf((float)ih8(key, start + i) * c);
}

OR_API int or_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
