/*
 * cpu_moe_port.c — AVX-512 BF16 + OpenMP port of solar_hybrid/cpu_moe.cpp:38-96 (the CPU baseline "port").
 *
 * TEST INFRASTRUCTURE ONLY: checked bit-for-bit against the scalar restatement in moe_oracle.c by the tests.  The
 * benchmark's cpu_baseline leg times it for the batched workloads (T > 1 tokens, cpu_moe.cpp's own use); batch 1 times
 * the reference's own cpu_kern.c build (oracle/_ref) or, where that cannot be loaded, the scalar restatement.
 * Built into its own library with AVX-512 flags so that the scalar oracle stays loadable on any x86-64 host.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#define OR_API __attribute__((visibility("default")))
static inline uint16_t f2bf_p(float f) { uint32_t u; memcpy(&u, &f, 4); u += 0x7FFFu + ((u >> 16) & 1u); return (uint16_t)(u >> 16); }
static inline float silu_mul(float g, float u) { return (g / (1.f + expf(-g))) * u; }

/* Same algorithm as cpu_moe.cpp: phase 1 work units = (expert, 64-row block of the 2F gate|up rows), dynamic
 * schedule; silu*mul to bf16; phase 2 = 32-row output blocks owned per thread (no atomics), experts in list order. */
#if defined(__AVX512BF16__) && defined(__AVX512F__)
#include <immintrin.h>
static inline float dot_avx(const uint16_t* a, const uint16_t* b, int n) {
    __m512 acc0 = _mm512_setzero_ps(), acc1 = _mm512_setzero_ps();
    int i = 0;
    for (; i + 64 <= n; i += 64) {
        acc0 = _mm512_dpbf16_ps(acc0, (__m512bh)_mm512_loadu_si512(a + i), (__m512bh)_mm512_loadu_si512(b + i));
        acc1 = _mm512_dpbf16_ps(acc1, (__m512bh)_mm512_loadu_si512(a + i + 32), (__m512bh)_mm512_loadu_si512(b + i + 32));
    }
    for (; i < n; i += 32)
        acc0 = _mm512_dpbf16_ps(acc0, (__m512bh)_mm512_loadu_si512(a + i), (__m512bh)_mm512_loadu_si512(b + i));
    return _mm512_reduce_add_ps(_mm512_add_ps(acc0, acc1));
}
OR_API int or_have_avx512bf16(void) { return 1; }
OR_API void or_cpu_moe_avx512(int T, int H, int F, int E, const uint16_t* x, const uint16_t* const* gus,
                              const uint16_t* const* ds, const int64_t* const* toks, const int* ntok,
                              const float* const* ws, float* out) {
    memset(out, 0, sizeof(float) * (size_t)T * H);
    if (E <= 0) return;
    int* off = (int*)malloc(sizeof(int) * (E + 1));
    off[0] = 0;
    for (int e = 0; e < E; e++) off[e + 1] = off[e] + ntok[e];
    const int R = off[E];
    uint16_t* act = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)R * F + 64);
    float* gb = (float*)malloc(sizeof(float) * (size_t)R * 2 * F + 64);
    const int RB = 64, nblk = (2 * F) / RB, HB = 32;
    #pragma omp parallel for schedule(dynamic, 1)
    for (int un = 0; un < E * nblk; un++) {
        const int e = un / nblk, b = un % nblk;
        for (int r = b * RB; r < (b + 1) * RB; r++)
            for (int j = 0; j < ntok[e]; j++)
                gb[(size_t)(off[e] + j) * 2 * F + r] = dot_avx(gus[e] + (size_t)r * H, x + (size_t)toks[e][j] * H, H);
    }
    #pragma omp parallel for schedule(static)
    for (int rj = 0; rj < R; rj++)
        for (int f = 0; f < F; f++)
            act[(size_t)rj * F + f] = f2bf_p(silu_mul(gb[(size_t)rj * 2 * F + f], gb[(size_t)rj * 2 * F + F + f]));
    #pragma omp parallel for schedule(dynamic, 1)
    for (int hb = 0; hb < H / HB; hb++)
        for (int e = 0; e < E; e++)
            for (int h = hb * HB; h < (hb + 1) * HB; h++)
                for (int j = 0; j < ntok[e]; j++) {
                    float* o = out + (size_t)toks[e][j] * H + h;
                    *o = fmaf(ws[e][j], dot_avx(ds[e] + (size_t)h * F, act + (size_t)(off[e] + j) * F, F), *o);
                }
    free(off); free(act); free(gb);
}
#else
#error "cpu_moe_port.c needs -mavx512f -mavx512bf16"
#endif

OR_API int or_port_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

