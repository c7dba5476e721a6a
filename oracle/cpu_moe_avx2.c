/*
 * cpu_moe_avx2.c -- CPU expert kernel timed as the CPU baseline.
 *
 * TEST/BENCH INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg and tests/
 * call it; the product library never does.
 *
 * It stands in for ktransformers' AVX2BF16_MOE (not vendored with the
 * reference and not fetchable offline).  It keeps that kernel's row contract
 * as the reference drives it (baselines/ktransformers/runtime.py:180-181,
 * native/native_layer_dispatch.cpp:68-69): a packed block of rows, each row r
 * run through expert selected[r] (k = 1) and scaled by coeff[r].
 *
 * Math: bf16 weights and activations widened to fp32 in AVX2 registers, fp32
 * FMA accumulation, h = silu(g)*u rounded to bf16, y rounded to bf16.
 * Threads: OpenMP (persistent libgomp pool), the caller's thread included.
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

static inline __m256 ld_bf16x8(const uint16_t *p) {
    __m128i v = _mm_loadu_si128((const __m128i *)p);
    return _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(v), 16));
}

static inline float hsum8(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
    lo = _mm_add_ps(lo, hi);
    lo = _mm_add_ps(lo, _mm_movehl_ps(lo, lo));
    lo = _mm_add_ss(lo, _mm_shuffle_ps(lo, lo, 1));
    return _mm_cvtss_f32(lo);
}

static inline uint16_t to_bf16(float f) { return orc_f32_to_bf16(f); }
static inline float from_bf16(uint16_t h) { return orc_bf16_to_f32(h); }

/* dot(w bf16[n], x fp32[n]); n % 32 == 0 */
static inline float dot_w_xf(const uint16_t *w, const float *x, int n) {
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    for (int i = 0; i < n; i += 32) {
        a0 = _mm256_fmadd_ps(ld_bf16x8(w + i), _mm256_loadu_ps(x + i), a0);
        a1 = _mm256_fmadd_ps(ld_bf16x8(w + i + 8), _mm256_loadu_ps(x + i + 8), a1);
        a2 = _mm256_fmadd_ps(ld_bf16x8(w + i + 16), _mm256_loadu_ps(x + i + 16), a2);
        a3 = _mm256_fmadd_ps(ld_bf16x8(w + i + 24), _mm256_loadu_ps(x + i + 24), a3);
    }
    return hsum8(_mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3)));
}

/* four activation rows against one weight row (weight loaded once) */
static inline void dot4_w_xf(const uint16_t *w, const float *x0, const float *x1,
                             const float *x2, const float *x3, int n, float out[4]) {
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    for (int i = 0; i < n; i += 8) {
        __m256 wv = ld_bf16x8(w + i);
        a0 = _mm256_fmadd_ps(wv, _mm256_loadu_ps(x0 + i), a0);
        a1 = _mm256_fmadd_ps(wv, _mm256_loadu_ps(x1 + i), a1);
        a2 = _mm256_fmadd_ps(wv, _mm256_loadu_ps(x2 + i), a2);
        a3 = _mm256_fmadd_ps(wv, _mm256_loadu_ps(x3 + i), a3);
    }
    out[0] = hsum8(a0); out[1] = hsum8(a1); out[2] = hsum8(a2); out[3] = hsum8(a3);
}

static inline float silu_f(float g) { return g / (1.0f + expf(-g)); }

static int have_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

/* One expert over m rows: xf fp32 [m,H] -> yout fp32 [m,H] (bf16-rounded values). */
static void expert_rows(const float *xf, int m, const uint16_t *base, int H, int I,
                        float *hf, float *yout, int nthreads) {
    const uint16_t *wg = base, *wu = base + (size_t)I * H, *wd = base + 2 * (size_t)I * H;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int i = 0; i < I; ++i) {
        int r = 0;
        for (; r + 4 <= m; r += 4) {
            float g[4], u[4];
            const float *x0 = xf + (size_t)r * H;
            dot4_w_xf(wg + (size_t)i * H, x0, x0 + H, x0 + 2 * H, x0 + 3 * H, H, g);
            dot4_w_xf(wu + (size_t)i * H, x0, x0 + H, x0 + 2 * H, x0 + 3 * H, H, u);
            for (int q = 0; q < 4; ++q)
                hf[(size_t)(r + q) * I + i] = from_bf16(to_bf16(silu_f(g[q]) * u[q]));
        }
        for (; r < m; ++r) {
            float g = dot_w_xf(wg + (size_t)i * H, xf + (size_t)r * H, H);
            float u = dot_w_xf(wu + (size_t)i * H, xf + (size_t)r * H, H);
            hf[(size_t)r * I + i] = from_bf16(to_bf16(silu_f(g) * u));
        }
    }
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int j = 0; j < H; ++j) {
        int r = 0;
        for (; r + 4 <= m; r += 4) {
            float y[4];
            const float *h0 = hf + (size_t)r * I;
            dot4_w_xf(wd + (size_t)j * I, h0, h0 + I, h0 + 2 * I, h0 + 3 * I, I, y);
            for (int q = 0; q < 4; ++q) yout[(size_t)(r + q) * H + j] = from_bf16(to_bf16(y[q]));
        }
        for (; r < m; ++r)
            yout[(size_t)r * H + j] = from_bf16(to_bf16(dot_w_xf(wd + (size_t)j * I, hf + (size_t)r * I, I)));
    }
}

int cpu_moe_forward_rows(const uint16_t *x, int rows, const int64_t *selected,
                         const float *coeff, const uint16_t *const *slots, int H, int I,
                         uint16_t *out, int nthreads) {
    if (!have_avx2() || rows < 1 || H % 32 || I % 32 || nthreads < 1) return -1;
    /* stable grouping of rows by expert, as the packed native call sees them */
    int64_t maxe = 0;
    for (int r = 0; r < rows; ++r) {
        if (selected[r] < 0) return -1;
        if (selected[r] > maxe) maxe = selected[r];
    }
    int E = (int)maxe + 1;
    int *cnt = (int *)calloc((size_t)E + 1, sizeof(int));
    int *order = (int *)malloc(sizeof(int) * (size_t)rows);
    float *xf = (float *)malloc(sizeof(float) * (size_t)rows * H);
    float *hf = (float *)malloc(sizeof(float) * (size_t)rows * I);
    float *yf = (float *)malloc(sizeof(float) * (size_t)rows * H);
    if (!cnt || !order || !xf || !hf || !yf) {
        free(cnt); free(order); free(xf); free(hf); free(yf);
        return -1;
    }
    for (int r = 0; r < rows; ++r) cnt[selected[r] + 1]++;
    for (int e = 0; e < E; ++e) cnt[e + 1] += cnt[e];
    int *cur = (int *)malloc(sizeof(int) * (size_t)E);
    memcpy(cur, cnt, sizeof(int) * (size_t)E);
    for (int r = 0; r < rows; ++r) order[cur[selected[r]]++] = r;
    free(cur);
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int q = 0; q < rows; ++q) {
        const uint16_t *src = x + (size_t)order[q] * H;
        for (int j = 0; j < H; ++j) xf[(size_t)q * H + j] = from_bf16(src[j]);
    }
    for (int e = 0; e < E; ++e) {
        int m = cnt[e + 1] - cnt[e];
        if (!m) continue;
        expert_rows(xf + (size_t)cnt[e] * H, m, slots[e], H, I, hf + (size_t)cnt[e] * I,
                    yf + (size_t)cnt[e] * H, nthreads);
    }
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int q = 0; q < rows; ++q) {
        int r = order[q];
        float c = coeff ? coeff[r] : 1.0f;
        for (int j = 0; j < H; ++j) out[(size_t)r * H + j] = to_bf16(c * yf[(size_t)q * H + j]);
    }
    free(cnt); free(order); free(xf); free(hf); free(yf);
    return 0;
}

int cpu_moe_decode(const uint16_t *x, const int32_t *ids, const uint16_t *w, int k,
                   const uint16_t *const *slots, int H, int I, uint16_t *out, int nthreads) {
    if (!have_avx2() || k < 1 || k > 64 || H % 32 || I % 32 || nthreads < 1) return -1;
    float *xf = (float *)malloc(sizeof(float) * (size_t)H);
    float *hf = (float *)malloc(sizeof(float) * (size_t)k * I);
    if (!xf || !hf) {
        free(xf); free(hf);
        return -1;
    }
    for (int j = 0; j < H; ++j) xf[j] = from_bf16(x[j]);
    /* gate/up for all k experts, then down + weighted merge per output row */
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int q = 0; q < k * I; ++q) {
        int s = q / I, i = q % I;
        const uint16_t *base = slots[ids[s]];
        float g = dot_w_xf(base + (size_t)i * H, xf, H);
        float u = dot_w_xf(base + (size_t)I * H + (size_t)i * H, xf, H);
        hf[(size_t)s * I + i] = from_bf16(to_bf16(silu_f(g) * u));
    }
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int j = 0; j < H; ++j) {
        float acc = 0.0f;
        for (int s = 0; s < k; ++s) {
            const uint16_t *wd = slots[ids[s]] + 2 * (size_t)I * H;
            float y = from_bf16(to_bf16(dot_w_xf(wd + (size_t)j * I, hf + (size_t)s * I, I)));
            acc += from_bf16(w[s]) * y;
        }
        out[j] = to_bf16(acc);
    }
    free(xf); free(hf);
    return 0;
}
