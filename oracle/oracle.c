/*
 * oracle.c -- CPU restatement of PDScope's GPU MoE-layer arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (results are checked against it): never linked into the product
 * library.  Built by oracle/Makefile into oracle/liboracle.so and called from
 * tests/ through oracle/oracle.py.
 *
 * Compiled with -ffp-contract=off so that every fp32 expression below is
 * evaluated exactly as written (explicit fmaf() where a fused op is meant).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ bf16 */

float orc_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Round-to-nearest-even, the rounding torch applies in c10::BFloat16. */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* binary64 -> bf16 with one correct rounding.  binary64 -> binary32 with
 * round-to-odd, then binary32 -> bf16 to nearest even; since 24 >= 8 + 2 the
 * double rounding equals the direct rounding (Boldo & Melquiond, "Emulation
 * of FMA and correctly rounded sums: proved algorithms using rounding to
 * odd", IEEE TC 2008). */
uint16_t orc_f64_to_bf16(double d) {
    if (isnan(d)) return 0x7fc0u;
    float f = (float)d;
    if ((double)f != d && isfinite(f)) {
        uint32_t u;
        memcpy(&u, &f, 4);
        if (fabs((double)f) > fabs(d)) u -= 1u; /* truncate toward zero */
        u |= 1u;                                /* sticky (odd) bit */
        memcpy(&f, &u, 4);
    }
    return orc_f32_to_bf16(f);
}

/* exp(x) for x <= 0 in fp32 with a fixed operation sequence:
 * Cody-Waite reduction x = n*ln2 + r (ln2 split into a 13-bit head and a
 * tail, W. J. Cody & W. Waite, "Software Manual for the Elementary
 * Functions", 1980), then exp(r) by the degree-7 Taylor polynomial in
 * Horner form (coefficients 1/j!), then scaling by 2^n built from the
 * exponent field.  Results below 2^-125 are flushed to 0 so no subnormal is
 * ever produced (GPU and CPU agree regardless of denormal mode). */
float orc_expf(float x) {
    const float log2e = 0x1.715476p+0f;
    const float ln2_hi = 0x1.62ep-1f;
    const float ln2_lo = 0x1.0bfbe8p-15f;
    float n = rintf(x * log2e);
    if (!(n >= -125.0f)) return 0.0f;
    float r = fmaf(-n, ln2_hi, x);
    r = fmaf(-n, ln2_lo, r);
    float p = 0x1.a01a02p-13f;        /* 1/5040 */
    p = fmaf(p, r, 0x1.6c16c2p-10f);  /* 1/720 */
    p = fmaf(p, r, 0x1.111112p-7f);   /* 1/120 */
    p = fmaf(p, r, 0x1.555556p-5f);   /* 1/24 */
    p = fmaf(p, r, 0x1.555556p-3f);   /* 1/6 */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    uint32_t sb = (uint32_t)((int)n + 127) << 23;
    float s;
    memcpy(&s, &sb, 4);
    return p * s;
}

/* ---------------------------------------------------------------- A1 route */

static double dot_bf16_exact(const uint16_t *a, const uint16_t *b, int n) {
    double acc = 0.0;
    for (int i = 0; i < n; ++i)
        acc += (double)orc_bf16_to_f32(a[i]) * (double)orc_bf16_to_f32(b[i]);
    return acc;
}

/* qwen.py:147 logits = F.linear(inputs, gate): bf16 output of an fp32
 * accumulated product; restated as the exact sum rounded once. */
void orc_route_logits(const uint16_t *x, const uint16_t *gate, int T, int H, int E,
                      uint16_t *logits) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t)
        for (int e = 0; e < E; ++e)
            logits[(size_t)t * E + e] =
                orc_f64_to_bf16(dot_bf16_exact(x + (size_t)t * H, gate + (size_t)e * H, H));
}

/* Sum of v[0..E) in the wave64 order the GPU kernel uses: lane l first adds
 * v[l], v[l+64], ... in that order starting from 0, then an xor butterfly
 * over offsets 32,16,...,1 (every lane ends with the same value). */
static float wave64_sum(const float *v, int E) {
    float lane[64], next[64];
    for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int e = l; e < E; e += 64) acc = acc + v[e];
        lane[l] = acc;
    }
    for (int off = 32; off >= 1; off >>= 1) {
        for (int l = 0; l < 64; ++l) next[l] = lane[l] + lane[l ^ off];
        memcpy(lane, next, sizeof(lane));
    }
    return lane[0];
}

/* qwen.py:148-152: p = softmax(float(logits)), (w, ids) = topk(p, k) sorted,
 * w /= sum(w) when normalize, weights = bf16(w).  Ties in p select the lower
 * expert id first.  The optional fp32 bias is added to the float logit
 * before the softmax (a documented extension; the reference has none). */
int orc_route_from_logits(const uint16_t *logits, const float *bias, int T, int E, int k,
                          int normalize, int32_t *ids, uint16_t *weights, float *probs) {
    if (T < 0 || E < 1 || E > 1024 || k < 1 || k > E || k > 64) return -1;
    float *l = (float *)malloc(sizeof(float) * (size_t)E);
    float *ex = (float *)malloc(sizeof(float) * (size_t)E);
    float *p = (float *)malloc(sizeof(float) * (size_t)E);
    unsigned char *taken = (unsigned char *)malloc((size_t)E);
    if (!l || !ex || !p || !taken) {
        free(l); free(ex); free(p); free(taken);
        return -1;
    }
    for (int t = 0; t < T; ++t) {
        const uint16_t *row = logits + (size_t)t * E;
        float m = -INFINITY;
        for (int e = 0; e < E; ++e) {
            float v = orc_bf16_to_f32(row[e]);
            if (bias) v = v + bias[e];
            l[e] = v;
            if (v > m) m = v;
        }
        for (int e = 0; e < E; ++e) ex[e] = orc_expf(l[e] - m);
        float s = wave64_sum(ex, E);
        for (int e = 0; e < E; ++e) p[e] = ex[e] / s;
        if (probs) memcpy(probs + (size_t)t * E, p, sizeof(float) * (size_t)E);
        memset(taken, 0, (size_t)E);
        float sel[64];
        for (int j = 0; j < k; ++j) {
            int best = -1;
            for (int e = 0; e < E; ++e) {
                if (taken[e]) continue;
                if (best < 0 || p[e] > p[best]) best = e; /* strict: ties keep lower id */
            }
            taken[best] = 1;
            ids[(size_t)t * k + j] = best;
            sel[j] = p[best];
        }
        float denom = 0.0f;
        if (normalize)
            for (int j = 0; j < k; ++j) denom = denom + sel[j];
        for (int j = 0; j < k; ++j)
            weights[(size_t)t * k + j] = orc_f32_to_bf16(normalize ? sel[j] / denom : sel[j]);
    }
    free(l); free(ex); free(p); free(taken);
    return 0;
}

/* ------------------------------------------------------------ A2 predictor */

void orc_route_hist(const int32_t *ids, int n, int E, int32_t *hist) {
    for (int e = 0; e < E; ++e) hist[e] = 0;
    for (int i = 0; i < n; ++i)
        if (ids[i] >= 0 && ids[i] < E) hist[ids[i]]++;
}

/* ------------------------------------------------------------ A3 grouping */

/* pdscope_runtime.py:23-31: flat = selected.T (slot-major, f = s*T + t),
 * counts = bincount(flat), order = argsort(flat, stable=True),
 * tokens = order % T, positions = tokens*k + order // T.  A stable argsort
 * of small integer keys is a counting sort. */
int orc_pack(const int32_t *ids, int T, int k, int E, int32_t *counts, int32_t *offsets,
             int32_t *perm_token, int32_t *perm_pos, int32_t *row_of) {
    if (T < 1 || k < 1 || E < 1) return -1;
    int64_t n = (int64_t)T * k;
    for (int e = 0; e < E; ++e) counts[e] = 0;
    for (int64_t i = 0; i < n; ++i) {
        if (ids[i] < 0 || ids[i] >= E) return -1;
        counts[ids[i]]++;
    }
    offsets[0] = 0;
    for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t *cursor = (int32_t *)malloc(sizeof(int32_t) * (size_t)E);
    if (!cursor) return -1;
    memcpy(cursor, offsets, sizeof(int32_t) * (size_t)E);
    for (int s = 0; s < k; ++s)
        for (int t = 0; t < T; ++t) {
            int e = ids[(size_t)t * k + s];
            int r = cursor[e]++;
            perm_token[r] = t;
            perm_pos[r] = t * k + s;
            row_of[(size_t)t * k + s] = r;
        }
    free(cursor);
    return 0;
}

/* --------------------------------------------------------- A4 expert math */

static double silu_d(double g) { return g / (1.0 + exp(-g)); }

/* qwen.py:87-90 with torch's bf16 output rounding after every op. */
void orc_expert_forward(const uint16_t *x, int m, const uint16_t *wg, const uint16_t *wu,
                        const uint16_t *wd, int H, int I, uint16_t *y, uint16_t *h) {
    /* Every output element is one exact dot product rounded once, so the
     * work splits over (row, column) pairs: a single-row call uses every
     * thread and the result does not depend on the thread count. */
    uint16_t *hbuf = h ? h : (uint16_t *)malloc(sizeof(uint16_t) * (size_t)m * I);
    if (!hbuf) return;
    int64_t ni = (int64_t)m * I, nj = (int64_t)m * H;
#pragma omp parallel for schedule(static)
    for (int64_t ri = 0; ri < ni; ++ri) {
        int64_t r = ri / I, i = ri % I;
        const uint16_t *xr = x + (size_t)r * H;
        uint16_t g = orc_f64_to_bf16(dot_bf16_exact(xr, wg + (size_t)i * H, H));
        uint16_t u = orc_f64_to_bf16(dot_bf16_exact(xr, wu + (size_t)i * H, H));
        uint16_t a = orc_f64_to_bf16(silu_d(orc_bf16_to_f32(g)));
        hbuf[ri] = orc_f64_to_bf16((double)orc_bf16_to_f32(a) * (double)orc_bf16_to_f32(u));
    }
#pragma omp parallel for schedule(static)
    for (int64_t rj = 0; rj < nj; ++rj) {
        int64_t r = rj / H, j = rj % H;
        y[rj] = orc_f64_to_bf16(dot_bf16_exact(hbuf + (size_t)r * I, wd + (size_t)j * I, I));
    }
    if (!h) free(hbuf);
}

/* qwen.py:93-98 reference_fp32: float math with no intermediate rounding. */
void orc_expert_forward_fp(const uint16_t *x, int m, const uint16_t *wg, const uint16_t *wu,
                           const uint16_t *wd, int H, int I, float *y) {
#pragma omp parallel
    {
        double *hrow = (double *)malloc(sizeof(double) * (size_t)I);
#pragma omp for schedule(static)
        for (int r = 0; r < m; ++r) {
            const uint16_t *xr = x + (size_t)r * H;
            for (int i = 0; i < I; ++i) {
                double g = dot_bf16_exact(xr, wg + (size_t)i * H, H);
                double u = dot_bf16_exact(xr, wu + (size_t)i * H, H);
                hrow[i] = silu_d(g) * u;
            }
            for (int j = 0; j < H; ++j) {
                double acc = 0.0;
                const uint16_t *wr = wd + (size_t)j * I;
                for (int i = 0; i < I; ++i) acc += hrow[i] * (double)orc_bf16_to_f32(wr[i]);
                y[(size_t)r * H + j] = (float)acc;
            }
        }
        free(hrow);
    }
}

/* ---------------------------------------------------------------- A8 merge */

/* pdscope_runtime.py:450-469: out = sum over a token's k rows of w * y.  The
 * reference accumulates in bf16 through index_add_; restated here as the
 * exact weighted sum rounded once. */
void orc_merge(const uint16_t *y, const int32_t *row_of, const uint16_t *w, int T, int k,
               int H, const uint16_t *add_in, uint16_t *out) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t)
        for (int j = 0; j < H; ++j) {
            double acc = add_in ? (double)orc_bf16_to_f32(add_in[(size_t)t * H + j]) : 0.0;
            for (int s = 0; s < k; ++s) {
                int r = row_of[(size_t)t * k + s];
                acc += (double)orc_bf16_to_f32(w[(size_t)t * k + s]) *
                       (double)orc_bf16_to_f32(y[(size_t)r * H + j]);
            }
            out[(size_t)t * H + j] = orc_f64_to_bf16(acc);
        }
}

/* A8 reference merge and A9 GPU half: torch's bf16 index_add_, row by row.
 * out[tokens[r], j] = bf16(out[tokens[r], j] + bf16(rows[r, j] * w[r]))
 * for r = 0..n-1 in order, in bf16 arithmetic (each sum and product of two
 * bf16 values formed in fp32 and rounded to nearest even, as
 * c10::BFloat16's operators do).  Restates the per-expert merge
 * output.index_add_(0, tokens, (parts[e] * coeff[:, None]).to(bf16)) of
 * pdscope_runtime.py:466-468 applied expert by expert, and the
 * out.index_add_(0, tokens, scratch * weights[:, None]) of
 * native_layer_dispatch.cpp:88,129. */
void orc_index_add_bf16(uint16_t *out, int H, const int64_t *tokens, const uint16_t *rows,
                        const uint16_t *w, int64_t n) {
    for (int64_t r = 0; r < n; ++r) {
        uint16_t *o = out + (size_t)tokens[r] * H;
        const uint16_t *y = rows + (size_t)r * H;
        const float wr = orc_bf16_to_f32(w[r]);
        for (int j = 0; j < H; ++j) {
            const float prod = orc_bf16_to_f32(orc_f32_to_bf16(orc_bf16_to_f32(y[j]) * wr));
            o[j] = orc_f32_to_bf16(orc_bf16_to_f32(o[j]) + prod);
        }
    }
}

/* The reference's default merge (merge='reference', pdscope_runtime.py:466-468)
 * for one layer: out starts at zero and each expert's rows are index-added in
 * ascending expert id.  A token meets each expert at most once, so per token
 * this is its k weighted rows added one at a time in ascending expert id,
 * i.e. in ascending grouped row (rows are grouped by expert ascending).
 * add_in (nullable, shared experts) is added last, as a dense block adds its
 * shared-expert output after the routed sum. */
void orc_merge_ordered(const uint16_t *y, const int32_t *row_of, const uint16_t *w, int T, int k,
                       int H, const uint16_t *add_in, uint16_t *out) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
        int r[64], s_of[64];
        for (int s = 0; s < k; ++s) {
            r[s] = row_of[(size_t)t * k + s];
            s_of[s] = s;
        }
        for (int a = 1; a < k; ++a) /* insertion sort by grouped row */
            for (int b = a; b > 0 && r[b - 1] > r[b]; --b) {
                int tr = r[b], ts = s_of[b];
                r[b] = r[b - 1]; s_of[b] = s_of[b - 1];
                r[b - 1] = tr; s_of[b - 1] = ts;
            }
        for (int j = 0; j < H; ++j) {
            float acc = 0.0f;
            for (int q = 0; q < k; ++q) {
                const float wr = orc_bf16_to_f32(w[(size_t)t * k + s_of[q]]);
                const float prod =
                    orc_bf16_to_f32(orc_f32_to_bf16(orc_bf16_to_f32(y[(size_t)r[q] * H + j]) * wr));
                acc = orc_bf16_to_f32(orc_f32_to_bf16(acc + prod));
            }
            if (add_in) acc = orc_bf16_to_f32(orc_f32_to_bf16(acc + orc_bf16_to_f32(add_in[(size_t)t * H + j])));
            out[(size_t)t * H + j] = orc_f32_to_bf16(acc);
        }
    }
}

/* ---------------------------------------------------------------- layer */

int orc_moe_layer(const uint16_t *x, int T, int H, int I, int E, int k, int normalize,
                  const uint16_t *gate, const float *bias, const uint16_t *const *slots,
                  uint16_t *out, uint16_t *logits_out, int32_t *ids_out, uint16_t *w_out) {
    if (T < 1 || H < 1 || I < 1 || E < 1 || k < 1 || k > E) return -1;
    size_t n = (size_t)T * k;
    uint16_t *logits = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)T * E);
    int32_t *ids = (int32_t *)malloc(sizeof(int32_t) * n);
    uint16_t *w = (uint16_t *)malloc(sizeof(uint16_t) * n);
    int32_t *counts = (int32_t *)malloc(sizeof(int32_t) * (size_t)E);
    int32_t *offsets = (int32_t *)malloc(sizeof(int32_t) * (size_t)(E + 1));
    int32_t *ptok = (int32_t *)malloc(sizeof(int32_t) * n);
    int32_t *ppos = (int32_t *)malloc(sizeof(int32_t) * n);
    int32_t *row_of = (int32_t *)malloc(sizeof(int32_t) * n);
    uint16_t *xg = (uint16_t *)malloc(sizeof(uint16_t) * n * (size_t)H);
    uint16_t *y = (uint16_t *)malloc(sizeof(uint16_t) * n * (size_t)H);
    int rc = -1;
    if (!logits || !ids || !w || !counts || !offsets || !ptok || !ppos || !row_of || !xg || !y)
        goto done;
    orc_route_logits(x, gate, T, H, E, logits);
    if (orc_route_from_logits(logits, bias, T, E, k, normalize, ids, w, NULL)) goto done;
    if (orc_pack(ids, T, k, E, counts, offsets, ptok, ppos, row_of)) goto done;
    for (size_t r = 0; r < n; ++r)
        memcpy(xg + r * H, x + (size_t)ptok[r] * H, sizeof(uint16_t) * (size_t)H);
    for (int e = 0; e < E; ++e) {
        int m = counts[e];
        if (!m) continue;
        const uint16_t *base = slots[e];
        size_t ih = (size_t)I * H;
        orc_expert_forward(xg + (size_t)offsets[e] * H, m, base, base + ih, base + 2 * ih, H, I,
                           y + (size_t)offsets[e] * H, NULL);
    }
    orc_merge(y, row_of, w, T, k, H, NULL, out);
    if (logits_out) memcpy(logits_out, logits, sizeof(uint16_t) * (size_t)T * E);
    if (ids_out) memcpy(ids_out, ids, sizeof(int32_t) * n);
    if (w_out) memcpy(w_out, w, sizeof(uint16_t) * n);
    rc = 0;
done:
    free(logits); free(ids); free(w); free(counts); free(offsets);
    free(ptok); free(ppos); free(row_of); free(xg); free(y);
    return rc;
}
