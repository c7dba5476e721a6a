/*
 * oracle.h -- CPU restatement of PDScope's GPU MoE-layer arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only to check results against.
 *
 * Every function cites the reference line it restates.  All bf16 values are
 * raw uint16_t bit patterns (the upper half of an IEEE binary32).
 *
 * Rounding conventions (documented choices, see the .c file):
 *   - "exact then round": dot products are accumulated in binary64 (each
 *     bf16*bf16 product is exact there) and rounded ONCE to bf16 with
 *     round-to-nearest-even (via round-to-odd to binary32, which makes the
 *     two-step rounding equal to a single correct rounding).
 *   - softmax uses orc_expf(), a Cody-Waite reduced degree-7 Taylor exp
 *     whose fp32 operation sequence is fixed, so the same value can be
 *     recomputed bit-for-bit by the GPU kernel.
 */
#ifndef PDSCOPE_ORACLE_H
#define PDSCOPE_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 helpers */
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);      /* round to nearest even */
uint16_t orc_f64_to_bf16(double d);     /* single correct rounding */
float orc_expf(float x);                /* x <= 0 domain, flushes below 2^-126 */

/* A1 logits: logits[t,e] = bf16(sum_h x[t,h]*gate[e,h])
 * (expertbench/adapters/qwen.py:147, F.linear with fp32 accumulation). */
void orc_route_logits(const uint16_t *x, const uint16_t *gate, int T, int H, int E,
                      uint16_t *logits);

/* A1 softmax/top-k/renorm from given bf16 logits (qwen.py:148-152).
 * bias (nullable, fp32 [E]) is added to float(logit) before the softmax.
 * ids are sorted by (probability desc, expert id asc).  probs (nullable)
 * receives the full fp32 softmax row [T,E].  Returns 0 or -1 on bad args. */
int orc_route_from_logits(const uint16_t *logits, const float *bias, int T, int E, int k,
                          int normalize, int32_t *ids, uint16_t *weights, float *probs);

/* A2 predictor histogram (pdscope_runtime.py:245-249): hist[e] = #(ids == e). */
void orc_route_hist(const int32_t *ids, int n, int E, int32_t *hist);

/* A3 grouping (pdscope_runtime.py:16-39, qwen.py:168-174).  ids is [T,k]
 * row-major.  Stable order over slot-major flat index f = s*T + t, grouped by
 * expert ascending.  counts[E], offsets[E+1], perm_token[T*k], perm_pos[T*k]
 * (= t*k+s) and row_of[T*k] (row_of[t*k+s] = grouped row).  Returns 0/-1. */
int orc_pack(const int32_t *ids, int T, int k, int E, int32_t *counts, int32_t *offsets,
             int32_t *perm_token, int32_t *perm_pos, int32_t *row_of);

/* A4 expert formula (qwen.py:87-90) with torch's bf16 roundings after each
 * op: g,u = bf16(x.W^T); a = bf16(silu(g)); h = bf16(a*u); y = bf16(h.Wd^T).
 * x [m,H]; wg,wu [I,H]; wd [H,I]; y [m,H]; h (nullable) [m,I]. */
void orc_expert_forward(const uint16_t *x, int m, const uint16_t *wg, const uint16_t *wu,
                        const uint16_t *wd, int H, int I, uint16_t *y, uint16_t *h);

/* A4 FP32 twin (qwen.py:93-98): no intermediate rounding, binary64 math,
 * output float [m,H]. */
void orc_expert_forward_fp(const uint16_t *x, int m, const uint16_t *wg, const uint16_t *wu,
                           const uint16_t *wd, int H, int I, float *y);

/* A8 merge (pdscope_runtime.py:450-469): out[t] = bf16(sum_s w[t,s]*y[row_of[t*k+s]]),
 * summed exactly then rounded once.  If add_in (nullable, [T,H] bf16) is given
 * it is added unweighted (shared experts). */
void orc_merge(const uint16_t *y, const int32_t *row_of, const uint16_t *w, int T, int k,
               int H, const uint16_t *add_in, uint16_t *out);

/* torch bf16 index_add_ row by row: out[tokens[r]] = bf16(out + bf16(rows[r] * w[r])),
 * r = 0..n-1 in order (pdscope_runtime.py:466-468, native_layer_dispatch.cpp:88,129). */
void orc_index_add_bf16(uint16_t *out, int H, const int64_t *tokens, const uint16_t *rows,
                        const uint16_t *w, int64_t n);

/* The reference's default merge: per token its k weighted rows added in bf16, one
 * at a time, in ascending expert id (= ascending grouped row); add_in added last. */
void orc_merge_ordered(const uint16_t *y, const int32_t *row_of, const uint16_t *w, int T, int k,
                       int H, const uint16_t *add_in, uint16_t *out);

/* Whole layer: route -> pack -> experts -> merge.  slots[e] points at expert
 * e's gate|up|down block (row-major [I,H],[I,H],[H,I]).  Outputs are optional
 * (nullable) except out.  Returns 0/-1. */
int orc_moe_layer(const uint16_t *x, int T, int H, int I, int E, int k, int normalize,
                  const uint16_t *gate, const float *bias, const uint16_t *const *slots,
                  uint16_t *out, uint16_t *logits_out, int32_t *ids_out, uint16_t *w_out);

/* CPU baseline stand-in for ktransformers AVX2BF16_MOE.forward_task
 * (baselines/ktransformers/runtime.py:180-181): rows of a packed input, each
 * row r processed by expert selected[r] and scaled by coeff[r].
 * Multi-threaded AVX2 (nthreads workers).  fp32 accumulation, bf16 h/y.
 * Returns 0, or -1 when AVX2/FMA is unavailable. */
int cpu_moe_forward_rows(const uint16_t *x, int rows, const int64_t *selected,
                         const float *coeff, const uint16_t *const *slots, int H, int I,
                         uint16_t *out, int nthreads);

/* Same kernel, one token through k experts, merged with weights (decode). */
int cpu_moe_decode(const uint16_t *x, const int32_t *ids, const uint16_t *w, int k,
                   const uint16_t *const *slots, int H, int I, uint16_t *out, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
