/*
 * pdscope_moe.h -- C-ABI of libpdscope_moe.so, the gfx950 MoE-layer path.
 *
 * Plain pointers and sizes only.  Every device pointer is a HIP device
 * address (hipMalloc / torch CUDA tensor storage); `stream` is a hipStream_t
 * (NULL = legacy default stream).  bf16 tensors are row-major arrays of
 * 16-bit bfloat16 bit patterns.
 *
 * Return value: 0 on success, 1 for an invalid argument, 2 for a HIP runtime
 * error; pdscope_last_error() then returns a thread-local message.  No entry
 * point allocates device memory, synchronises the device or reads device
 * memory on the host, so every launch sequence can be captured in a hipGraph.
 * Work is stream-ordered on `stream`.
 *
 * Expert weights are addressed through a device table `slots[E]` of base
 * pointers; expert e's block holds gate_proj [I,H], up_proj [I,H] and
 * down_proj [H,I] back to back (bf16, row-major), the order of
 * PROJECTIONS in expertbench/adapters/qwen.py:27 and of the per-expert
 * copy in expertbench/executor.py:344-357.  Cache slots and demand staging
 * slots are therefore addressed uniformly.
 */
#ifndef PDSCOPE_MOE_H
#define PDSCOPE_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message for the last failing call on this thread ("" if none). */
const char *pdscope_last_error(void);

/* Library version string. */
const char *pdscope_version(void);

/* Bytes of zero-initialised device workspace pdscope_route_topk needs for
 * T <= 8 tokens (the caller zero-fills it once; the kernels leave it zeroed). */
size_t pdscope_route_workspace_bytes(void);

/* Bytes of workspace pdscope_route_topk needs for T tokens of hidden size H
 * and E experts: the zeroed 256-byte block above, followed (T > 8) by the
 * split-K partial logits.  Zero-fill once at allocation. */
size_t pdscope_route_workspace_size(int T, int H, int E);

/*
 * A1 router: replaces `route` (expertbench/adapters/qwen.py:140-152).
 *   logits[t,e] = bf16(sum_h x[t,h] * gate[e,h])     (fp32 accumulation)
 *   p = softmax(float(logits[t,:]) + bias)           (fp32; bias nullable)
 *   ids[t,:]    = top-k experts by p, ties -> lower expert id, sorted
 *   weights     = bf16(p_sel / sum(p_sel)) if normalize else bf16(p_sel)
 * x [T,H] bf16, gate [E,H] bf16, bias [E] fp32 or NULL, logits [T,E] bf16,
 * ids [T,k] int32, weights [T,k] bf16, probs [T,E] fp32 or NULL.
 * Limits: E % 32 == 0, E <= 256, 1 <= k <= min(E, 16), H % 16 == 0.
 * workspace: pdscope_route_workspace_size(T, H, E) bytes, zero-filled once.
 * T > 8 runs two launches (split-K MFMA partial logits, then one wave per
 * token sums them in a fixed order and routes); T <= 8 one GEMV launch.
 */
int pdscope_route_topk(const void *x, const void *gate, const float *bias, int T, int H, int E,
                       int k, int normalize, void *logits, int32_t *ids, void *weights,
                       float *probs, void *workspace, void *stream);

/*
 * A2 gate-fallback predictor histogram: replaces the Counter over
 * route(x, next_gate).selected (expertbench/pdscope_runtime.py:245-249).
 * hist[e] = number of (t, slot) with ids[t,slot] == e; hist is overwritten.
 */
int pdscope_route_hist(const int32_t *ids, int n, int E, int32_t *hist, void *stream);

/*
 * A3 ragged grouping: replaces compact_expert_groups
 * (expertbench/pdscope_runtime.py:16-39) and expert_groups
 * (expertbench/adapters/qwen.py:155-174).
 * Stable order over the slot-major flat index f = s*T + t, grouped by expert
 * ascending.  Outputs: counts[E], offsets[E+1] (exclusive prefix sum),
 * perm_token[T*k] (token of each grouped row), perm_pos[T*k] (= t*k + s) and
 * row_of[T*k] (grouped row of position t*k+s).  Requires E <= 256.
 * workspace: pdscope_pack_workspace_size(T, k, E) bytes (NULL when that is
 * 0: small inputs run one workgroup; larger ones two multi-block launches).
 */
size_t pdscope_pack_workspace_size(int T, int k, int E);
int pdscope_pack(const int32_t *ids, int T, int k, int E, int32_t *counts, int32_t *offsets,
                 int32_t *perm_token, int32_t *perm_pos, int32_t *row_of, void *workspace, void *stream);

/*
 * pdscope_pack without a workspace argument and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under hipGraph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments and outputs as pdscope_pack (bit
 * for bit); the multi-block path's per-chunk counts live in a library-owned
 * static device array of 512 KiB per GPU whose address is looked up once per
 * device: by pdscope_pack_static_max_ids() with that device current (call it
 * at set-up, before any capture; it returns 0 if the lookup fails), else by
 * the first multi-block call.  Limit: T*k <= pdscope_pack_static_max_ids()
 * (1048576 ids);
 * larger inputs return 1 (EINVAL).  Every call on one GPU shares that GPU's
 * array, so calls that overlap in time on one GPU (several streams or
 * threads) race; nothing in the array has to be cleared between calls.
 */
size_t pdscope_pack_static_max_ids(void);
int pdscope_pack_static(const int32_t *ids, int T, int k, int E, int32_t *counts, int32_t *offsets,
                        int32_t *perm_token, int32_t *perm_pos, int32_t *row_of, void *stream);

/*
 * Tile schedule for pdscope_swiglu_grouped over a subset of experts:
 * tile_start[i] = sum_{j<i} ceil(counts[sel[j]] / block_m), i = 0..nsel.
 * counts has E entries; a sel entry outside [0, E) counts as an expert with
 * no rows (the same holds for the balanced schedules below and for the
 * schedule written by pdscope_pack_schedule_balanced).
 * block_m is the row tile the grouped call will use (see
 * pdscope_grouped_block_m).
 */
int pdscope_schedule(const int32_t *counts, int E, const int32_t *sel, int nsel, int block_m,
                     int32_t *tile_start, void *stream);

/*
 * Balanced tile schedule: the grouped kernels cut the tile list (in sel
 * order) into 8 contiguous equal-count pieces, one per XCD.  This orders the
 * experts so those pieces hold similar work and start with their largest
 * experts: rank the selected experts by rows (descending, ties by position),
 * deal rank r to group (r/8 even ? r%8 : 7-r%8), concatenate the groups.
 * order[nsel] receives the experts in that order and tile_start[nsel+1] the
 * m-tile prefix over order; pass `order` as sel to pdscope_swiglu_grouped*.
 * No counterpart in the reference (its experts run one launch each).
 * Limits: nsel <= 256.
 */
int pdscope_schedule_balanced(const int32_t *counts, int E, const int32_t *sel, int nsel, int block_m,
                              int32_t *order, int32_t *tile_start, void *stream);

/*
 * pdscope_schedule_balanced for a gate/up and a down launch whose row tiles
 * differ, in one launch: the order depends on the rows only, so both
 * launches take `order`; tile_start is its m-tile prefix for block_m and
 * tile_start2 for block_m2.  No counterpart in the reference.
 */
int pdscope_schedule_balanced_pair(const int32_t *counts, int E, const int32_t *sel, int nsel, int block_m,
                                   int block_m2, int32_t *order, int32_t *tile_start, int32_t *tile_start2,
                                   void *stream);

/*
 * pdscope_pack followed by the balanced schedule of `sel` over the counts it
 * produces (pdscope_schedule_balanced, or _pair when block_m2 != 0 with
 * tile_start2), computed inside the pack launch by one extra workgroup (it
 * counts the ids itself, or sums the per-chunk counts of the multi-block path)
 * beside the scatter, so the schedule costs no launch of its own.  Outputs as
 * the two calls give them.  No counterpart in the reference.
 */
int pdscope_pack_schedule_balanced(const int32_t *ids, int T, int k, int E, int32_t *counts, int32_t *offsets,
                                   int32_t *perm_token, int32_t *perm_pos, int32_t *row_of, void *workspace,
                                   const int32_t *sel, int nsel, int block_m, int block_m2, int32_t *order,
                                   int32_t *tile_start, int32_t *tile_start2, void *stream);

/* Row tile (32, 64, 128, 256 or 384) for `rows_hint` average rows per
 * selected expert: <= 16 rows 32, <= 64 rows 64, <= 124 rows 128, <= 192 rows
 * 256, <= 320 rows 384 (one tile holds a typical expert, so its weights
 * stream once), 256 above.  No reference counterpart: the reference launches
 * one torch GEMM chain per expert (expertbench/adapters/qwen.py:87-90). */
int pdscope_grouped_block_m(int rows_hint);

/* As pdscope_grouped_block_m(mean_rows), except that a launch whose largest
 * expert has more than 768 rows keeps the 256-row tile instead of 384: the
 * 384-row tile is 128 columns wide and reads every activation row twice as
 * often, which costs more than it saves once a few experts span several
 * row tiles (skewed routing). */
int pdscope_grouped_block_m_max(int mean_rows, int max_rows);

/*
 * A4 grouped SwiGLU for prefill: replaces expert_forward
 * (expertbench/adapters/qwen.py:87-90) over every selected expert, as
 * launched per expert by ExpertExecutor.gpu (expertbench/executor.py:454-488).
 * For each selected expert e and each grouped row r in
 * [offsets[e], offsets[e+1]):
 *   g,u  = bf16(x[perm_token[r]] . gate_e^T), bf16(x[perm_token[r]] . up_e^T)
 *   h[r] = bf16(bf16(silu(g)) * u)                    (h_ws [T*k, I] bf16)
 *   y[r] = bf16(h[r] . down_e^T)                      (y [T*k, H] bf16)
 * bf16 MFMA with fp32 accumulation.  max_tiles bounds sum ceil(m_e/block_m)
 * (e.g. ceil(rows/block_m) + nsel); tiles beyond tile_start[nsel] exit.
 * block_m: 32, 64, 128 or 256, the row tile pdscope_schedule used.
 * Limits: H % 256 == 0 and I % 128 == 0 (every row tile is 256 columns
 * wide: 128 gate + 128 up columns, or 256 output columns).
 */
int pdscope_swiglu_grouped(const void *x, const int32_t *perm_token, const int32_t *offsets,
                           const int32_t *sel, int nsel, const int32_t *tile_start,
                           int max_tiles, int block_m, const void *const *slots, int H, int I,
                           void *h_ws, void *y, void *stream);

/* The two launches of pdscope_swiglu_grouped, separately (same arguments):
 * gate/up + SwiGLU into h_ws, then down into y.  Lets a caller overlap or
 * time them individually. */
int pdscope_swiglu_grouped_gateup(const void *x, const int32_t *perm_token, const int32_t *offsets,
                                  const int32_t *sel, int nsel, const int32_t *tile_start, int max_tiles,
                                  int block_m, const void *const *slots, int H, int I, void *h_ws,
                                  void *stream);
int pdscope_swiglu_grouped_down(const void *h_ws, const int32_t *offsets, const int32_t *sel, int nsel,
                                const int32_t *tile_start, int max_tiles, int block_m,
                                const void *const *slots, int H, int I, void *y, void *stream);

/*
 * A8 fused weighted merge: replaces the index_add_ merge
 * (expertbench/pdscope_runtime.py:450-469).
 *   out[t,:] = bf16( add_in[t,:] + sum_s w[t,s] * y[row_of[t*k+s],:] )
 * summed in fp32 in slot order s = 0..k-1 and rounded once; deterministic.
 * add_in (nullable) is added unweighted (shared experts).
 */
int pdscope_merge(const void *y, const int32_t *row_of, const void *w, int T, int k, int H,
                  const void *add_in, void *out, void *stream);

/*
 * A8 in the arithmetic of the reference's default merge (merge='reference',
 * expertbench/pdscope_runtime.py:454-468: a zero output and one bf16
 * index_add_ of parts[e] * coeff per expert, experts in ascending id).  A
 * token meets an expert at most once, so per token its k rows are added in
 * ascending expert id (= ascending grouped row):
 *   acc = 0;  acc = bf16(acc + bf16(w[t,s] * y[row,:]))  for each row;
 *   out[t,:] = add_in ? bf16(acc + add_in[t,:]) : acc    (add_in added last).
 * Same arguments as pdscope_merge; deterministic, bit-exact with that
 * sequence of index_add_ calls.
 */
int pdscope_merge_ordered(const void *y, const int32_t *row_of, const void *w, int T, int k, int H,
                          const void *add_in, void *out, void *stream);

/*
 * A4+A8 for one decode token (T == 1): replaces the per-expert decode
 * submissions (expertbench/pdscope_runtime.py:326-350, executor.py:454-488,
 * including the resident-graph replay of executor.py:113-138) and the merge.
 *   h_s  = bf16(bf16(silu(bf16(x.gate_s^T))) * bf16(x.up_s^T))  (h_ws [k,I])
 *   y_s  = bf16(h_s . down_s^T)
 *   merge_mode 0: out = bf16( sum_s w[s] * y_s ), fp32 in slot order, one rounding
 *   merge_mode 1: the y_s added in ascending expert id in bf16 arithmetic, as
 *                 pdscope_merge_ordered (the reference's default merge)
 * for the k experts ids[0..k). Streaming GEMV, weights read once.
 * Limits: H % 8 == 0, H <= 4096, I % 8 == 0, k <= 16, k*I*2 <= 64 KiB.
 */
int pdscope_swiglu_decode(const void *x, const int32_t *ids, const void *w, int k,
                          const void *const *slots, int H, int I, void *h_ws, void *out,
                          int merge_mode, void *stream);

/*
 * A1+A4+A8 for one decode token in ONE launch: replaces route
 * (expertbench/adapters/qwen.py:140-152), the per-expert decode submissions
 * (expertbench/pdscope_runtime.py:326-350, executor.py:454-488, including the
 * resident-graph replay of executor.py:113-138) and the merge
 * (pdscope_runtime.py:450-469).  Results are bitwise those of
 * pdscope_route_topk followed by pdscope_swiglu_decode (same arguments,
 * merge_mode as there).
 * x [H], gate [E,H], bias [E] fp32 or NULL, logits [E] bf16, ids [k] int32,
 * weights [k] bf16, probs [E] fp32 or NULL, h_ws [k*I] bf16, out [H] bf16.
 * workspace: pdscope_decode_workspace_bytes() bytes, zero-filled once by the
 * caller and then owned by the kernel (per-block epochs and the words that
 * carry logits and h between blocks; nothing to reset between launches).
 * One workspace serves every launch of one hidden size H on one stream;
 * launches that overlap in time, or of another H, need their own.
 * 32-bit word 1024 of the workspace is a sticky error flag: non-zero if a
 * bounded internal wait gave up (the output is then invalid).
 * Returns 1 (EINVAL) for shapes outside the kernel (see
 * pdscope_decode_layer_supported; E must be even, k <= 8) and when its grid
 * of H/4 blocks cannot be resident at once on the current device.
 */
size_t pdscope_decode_workspace_bytes(void);
int pdscope_decode_layer_supported(int H, int I, int E, int k);

/*
 * Whether pdscope_decode_layer_chained can run this shape on the current
 * device: the checks of pdscope_decode_layer_supported, the next-layer
 * predictor's grid condition when with_predictor is non-zero, and the
 * co-residency of the chained variant's grid (it has its own registers and
 * static LDS).  Replaces the graph-capture precondition of the reference's
 * resident expert graphs (expertbench/executor.py:42-146), which only
 * capture what can replay.
 */
int pdscope_decode_layer_chained_supported(int H, int I, int E, int k, int with_predictor);
int pdscope_decode_layer(const void *x, const void *gate, const float *bias, int H, int E, int k,
                         int normalize, int merge_mode, const void *const *slots, int I, void *logits,
                         int32_t *ids, void *weights, float *probs, void *h_ws, void *out, void *workspace,
                         void *stream);

/*
 * pdscope_decode_layer for one layer of a chain of decode layers, with the
 * residual sum and the next layer's gate-fallback prediction folded in:
 * replaces, besides what pdscope_decode_layer replaces, the predictor route
 * route(inputs, next_gate, top_k, normalize) of
 * expertbench/pdscope_runtime.py:245-249 (the ids that pick the next layer's
 * prefetches).
 *   resid, x_out   both NULL, or both [H] bf16: the layer input is then
 *                  bf16(x + resid) (fp32 sum, one rounding), written to x_out;
 *   next_gate, pred_out  both NULL, or [E,H] bf16 and [k] int32: pred_out
 *                  receives the top-k of next_gate . input (no bias), the
 *                  ids pdscope_route_topk gives for that gate and input.
 *                  Needs E <= H/2.
 * Every other argument and output is as in pdscope_decode_layer, and with
 * all four NULL the call is pdscope_decode_layer.
 */
int pdscope_decode_layer_chained(const void *x, const void *resid, void *x_out, const void *gate,
                                 const float *bias, int H, int E, int k, int normalize, int merge_mode,
                                 const void *const *slots, int I, const void *next_gate, int32_t *pred_out,
                                 void *logits, int32_t *ids, void *weights, float *probs, void *h_ws, void *out,
                                 void *workspace, void *stream);

/*
 * A bound resident decode layer: replaces the per-expert resident graph
 * replay of the reference (ResidentExpertGraphs.__call__,
 * expertbench/executor.py:113-135: input copy, replay, output copy) together
 * with the routing read-back that reveals the demand
 * (expertbench/pdscope_runtime.py:25-26, :249).
 *
 * pdscope_decode_bind checks and plans every argument of
 * pdscope_decode_layer_chained that stays put from one token to the next
 * (resid / x_out are not bound: NULL) and keeps them in a host record
 * (*binding, freed by pdscope_decode_unbind); the pointed-to buffers must
 * outlive it.  ids [k] int32 is device scratch of the binding; host_ids
 * (2k words) and host_error (1 word) must be pinned host memory
 * (hipHostMalloc), else the call fails.
 *
 * pdscope_decode_run enqueues on `stream`, on the binding's device, a token
 * numbered seq (1 .. 32767, else EINVAL): the fused decode kernel (inputs x,
 * outputs out / logits / weights as in pdscope_decode_layer), which stores
 * host_ids[0,k) = (seq << 16) | routed id as soon as its routing is final,
 * before the kernel completes (and, when selected != NULL, selected[0,k) =
 * the routed ids as int64 on the device), and host_ids[k,2k) = (seq << 16) |
 * predicted id (when bound with next_gate); then a one-wave kernel that
 * stores *host_error = (seq << 16) | the workspace's sticky error word.
 * Each word is valid once it carries seq in its upper half (no fence orders
 * them).  *host_error is stored after the decode kernel completed, so a host
 * that reads seq there knows the launch (and anything the stream ordered
 * before it) has completed, and finds the other words tagged too.  Two
 * launches per token, no graph: replaying a captured graph of the same
 * kernel costs the host several times more.  Calls that share a binding or
 * its workspace must be ordered on one stream.
 */
typedef struct pdscope_decode_binding pdscope_decode_binding;
int pdscope_decode_bind(const void *gate, const float *bias, int H, int E, int k, int normalize, int merge_mode,
                        const void *const *slots, int I, const void *next_gate, int32_t *pred_out, int32_t *ids,
                        float *probs, void *h_ws, void *workspace, int32_t *host_ids, int32_t *host_error,
                        pdscope_decode_binding **binding);
int pdscope_decode_run(const pdscope_decode_binding *binding, const void *x, void *out, void *logits,
                       void *weights, int64_t *selected, int32_t seq, void *stream);
void pdscope_decode_unbind(pdscope_decode_binding *binding);

/*
 * A7 demand staging: replaces the three per-projection non_blocking copies
 * (expertbench/executor.py:341-363).  One hipMemcpyAsync of `bytes` from
 * page-locked host memory into a cache or staging slot on `stream`, then
 * hipEventRecord(event) when event != NULL.
 */
int pdscope_stage_expert(void *dst_slot, const void *pinned_src, size_t bytes, void *event,
                         void *stream);

/*
 * A9 native CPU-group tail, GPU half: replaces the stage + index_add_ of
 * finish_and_merge / submit_and_merge (native/native_layer_dispatch.cpp:83-88,
 * 124-129).  Copies host block [rows, row_bytes] into device scratch, then
 * for r = 0..rows-1 in order: out[tokens[r],:] += bf16(scratch[r,:]*weights[r])
 * with bf16 accumulation (one valid order of the reference's index_add_).
 * tokens int64 [rows], weights bf16 [rows], out bf16 [out_rows, row_bytes/2];
 * a row whose token lies outside [0, out_rows) is skipped.
 */
int pdscope_stage_merge(const void *host_block, int64_t rows, int64_t row_bytes, void *scratch,
                        void *out, const int64_t *tokens, const void *weights, int64_t out_rows,
                        void *stream);

/*
 * A9 native CPU-group tail, host half: replaces fill_packed and the id /
 * coefficient / count setup of submit_group (native/native_layer_dispatch.cpp:
 * 34-40, 59-67).  Copies `row` (row_bytes) into packed[r] for r < rows, sets
 * selected[r] = ids[r], coeff[r] = 1.0f and *count = rows.  Host memory only.
 */
int pdscope_dispatch_pack(const void *row, int64_t rows, int64_t row_bytes, void *packed, int32_t *count,
                          int64_t *selected, float *coeff, const int64_t *ids);

#ifdef __cplusplus
}
#endif
#endif /* PDSCOPE_MOE_H */
