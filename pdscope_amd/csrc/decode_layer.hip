// K4f: the whole T == 1 MoE layer in one persistent launch: router logits,
// softmax / top-k / renorm, the SwiGLU gate/up GEMV of the k routed experts
// and their down projection with the weighted merge.
// Restates, for one decode token, route (expertbench/adapters/qwen.py:140-152),
// the per-expert decode submissions of PDScopeCudaRuntime.forward
// (expertbench/pdscope_runtime.py:326-350; expert_forward, qwen.py:87-90) and
// the merge (pdscope_runtime.py:450-469).
//
// Grid: one wave per output column (H / 4 blocks of 4 waves), sized so that
// every block is resident at once (checked against the occupancy of this
// kernel on the current device).  Phases:
//   1. blocks 0 .. E/4-1: one wave per router row -> bf16 logit;
//   2. wave 0 of every block collects the E logits and picks the experts
//      itself, so no further hop publishes the routing: without a logit bias
//      by unique bf16-logit keys, each rank stored as soon as it is known,
//      then checked against the softmax probabilities while the rows stream
//      (on a mismatch the exact top-k replaces the pick and the rows it
//      changes are computed again); with a bias, the exact softmax / top-k;
//   3. every wave issues the loads of its P (gate, up) row pairs of the
//      routed experts (16-byte non-temporal loads) once the rank of its rows
//      is picked;
//   4. gate/up dot products -> h; then the wave issues its down-projection
//      rows (two slots x four output columns), which land while h is
//      handed between blocks;
//   5. every block collects all of h, finishes its down rows and merges:
//      merge_mode 0: out[j] = bf16(sum_s w_s * y_s[j]) in fp32, slot order,
//      one rounding; merge_mode 1 (the reference's merge arithmetic,
//      expertbench/pdscope_runtime.py:466-468): y_s added in ascending
//      expert id, acc = bf16(acc + bf16(w_s * y_s[j])); y_s = bf16(h_s . down_s[j]).
//
// Cross-block hand-off without read-modify-write atomics.  Same-address
// atomics from hundreds of blocks serialise at the memory side (~14 ns
// each), and a release fence per block writes back the whole XCD L2, so a
// counter barrier costs several microseconds.  Instead every published
// value is one 32-bit word (epoch << 16 | bf16 bits) written with
// device-scope relaxed stores (write-through) and read with device-scope
// relaxed loads until its epoch is the current one.  A value and its
// validity travel in one word, so no ordering between locations is needed.
// Each block publishes its words from its last wave, in 8-byte stores
// (logits: 4 per block in a line of their own, one thread; h: 4P
// consecutive words, 2P threads), and polls with the other waves.
// The epoch is a per-block counter kept in the workspace (all blocks of a
// launch see the same value because every launch runs every block once);
// it cycles through 1..65535, never 0, so a zero-filled workspace holds no
// valid word.  Polling is bounded: each thread has kSpinBudget polls for the
// whole launch; when they are spent it sets the sticky error word and uses
// what it read, so the launch always drains.  Because the epochs advance
// per block, one workspace serves one grid size (one H) on one stream.
//
// Per-lane arithmetic order equals route_gemv_kernel, decode_gateup_kernel
// and decode_down_kernel, so the result is bitwise the result of the
// three-launch path (pdscope_route_topk + pdscope_swiglu_decode).
#include <mutex>
#include <new>
#include <unordered_map>

#include "common.h"
#include "topk.h"

namespace pd {

// Polls one thread may spend over the whole launch (a normal launch needs a
// few hundred at most); once spent, the thread stops waiting.
constexpr uint32_t kSpinBudget = 1u << 16;

// First thread of the last wave of a block: it publishes the block's words
// and that wave takes no part in polling.  On gfx9 the vector-memory counter
// covers stores as well as loads, so a wave that has just stored would see
// each of its polls wait for its stores to be acknowledged (write-through to
// memory, slow while the weight stream saturates HBM); for the same reason
// the logits and h_ws outputs are stored at the end of the launch.
constexpr int kPublisher = 192;

constexpr int kDecodeMaxK = 8;
constexpr int kDecodeMaxE = 256;
constexpr int kDecodeMaxBlocks = 1024;
constexpr int kDecodeMaxKI = 16384;  // k * I words of h

// Workspace layout in 32-bit words (zero-filled once by the caller).
constexpr int kWsEpoch = 0;                          // [kDecodeMaxBlocks] per-block epoch
constexpr int kWsError = kDecodeMaxBlocks;           // sticky error word
constexpr int kWsLogit = kWsError + 32;              // [kDecodeMaxE / 4] lines of 4 published logits
constexpr int kWsH = kWsLogit + kDecodeMaxE * 8;     // [kDecodeMaxKI] published h
constexpr int kWsPLogit = kWsH + kDecodeMaxKI;       // [kDecodeMaxE / 4] lines of next-layer predictor logits
constexpr int kWsWords = kWsPLogit + kDecodeMaxE * 8;

__device__ __forceinline__ uint64_t load_pair(const uint32_t *w) {
    return __hip_atomic_load(reinterpret_cast<const uint64_t *>(w), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool pair_ready(uint64_t v, uint32_t epoch) {
    return ((uint32_t)v >> 16) == epoch && (uint32_t)(v >> 48) == epoch;
}

// Poll the word pair at w until both words carry `epoch`, keeping four
// polls in flight: the oldest is checked when it returns and re-issued at
// once, so the pair is seen about a quarter of a round trip after it became
// visible instead of up to a whole one.  The four loads live in fixed
// registers and the loop is uniform over the active lanes (a lane latches
// its value when ready; the loop ends when every active lane has one), so
// the compiler's wait analysis keeps three newer polls in flight at each
// check.  Loads left in flight on return are harmless (later waits cover
// them).  Every round spends one unit of budget; when it runs out the
// sticky error word is set (a lane without a current value then returns 0).
__device__ __forceinline__ uint64_t poll_pair(const uint32_t *w, uint32_t epoch, uint32_t *err, uint32_t &budget) {
    uint64_t p0 = load_pair(w), p1 = load_pair(w), p2 = load_pair(w), p3 = load_pair(w);
    uint64_t got = 0;
    bool have = false;
    for (;;) {
#define PD_POLL_STEP(P)                              \
        {                                            \
            const bool r = !have && pair_ready(P, epoch); \
            got = r ? P : got;                       \
            have = have || r;                        \
        }                                            \
        if (__ballot(!have) == 0) return got;        \
        P = load_pair(w);
        PD_POLL_STEP(p0)
        PD_POLL_STEP(p1)
        PD_POLL_STEP(p2)
        PD_POLL_STEP(p3)
#undef PD_POLL_STEP
        if (budget == 0) {
            __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return got;
        }
        --budget;
    }
}

// Collect `count` published words starting at w (count even, w 8-byte
// aligned) into dst (LDS, 16-bit values), cooperatively: thread t takes the
// word pairs t, t + nthreads, ...  B pair loads are issued together, then
// the ones not yet current are re-read until they are.  `budget` is the
// calling thread's remaining poll allowance for the launch.
template <int B>
__device__ __forceinline__ void collect(const uint32_t *w, int count, int t, int nthreads, uint32_t epoch,
                                        uint32_t *err, uint32_t &budget, uint16_t *dst) {
    const int pairs = count >> 1;
    for (int j0 = t; j0 < pairs; j0 += B * nthreads) {
        uint64_t v[B];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int j = j0 + b * nthreads;
            v[b] = j < pairs ? load_pair(w + 2 * j) : 0;
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int j = j0 + b * nthreads;
            if (j >= pairs) continue;
            if (!pair_ready(v[b], epoch)) v[b] = poll_pair(w + 2 * j, epoch, err, budget);
            dst[2 * j] = (uint16_t)v[b];
            dst[2 * j + 1] = (uint16_t)(v[b] >> 32);
        }
    }
}

// g[p] = sum over the H row of gate row p times x, u[p] likewise for the up
// row: per lane over its chunks in order, then across the wave.  The 2P
// chains are independent and interleaved so that their latencies overlap.
template <int P, int NCH>
__device__ __forceinline__ void gate_up_dots(const uint4 (&gv)[P][NCH], const uint4 (&uv)[P][NCH],
                                             const uint4 (&xv)[NCH], int C, int lane, float (&g)[P], float (&u)[P]) {
#pragma unroll
    for (int p = 0; p < P; ++p) g[p] = u[p] = 0.0f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        if (lane + 64 * j < C) {
#pragma unroll
            for (int p = 0; p < P; ++p) {
                g[p] = dot8(gv[p][j], xv[j], g[p]);
                u[p] = dot8(uv[p][j], xv[j], u[p]);
            }
        }
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
        g[p] = wave_sum_dpp(g[p]);
        u[p] = wave_sum_dpp(u[p]);
    }
}

// x_eff = bf16(x + r) for the 8 bf16 pairs of two uint4 (fp32 sum, one
// round-to-nearest-even rounding by the hardware pair convert)
__device__ __forceinline__ uint4 add_bf16x8(uint4 a, uint4 r) {
    auto pair = [](uint32_t u, uint32_t v) { return f2bf2_hw(lo_bf(u) + lo_bf(v), hi_bf(u) + hi_bf(v)); };
    return make_uint4(pair(a.x, r.x), pair(a.y, r.y), pair(a.z, r.z), pair(a.w, r.w));
}

// NCH: 16-byte chunks per lane of an H row (>= H/8/64); P: gate/up row pairs
// per wave (>= k*I / waves); DC: 16-byte chunks per half-wave lane of a
// down row (>= I/8/32).  Larger values than needed are masked.
//
// Optional inputs (all may be null):
//   resid    the layer input is x_eff = bf16(x + resid) (a residual stream);
//            x_out receives x_eff (block 0) for the next layer's residual;
//   next_gate / pred_out  the gate-fallback predictor of the next layer:
//            top-k of next_gate . x_eff (no bias) into pred_out[k];
//   host_words  pinned host words for a host that waits on this launch:
//            [0, k) the routed ids, stored as soon as block 0 holds the final
//            routing (well before the launch ends), [k, 2k) the prediction,
//            each as (tag << 16) | id with a system-scope store, so a word is
//            valid once it carries the caller's tag; selected (int64 [k],
//            device) receives the routed ids at the same point.
template <int NCH, int P, int DC, bool CHAIN>
__global__ __launch_bounds__(256, 2) void decode_layer_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ resid, uint16_t *__restrict__ x_out,
    const uint16_t *__restrict__ gate, const float *__restrict__ bias, int H, int E, int k, int normalize,
    int merge_mode, const uint16_t *const *__restrict__ slots, int I, const uint16_t *__restrict__ next_gate,
    int32_t *__restrict__ pred_out, uint16_t *__restrict__ logits, int32_t *__restrict__ ids,
    uint16_t *__restrict__ weights, float *__restrict__ probs, uint16_t *__restrict__ h_ws,
    uint16_t *__restrict__ out, uint32_t *ws, int32_t *host_words, int64_t *__restrict__ selected, uint32_t tag) {
    extern __shared__ uint4 s_h[];       // k * I bf16
    __shared__ float s_logit[kDecodeMaxE];
    __shared__ float s_plogit[CHAIN ? kDecodeMaxE : 1];  // the next layer's predictor logits (last block)
    __shared__ uint32_t s_pub[16];
    __shared__ float s_y[kDecodeMaxK * 4];
    __shared__ const uint16_t *s_slot[kDecodeMaxE];
    __shared__ TopkScratch s_tk;
    __shared__ TopkScratch s_tk2;  // the exact routing when the logit-key one fails its check
    __shared__ int s_redo;
    __shared__ uint32_t s_epoch;

    const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
    const int C = H >> 3, CI = I >> 3;
    const int RB = (E + 3) / 4;
    uint32_t *err = ws + kWsError;
    uint32_t budget = kSpinBudget;

    // router rows first (blocks 0 .. RB-1): their latency starts the chain;
    // with a next gate, blocks RB .. 2RB-1 compute the next layer's
    // predictor logits
    const bool routes = (int)blockIdx.x < RB;
    const bool predicts = CHAIN && next_gate != nullptr && !routes && (int)blockIdx.x < 2 * RB;
    const int e_route = (routes ? (int)blockIdx.x : (int)blockIdx.x - RB) * 4 + wave;
    uint4 wv[NCH];
    if (routes || predicts) {
        const uint16_t *src = routes ? gate : next_gate;
        const uint4 *wrow = reinterpret_cast<const uint4 *>(src + (size_t)min(e_route, E - 1) * H);
#pragma unroll
        for (int j = 0; j < NCH; ++j) wv[j] = wrow[min(lane + 64 * j, C - 1)];
    }
    uint4 xv[NCH], rv[NCH];
#pragma unroll
    for (int j = 0; j < NCH; ++j) xv[j] = reinterpret_cast<const uint4 *>(x)[min(lane + 64 * j, C - 1)];
    const bool has_resid = CHAIN && resid != nullptr;
    if (has_resid) {
#pragma unroll
        for (int j = 0; j < NCH; ++j) rv[j] = reinterpret_cast<const uint4 *>(resid)[min(lane + 64 * j, C - 1)];
    }
    // then the small words: this block's epoch and the slot table (one wait
    // covers them and the rows above)
    if (tid == 0) {
        uint32_t ep = (__hip_atomic_load(ws + kWsEpoch + blockIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u) &
                      0xffffu;
        s_epoch = ep ? ep : 1u;
    }
    for (int e = tid; e < E; e += blockDim.x) s_slot[e] = slots[e];
    if (tid < 16) s_tk.seli[tid] = -1;  // no expert picked yet (see the rows below)
    __syncthreads();
    const uint32_t epoch = s_epoch;
    // the residual sum: now where the router dot needs it, else while the
    // gate/up rows stream
    const bool add_now = has_resid && (routes || predicts);
    if (add_now) {
#pragma unroll
        for (int j = 0; j < NCH; ++j) xv[j] = add_bf16x8(xv[j], rv[j]);
    }

    // ---- 1. router (or predictor) logits: block r computes experts
    // 4r..4r+3 and publishes them as one 16-byte write into a 128-byte line
    // of its own (one writer per line: partial writes of one line by many
    // agents serialise)
    if (routes || predicts) {
        const int e = e_route;
        uint32_t b = 0;
        if (e < E) {
            float a = 0.0f;
#pragma unroll
            for (int j = 0; j < NCH; ++j)
                if (lane + 64 * j < C) a = dot8(xv[j], wv[j], a);
            a = wave_sum_dpp(a);
            b = f2bf(a);
        }
        if (lane == 0) s_pub[wave] = (epoch << 16) | b;
        __syncthreads();
        if (tid == kPublisher) {
            uint64_t *line = reinterpret_cast<uint64_t *>(
                ws + (routes ? kWsLogit + blockIdx.x * 32 : kWsPLogit + (blockIdx.x - RB) * 32));
            __hip_atomic_store(line, (uint64_t)s_pub[0] | ((uint64_t)s_pub[1] << 32), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(line + 1, (uint64_t)s_pub[2] | ((uint64_t)s_pub[3] << 32), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }

    // Block b owns the 4P consecutive (gate, up) row pairs q = 4P*b + P*wave + p
    // of the k*I slot-major rows; slot s = q / I.
    const int KI = k * I;
    const int q0 = blockIdx.x * 4 * P + wave * P;

    // ---- 2. routing, computed by every block from the published logits
    // (one wave collects them: pair j holds experts 2j, 2j+1 and sits in the
    // line of route block j/2)
    if (wave == 0) {
        for (int j = lane; j < 2 * RB; j += 64) {
            const uint32_t *w = ws + kWsLogit + (j >> 1) * 32 + (j & 1) * 2;
            const uint64_t v = poll_pair(w, epoch, err, budget);
            if (2 * j < E) s_logit[2 * j] = bf2f((uint32_t)v & 0xffffu);
            if (2 * j + 1 < E) s_logit[2 * j + 1] = bf2f((uint32_t)(v >> 32) & 0xffffu);
        }
    }
    __syncthreads();
    // Without a logit bias the experts are picked first by their bf16 logits
    // (topk_by_logit_keys: the rows below start streaming ~0.5 us earlier),
    // and wave 0 checks the pick against the probabilities while its rows
    // stream; when the check fails (distinct logits with equal
    // probabilities), the exact routing is computed and the rows whose
    // expert it changes are computed again before h is published.
    const bool pub = blockIdx.x == 0;
    const bool by_keys = bias == nullptr;
    int rk[4];
    if (wave == 0) {
        if (by_keys) {
            if (E <= 128)
                topk_by_logit_keys<2>(s_logit, E, k, &s_tk, rk);
            else
                topk_by_logit_keys<4>(s_logit, E, k, &s_tk, rk);
        } else if (E <= 128) {
            topk_token<2>(s_logit, bias, E, k, normalize, 0, pub ? ids : nullptr, pub ? weights : nullptr,
                          pub ? probs : nullptr, &s_tk);
        } else {
            topk_token<4>(s_logit, bias, E, k, normalize, 0, pub ? ids : nullptr, pub ? weights : nullptr,
                          pub ? probs : nullptr, &s_tk);
        }
    }
    // with the logit-key pick each wave waits (below) only for the ranks of its
    // own rows, which wave 0 stores round by round: a block whose rows belong
    // to an early rank starts streaming before the pick is complete
    if (!by_keys) __syncthreads();

    // ---- 3. the gate/up rows this wave computes
    uint4 gv[P][NCH], uv[P][NCH];
    bool has[P];
    auto issue_rows = [&](TopkScratch &tk) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int q = min(q0 + p, KI - 1);
            const int sl = q / I, i = q - sl * I;
            int e = __hip_atomic_load(&tk.seli[sl], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
            // rank sl not picked yet (logit-key pick in progress): wave 0 stores
            // every rank after its bounded polls, so this ends; the wait still
            // spends the thread's poll budget, and an exhausted budget sets the
            // error word and reads expert 0 (in bounds)
            while (e < 0) {
                if (budget == 0) {
                    __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    e = 0;
                    break;
                }
                --budget;
                __builtin_amdgcn_s_sleep(1);
                e = __hip_atomic_load(&tk.seli[sl], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            const uint16_t *base = s_slot[e];
            // an expert without a ready copy reads the activation row instead
            // (H elements, in bounds) and contributes h = 0
            has[p] = base != nullptr;
            const uint16_t *grow = base ? base + (size_t)i * H : x;
            const uint16_t *urow = base ? base + (size_t)(I + i) * H : x;
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
                gv[p][j] = ld_nt(grow + 8 * min(lane + 64 * j, C - 1));
                uv[p][j] = ld_nt(urow + 8 * min(lane + 64 * j, C - 1));
            }
        }
    };
    // ---- 4. gate/up -> h
    // h = bf16(silu(bf16(g)) * bf16(u)), lane 0 for the wave's P rows.  (One
    // lane per row would publish earlier, but then the down rows below start
    // earlier too and slow the blocks whose gate/up rows are still streaming:
    // the last block's h, which every block waits for, comes later.)
    auto finish_rows = [&]() __attribute__((always_inline)) {
        float g[P], u[P];
        gate_up_dots<P, NCH>(gv, uv, xv, C, lane, g, u);
        if (lane == 0) {
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const float a = bf16_round(silu_f32(bf16_round(g[p])));
                const uint32_t hb = has[p] ? f2bf(a * bf16_round(u[p])) : 0u;
                s_pub[wave * P + p] = (epoch << 16) | hb;
            }
        }
    };
    issue_rows(s_tk);
    if (wave == 0) {
        bool exact = true;
        if (by_keys) {
            exact = E <= 128 ? topk_verify_finish<2>(s_logit, E, k, normalize, 0, pub ? ids : nullptr,
                                                     pub ? weights : nullptr, pub ? probs : nullptr, &s_tk, rk)
                             : topk_verify_finish<4>(s_logit, E, k, normalize, 0, pub ? ids : nullptr,
                                                     pub ? weights : nullptr, pub ? probs : nullptr, &s_tk, rk);
            if (!exact) {
                if (E <= 128)
                    topk_token<2>(s_logit, nullptr, E, k, normalize, 0, pub ? ids : nullptr, pub ? weights : nullptr,
                                  pub ? probs : nullptr, &s_tk2);
                else
                    topk_token<4>(s_logit, nullptr, E, k, normalize, 0, pub ? ids : nullptr, pub ? weights : nullptr,
                                  pub ? probs : nullptr, &s_tk2);
            }
        }
        if (lane == 0) s_redo = exact ? 0 : 1;
        // block 0 holds the final routing: hand it to a waiting host now
        if (pub && host_words && lane < k) {
            const int32_t e = exact ? s_tk.seli[lane] : s_tk2.seli[lane];
            if (selected) selected[lane] = (int64_t)e;
            __hip_atomic_store(host_words + lane, (int32_t)((tag << 16) | (uint32_t)e), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
    if (has_resid && !add_now) {
#pragma unroll
        for (int j = 0; j < NCH; ++j) xv[j] = add_bf16x8(xv[j], rv[j]);
    }
    finish_rows();
    __syncthreads();
    if (s_redo) {
        // the exact routing replaces the logit-key pick: rows of a changed
        // slot are loaded and computed again (block-uniform branch)
        bool changed = false;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int sl = min(q0 + p, KI - 1) / I;
            changed |= s_tk2.seli[sl] != s_tk.seli[sl];
        }
        if (changed) {
            issue_rows(s_tk2);
            finish_rows();
        }
        __syncthreads();
        if (tid < k) {
            s_tk.seli[tid] = s_tk2.seli[tid];
            s_tk.selp[tid] = s_tk2.selp[tid];
            s_tk.selw[tid] = s_tk2.selw[tid];
        }
        __syncthreads();
    }
    // the block's 4P words go out as 8-byte writes by the last wave's first
    // 2P threads
    if (tid >= kPublisher && tid < kPublisher + 2 * P) {
        const int t2 = tid - kPublisher;
        const int qb = blockIdx.x * 4 * P + 2 * t2;
        if (qb < KI) {
            __hip_atomic_store(reinterpret_cast<uint64_t *>(ws + kWsH + qb),
                               (uint64_t)s_pub[2 * t2] | ((uint64_t)s_pub[2 * t2 + 1] << 32), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }

    // down rows, issued once the block has published its h words (the
    // gate/up rows feed the h hand-off, the critical path; down rows issued
    // while other waves' or blocks' gate/up rows stream delay them; these
    // land during the hand-off): block b owns output columns 4b..4b+3;
    // half-wave (wave w, half h) owns slot s = 2w + h and reads that
    // expert's 4 rows, so a wave touches two experts' pages instead of k
    const int half = lane >> 5, hl = lane & 31;
    const int slot = 2 * wave + half;
    const size_t IH2 = 2 * (size_t)I * H;
    const uint16_t *dbase = slot < k ? s_slot[s_tk.seli[slot]] : nullptr;
    const bool dhas = dbase != nullptr;
    uint4 dv[4][DC];
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
        const int col = min((int)blockIdx.x * 4 + c4, H - 1);
        // no copy (or no expert): read the router rows instead (E*H >= I elements, in bounds)
        const uint16_t *row = dhas ? dbase + IH2 + (size_t)col * I : gate;
#pragma unroll
        for (int c = 0; c < DC; ++c) dv[c4][c] = ld_nt(row + 8 * min(hl + 32 * c, CI - 1));
    }

    // ---- 5. collect h (the other waves), then down + merge
    if (tid < kPublisher)
        collect<8>(ws + kWsH, KI, tid, kPublisher, epoch, err, budget, reinterpret_cast<uint16_t *>(s_h));
    // meanwhile the last block's publisher wave routes the next layer from
    // the predictor logits (published early in the launch) into pred_out
    if (CHAIN && next_gate && blockIdx.x == gridDim.x - 1 && tid >= kPublisher) {
        for (int j = lane; j < 2 * RB; j += 64) {
            const uint32_t *w = ws + kWsPLogit + (j >> 1) * 32 + (j & 1) * 2;
            const uint64_t v = poll_pair(w, epoch, err, budget);
            if (2 * j < E) s_plogit[2 * j] = bf2f((uint32_t)v & 0xffffu);
            if (2 * j + 1 < E) s_plogit[2 * j + 1] = bf2f((uint32_t)(v >> 32) & 0xffffu);
        }
        wave_lds_sync();
        if (E <= 128)
            topk_token<2>(s_plogit, nullptr, E, k, normalize, 0, pred_out, nullptr, nullptr, &s_tk2);
        else
            topk_token<4>(s_plogit, nullptr, E, k, normalize, 0, pred_out, nullptr, nullptr, &s_tk2);
        if (host_words && lane < k)
            __hip_atomic_store(host_words + k + lane, (int32_t)((tag << 16) | (uint32_t)s_tk2.seli[lane]),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    __syncthreads();
    // y[s][c] = bf16(h_s . down_s[col c]), each half-wave its own slot: the
    // slot's h chunks are read once, and the four column chains (each in
    // chunk order) are interleaved so their latencies overlap
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (slot < k) {
        uint4 hv[DC];
#pragma unroll
        for (int c = 0; c < DC; ++c) hv[c] = s_h[slot * CI + min(hl + 32 * c, CI - 1)];
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            if (hl + 32 * c < CI) {
#pragma unroll
                for (int c4 = 0; c4 < 4; ++c4) acc[c4] = dot8(dv[c4][c], hv[c], acc[c4]);
            }
        }
        if (!dhas) acc[0] = acc[1] = acc[2] = acc[3] = 0.0f;
    }
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
        acc[c4] = half_sum_dpp(acc[c4]);  // lanes 31 / 63 hold the sums of the two halves
        if (hl == 31 && slot < k) s_y[slot * 4 + c4] = bf16_round(acc[c4]);
    }
    __syncthreads();
    // merge, one lane per column
    if (tid < 4) {
        const int col = blockIdx.x * 4 + tid;
        float total = 0.0f;
        if (merge_mode) {
            int prev = -1;
            for (int n = 0; n < k; ++n) {  // the next larger expert id each round
                int best = 0x7fffffff, bs = 0;
                for (int s2 = 0; s2 < k; ++s2) {
                    const int e = s_tk.seli[s2];
                    if (e > prev && e < best) {
                        best = e;
                        bs = s2;
                    }
                }
                prev = best;
                total = bf16_round(total + bf16_round(bf2f(s_tk.selw[bs]) * s_y[bs * 4 + tid]));
            }
        } else {
            for (int s2 = 0; s2 < k; ++s2) total = __builtin_fmaf(bf2f(s_tk.selw[s2]), s_y[s2 * 4 + tid], total);
        }
        if (col < H) out[col] = (uint16_t)f2bf(total);
    }
    // outputs off the critical path: the logits (block 0, from the collected
    // words), this block's h values and the effective input
    if (blockIdx.x == 0) {
        for (int e = tid; e < E; e += blockDim.x) logits[e] = (uint16_t)(__float_as_uint(s_logit[e]) >> 16);
        if (CHAIN && x_out && wave == 0) {
#pragma unroll
            for (int j = 0; j < NCH; ++j)
                if (lane + 64 * j < C) reinterpret_cast<uint4 *>(x_out)[lane + 64 * j] = xv[j];
        }
    }
    if (tid < 4 * P) {
        const int q = blockIdx.x * 4 * P + tid;
        if (q < KI) h_ws[q] = (uint16_t)s_pub[tid];
    }
    // without a next gate, block 0 marks the predictor words invalid (epoch
    // 0 is never current), so that words left by an earlier predicting
    // launch cannot pass for a later one's when the 16-bit epoch wraps
    if (CHAIN && !next_gate && blockIdx.x == 0 && tid < 2 * RB)
        __hip_atomic_store(reinterpret_cast<uint64_t *>(ws + kWsPLogit + (tid >> 1) * 32 + (tid & 1) * 2), 0ull,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) __hip_atomic_store(ws + kWsEpoch + blockIdx.x, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

typedef void (*DecodeLayerFn)(const uint16_t *, const uint16_t *, uint16_t *, const uint16_t *, const float *, int,
                              int, int, int, int, const uint16_t *const *, int, const uint16_t *,
                              int32_t *, uint16_t *, int32_t *, uint16_t *, float *, uint16_t *, uint16_t *,
                              uint32_t *, int32_t *, int64_t *, uint32_t);

struct DecodePlan {
    DecodeLayerFn fn;        // plain launch
    DecodeLayerFn fn_chain;  // with the residual / next-layer predictor code
    int blocks;
    size_t lds;
};

// Instantiations (NCH, P, DC), chosen as the smallest that covers the shape
// with P * NCH <= 16 (register budget of two blocks per CU).
static int pick_decode(int H, int I, int k, DecodePlan *plan, std::string *why) {
    const int C = H / 8, CI = I / 8;
    const int blocks = (H + 3) / 4;
    const int waves = blocks * 4;
    const int nch_need = (C + 63) / 64, p_need = (k * I + waves - 1) / waves, dc_need = (CI + 31) / 32;
    const int nch = nch_need <= 2 ? 2 : nch_need <= 4 ? 4 : nch_need <= 8 ? 8 : 0;
    const int dc = dc_need <= 3 ? 3 : dc_need <= 6 ? 6 : 0;
    int p = p_need <= 2 ? 2 : p_need <= 3 ? 3 : p_need <= 4 ? 4 : 0;
    if (nch == 8 && p > 2) p = 0;
    if (!nch || !dc || !p || blocks > kDecodeMaxBlocks || k * I > kDecodeMaxKI) {
        *why = "decode_layer: shape outside the fused kernel (needs H <= 4096, I <= 1536, k*I <= 4*H)";
        return kEInval;
    }
    DecodeLayerFn fn = nullptr, fn_chain = nullptr;
#define PD_DL(N, PP, D)                                     \
    if (nch == N && p == PP && dc == D) {                   \
        fn = decode_layer_kernel<N, PP, D, false>;          \
        fn_chain = decode_layer_kernel<N, PP, D, true>;     \
    }
    PD_DL(2, 2, 3) PD_DL(2, 3, 3) PD_DL(2, 4, 3) PD_DL(2, 2, 6) PD_DL(2, 3, 6) PD_DL(2, 4, 6)
    PD_DL(4, 2, 3) PD_DL(4, 3, 3) PD_DL(4, 4, 3) PD_DL(4, 2, 6) PD_DL(4, 3, 6) PD_DL(4, 4, 6)
    PD_DL(8, 2, 3) PD_DL(8, 2, 6)
#undef PD_DL
    if (!fn) {
        *why = "decode_layer: no instantiation for this shape";
        return kEInval;
    }
    plan->fn = fn;
    plan->fn_chain = fn_chain;
    plan->blocks = blocks;
    plan->lds = (size_t)k * I * 2;
    return kOk;
}

// Blocks of `fn` that can be resident at once on the current device.
static int resident_blocks(DecodeLayerFn fn, size_t lds, std::string *why) {
    static std::mutex mu;
    static std::unordered_map<uint64_t, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        *why = "decode_layer: hipGetDevice failed";
        return -1;
    }
    const uint64_t key = ((uint64_t)(uintptr_t)fn * 31u + lds) * 64u + (uint64_t)dev;
    {
        std::lock_guard<std::mutex> lock(mu);
        auto it = cache.find(key);
        if (it != cache.end()) return it->second;
    }
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(fn), 256, lds) !=
            hipSuccess) {
        *why = "decode_layer: occupancy query failed";
        return -1;
    }
    const int n = cus * per_cu;
    std::lock_guard<std::mutex> lock(mu);
    cache[key] = n;
    return n;
}

}  // namespace pd

using namespace pd;

PD_API size_t pdscope_decode_workspace_bytes(void) { return (size_t)kWsWords * 4; }

PD_API int pdscope_decode_layer_supported(int H, int I, int E, int k) {
    if (H < 16 || H % 16 || I < 8 || I % 8 || E < 2 || E > kDecodeMaxE || E % 2 || k < 1 || k > kDecodeMaxK ||
        k > E)
        return 0;
    if ((size_t)I > (size_t)E * H || (E + 3) / 4 > (H + 3) / 4) return 0;
    DecodePlan plan;
    std::string why;
    if (pick_decode(H, I, k, &plan, &why) != kOk) return 0;
    const int n = resident_blocks(plan.fn, plan.lds, &why);
    return n >= plan.blocks ? 1 : 0;
}

PD_API int pdscope_decode_layer_chained_supported(int H, int I, int E, int k, int with_predictor) {
    if (!pdscope_decode_layer_supported(H, I, E, k)) return 0;
    if (with_predictor && 2 * ((E + 3) / 4) > (H + 3) / 4) return 0;
    DecodePlan plan;
    std::string why;
    if (pick_decode(H, I, k, &plan, &why) != kOk) return 0;
    // the chained variant has its own registers and static LDS
    const int n = resident_blocks(plan.fn_chain, plan.lds, &why);
    return n >= plan.blocks ? 1 : 0;
}

// Argument checks and plan shared by every entry point; the kernel variant
// (plain, or with the residual / next-layer predictor code) goes to *fn.
static int plan_decode_layer(const void *x, bool chain, const void *gate, int H, int E, int k, int merge_mode,
                             const void *const *slots, int I, const void *next_gate, const int32_t *pred_out,
                             const void *logits, const int32_t *ids, const void *weights, const void *h_ws,
                             const void *out, const void *workspace, DecodePlan *plan, DecodeLayerFn *fn) {
    if (!x || !gate || !slots || !logits || !ids || !weights || !h_ws || !out || !workspace)
        return fail(kEInval, "decode_layer: null pointer");
    if (H < 16 || H % 16) return fail(kEInval, "decode_layer: need H % 16 == 0");
    if (I < 8 || I % 8) return fail(kEInval, "decode_layer: need I % 8 == 0");
    if (E < 2 || E > kDecodeMaxE || E % 2) return fail(kEInval, "decode_layer: need even E <= 256");
    if (k < 1 || k > kDecodeMaxK || k > E) return fail(kEInval, "decode_layer: need 1 <= k <= min(E, 8)");
    if (merge_mode != 0 && merge_mode != 1) return fail(kEInval, "decode_layer: merge_mode must be 0 or 1");
    if ((size_t)I > (size_t)E * H) return fail(kEInval, "decode_layer: need I <= E*H");
    if ((size_t)k * I * 2 > 64 * 1024) return fail(kEInval, "decode_layer: k*I*2 must fit 64 KiB of LDS");
    if ((E + 3) / 4 > (H + 3) / 4) return fail(kEInval, "decode_layer: need E <= H");
    if (!next_gate != !pred_out) return fail(kEInval, "decode_layer: next_gate and pred_out go together");
    if (next_gate && 2 * ((E + 3) / 4) > (H + 3) / 4)
        return fail(kEInval, "decode_layer: the next-layer predictor needs E <= H/2");
    std::string why;
    if (pick_decode(H, I, k, plan, &why) != kOk) return fail(kEInval, why);
    *fn = chain ? plan->fn_chain : plan->fn;
    const int resident = resident_blocks(*fn, plan->lds, &why);
    if (resident < 0) return fail(kEHip, why);
    if (resident < plan->blocks)
        return fail(kEInval, "decode_layer: the grid would not be resident at once on this device");
    return kOk;
}

// Shared by both entry points: checks, plan, launch.
static int launch_decode_layer(const void *x, const void *resid, void *x_out, const void *gate, const float *bias,
                               int H, int E, int k, int normalize, int merge_mode, const void *const *slots, int I,
                               const void *next_gate, int32_t *pred_out, void *logits,
                               int32_t *ids, void *weights, float *probs, void *h_ws, void *out, void *workspace,
                               void *stream) {
    DecodePlan plan;
    DecodeLayerFn fn = nullptr;
    const int rc = plan_decode_layer(x, resid || next_gate, gate, H, E, k, merge_mode, slots, I, next_gate, pred_out,
                                     logits, ids, weights, h_ws, out, workspace, &plan, &fn);
    if (rc != kOk) return rc;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    fn<<<plan.blocks, 256, plan.lds, s>>>(
        (const uint16_t *)x, (const uint16_t *)resid, (uint16_t *)x_out, (const uint16_t *)gate, bias, H, E, k,
        normalize, merge_mode, (const uint16_t *const *)slots, I, (const uint16_t *)next_gate, pred_out,
        (uint16_t *)logits, ids, (uint16_t *)weights, probs, (uint16_t *)h_ws, (uint16_t *)out,
        (uint32_t *)workspace, nullptr, nullptr, 0u);
    return check_launch("decode_layer_kernel");
}

PD_API int pdscope_decode_layer(const void *x, const void *gate, const float *bias, int H, int E, int k,
                                int normalize, int merge_mode, const void *const *slots, int I, void *logits,
                                int32_t *ids, void *weights, float *probs, void *h_ws, void *out, void *workspace,
                                void *stream) {
    return launch_decode_layer(x, nullptr, nullptr, gate, bias, H, E, k, normalize, merge_mode, slots, I, nullptr,
                               nullptr, logits, ids, weights, probs, h_ws, out, workspace, stream);
}

PD_API int pdscope_decode_layer_chained(const void *x, const void *resid, void *x_out, const void *gate,
                                        const float *bias, int H, int E, int k, int normalize, int merge_mode,
                                        const void *const *slots, int I, const void *next_gate,
                                        int32_t *pred_out, void *logits, int32_t *ids,
                                        void *weights, float *probs, void *h_ws, void *out, void *workspace,
                                        void *stream) {
    if (!resid != !x_out) return fail(kEInval, "decode_layer_chained: resid and x_out go together");
    return launch_decode_layer(x, resid, x_out, gate, bias, H, E, k, normalize, merge_mode, slots, I, next_gate,
                               pred_out, logits, ids, weights, probs, h_ws, out, workspace, stream);
}

// ---------------------------------------------------------------- bound decode layer
//
// A resident decode layer whose gate, slot table, predictor gate and device
// buffers stay put from one token to the next is checked and planned once
// (pdscope_decode_bind); each token is then one call of pdscope_decode_run,
// numbered by the caller (seq, 1 .. 32767): the fused decode kernel, which
// stores the routed ids and the next-layer prediction into pinned host words
// as (seq << 16) | id as soon as it holds them, and the routed ids as int64
// into the caller's device tensor; then a one-wave kernel that stores the
// sticky error word as (seq << 16) | word.  Every word validates itself by
// its tag, so no fence orders them; the error word is stored after the layer
// kernel completed (stream order), so a host that reads seq in it knows the
// launch has completed.  A host may act on the routed ids before that, while
// the layer kernel still runs.  On this device a direct launch costs the
// host about 3 us against about 23 us for replaying a captured graph of the
// same kernel.

namespace pd {

__global__ __launch_bounds__(64) void decode_error_readback_kernel(const uint32_t *__restrict__ err,
                                                                   int32_t *host_err, uint32_t tag) {
    if (threadIdx.x == 0) {
        const uint32_t w = __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(host_err, (int32_t)((tag << 16) | (w & 0xffffu)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

}  // namespace pd

struct pdscope_decode_binding {
    DecodeLayerFn fn;
    int blocks;
    size_t lds;
    int device;
    const uint16_t *gate;
    const float *bias;
    int H, E, k, normalize, merge_mode, I;
    const uint16_t *const *slots;
    const uint16_t *next_gate;
    int32_t *pred_out;
    int32_t *ids;
    float *probs;
    uint16_t *h_ws;
    uint32_t *workspace;
    int32_t *host_ids;   // device addresses of the pinned read-back words
    int32_t *host_err;
};

// Device address of a word of pinned host memory (an error if it is not).
static int pinned_device_address(void *host, int32_t **dev, const char *what) {
    void *d = nullptr;
    if (hipHostGetDevicePointer(&d, host, 0) != hipSuccess || !d) {
        (void)hipGetLastError();
        return fail(kEInval, std::string("decode_bind: ") + what + " must be pinned host memory");
    }
    *dev = static_cast<int32_t *>(d);
    return kOk;
}

PD_API int pdscope_decode_bind(const void *gate, const float *bias, int H, int E, int k, int normalize,
                               int merge_mode, const void *const *slots, int I, const void *next_gate,
                               int32_t *pred_out, int32_t *ids, float *probs, void *h_ws, void *workspace,
                               int32_t *host_ids, int32_t *host_error, pdscope_decode_binding **binding) {
    if (!binding) return fail(kEInval, "decode_bind: null binding out-pointer");
    *binding = nullptr;
    if (!host_ids || !host_error) return fail(kEInval, "decode_bind: null read-back pointer");
    DecodePlan plan;
    DecodeLayerFn fn = nullptr;
    // x, logits, weights and out arrive with each run: stand-ins pass the null checks here
    const void *later = gate;
    int rc = plan_decode_layer(later, next_gate != nullptr, gate, H, E, k, merge_mode, slots, I, next_gate, pred_out,
                               later, ids, later, h_ws, later, workspace, &plan, &fn);
    if (rc != kOk) return rc;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(kEHip, "decode_bind: hipGetDevice failed");
    int32_t *dh = nullptr, *de = nullptr;
    if ((rc = pinned_device_address(host_ids, &dh, "host_ids")) != kOk) return rc;
    if ((rc = pinned_device_address(host_error, &de, "host_error")) != kOk) return rc;
    auto *b = new (std::nothrow) pdscope_decode_binding;
    if (!b) return fail(kEInval, "decode_bind: out of host memory");
    *b = pdscope_decode_binding{fn, plan.blocks, plan.lds, dev, (const uint16_t *)gate, bias, H, E, k, normalize,
                                merge_mode, I, (const uint16_t *const *)slots, (const uint16_t *)next_gate,
                                pred_out, ids, probs, (uint16_t *)h_ws, (uint32_t *)workspace, dh, de};
    *binding = b;
    return kOk;
}

PD_API int pdscope_decode_run(const pdscope_decode_binding *b, const void *x, void *out, void *logits,
                              void *weights, int64_t *selected, int32_t seq, void *stream) {
    if (!b) return fail(kEInval, "decode_run: null binding");
    if (!x || !out || !logits || !weights) return fail(kEInval, "decode_run: null pointer");
    if (seq < 1 || seq > 0x7fff) return fail(kEInval, "decode_run: seq must be in 1 .. 32767");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev != b->device)
        return fail(kEInval, "decode_run: the binding belongs to another device");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    b->fn<<<b->blocks, 256, b->lds, s>>>(
        (const uint16_t *)x, nullptr, nullptr, b->gate, b->bias, b->H, b->E, b->k, b->normalize, b->merge_mode,
        b->slots, b->I, b->next_gate, b->pred_out, (uint16_t *)logits, b->ids, (uint16_t *)weights, b->probs,
        b->h_ws, (uint16_t *)out, b->workspace, b->host_ids, selected, (uint32_t)seq);
    int rc = check_launch("decode_layer_kernel");
    if (rc != kOk) return rc;
    decode_error_readback_kernel<<<1, 64, 0, s>>>(b->workspace + kWsError, b->host_err, (uint32_t)seq);
    return check_launch("decode_error_readback_kernel");
}

PD_API void pdscope_decode_unbind(pdscope_decode_binding *b) { delete b; }
