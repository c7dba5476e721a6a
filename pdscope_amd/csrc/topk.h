// Softmax + top-k + renormalisation of one token's router logits by one
// wave64 (the selection of expertbench/adapters/qwen.py:148-151).
#pragma once

#include "common.h"

namespace pd {

// Per-wave LDS scratch of the top-k selection.  After topk_token returns,
// seli[0..k) holds the selected experts in rank order, selp[0..k) their
// probabilities and selw[0..k) their final bf16 weights.
struct TopkScratch {
    float selp[16];
    int seli[16];
    uint16_t selw[16];
};

// Make this wave's LDS writes visible to its other lanes before they read.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Wave-wide max through DPP (no LDS round trips): row_shr 1/2/4/8 leave
// each row's max in its lane 15, row_bcast 15/31 carry it to lane 63, which
// is read back as a uniform value.  Lanes without a DPP source read the
// identity of max (INT_MIN), so each step is one v_max_i32 with a DPP operand.
__device__ __forceinline__ int dpp_max_i32(int v) {
    constexpr int kId = (int)0x80000000;
    v = max(v, __builtin_amdgcn_update_dpp(kId, v, 0x111, 0xf, 0xf, false));  // row_shr:1
    v = max(v, __builtin_amdgcn_update_dpp(kId, v, 0x112, 0xf, 0xf, false));  // row_shr:2
    v = max(v, __builtin_amdgcn_update_dpp(kId, v, 0x114, 0xf, 0xf, false));  // row_shr:4
    v = max(v, __builtin_amdgcn_update_dpp(kId, v, 0x118, 0xf, 0xf, false));  // row_shr:8
    v = max(v, __builtin_amdgcn_update_dpp(kId, v, 0x142, 0xa, 0xf, false));  // row_bcast:15
    v = max(v, __builtin_amdgcn_update_dpp(kId, v, 0x143, 0xc, 0xf, false));  // row_bcast:31
    return __builtin_amdgcn_readlane(v, 63);
}

// Wave-wide max of fp32 values that are not NaN, through dpp_max_i32 on an
// order-preserving integer image of the bits (negative values have their
// magnitude bits flipped).  Among equal maxima +0 beats -0.
__device__ __forceinline__ float dpp_max_f32(float f) {
    const int b = __float_as_int(f);
    const int m = dpp_max_i32(b ^ ((b >> 31) & 0x7fffffff));
    return __int_as_float(m ^ ((m >> 31) & 0x7fffffff));
}

// Softmax of one token's logits by one wave.  lrow: E logits of the token
// (bf16 values held as fp32, in LDS).  Lane l owns experts l, l+64, ...;
// the softmax denominator is summed per lane in that order and then by an
// xor butterfly over offsets 32..1, an order that is fixed and reproduced by
// the host-side oracle.  p[j] is the probability of expert lane + 64 j (0
// where that is >= E); probs row t is written when non-null.
template <int J>
__device__ __forceinline__ void softmax_wave(const float *lrow, const float *__restrict__ bias, int E, int t,
                                             float *__restrict__ probs, float (&p)[J]) {
#pragma clang fp contract(off)
    const int lane = lane_id();
    float v[J];
    float m = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < J; ++j) {
        int e = lane + 64 * j;
        float val = -__builtin_inff();
        if (e < E) {
            val = lrow[e];
            if (bias) val = val + bias[e];
        }
        v[j] = val;
        m = fmaxf(m, val);
    }
    m = dpp_max_f32(m);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        int e = lane + 64 * j;
        float ex = 0.0f;
        if (e < E) {
            ex = route_expf(v[j] - m);
            acc = acc + ex;
        }
        p[j] = ex;
    }
    const float S = wave_sum(acc);
#pragma unroll
    for (int j = 0; j < J; ++j) {
        p[j] = p[j] / S;
        const int e = lane + 64 * j;
        if (e < E && probs) probs[(size_t)t * E + e] = p[j];
    }
}

// Softmax + selection of one token by one wave.  Selection: k rounds of a
// wave-wide max over the probabilities' bit patterns (p >= 0, so integer
// order is float order; taken candidates drop to -1); among equal maxima the
// lowest expert id wins (ballot, first set lane of the lowest j).  This is
// the total order "higher probability first, lower expert id on ties", so
// the k rounds give the sorted top-k.  ids / weights / probs (global, row t)
// are written when non-null.
template <int J>
__device__ __forceinline__ void topk_token(const float *lrow, const float *__restrict__ bias, int E, int k,
                                           int normalize, int t, int32_t *__restrict__ ids,
                                           uint16_t *__restrict__ weights, float *__restrict__ probs,
                                           TopkScratch *sc) {
#pragma clang fp contract(off)
    const int lane = lane_id();
    float p[J];
    softmax_wave<J>(lrow, bias, E, t, probs, p);
    int hi[J];
#pragma unroll
    for (int j = 0; j < J; ++j) hi[j] = lane + 64 * j < E ? (int)__float_as_uint(p[j]) : -1;
    float myp = 0.0f, denom = 0.0f;
    int myid = 0;
    for (int r = 0; r < k; ++r) {
        int lm = hi[0];
#pragma unroll
        for (int j = 1; j < J; ++j) lm = max(lm, hi[j]);
        const int mx = dpp_max_i32(lm);
        int sel = -1;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const unsigned long long b = __ballot(hi[j] == mx);
            if (sel < 0 && b) sel = 64 * j + __ffsll(b) - 1;
        }
#pragma unroll
        for (int j = 0; j < J; ++j)
            if (lane + 64 * j == sel) hi[j] = -1;
        const float pv = __int_as_float(mx);
        if (normalize) denom = denom + pv;
        if (lane == r) {
            myp = pv;
            myid = sel;
        }
    }
    if (lane < k) {
        const uint16_t wb = (uint16_t)f2bf(normalize ? myp / denom : myp);
        sc->selp[lane] = myp;
        sc->seli[lane] = myid;
        sc->selw[lane] = wb;
        if (ids) ids[(size_t)t * k + lane] = myid;
        if (weights) weights[(size_t)t * k + lane] = wb;
    }
    wave_lds_sync();
}

// Order-preserving key of a bf16 logit (held as fp32) and its expert id:
// larger logit first, equal logits lower id first; keys of distinct experts
// differ.  The bf16 bits map to an unsigned order (sign set: complement;
// else set the sign), the id fills the low half as 0xffff - e, and the top
// bit flips so signed integer order is that unsigned order.
__device__ __forceinline__ int logit_key(float v, int e) {
    const uint32_t b = __float_as_uint(v) >> 16;
    const uint32_t o = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
    return (int)(((o << 16) | (0xffffu - (uint32_t)e)) ^ 0x80000000u);
}

// First half of the two-step routing of one token by one wave (no logit
// bias): the k experts of largest bf16 logit (equal logits: lower id) in
// that order, by k rounds of a wave-wide max over unique keys (no ballot
// per round), into sc->seli.  Each round's expert is stored at once with
// workgroup-scope release, so other waves of the block may wait for just the
// ranks they need (sc->seli[r] < 0 until then, when the caller cleared it).
// rank[j] receives the rank of expert lane + 64 j, -1 if not taken.  The softmax is increasing in the logit, so
// this is the probability top-k except where distinct logits give equal
// probabilities; topk_verify_finish detects exactly those cases.
template <int J>
__device__ __forceinline__ void topk_by_logit_keys(const float *lrow, int E, int k, TopkScratch *sc,
                                                   int (&rank)[4]) {
    const int lane = lane_id();
    int key[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int e = lane + 64 * j;
        key[j] = e < E ? logit_key(lrow[e], e) : (int)0x80000000;
        rank[j] = -1;
    }
    for (int r = 0; r < k; ++r) {
        int lm = key[0];
#pragma unroll
        for (int j = 1; j < J; ++j) lm = max(lm, key[j]);
        const int sel = 0xffff - (dpp_max_i32(lm) & 0xffff);
#pragma unroll
        for (int j = 0; j < J; ++j)
            if (lane + 64 * j == sel) {
                key[j] = (int)0x80000000;
                rank[j] = r;
            }
        if (lane == 0) __hip_atomic_store(&sc->seli[r], sel, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    wave_lds_sync();
}

// Second half: the softmax (probs row t written when non-null), then a check
// that sc->seli is the top-k of topk_token -- ranks descending in
// (probability, -id), and the last one above every expert not taken in that
// order.  If so, the probabilities and weights go to sc->selp / selw (and
// ids / weights row t when non-null) with topk_token's arithmetic (the
// renormalising sum in rank order) and it returns true; else it writes
// nothing more and returns false, and the caller runs topk_token.
template <int J>
__device__ __forceinline__ bool topk_verify_finish(const float *lrow, int E, int k, int normalize, int t,
                                                   int32_t *__restrict__ ids, uint16_t *__restrict__ weights,
                                                   float *__restrict__ probs, TopkScratch *sc,
                                                   const int (&rank)[4]) {
#pragma clang fp contract(off)
    const int lane = lane_id();
    float p[J];
    softmax_wave<J>(lrow, nullptr, E, t, probs, p);
#pragma unroll
    for (int j = 0; j < J; ++j)
        if (rank[j] >= 0) sc->selp[rank[j]] = p[j];
    wave_lds_sync();
    bool bad = false;
    if (lane + 1 < k) {
        const float a = sc->selp[lane], b = sc->selp[lane + 1];
        bad = !(a > b || (a == b && sc->seli[lane] < sc->seli[lane + 1]));
    }
    // the largest probability not taken (bit patterns: p >= 0), -1 if none
    int um = -1;
#pragma unroll
    for (int j = 0; j < J; ++j)
        if (lane + 64 * j < E && rank[j] < 0) um = max(um, (int)__float_as_uint(p[j]));
    const int M = dpp_max_i32(um);
    const int last = (int)__float_as_uint(sc->selp[k - 1]);
    if (last < M) {
        bad = true;
    } else if (last == M) {
        // the lowest expert id not taken with that probability must come after
        int emin = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const unsigned long long bm =
                __ballot(lane + 64 * j < E && rank[j] < 0 && (int)__float_as_uint(p[j]) == M);
            if (bm && emin == 0x7fffffff) emin = 64 * j + __ffsll(bm) - 1;
        }
        if (sc->seli[k - 1] > emin) bad = true;
    }
    if (__ballot(bad)) return false;
    float denom = 0.0f;
    if (normalize)
        for (int r = 0; r < k; ++r) denom = denom + sc->selp[r];
    if (lane < k) {
        const float myp = sc->selp[lane];
        const uint16_t wb = (uint16_t)f2bf(normalize ? myp / denom : myp);
        sc->selw[lane] = wb;
        if (ids) ids[(size_t)t * k + lane] = sc->seli[lane];
        if (weights) weights[(size_t)t * k + lane] = wb;
    }
    wave_lds_sync();
    return true;
}

// Block-level wrapper for one token: wave 0 routes, the block waits.  Must
// be reached by the whole block; sc is then valid for every thread.
template <int J>
__device__ __forceinline__ void topk_block(const float *lrow, const float *__restrict__ bias, int E, int k,
                                           int normalize, int32_t *__restrict__ ids, uint16_t *__restrict__ weights,
                                           float *__restrict__ probs, TopkScratch *sc) {
    if (threadIdx.x < 64) topk_token<J>(lrow, bias, E, k, normalize, 0, ids, weights, probs, sc);
    __syncthreads();
}

}  // namespace pd
