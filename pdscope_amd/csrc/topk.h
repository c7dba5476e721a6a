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
