// K1: router logits + fp32 softmax + top-k (ties -> lower id) + renorm.
// Restates expertbench/adapters/qwen.py:140-152 (route) on gfx950, and the
// predictor histogram of expertbench/pdscope_runtime.py:245-249.
#include "common.h"

namespace pd {

// Softmax + top-k + renormalisation for one token, executed by one wave64.
// lrow: E logits of the token (bf16 values held as fp32, in LDS).
// Lane l owns experts l, l+64, ...; the softmax denominator is summed
// per lane in that order and then by an xor butterfly, an order that is
// fixed and reproduced by the host-side checker.
template <int J>
__device__ __forceinline__ void topk_token(const float *lrow, const float *__restrict__ bias, int E, int k,
                           int normalize, int t, int32_t *__restrict__ ids,
                           uint16_t *__restrict__ weights, float *__restrict__ probs) {
#pragma clang fp contract(off)
    const int lane = lane_id();
    float v[J], p[J];
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
    m = wave_max(m);
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
        int e = lane + 64 * j;
        if (probs && e < E) probs[(size_t)t * E + e] = p[j];
    }
    uint32_t taken = 0;
    float wsel[16];
    int isel[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        if (r < k) {
            uint64_t best = 0;
#pragma unroll
            for (int j = 0; j < J; ++j) {
                int e = lane + 64 * j;
                if (e < E && !((taken >> j) & 1u)) {
                    uint64_t key = ((uint64_t)__float_as_uint(p[j]) << 32) | (0xffffffffu - (uint32_t)e);
                    best = key > best ? key : best;
                }
            }
            best = wave_max_u64(best);
            int e = (int)(0xffffffffu - (uint32_t)best);
            if ((e & 63) == lane) taken |= 1u << (e >> 6);
            isel[r] = e;
            wsel[r] = __uint_as_float((uint32_t)(best >> 32));
        }
    }
    float denom = 0.0f;
    if (normalize) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (r < k) denom = denom + wsel[r];
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (r < k) {
                ids[(size_t)t * k + r] = isel[r];
                weights[(size_t)t * k + r] = (uint16_t)f2bf(normalize ? wsel[r] / denom : wsel[r]);
            }
    }
}

template <int J>
__device__ __forceinline__ void topk_tokens_block(const float *s_logit, int ntok, int E, const float *bias, int k,
                                  int normalize, int t0, int32_t *ids, uint16_t *weights,
                                  float *probs) {
    const int wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    for (int tt = wave; tt < ntok; tt += nwaves)
        topk_token<J>(s_logit + tt * E, bias, E, k, normalize, t0 + tt, ids, weights, probs);
}

__device__ __forceinline__ void topk_dispatch(const float *s_logit, int ntok, int E, const float *bias, int k,
                              int normalize, int t0, int32_t *ids, uint16_t *weights, float *probs) {
    if (E <= 64)
        topk_tokens_block<1>(s_logit, ntok, E, bias, k, normalize, t0, ids, weights, probs);
    else if (E <= 128)
        topk_tokens_block<2>(s_logit, ntok, E, bias, k, normalize, t0, ids, weights, probs);
    else
        topk_tokens_block<4>(s_logit, ntok, E, bias, k, normalize, t0, ids, weights, probs);
}

constexpr int kGemvMaxT = 8;

// Small-T path (decode): one wave per expert row; each wave streams its
// router row once and dots it with the <= 8 token rows.  The last block to
// finish (device-scope counter in the workspace, reset by that block) runs
// the softmax/top-k for every token.
__global__ __launch_bounds__(256) void route_gemv_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ gate, const float *__restrict__ bias,
    int T, int H, int E, int k, int normalize, uint16_t *__restrict__ logits,
    int32_t *__restrict__ ids, uint16_t *__restrict__ weights, float *__restrict__ probs,
    uint32_t *__restrict__ counter) {
    __shared__ float s_logit[kGemvMaxT * 256];
    __shared__ int s_last;
    const int lane = lane_id();
    const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int C = H >> 3;  // 16-byte chunks per row
    if (e < E) {
        const uint4 *wrow = reinterpret_cast<const uint4 *>(gate + (size_t)e * H);
        float acc[kGemvMaxT];
#pragma unroll
        for (int t = 0; t < kGemvMaxT; ++t) acc[t] = 0.0f;
        for (int c = lane; c < C; c += 64) {
            uint4 wv = wrow[c];
#pragma unroll
            for (int t = 0; t < kGemvMaxT; ++t)
                if (t < T) acc[t] = dot8(reinterpret_cast<const uint4 *>(x + (size_t)t * H)[c], wv, acc[t]);
        }
#pragma unroll
        for (int t = 0; t < kGemvMaxT; ++t) {
            if (t < T) {
                float s = wave_sum(acc[t]);
                if (lane == 0) logits[(size_t)t * E + e] = (uint16_t)f2bf(s);
            }
        }
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t prev = atomicAdd(counter, 1u);
        s_last = (prev == gridDim.x - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int i = threadIdx.x; i < T * E; i += blockDim.x) s_logit[i] = bf2f(logits[i]);
    __syncthreads();
    topk_dispatch(s_logit, T, E, bias, k, normalize, 0, ids, weights, probs);
    if (threadIdx.x == 0) atomicExch(counter, 0u);
}

// Prefill path: a block owns 32 tokens and all E experts.  Logits come from
// v_mfma_f32_32x32x16_bf16 (wave w computes expert blocks w, w+4, ...), are
// rounded to bf16, staged in LDS and routed in the same block.
__global__ __launch_bounds__(256) void route_mfma_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ gate, const float *__restrict__ bias,
    int T, int H, int E, int k, int normalize, uint16_t *__restrict__ logits,
    int32_t *__restrict__ ids, uint16_t *__restrict__ weights, float *__restrict__ probs) {
    __shared__ float s_logit[32 * 256];
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * 32;
    const int ntok = min(32, T - t0);
    const int trow = t0 + min(lane & 31, ntok - 1);
    const int kofs = (lane >> 5) * 8;
    const int NB = E >> 5;
    const uint16_t *xrow = x + (size_t)trow * H + kofs;
    for (int nb = wave; nb < NB; nb += 4) {
        const uint16_t *grow = gate + (size_t)(nb * 32 + (lane & 31)) * H + kofs;
        f32x16_t acc = {};
#pragma unroll 8
        for (int k0 = 0; k0 < H; k0 += 16) {
            bf16x8_t a = *reinterpret_cast<const bf16x8_t *>(xrow + k0);
            bf16x8_t b = *reinterpret_cast<const bf16x8_t *>(grow + k0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            int tt = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
            int e = nb * 32 + (lane & 31);
            uint32_t hb = f2bf(acc[r]);
            s_logit[tt * E + e] = bf2f(hb);
            if (tt < ntok) logits[(size_t)(t0 + tt) * E + e] = (uint16_t)hb;
        }
    }
    __syncthreads();
    topk_dispatch(s_logit, ntok, E, bias, k, normalize, t0, ids, weights, probs);
}

__global__ __launch_bounds__(1024) void route_hist_kernel(const int32_t *__restrict__ ids, int n, int E,
                                                          int32_t *__restrict__ hist) {
    __shared__ int32_t s_hist[1024];
    for (int e = threadIdx.x; e < E; e += blockDim.x) s_hist[e] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        int e = ids[i];
        if (e >= 0 && e < E) atomicAdd(&s_hist[e], 1);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) hist[e] = s_hist[e];
}

}  // namespace pd

using namespace pd;

PD_API size_t pdscope_route_workspace_bytes(void) { return 256; }

PD_API int pdscope_route_topk(const void *x, const void *gate, const float *bias, int T, int H, int E,
                              int k, int normalize, void *logits, int32_t *ids, void *weights,
                              float *probs, void *workspace, void *stream) {
    if (!x || !gate || !logits || !ids || !weights) return fail(kEInval, "route: null tensor pointer");
    if (T < 1 || H < 16 || H % 16) return fail(kEInval, "route: need T >= 1 and H % 16 == 0");
    if (E < 32 || E > 256 || E % 32) return fail(kEInval, "route: need E % 32 == 0 and E <= 256");
    if (k < 1 || k > 16 || k > E) return fail(kEInval, "route: need 1 <= k <= min(E, 16)");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (T <= kGemvMaxT) {
        if (!workspace) return fail(kEInval, "route: small-T path needs the zeroed workspace");
        route_gemv_kernel<<<(E + 3) / 4, 256, 0, s>>>(
            (const uint16_t *)x, (const uint16_t *)gate, bias, T, H, E, k, normalize,
            (uint16_t *)logits, ids, (uint16_t *)weights, probs, (uint32_t *)workspace);
        return check_launch("route_gemv_kernel");
    }
    route_mfma_kernel<<<(T + 31) / 32, 256, 0, s>>>((const uint16_t *)x, (const uint16_t *)gate, bias, T,
                                                    H, E, k, normalize, (uint16_t *)logits, ids,
                                                    (uint16_t *)weights, probs);
    return check_launch("route_mfma_kernel");
}

PD_API int pdscope_route_hist(const int32_t *ids, int n, int E, int32_t *hist, void *stream) {
    if (!ids || !hist || n < 0 || E < 1 || E > 1024) return fail(kEInval, "route_hist: bad arguments");
    route_hist_kernel<<<1, 1024, 0, reinterpret_cast<hipStream_t>(stream)>>>(ids, n, E, hist);
    return check_launch("route_hist_kernel");
}
