// K1: router logits + fp32 softmax + top-k (ties -> lower id) + renorm.
// Restates expertbench/adapters/qwen.py:140-152 (route) on gfx950, and the
// predictor histogram of expertbench/pdscope_runtime.py:245-249.
#include "common.h"
#include "topk.h"

namespace pd {

template <int J>
__device__ __forceinline__ void topk_tokens_block(const float *s_logit, int ntok, int E, const float *bias, int k,
                                                  int normalize, int t0, int32_t *ids, uint16_t *weights,
                                                  float *probs, TopkScratch *s_tk) {
    const int wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    for (int tt = wave; tt < ntok; tt += nwaves)
        topk_token<J>(s_logit + tt * E, bias, E, k, normalize, t0 + tt, ids, weights, probs, s_tk + wave);
}

__device__ __forceinline__ void topk_dispatch(const float *s_logit, int ntok, int E, const float *bias, int k,
                                              int normalize, int t0, int32_t *ids, uint16_t *weights, float *probs,
                                              TopkScratch *s_tk) {
    if (E <= 64)
        topk_tokens_block<1>(s_logit, ntok, E, bias, k, normalize, t0, ids, weights, probs, s_tk);
    else if (E <= 128)
        topk_tokens_block<2>(s_logit, ntok, E, bias, k, normalize, t0, ids, weights, probs, s_tk);
    else
        topk_tokens_block<4>(s_logit, ntok, E, bias, k, normalize, t0, ids, weights, probs, s_tk);
}

constexpr int kGemvMaxT = 8;

// Small-T path (decode): one wave per expert row; each wave streams its
// router row once and dots it with the <= 8 token rows.  The last block to
// finish (device-scope counter in the workspace, reset by that block) runs
// the softmax/top-k for every token.
template <int NCH>
__global__ __launch_bounds__(256) void route_gemv_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ gate, const float *__restrict__ bias,
    int T, int H, int E, int k, int normalize, uint16_t *__restrict__ logits,
    int32_t *__restrict__ ids, uint16_t *__restrict__ weights, float *__restrict__ probs,
    uint32_t *__restrict__ counter) {
    __shared__ float s_logit[kGemvMaxT * 256];
    __shared__ TopkScratch s_tk[4];
    __shared__ int s_last;
    const int lane = lane_id();
    const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int C = H >> 3;  // 16-byte chunks per row; lane owns chunks lane + 64*j
    if (e < E) {
        const uint4 *wrow = reinterpret_cast<const uint4 *>(gate + (size_t)e * H);
        uint4 wv[NCH];
#pragma unroll
        for (int j = 0; j < NCH; ++j) wv[j] = wrow[min(lane + 64 * j, C - 1)];
        for (int t = 0; t < T; ++t) {
            const uint4 *xrow = reinterpret_cast<const uint4 *>(x + (size_t)t * H);
            uint4 xv[NCH];
#pragma unroll
            for (int j = 0; j < NCH; ++j) xv[j] = xrow[min(lane + 64 * j, C - 1)];
            float a = 0.0f;
#pragma unroll
            for (int j = 0; j < NCH; ++j)
                if (lane + 64 * j < C) a = dot8(xv[j], wv[j], a);
            a = wave_sum(a);
            if (lane == 0) logits[(size_t)t * E + e] = (uint16_t)f2bf(a);
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
    topk_dispatch(s_logit, T, E, bias, k, normalize, 0, ids, weights, probs, s_tk);
    if (threadIdx.x == 0) atomicExch(counter, 0u);
}

// Prefill path: a block owns 32 tokens and all E = 32*NB experts.  The four
// waves split H into quarters; each wave runs NB independent
// v_mfma_f32_32x32x16_bf16 accumulator chains over its quarter with the next
// step's operands prefetched into registers.  The four partial sums are
// added in LDS in wave order (a fixed order, so logits are deterministic),
// rounded to bf16 and routed in the same block.
template <int NB>
__global__ __launch_bounds__(256) void route_mfma_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ gate, const float *__restrict__ bias,
    int T, int H, int k, int normalize, uint16_t *__restrict__ logits, int32_t *__restrict__ ids,
    uint16_t *__restrict__ weights, float *__restrict__ probs) {
    constexpr int E = NB * 32;
    extern __shared__ float s_part[];  // [32][E]: summed partials, then bf16-rounded logits
    __shared__ TopkScratch s_tk[4];
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * 32;
    const int ntok = min(32, T - t0);
    const int trow = t0 + min(lane & 31, ntok - 1);
    const int kq = H >> 2;
    const int kbase = wave * kq + (lane >> 5) * 8;
    const uint16_t *xrow = x + (size_t)trow * H + kbase;
    const uint16_t *grow = gate + (size_t)(lane & 31) * H + kbase;
    const size_t gstride = (size_t)32 * H;

    f32x16_t acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x16_t{};
    bf16x8_t a_cur = *reinterpret_cast<const bf16x8_t *>(xrow);
    bf16x8_t b_cur[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) b_cur[nb] = *reinterpret_cast<const bf16x8_t *>(grow + nb * gstride);
    for (int k0 = 16; k0 <= kq; k0 += 16) {
        bf16x8_t a_nxt = a_cur, b_nxt[NB];
        const bool more = k0 < kq;
        if (more) a_nxt = *reinterpret_cast<const bf16x8_t *>(xrow + k0);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            b_nxt[nb] = b_cur[nb];
            if (more) b_nxt[nb] = *reinterpret_cast<const bf16x8_t *>(grow + nb * gstride + k0);
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_cur, b_cur[nb], acc[nb], 0, 0, 0);
        a_cur = a_nxt;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) b_cur[nb] = b_nxt[nb];
    }
    // fixed-order reduction ((p0 + p1) + p2) + p3: the waves add their
    // partials into one LDS tile in turn
#pragma unroll 1
    for (int w = 0; w < 4; ++w) {
        if (wave == w) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int tt = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                    float *dst = s_part + tt * E + nb * 32 + (lane & 31);
                    *dst = (w == 0) ? acc[nb][r] : *dst + acc[nb][r];
                }
        }
        __syncthreads();
    }
    for (int i = threadIdx.x; i < 32 * E; i += 256) {
        const uint32_t hb = f2bf(s_part[i]);
        s_part[i] = bf2f(hb);
        const int tt = i / E;
        if (tt < ntok) logits[(size_t)(t0 + tt) * E + (i - tt * E)] = (uint16_t)hb;
    }
    __syncthreads();
    topk_tokens_block<(NB * 32 + 63) / 64>(s_part, ntok, E, bias, k, normalize, t0, ids,
                                                                 weights, probs, s_tk);
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
        const int nch = (H / 8 + 63) / 64;
        switch (nch) {
#define PD_RG(N)                                                                                           \
    case N:                                                                                                \
        route_gemv_kernel<N><<<(E + 3) / 4, 256, 0, s>>>((const uint16_t *)x, (const uint16_t *)gate, bias, T, H, E, k, \
                                                         normalize, (uint16_t *)logits, ids, (uint16_t *)weights,  \
                                                         probs, (uint32_t *)workspace);                    \
        break;
            PD_RG(1) PD_RG(2) PD_RG(3) PD_RG(4) PD_RG(5) PD_RG(6) PD_RG(7) PD_RG(8)
#undef PD_RG
        default:
            return fail(kEInval, "route: small-T path needs H <= 4096");
        }
        return check_launch("route_gemv_kernel");
    }
    if (H % 64) return fail(kEInval, "route: prefill path needs H % 64 == 0");
    const size_t lds = (size_t)32 * E * sizeof(float);
    const int blocks = (T + 31) / 32;
    switch (E / 32) {
#define PD_RT(NB)                                                                                          \
    case NB:                                                                                               \
        route_mfma_kernel<NB><<<blocks, 256, lds, s>>>((const uint16_t *)x, (const uint16_t *)gate, bias, T, H, k, \
                                                      normalize, (uint16_t *)logits, ids, (uint16_t *)weights,     \
                                                      probs);                                              \
        break;
        PD_RT(1) PD_RT(2) PD_RT(3) PD_RT(4) PD_RT(5) PD_RT(6) PD_RT(7) PD_RT(8)
#undef PD_RT
    default:
        return fail(kEInval, "route: unsupported E");
    }
    return check_launch("route_mfma_kernel");
}

PD_API int pdscope_route_hist(const int32_t *ids, int n, int E, int32_t *hist, void *stream) {
    if (!ids || !hist || n < 0 || E < 1 || E > 1024) return fail(kEInval, "route_hist: bad arguments");
    route_hist_kernel<<<1, 1024, 0, reinterpret_cast<hipStream_t>(stream)>>>(ids, n, E, hist);
    return check_launch("route_hist_kernel");
}
