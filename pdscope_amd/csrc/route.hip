// K1: router logits + fp32 softmax + top-k (ties -> lower id) + renorm.
// Restates expertbench/adapters/qwen.py:140-152 (route) on gfx950, and the
// predictor histogram of expertbench/pdscope_runtime.py:245-249.
// T <= 8: one GEMV launch whose last block routes every token.  T > 8:
// split-K MFMA partial logits, then one wave per token sums them in a fixed
// order and routes.
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
            a = wave_sum_dpp(a);
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

// Prefill path, two launches.
// route_partial_kernel: split-K logits.  Block (token tile of 32, K chunk ks)
// has E/32 waves; wave w computes the 32 x 32 tile of tokens x experts
// [32w, 32w + 32) over its K chunk of 16*STEPS elements with
// v_mfma_f32_32x32x16_bf16, all operand loads issued up front (one memory
// latency per block), and stores the fp32 partial to part[ks][t][e].
template <int STEPS>
__global__ __launch_bounds__(512) void route_partial_kernel(const uint16_t *__restrict__ x,
                                                            const uint16_t *__restrict__ gate, int T, int H, int E,
                                                            float *__restrict__ part) {
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * 32, ks = blockIdx.y;
    const int k0 = ks * STEPS * 16 + (lane >> 5) * 8;
    const int trow = min(t0 + (lane & 31), T - 1);
    const int e = wave * 32 + (lane & 31);
    const uint16_t *xa = x + (size_t)trow * H + k0;
    const uint16_t *gb = gate + (size_t)e * H + k0;
    bf16x8_t a[STEPS], b[STEPS];
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
        a[st] = *reinterpret_cast<const bf16x8_t *>(xa + 16 * st);
        b[st] = *reinterpret_cast<const bf16x8_t *>(gb + 16 * st);
    }
    f32x16_t acc = f32x16_t{};
#pragma unroll
    for (int st = 0; st < STEPS; ++st) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[st], b[st], acc, 0, 0, 0);
    // lane holds expert column e, token rows (r/4)*8 + (lane/32)*4 + r%4
    float *dst = part + (size_t)ks * T * E + e;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int t = t0 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (t < T) dst[(size_t)t * E] = acc[r];
    }
}

// route_partial_lds_kernel: the same partials for large T with less
// traffic.  Block (128 tokens, K chunk ks) stages the 256-element chunk of
// every router row in LDS once, by direct-to-LDS loads (lane l of a load
// fills bytes 16 l of a 1 KB piece), and its 4 waves each take 32 tokens
// against all E experts.  The chunk is read once per 128 tokens instead of
// once per 32, and the token rows once per block instead of once per wave.
// LDS row r (512 bytes) holds its logical 16-byte chunk c in slot
// c ^ (r % 16), so the 16 rows of a fragment read hit 16 distinct bank
// groups.  Each partial is the same MFMA chain as in route_partial_kernel.
__global__ __launch_bounds__(256) void route_partial_lds_kernel(const uint16_t *__restrict__ x,
                                                                const uint16_t *__restrict__ gate, int T, int H,
                                                                int E, float *__restrict__ part) {
    constexpr int STEPS = 16, KC = 16 * STEPS;  // K elements per chunk
    constexpr int ROWB = KC * 2;                // 512 bytes per router row
    __shared__ __attribute__((aligned(1024))) uint8_t s_gate[256 * ROWB];  // E <= 256 rows
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    const int ks = blockIdx.y;
    const int t0 = blockIdx.x * 128 + wave * 32;
    const int kbase = ks * KC;
    // the router chunk: E/2 pieces of 1 KB (two rows each), E/8 per wave;
    // lane l writes slot l % 32 of row 2 p + l / 32, i.e. logical chunk
    // (l % 32) ^ (row % 16)
    for (int pc = wave; pc < E / 2; pc += 4) {
        const int row = 2 * pc + (lane >> 5);
        const int c = (lane & 31) ^ (row & 15);
        const uint16_t *src = gate + (size_t)row * H + kbase + c * 8;
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(uintptr_t)src,
                                         (__attribute__((address_space(3))) void *)(uint32_t)(uintptr_t)(
                                             s_gate + pc * 1024),
                                         16, 0, 0);
    }
    // this wave's token rows
    const int trow = min(t0 + (lane & 31), T - 1);
    const uint16_t *xa = x + (size_t)trow * H + kbase + (lane >> 5) * 8;
    bf16x8_t a[STEPS];
#pragma unroll
    for (int st = 0; st < STEPS; ++st) a[st] = *reinterpret_cast<const bf16x8_t *>(xa + 16 * st);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's chunk pieces and token rows have landed
    __syncthreads();
    const int ET = E / 32;
    f32x16_t acc[8];
#pragma unroll
    for (int et = 0; et < 8; ++et) acc[et] = f32x16_t{};
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
        const int c = st * 2 + (lane >> 5);
#pragma unroll
        for (int et = 0; et < 8; ++et) {
            if (et < ET) {
                const int row = et * 32 + (lane & 31);
                const bf16x8_t b =
                    *reinterpret_cast<const bf16x8_t *>(s_gate + row * ROWB + ((c ^ (row & 15)) << 4));
                acc[et] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[st], b, acc[et], 0, 0, 0);
            }
        }
    }
    // lane holds expert column et*32 + (lane & 31), token rows (r/4)*8 + (lane/32)*4 + r%4
    float *dst = part + (size_t)ks * T * E;
#pragma unroll
    for (int et = 0; et < 8; ++et) {
        if (et >= ET) continue;
        const int e = et * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = t0 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
            if (t < T) dst[(size_t)t * E + e] = acc[et][r];
        }
    }
}

// route_finish_kernel: one wave per token sums the KS partials in chunk
// order, rounds to the bf16 logit and runs the softmax / top-k / renorm.
// The partials are loaded eight chunks at a time before they are added (one
// memory latency per eight chunks, not per chunk).
template <int J>
__global__ __launch_bounds__(256) void route_finish_kernel(const float *__restrict__ part, int KS, int T, int E,
                                                           const float *__restrict__ bias, int k, int normalize,
                                                           uint16_t *__restrict__ logits, int32_t *__restrict__ ids,
                                                           uint16_t *__restrict__ weights, float *__restrict__ probs) {
    __shared__ float s_logit[4][64 * J];
    __shared__ TopkScratch s_tk[4];
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wave;
    if (t >= T) return;
    float v[J];
#pragma unroll
    for (int j = 0; j < J; ++j) v[j] = 0.0f;
    for (int ks0 = 0; ks0 < KS; ks0 += 8) {
        float pv[8][J];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float *row = part + ((size_t)(ks0 + u) * T + t) * E;
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int e = lane + 64 * j;
                pv[u][j] = (ks0 + u < KS && e < E) ? row[e] : 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
#pragma unroll
            for (int j = 0; j < J; ++j)
                if (ks0 + u < KS && lane + 64 * j < E) v[j] = v[j] + pv[u][j];
        }
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int e = lane + 64 * j;
        if (e < E) {
            const uint32_t hb = f2bf(v[j]);
            logits[(size_t)t * E + e] = (uint16_t)hb;
            s_logit[wave][e] = bf2f(hb);
        }
    }
    wave_lds_sync();
    topk_token<J>(s_logit[wave], bias, E, k, normalize, t, ids, weights, probs, &s_tk[wave]);
}

// Token count from which the partial logits use the LDS-staged kernel.
constexpr int kRouteStagedMinT = 2048;

// K chunk of the split-K router: 256 elements (16 MFMA steps) when H allows.
static int route_kchunk(int H) {
    for (int kc = 256; kc >= 16; kc >>= 1)
        if (H % kc == 0) return kc;
    return 0;
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

// Bytes of workspace pdscope_route_topk needs for T tokens: the zeroed
// 256-byte counter of the small-T path, then (T > 8) the split-K partial
// logits (fp32, H / kchunk x T x E).
PD_API size_t pdscope_route_workspace_size(int T, int H, int E) {
    if (T <= kGemvMaxT) return 256;
    const int kc = route_kchunk(H);
    if (kc == 0 || E < 1) return 256;
    return 256 + (size_t)(H / kc) * (size_t)T * (size_t)E * sizeof(float);
}

PD_API int pdscope_route_topk(const void *x, const void *gate, const float *bias, int T, int H, int E,
                              int k, int normalize, void *logits, int32_t *ids, void *weights,
                              float *probs, void *workspace, void *stream) {
    if (!x || !gate || !logits || !ids || !weights) return fail(kEInval, "route: null tensor pointer");
    if (T < 1 || H < 16 || H % 16) return fail(kEInval, "route: need T >= 1 and H % 16 == 0");
    if (E < 32 || E > 256 || E % 32) return fail(kEInval, "route: need E % 32 == 0 and E <= 256");
    if (k < 1 || k > 16 || k > E) return fail(kEInval, "route: need 1 <= k <= min(E, 16)");
    if (!workspace) return fail(kEInval, "route: workspace (pdscope_route_workspace_size bytes) is required");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (T <= kGemvMaxT) {
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
    const int kc = route_kchunk(H);
    const int KS = H / kc;
    float *part = reinterpret_cast<float *>(static_cast<char *>(workspace) + 256);
    const dim3 g1((T + 31) / 32, KS);
    const int threads = (E / 32) * 64;
    // large T: 128 tokens per block over an LDS-staged router chunk
    // (needs the 256-element chunk)
    const bool staged = T >= kRouteStagedMinT && kc == 256;
    if (staged) {
        const dim3 gs((T + 127) / 128, KS);
        route_partial_lds_kernel<<<gs, 256, 0, s>>>((const uint16_t *)x, (const uint16_t *)gate, T, H, E, part);
    } else {
    switch (kc / 16) {
#define PD_RP(ST)                                                                                           \
    case ST:                                                                                                \
        route_partial_kernel<ST><<<g1, threads, 0, s>>>((const uint16_t *)x, (const uint16_t *)gate, T, H, E, part); \
        break;
        PD_RP(1) PD_RP(2) PD_RP(4) PD_RP(8) PD_RP(16)
#undef PD_RP
    default:
        return fail(kEInval, "route: unsupported K chunk");
    }
    }
    int rc = check_launch(staged ? "route_partial_lds_kernel" : "route_partial_kernel");
    if (rc) return rc;
    const int g2 = (T + 3) / 4;
    if (E <= 64)
        route_finish_kernel<1><<<g2, 256, 0, s>>>(part, KS, T, E, bias, k, normalize, (uint16_t *)logits, ids,
                                                 (uint16_t *)weights, probs);
    else if (E <= 128)
        route_finish_kernel<2><<<g2, 256, 0, s>>>(part, KS, T, E, bias, k, normalize, (uint16_t *)logits, ids,
                                                 (uint16_t *)weights, probs);
    else
        route_finish_kernel<4><<<g2, 256, 0, s>>>(part, KS, T, E, bias, k, normalize, (uint16_t *)logits, ids,
                                                 (uint16_t *)weights, probs);
    return check_launch("route_finish_kernel");
}

PD_API int pdscope_route_hist(const int32_t *ids, int n, int E, int32_t *hist, void *stream) {
    if (!ids || !hist || n < 0 || E < 1 || E > 1024) return fail(kEInval, "route_hist: bad arguments");
    route_hist_kernel<<<1, 1024, 0, reinterpret_cast<hipStream_t>(stream)>>>(ids, n, E, hist);
    return check_launch("route_hist_kernel");
}
