// K4: T == 1 decode expert FFN as a coalesced streaming GEMV, with the
// weighted merge fused into the down projection.
// Restates, for one token and its k routed experts, expert_forward
// (expertbench/adapters/qwen.py:87-90) as submitted per expert by the decode
// loop (expertbench/pdscope_runtime.py:326-350) and the merge
// (pdscope_runtime.py:450-469).
//
// Launch 1 (gate/up): one wave per two (expert, intermediate) items; every
//   lane streams 16-byte chunks of the gate and up rows (4 KiB rows at
//   H = 2048 are 4 chunks per lane), so each wave keeps 16 loads in flight.
//   h[s,i] = bf16(bf16(silu(bf16(g))) * bf16(u))  ->  h_ws [k, I]
// Launch 2 (down + merge): each 32-lane half-wave owns one expert row of
//   down_s (I bf16); a wave walks the k experts in pairs for its output
//   column j, rounds each expert's y to bf16 (the expert output dtype) and
//   accumulates w_s * y_s in fp32 in slot order (merge_mode 0:
//   out[j] = bf16(sum_s w_s * y_s[j]), one rounding), or keeps the y_s and
//   adds them in ascending expert id in bf16 arithmetic (merge_mode 1, the
//   reference's merge, expertbench/pdscope_runtime.py:466-468:
//   acc = bf16(acc + bf16(w_s * y_s[j]))).  h (k*I bf16) is staged in LDS
//   once per block.
#include "common.h"

namespace pd {

template <int NJ>
__global__ __launch_bounds__(256) void decode_gateup_kernel(const uint16_t *__restrict__ x,
                                                            const int32_t *__restrict__ ids,
                                                            const uint16_t *const *__restrict__ slots, int H,
                                                            int I, int k, uint16_t *__restrict__ h_ws) {
    const int lane = lane_id();
    const int q0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 2;
    const int items = k * I;
    if (q0 >= items) return;
    // lane owns 16-byte chunks lane + 64*j (j < NJ) of each H-row; when H is
    // not a multiple of 512 the tail chunks are clamped and masked out
    const int C = H >> 3;
    uint4 xv[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) xv[j] = reinterpret_cast<const uint4 *>(x)[min(lane + 64 * j, C - 1)];
    uint4 gv[2][NJ], uv[2][NJ];
    bool ok[2];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int q = min(q0 + it, items - 1);
        const int s = q / I, i = q - s * I;
        const uint16_t *base = slots[ids[s]];
        // an expert without a ready copy reads the activation row instead
        // (H elements, in bounds) and contributes h = 0
        ok[it] = base != nullptr;
        const uint4 *grow = ok[it] ? reinterpret_cast<const uint4 *>(base + (size_t)i * H)
                                   : reinterpret_cast<const uint4 *>(x);
        const uint4 *urow = ok[it] ? reinterpret_cast<const uint4 *>(base + (size_t)(I + i) * H)
                                   : reinterpret_cast<const uint4 *>(x);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            gv[it][j] = ld_nt(grow + min(lane + 64 * j, C - 1));
            uv[it][j] = ld_nt(urow + min(lane + 64 * j, C - 1));
        }
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            if (lane + 64 * j < C) {
                g = dot8(gv[it][j], xv[j], g);
                u = dot8(uv[it][j], xv[j], u);
            }
        }
        g = wave_sum_dpp(g);
        u = wave_sum_dpp(u);
        const int q = q0 + it;
        if (lane == 0 && q < items) {
            const float a = bf16_round(silu_f32(bf16_round(g)));
            h_ws[q] = ok[it] ? (uint16_t)f2bf(a * bf16_round(u)) : (uint16_t)0;
        }
    }
}

// CPL = 16-byte chunks per lane per expert row (ceil(I / 8 / 32))
template <int CPL>
__global__ __launch_bounds__(256) void decode_down_kernel(const uint16_t *__restrict__ h_ws,
                                                          const int32_t *__restrict__ ids,
                                                          const uint16_t *__restrict__ w,
                                                          const uint16_t *const *__restrict__ slots, int H,
                                                          int I, int k, int merge_mode,
                                                          uint16_t *__restrict__ out) {
    extern __shared__ uint4 s_h[];
    __shared__ float s_ys[4][16];  // per wave: bf16 y of each slot (merge_mode 1)
    const int CI = I >> 3;
    for (int idx = threadIdx.x; idx < k * CI; idx += blockDim.x)
        s_h[idx] = reinterpret_cast<const uint4 *>(h_ws)[idx];
    __syncthreads();
    const int lane = lane_id(), half = lane >> 5, hl = lane & 31;
    const int j = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (j >= H) return;
    const size_t IH2 = 2 * (size_t)I * H;
    float total = 0.0f;
    for (int p = 0; p < k; p += 2) {
        const int s = p + half;
        float acc = 0.0f;
        if (s < k) {
            const uint16_t *base = slots[ids[s]];
            // no ready copy: read h itself (k*I elements, in bounds) and add 0
            const uint4 *row = base ? reinterpret_cast<const uint4 *>(base + IH2 + (size_t)j * I)
                                    : reinterpret_cast<const uint4 *>(h_ws);
            uint4 wv[CPL];
#pragma unroll
            for (int c = 0; c < CPL; ++c) wv[c] = ld_nt(row + min(hl + 32 * c, CI - 1));
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int ch = hl + 32 * c;
                if (ch < CI) acc = dot8(wv[c], s_h[s * CI + ch], acc);
            }
            if (!base) acc = 0.0f;
        }
        acc = half_sum_dpp(acc);  // lanes 31 / 63 hold the sums of the two halves
        const float even = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 31));
        const float odd = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 63));
        if (lane == 0) {
            total = __builtin_fmaf(bf2f(w[p]), bf16_round(even), total);
            if (p + 1 < k) total = __builtin_fmaf(bf2f(w[p + 1]), bf16_round(odd), total);
            s_ys[threadIdx.x >> 6][p] = bf16_round(even);
            if (p + 1 < k) s_ys[threadIdx.x >> 6][p + 1] = bf16_round(odd);
        }
    }
    if (lane == 0 && merge_mode) {
        const float *ys = s_ys[threadIdx.x >> 6];
        total = 0.0f;
        int prev = -1;
        for (int n = 0; n < k; ++n) {  // the next larger expert id each round
            int best = 0x7fffffff, bs = 0;
            for (int s = 0; s < k; ++s) {
                const int e = ids[s];
                if (e > prev && e < best) {
                    best = e;
                    bs = s;
                }
            }
            prev = best;
            total = bf16_round(total + bf16_round(bf2f(w[bs]) * ys[bs]));
        }
    }
    if (lane == 0) out[j] = (uint16_t)f2bf(total);
}

}  // namespace pd

using namespace pd;

PD_API int pdscope_swiglu_decode(const void *x, const int32_t *ids, const void *w, int k,
                                 const void *const *slots, int H, int I, void *h_ws, void *out,
                                 int merge_mode, void *stream) {
    if (!x || !ids || !w || !slots || !h_ws || !out) return fail(kEInval, "decode: null pointer");
    if (merge_mode != 0 && merge_mode != 1) return fail(kEInval, "decode: merge_mode must be 0 or 1");
    if (k < 1 || k > 16) return fail(kEInval, "decode: need 1 <= k <= 16");
    if (H < 8 || H % 8 || H > 4096) return fail(kEInval, "decode: need H % 8 == 0 and H <= 4096");
    if (I < 8 || I % 8 || I > 8192) return fail(kEInval, "decode: need I % 8 == 0 and I <= 8192");
    if ((size_t)k * I * 2 > 64 * 1024) return fail(kEInval, "decode: k*I*2 must fit 64 KiB of LDS");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const uint16_t *xp = (const uint16_t *)x;
    const uint16_t *const *sp = (const uint16_t *const *)slots;
    const int waves = (k * I + 1) / 2;
    const int blocks = (waves + 3) / 4;
    switch ((H / 8 + 63) / 64) {
#define PD_GU(NJ)                                                                                          \
    case NJ:                                                                                               \
        decode_gateup_kernel<NJ><<<blocks, 256, 0, s>>>(xp, ids, sp, H, I, k, (uint16_t *)h_ws);           \
        break;
        PD_GU(1) PD_GU(2) PD_GU(3) PD_GU(4) PD_GU(5) PD_GU(6) PD_GU(7) PD_GU(8)
#undef PD_GU
    default:
        return fail(kEInval, "decode: unsupported H");
    }
    int rc = check_launch("decode_gateup_kernel");
    if (rc) return rc;
    const int cpl = ((I >> 3) + 31) / 32;
    const size_t lds = (size_t)k * I * 2;
    const int dblocks = (H + 3) / 4;
    switch (cpl) {
#define PD_DN(C)                                                                                           \
    case C:                                                                                                \
        decode_down_kernel<C><<<dblocks, 256, lds, s>>>((const uint16_t *)h_ws, ids, (const uint16_t *)w, sp, H, \
                                                        I, k, merge_mode, (uint16_t *)out);                \
        break;
        PD_DN(1) PD_DN(2) PD_DN(3) PD_DN(4) PD_DN(5) PD_DN(6) PD_DN(7) PD_DN(8)
#undef PD_DN
    default:
        if (cpl <= 32) {
            decode_down_kernel<32><<<dblocks, 256, lds, s>>>((const uint16_t *)h_ws, ids, (const uint16_t *)w, sp,
                                                             H, I, k, merge_mode, (uint16_t *)out);
        } else {
            return fail(kEInval, "decode: unsupported I");
        }
    }
    return check_launch("decode_down_kernel");
}
