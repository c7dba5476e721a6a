// K3: grouped SwiGLU expert FFN for prefill on bf16 MFMA (gfx950).
// Restates expert_forward (expertbench/adapters/qwen.py:87-90) for every
// selected expert at once, replacing the per-expert launches of
// ExpertExecutor.gpu (expertbench/executor.py:454-488).
//
// Two launches per call:
//   gate/up : h[r,i] = bf16(bf16(silu(bf16(x_r.gate_i))) * bf16(x_r.up_i))
//             the A rows are gathered through perm_token, the B tile holds
//             BN/2 gate rows and the matching BN/2 up rows, so the SwiGLU
//             epilogue pairs accumulators of the same lane;
//   down    : y[r,n] = bf16(h_r . down_n)
// Both operands are K-contiguous ([rows, K] activations, [out, in] weights),
// so every 16-byte global load feeds one MFMA lane directly.  Tiles go
// through double-buffered LDS with a 16-byte-chunk XOR swizzle
// (chunk c of row r lives at c ^ (r & 7)) so the 32 lanes reading one
// column of chunks hit distinct banks.  MFMA: v_mfma_f32_32x32x16_bf16.
#include "common.h"

namespace pd {

constexpr int kBK = 64;  // K elements per LDS stage (8 chunks of 16 B)

__device__ __forceinline__ int swz(int row, int chunk) { return row * kBK + ((chunk ^ (row & 7)) << 3); }

template <int BM, int BN, int WM, int WN, bool GATEUP>
__global__ __launch_bounds__(256, 2) void grouped_kernel(
    const uint16_t *__restrict__ a_src, const int32_t *__restrict__ perm_token,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ sel, int nsel,
    const int32_t *__restrict__ tile_start, const uint16_t *const *__restrict__ slots, int H, int I,
    uint16_t *__restrict__ out) {
    static_assert(WM * WN == 4, "4 waves");
    constexpr int TM = BM / WM, TN = BN / WN;  // wave tile
    constexpr int MB = TM / 32, NB = TN / 32;  // 32x32 MFMA blocks per wave
    static_assert(MB >= 1 && NB >= 1 && (!GATEUP || NB % 2 == 0), "wave tiling");
    constexpr int A_PER = BM * 8 / 256, B_PER = BN * 8 / 256;  // 16-byte chunks per thread per stage
    static_assert(A_PER >= 1 && B_PER >= 1, "tile too small");

    __shared__ __attribute__((aligned(16))) uint16_t s_a[2][BM * kBK];
    __shared__ __attribute__((aligned(16))) uint16_t s_b[2][BN * kBK];

    // ---- XCD-aware tile order: blocks are dispatched round-robin over the 8
    // XCDs (block b -> XCD b % 8).  m-tile mt is pinned to XCD mt % 8 and its
    // n-tiles are consecutive blocks of that XCD, so the gathered activation
    // rows of an m-tile are fetched into one L2 and reused by every n-tile.
    const int ntn = GATEUP ? I / (BN / 2) : H / BN;
    const int xcd = blockIdx.x & 7, pos = blockIdx.x >> 3;
    const int jm = pos / ntn, nt = pos - jm * ntn;
    const int bx = jm * 8 + xcd;
    if (bx >= tile_start[nsel]) return;
    // ---- locate (expert, m-tile): binary search over the tile prefix
    int lo = 0, hi = nsel - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (tile_start[mid] <= bx) lo = mid;
        else hi = mid - 1;
    }
    const int e = sel[lo];
    const int row_end = offsets[e + 1];
    const int m0 = offsets[e] + (bx - tile_start[lo]) * BM;
    const int K = GATEUP ? H : I;
    const int n0 = nt * (GATEUP ? BN / 2 : BN);  // first intermediate (gate/up) or output column
    const uint16_t *base = slots[e];
    if (base == nullptr) return;  // no ready copy of this expert: never dereference
    const size_t IH = (size_t)I * H;

    // ---- per-thread global row pointers (fixed over the K loop)
    const int tid = threadIdx.x;
    const uint16_t *a_ptr[A_PER];
    const uint16_t *b_ptr[B_PER];
#pragma unroll
    for (int q = 0; q < A_PER; ++q) {
        const int id = q * 256 + tid, r = id >> 3, c = id & 7;
        const int row = min(m0 + r, row_end - 1);
        if (GATEUP) a_ptr[q] = a_src + (size_t)perm_token[row] * H + c * 8;
        else a_ptr[q] = a_src + (size_t)row * I + c * 8;
    }
#pragma unroll
    for (int q = 0; q < B_PER; ++q) {
        const int id = q * 256 + tid, r = id >> 3, c = id & 7;
        if (GATEUP) {
            const int i = n0 + (r < BN / 2 ? r : r - BN / 2);
            b_ptr[q] = base + (r < BN / 2 ? 0 : IH) + (size_t)i * H + c * 8;
        } else {
            b_ptr[q] = base + 2 * IH + (size_t)(n0 + r) * I + c * 8;
        }
    }

    u32x4_t ra[A_PER], rb[B_PER];
#define PD_GLOAD(k0)                                                                            \
    do {                                                                                        \
        _Pragma("unroll") for (int q = 0; q < A_PER; ++q) ra[q] = *gptr(a_ptr[q] + (k0));      \
        _Pragma("unroll") for (int q = 0; q < B_PER; ++q) rb[q] = *gptr(b_ptr[q] + (k0));      \
    } while (0)
#define PD_LSTORE(buf)                                                                          \
    do {                                                                                        \
        _Pragma("unroll") for (int q = 0; q < A_PER; ++q) {                                    \
            const int id_ = q * 256 + tid;                                                      \
            *reinterpret_cast<u32x4_t *>(&s_a[buf][swz(id_ >> 3, id_ & 7)]) = ra[q];          \
        }                                                                                       \
        _Pragma("unroll") for (int q = 0; q < B_PER; ++q) {                                    \
            const int id_ = q * 256 + tid;                                                      \
            *reinterpret_cast<u32x4_t *>(&s_b[buf][swz(id_ >> 3, id_ & 7)]) = rb[q];          \
        }                                                                                       \
    } while (0)

    const int lane = lane_id(), wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int lrow = lane & 31, lhalf = lane >> 5;

    f32x16_t acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = f32x16_t{};

    // B-tile row of the wave's n-block nb (gate/up pairs share a lane layout)
#define PD_BROW(nb)                                                                              \
    (GATEUP ? ((nb) < NB / 2 ? wn * (TN / 2) + (nb) * 32 : BN / 2 + wn * (TN / 2) + ((nb) - NB / 2) * 32) \
            : wn * TN + (nb) * 32)

    const int KT = K / kBK;
    PD_GLOAD(0);
    PD_LSTORE(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < KT) PD_GLOAD((kt + 1) * kBK);
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            const int chunk = kk * 2 + lhalf;
            bf16x8_t af[MB], bfr[NB];
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const int row = wm * TM + i * 32 + lrow;
                af[i] = *reinterpret_cast<const bf16x8_t *>(&s_a[buf][swz(row, chunk)]);
            }
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int row = PD_BROW(j) + lrow;
                bfr[j] = *reinterpret_cast<const bf16x8_t *>(&s_b[buf][swz(row, chunk)]);
            }
#pragma unroll
            for (int i = 0; i < MB; ++i)
#pragma unroll
                for (int j = 0; j < NB; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < KT) PD_LSTORE(buf ^ 1);
        __syncthreads();
    }

#undef PD_GLOAD
#undef PD_LSTORE
#undef PD_BROW
    // ---- epilogue: lane holds column (lane & 31), rows (r/4)*8 + (lane/32)*4 + r%4
#pragma unroll
    for (int i = 0; i < MB; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + wm * TM + i * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
            if (row >= row_end) continue;
            if (GATEUP) {
#pragma unroll
                for (int j = 0; j < NB / 2; ++j) {
                    const int col = n0 + wn * (TN / 2) + j * 32 + lrow;
                    const float g = bf16_round(acc[i][j][r]);
                    const float u = bf16_round(acc[i][j + NB / 2][r]);
                    const float a = bf16_round(silu_f32(g));
                    out[(size_t)row * I + col] = (uint16_t)f2bf(a * u);
                }
            } else {
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const int col = n0 + wn * TN + j * 32 + lrow;
                    out[(size_t)row * H + col] = (uint16_t)f2bf(acc[i][j][r]);
                }
            }
        }
    }
}

// phase: 1 = gate/up only, 2 = down only, 3 = both
template <int BM, int BN, int WM, int WN>
int launch_grouped(int phase, const uint16_t *x, const int32_t *perm_token, const int32_t *offsets,
                   const int32_t *sel, int nsel, const int32_t *tile_start, int max_tiles,
                   const uint16_t *const *slots, int H, int I, uint16_t *h_ws, uint16_t *y, hipStream_t s) {
    if (I % (BN / 2) || H % BN) return fail(kEInval, "grouped: I must divide by BN/2 and H by BN");
    if (phase & 1) {
        const unsigned g1 = (unsigned)((max_tiles + 7) / 8 * 8) * (unsigned)(I / (BN / 2));
        grouped_kernel<BM, BN, WM, WN, true><<<g1, 256, 0, s>>>(x, perm_token, offsets, sel, nsel, tile_start,
                                                                 slots, H, I, h_ws);
        int rc = check_launch("grouped_kernel<gateup>");
        if (rc) return rc;
    }
    if (phase & 2) {
        const unsigned g2 = (unsigned)((max_tiles + 7) / 8 * 8) * (unsigned)(H / BN);
        grouped_kernel<BM, BN, WM, WN, false><<<g2, 256, 0, s>>>(h_ws, nullptr, offsets, sel, nsel, tile_start,
                                                                  slots, H, I, y);
        return check_launch("grouped_kernel<down>");
    }
    return kOk;
}

int grouped_entry(int phase, const void *x, const int32_t *perm_token, const int32_t *offsets, const int32_t *sel,
                  int nsel, const int32_t *tile_start, int max_tiles, int block_m, const void *const *slots, int H,
                  int I, void *h_ws, void *y, void *stream) {
    if (((phase & 1) && (!x || !perm_token)) || !offsets || !sel || !tile_start || !slots || !h_ws ||
        ((phase & 2) && !y))
        return fail(kEInval, "grouped: null pointer");
    if (nsel < 1 || max_tiles < 1) return fail(kEInval, "grouped: need nsel >= 1 and max_tiles >= 1");
    if (H % 64 || I % 64 || H < 64 || I < 64) return fail(kEInval, "grouped: need H % 64 == 0 and I % 64 == 0");
    if (max_tiles > (1 << 22)) return fail(kEInval, "grouped: max_tiles too large");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const uint16_t *xp = (const uint16_t *)x;
    const uint16_t *const *sp = (const uint16_t *const *)slots;
    switch (block_m) {
    case 32:
        return launch_grouped<32, 256, 1, 4>(phase, xp, perm_token, offsets, sel, nsel, tile_start, max_tiles, sp, H,
                                             I, (uint16_t *)h_ws, (uint16_t *)y, s);
    case 64:
        return launch_grouped<64, 128, 2, 2>(phase, xp, perm_token, offsets, sel, nsel, tile_start, max_tiles, sp, H,
                                             I, (uint16_t *)h_ws, (uint16_t *)y, s);
    case 128:
        return launch_grouped<128, 128, 2, 2>(phase, xp, perm_token, offsets, sel, nsel, tile_start, max_tiles, sp,
                                              H, I, (uint16_t *)h_ws, (uint16_t *)y, s);
    default:
        return fail(kEInval, "grouped: block_m must be 32, 64 or 128");
    }
}

}  // namespace pd

using namespace pd;

// Weights are re-read once per m-tile of an expert, so the row tile should
// cover a typical expert in one tile; 32 only for very thin experts.
PD_API int pdscope_grouped_block_m(int rows_hint) {
    if (rows_hint <= 16) return 32;
    if (rows_hint <= 80) return 64;
    return 128;
}

PD_API int pdscope_swiglu_grouped(const void *x, const int32_t *perm_token, const int32_t *offsets,
                                  const int32_t *sel, int nsel, const int32_t *tile_start, int max_tiles,
                                  int block_m, const void *const *slots, int H, int I, void *h_ws, void *y,
                                  void *stream) {
    return grouped_entry(3, x, perm_token, offsets, sel, nsel, tile_start, max_tiles, block_m, slots, H, I, h_ws, y,
                         stream);
}

PD_API int pdscope_swiglu_grouped_gateup(const void *x, const int32_t *perm_token, const int32_t *offsets,
                                         const int32_t *sel, int nsel, const int32_t *tile_start, int max_tiles,
                                         int block_m, const void *const *slots, int H, int I, void *h_ws,
                                         void *stream) {
    return grouped_entry(1, x, perm_token, offsets, sel, nsel, tile_start, max_tiles, block_m, slots, H, I, h_ws,
                         nullptr, stream);
}

PD_API int pdscope_swiglu_grouped_down(const void *h_ws, const int32_t *offsets, const int32_t *sel, int nsel,
                                       const int32_t *tile_start, int max_tiles, int block_m,
                                       const void *const *slots, int H, int I, void *y, void *stream) {
    return grouped_entry(2, nullptr, nullptr, offsets, sel, nsel, tile_start, max_tiles, block_m, slots, H, I,
                         const_cast<void *>(h_ws), y, stream);
}
