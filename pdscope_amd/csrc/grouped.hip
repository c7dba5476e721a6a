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
// so every 16-byte chunk feeds one MFMA lane directly.  Tiles stream into
// multi-stage LDS rings by direct-to-LDS loads (global_load_lds_dwordx4)
// with a 16-byte-chunk XOR swizzle applied on the source side (see Geo),
// so fragment reads are bank-conflict free.
// MFMA: v_mfma_f32_32x32x16_bf16, fp32 accumulation.
#include <type_traits>

#include "common.h"

namespace pd {

// LDS tile geometry for a K step of BK bf16 elements: a tile row is BK * 2
// bytes (CPR chunks of 16 B); one wave-wide direct-to-LDS load fills 1 KB,
// i.e. RPI consecutive rows.  With 64 banks of 4 bytes, a 16-byte fragment
// read serves 16 lanes (16 consecutive rows, one logical chunk) per cycle;
// rows share a 256-byte bank line in groups of RPL, so chunk c of row r is
// stored in slot c ^ ((r / RPL) % CPR) and the 16 rows of a fragment read
// land in 16 distinct 16-byte bank groups (conflict free).
template <int BK>
struct Geo {
    static constexpr int RB = BK * 2;
    static constexpr int CPR = BK / 8;
    static constexpr int RPI = 1024 / RB;
    static constexpr int RPL = 256 / RB;
    static __device__ __forceinline__ int key(int r) { return (r / RPL) % CPR; }
    static __device__ __forceinline__ int off(int r, int c) { return r * RB + ((c ^ key(r)) << 4); }
};

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void g_void_t;

// One wave-wide direct-to-LDS load: lane l's 16 bytes at src land at
// dst + 16 l (dst is wave-uniform), bypassing the registers.  AUX is the
// cache-policy field: kDeviceScope (sc1) makes the load device-coherent, so
// it is served by the L2 without allocating in the CU's vector L1.  Weight
// tiles are read once per CU and use it (measured: about 10% faster grouped
// launches at T=4096 than with L1 allocation, while nt, the streaming hint,
// was slower); activation tiles keep the default.
constexpr int kDeviceScope = 16;
template <int AUX = 0>
__device__ __forceinline__ void load_lds16(const uint16_t *src, uint8_t *dst) {
    __builtin_amdgcn_global_load_lds((g_void_t *)(uintptr_t)src, (lds_void_t *)(uint32_t)(uintptr_t)dst, 16, 0, AUX);
}

// Hides a per-lane load offset from loop-invariant code motion, so each
// 64-bit address (uniform base + offset) is formed next to its load instead
// of being hoisted out of the K loop as a live register pair per load.
__device__ __forceinline__ void opaque(uint32_t &v) { asm volatile("" : "+v"(v)); }

// Wait until at most n vector-memory operations of this wave are in flight
// (n is a compile-time constant in every use).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// wait_vm<n> for a wave-uniform n in [0, 24] known only at run time
__device__ __forceinline__ void wait_vm_rt(int n) {
#define PD_W(K) else if (n == K) wait_vm<K>();
    if (n <= 0) wait_vm<0>();
    PD_W(1) PD_W(2) PD_W(3) PD_W(4) PD_W(5) PD_W(6) PD_W(7) PD_W(8) PD_W(9) PD_W(10) PD_W(11) PD_W(12)
    PD_W(13) PD_W(14) PD_W(15) PD_W(16) PD_W(17) PD_W(18) PD_W(19) PD_W(20) PD_W(21) PD_W(22) PD_W(23)
    else wait_vm<24>();
#undef PD_W
}

// Workgroup barrier for the LDS ring.  __syncthreads() would also wait for
// every outstanding direct-to-LDS load (its release fence covers them) and
// drain the pipeline; here the caller waits for exactly the stage it needs
// (wait_stage), this wave's LDS reads are complete (lgkmcnt 0) before the
// slot they read can be refilled, and the memory clobber keeps the
// compiler from moving LDS accesses across the barrier.
__device__ __forceinline__ void ring_barrier() {
    // lgkmcnt(0) through the builtin, so the compiler's own wait analysis
    // knows every earlier LDS read has completed here
    __builtin_amdgcn_s_waitcnt(0xc07f);
    asm volatile("s_barrier" ::: "memory");
}

// Wait until the stage to be consumed has landed, `younger` (0 .. S-2)
// later stages of LPW loads each being allowed to stay in flight.
template <int S, int LPW, int Y = S - 2>
__device__ __forceinline__ void wait_stage(int younger) {
    if constexpr (Y <= 0) {
        wait_vm<0>();
    } else {
        if (younger >= Y) {
            wait_vm<Y * LPW>();
            return;
        }
        wait_stage<S, LPW, Y - 1>(younger);
    }
}

// Tile BM x BN x BK, WM x WN waves (4 or 8: with 8, two waves share each
// SIMD so one wave's MFMAs cover the other's LDS reads, waits and
// epilogue).  OCC is the number of workgroups per CU the tile is sized for
// (LDS and registers): with 2, one workgroup's ring fill and epilogue
// overlap the other's K loop.  The A tile (activation rows) and the B tile (weight rows)
// stream into two LDS rings of SA and SB stages by direct-to-LDS loads.
// With SA == SB every wave loads its share of both.  With SA != SB
// (8 waves) the first half of the waves loads only A and the second half
// only B: a wave's load counter completes in issue order, so a wave that
// loads both operands cannot keep the slow weight stream (HBM) further
// ahead than the fast activation gathers (L2 / Infinity Cache); split
// roles let the B ring run SB-1 stages ahead on its own.  Every wave
// computes.  ILV deals the tile's 32-row blocks to the WM wave rows
// round-robin (block b to wave row b % WM) instead of in contiguous runs, so
// a tile whose experts fill only part of its rows keeps the MFMA work of
// every SIMD about equal.  Tiles are numbered (m-tile, n-tile) with n fastest and the
// tile range is cut into 8 contiguous pieces, one per XCD (block b runs on
// XCD b % 8): all n-tiles of an m-tile share the gathered activation rows
// in one L2, and the m-tiles of one expert read the same weight tiles at
// the same time from one L2.
template <int BM, int BN, int BK, int WM, int WN, int SA, int SB, bool ILV, bool GATEUP, int OCC, int FK>
__global__ __launch_bounds__(64 * WM * WN, OCC == 1 ? 1 : OCC * WM * WN / 4) void grouped_kernel(
    const uint16_t *__restrict__ a_src, const int32_t *__restrict__ perm_token,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ sel, int nsel,
    const int32_t *__restrict__ tile_start, const uint16_t *const *__restrict__ slots, int H, int I,
    uint16_t *__restrict__ out) {
    constexpr int NW = WM * WN;
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    constexpr bool SPLIT = SA != SB;
    static_assert(!SPLIT || NW == 8, "split load roles need 8 waves");
    constexpr int TM = BM / WM, TN = BN / WN;  // wave tile
    constexpr int MB = TM / 32, NB = TN / 32;  // 32x32 MFMA blocks per wave
    static_assert(MB >= 1 && NB >= 1 && (!GATEUP || NB % 2 == 0), "wave tiling");
    static_assert(MB <= 4, "the live row-block dispatch below covers up to 4 row blocks per wave");
    typedef Geo<BK> G;
    constexpr int NWA = SPLIT ? NW / 2 : NW, NWB = SPLIT ? NW / 2 : NW;  // waves loading A / B
    constexpr int AL = BM / G::RPI / NWA, BL = BN / G::RPI / NWB;  // 1 KB loads per loading wave per stage
    static_assert(AL >= 1 && BL >= 1 && AL * G::RPI * NWA == BM && BL * G::RPI * NWB == BN, "tile / load shape");
    static_assert(!SPLIT || (SA - 1) * AL <= 24, "A-wave waits count live loads up to wait_vm_rt's range");
    constexpr int ASTAGE = BM * G::RB, BSTAGE = BN * G::RB;
    static_assert(OCC * (SA * ASTAGE + SB * BSTAGE) <= 160 * 1024, "LDS of OCC workgroups per CU");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[SA * ASTAGE + SB * BSTAGE];
    uint8_t *const ring_a = smem;
    uint8_t *const ring_b = smem + SA * ASTAGE;

    // ---- tile -> (m-tile, n-tile)
    const int NT = GATEUP ? I / (BN / 2) : H / BN;
    const int total = tile_start[nsel] * NT;
    const int per_xcd = (total + 7) >> 3;
    const int pos = blockIdx.x >> 3;
    if (pos >= per_xcd) return;
    const int t = (blockIdx.x & 7) * per_xcd + pos;
    if (t >= total) return;
    const int mt = t / NT, nt = t - mt * NT;
    // the expert position of m-tile mt: the last lo with tile_start[lo] <= mt.
    // tile_start is non-decreasing with tile_start[0] = 0, so lo is the count
    // of j in [1, nsel) with tile_start[j] <= mt: independent loads and a
    // ballot per 64 entries instead of a chain of dependent loads
    int lo = 0;
#pragma unroll 4
    for (int base = 1; base < nsel; base += 64) {
        const int j = base + (threadIdx.x & 63);
        lo += __popcll(__ballot(j < nsel && tile_start[j] <= mt));
    }
    lo = __builtin_amdgcn_readfirstlane(lo);
    const int e = sel[lo];
    const int row_end = offsets[e + 1];
    const int m0 = offsets[e] + (mt - tile_start[lo]) * BM;
    const int K = GATEUP ? H : I;
    const int n0 = nt * (GATEUP ? BN / 2 : BN);  // first intermediate (gate/up) or output column
    const uint16_t *base = slots[e];
    if (base == nullptr) return;  // no ready copy of this expert: never dereference
    const size_t IH = (size_t)I * H;

    // ---- per-lane source rows: load q of A-wave wa covers A rows
    // RPI(wa + NWA q) .. +RPI-1 (B likewise with wb, NWB); lane l takes row
    // +l/CPR and the logical chunk that belongs in slot l % CPR of that row
    // (the swizzle).
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool a_role = !SPLIT || wave < NWA;
    const int wa = wave, wb = SPLIT ? wave - NWA : wave;
    const int rl = lane / G::CPR, slot = lane % G::CPR;
    // A loads whose rows all lie past the expert's last row are not issued (split roles only: there an A wave's load count per stage
    // is its own, and its waits count its live loads); their LDS rows keep
    // stale values, which reach only accumulator rows the epilogue skips
    const int live_groups = (min(row_end - m0, BM) + G::RPI - 1) / G::RPI;
    const int a_live = SPLIT ? __builtin_amdgcn_readfirstlane(
                                   min(AL, max(0, (live_groups - wa + NWA - 1) / NWA)))
                             : AL;
    // Load addresses.  Load q of a wave covers rows (w + NW q) RPI .. + RPI-1 of
    // its tile, and NW RPI is a multiple of the swizzle period (16 rows), so
    // a lane's row within the group and its swizzled chunk are the same for
    // every q: a per-lane byte offset plus a wave-uniform part per q.  Only the
    // gathered gate/up activation rows need a register per load (their token
    // offsets, in 16-byte units from a_src: 2^32 units cover 64 GiB).
    static_assert((NWA * G::RPI) % 16 == 0 && (NWB * G::RPI) % 16 == 0, "swizzle period");
    const uint32_t a_cs = (uint32_t)(slot ^ G::key(wa * G::RPI + rl));
    const uint32_t b_cs = (uint32_t)(slot ^ G::key(wb * G::RPI + rl));
    uint32_t lp[GATEUP ? AL : 1];
    if (GATEUP && a_role) {
#pragma unroll
        for (int q = 0; q < AL; ++q) {
            const int gr = min(m0 + (wa + NWA * q) * G::RPI + rl, row_end - 1);
            lp[q] = (uint32_t)perm_token[gr] * (uint32_t)(H / 8) + a_cs;
        }
    }
    // B: the lane's row and chunk in bytes from the first row of its load group
    const uint32_t b_lane = (uint32_t)rl * (uint32_t)(K * 2) + b_cs * 16u;
    // B: byte offset of load q's first row in the expert's block
    auto b_row0 = [&](int q) __attribute__((always_inline)) {
        const int rb = (wb + NWB * q) * G::RPI;
        if (GATEUP)
            return rb < BN / 2 ? (size_t)(n0 + rb) * H * 2 : (size_t)IH * 2 + (size_t)(n0 + rb - BN / 2) * H * 2;
        return (size_t)IH * 4 + (size_t)(n0 + rb) * I * 2;
    };
    const uint8_t *const a_base = reinterpret_cast<const uint8_t *>(a_src);
    const uint8_t *const b_base = reinterpret_cast<const uint8_t *>(base);
    auto issue_a = [&](int kt) __attribute__((always_inline)) {
        uint8_t *st = ring_a + (kt % SA) * ASTAGE;
        const uint8_t *b = a_base + kt * (BK * 2);
#pragma unroll
        for (int q = 0; q < AL; ++q)
            if (q < a_live) {
                if (GATEUP) {
                    uint32_t o = lp[GATEUP ? q : 0];
                    opaque(o);
                    load_lds16(reinterpret_cast<const uint16_t *>(b + (size_t)o * 16), st + (wa + NWA * q) * 1024);
                } else {
                    // h rows in grouped order; rows past the expert's end (all
                    // of a dead group's, with unified roles) repeat its last row
                    const int gr = min(m0 + (wa + NWA * q) * G::RPI + rl, row_end - 1);
                    uint32_t o = (uint32_t)gr * (uint32_t)(I / 8) + a_cs;
                    opaque(o);
                    load_lds16(reinterpret_cast<const uint16_t *>(b + (size_t)o * 16), st + (wa + NWA * q) * 1024);
                }
            }
    };
    auto issue_b = [&](int kt) __attribute__((always_inline)) {
        uint8_t *st = ring_b + (kt % SB) * BSTAGE;
        const uint8_t *b = b_base + kt * (BK * 2);
#pragma unroll
        for (int q = 0; q < BL; ++q) {
            uint32_t o = b_lane;
            opaque(o);
            load_lds16<kDeviceScope>(reinterpret_cast<const uint16_t *>(b + b_row0(q) + o), st + (wb + NWB * q) * 1024);
        }
    };

    const int wm = wave / WN, wn = wave % WN;
    const int lrow = lane & 31, lhalf = lane >> 5;
    f32x16_t acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = f32x16_t{};

    // B-tile row of the wave's n-block nb (gate/up pairs share a lane layout)
    auto brow = [&](int nb) {
        return GATEUP ? (nb < NB / 2 ? wn * (TN / 2) + nb * 32 : BN / 2 + wn * (TN / 2) + (nb - NB / 2) * 32)
                      : wn * TN + nb * 32;
    };

    // tile row of this wave's i-th 32-row block
    auto rblk = [&](int i) { return ILV ? (i * WM + wm) * 32 : wm * TM + i * 32; };
    // 32-row blocks of this wave that hold rows of the expert: a tail m-tile
    // of a few rows runs MFMAs and fragment reads on its live blocks only.
    // The count is wave-uniform; the K loop is specialised for each count so
    // every version stays straight-line code.
    const int live_blocks = (row_end - m0 + 31) / 32;
    const int mb_live = __builtin_amdgcn_readfirstlane(
        ILV ? min(MB, max(0, (live_blocks - wm + WM - 1) / WM)) : min(MB, max(0, (row_end - m0 - wm * TM + 31) / 32)));
    const int KT = K / BK;
    // Software-pipelined K loop.  Slot kt % SA of the A ring and kt % SB of
    // the B ring hold stage kt; the stages up to kt+SA-1 / kt+SB-1 are in
    // flight while stage kt is consumed, and the LDS reads of stage kt+1
    // overlap stage kt's MFMAs.
    // ROLE 0: this wave loads both operands (SA == SB); 1: A only; 2: B only
    auto kloop = [&](auto live, auto role_c) __attribute__((always_inline)) {
        constexpr int L = decltype(live)::value;
        constexpr int ROLE = decltype(role_c)::value;
        // a stage of BK is consumed in SUB fragment steps of BKF = FK (16:
        // one MFMA K step, 32: two), so the fragment registers do not grow
        // with BK
        static_assert(FK == 16 || FK == 32, "fragment step of one or two MFMA K steps");
        constexpr int BKF = BK < FK ? BK : FK;
        constexpr int SUB = BK / BKF;
        constexpr int KK = BKF / 16;
        bf16x8_t af[2][KK][MB], bfr[2][KK][NB];
        auto read_frags = [&](int kt, int sub, int buf) __attribute__((always_inline)) {
            const uint8_t *sa = ring_a + (kt % SA) * ASTAGE;
            const uint8_t *sb = ring_b + (kt % SB) * BSTAGE;
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                const int c = (sub * KK + kk) * 2 + lhalf;
#pragma unroll
                for (int i = 0; i < L; ++i)
                    af[buf][kk][i] = *reinterpret_cast<const bf16x8_t *>(sa + G::off(rblk(i) + lrow, c));
#pragma unroll
                for (int j = 0; j < NB; ++j)
                    bfr[buf][kk][j] = *reinterpret_cast<const bf16x8_t *>(sb + G::off(brow(j) + lrow, c));
            }
        };
        auto mfmas = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
            for (int kk = 0; kk < KK; ++kk)
#pragma unroll
                for (int i = 0; i < L; ++i)
#pragma unroll
                    for (int j = 0; j < NB; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[buf][kk][i], bfr[buf][kk][j],
                                                                            acc[i][j], 0, 0, 0);
        };
        // prologue: every ring filled, stage 0 landed
        if constexpr (ROLE == 1) {
#pragma unroll
            for (int s0 = 0; s0 < SA; ++s0)
                if (s0 < KT) issue_a(s0);
            wait_vm_rt(min(SA - 1, KT - 1) * a_live);
        } else if constexpr (ROLE == 2) {
#pragma unroll
            for (int s0 = 0; s0 < SB; ++s0)
                if (s0 < KT) issue_b(s0);
            wait_stage<SB + 1, BL>(min(SB - 1, KT - 1));
        } else {
#pragma unroll
            for (int s0 = 0; s0 < SA; ++s0)
                if (s0 < KT) {
                    issue_a(s0);
                    issue_b(s0);
                }
            wait_stage<SA + 1, AL + BL>(min(SA - 1, KT - 1));
        }
        ring_barrier();
        if constexpr (L > 0) read_frags(0, 0, 0);
        // one pipeline step consuming stage kt from fragment buffer CUR:
        // wait for stage kt+1 of this wave's ring(s), synchronise the block
        // (every wave has then also finished reading stage kt, whose
        // fragments are in registers), refill stage kt's slots with stages
        // kt+SA / kt+SB, read stage kt+1's fragments and run stage kt's MFMAs.
        // STEADY: stages kt+1, kt+SA and kt+SB exist (known at compile time).
        // The steady-state loop then has no path around the barrier; such a
        // path joins the loop header, and the compiler's wait analysis would
        // make this stage's MFMAs wait for the next stage's fragment reads.
        auto step = [&](int kt, auto cur_c, auto steady_c) __attribute__((always_inline)) {
            constexpr int CUR0 = decltype(cur_c)::value;
            constexpr bool STEADY = decltype(steady_c)::value;
            // the stage's sub-steps before its last: read the next sub-step's
            // fragments, run this one's MFMAs (no wait: the stage has landed)
#pragma unroll
            for (int sub = 0; sub + 1 < SUB; ++sub) {
                const int cb = CUR0 ^ (sub & 1);
                if constexpr (L > 0) read_frags(kt, sub + 1, cb ^ 1);
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (L > 0) mfmas(cb);
                __builtin_amdgcn_sched_barrier(0);
            }
            constexpr int CUR = CUR0 ^ ((SUB - 1) & 1);
            if (STEADY || kt + 1 < KT) {
                if constexpr (ROLE == 1) {
                    if constexpr (STEADY) wait_vm_rt((SA - 2) * a_live);
                    else wait_vm_rt(min(SA - 2, KT - 2 - kt) * a_live);
                } else if constexpr (ROLE == 2) {
                    if constexpr (STEADY) wait_stage<SB, BL>(SB - 2);
                    else wait_stage<SB, BL>(min(SB - 2, KT - 2 - kt));
                } else {
                    if constexpr (STEADY) wait_stage<SA, AL + BL>(SA - 2);
                    else wait_stage<SA, AL + BL>(min(SA - 2, KT - 2 - kt));
                }
                ring_barrier();
                // into stage kt's slots, read out before the barrier
                if constexpr (ROLE == 1) {
                    if (STEADY || kt + SA < KT) issue_a(kt + SA);
                } else if constexpr (ROLE == 2) {
                    if (STEADY || kt + SB < KT) issue_b(kt + SB);
                } else {
                    if (STEADY || kt + SA < KT) {
                        issue_a(kt + SA);
                        issue_b(kt + SA);
                    }
                }
                if constexpr (L > 0) read_frags(kt + 1, 0, CUR ^ 1);
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the next stage's reads ahead of these MFMAs
            if constexpr (L > 0) mfmas(CUR);
            // and keep these MFMAs ahead of the next step's wait and barrier:
            // sunk below them, they would leave the next stage's fragment
            // reads nothing to hide behind before that barrier's lgkmcnt(0)
            __builtin_amdgcn_sched_barrier(0);
        };
        using C0 = std::integral_constant<int, 0>;
        using Steady = std::true_type;
        using Tail = std::false_type;
        // unrolled by two so the fragment buffers are indexed statically
        int kt = 0;
        constexpr int SMAX = SA > SB ? SA : SB;
        // the buffer of a stage's first sub-step alternates with SUB odd
        using CN = std::integral_constant<int, SUB & 1>;
        for (; kt + 1 + SMAX < KT; kt += 2) {
            step(kt, C0{}, Steady{});
            step(kt + 1, CN{}, Steady{});
        }
        for (; kt + 1 < KT; kt += 2) {
            step(kt, C0{}, Tail{});
            step(kt + 1, CN{}, Tail{});
        }
        if (kt < KT) step(kt, C0{}, Tail{});
    };
    // one straight-line K loop per load role (both roles pass the same
    // barriers, once per step) and per live row-block count
    auto run = [&](auto live) __attribute__((always_inline)) {
        if constexpr (SPLIT) {
            if (a_role) kloop(live, std::integral_constant<int, 1>{});
            else kloop(live, std::integral_constant<int, 2>{});
        } else {
            kloop(live, std::integral_constant<int, 0>{});
        }
    };
    if (mb_live >= MB) run(std::integral_constant<int, MB>{});
    else if (mb_live == 0) run(std::integral_constant<int, 0>{});
    else if constexpr (MB >= 2) {
        if (mb_live == 1) run(std::integral_constant<int, 1>{});
        else if constexpr (MB >= 3) {
            if (mb_live == 2) run(std::integral_constant<int, 2>{});
            else if constexpr (MB >= 4) {
                if (mb_live == 3) run(std::integral_constant<int, 3>{});
            }
        }
    }

    // ---- epilogue: lane holds column (lane & 31), rows (r/4)*8 + (lane/32)*4 + r%4
#pragma unroll
    for (int i = 0; i < MB; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + rblk(i) + (r >> 2) * 8 + lhalf * 4 + (r & 3);
            if (row >= row_end) continue;
            if (GATEUP) {
#pragma unroll
                for (int j = 0; j < NB / 2; ++j) {
                    const int col = n0 + wn * (TN / 2) + j * 32 + lrow;
                    // g and u rounded by one conversion
                    const uint32_t gu = f2bf2_hw(acc[i][j][r], acc[i][j + NB / 2][r]);
                    const float g = __uint_as_float(gu << 16);
                    const float u = __uint_as_float(gu & 0xffff0000u);
                    const float a = bf16_round_hw(silu_fast(g));
                    out[(size_t)row * I + col] = (uint16_t)f2bf_hw(a * u);
                }
            } else {
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const int col = n0 + wn * TN + j * 32 + lrow;
                    out[(size_t)row * H + col] = (uint16_t)f2bf_hw(acc[i][j][r]);
                }
            }
        }
    }
}

// phase: 1 = gate/up only, 2 = down only, 3 = both
// PH: the phases (1 gate/up, 2 down) this tile configuration serves
template <int BM, int BN, int BK, int WM, int WN, int SA, int SB, bool ILV = false, int PH = 3, int OCC = 1,
          int FK = 32>
int launch_grouped(int phase, const uint16_t *x, const int32_t *perm_token, const int32_t *offsets,
                   const int32_t *sel, int nsel, const int32_t *tile_start, int max_tiles,
                   const uint16_t *const *slots, int H, int I, uint16_t *h_ws, uint16_t *y, hipStream_t s) {
    if (I % (BN / 2) || H % BN || H % BK || I % BK)
        return fail(kEInval, "grouped: I must divide by BN/2, H by BN, and both by the K step");
    // grid: every (m-tile, n-tile) the bound allows, a multiple of 8 so each
    // XCD's contiguous piece of the tile range has blocks
    if constexpr ((PH & 1) != 0) if (phase & 1) {
        const size_t n1 = (size_t)max_tiles * (size_t)(I / (BN / 2));
        const unsigned g1 = (unsigned)((n1 + 7) / 8 * 8);
        grouped_kernel<BM, BN, BK, WM, WN, SA, SB, ILV, true, OCC, FK><<<g1, 64 * WM * WN, 0, s>>>(x, perm_token, offsets, sel, nsel, tile_start,
                                                                    slots, H, I, h_ws);
        int rc = check_launch("grouped_kernel<gateup>");
        if (rc) return rc;
    }
    if constexpr ((PH & 2) != 0) if (phase & 2) {
        const size_t n2 = (size_t)max_tiles * (size_t)(H / BN);
        const unsigned g2 = (unsigned)((n2 + 7) / 8 * 8);
        grouped_kernel<BM, BN, BK, WM, WN, SA, SB, ILV, false, OCC, FK><<<g2, 64 * WM * WN, 0, s>>>(h_ws, nullptr, offsets, sel, nsel, tile_start,
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
        return launch_grouped<32, 256, 64, 1, 4, 4, 4>(phase, xp, perm_token, offsets, sel, nsel, tile_start, max_tiles, sp,
                                                H, I, (uint16_t *)h_ws, (uint16_t *)y, s);
    case 64: {
        // gate/up: split load roles, 3 + 4 stages, one workgroup per CU; down
        // (K = I, a short K loop): every wave loads both operands, 2 + 2
        // stages, two workgroups per CU (T=512: 79.6 against 85.3 us)
        int rc = kOk;
        if (phase & 1)
            rc = launch_grouped<64, 256, 64, 2, 4, 3, 4, false, 1>(1, xp, perm_token, offsets, sel, nsel, tile_start,
                                                                   max_tiles, sp, H, I, (uint16_t *)h_ws,
                                                                   (uint16_t *)y, s);
        if (rc == kOk && (phase & 2))
            rc = launch_grouped<64, 256, 64, 2, 4, 2, 2, false, 2, 2>(2, xp, perm_token, offsets, sel, nsel, tile_start,
                                                                      max_tiles, sp, H, I, (uint16_t *)h_ws,
                                                                      (uint16_t *)y, s);
        return rc;
    }
    case 128:
        return launch_grouped<128, 256, 64, 2, 4, 3, 3>(phase, xp, perm_token, offsets, sel, nsel, tile_start, max_tiles,
                                                 sp, H, I, (uint16_t *)h_ws, (uint16_t *)y, s);
    case 256:
        // 128-byte row pieces (BK 64) halve the L2 requests of the 64-byte
        // ones; each CU keeps about 64 requests in flight, so the bytes per
        // request set its fill rate.  Fragments are read one MFMA K step (16)
        // ahead, which keeps the tile within 256 VGPRs without spills, and
        // split load roles with 2 + 3 stages fill the 160 KB of LDS
        // (T=4096, Zipf routing: gate/up 338 -> 299 us, down 199 -> 173 us;
        // uniform: down 190 -> 161 us; bit-identical)
        return launch_grouped<256, 256, 64, 2, 4, 2, 3, false, 3, 1, 16>(phase, xp, perm_token, offsets, sel, nsel,
                                                                         tile_start, max_tiles, sp, H, I,
                                                                         (uint16_t *)h_ws, (uint16_t *)y, s);
    case 384:
        return launch_grouped<384, 128, 64, 4, 2, 2, 4, true>(phase, xp, perm_token, offsets, sel, nsel, tile_start,
                                                       max_tiles, sp, H, I, (uint16_t *)h_ws, (uint16_t *)y, s);
    default:
        return fail(kEInval, "grouped: block_m must be 32, 64, 128, 256 or 384");
    }
}

}  // namespace pd

using namespace pd;

// The row tile should cover a typical expert in one tile (weights are then
// read once per expert and n-tile); 32 only for very thin experts.
PD_API int pdscope_grouped_block_m(int rows_hint) {
    if (rows_hint <= 16) return 32;
    // whole Qwen-shaped layers (pack + gate/up + down + merge), uniform
    // routing, back to back: 24..40 mean rows run fastest on 64-row tiles,
    // 48..96 on 128-row tiles (64 rows: 271 against 292 us), 112 and above on
    // the 256-row tile (112: 309 against 320 us; the DeepSeek-V2-Lite mixed
    // batch, 122 mean rows of 17 MB experts: 332 against 355 us)
    if (rows_hint <= 44) return 64;
    if (rows_hint <= 104) return 128;
    if (rows_hint <= 192) return 256;
    // one 384-row tile holds an expert of the typical 200..320 rows (no
    // tail tile re-reading its weights); beyond that 256x256 tiles read the
    // activation rows fewer times
    if (rows_hint <= 320) return 384;
    return 256;
}

PD_API int pdscope_grouped_block_m_max(int mean_rows, int max_rows) {
    const int bm = pdscope_grouped_block_m(mean_rows);
    return bm == 384 && max_rows > 768 ? 256 : bm;
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
