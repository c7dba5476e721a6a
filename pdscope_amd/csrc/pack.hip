// K2: expert-sorted ragged packing.  Restates compact_expert_groups
// (expertbench/pdscope_runtime.py:16-39): a stable sort of the slot-major
// flat expert ids (f = s*T + t), i.e. a counting sort.
//
// Up to one chunk of ids (small T): one workgroup of 16 waves (below);
// larger inputs: one workgroup per chunk in two launches (further down).
// One workgroup of 16 waves.  Each wave owns a contiguous segment of the
// flat index space.  Pass 1 counts the segment per expert: a wave splits its
// 64 ids into equal-id groups with 8 ballots (one per id bit); the lowest
// lane of each group adds the group size to the wave's private LDS row.
// A scan over (expert, wave) turns the counts into per-wave write bases.
// Pass 2 repeats the ballots; a lane's grouped row is its wave base plus the
// number of equal ids in lower lanes, so the order inside an expert stays
// (slot, token) ascending.
#include <mutex>

#include "common.h"

namespace pd {

constexpr int kPackWaves = 16;
constexpr int kPackMaxE = 256;

__device__ __forceinline__ uint64_t group_mask(int e, bool valid) {
    uint64_t m = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        uint64_t bb = __ballot((e >> b) & 1);
        m &= ((e >> b) & 1) ? bb : ~bb;
    }
    return m;
}

// inclusive scan of one value per thread over the first 256 threads
__device__ int block_scan256(int v, int *s_wsum) {
    const int lane = lane_id(), wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        int o = __shfl_up(v, off, kWave);
        if (lane >= off) v += o;
    }
    if (lane == 63 && wave < 4) s_wsum[wave] = v;
    __syncthreads();
    int add = 0;
    for (int w = 0; w < wave && w < 4; ++w) add += s_wsum[w];
    __syncthreads();
    return v + add;
}

// The balanced order and tile prefixes, computed by threads 0..255 of the
// calling block (every thread of the block must call it: it synchronises).
// rows[e]: rows of expert e < E (global or LDS); a sel entry outside [0, E)
// counts as an expert with no rows (no tiles: the grouped launch never
// addresses it).  s_rows / s_at: 256 ints of LDS each (s_rows 16-byte
// aligned), s_wsum: 4 ints.
__device__ void balanced_schedule(const int32_t *rows, int E, const int32_t *__restrict__ sel, int nsel, int bm,
                                  int32_t *__restrict__ order, int32_t *__restrict__ tile_start, int bm2,
                                  int32_t *__restrict__ tile_start2, int *s_rows, int *s_at, int *s_wsum) {
    const int i = threadIdx.x;
    if (i < 256) {
        const int e = i < nsel ? sel[i] : -1;
        // -1 past nsel: never ranks above a real expert
        s_rows[i] = i < nsel ? ((unsigned)e < (unsigned)E ? rows[e] : 0) : -1;
    }
    __syncthreads();
    if (i < nsel) {
        const int c = s_rows[i];
        int r = 0;
        // four rows per LDS read (broadcast)
        for (int j = 0; j < nsel; j += 4) {
            const int4 q = *reinterpret_cast<const int4 *>(s_rows + j);
            r += (q.x > c) | ((q.x == c) & (j < i));
            r += (q.y > c) | ((q.y == c) & (j + 1 < i));
            r += (q.z > c) | ((q.z == c) & (j + 2 < i));
            r += (q.w > c) | ((q.w == c) & (j + 3 < i));
        }
        const int full = nsel >> 3, rem = nsel & 7;
        const int rd = r >> 3, w = r & 7;
        const int g = (rd & 1) ? 7 - w : w;
        // groups before g: `full` members each, plus one if the last (partial)
        // round reaches them (round `full` deals to 0.. upward when even, 7.. downward when odd)
        int before = g * full;
        if (rem) before += (full & 1) ? max(0, g - (8 - rem)) : min(g, rem);
        s_at[before + rd] = i;
    }
    __syncthreads();
    int tiles = 0, tiles2 = 0;
    if (i < nsel) {
        const int si = s_at[i];
        order[i] = sel[si];
        tiles = (s_rows[si] + bm - 1) / bm;
        if (tile_start2) tiles2 = (s_rows[si] + bm2 - 1) / bm2;
    }
    const int incl = block_scan256(tiles, s_wsum);
    if (i == 0) tile_start[0] = 0;
    if (i < nsel) tile_start[i + 1] = incl;
    if (tile_start2) {  // uniform: the whole block takes this branch
        const int incl2 = block_scan256(tiles2, s_wsum);
        if (i == 0) tile_start2[0] = 0;
        if (i < nsel) tile_start2[i + 1] = incl2;
    }
}

// 64-id chunks per wave held in registers: the single-workgroup kernel runs up
// to 2048 ids (two chunks per wave, one pass); loading more chunks than a
// wave's segment holds cost 2.7-6 us per call at T*k = 512..2048
constexpr int kPackRC = 2;

// Load up to kPackRC chunks of the wave's segment (expert id, or -1 outside
// the segment / outside [0, E)) with every load in flight at once.
__device__ __forceinline__ void pack_load(const int32_t *__restrict__ ids, int T, int k, int E, int sc, int end,
                                          int lane, int (&idv)[kPackRC]) {
    // Addresses are clamped into the segment so every load is unconditional
    // and all kPackRC loads are in flight together; out-of-segment lanes are
    // masked afterwards.
    const int last = max(end - 1, 0);
    int raw[kPackRC];
#pragma unroll
    for (int c = 0; c < kPackRC; ++c) {
        const int f = min(sc + c * 64 + lane, last);
        const int s = f / T, t = f - s * T;
        raw[c] = ids[(size_t)t * k + s];
    }
#pragma unroll
    for (int c = 0; c < kPackRC; ++c) {
        const int f = sc + c * 64 + lane;
        const int e = raw[c];
        idv[c] = (f < end && e >= 0 && e < E) ? e : -1;
    }
}

// Balanced schedule requested together with a pack (order == nullptr: none).
struct PackSchedule {
    const int32_t *sel;
    int nsel, bm, bm2;
    int32_t *order, *tile_start, *tile_start2;
};

// The schedule from the per-expert totals `tot` held by threads e < E.
__device__ void pack_then_schedule(const PackSchedule &ps, int E, int tot) {
    __shared__ __align__(16) int s_tot[kPackMaxE];
    __shared__ __align__(16) int s_rows[256];
    __shared__ int s_at[256];
    __shared__ int s_ws2[4];
    if (threadIdx.x < E) s_tot[threadIdx.x] = tot;
    __syncthreads();
    balanced_schedule(s_tot, E, ps.sel, ps.nsel, ps.bm, ps.order, ps.tile_start, ps.bm2, ps.tile_start2, s_rows,
                      s_at, s_ws2);
}

__global__ __launch_bounds__(1024) void pack_kernel(const int32_t *__restrict__ ids, int T, int k, int E,
                                                    int32_t *__restrict__ counts, int32_t *__restrict__ offsets,
                                                    int32_t *__restrict__ perm_token,
                                                    int32_t *__restrict__ perm_pos,
                                                    int32_t *__restrict__ row_of, PackSchedule ps) {
    __shared__ int32_t s_cnt[kPackWaves][kPackMaxE];
    __shared__ int s_wsum[4];
    const int n = T * k;
    const int wave = threadIdx.x >> 6, lane = lane_id();
    const int seg = ((n + kPackWaves * 64 - 1) / (kPackWaves * 64)) * 64;
    const int beg = min(wave * seg, n), end = min(beg + seg, n);
    const uint64_t below = (1ull << lane) - 1ull;
    const bool one_pass = (end - beg) <= kPackRC * 64;
    int idv[kPackRC];

    for (int e = lane; e < E; e += 64) s_cnt[wave][e] = 0;
    __syncthreads();
    // pass 1: per-wave counts
    for (int sc = beg; sc < end; sc += kPackRC * 64) {
        pack_load(ids, T, k, E, sc, end, lane, idv);
#pragma unroll
        for (int c = 0; c < kPackRC; ++c) {
            if (sc + c * 64 >= end) break;
            const int e = idv[c];
            const uint64_t m = group_mask(e < 0 ? 0 : e, e >= 0);
            if (e >= 0 && !(m & below)) s_cnt[wave][e] += __popcll(m);
        }
    }
    __syncthreads();
    int tot = 0;
    if (threadIdx.x < E)
        for (int w = 0; w < kPackWaves; ++w) tot += s_cnt[w][threadIdx.x];
    // a second workgroup (launched with a schedule only) counts as well and
    // writes the schedule while the first scatters
    if (blockIdx.x == 1) {
        pack_then_schedule(ps, E, tot);
        return;
    }
    const int incl = block_scan256(threadIdx.x < 256 ? tot : 0, s_wsum);
    if (threadIdx.x < E) {
        const int e = threadIdx.x;
        int run = incl - tot;
        counts[e] = tot;
        offsets[e] = run;
        if (e == E - 1) offsets[E] = incl;
        for (int w = 0; w < kPackWaves; ++w) {
            int c = s_cnt[w][e];
            s_cnt[w][e] = run;
            run += c;
        }
    }
    __syncthreads();
    // pass 2: stable scatter
    for (int sc = beg; sc < end; sc += kPackRC * 64) {
        if (!one_pass) pack_load(ids, T, k, E, sc, end, lane, idv);
#pragma unroll
        for (int c = 0; c < kPackRC; ++c) {
            if (sc + c * 64 >= end) break;
            const int e = idv[c];
            const uint64_t m = group_mask(e < 0 ? 0 : e, e >= 0);
            if (e >= 0) {
                const int f = sc + c * 64 + lane;
                const int s = f / T, t = f - s * T;
                const int pos = s_cnt[wave][e] + __popcll(m & below);
                perm_token[pos] = t;
                perm_pos[pos] = t * k + s;
                row_of[(size_t)t * k + s] = pos;
                if (!(m & below)) s_cnt[wave][e] += __popcll(m);
            }
        }
    }
}

// Multi-block variant for large T*k: the flat index space is cut into
// chunks of kPackWaves * 64 * kChunkRC ids (one chunk per block, one
// 64*kChunkRC segment per wave).  pack_count_kernel writes each chunk's
// per-expert counts to hist[chunk][e]; pack_scatter_kernel recounts its
// chunk per wave, turns hist into the chunk's bases (expert offset plus the
// counts of earlier chunks) and scatters exactly as the single-block kernel,
// so the grouping is identical.
constexpr int kChunkRC = 2;
constexpr int kChunkIds = kPackWaves * 64 * kChunkRC;

__device__ __forceinline__ void chunk_load(const int32_t *__restrict__ ids, int T, int k, int E, int beg, int end,
                                           int lane, int (&idv)[kChunkRC]) {
    const int last = max(end - 1, 0);
    int raw[kChunkRC];
#pragma unroll
    for (int c = 0; c < kChunkRC; ++c) {
        const int f = min(beg + c * 64 + lane, last);
        const int s = f / T, t = f - s * T;
        raw[c] = ids[(size_t)t * k + s];
    }
#pragma unroll
    for (int c = 0; c < kChunkRC; ++c) {
        const int f = beg + c * 64 + lane;
        const int e = raw[c];
        idv[c] = (f < end && e >= 0 && e < E) ? e : -1;
    }
}

// per-wave counts of this wave's segment into s_cnt[wave][*] (zeroed here)
__device__ __forceinline__ void chunk_count(const int (&idv)[kChunkRC], int beg, int end, int E, int wave, int lane,
                                            int32_t (*s_cnt)[kPackMaxE]) {
    const uint64_t below = (1ull << lane) - 1ull;
    for (int e = lane; e < E; e += 64) s_cnt[wave][e] = 0;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int c = 0; c < kChunkRC; ++c) {
        if (beg + c * 64 >= end) break;
        const int e = idv[c];
        const uint64_t m = group_mask(e < 0 ? 0 : e, e >= 0);
        if (e >= 0 && !(m & below)) s_cnt[wave][e] += __popcll(m);
    }
}

__global__ __launch_bounds__(1024) void pack_count_kernel(const int32_t *__restrict__ ids, int T, int k, int E,
                                                          int32_t *__restrict__ hist) {
    __shared__ int32_t s_cnt[kPackWaves][kPackMaxE];
    const int n = T * k;
    const int wave = threadIdx.x >> 6, lane = lane_id();
    const int beg = min((int)blockIdx.x * kChunkIds + wave * 64 * kChunkRC, n);
    const int end = min(beg + 64 * kChunkRC, n);
    int idv[kChunkRC];
    chunk_load(ids, T, k, E, beg, end, lane, idv);
    chunk_count(idv, beg, end, E, wave, lane, s_cnt);
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        int tot = 0;
        for (int w = 0; w < kPackWaves; ++w) tot += s_cnt[w][e];
        hist[(size_t)blockIdx.x * E + e] = tot;
    }
}

__global__ __launch_bounds__(1024) void pack_scatter_kernel(const int32_t *__restrict__ ids, int T, int k, int E,
                                                            const int32_t *__restrict__ hist, int nchunk,
                                                            int32_t *__restrict__ counts,
                                                            int32_t *__restrict__ offsets,
                                                            int32_t *__restrict__ perm_token,
                                                            int32_t *__restrict__ perm_pos,
                                                            int32_t *__restrict__ row_of, PackSchedule ps) {
    __shared__ int32_t s_cnt[kPackWaves][kPackMaxE];
    __shared__ int s_wsum[4];
    if ((int)blockIdx.x == nchunk) {
        // the extra workgroup of a launch with a schedule: totals from the
        // per-chunk counts, then the schedule, beside the scatter
        int tot = 0;
        if (threadIdx.x < E)
            for (int b = 0; b < nchunk; ++b) tot += hist[(size_t)b * E + threadIdx.x];
        pack_then_schedule(ps, E, tot);
        return;
    }
    const int n = T * k;
    const int wave = threadIdx.x >> 6, lane = lane_id();
    const int beg = min((int)blockIdx.x * kChunkIds + wave * 64 * kChunkRC, n);
    const int end = min(beg + 64 * kChunkRC, n);
    const uint64_t below = (1ull << lane) - 1ull;
    int idv[kChunkRC];
    chunk_load(ids, T, k, E, beg, end, lane, idv);
    chunk_count(idv, beg, end, E, wave, lane, s_cnt);
    int tot = 0, pre = 0;
    if (threadIdx.x < E) {
        const int e = threadIdx.x;
        for (int b = 0; b < nchunk; ++b) {
            const int c = hist[(size_t)b * E + e];
            tot += c;
            if (b < (int)blockIdx.x) pre += c;
        }
    }
    __syncthreads();
    const int incl = block_scan256(threadIdx.x < 256 ? tot : 0, s_wsum);
    if (threadIdx.x < E) {
        const int e = threadIdx.x;
        const int off = incl - tot;
        if (blockIdx.x == 0) {
            counts[e] = tot;
            offsets[e] = off;
            if (e == E - 1) offsets[E] = incl;
        }
        int run = off + pre;
        for (int w = 0; w < kPackWaves; ++w) {
            const int c = s_cnt[w][e];
            s_cnt[w][e] = run;
            run += c;
        }
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kChunkRC; ++c) {
        if (beg + c * 64 >= end) break;
        const int e = idv[c];
        const uint64_t m = group_mask(e < 0 ? 0 : e, e >= 0);
        if (e >= 0) {
            const int f = beg + c * 64 + lane;
            const int s = f / T, t = f - s * T;
            const int pos = s_cnt[wave][e] + __popcll(m & below);
            perm_token[pos] = t;
            perm_pos[pos] = t * k + s;
            row_of[(size_t)t * k + s] = pos;
            if (!(m & below)) s_cnt[wave][e] += __popcll(m);
        }
    }
}

// a sel entry outside [0, E) counts as an expert with no rows
__global__ __launch_bounds__(256) void schedule_kernel(const int32_t *__restrict__ counts, int E,
                                                       const int32_t *__restrict__ sel, int nsel, int bm,
                                                       int32_t *__restrict__ tile_start) {
    __shared__ int s_wsum[4];
    __shared__ int s_carry;
    if (threadIdx.x == 0) {
        s_carry = 0;
        tile_start[0] = 0;
    }
    __syncthreads();
    for (int base = 0; base < nsel; base += 256) {
        const int i = base + threadIdx.x;
        const int e = i < nsel ? sel[i] : -1;
        const int tiles = (unsigned)e < (unsigned)E ? (counts[e] + bm - 1) / bm : 0;
        const int incl = block_scan256(tiles, s_wsum);
        if (i < nsel) tile_start[i + 1] = s_carry + incl;
        __syncthreads();
        if (threadIdx.x == 255) s_carry += incl;
        __syncthreads();
    }
}

// Balanced tile order for the grouped kernel, which cuts its tile list (in
// sel order) into 8 contiguous equal-count pieces, one per XCD, dispatched in
// order.  The selected experts are ranked by rows (descending, then by
// position), rank r is dealt to group (r / 8 even ? r % 8 : 7 - r % 8) and
// the groups are concatenated: every piece then holds a similar mix of large
// and small experts (similar work) and starts with its largest ones, so the
// short tiles run last.  order[i] is the expert at position i of that list,
// tile_start its m-tile prefix (as schedule_kernel over `order`).  nsel <= 256.
// With tile_start2, the same order's m-tile prefix for a second row tile bm2
// (the order depends on the rows only, not on the tile).
__global__ __launch_bounds__(256) void schedule_balanced_kernel(const int32_t *__restrict__ counts, int E,
                                                                const int32_t *__restrict__ sel, int nsel, int bm,
                                                                int32_t *__restrict__ order,
                                                                int32_t *__restrict__ tile_start, int bm2,
                                                                int32_t *__restrict__ tile_start2) {
    __shared__ __align__(16) int s_rows[256];
    __shared__ int s_at[256];  // list position -> sel position
    __shared__ int s_wsum[4];
    balanced_schedule(counts, E, sel, nsel, bm, order, tile_start, bm2, tile_start2, s_rows, s_at, s_wsum);
}

}  // namespace pd

using namespace pd;

// above this many ids the two-launch multi-block path is used
constexpr int kPackMultiMin = kChunkIds;

PD_API size_t pdscope_pack_workspace_size(int T, int k, int E) {
    if (T < 1 || k < 1 || E < 1) return 0;
    const int64_t n = (int64_t)T * k;
    if (n <= kPackMultiMin) return 0;
    return (size_t)((n + kChunkIds - 1) / kChunkIds) * (size_t)E * sizeof(int32_t);
}

static int pack_launch(const int32_t *ids, int T, int k, int E, int32_t *counts, int32_t *offsets,
                       int32_t *perm_token, int32_t *perm_pos, int32_t *row_of, void *workspace, PackSchedule ps,
                       void *stream) {
    if (!ids || !counts || !offsets || !perm_token || !perm_pos || !row_of)
        return fail(kEInval, "pack: null pointer");
    if (T < 1 || k < 1 || E < 1 || E > kPackMaxE) return fail(kEInval, "pack: need T,k >= 1 and 1 <= E <= 256");
    if ((int64_t)T * k > (1ll << 30)) return fail(kEInval, "pack: T*k too large");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int n = T * k;
    if (n <= kPackMultiMin) {
        pack_kernel<<<ps.order ? 2 : 1, 1024, 0, s>>>(ids, T, k, E, counts, offsets, perm_token, perm_pos, row_of, ps);
        return check_launch("pack_kernel");
    }
    if (!workspace) return fail(kEInval, "pack: T*k above the single-block size needs pdscope_pack_workspace_size bytes");
    const int nchunk = (n + kChunkIds - 1) / kChunkIds;
    int32_t *hist = static_cast<int32_t *>(workspace);
    pack_count_kernel<<<nchunk, 1024, 0, s>>>(ids, T, k, E, hist);
    int rc = check_launch("pack_count_kernel");
    if (rc) return rc;
    pack_scatter_kernel<<<nchunk + (ps.order ? 1 : 0), 1024, 0, s>>>(ids, T, k, E, hist, nchunk, counts, offsets, perm_token, perm_pos,
                                                row_of, ps);
    return check_launch("pack_scatter_kernel");
}

PD_API int pdscope_pack(const int32_t *ids, int T, int k, int E, int32_t *counts, int32_t *offsets,
                        int32_t *perm_token, int32_t *perm_pos, int32_t *row_of, void *workspace, void *stream) {
    return pack_launch(ids, T, k, E, counts, offsets, perm_token, perm_pos, row_of, workspace,
                       PackSchedule{nullptr, 0, 0, 0, nullptr, nullptr, nullptr}, stream);
}

PD_API int pdscope_pack_schedule_balanced(const int32_t *ids, int T, int k, int E, int32_t *counts,
                                          int32_t *offsets, int32_t *perm_token, int32_t *perm_pos,
                                          int32_t *row_of, void *workspace, const int32_t *sel, int nsel,
                                          int block_m, int block_m2, int32_t *order, int32_t *tile_start,
                                          int32_t *tile_start2, void *stream) {
    if (!sel || !order || !tile_start || nsel < 0 || nsel > 256 || (block_m2 != 0) != (tile_start2 != nullptr))
        return fail(kEInval, "pack_schedule_balanced: bad schedule arguments (nsel 0..256; block_m2 with tile_start2)");
    for (int b : {block_m, block_m2 ? block_m2 : block_m})
        if (b != 32 && b != 64 && b != 128 && b != 256 && b != 384)
            return fail(kEInval, "pack_schedule_balanced: block sizes must be 32, 64, 128, 256 or 384");
    return pack_launch(ids, T, k, E, counts, offsets, perm_token, perm_pos, row_of, workspace,
                       PackSchedule{sel, nsel, block_m, block_m2, order, tile_start, tile_start2}, stream);
}

// ---------------------------------------------------------------- no-allocation variant
//
// pdscope_pack_static: pdscope_pack whose multi-block path keeps its
// per-chunk counts in a library-owned device array instead of a caller
// workspace.  The count launch writes hist[c][e] for every chunk c < nchunk
// and expert e < E before the scatter launch reads them, so nothing in the
// array has to start at zero and a call never depends on what an earlier
// call left there.  Every call on one GPU shares that GPU's array: calls that
// overlap in time on one GPU race.
constexpr int kPackStaticMaxIds = 1 << 20;
constexpr int kPackStaticWords = (kPackStaticMaxIds / kChunkIds) * kPackMaxE;  // 512 KiB

static __device__ __align__(256) int32_t scratch[kPackStaticWords];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static int32_t *g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device, looked up once per
// device with that device current (the array's host-side name is not a
// device address and must never be passed to a kernel).
static int pack_scratch(int32_t **out) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return fail(kEHip, std::string("pack_static: hipGetDevice: ") + hipGetErrorString(err));
    if (dev < 0 || dev >= kMaxDevices) return fail(kEInval, "pack_static: device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !p)
            return fail(kEHip, std::string("pack_static: hipGetSymbolAddress: ") + hipGetErrorString(err));
        g_scratch_ptr[dev] = static_cast<int32_t *>(p);
    }
    *out = g_scratch_ptr[dev];
    return kOk;
}

// The id limit of pdscope_pack_static.  Also resolves the static array's
// address on the current device, so a caller that sizes its inputs at set-up
// pays that lookup there, outside any stream capture; returns 0 (with the
// error message set) if the lookup fails.
PD_API size_t pdscope_pack_static_max_ids(void) {
    int32_t *p = nullptr;
    if (pack_scratch(&p) != kOk) return 0;
    return (size_t)kPackStaticMaxIds;
}

PD_API int pdscope_pack_static(const int32_t *ids, int T, int k, int E, int32_t *counts, int32_t *offsets,
                               int32_t *perm_token, int32_t *perm_pos, int32_t *row_of, void *stream) {
    if (!ids || !counts || !offsets || !perm_token || !perm_pos || !row_of)
        return fail(kEInval, "pack_static: null pointer");
    if (T < 1 || k < 1 || E < 1 || E > kPackMaxE)
        return fail(kEInval, "pack_static: need T,k >= 1 and 1 <= E <= 256");
    if ((int64_t)T * k > kPackStaticMaxIds)
        return fail(kEInval, "pack_static: T*k exceeds the static scratch limit of 1048576 ids");
    const int n = T * k;
    if (n <= kPackMultiMin) return pdscope_pack(ids, T, k, E, counts, offsets, perm_token, perm_pos, row_of, nullptr,
                                                stream);
    int32_t *hist = nullptr;
    const int rc = pack_scratch(&hist);
    if (rc) return rc;
    return pdscope_pack(ids, T, k, E, counts, offsets, perm_token, perm_pos, row_of, hist, stream);
}

PD_API int pdscope_schedule(const int32_t *counts, int E, const int32_t *sel, int nsel, int block_m,
                            int32_t *tile_start, void *stream) {
    if (!counts || !sel || !tile_start || nsel < 0 || E < 1) return fail(kEInval, "schedule: bad arguments");
    if (block_m != 32 && block_m != 64 && block_m != 128 && block_m != 256 && block_m != 384)
        return fail(kEInval, "schedule: block_m must be 32, 64, 128, 256 or 384");
    schedule_kernel<<<1, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(counts, E, sel, nsel, block_m, tile_start);
    return check_launch("schedule_kernel");
}

PD_API int pdscope_schedule_balanced(const int32_t *counts, int E, const int32_t *sel, int nsel, int block_m,
                                     int32_t *order, int32_t *tile_start, void *stream) {
    if (!counts || !sel || !order || !tile_start || nsel < 0 || nsel > 256 || E < 1)
        return fail(kEInval, "schedule_balanced: bad arguments (nsel must be 0..256)");
    if (block_m != 32 && block_m != 64 && block_m != 128 && block_m != 256 && block_m != 384)
        return fail(kEInval, "schedule_balanced: block_m must be 32, 64, 128, 256 or 384");
    schedule_balanced_kernel<<<1, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(counts, E, sel, nsel, block_m,
                                                                                   order, tile_start, 0, nullptr);
    return check_launch("schedule_balanced_kernel");
}

PD_API int pdscope_schedule_balanced_pair(const int32_t *counts, int E, const int32_t *sel, int nsel, int block_m,
                                          int block_m2, int32_t *order, int32_t *tile_start, int32_t *tile_start2,
                                          void *stream) {
    if (!counts || !sel || !order || !tile_start || !tile_start2 || nsel < 0 || nsel > 256 || E < 1)
        return fail(kEInval, "schedule_balanced_pair: bad arguments (nsel must be 0..256)");
    for (int b : {block_m, block_m2})
        if (b != 32 && b != 64 && b != 128 && b != 256 && b != 384)
            return fail(kEInval, "schedule_balanced_pair: block sizes must be 32, 64, 128, 256 or 384");
    schedule_balanced_kernel<<<1, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(counts, E, sel, nsel, block_m,
                                                                                   order, tile_start, block_m2,
                                                                                   tile_start2);
    return check_launch("schedule_balanced_kernel");
}
