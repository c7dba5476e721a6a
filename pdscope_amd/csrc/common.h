// Shared device helpers for the gfx950 MoE-layer kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#define PD_API extern "C" __attribute__((visibility("default")))

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

namespace pd {

constexpr int kWave = 64;

// ---------------------------------------------------------------- errors

void set_error(const std::string &msg);
int fail(int code, const std::string &msg);
int check_launch(const char *what);

enum : int { kOk = 0, kEInval = 1, kEHip = 2 };

// ---------------------------------------------------------------- bf16

__device__ __forceinline__ float bf2f(uint32_t h16) { return __uint_as_float(h16 << 16); }

// round-to-nearest-even fp32 -> bf16 (same rule as torch's c10::BFloat16)
__device__ __forceinline__ uint32_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float bf16_round(float f) { return bf2f(f2bf(f)); }

// The same round-to-nearest-even conversion by gfx950's v_cvt_pk_bf16_f32
// (equal to f2bf for every finite value and infinity): for epilogues that
// convert many values per lane.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t f2bf_hw(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ float bf16_round_hw(float f) { return (float)(__bf16)f; }
// lo in bits 0-15, hi in bits 16-31
__device__ __forceinline__ uint32_t f2bf2_hw(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

// low / high bf16 of a packed 32-bit word, widened to fp32
__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Global-address-space views.  Pointers read from memory (slot tables) are
// generic to the compiler, which then emits flat loads; flat loads also
// count against the LDS wait counter, so every LDS wait would drain them.
// Casting to address space 1 keeps them global loads.
typedef __attribute__((address_space(1))) const u32x4_t g_u32x4_t;

__device__ __forceinline__ const g_u32x4_t *gptr(const void *p) {
    return (const g_u32x4_t *)(reinterpret_cast<uintptr_t>(p));
}

// 16-byte streaming load that bypasses cache allocation (weights read once)
__device__ __forceinline__ uint4 ld_nt(const void *p) {
    u32x4_t v = __builtin_nontemporal_load(gptr(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// plain 16-byte global load
__device__ __forceinline__ uint4 ld_g(const void *p) {
    u32x4_t v = *gptr(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// dot of 8 bf16 pairs packed in two uint4, accumulated in word order into
// acc by four v_dot2_f32_bf16 (each adds the two bf16 products of one 32-bit
// word pair to acc).  One instruction per two pairs instead of six (unpack
// and fma); measured on gfx950 it matches the exactly rounded two-product
// sum more often than an fma chain does and keeps denormals.
__device__ __forceinline__ float dot2w(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), acc,
                                           false);
}
__device__ __forceinline__ float dot8(const uint4 a, const uint4 b, float acc) {
    acc = dot2w(a.x, b.x, acc);
    acc = dot2w(a.y, b.y, acc);
    acc = dot2w(a.z, b.z, acc);
    acc = dot2w(a.w, b.w, acc);
    return acc;
}

// ---------------------------------------------------------------- wave ops

// Sum over the wave by an xor butterfly, offsets 32, 16, 8, 4, 2, 1: each
// step adds lane a's value and lane a^d's, so after it the lanes that differ
// only in the bits already reduced hold identical values, and every lane
// ends with the same total.  The steps run without LDS: v_permlane32_swap /
// v_permlane16_swap hand each lane the value of lane a^32 / a^16 (in the
// one or the other output register, whose per-lane sum is then v_a +
// v_(a^d) in some operand order; fp32 addition commutes), and row_ror 8, 4,
// 2, 1 read a lane of the same 16-lane row that differs from a^d only in
// bits whose lanes already agree.  The result is bit-identical to the
// shuffle butterfly v += shfl_xor(v, d).
__device__ __forceinline__ float wave_sum(float v) {
    auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
    auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    v = v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, true));  // row_ror:8
    v = v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xf, 0xf, true));  // row_ror:4
    v = v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x122, 0xf, 0xf, true));  // row_ror:2
    v = v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x121, 0xf, 0xf, true));  // row_ror:1
    return v;
}

// Sums through DPP lane moves (no LDS round trips, unlike the shuffles
// above).  Fixed order: neighbours (xor 1), then pairs (xor 2) within quads,
// then lane i with 7-i of each half-row and with 15-i of each row, after
// which every lane of a 16-lane row holds the row sum; row_bcast 15 then
// adds row 0 into row 1 and row 2 into row 3 (rows 1 and 3 hold the sums of
// lanes 0-31 and 32-63), and row_bcast 31 adds lanes 0-31 into row 3.
// Lanes a move does not reach add +0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// sum of each 32-lane half: lanes 16-31 hold lanes 0-31's, lanes 48-63 lanes 32-63's
__device__ __forceinline__ float half_sum_dpp(float v) {
    v = dpp_add<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xf>(v);  // row_half_mirror
    v = dpp_add<0x140, 0xf>(v);  // row_mirror
    return dpp_add<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
}

// sum over the wave, returned to every lane
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = dpp_add<0x143, 0xc>(half_sum_dpp(v));  // row_bcast:31 into rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// exp(x) for x <= 0 with a fixed fp32 operation sequence: Cody-Waite
// reduction x = n*ln2 + r with ln2 split into a 13-bit head and a tail, the
// degree-7 Taylor polynomial of exp(r) in Horner form, and scaling by 2^n
// built in the exponent field.  Results below 2^-125 flush to 0, so the value
// never depends on the denormal mode.  The host-side oracle evaluates the
// same sequence, which makes routing probabilities reproducible bit for bit.
__device__ __forceinline__ float route_expf(float x) {
#pragma clang fp contract(off)
    const float log2e = 0x1.715476p+0f;
    const float ln2_hi = 0x1.62ep-1f;
    const float ln2_lo = 0x1.0bfbe8p-15f;
    float n = __builtin_rintf(x * log2e);
    if (!(n >= -125.0f)) return 0.0f;
    float r = __builtin_fmaf(-n, ln2_hi, x);
    r = __builtin_fmaf(-n, ln2_lo, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    float s = __uint_as_float((uint32_t)((int)n + 127) << 23);
    return p * s;
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

// silu with the hardware exp2 and reciprocal (about 1 ulp each): for epilogues
// whose result is rounded to bf16 right away
__device__ __forceinline__ float silu_fast(float g) {
    const float e = __builtin_amdgcn_exp2f(-g * 0x1.715476p+0f);
    return g * __builtin_amdgcn_rcpf(1.0f + e);
}

}  // namespace pd
