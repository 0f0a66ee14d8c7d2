// dev_reduce.h — cross-lane sums over DPP lane permutes (VALU only, no LDS traffic) for
// gfx950's 64-lane wavefronts. Every lane that takes part must be active; a 16-lane
// group is one DPP row (lanes 16j .. 16j+15).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace gehtp {
namespace dev {

// DPP controls used below (GCN/CDNA DPP encoding).
constexpr int kDppQuadSwap1 = 0xB1;       // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuadSwap2 = 0x4E;       // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppRowHalfMirror = 0x141;  // lane i <-> 7 - i within each 8 lanes
constexpr int kDppRowMirror = 0x140;      // lane i <-> 15 - i within each 16 lanes

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

template <int CTRL>
__device__ __forceinline__ double dpp(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Sum over each 16-lane group; every lane of the group gets the same value (each step
// adds the same two operands in every lane, in either order).
template <typename T>
__device__ __forceinline__ T row_sum16(T v) {
    v += dpp<kDppQuadSwap1>(v);
    v += dpp<kDppQuadSwap2>(v);
    v += dpp<kDppRowHalfMirror>(v);
    v += dpp<kDppRowMirror>(v);
    return v;
}

template <typename T>
__device__ __forceinline__ T row_max16(T v) {
    v = fmax(v, dpp<kDppQuadSwap1>(v));
    v = fmax(v, dpp<kDppQuadSwap2>(v));
    v = fmax(v, dpp<kDppRowHalfMirror>(v));
    v = fmax(v, dpp<kDppRowMirror>(v));
    return v;
}

__device__ __forceinline__ float read_lane(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ double read_lane(double v, int lane) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), lane);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Sum / max of all 64 lanes, the same value in every lane: 16-lane reductions, then
// the four group results combined in lane order.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
    v = row_sum16(v);
    return ((read_lane(v, 0) + read_lane(v, 16)) + read_lane(v, 32)) + read_lane(v, 48);
}

__device__ __forceinline__ float wave_max(float v) {
    v = row_max16(v);
    return fmaxf(fmaxf(read_lane(v, 0), read_lane(v, 16)), fmaxf(read_lane(v, 32), read_lane(v, 48)));
}

// max(a, b, c) as one v_max3_f32. fmaxf on values the compiler cannot prove canonical
// (MFMA results, for one) gets a NaN-quieting v_max_f32 x, x, x per operand first; for
// inputs that are never NaN this gives the same value in one instruction.
__device__ __forceinline__ float max3_nonan(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// v[l] + v[l^16] + v[l^32] + v[l^48] in every lane: the same position in the four
// 16-lane rows, summed with gfx950's row swaps (v_permlane32_swap: lanes 32-63 of the
// first operand trade with lanes 0-31 of the second; v_permlane16_swap: odd rows of the
// first trade with even rows of the second). With two copies of v as the operands,
// each lane ends up holding its partner's value in one of them. Written as inline asm
// with both registers read-write: the compiler builtin, given one value for both
// operands, treats its two results as equal and drops the partner. The s_nop covers
// the VALU-write -> permlane-read hazard, as the compiler's own lowering does.
__device__ __forceinline__ void permlane32_swap(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane16_swap(uint32_t& a, uint32_t& b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float cross_row_sum(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    permlane32_swap(a, b);
    v = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
    a = __builtin_bit_cast(uint32_t, v);
    b = a;
    permlane16_swap(a, b);
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
// v[l] + v[l^16] in every lane: the two 16-lane rows of each half-wave.
__device__ __forceinline__ float pair_row_sum(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    permlane16_swap(a, b);
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

}  // namespace dev
}  // namespace gehtp
