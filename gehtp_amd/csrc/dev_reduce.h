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

__device__ __forceinline__ double read_lane(double v, int lane) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), lane);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Sum of all 64 lanes, the same value in every lane: 16-lane sums, then the four group
// sums added in lane order.
__device__ __forceinline__ double wave_sum(double v) {
    v = row_sum16(v);
    return ((read_lane(v, 0) + read_lane(v, 16)) + read_lane(v, 32)) + read_lane(v, 48);
}

}  // namespace dev
}  // namespace gehtp
