// dpp.h - wave-level reductions with DPP lane permutations (no LDS
// round trip): quad swaps 0xB1/0x4E, row_half_mirror 0x141, row_mirror
// 0x140, row_bcast:15 0x142 (rows 1, 3) and row_bcast:31 0x143 (rows 2, 3).
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>

namespace eahmmf {

template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_fmax_step(float a, float fill) {
    return fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, fill),
                                                                          __builtin_bit_cast(int, a), CTRL, ROWS, 0xF,
                                                                          false)));
}

// wave64 max with DPP row operations; lane 63 collects the total, which is
// then broadcast.  Controls: 0xB1/0x4E quad permutes, 0x141 row_half_mirror,
// 0x140 row_mirror, 0x142 row_bcast:15 (rows 1,3), 0x143 row_bcast:31 (rows 2,3).
__device__ __forceinline__ float dpp_max(float v) {
    v = dpp_fmax_step<0xB1, 0xF>(v, v);
    v = dpp_fmax_step<0x4E, 0xF>(v, v);
    v = dpp_fmax_step<0x141, 0xF>(v, -INFINITY);
    v = dpp_fmax_step<0x140, 0xF>(v, -INFINITY);
    v = dpp_fmax_step<0x142, 0xA>(v, -INFINITY);
    v = dpp_fmax_step<0x143, 0xC>(v, -INFINITY);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// wave64 maximum of unsigned words with the same DPP steps (0 is the
// identity), returned in every lane.
__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// v + v of the lane DPP control CTRL names, in rows ROWS (others add 0).
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp_add_step(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xF,
                                                                     false));
}

// Sum over each aligned group of W lanes (W a power of two <= 64) with DPP
// steps: quad swaps, row_half_mirror, row_mirror, row_bcast:15 and :31.  The
// group's last lane holds the total (for W <= 16 every lane of the group).
template <int W>
__device__ __forceinline__ float group_sum(float v) {
    if (W >= 2) v = dpp_add_step<0xB1>(v);
    if (W >= 4) v = dpp_add_step<0x4E>(v);
    if (W >= 8) v = dpp_add_step<0x141>(v);
    if (W >= 16) v = dpp_add_step<0x140>(v);
    if (W >= 32) v = dpp_add_step<0x142, 0xA>(v);
    if (W >= 64) v = dpp_add_step<0x143, 0xC>(v);
    return v;
}

// The same for ints and a run-time group size T (uniform): the group's last
// lane holds the total.
__device__ __forceinline__ int group_sum_i(int v, int T) {
    if (T >= 2) v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
    if (T >= 4) v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
    if (T >= 8) v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
    if (T >= 16) v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);
    if (T >= 32) v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
    if (T >= 64) v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
    return v;
}

// group_sum with the total in every lane of the group.
template <int W>
__device__ __forceinline__ float group_sum_all(float v) {
    v = group_sum<W>(v);
    if constexpr (W == 64) {
        v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
    } else if constexpr (W == 32) {
        const float lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 31));
        const float hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
        v = (__lane_id() < 32) ? lo : hi;
    }
    return v;
}

}  // namespace eahmmf
