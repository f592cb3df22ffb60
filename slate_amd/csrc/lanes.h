// lanes.h -- cross-lane sums and maxima of a 64-lane wave built from DPP
// moves (quad_perm, row_half_mirror, row_mirror, row_ror) and lane reads,
// so they use no LDS crossbar traffic (ds_bpermute / ds_swizzle).
#pragma once
#include "common.h"

namespace slate_hip {

// v of the lane that DPP control CTRL names (all rows and banks enabled;
// every control used here names a lane inside the same 16-lane row).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

constexpr int DPP_QUAD_XOR1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;
constexpr int DPP_ROW_ROR8 = 0x128;

// Over each aligned group of 8 lanes; every lane of the group gets the result.
__device__ __forceinline__ float group8_sum(float v) {
    v += dpp_mov<DPP_QUAD_XOR1>(v);
    v += dpp_mov<DPP_QUAD_XOR2>(v);
    v += dpp_mov<DPP_ROW_HALF_MIRROR>(v);
    return v;
}
__device__ __forceinline__ float group8_max(float v) {
    v = fmaxf(v, dpp_mov<DPP_QUAD_XOR1>(v));
    v = fmaxf(v, dpp_mov<DPP_QUAD_XOR2>(v));
    v = fmaxf(v, dpp_mov<DPP_ROW_HALF_MIRROR>(v));
    return v;
}

// Over each 16-lane row; every lane of the row gets the result.
__device__ __forceinline__ float row16_sum(float v) {
    v = group8_sum(v);
    return v + dpp_mov<DPP_ROW_MIRROR>(v);
}
__device__ __forceinline__ float row16_max(float v) {
    v = group8_max(v);
    return fmaxf(v, dpp_mov<DPP_ROW_MIRROR>(v));
}

__device__ __forceinline__ float lane_read(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Over the whole wave (all lanes active); the result is wave-uniform.
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    return (lane_read(v, 0) + lane_read(v, 16)) + (lane_read(v, 32) + lane_read(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = row16_max(v);
    return fmaxf(fmaxf(lane_read(v, 0), lane_read(v, 16)), fmaxf(lane_read(v, 32), lane_read(v, 48)));
}

// Over the wave when v is the same in all lanes of each aligned 8-lane group
// (each group counted once).
__device__ __forceinline__ float wave_groups_sum(float v) {
    v += dpp_mov<DPP_ROW_ROR8>(v);
    return (lane_read(v, 0) + lane_read(v, 16)) + (lane_read(v, 32) + lane_read(v, 48));
}
__device__ __forceinline__ float wave_groups_max(float v) {
    v = fmaxf(v, dpp_mov<DPP_ROW_ROR8>(v));
    return fmaxf(fmaxf(lane_read(v, 0), lane_read(v, 16)), fmaxf(lane_read(v, 32), lane_read(v, 48)));
}

}  // namespace slate_hip
