// Wavefront (64-lane) reductions through DPP lane moves and lane reads: no LDS round trips.
// The summation order is fixed (same instructions every call), so results are repeatable.
#pragma once
#include <hip/hip_runtime.h>

namespace lg {

template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over all 64 lanes; every lane receives the (wave-uniform) total.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]: pairs
  v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]: quads
  v += dpp_move<0x141>(v);  // row_half_mirror: 8 lanes
  v += dpp_move<0x140>(v);  // row_mirror: 16 lanes (each row holds its sum)
  return ((lane_value(v, 0) + lane_value(v, 16)) + lane_value(v, 32)) + lane_value(v, 48);
}

}  // namespace lg

namespace lg {

template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_move_rows(float v) {  // rows outside ROWS receive 0
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xF, false));
}

// Sum over each group of 8 consecutive lanes (every lane of the group receives it).
__device__ __forceinline__ float group8_sum(float v) {
  v += dpp_move<0xB1>(v);
  v += dpp_move<0x4E>(v);
  v += dpp_move<0x141>(v);
  return v;
}

// Sum over each 16-lane row (every lane of the row receives it).
__device__ __forceinline__ float row_sum(float v) {
  v = group8_sum(v);
  v += dpp_move<0x140>(v);
  return v;
}

// Maximum over each 16-lane row (every lane of the row receives it).
__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));
  v = fmaxf(v, dpp_move<0x4E>(v));
  v = fmaxf(v, dpp_move<0x141>(v));
  v = fmaxf(v, dpp_move<0x140>(v));
  return v;
}

// Native 4-float vector (register operand of the 16x16x4 f32 MFMA; copies stay in registers).
typedef float float4v __attribute__((ext_vector_type(4)));

// Sum over each 32-lane half of the wave; valid in rows 1 and 3 (lanes 16-31 and 48-63).
__device__ __forceinline__ float half_sum_odd_rows(float v) {
  v = row_sum(v);
  v += dpp_move_rows<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  return v;
}

// Maximum over all 64 lanes (wave-uniform result).
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));
  v = fmaxf(v, dpp_move<0x4E>(v));
  v = fmaxf(v, dpp_move<0x141>(v));
  v = fmaxf(v, dpp_move<0x140>(v));
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

}  // namespace lg
