// sidon_wave.h -- wavefront (64-lane) reductions for the library's kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace sidon {

// Sum of v over the 64 lanes, returned in every lane.  Within each row of 16
// lanes four DPP steps (quad swaps, half-row and row mirrors) leave the row
// sum in every lane of the row; the four row sums are then read as scalars.
// No LDS round trip, so independent reductions overlap freely.
template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), kCtrl, 0xf, 0xf, false));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<0xb1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_mov<0x4e>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  auto lane = [](float x, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
  };
  return (lane(v, 0) + lane(v, 16)) + (lane(v, 32) + lane(v, 48));
}

}  // namespace sidon
