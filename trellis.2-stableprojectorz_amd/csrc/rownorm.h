// Device helpers shared by the LayerNorm row pass (rowops.hip) and the conv epilogue that
// normalizes whole rows (conv.hip), so that both compute the same bits: the wave64 butterfly sum
// and SiLU as x * 1/(1+exp(-x)) (src/dense/ops/silu.ts:25-29).
#pragma once

#include <hip/hip_runtime.h>

namespace tsc {

__device__ __forceinline__ float rn_wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// The butterfly restricted to aligned groups of G lanes.  When only the first n <= G lanes of a
// group hold nonzero values it returns the bits rn_wave_sum returns for those values in lanes
// 0..n-1 of a wave: the wave's wider steps only add exact zeros.
template <int G>
__device__ __forceinline__ float rn_group_sum(float v) {
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float rn_silu(float x) { return x * (1.0f / (1.0f + __expf(-x))); }

}  // namespace tsc
