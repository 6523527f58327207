// Pieces shared by the two neighbor-map builds (map_build.hip, map_radix.hip).
#pragma once

#include <algorithm>

#include "tsc_internal.h"

namespace tsc {
namespace mapk {

// key = ((b*X+x)*Y+y)*Z+z; false (and no key) when the voxel lies outside the grid.
template <typename K>
__device__ __forceinline__ bool pack_key(int4 c, int32_t B, int32_t X, int32_t Y, int32_t Z,
                                         K* key) {
  if ((uint32_t)c.x >= (uint32_t)B || (uint32_t)c.y >= (uint32_t)X ||
      (uint32_t)c.z >= (uint32_t)Y || (uint32_t)c.w >= (uint32_t)Z)
    return false;
  *key = (((K)c.x * X + c.y) * Y + c.z) * Z + c.w;
  return true;
}

// Column-parallel neighbor fill.  Each voxel (sorted position i) gets 9 lanes, one per neighbor
// column (kd, kh); a wave serves 7 voxels (63 lanes).  Lane (i, kd, kh) resolves the three z taps
// v = kd*9 + kh*3 + {0,1,2} through Lookup::column and writes them to nbr[row*27 + 3*(kd*3+kh)],
// so the 9 lanes of a voxel together write its 108-byte row.  Compared with one thread per voxel
// this puts 9x more independent probes in flight and needs no LDS staging.  Sorted positions are
// spread XCD-contiguously so each XCD's L2 holds one spatial region of the probed structures.
constexpr int kFillLanes = 9;
constexpr int kFillVoxPerWave = 7;
constexpr int kFillThreads = 256;
constexpr int kFillVoxPerBlock = kFillVoxPerWave * (kFillThreads / 64);

template <typename K, typename Lookup>
__global__ void __launch_bounds__(kFillThreads)
    fill_columns_kernel(const K* __restrict__ keys, const int32_t* __restrict__ perm,
                        const int* __restrict__ count_dev, int64_t count_host, K sentinel,
                        int32_t X, int32_t Y, int32_t Z, int32_t dD, int32_t dH, int32_t dW,
                        Lookup lk, int32_t per_xcd, int32_t* __restrict__ nbr,
                        uint32_t* __restrict__ status) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int slot = lane / kFillLanes, col = lane - slot * kFillLanes;
  if (slot >= kFillVoxPerWave) return;
  const int64_t logical = (int64_t)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  const int64_t i = (logical * (kFillThreads / 64) + wid) * kFillVoxPerWave + slot;
  const int64_t count = count_dev ? (int64_t)count_dev[0] : count_host;
  if (i >= count) return;
  const K key = keys[i];
  if (key == sentinel) {  // out-of-range voxel (radix path): reported, no row written
    if (col == 0) atomicOr(status, TSC_MAP_OUT_OF_RANGE);
    return;
  }
  if (status && col == 0 && i > 0 && keys[i - 1] == key) atomicOr(status, TSC_MAP_DUPLICATE);
  const int32_t row = perm[i];
  K t = key;
  const int32_t z = (int32_t)(t % (K)Z);
  t /= (K)Z;
  const K column = t;  // (b*X + x)*Y + y
  const int32_t y = (int32_t)(t % (K)Y);
  t /= (K)Y;
  const int32_t x = (int32_t)(t % (K)X);
  const int kd = col / 3, kh = col - kd * 3;
  const int32_t nx = x + (kd - 1) * dD, ny = y + (kh - 1) * dH;
  int32_t v[3] = {-1, -1, -1};
  if ((uint32_t)nx < (uint32_t)X && (uint32_t)ny < (uint32_t)Y) {
    // key of (nx, ny, z) in the same batch
    const K kc = (K)((int64_t)key + (int64_t)((kd - 1) * dD) * ((int64_t)Y * Z) +
                     (int64_t)((kh - 1) * dH) * Z);
    const K nc = (K)((int64_t)column + (int64_t)((kd - 1) * dD) * Y + (kh - 1) * dH);
    lk.column(kc, nc, z, Z, dW, v);
  }
  if (col == 4) v[1] = row;  // tap 13 is the voxel itself
  int32_t* dst = nbr + (int64_t)row * 27 + col * 3;
  dst[0] = v[0];
  dst[1] = v[1];
  dst[2] = v[2];
}

inline int32_t fill_per_xcd(int64_t n) {
  const int64_t blocks = (n + kFillVoxPerBlock - 1) / kFillVoxPerBlock;
  return (int32_t)((std::max<int64_t>(blocks, 1) + 7) / 8);
}

}  // namespace mapk
}  // namespace tsc
