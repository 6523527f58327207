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

// Division by a divisor fixed for the whole launch, as a multiply-high and shifts (Granlund and
// Montgomery, "Division by invariant integers using multiplication", PLDI 1994, fig. 4.1):
// with l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1, for every 32-bit n
//   n / d = (t + ((n - t) >> min(l,1))) >> max(l-1,0),   t = mulhi(m, n).
// Integer division by a runtime value is a ~30-instruction sequence on the GPU; the fills
// decode three of them per probe.
struct FastDiv {
  uint32_t d = 1, m = 1;
  int s1 = 0, s2 = 0;
  static FastDiv make(uint32_t d) {
    FastDiv f;
    int l = 0;
    while (l < 32 && (uint64_t(1) << l) < d) ++l;
    f.d = d;
    f.m = (uint32_t)(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
    f.s1 = l < 1 ? l : 1;
    f.s2 = l > 1 ? l - 1 : 0;
    return f;
  }
  __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t t = __umulhi(m, n);
#else
    const uint32_t t = (uint32_t)(((uint64_t)m * n) >> 32);
#endif
    return (t + ((n - t) >> s1)) >> s2;
  }
};

// Splits a packed key into (column = (b*X + x)*Y + y, x, y, z).  32-bit keys use FastDiv; 64-bit
// keys (grids of 2^31 cells or more) divide directly.
template <typename K>
struct KeyCoder {
  int32_t X, Y, Z;
  FastDiv fx, fy, fz;
  static KeyCoder make(int32_t X, int32_t Y, int32_t Z) {
    return KeyCoder{X, Y, Z, FastDiv::make((uint32_t)X), FastDiv::make((uint32_t)Y),
                    FastDiv::make((uint32_t)Z)};
  }
  __device__ __forceinline__ void decode(K key, K* column, int32_t* x, int32_t* y,
                                         int32_t* z) const {
    if constexpr (sizeof(K) == 4) {
      const uint32_t k = (uint32_t)key;
      const uint32_t c = fz.div(k);
      const uint32_t by = fy.div(c);
      *column = (K)c;
      *z = (int32_t)(k - c * (uint32_t)Z);
      *y = (int32_t)(c - by * (uint32_t)Y);
      *x = (int32_t)(by - fx.div(by) * (uint32_t)X);
    } else {
      K t = key;
      *z = (int32_t)(t % (K)Z);
      t /= (K)Z;
      *column = t;
      *y = (int32_t)(t % (K)Y);
      t /= (K)Y;
      *x = (int32_t)(t % (K)X);
    }
  }
  __device__ __forceinline__ int32_t z_of(K key) const {
    if constexpr (sizeof(K) == 4) {
      const uint32_t k = (uint32_t)key;
      return (int32_t)(k - fz.div(k) * (uint32_t)Z);
    } else {
      return (int32_t)(key % (K)Z);
    }
  }
  __device__ __forceinline__ K column_of(K key) const {
    if constexpr (sizeof(K) == 4) return (K)fz.div((uint32_t)key);
    else return key / (K)Z;
  }
};

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
                        KeyCoder<K> kc_, int32_t dD, int32_t dH, int32_t dW,
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
  const int32_t X = kc_.X, Y = kc_.Y, Z = kc_.Z;
  K column;  // (b*X + x)*Y + y
  int32_t x, y, z;
  kc_.decode(key, &column, &x, &y, &z);
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
