// Neighbor-map build for submanifold 3x3x3 sparse convolution on gfx950.
//
// Semantics follow the reference's pass0/pass1 (src/sparse/ops/conv3d_wgsl.ts:44-128) and the
// Python hashmap_fallback (sorted flat_idx + searchsorted, README.md:111): for every voxel row n
// and tap v = kd*9+kh*3+kw, nbr[n*27+v] is the ORIGINAL row index of the voxel at
// (x+(kd-1)dD, y+(kh-1)dH, z+(kw-1)dW) in the same batch, or -1 when absent / out of
// [0,X)x[0,Y)x[0,Z).  The packed key includes the batch index: key = ((b*X+x)*Y+y)*Z+z.
//
// Bitmap path (grid of B*X*Y*Z cells small enough for a bitmap):
//   1. clear   : zero the occupancy bitmap (one bit per cell) and the status word
//   2. mark    : per voxel, atomicOr its bit; duplicates / out-of-range coords set status bits
//   3. scan    : exclusive prefix of popcounts per 128-bit group -> rank of every occupied cell
//                (the rank of a key is its position in the sorted unique key list)
//   4. place   : per voxel, sorted_keys[rank] = key, perm[rank] = row  (a counting sort)
//   5. fill    : per sorted position (spatially coherent lookups), 27 bitmap probes -> perm
// Algorithmic HBM bytes: 16 B/voxel coords in + 108 B/voxel table out + key-size B/voxel keys.

#include <algorithm>

#include "map_common.h"

namespace tsc {
namespace {

constexpr int kThreads = 256;
constexpr int kScanItems = 4;                       // 128-bit groups per thread in the scan
constexpr int kScanTile = kThreads * kScanItems;    // groups per scan block

__device__ __forceinline__ int popc4_below(uint4 w, uint32_t word, uint32_t bit) {
  // Number of set bits in group w strictly below (word, bit).
  uint32_t m = (bit == 0) ? 0u : (0xffffffffu >> (32 - bit));
  int r = 0;
  r += (word > 0) ? __popc(w.x) : __popc(w.x & m);
  if (word >= 1) r += (word > 1) ? __popc(w.y) : __popc(w.y & m);
  if (word >= 2) r += (word > 2) ? __popc(w.z) : __popc(w.z & m);
  if (word >= 3) r += __popc(w.w & m);
  return r;
}

__device__ __forceinline__ uint32_t pick_word(uint4 w, uint32_t word) {
  return word == 0 ? w.x : word == 1 ? w.y : word == 2 ? w.z : w.w;
}

__global__ void __launch_bounds__(kThreads) clear_kernel(uint4* __restrict__ bits, int64_t groups,
                                                         uint32_t* __restrict__ status) {
  int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x;
  if (i == 0) status[0] = 0u;
  int64_t stride = (int64_t)gridDim.x * kThreads;
  for (; i < groups; i += stride) bits[i] = make_uint4(0u, 0u, 0u, 0u);
}

template <typename K>
__device__ __forceinline__ bool pack_key(int4 c, int32_t B, int32_t X, int32_t Y, int32_t Z,
                                         K* key) {
  if ((uint32_t)c.x >= (uint32_t)B || (uint32_t)c.y >= (uint32_t)X ||
      (uint32_t)c.z >= (uint32_t)Y || (uint32_t)c.w >= (uint32_t)Z)
    return false;
  *key = (((K)c.x * X + c.y) * Y + c.z) * Z + c.w;
  return true;
}

template <typename K>
__global__ void __launch_bounds__(kThreads)
    mark_kernel(const int4* __restrict__ coords, int64_t N, int32_t B, int32_t X, int32_t Y,
                int32_t Z, uint32_t* __restrict__ words, uint32_t* __restrict__ status) {
  int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x;
  if (i >= N) return;
  K key;
  if (!pack_key<K>(coords[i], B, X, Y, Z, &key)) {
    atomicOr(status, TSC_MAP_OUT_OF_RANGE);
    return;
  }
  uint32_t bit = 1u << (uint32_t)(key & 31);
  uint32_t old = atomicOr(&words[key >> 5], bit);
  if (old & bit) atomicOr(status, TSC_MAP_DUPLICATE);
}

__device__ __forceinline__ int group_popc(uint4 w) {
  return __popc(w.x) + __popc(w.y) + __popc(w.z) + __popc(w.w);
}

// Inclusive wave64 scan.
__device__ __forceinline__ int wave_incl_scan(int v) {
  int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int t = __shfl_up(v, off, 64);
    if (lane >= off) v += t;
  }
  return v;
}

// Block-wide exclusive scan of one int per thread (kThreads threads); returns the exclusive
// prefix and writes the block total to *total.
__device__ __forceinline__ int block_excl_scan(int v, int* total) {
  __shared__ int wsum[kThreads / 64];
  int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  int incl = wave_incl_scan(v);
  if (lane == 63) wsum[wid] = incl;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) {
    int s = wsum[w];
    if (w < wid) base += s;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return base + incl - v;
}

__global__ void __launch_bounds__(kThreads)
    scan_reduce_kernel(const uint4* __restrict__ bits, int64_t groups, int* __restrict__ blk_sums) {
  int64_t g0 = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
  int s = 0;
#pragma unroll
  for (int j = 0; j < kScanItems; ++j)
    if (g0 + j < groups) s += group_popc(bits[g0 + j]);
  int total;
  block_excl_scan(s, &total);
  if (threadIdx.x == 0) blk_sums[blockIdx.x] = total;
}

// Single block: exclusive scan of blk_sums in place; count[0] = grand total.
__global__ void __launch_bounds__(1024) scan_blocks_kernel(int* __restrict__ blk_sums, int nblk,
                                                           int* __restrict__ count) {
  __shared__ int wsum[16];
  __shared__ int carry_s;
  if (threadIdx.x == 0) carry_s = 0;
  __syncthreads();
  int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  for (int base = 0; base < nblk; base += 1024) {
    int i = base + threadIdx.x;
    int v = (i < nblk) ? blk_sums[i] : 0;
    int incl = wave_incl_scan(v);
    if (lane == 63) wsum[wid] = incl;
    __syncthreads();
    int pre = 0, tot = 0;
    for (int w = 0; w < 16; ++w) {
      if (w < wid) pre += wsum[w];
      tot += wsum[w];
    }
    int carry = carry_s;
    if (i < nblk) blk_sums[i] = carry + pre + incl - v;
    __syncthreads();
    if (threadIdx.x == 0) carry_s = carry + tot;
    __syncthreads();
  }
  if (threadIdx.x == 0) count[0] = carry_s;
}

__global__ void __launch_bounds__(kThreads)
    scan_down_kernel(const uint4* __restrict__ bits, int64_t groups,
                     const int* __restrict__ blk_offs, int* __restrict__ prefix) {
  int64_t g0 = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
  int c[kScanItems];
  int s = 0;
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) {
    c[j] = (g0 + j < groups) ? group_popc(bits[g0 + j]) : 0;
    s += c[j];
  }
  int total;
  int run = blk_offs[blockIdx.x] + block_excl_scan(s, &total);
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) {
    if (g0 + j < groups) prefix[g0 + j] = run;
    run += c[j];
  }
}

template <typename K>
__device__ __forceinline__ int rank_of(K key, const uint4* __restrict__ bits,
                                       const int* __restrict__ prefix, bool* present) {
  int64_t g = (int64_t)(key >> 7);
  uint4 w = bits[g];
  uint32_t word = (uint32_t)(key >> 5) & 3u, bit = (uint32_t)key & 31u;
  *present = (pick_word(w, word) >> bit) & 1u;
  return prefix[g] + popc4_below(w, word, bit);
}

template <typename K>
__global__ void __launch_bounds__(kThreads)
    place_kernel(const int4* __restrict__ coords, int64_t N, int32_t B, int32_t X, int32_t Y,
                 int32_t Z, const uint4* __restrict__ bits, const int* __restrict__ prefix,
                 K* __restrict__ keys, int32_t* __restrict__ perm) {
  int64_t i = blockIdx.x * (int64_t)kThreads + threadIdx.x;
  if (i >= N) return;
  K key;
  if (!pack_key<K>(coords[i], B, X, Y, Z, &key)) return;
  bool present;
  int r = rank_of<K>(key, bits, prefix, &present);
  keys[r] = key;
  perm[r] = (int32_t)i;
}

// Bitmap probe for the column-parallel fill: one 16-byte group load plus its prefix serves the
// three z taps of a neighbor column (a second group only when a tap crosses a 128-cell
// boundary); present cells read their original row through perm[rank].
template <typename K>
struct BitmapLookup {
  const uint4* __restrict__ bits;
  const int* __restrict__ prefix;
  const int32_t* __restrict__ perm;
  __device__ __forceinline__ void column(K kc, K /*column id*/, int32_t z, int32_t Z, int32_t dW,
                                         int32_t v[3]) const {
    const int64_t g = (int64_t)(kc >> 7);
    const uint4 w = bits[g];
    const int p = prefix[g];
#pragma unroll
    for (int kw = 0; kw < 3; ++kw) {
      const int32_t nz = z + (kw - 1) * dW;
      if (kw == 1 || (uint32_t)nz >= (uint32_t)Z) continue;  // centre handled below
      const K kt = (K)((int64_t)kc + (kw - 1) * dW);
      const int64_t gt = (int64_t)(kt >> 7);
      uint4 wt = w;
      int pt = p;
      if (gt != g) {
        wt = bits[gt];
        pt = prefix[gt];
      }
      const uint32_t word = (uint32_t)(kt >> 5) & 3u, bit = (uint32_t)kt & 31u;
      if ((pick_word(wt, word) >> bit) & 1u) v[kw] = perm[pt + popc4_below(wt, word, bit)];
    }
    const uint32_t word = (uint32_t)(kc >> 5) & 3u, bit = (uint32_t)kc & 31u;
    if ((pick_word(w, word) >> bit) & 1u) v[1] = perm[p + popc4_below(w, word, bit)];
  }
};

inline unsigned grid_for(int64_t n, int per_block) {
  int64_t b = (n + per_block - 1) / per_block;
  return (unsigned)(b < 1 ? 1 : b);
}

template <typename K>
int bitmap_impl(tsc_ctx* ctx, const int32_t* coords, int64_t N, int32_t B, int32_t X, int32_t Y,
                int32_t Z, const int32_t dil[3], void* keys_out, int32_t* perm_out,
                int32_t* nbr_out, uint32_t* status_dev) {
  const int64_t cells = (int64_t)B * X * Y * Z;
  const int64_t groups = (cells + 127) / 128;
  const int64_t nblk = (groups + kScanTile - 1) / kScanTile;
  // Workspace: bitmap, prefix, block sums, count, and keys/perm when the caller wants none.
  size_t need = align_up((size_t)groups * 16, 256) + align_up((size_t)groups * 4, 256) +
                align_up((size_t)nblk * 4, 256) + 256;
  if (!keys_out) need += align_up((size_t)N * sizeof(K), 256);
  if (!perm_out) need += align_up((size_t)N * 4, 256);
  void* ws;
  int st = workspace(ctx, need, &ws);
  if (st) return st;
  Carve cv(ws);
  uint4* bits = cv.take<uint4>(groups);
  int* prefix = cv.take<int>(groups);
  int* blk = cv.take<int>(nblk);
  int* count = cv.take<int>(64);
  K* keys = keys_out ? (K*)keys_out : cv.take<K>(N);
  int32_t* perm = perm_out ? perm_out : cv.take<int32_t>(N);

  hipStream_t s = ctx->stream;
  unsigned clear_blocks = (unsigned)std::min<int64_t>((groups + kThreads - 1) / kThreads, 4096);
  if (clear_blocks < 1) clear_blocks = 1;
  {
    ProfScope p(ctx, "map_clear");
    clear_kernel<<<clear_blocks, kThreads, 0, s>>>(bits, groups, status_dev);
  }
  if (N > 0) {
    ProfScope p(ctx, "map_mark");
    mark_kernel<K><<<grid_for(N, kThreads), kThreads, 0, s>>>((const int4*)coords, N, B, X, Y, Z,
                                                             (uint32_t*)bits, status_dev);
  }
  {
    ProfScope p(ctx, "map_scan_reduce");
    scan_reduce_kernel<<<(unsigned)nblk, kThreads, 0, s>>>(bits, groups, blk);
  }
  {
    ProfScope p(ctx, "map_scan_blocks");
    scan_blocks_kernel<<<1, 1024, 0, s>>>(blk, (int)nblk, count);
  }
  {
    ProfScope p(ctx, "map_scan_down");
    scan_down_kernel<<<(unsigned)nblk, kThreads, 0, s>>>(bits, groups, blk, prefix);
  }
  if (N > 0) {
    {
      ProfScope p(ctx, "map_place");
      place_kernel<K><<<grid_for(N, kThreads), kThreads, 0, s>>>(
          (const int4*)coords, N, B, X, Y, Z, bits, prefix, keys, perm);
    }
    ProfScope p(ctx, "map_fill");
    const int32_t per_xcd = mapk::fill_per_xcd(N);
    mapk::fill_columns_kernel<K, BitmapLookup<K>><<<(unsigned)per_xcd * 8u, mapk::kFillThreads, 0, s>>>(
        keys, perm, count, 0, (K)-1, mapk::KeyCoder<K>::make(X, Y, Z), dil[0], dil[1], dil[2],
        BitmapLookup<K>{bits, prefix, perm}, per_xcd, nbr_out, nullptr);
  }
  return check_hip(hipGetLastError(), "map_build_bitmap launch");
}

}  // namespace

int map_build_bitmap(tsc_ctx* ctx, const int32_t* coords, int64_t N, int32_t B, int32_t X,
                     int32_t Y, int32_t Z, const int32_t dil[3], void* keys_out, int32_t* perm_out,
                     int32_t* nbr_out, uint32_t* status_dev) {
  const int64_t cells = (int64_t)B * X * Y * Z;
  if (cells < (int64_t(1) << 31))
    return bitmap_impl<int32_t>(ctx, coords, N, B, X, Y, Z, dil, keys_out, perm_out, nbr_out,
                                status_dev);
  return bitmap_impl<int64_t>(ctx, coords, N, B, X, Y, Z, dil, keys_out, perm_out, nbr_out,
                              status_dev);
}

}  // namespace tsc
