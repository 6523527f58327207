// Neighbor-map build by radix sort of packed keys (no global atomics, no grid-sized memsets).
//
// Same outputs as the bitmap path (sorted unique keys, their rows, the (N,27) neighbor table; see
// map_build.hip for the semantics and reference citations).  Keys have nbits = bitlen(cells-1)
// bits; the top TB = min(nbits, 10) bits select one of 2^TB buckets.  Steps of the map build (up
// to 2048 tiles of 8192 voxels, i.e. 16.7 M voxels):
//   pack_sort  coords -> (key, row), reordered inside each 8192-row tile by bucket digit and
//              written back over the tile, with the tile's digit starts and an out-of-range flag
//              (out-of-range coordinates are clamped to the last cell, so every key stays below
//              2^nbits, and reported through the flag).
//   bucket     one block per bucket: gathers the bucket's run from every tile, sorts it by an
//              LDS bitmap of its key range (rank = set bits below; stable LSD passes for repeated
//              keys or buckets past 65536) and writes the sorted keys and rows, plus col_start[c]
//              for the (b,x,y) columns whose first key c*Z falls in the bucket's key range; block
//              0 folds the tile flags into the status word.
//   fill       window fill from LDS (below), or the column-parallel fill over the whole sorted
//              array when the column table would be much larger than the voxel set.
// Larger sets, and the gather plan's Morton sort (sort_rows_morton, no column starts; its buckets
// are uneven), run pack (histograms only), scan (per-bucket offsets over tiles), partition
// (scatter into contiguous buckets) and the same bucket kernel reading the partitioned copy.

#include <algorithm>
#include <type_traits>

#include "map_common.h"

namespace tsc {
namespace {

constexpr int RT = 256;             // threads per block
constexpr int RI = 16;              // items per thread
constexpr int RTILE = RT * RI;      // elements per tile
constexpr int WAVES = RT / 64;
constexpr int TBMAX = 10;           // bucket digit bits
constexpr int NBMAX = 1 << TBMAX;   // buckets
constexpr int LBITS = 9;            // local pass digit bits
constexpr int LNB = 1 << LBITS;
constexpr int LPT = LNB / RT;       // local digits owned per thread
constexpr int PT = 1024;            // pack / partition threads per block
constexpr int PI = 8;               // pack / partition items per thread (512 x 16: Morton pack
                                    // 19.6 -> 14.7 us at 1.5 M voxels, the others equal)
constexpr int PTILE = PT * PI;      // pack / partition tile

template <typename K>
__device__ __forceinline__ int digit_of(K k, int shift, int mask) {
  return (int)((k >> shift) & (K)mask);
}

__global__ void clear_status_kernel(uint32_t* status) {
  if (threadIdx.x == 0) status[0] = 0u;
}

// Key generators for pack_kernel.  PackedKey: the (b, x, y, z) cell index of the neighbor map,
// clamped to the last cell (and reported) when out of range.  MortonKey: the gather plan's
// (batch, Z-curve) key over the low `bits` bits of x, y, z (z lowest), its lowest `shift` bits
// dropped when the pair is wider than 64 bits, masked to the sort's key width.
template <typename K>
struct PackedKey {
  int32_t B, X, Y, Z;
  K last_cell;
  __device__ __forceinline__ bool operator()(int4 c, K* key) const {
    if (mapk::pack_key<K>(c, B, X, Y, Z, key)) return true;
    *key = last_cell;
    return false;
  }
};

// Spreads the low 21 bits of v to every third bit (bit i -> bit 3i), by the shift-and-mask
// sequence of "bit interleaving by magic numbers" (each step halves the width of the groups).
__device__ __forceinline__ uint64_t spread3(uint32_t v) {
  uint64_t x = v & 0x1fffffu;
  x = (x | x << 32) & 0x001f00000000ffffull;
  x = (x | x << 16) & 0x001f0000ff0000ffull;
  x = (x | x << 8) & 0x100f00f00f00f00full;
  x = (x | x << 4) & 0x10c30c30c30c30c3ull;
  x = (x | x << 2) & 0x1249249249249249ull;
  return x;
}

template <typename K>
struct MortonKey {
  int bits, shift;
  uint64_t mask;
  __device__ __forceinline__ bool operator()(int4 c, K* key) const {
    const uint32_t lo = (uint32_t)((1u << bits) - 1u);
    const uint64_t m = spread3((uint32_t)c.w & lo) | spread3((uint32_t)c.z & lo) << 1 |
                       spread3((uint32_t)c.y & lo) << 2;
    const uint64_t k = ((uint64_t)(uint32_t)c.x << (3 * bits - shift)) | (m >> shift);
    *key = (K)(k & mask);
    return true;
  }
};

template <typename K, typename Gen>
__global__ void __launch_bounds__(PT)
    pack_kernel(const int4* __restrict__ coords, int64_t N, Gen gen, K* __restrict__ keys,
                int32_t* __restrict__ vals, int shift, int dbits, int* __restrict__ counts,
                int ntiles, int* __restrict__ oob_tile) {
  __shared__ int hist[NBMAX];
  const int nb = 1 << dbits, mask = nb - 1;
  for (int d = threadIdx.x; d < nb; d += PT) hist[d] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * PTILE;
  int oob = 0;
  // All PI coordinate loads are issued before the first store, and full tiles run without
  // per-item branches: one vmcnt counts loads and stores, and across branches the compiler
  // falls back to waiting for everything, which would serialise the items on store latency.
  int4 c[PI];
  auto item = [&](int j, int64_t e) {
    K key;
    if (!gen(c[j], &key)) oob = 1;
    keys[e] = key;
    vals[e] = (int32_t)e;
    atomicAdd(&hist[digit_of<K>(key, shift, mask)], 1);  // LDS atomic
  };
  if (base + PTILE <= N) {
#pragma unroll
    for (int j = 0; j < PI; ++j) c[j] = coords[base + j * PT + threadIdx.x];
#pragma unroll
    for (int j = 0; j < PI; ++j) item(j, base + j * PT + threadIdx.x);
  } else {
#pragma unroll
    for (int j = 0; j < PI; ++j) {
      const int64_t e = base + j * PT + threadIdx.x;
      c[j] = e < N ? coords[e] : make_int4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < PI; ++j) {
      const int64_t e = base + j * PT + threadIdx.x;
      if (e < N) item(j, e);
    }
  }
  oob = __syncthreads_or(oob);
  for (int d = threadIdx.x; d < nb; d += PT) counts[(int64_t)d * ntiles + blockIdx.x] = hist[d];
  if (threadIdx.x == 0) oob_tile[blockIdx.x] = oob;
}

__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(v, off, 64);
    if (lane >= off) v += t;
  }
  return v;
}

// Exclusive scan of v over the block's NW waves; *total receives the block sum.
template <int NW = WAVES>
__device__ __forceinline__ int block_excl_scan(int v, int* wsum, int* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int incl = wave_incl_scan(v);
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  int pre = incl - v, tot = 0;
#pragma unroll
  for (int ww = 0; ww < NW; ++ww) {
    if (ww < w) pre += wsum[ww];
    tot += wsum[ww];
  }
  __syncthreads();
  *total = tot;
  return pre;
}

// Block d: exclusive scan over tiles of bucket d's counts (in place) and totals[d] = its sum.
// Block 0 also sets the status word from the pack kernel's out-of-range tile flags (the fill
// adds the duplicate bit later in stream order).
__global__ void __launch_bounds__(RT)
    scan_kernel(int* __restrict__ counts, int ntiles, int* __restrict__ totals,
                const int* __restrict__ oob_tile, uint32_t* __restrict__ status) {
  __shared__ int wsum[WAVES];
  int* c = counts + (int64_t)blockIdx.x * ntiles;
  int carry = 0;
  for (int base = 0; base < ntiles; base += RT) {
    const int i = base + threadIdx.x;
    const int v = (i < ntiles) ? c[i] : 0;
    int tot;
    const int pre = block_excl_scan(v, wsum, &tot);
    if (i < ntiles) c[i] = carry + pre;
    carry += tot;
  }
  if (threadIdx.x == 0) totals[blockIdx.x] = carry;
  if (blockIdx.x == 0) {
    int any = 0;
    for (int i = threadIdx.x; i < ntiles; i += RT) any |= oob_tile[i];
    any = __syncthreads_or(any);
    if (threadIdx.x == 0) status[0] = any ? (uint32_t)TSC_MAP_OUT_OF_RANGE : 0u;
  }
}

// Stable ranks of one wave's RI items (lanes = consecutive elements, items in order) among equal
// digits: peers = lanes with the same digit (one ballot per digit bit), rank = popcount of the
// lower peers + the wave's running count of that digit (cnt, in LDS, advanced by the first peer).
template <typename K, int N_ITEMS>
__device__ __forceinline__ void wave_rank(const K (&kk)[N_ITEMS], int64_t first, int64_t limit,
                                          int shift, int dbits, int* cnt, int (&lr)[N_ITEMS]) {
  const int lane = threadIdx.x & 63;
  const int mask = (1 << dbits) - 1;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int j = 0; j < N_ITEMS; ++j) {
    const bool valid = first + j * 64 + lane < limit;
    const int d = digit_of<K>(kk[j], shift, mask);
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < dbits; ++b) {
      const bool bit = (d >> b) & 1;
      const uint64_t m = __ballot(valid && bit);
      peers &= bit ? m : ~m;
    }
    lr[j] = 0;
    if (valid) {
      const int before = __popcll(peers & lt_mask);
      const int c = cnt[d];
      lr[j] = c + before;
      if (before == 0) cnt[d] = c + __popcll(peers);
    }
  }
}

// Partition by bucket digit.  Order inside a bucket does not matter (the bucket kernel sorts it
// completely), so an element's slot among its tile's elements of the same digit comes from an
// LDS atomic.  The tile is reordered by digit in LDS and written as contiguous runs at
// (all elements of smaller digits) + (this digit in earlier tiles).
template <typename K>
__global__ void __launch_bounds__(PT)
    partition_kernel(const K* __restrict__ ksrc, const int32_t* __restrict__ vsrc, int64_t N,
                     int shift, int dbits, const int* __restrict__ offs,
                     const int* __restrict__ totals, int ntiles, K* __restrict__ kdst,
                     int32_t* __restrict__ vdst, int* __restrict__ bstart) {
  constexpr int PDPT = NBMAX / PT;  // bucket digits owned per thread in the prefix
  __shared__ int lcnt[NBMAX];
  __shared__ int dstart[NBMAX];
  __shared__ int gbase[NBMAX];
  __shared__ int wsum[PT / 64];
  __shared__ K sk[PTILE];
  __shared__ int32_t sv[PTILE];
  const int nb = 1 << dbits, mask = nb - 1;
  const int tid = threadIdx.x;
  for (int i = tid; i < NBMAX; i += PT) lcnt[i] = 0;
  __syncthreads();
  const int64_t tile0 = (int64_t)blockIdx.x * PTILE;
  K kk[PI];
  int32_t vv[PI];
  int slot[PI];
#pragma unroll
  for (int j = 0; j < PI; ++j) {
    const int64_t e = tile0 + j * PT + tid;
    const bool valid = e < N;
    kk[j] = valid ? ksrc[e] : (K)0;
    vv[j] = valid ? vsrc[e] : 0;
  }
#pragma unroll
  for (int j = 0; j < PI; ++j) {
    const int64_t e = tile0 + j * PT + tid;
    slot[j] = e < N ? atomicAdd(&lcnt[digit_of<K>(kk[j], shift, mask)], 1) : 0;
  }
  __syncthreads();
  // Thread t owns digits [t*PDPT, (t+1)*PDPT): tile-local start of each digit and its global start.
  int loc[PDPT];
  int tsum = 0, gsum = 0;
#pragma unroll
  for (int q = 0; q < PDPT; ++q) {
    const int d = tid * PDPT + q;
    loc[q] = lcnt[d];
    tsum += loc[q];
    gsum += d < nb ? totals[d] : 0;
  }
  int dummy;
  int pre = block_excl_scan<PT / 64>(tsum, wsum, &dummy);
  int gpre = block_excl_scan<PT / 64>(gsum, wsum, &dummy);
#pragma unroll
  for (int q = 0; q < PDPT; ++q) {
    const int d = tid * PDPT + q;
    dstart[d] = pre;
    pre += loc[q];
    if (d < nb) {
      gbase[d] = gpre + offs[(int64_t)d * ntiles + blockIdx.x];
      if (blockIdx.x == 0) bstart[d] = gpre;  // bucket start, for the bucket kernel
      gpre += totals[d];
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < PI; ++j) {
    const int64_t e = tile0 + j * PT + tid;
    if (e < N) {
      const int p = dstart[digit_of<K>(kk[j], shift, mask)] + slot[j];
      sk[p] = kk[j];
      sv[p] = vv[j];
    }
  }
  __syncthreads();
  const int64_t rem = N - tile0;
  const int tile_n = rem < PTILE ? (int)rem : PTILE;
  for (int i = tid; i < tile_n; i += PT) {
    const K k = sk[i];
    const int d = digit_of<K>(k, shift, mask);
    const int64_t pos = (int64_t)gbase[d] + (i - dstart[d]);
    kdst[pos] = k;
    vdst[pos] = sv[i];
  }
}

// Gather pipeline (at most kGatherTiles tiles): pack and a tile-local sort by bucket digit in one
// kernel.  The tile's (key, row) pairs are formed as in pack_kernel, reordered by digit in LDS
// (slots from LDS atomics, as in partition_kernel) and written back over the tile's own range as
// one coalesced run.  toff[tile * (nb + 1) + d] = the tile's first position of digit d (d <= nb,
// toff[nb] = the tile's size), so bucket d's elements are the runs [toff[d], toff[d + 1]) of
// every tile, and its start in the sorted output is the sum of the tiles' toff[d].  No global
// scatter and no scan launch: the bucket kernel gathers the runs itself.
constexpr int kGatherTiles = 2048;  // runs per bucket: 8 per thread of the bucket kernel

template <typename K, typename Gen>
__global__ void __launch_bounds__(PT)
    pack_sort_kernel(const int4* __restrict__ coords, int64_t N, Gen gen, int shift, int dbits,
                     K* __restrict__ ktile, int32_t* __restrict__ vtile, int* __restrict__ toff,
                     int ntiles, int* __restrict__ oob_tile) {
  constexpr int PDPT = NBMAX / PT;
  __shared__ int lcnt[NBMAX];
  __shared__ int dstart[NBMAX];
  __shared__ int wsum[PT / 64];
  __shared__ K sk[PTILE];
  __shared__ int32_t sv[PTILE];
  const int nb = 1 << dbits, mask = nb - 1;
  const int tid = threadIdx.x;
  for (int i = tid; i < NBMAX; i += PT) lcnt[i] = 0;
  __syncthreads();
  const int64_t tile0 = (int64_t)blockIdx.x * PTILE;
  const int64_t rem = N - tile0;
  const int tile_n = rem < PTILE ? (int)rem : PTILE;
  // Every coordinate load is issued before the first use (indices past the tile re-read its
  // last element, never used).
  int4 c[PI];
#pragma unroll
  for (int j = 0; j < PI; ++j) c[j] = coords[tile0 + min(j * PT + tid, tile_n - 1)];
  K kk[PI];
  int slot[PI];
  int oob = 0;
#pragma unroll
  for (int j = 0; j < PI; ++j) {
    K key = (K)0;
    slot[j] = 0;
    if (j * PT + tid < tile_n) {
      if (!gen(c[j], &key)) oob = 1;
      slot[j] = atomicAdd(&lcnt[digit_of<K>(key, shift, mask)], 1);  // LDS atomic
    }
    kk[j] = key;
  }
  oob = __syncthreads_or(oob);
  // Tile-local digit starts: thread t owns digits [t*PDPT, (t+1)*PDPT).
  int loc[PDPT];
  int tsum = 0;
#pragma unroll
  for (int q = 0; q < PDPT; ++q) {
    const int d = tid * PDPT + q;
    loc[q] = d < nb ? lcnt[d] : 0;
    tsum += loc[q];
  }
  int dummy;
  int pre = block_excl_scan<PT / 64>(tsum, wsum, &dummy);
#pragma unroll
  for (int q = 0; q < PDPT; ++q) {
    const int d = tid * PDPT + q;
    if (d < nb) {
      dstart[d] = pre;
      toff[(int64_t)blockIdx.x * (nb + 1) + d] = pre;
    }
    pre += loc[q];
  }
  if (tid == 0) {
    toff[(int64_t)blockIdx.x * (nb + 1) + nb] = tile_n;
    oob_tile[blockIdx.x] = oob;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < PI; ++j) {
    const int i = j * PT + tid;
    if (i < tile_n) {
      const int p = dstart[digit_of<K>(kk[j], shift, mask)] + slot[j];
      sk[p] = kk[j];
      sv[p] = (int32_t)(tile0 + i);
    }
  }
  __syncthreads();
  for (int i = tid; i < tile_n; i += PT) {
    ktile[tile0 + i] = sk[i];
    vtile[tile0 + i] = sv[i];
  }
}

// First index in [lo, hi) with keys[idx] >= t.
template <typename K>
__device__ __forceinline__ int64_t lower_bound(const K* keys, int64_t lo, int64_t hi, K t) {
  while (lo < hi) {
    const int64_t mid = lo + ((hi - lo) >> 1);
    if (keys[mid] < t) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// Exclusive scan of the LNB-bin histogram in run[] (in place), LPT bins per thread.
__device__ __forceinline__ void scan_bins(int* run, int* wsum) {
  const int tid = threadIdx.x;
  int c[LPT], sum = 0;
#pragma unroll
  for (int q = 0; q < LPT; ++q) {
    c[q] = run[tid * LPT + q];
    sum += c[q];
  }
  int tot;
  int pre = block_excl_scan(sum, wsum, &tot);
#pragma unroll
  for (int q = 0; q < LPT; ++q) {
    run[tid * LPT + q] = pre;
    pre += c[q];
  }
}

// wcnt[w][d] (each wave's count of digit d) -> each wave's exclusive offset among the waves;
// returns the per-thread totals of its LPT digits in cnt.
__device__ __forceinline__ void wave_offsets(int (*wcnt)[LNB], int (&cnt)[LPT]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int q = 0; q < LPT; ++q) {
    const int d = tid * LPT + q;
    int r = 0;
#pragma unroll
    for (int ww = 0; ww < WAVES; ++ww) {
      const int x = wcnt[ww][d];
      wcnt[ww][d] = r;
      r += x;
    }
    cnt[q] = r;
  }
}

// One block per bucket b (see the file comment).  The bucket occupies [start, start+size) of
// (k0, v0) after the partition.
//  * size <= 65536 and lb <= kBitmapBits (every int32-key grid up to 2^27 cells): each thread
//    sets bit (key mod 2^lb) of an LDS bitmap of the bucket's key range for its elements (held
//    in registers up to RTILE elements, else read in chunks of RTILE).  With unique keys an
//    element's sorted position is the number of set bits below its own (per-word prefix counts
//    + one popcount), and so is every column start:
//    col_start[c] = start + (set bits below c*Z - (b << lb)).
//  * otherwise, or when the bitmap finds a repeated key: stable LSD passes over the bucket's
//    remaining bits (at most 9 per pass) through global memory in chunks of RTILE (histogram of
//    the pass digit, exclusive scan, wave_rank over wave-contiguous runs, scatter), alternating
//    between (k0, v0) and (k1, v1), the last pass writing (kout, vout); equal keys end up
//    adjacent for the fill's duplicate check.  Column starts then come from binary searches of
//    the sorted bucket.
constexpr int kBitmapBits = 17;
constexpr int kBitmapWords = (1 << kBitmapBits) / 32;

// Source of the buckets in the gather pipeline: pack_sort_kernel's tile-sorted pairs and digit
// starts (ktile == nullptr: the partitioned layout, bucket b at [bstart[b], + totals[b]) of k0).
template <typename K>
struct GatherSrc {
  const K* ktile;
  const int32_t* vtile;
  const int* toff;
  int ntiles;
  const int* oob_tile;  // folded into *status by block 0
  uint32_t* status;
};

template <typename K>
__global__ void __launch_bounds__(RT)
    bucket_sort_kernel(K* k0, int32_t* v0, K* k1, int32_t* v1, K* __restrict__ kout,
                       int32_t* __restrict__ vout, const int* __restrict__ totals,
                       const int* __restrict__ bstart, int nbk,
                       int lb, int64_t cells, int64_t Z, int64_t ncol, int64_t n,
                       int32_t* __restrict__ col_start, GatherSrc<K> gs) {
  // smem: the key bitmap, or the LSD digit counters run[LNB] + wcnt[WAVES][LNB]; before either,
  // the gather pipeline's expanded source positions of the bucket's elements.
  __shared__ __attribute__((aligned(16))) uint32_t smem[kBitmapWords];
  __shared__ __attribute__((aligned(16))) uint16_t wpre[kBitmapWords];  // set bits before each word
  __shared__ int wsum[WAVES];
  static_assert(kBitmapWords >= LNB * (WAVES + 1), "LSD counters alias the bitmap");
  uint32_t* bits = smem;
  int* run = (int*)smem;
  int(*wcnt)[LNB] = (int(*)[LNB])((int*)smem + LNB);
  const int tid = threadIdx.x;
  // Block i runs on XCD i mod 8: each XCD takes a contiguous eighth of the buckets, so the
  // neighboring buckets that share cache lines of the tiles' runs (and of the digit starts) are
  // fetched into one L2.
  const int b = (nbk & 7) == 0 ? (int)(blockIdx.x & 7) * (nbk >> 3) + (int)(blockIdx.x >> 3)
                               : (int)blockIdx.x;
  const int passes = (lb + LBITS - 1) / LBITS;
  const int pbits = passes ? (lb + passes - 1) / passes : 0;
  const K lmask = (K)(((uint64_t)1 << lb) - 1);
  const bool gather = gs.ktile != nullptr;
  int64_t start;
  int size;
  // Gather pipeline: run t of the bucket (tile t's elements of digit b, thread t % RT's run
  // k = t / RT) holds the bucket's elements [rb0[k], rb0[k] + rl[k]), read from tile t at
  // t*PTILE + ra[k].  The source positions of RTILE elements at a time are expanded into LDS
  // (pos[i]), so each element costs one LDS read.
  constexpr int kRunsPerThread = (kGatherTiles + RT - 1) / RT;
  int* const pos = (int*)smem;  // [RTILE] expanded source positions, before the bitmap
  static_assert(RTILE <= kBitmapWords, "expanded positions fit the bitmap's words");
  int ra[kRunsPerThread], rl[kRunsPerThread], rb0[kRunsPerThread];
  if (gather) {
    const int nt = gs.ntiles;
    int carry = 0, below = 0;
#pragma unroll
    for (int k = 0; k < kRunsPerThread; ++k) {
      ra[k] = rl[k] = rb0[k] = 0;
      if (k * RT >= nt) continue;  // uniform
      const int t = k * RT + tid;
      if (t < nt) {
        ra[k] = gs.toff[(int64_t)t * (nbk + 1) + b];
        rl[k] = gs.toff[(int64_t)t * (nbk + 1) + b + 1] - ra[k];
      }
      int tot;
      rb0[k] = carry + block_excl_scan(rl[k], wsum, &tot);
      carry += tot;
      below += ra[k];
    }
    int tot_below;
    (void)block_excl_scan(below, wsum, &tot_below);  // elements of smaller digits: the start
    start = tot_below;
    size = carry;
    if (b == 0 && gs.status) {
      int any = 0;
      for (int t = tid; t < nt; t += RT) any |= gs.oob_tile[t];
      any = __syncthreads_or(any);
      if (tid == 0) gs.status[0] = any ? (uint32_t)TSC_MAP_OUT_OF_RANGE : 0u;
    }
  } else {
    start = bstart[b];
    size = totals[b];
  }
  // 16-bit word prefixes hold ranks below 65536: larger buckets take the LSD path.
  const bool bitmap_ok = size <= 65536 && lb <= kBitmapBits && passes > 0;
  // A bucket of at most RTILE elements stays in registers; a larger one is read in chunks of
  // RTILE twice (bits, then ranks) and written by rank straight to the outputs.
  const bool in_regs = bitmap_ok && size <= RTILE;
  K kk[RI];
  int32_t vv[RI];
  if (gather) {
    const int nt = gs.ntiles;
    // Chunks of RTILE elements (one chunk when the bucket stays in registers): positions of the
    // chunk's elements into LDS, then one read per element.
    for (int c0 = 0; c0 < size; c0 += RTILE) {  // uniform
      const int c1 = min(size, c0 + RTILE);
#pragma unroll
      for (int k = 0; k < kRunsPerThread; ++k) {
        const int t = k * RT + tid;
        if (t >= nt) continue;
        const int lo = max(rb0[k], c0), hi = min(rb0[k] + rl[k], c1);
        for (int e = lo; e < hi; ++e) pos[e - c0] = t * PTILE + ra[k] + (e - rb0[k]);
      }
      __syncthreads();
      if (in_regs) {
#pragma unroll
        for (int j = 0; j < RI; ++j) {
          const int i = j * RT + tid;
          if (i < size) {
            const int q = pos[i];
            kk[j] = gs.ktile[q];
            vv[j] = gs.vtile[q];
          }
        }
      } else {
        // Every other path reads the bucket from (k0, v0): assemble it there first.
        for (int i = c0 + tid; i < c1; i += RT) {
          const int q = pos[i - c0];
          k0[start + i] = gs.ktile[q];
          v0[start + i] = gs.vtile[q];
        }
      }
      __syncthreads();
    }
  } else if (in_regs) {
#pragma unroll
    for (int j = 0; j < RI; ++j) {
      const int i = j * RT + tid;
      if (i < size) {
        kk[j] = k0[start + i];
        vv[j] = v0[start + i];
      }
    }
  }

  bool by_bitmap = false;
  if (bitmap_ok) {
    const int nwords = ((1 << lb) + 31) / 32;
    for (int i = tid; i < nwords; i += RT) bits[i] = 0u;
    __syncthreads();
    int loc[RI];
    int dup = 0;
    if (in_regs) {
#pragma unroll
      for (int j = 0; j < RI; ++j) {
        const int i = j * RT + tid;
        if (i < size) {
          loc[j] = (int)(kk[j] & lmask);
          const uint32_t bit = 1u << (loc[j] & 31);
          dup |= (atomicOr(&bits[loc[j] >> 5], bit) & bit) != 0u;
        }
      }
    } else {
      for (int c0 = 0; c0 < size; c0 += RTILE) {
#pragma unroll
        for (int j = 0; j < RI; ++j) {
          const int i = c0 + j * RT + tid;
          kk[j] = i < size ? k0[start + i] : (K)0;
        }
#pragma unroll
        for (int j = 0; j < RI; ++j) {
          if (c0 + j * RT + tid < size) {
            const int l = (int)(kk[j] & lmask);
            const uint32_t bit = 1u << (l & 31);
            dup |= (atomicOr(&bits[l >> 5], bit) & bit) != 0u;
          }
        }
      }
    }
    dup = __syncthreads_or(dup);
    if (!dup) {
      // Per-word prefix counts: thread t owns words [t*wpt, (t+1)*wpt), one block scan of the
      // per-thread totals.  At the full bitmap (16 words per thread) the words are read and the
      // 16-bit prefixes written as 16-byte vectors.
      const int wpt = (nwords + RT - 1) / RT;
      constexpr int kWpt = kBitmapWords / RT;
      int cw[kWpt];
      if (wpt == kWpt) {
        const uint4* bv = (const uint4*)bits + tid * (kWpt / 4);
#pragma unroll
        for (int q = 0; q < kWpt / 4; ++q) {
          const uint4 x = bv[q];
          cw[4 * q] = __popc(x.x);
          cw[4 * q + 1] = __popc(x.y);
          cw[4 * q + 2] = __popc(x.z);
          cw[4 * q + 3] = __popc(x.w);
        }
      } else {
#pragma unroll
        for (int q = 0; q < kWpt; ++q) {
          const int wi = tid * wpt + q;
          cw[q] = (q < wpt && wi < nwords) ? __popc(bits[wi]) : 0;
        }
      }
      int sum = 0;
#pragma unroll
      for (int q = 0; q < kWpt; ++q) sum += cw[q];
      int tot;
      int pre = block_excl_scan(sum, wsum, &tot);
      if (wpt == kWpt) {
        uint32_t pk[kWpt / 2];
#pragma unroll
        for (int q = 0; q < kWpt / 2; ++q) {
          const uint32_t lo = (uint32_t)pre;
          pre += cw[2 * q];
          pk[q] = lo | ((uint32_t)pre << 16);
          pre += cw[2 * q + 1];
        }
        uint4* wp = (uint4*)wpre + tid * (kWpt / 8);
#pragma unroll
        for (int q = 0; q < kWpt / 8; ++q)
          wp[q] = make_uint4(pk[4 * q], pk[4 * q + 1], pk[4 * q + 2], pk[4 * q + 3]);
      } else {
#pragma unroll
        for (int q = 0; q < kWpt; ++q) {
          const int wi = tid * wpt + q;
          if (q < wpt && wi < nwords) {
            wpre[wi] = (uint16_t)pre;
            pre += cw[q];
          }
        }
      }
      __syncthreads();
      // Rank of local key l among the bucket's keys: set bits below it.
      auto rank = [&](int l) {
        const int wi = l >> 5;
        return (int)wpre[wi] + __popc(bits[wi] & ((1u << (l & 31)) - 1u));
      };
      // Column starts from the bitmap, before the staging below overwrites it: columns whose
      // first key c*Z lies in this bucket's key range [b << lb, (b+1) << lb).
      if (col_start) {
        const int64_t key_lo = (int64_t)b << lb;
        const int64_t key_hi = std::min<int64_t>((int64_t)(b + 1) << lb, cells);
        const int64_t c_lo = (key_lo + Z - 1) / Z, c_hi = (key_hi + Z - 1) / Z;
        for (int64_t c = c_lo + tid; c < c_hi; c += RT)
          col_start[c] = (int32_t)(start + rank((int)(c * Z - key_lo)));
      }
      if (in_regs) {
        int rk[RI];
#pragma unroll
        for (int j = 0; j < RI; ++j)
          if (j * RT + tid < size) rk[j] = rank(loc[j]);
        if constexpr (sizeof(K) == 4) {
          // Stage keys, then rows, in sorted order through LDS (the bitmap is no longer
          // needed) so that the global writes are coalesced runs instead of one cache line per
          // element.
          int32_t* st = (int32_t*)smem;
          static_assert(kBitmapWords >= RTILE, "staging holds a full bucket");
          __syncthreads();
#pragma unroll
          for (int j = 0; j < RI; ++j)
            if (j * RT + tid < size) st[rk[j]] = (int32_t)kk[j];
          __syncthreads();
          for (int i = tid; i < size; i += RT) kout[start + i] = (K)st[i];
          __syncthreads();
#pragma unroll
          for (int j = 0; j < RI; ++j)
            if (j * RT + tid < size) st[rk[j]] = vv[j];
          __syncthreads();
          for (int i = tid; i < size; i += RT) vout[start + i] = st[i];
        } else {
#pragma unroll
          for (int j = 0; j < RI; ++j) {
            if (j * RT + tid < size) {
              kout[start + rk[j]] = kk[j];
              vout[start + rk[j]] = vv[j];
            }
          }
        }
      } else {
        for (int c0 = 0; c0 < size; c0 += RTILE) {
#pragma unroll
          for (int j = 0; j < RI; ++j) {
            const int i = c0 + j * RT + tid;
            kk[j] = i < size ? k0[start + i] : (K)0;
            vv[j] = i < size ? v0[start + i] : 0;
          }
#pragma unroll
          for (int j = 0; j < RI; ++j) {
            if (c0 + j * RT + tid < size) {
              const int r = rank((int)(kk[j] & lmask));
              kout[start + r] = kk[j];
              vout[start + r] = vv[j];
            }
          }
        }
      }
      by_bitmap = true;
    } else if (gather && in_regs) {
      // A repeated key: the LSD path reads the bucket from (k0, v0).
#pragma unroll
      for (int j = 0; j < RI; ++j) {
        const int i = j * RT + tid;
        if (i < size) {
          k0[start + i] = kk[j];
          v0[start + i] = vv[j];
        }
      }
    }
  }
  if (!by_bitmap) {
    const int lane = tid & 63, w = tid >> 6;
    for (int p = 0; p < passes; ++p) {
      const int shift = p * pbits;
      const int dbits = min(pbits, lb - shift);
      const int mask = (1 << dbits) - 1;
      const bool last = p == passes - 1;
      const K* ks = (p & 1) ? k1 : k0;
      const int32_t* vs = (p & 1) ? v1 : v0;
      K* kd = last ? kout : ((p & 1) ? k0 : k1);
      int32_t* vd = last ? vout : ((p & 1) ? v0 : v1);
      __syncthreads();
      for (int d = tid; d < LNB; d += RT) run[d] = 0;
      __syncthreads();
      for (int i = tid; i < size; i += RT)
        atomicAdd(&run[digit_of<K>(ks[start + i], shift, mask)], 1);
      __syncthreads();
      scan_bins(run, wsum);
      for (int c0 = 0; c0 < size; c0 += RTILE) {
        for (int i = tid; i < WAVES * LNB; i += RT) (&wcnt[0][0])[i] = 0;
        __syncthreads();
        const int wfirst = c0 + w * (RI * 64);
        const int wlimit = min(size, wfirst + RI * 64);
        K kk[RI];
        int32_t vv[RI];
        int lr[RI];
#pragma unroll
        for (int j = 0; j < RI; ++j) {
          const int e = wfirst + j * 64 + lane;
          const bool valid = e < wlimit;
          kk[j] = valid ? ks[start + e] : (K)0;
          vv[j] = valid ? vs[start + e] : 0;
        }
        wave_rank<K, RI>(kk, wfirst, wlimit, shift, dbits, wcnt[w], lr);
        __syncthreads();
        int cnt[LPT];
        wave_offsets(wcnt, cnt);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < RI; ++j) {
          const int e = wfirst + j * 64 + lane;
          if (e < wlimit) {
            const int d = digit_of<K>(kk[j], shift, mask);
            const int pos = run[d] + wcnt[w][d] + lr[j];
            kd[start + pos] = kk[j];
            vd[start + pos] = vv[j];
          }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < LPT; ++q) run[tid * LPT + q] += cnt[q];
        __syncthreads();
      }
    }
    if (passes == 0) {
      for (int i = tid; i < size; i += RT) {
        kout[start + i] = k0[start + i];
        vout[start + i] = v0[start + i];
      }
    }
  }
  if (!col_start) return;
  if (b == nbk - 1 && tid == 0) col_start[ncol] = (int32_t)n;
  if (by_bitmap) return;
  __syncthreads();
  // Columns whose first key c*Z lies in this bucket's key range [b << lb, (b+1) << lb).
  const int64_t key_lo = (int64_t)b << lb;
  const int64_t key_hi = std::min<int64_t>((int64_t)(b + 1) << lb, cells);
  const int64_t c_lo = (key_lo + Z - 1) / Z, c_hi = (key_hi + Z - 1) / Z;
  for (int64_t c = c_lo + tid; c < c_hi; c += RT)
    col_start[c] = (int32_t)(start + lower_bound<K>(kout + start, 0, size, (K)(c * Z)));
}

// Column-index probe for the column-parallel fill: the neighbor column's keys occupy
// [col_start[nc], col_start[nc+1]) of the sorted array (or the whole array without a column
// table); one lower_bound finds the first key >= the lowest wanted z, then a short forward walk
// picks up the (up to three) wanted taps.
template <typename K, bool USE_COLS>
struct ColumnLookup {
  const K* __restrict__ keys;
  const int32_t* __restrict__ col_start;
  const int32_t* __restrict__ perm;
  int64_t n;
  __device__ __forceinline__ void column(K kc, K nc, int32_t z, int32_t Z, int32_t dW,
                                         int32_t v[3]) const {
    int64_t lo = 0, hi = n;
    if (USE_COLS) {
      lo = col_start[nc];
      hi = col_start[nc + 1];
    }
    const bool has_lo = z - dW >= 0, has_hi = z + dW < Z;
    const K first = has_lo ? (K)(kc - dW) : kc;
    const K last = has_hi ? (K)(kc + dW) : kc;
    for (int64_t q = lower_bound<K>(keys, lo, hi, first); q < hi; ++q) {
      const K k = keys[q];
      if (k > last) break;
      if (k == kc) v[1] = perm[q];
      else if (has_lo && k == (K)(kc - dW)) v[0] = perm[q];
      else if (has_hi && k == (K)(kc + dW)) v[2] = perm[q];
    }
  }
};

// Window fill: a block owns VOX = ROUNDS * 28 consecutive sorted voxels (112).  Their columns span
// [c_first, c_last]; every neighbor column with offset (kd-1)*dD along x lies in
// [c_first + (kd-1)*dD*Y - dH, c_last + (kd-1)*dD*Y + dH], and the sorted voxels of those
// columns are one contiguous run of the sorted arrays.  Phase 1 decodes the block's voxels (two
// per thread, all loads issued together: column, z, row, a 9-bit mask of in-grid neighbor
// columns, the duplicate check), then copies, per kd, that run's rows and keys relative to the
// window's first column (j*Z + z for the j-th column of the window; keys are unique, so a
// relative key names one voxel) plus the column starts into LDS, and takes the longest column
// of the three windows from the same column-start loads.  Phase 2 resolves every probe from
// LDS with 9 lanes per voxel (one per neighbor column): a binary search for the first key >= the
// lowest wanted one in the column, then the next three entries compared as keys (an entry of
// another column or a sentinel cannot equal a wanted key).  Each lane runs ILP voxels' searches
// side by side, so ILP independent LDS chains are in flight per lane.  Blocks of a few hundred
// voxels would amortise phase 1's chain of dependent global loads (own keys -> column starts ->
// windows, several microseconds per block under the fill's write traffic) but measured slower
// (fewer blocks per CU keep fewer scattered stores in flight); 112 voxels is the default.  A kd
// window that does not fit (very sparse or very dense regions, or Z so large that window keys
// overflow 31 bits) falls back to the global column lookup for that kd only.
constexpr int kWinIlp = 4;

// THREADS per block (2 or 4 waves), ROUNDS of 7 voxels per wave; CAPE / CAPC = voxels / columns
// per kd window, sized so that the LDS lets the wave limit (32 per CU) decide the blocks per CU.
template <int ROUNDS, int THREADS>
struct WinCfg {
  static constexpr int WAVES = THREADS / 64;
  static constexpr int VOX = ROUNDS * mapk::kFillVoxPerWave * WAVES;
  static constexpr int CAPE = THREADS == 128 ? 240 : ROUNDS >= 16 ? 1024 : ROUNDS >= 8 ? 640 : 464;
  static constexpr int CAPC = THREADS == 128 ? 96 : ROUNDS >= 16 ? 256 : ROUNDS >= 8 ? 128 : 432;
  static_assert(VOX <= 2 * THREADS, "two voxels per thread in the decode");
  static_assert(ROUNDS % kWinIlp == 0, "rounds come in groups of ILP");
};

template <typename K, int ROUNDS, int THREADS>
__global__ void __launch_bounds__(THREADS)
    fill_window_kernel(const K* __restrict__ keys, const int32_t* __restrict__ perm,
                       const int32_t* __restrict__ col_start, int64_t n, mapk::KeyCoder<K> kc_,
                       int32_t dD, int32_t dH, int32_t dW, int64_t ncol, int32_t per_xcd,
                       int32_t* __restrict__ nbr, uint32_t* __restrict__ status) {
  using Cfg = WinCfg<ROUNDS, THREADS>;
  constexpr int kWinThreads = THREADS;
  constexpr int VOX = Cfg::VOX, CAPE = Cfg::CAPE, CAPC = Cfg::CAPC;
  using I = typename std::conditional<sizeof(K) == 4, int32_t, int64_t>::type;  // column index
  // Window keys / rows at [1, ne], slot 0 readable (never used), sentinels after the run: the
  // probe reads up to 2 past a column's end and its search one before the column's start.
  __shared__ int32_t lk[3][CAPE + 5];
  __shared__ int32_t lp[3][CAPE + 5];
  __shared__ int32_t lcs[3][CAPC + 1];
  __shared__ I w_lo[3];
  __shared__ int32_t w_e0[3], w_ne[3], w_nc[3];
  __shared__ I c_range[2];
  __shared__ int32_t w_maxlen;  // longest column in the three windows
  __shared__ I vcol[VOX];       // absolute column (the global-lookup path)
  __shared__ int4 vinfo[VOX];   // column - c_first, z, row, in-grid neighbor-column mask
  const int tid = threadIdx.x;
  const int32_t X = kc_.X, Y = kc_.Y, Z = kc_.Z;
  const int64_t logical = (int64_t)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  const int64_t i0 = logical * VOX;
  if (i0 >= n) return;  // uniform per block
  const int nv = (int)((i0 + VOX < n) ? VOX : n - i0);
  // Every thread decodes the block's first key (one broadcast load) for relative columns.
  K first_col;
  {
    int32_t x, y, z;
    kc_.decode(keys[i0], &first_col, &x, &y, &z);
  }
  int dup = 0;
  {
    K kk[2], kp[2];
    int32_t rr[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = tid + h * kWinThreads;
      const bool live = j < nv;
      kk[h] = live ? keys[i0 + j] : (K)0;
      kp[h] = (live && i0 + j > 0) ? keys[i0 + j - 1] : (K)-1;
      rr[h] = live ? perm[i0 + j] : -1;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = tid + h * kWinThreads;
      if (j >= nv) continue;
      K column;
      int32_t x, y, z;
      kc_.decode(kk[h], &column, &x, &y, &z);
      int m = 0;
#pragma unroll
      for (int kd = 0; kd < 3; ++kd) {
#pragma unroll
        for (int kh = 0; kh < 3; ++kh) {
          const bool in = (uint32_t)(x + (kd - 1) * dD) < (uint32_t)X &&
                          (uint32_t)(y + (kh - 1) * dH) < (uint32_t)Y;
          m |= (int)in << (kd * 3 + kh);
        }
      }
      vcol[j] = (I)column;
      vinfo[j] = make_int4((int32_t)(column - first_col), z, rr[h], m);
      if (kp[h] == kk[h]) dup = 1;
      if (j == nv - 1) c_range[1] = (I)column;
    }
  }
  if (tid == 0) {
    c_range[0] = (I)first_col;
    w_maxlen = 0;
  }
  dup = __syncthreads_or(dup);
  if (dup && tid == 0) atomicOr(status, TSC_MAP_DUPLICATE);
  if (tid < 3) {
    const int64_t shiftc = (int64_t)(tid - 1) * dD * Y;
    int64_t lo = (int64_t)c_range[0] + shiftc - dH, hi = (int64_t)c_range[1] + shiftc + dH;
    if (lo < 0) lo = 0;
    if (hi > ncol - 1) hi = ncol - 1;
    int32_t e0 = 0, ne = 0, nc = 0;
    // Window keys (j*Z + z) must stay below 2^31 - 1 (the sentinel).
    const bool keys31 = (int64_t)(CAPC + 1) * Z < (int64_t)INT32_MAX;
    if (lo <= hi && hi - lo + 1 <= CAPC && keys31) {
      e0 = col_start[lo];
      ne = col_start[hi + 1] - e0;
      nc = (int32_t)(hi - lo + 1);
      if (ne > CAPE) {
        nc = -1;
        ne = 0;  // nothing copied (the sentinels then sit at the window's start)
      }
    } else if (lo <= hi) {
      nc = -1;
    }
    w_lo[tid] = (I)lo;
    w_e0[tid] = e0;
    w_ne[tid] = ne;
    w_nc[tid] = nc;  // -1: window does not fit, probes of this kd go to global memory
  }
  __syncthreads();
  {
    // Column starts (and the longest column), keys and rows of the three windows: every load of
    // this phase is issued before the first LDS store (one round trip instead of one per window
    // and array).  Each thread takes column entries j = tid + 256u (u < CU) and window entries
    // j = tid + 256u (u < EU) of every window; indices past a window's end are clamped to its last
    // entry (or to entry 0 of an empty window) so that every load is unconditional.
    constexpr int CU = (CAPC + 1 + kWinThreads - 1) / kWinThreads;
    constexpr int EU = (CAPE + kWinThreads - 1) / kWinThreads;
    int32_t ca[3][CU], cb[3][CU], pv[3][EU];
    K kv[3][EU];
#pragma unroll
    for (int w = 0; w < 3; ++w) {
      const int nc = w_nc[w] > 0 ? w_nc[w] : 0;
      const int64_t lo = w_nc[w] > 0 ? (int64_t)w_lo[w] : 0;
      const int ne = w_nc[w] > 0 ? w_ne[w] : 0;
      const int64_t e0 = ne > 0 ? w_e0[w] : 0;
#pragma unroll
      for (int u = 0; u < CU; ++u) {
        const int j = min(tid + u * kWinThreads, nc);
        ca[w][u] = col_start[lo + j];
        cb[w][u] = col_start[lo + min(j + 1, nc)];
      }
#pragma unroll
      for (int u = 0; u < EU; ++u) {
        const int j = min(tid + u * kWinThreads, ne > 0 ? ne - 1 : 0);
        kv[w][u] = keys[e0 + j];
        pv[w][u] = perm[e0 + j];
      }
    }
    int mx = 0;
#pragma unroll
    for (int w = 0; w < 3; ++w) {
      const int nc = w_nc[w];
      if (nc <= 0) continue;  // empty (lo > hi) or not fitting: nothing copied
      const int32_t e0 = w_e0[w], ne = w_ne[w];
      const K kbase = (K)w_lo[w] * (K)Z;  // key of the window's first column at z = 0
#pragma unroll
      for (int u = 0; u < CU; ++u) {
        const int j = tid + u * kWinThreads;
        if (j <= nc) {
          lcs[w][j] = ca[w][u] - e0;
          mx = max(mx, cb[w][u] - ca[w][u]);
        }
      }
#pragma unroll
      for (int u = 0; u < EU; ++u) {
        const int j = tid + u * kWinThreads;
        if (j < ne) {
          lk[w][1 + j] = (int32_t)(kv[w][u] - kbase);
          lp[w][1 + j] = pv[w][u];
        }
      }
    }
    // Sentinels after every window's run, also for empty and global-lookup windows (whose lanes
    // still read entries 0..2 and must find no key they want).
    if (tid < 12) lk[tid >> 2][1 + w_ne[tid >> 2] + (tid & 3)] = INT32_MAX;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = max(mx, __shfl_xor(mx, off, 64));
    if ((tid & 63) == 0 && mx > 0) atomicMax(&w_maxlen, mx);
  }
  __syncthreads();

  const int lane = tid & 63, wid = tid >> 6;
  const int slot = lane / mapk::kFillLanes, col = lane - slot * mapk::kFillLanes;
  if (slot >= mapk::kFillVoxPerWave) return;  // no barrier follows
  const int kd = col / 3, kh = col - kd * 3;
  const int nc_w = w_nc[kd];
  const I lo_w = w_lo[kd];
  const I off = (I)(kd - 1) * dD * Y + (I)(kh - 1) * dH;
  const int32_t* const wk = lk[kd] + 1;
  const int32_t* const wp = lp[kd] + 1;
  const int32_t* const wc = lcs[kd];
  const int li0 = wid * ROUNDS * mapk::kFillVoxPerWave + slot;
  if (dW == 1 && w_nc[0] >= 0 && w_nc[1] >= 0 && w_nc[2] >= 0) {
    // Every window fits (block-uniform): branch-free probes.  The neighbor column is window
    // column j = (column - c_first) + jofs (an in-grid neighbor column always lies in the
    // window) and the wanted keys are t - 1, t, t + 1 with t = j*Z + z.  The first entry >= t - 1
    // comes from a binary search over the column with a block-uniform step count (powers of two
    // below the longest column); the three keys can only be that entry and the next two.
    // Out-of-grid lanes search an empty range and want negative keys, which match nothing.
    const int jofs = (int)((I)c_range[0] + off - lo_w);
    const int maxlen = w_maxlen;
    int steps = 0;
    while ((2 << steps) <= maxlen) ++steps;  // 2^steps <= maxlen < 2^(steps+1)
    const int top = maxlen > 0 ? 1 << steps : 0;
    for (int g = 0; g < ROUNDS; g += kWinIlp) {
      int pos[kWinIlp], e[kWinIlp], first[kWinIlp], t[kWinIlp], zz[kWinIlp], row[kWinIlp];
      bool live[kWinIlp];
#pragma unroll
      for (int u = 0; u < kWinIlp; ++u) {
        const int li = li0 + (g + u) * mapk::kFillVoxPerWave;
        live[u] = li < nv;
        const int4 vi = vinfo[live[u] ? li : 0];
        row[u] = vi.z;
        zz[u] = vi.y;
        const bool inb = live[u] && ((vi.w >> col) & 1);
        const int j = inb ? vi.x + jofs : 0;
        pos[u] = inb ? wc[j] : 0;
        e[u] = inb ? wc[j + 1] : 0;
        t[u] = inb ? j * Z + zz[u] : -4;
        first[u] = zz[u] > 0 ? t[u] - 1 : t[u];
      }
      for (int st = top; st > 0; st >>= 1) {  // uniform trip count, no lane branches
#pragma unroll
        for (int u = 0; u < kWinIlp; ++u) {
          const int tt = pos[u] + st;
          const int32_t kv = wk[(tt < e[u] ? tt : e[u]) - 1];  // index >= a - 1 >= -1
          pos[u] = ((tt <= e[u]) & (kv < first[u])) ? tt : pos[u];
        }
      }
#pragma unroll
      for (int u = 0; u < kWinIlp; ++u) {
        // pos <= e <= ne: pos + 2 reads a later column's key or a sentinel at worst.
        const int p = pos[u];
        const int32_t k0 = wk[p], k1 = wk[p + 1], k2 = wk[p + 2];
        const int32_t p0 = wp[p], p1 = wp[p + 1], p2 = wp[p + 2];
        const int32_t tm = zz[u] > 0 ? t[u] - 1 : -4, tp = zz[u] + 1 < Z ? t[u] + 1 : -4;
        const int32_t v0 = k0 == tm ? p0 : -1;
        int32_t v1 = k1 == t[u] ? p1 : -1;
        v1 = k0 == t[u] ? p0 : v1;
        int32_t v2 = k2 == tp ? p2 : -1;
        v2 = k1 == tp ? p1 : v2;
        v2 = k0 == tp ? p0 : v2;
        if (col == 4) v1 = row[u];  // tap 13 is the voxel itself
        if (live[u]) {
          int32_t* dst = nbr + (int64_t)row[u] * 27 + col * 3;
          dst[0] = v0;
          dst[1] = v1;
          dst[2] = v2;
        }
      }
    }
    return;
  }
  const int nscan = 2 * dW + 1;
  ColumnLookup<K, true> glk{keys, col_start, perm, n};
  for (int r = 0; r < ROUNDS; ++r) {
    const int li = li0 + r * mapk::kFillVoxPerWave;
    if (li >= nv) break;
    const int4 vi = vinfo[li];
    const int32_t row = vi.z;
    int32_t v0 = -1, v1 = -1, v2 = -1;
    if ((vi.w >> col) & 1) {
      const I ncl = vcol[li] + off;
      const int32_t z = vi.y;
      const bool has_lo = z - dW >= 0, has_hi = z + dW < Z;
      if (nc_w > 0) {
        const int j = (int)(ncl - lo_w);
        int a = wc[j];
        int b = wc[j + 1];
        const int e = b;
        const int32_t base = j * Z;  // window key of (column j, z = 0)
        const int32_t first = base + (has_lo ? z - dW : z);
        while (a < b) {  // first entry with key >= first
          const int mid = (a + b) >> 1;
          if (wk[mid] < first) a = mid + 1;
          else b = mid;
        }
        const int32_t last = base + (has_hi ? z + dW : z);
        for (int s = 0; s < nscan; ++s, ++a) {
          if (a >= e) break;
          const int32_t kk = wk[a];
          if (kk > last) break;
          const int32_t p = wp[a];
          const int32_t zz = kk - base;
          if (zz == z) v1 = p;
          else if (has_lo && zz == z - dW) v0 = p;
          else if (has_hi && zz == z + dW) v2 = p;
        }
      } else {
        int32_t v[3] = {-1, -1, -1};
        glk.column((K)((K)ncl * Z + z), (K)ncl, z, Z, dW, v);
        v0 = v[0];
        v1 = v[1];
        v2 = v[2];
      }
    }
    if (col == 4) v1 = row;  // tap 13 is the voxel itself
    int32_t* dst = nbr + (int64_t)row * 27 + col * 3;
    dst[0] = v0;
    dst[1] = v1;
    dst[2] = v2;
  }
}

inline int bit_length(uint64_t v) {
  int b = 0;
  while (v) {
    ++b;
    v >>= 1;
  }
  return b;
}

// Voxels per fill block: 112.  Measured on map512: 224 voxels (7 blocks per CU) +6 % and 448
// voxels (4 blocks per CU) +22 % fill time.
// Threads per fill block: 256 (4 waves, 8 blocks per CU).  2-wave blocks of the same 112 voxels
// (16 blocks per CU, twice the dependent load chains in flight) measured 9 % slower.
constexpr int kFillThreads = 256;
constexpr int kFillRounds = 1024 / kFillThreads;  // 112 voxels per block

// Sort buffers carved from one workspace: (kA, vA) and (kB, vB) ping-pong copies of the pairs
// (plus (kC, vC) for the gather pipeline), per-(bucket, tile) counts or the tiles' digit starts,
// bucket totals and starts, per-tile out-of-range flags.
template <typename K>
struct SortBufs {
  K *kA, *kB, *kC;
  int32_t *vA, *vB, *vC;
  int *counts, *totals, *oob_tile, *bstart;
  // The gather pipeline keeps the tile-sorted pairs (kA, vA) intact while buckets are sorted, so
  // its LSD passes ping-pong between (kB, vB) and a third copy (kC, vC); counts holds the tiles'
  // digit starts, ntiles x (nb + 1).
  // want_gather: the caller's keys suit the gather pipeline (see sort_stages).
  static bool gather(int64_t N, bool want_gather) {
    return want_gather && (N + PTILE - 1) / PTILE <= kGatherTiles;
  }
  static size_t bytes(int64_t N, int nb, bool want_gather) {
    const int64_t ntiles = (N + PTILE - 1) / PTILE;
    const int copies = gather(N, want_gather) ? 3 : 2;
    return copies * (align_up((size_t)N * sizeof(K), 256) + align_up((size_t)N * 4, 256)) +
           align_up((size_t)(nb + 1) * ntiles * 4, 256) + 2 * align_up((size_t)nb * 4, 256) +
           align_up((size_t)ntiles * 4, 256);
  }
  void carve(Carve& cv, int64_t N, int nb, bool want_gather) {
    const int64_t ntiles = (N + PTILE - 1) / PTILE;
    kA = cv.take<K>(N);
    vA = cv.take<int32_t>(N);
    kB = cv.take<K>(N);
    vB = cv.take<int32_t>(N);
    kC = nullptr;
    vC = nullptr;
    if (gather(N, want_gather)) {
      kC = cv.take<K>(N);
      vC = cv.take<int32_t>(N);
    }
    counts = cv.take<int>((int64_t)(nb + 1) * ntiles);
    totals = cv.take<int>(nb);
    oob_tile = cv.take<int>(ntiles);
    bstart = cv.take<int>(nb);
  }
};

// Sort of (gen(coords[i]), i) for i < N (N > 0) by keys below 2^nbits, at most TBMAX bucket bits.
// Buffers carved for the gather pipeline (up to kGatherTiles tiles): pack with the tile-local
// digit sort, then buckets gathering their runs -- two launches, for evenly filled buckets such
// as the map's x-slab buckets of a surface (1.5 M-voxel shell: 39 against 54 us for the four
// launches below).  Otherwise pack, scan, partition, buckets: the Morton order's buckets hold up
// to 12 k voxels, which the gather path assembles one block per bucket (63 against 49 us for
// partition + buckets).  Sorted pairs go to (kOut, vOut), the column starts to cols when it is
// not null (for the map's (b, x, y) columns of Z keys each), the out-of-range flag to *status.
// names[] are the profiler names of the four stages.
template <typename K, typename Gen>
void sort_stages(tsc_ctx* ctx, const int32_t* coords, int64_t N, Gen gen, int nbits,
                 const SortBufs<K>& sb, K* kOut, int32_t* vOut, int64_t cells, int64_t Z,
                 int64_t ncol, int32_t* cols, uint32_t* status, const char* const names[4]) {
  const int tb = std::min(nbits, TBMAX);
  const int lb = nbits - tb;
  const int nbk = 1 << tb;
  const int64_t ntiles = (N + PTILE - 1) / PTILE;
  hipStream_t s = ctx->stream;
  if (sb.kC) {  // carved for the gather pipeline
    {
      ProfScope p(ctx, names[0]);
      pack_sort_kernel<K, Gen><<<(unsigned)ntiles, PT, 0, s>>>(
          (const int4*)coords, N, gen, lb, tb, sb.kA, sb.vA, sb.counts, (int)ntiles, sb.oob_tile);
    }
    ProfScope ps(ctx, names[3]);
    bucket_sort_kernel<K><<<(unsigned)nbk, RT, 0, s>>>(
        sb.kB, sb.vB, sb.kC, sb.vC, kOut, vOut, nullptr, nullptr, nbk, lb, cells, Z, ncol, N,
        cols, GatherSrc<K>{sb.kA, sb.vA, sb.counts, (int)ntiles, sb.oob_tile, status});
    return;
  }
  {
    ProfScope p(ctx, names[0]);
    pack_kernel<K, Gen><<<(unsigned)ntiles, PT, 0, s>>>(
        (const int4*)coords, N, gen, sb.kA, sb.vA, lb, tb, sb.counts, (int)ntiles, sb.oob_tile);
  }
  {
    ProfScope ps(ctx, names[1]);
    scan_kernel<<<(unsigned)nbk, RT, 0, s>>>(sb.counts, (int)ntiles, sb.totals, sb.oob_tile,
                                             status);
  }
  {
    ProfScope ps(ctx, names[2]);
    partition_kernel<K><<<(unsigned)ntiles, PT, 0, s>>>(
        sb.kA, sb.vA, N, lb, tb, sb.counts, sb.totals, (int)ntiles, sb.kB, sb.vB, sb.bstart);
  }
  {
    ProfScope ps(ctx, names[3]);
    bucket_sort_kernel<K><<<(unsigned)nbk, RT, 0, s>>>(
        sb.kB, sb.vB, sb.kA, sb.vA, kOut, vOut, sb.totals, sb.bstart, nbk, lb, cells, Z, ncol, N,
        cols, GatherSrc<K>{nullptr, nullptr, nullptr, 0, nullptr, nullptr});
  }
}

template <typename K>
int radix_impl(tsc_ctx* ctx, const int32_t* coords, int64_t N, int32_t B, int32_t X, int32_t Y,
               int32_t Z, const int32_t dil[3], void* keys_out, int32_t* perm_out,
               int32_t* nbr_out, uint32_t* status_dev) {
  const int64_t cells = (int64_t)B * X * Y * Z;
  const int nbits = std::max(1, bit_length((uint64_t)(cells - 1)));
  const int64_t ncol = (int64_t)B * X * Y;
  const bool use_cols = ncol <= std::max<int64_t>(16 * N, int64_t(1) << 22);
  size_t need = SortBufs<K>::bytes(N, NBMAX, true) +
                (use_cols ? align_up((size_t)(ncol + 1) * 4, 256) : 0);
  if (!keys_out) need += align_up((size_t)N * sizeof(K), 256);
  if (!perm_out) need += align_up((size_t)N * 4, 256);
  void* ws;
  int st = workspace(ctx, need, &ws);
  if (st) return st;
  Carve cv(ws);
  SortBufs<K> sb;
  sb.carve(cv, N, NBMAX, true);
  int32_t* cols = use_cols ? cv.take<int32_t>(ncol + 1) : nullptr;
  K* kOut = keys_out ? (K*)keys_out : cv.take<K>(N);
  int32_t* vOut = perm_out ? perm_out : cv.take<int32_t>(N);

  hipStream_t s = ctx->stream;
  if (N == 0) {
    clear_status_kernel<<<1, 64, 0, s>>>(status_dev);
    return check_hip(hipGetLastError(), "map_build_radix launch");
  }
  static const char* const names[4] = {"radix_pack", "radix_scan", "radix_partition",
                                       "radix_buckets"};
  sort_stages<K>(ctx, coords, N, PackedKey<K>{B, X, Y, Z, (K)(cells - 1)}, nbits, sb, kOut, vOut,
                 cells, Z, ncol, cols, status_dev, names);
  {
    ProfScope ps(ctx, "radix_fill");
    const K no_sentinel = (K)-1;  // out-of-range voxels were clamped in pack
    if (use_cols) {
      constexpr int R = kFillRounds, T = kFillThreads;
      const int64_t blocks = (N + WinCfg<R, T>::VOX - 1) / WinCfg<R, T>::VOX;
      const int32_t per_xcd = (int32_t)((blocks + 7) / 8);
      fill_window_kernel<K, R, T><<<(unsigned)per_xcd * 8u, T, 0, s>>>(
          kOut, vOut, cols, N, mapk::KeyCoder<K>::make(X, Y, Z), dil[0], dil[1], dil[2], ncol,
          per_xcd, nbr_out, status_dev);
    } else {
      const int32_t per_xcd = mapk::fill_per_xcd(N);
      const unsigned grid = (unsigned)per_xcd * 8u;
      mapk::fill_columns_kernel<K, ColumnLookup<K, false>><<<grid, mapk::kFillThreads, 0, s>>>(
          kOut, vOut, nullptr, N, no_sentinel, mapk::KeyCoder<K>::make(X, Y, Z), dil[0], dil[1],
          dil[2], ColumnLookup<K, false>{kOut, nullptr, vOut, N}, per_xcd, nbr_out, status_dev);
    }
  }
  return check_hip(hipGetLastError(), "map_build_radix launch");
}

}  // namespace

int map_build_radix(tsc_ctx* ctx, const int32_t* coords, int64_t N, int32_t B, int32_t X,
                    int32_t Y, int32_t Z, const int32_t dil[3], void* keys_out, int32_t* perm_out,
                    int32_t* nbr_out, uint32_t* status_dev) {
  const int64_t cells = (int64_t)B * X * Y * Z;
  if (cells < (int64_t(1) << 31))
    return radix_impl<int32_t>(ctx, coords, N, B, X, Y, Z, dil, keys_out, perm_out, nbr_out,
                               status_dev);
  return radix_impl<int64_t>(ctx, coords, N, B, X, Y, Z, dil, keys_out, perm_out, nbr_out,
                             status_dev);
}

namespace {

// Morton keys of up to 32 bits sort as uint32, wider ones as uint64.  A 512^3 shell's Z-curve puts
// up to 12 k voxels under one 10-bit prefix; the bucket kernel's bitmap rank takes them in chunks
// (measured on that shell: 10 bucket bits 68 us for the four stages, 12 bits 86 us, where the
// larger partition and pack histograms cost more than the smaller buckets save).
template <typename K>
int morton_impl(tsc_ctx* ctx, const int32_t* coords, int64_t N, int bits, int shift, int nbits,
                int32_t* rows_out) {
  const size_t need = SortBufs<K>::bytes(N, NBMAX, false) + align_up((size_t)N * sizeof(K), 256) +
                      256;
  void* ws;
  int st = workspace(ctx, need, &ws);
  if (st) return st;
  Carve cv(ws);
  SortBufs<K> sb;
  sb.carve(cv, N, NBMAX, false);
  K* kOut = cv.take<K>(N);
  uint32_t* status = cv.take<uint32_t>(1);  // the scan's flag word; Morton keys never set it
  const uint64_t mask = nbits >= 64 ? ~0ull : ((1ull << nbits) - 1);
  static const char* const names[4] = {"morton_pack", "morton_scan", "morton_partition",
                                       "morton_buckets"};
  sort_stages<K>(ctx, coords, N, MortonKey<K>{bits, shift, mask}, nbits, sb, kOut, rows_out,
                 (int64_t)0, (int64_t)1, (int64_t)0, nullptr, status, names);
  return check_hip(hipGetLastError(), "gather plan sort");
}

}  // namespace

namespace {

// The store side of fill_window_kernel alone (a measurement kernel; no product path runs it): the
// same blocks of 112 consecutive sorted voxels dealt to the XCDs in contiguous runs, the same
// 7 voxels per wave over 4 rounds, and the same 9 lanes x 12 bytes of each voxel's 108-byte row
// at its original row rows[i] (i when rows is null).  rows[i] is its only load, so its time is
// what the fill would take if its window copies and searches cost nothing: the floor of a table
// laid out in the caller's row order.  The words written are (-1, row, -1) per lane.
__global__ void __launch_bounds__(kFillThreads)
    write_floor_kernel(const int32_t* __restrict__ rows, int64_t n, int32_t per_xcd,
                       int32_t* __restrict__ out) {
  constexpr int VOX = kFillRounds * mapk::kFillVoxPerWave * (kFillThreads / 64);
  const int64_t i0 = ((int64_t)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3)) * VOX;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int slot = lane / mapk::kFillLanes, col = lane - slot * mapk::kFillLanes;
  if (slot >= mapk::kFillVoxPerWave) return;
  const int li0 = wid * kFillRounds * mapk::kFillVoxPerWave + slot;
#pragma unroll
  for (int r = 0; r < kFillRounds; ++r) {
    const int64_t i = i0 + li0 + r * mapk::kFillVoxPerWave;
    if (i >= n) break;
    const int32_t row = rows ? rows[i] : (int32_t)i;
    if (row < 0 || row >= n) continue;
    int32_t* dst = out + (int64_t)row * 27 + col * 3;
    dst[0] = -1;
    dst[1] = row;
    dst[2] = -1;
  }
}

}  // namespace

int map_write_floor_launch(tsc_ctx* ctx, const int32_t* rows, int64_t N, int32_t* out) {
  if (N == 0) return TSC_OK;
  constexpr int VOX = kFillRounds * mapk::kFillVoxPerWave * (kFillThreads / 64);
  const int64_t blocks = (N + VOX - 1) / VOX;
  const int32_t per_xcd = (int32_t)((blocks + 7) / 8);
  ProfScope ps(ctx, "map_write_floor");
  write_floor_kernel<<<(unsigned)per_xcd * 8u, kFillThreads, 0, ctx->stream>>>(rows, N, per_xcd,
                                                                               out);
  return check_hip(hipGetLastError(), "map_write_floor launch");
}

int sort_rows_morton(tsc_ctx* ctx, const int32_t* coords, int64_t N, int bits, int shift,
                     int nbits, int32_t* rows_out) {
  if (N == 0) return TSC_OK;
  return nbits <= 32 ? morton_impl<uint32_t>(ctx, coords, N, bits, shift, nbits, rows_out)
                     : morton_impl<uint64_t>(ctx, coords, N, bits, shift, nbits, rows_out);
}

}  // namespace tsc
