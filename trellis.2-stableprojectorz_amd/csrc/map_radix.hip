// Neighbor-map build by LSD radix sort of packed keys (no global atomics, no grid-sized memsets).
//
// Same outputs as the bitmap path (sorted unique keys, their rows, the (N,27) neighbor table; see
// map_build.hip for the semantics and reference citations).  Steps:
//   pack      coords -> (key, row) in input order; histogram of the first digit per 4096-tile.
//             Out-of-range coordinates get key = cells (sorts last) and are reported later.
//   P passes  stable LSD counting sort on D-bit digits (D <= 8, P = ceil(bits/8)):
//               scan     exclusive scan of the digit-major (digit, tile) histogram
//               scatter  per tile: wave-ballot multisplit gives each element its stable rank
//                        among equal digits (one ballot per digit bit -> peer mask -> popcount),
//                        the tile is reordered by digit in LDS and written as contiguous runs
//               hist     per-tile histogram of the next digit
//   columns   col_start[c] = first sorted position whose key >= c*Z, for every (b,x,y) column c;
//             each block binary-searches its 256 columns inside a range found once per block
//   fill      per sorted position: 9 neighbor columns -> binary search of the three z taps
//             inside the column's [start, end) range; present neighbors read perm; duplicate
//             keys and out-of-range rows set status bits; rows written via LDS staging.
// When the column table would be much larger than the voxel set (very sparse, huge grids) the
// fill searches the whole sorted array instead of a column range.

#include <algorithm>

#include "map_common.h"

namespace tsc {
namespace {

constexpr int RT = 256;             // threads per block
constexpr int RI = 16;              // items per thread
constexpr int RTILE = RT * RI;      // elements per tile
constexpr int WAVES = RT / 64;
constexpr int NBMAX = 256;          // max bins per digit (8-bit digits)

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
__device__ __forceinline__ int digit_of(K k, int shift, int mask) {
  return (int)((k >> shift) & (K)mask);
}

__global__ void clear_status_kernel(uint32_t* status) {
  if (threadIdx.x == 0) status[0] = 0u;
}

template <typename K>
__global__ void __launch_bounds__(RT)
    pack_kernel(const int4* __restrict__ coords, int64_t N, int32_t B, int32_t X, int32_t Y,
                int32_t Z, K sentinel, K* __restrict__ keys, int32_t* __restrict__ vals, int shift,
                int dbits, int* __restrict__ counts, int ntiles, uint32_t* __restrict__ status) {
  __shared__ int hist[NBMAX];
  const int nb = 1 << dbits, mask = nb - 1;
  for (int d = threadIdx.x; d < nb; d += RT) hist[d] = 0;
  if (blockIdx.x == 0 && threadIdx.x == 0) status[0] = 0u;  // nothing else writes it yet
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * RTILE;
#pragma unroll 4
  for (int j = 0; j < RI; ++j) {
    const int64_t e = base + j * RT + threadIdx.x;
    if (e < N) {
      K key;
      if (!pack_key<K>(coords[e], B, X, Y, Z, &key)) key = sentinel;
      keys[e] = key;
      vals[e] = (int32_t)e;
      atomicAdd(&hist[digit_of<K>(key, shift, mask)], 1);  // LDS atomic
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < nb; d += RT) counts[(int64_t)d * ntiles + blockIdx.x] = hist[d];
}

template <typename K>
__global__ void __launch_bounds__(RT)
    hist_kernel(const K* __restrict__ keys, int64_t N, int shift, int dbits,
                int* __restrict__ counts, int ntiles) {
  __shared__ int hist[NBMAX];
  const int nb = 1 << dbits, mask = nb - 1;
  for (int d = threadIdx.x; d < nb; d += RT) hist[d] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * RTILE;
#pragma unroll 4
  for (int j = 0; j < RI; ++j) {
    const int64_t e = base + j * RT + threadIdx.x;
    if (e < N) atomicAdd(&hist[digit_of<K>(keys[e], shift, mask)], 1);
  }
  __syncthreads();
  for (int d = threadIdx.x; d < nb; d += RT) counts[(int64_t)d * ntiles + blockIdx.x] = hist[d];
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

// Block d: exclusive scan over tiles of digit d's counts (in place) and totals[d] = its sum.
// Coalesced: each round loads 256 consecutive counts, one per thread.
__global__ void __launch_bounds__(RT)
    scan_kernel(int* __restrict__ counts, int ntiles, int* __restrict__ totals) {
  __shared__ int wsum[WAVES];
  __shared__ int carry_s;
  int* c = counts + (int64_t)blockIdx.x * ntiles;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (threadIdx.x == 0) carry_s = 0;
  __syncthreads();
  for (int base = 0; base < ntiles; base += RT) {
    const int i = base + threadIdx.x;
    const int v = (i < ntiles) ? c[i] : 0;
    const int incl = wave_incl_scan(v);
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    int pre = carry_s, tot = 0;
#pragma unroll
    for (int ww = 0; ww < WAVES; ++ww) {
      if (ww < w) pre += wsum[ww];
      tot += wsum[ww];
    }
    if (i < ntiles) c[i] = pre + incl - v;
    __syncthreads();
    if (threadIdx.x == 0) carry_s += tot;
    __syncthreads();
  }
  if (threadIdx.x == 0) totals[blockIdx.x] = carry_s;
}

// One stable counting-sort pass over a tile of RTILE elements.  Wave w owns the contiguous
// sub-tile [w*RI*64, (w+1)*RI*64) and walks it item by item (lanes = consecutive elements), so
// element order = (wave, item, lane) and ranks are stable.
template <typename K>
__global__ void __launch_bounds__(RT)
    scatter_kernel(const K* __restrict__ ksrc, const int32_t* __restrict__ vsrc, int64_t N,
                   int shift, int dbits, const int* __restrict__ offs,
                   const int* __restrict__ totals, int ntiles,
                   K* __restrict__ kdst, int32_t* __restrict__ vdst) {
  __shared__ int wcnt[WAVES][NBMAX];
  __shared__ int dstart[NBMAX];
  __shared__ int gbase[NBMAX];
  __shared__ int wsum[WAVES], gsum[WAVES];
  __shared__ K sk[RTILE];
  __shared__ int32_t sv[RTILE];
  const int nb = 1 << dbits, mask = nb - 1;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int i = tid; i < WAVES * NBMAX; i += RT) (&wcnt[0][0])[i] = 0;
  __syncthreads();
  const int64_t tile0 = (int64_t)blockIdx.x * RTILE;
  const int64_t wbase = tile0 + (int64_t)w * (RI * 64);
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  K kk[RI];
  int32_t vv[RI];
  int lr[RI];
#pragma unroll
  for (int j = 0; j < RI; ++j) {
    const int64_t e = wbase + j * 64 + lane;
    const bool valid = e < N;
    kk[j] = valid ? ksrc[e] : (K)0;
    vv[j] = valid ? vsrc[e] : 0;
  }
#pragma unroll
  for (int j = 0; j < RI; ++j) {
    const int64_t e = wbase + j * 64 + lane;
    const bool valid = e < N;
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
      const int cnt = wcnt[w][d];
      lr[j] = cnt + before;
      if (before == 0) wcnt[w][d] = cnt + __popcll(peers);
    }
  }
  __syncthreads();
  // Per digit (thread tid = digit): exclusive prefix over waves, tile total, the tile-local start
  // of the digit, and its global start = (all elements of smaller digits) + (this digit in
  // earlier tiles).
  int tot = 0, gtot = 0;
  if (tid < nb) {
    int run = 0;
#pragma unroll
    for (int ww = 0; ww < WAVES; ++ww) {
      const int c = wcnt[ww][tid];
      wcnt[ww][tid] = run;
      run += c;
    }
    tot = run;
    gtot = totals[tid];
  }
  const int incl = wave_incl_scan(tot);
  const int gincl = wave_incl_scan(gtot);
  if (lane == 63) {
    wsum[w] = incl;
    gsum[w] = gincl;
  }
  __syncthreads();
  int pre = incl - tot, gpre = gincl - gtot;
  for (int ww = 0; ww < w; ++ww) {
    pre += wsum[ww];
    gpre += gsum[ww];
  }
  if (tid < nb) {
    dstart[tid] = pre;
    gbase[tid] = gpre + offs[(int64_t)tid * ntiles + blockIdx.x];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < RI; ++j) {
    const int64_t e = wbase + j * 64 + lane;
    if (e < N) {
      const int d = digit_of<K>(kk[j], shift, mask);
      const int p = dstart[d] + wcnt[w][d] + lr[j];
      sk[p] = kk[j];
      sv[p] = vv[j];
    }
  }
  __syncthreads();
  const int64_t rem = N - tile0;
  const int tile_n = rem < RTILE ? (int)rem : RTILE;
  for (int i = tid; i < tile_n; i += RT) {
    const K k = sk[i];
    const int d = digit_of<K>(k, shift, mask);
    const int64_t pos = (int64_t)gbase[d] + (i - dstart[d]);
    kdst[pos] = k;
    vdst[pos] = sv[i];
  }
}

// First index in [lo, hi) with keys[idx] >= t.
template <typename K>
__device__ __forceinline__ int64_t lower_bound(const K* __restrict__ keys, int64_t lo, int64_t hi,
                                               K t) {
  while (lo < hi) {
    const int64_t mid = lo + ((hi - lo) >> 1);
    if (keys[mid] < t) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// col_start[c] = lower_bound(keys, c*Z) for c in [0, ncol]; blocks own 256 consecutive columns
// and first bracket their key range with two searches over the whole array.
template <typename K>
__global__ void __launch_bounds__(RT)
    columns_kernel(const K* __restrict__ keys, int64_t n, int64_t Z, int64_t ncol,
                   int32_t* __restrict__ col_start) {
  __shared__ int64_t range[2];
  const int64_t c0 = (int64_t)blockIdx.x * RT;
  if (threadIdx.x < 2) {
    const int64_t cb = c0 + threadIdx.x * RT;
    range[threadIdx.x] = (cb > ncol) ? n : lower_bound<K>(keys, 0, n, (K)(cb * Z));
  }
  __syncthreads();
  const int64_t c = c0 + threadIdx.x;
  if (c <= ncol) col_start[c] = (int32_t)lower_bound<K>(keys, range[0], range[1], (K)(c * Z));
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

inline int bit_length(uint64_t v) {
  int b = 0;
  while (v) {
    ++b;
    v >>= 1;
  }
  return b;
}

template <typename K>
int radix_impl(tsc_ctx* ctx, const int32_t* coords, int64_t N, int32_t B, int32_t X, int32_t Y,
               int32_t Z, const int32_t dil[3], void* keys_out, int32_t* perm_out,
               int32_t* nbr_out, uint32_t* status_dev) {
  const int64_t cells = (int64_t)B * X * Y * Z;
  const K sentinel = (K)cells;  // above every valid key
  const int nbits = std::max(1, bit_length((uint64_t)cells));
  const int passes = (nbits + 7) / 8;
  const int dbits_full = (nbits + passes - 1) / passes;
  const int64_t ntiles = (N + RTILE - 1) / RTILE;
  const int64_t ncol = (int64_t)B * X * Y;
  const bool use_cols = ncol <= std::max<int64_t>(16 * N, int64_t(1) << 22);
  const int64_t S = (int64_t)(1 << dbits_full) * ntiles;
  size_t need = 2 * align_up((size_t)N * sizeof(K), 256) + 2 * align_up((size_t)N * 4, 256) +
                align_up((size_t)S * 4, 256) + align_up(NBMAX * 4, 256) + (use_cols ? align_up((size_t)(ncol + 1) * 4, 256) : 0);
  if (!keys_out) need += align_up((size_t)N * sizeof(K), 256);
  if (!perm_out) need += align_up((size_t)N * 4, 256);
  void* ws;
  int st = workspace(ctx, need, &ws);
  if (st) return st;
  Carve cv(ws);
  K* kA = cv.take<K>(N);
  int32_t* vA = cv.take<int32_t>(N);
  K* kB = cv.take<K>(N);
  int32_t* vB = cv.take<int32_t>(N);
  int* counts = cv.take<int>(S);
  int* totals = cv.take<int>(NBMAX);
  int32_t* cols = use_cols ? cv.take<int32_t>(ncol + 1) : nullptr;
  K* kOut = keys_out ? (K*)keys_out : cv.take<K>(N);
  int32_t* vOut = perm_out ? perm_out : cv.take<int32_t>(N);

  hipStream_t s = ctx->stream;
  if (N == 0) {
    clear_status_kernel<<<1, 64, 0, s>>>(status_dev);
    return check_hip(hipGetLastError(), "map_build_radix launch");
  }
  {
    ProfScope p(ctx, "radix_pack");
    pack_kernel<K><<<(unsigned)ntiles, RT, 0, s>>>((const int4*)coords, N, B, X, Y, Z, sentinel,
                                                    kA, vA, 0, std::min(dbits_full, nbits),
                                                    counts, (int)ntiles, status_dev);
  }
  K* kc = kA;
  int32_t* vc = vA;
  for (int p = 0; p < passes; ++p) {
    const int shift = p * dbits_full;
    const int dbits = std::min(dbits_full, nbits - shift);
    K* kd = (p == passes - 1) ? kOut : (kc == kA ? kB : kA);
    int32_t* vd = (p == passes - 1) ? vOut : (vc == vA ? vB : vA);
    if (p > 0) {
      ProfScope ps(ctx, "radix_hist");
      hist_kernel<K><<<(unsigned)ntiles, RT, 0, s>>>(kc, N, shift, dbits, counts, (int)ntiles);
    }
    {
      ProfScope ps(ctx, "radix_scan");
      scan_kernel<<<(unsigned)(1 << dbits), RT, 0, s>>>(counts, (int)ntiles, totals);
    }
    {
      ProfScope ps(ctx, "radix_scatter");
      scatter_kernel<K><<<(unsigned)ntiles, RT, 0, s>>>(kc, vc, N, shift, dbits, counts, totals,
                                                         (int)ntiles, kd, vd);
    }
    kc = kd;
    vc = vd;
  }
  if (use_cols) {
    ProfScope ps(ctx, "radix_columns");
    columns_kernel<K><<<(unsigned)((ncol + 1 + RT - 1) / RT), RT, 0, s>>>(kOut, N, Z, ncol, cols);
  }
  {
    ProfScope ps(ctx, "radix_fill");
    const int32_t per_xcd = mapk::fill_per_xcd(N);
    const unsigned grid = (unsigned)per_xcd * 8u;
    if (use_cols)
      mapk::fill_columns_kernel<K, ColumnLookup<K, true>><<<grid, mapk::kFillThreads, 0, s>>>(
          kOut, vOut, nullptr, N, sentinel, X, Y, Z, dil[0], dil[1], dil[2],
          ColumnLookup<K, true>{kOut, cols, vOut, N}, per_xcd, nbr_out, status_dev);
    else
      mapk::fill_columns_kernel<K, ColumnLookup<K, false>><<<grid, mapk::kFillThreads, 0, s>>>(
          kOut, vOut, nullptr, N, sentinel, X, Y, Z, dil[0], dil[1], dil[2],
          ColumnLookup<K, false>{kOut, nullptr, vOut, N}, per_xcd, nbr_out, status_dev);
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

}  // namespace tsc
