// Row order for the conv kernels: rows sorted by their set of present neighbors.
//
// The conv kernels process output rows in tiles (32 to 256 consecutive entries of `order`) and
// skip a tap only when no row of the tile has that neighbor.  In key order a tile of a thin
// shell touches nearly all 27 taps although each row has ~9-17 neighbors, so most tap work is
// multiplication by absent (zero) rows.  The order sorts rows inside windows of 262144
// consecutive key-sorted rows (spatially grouped, so gathers keep some locality) by their 26-bit
// mask of present neighbors (corner taps in the top bits, then edges, then faces; tap 13, the
// row itself, is always present), ranked in the reflected binary (Gray) sequence: masks that share
// their leading taps sit next to each other, and consecutive ones differ in as few taps as the
// sequence allows, so a tile's union of taps stays close to one row's.  Ties keep key order.
//
// Stable LSD radix sort, three passes of <= 9 bits, over tiles of 16384 rows (16 per window):
//   mask     key = mask of row perm[i], val = perm[i]; tile histogram of digit 0
//   scan     per window: digit-major, tile-minor exclusive offsets of the 16 tiles' counts
//   scatter  per tile: wave-ballot stable ranks (one ballot per digit bit -> peer mask; popcount
//            of lower peers + the wave's running count; per-digit offsets across waves), written
//            to window start + offset of (tile, digit) + rank
//   hist     tile histogram of the next digit
// Processed taps / valid taps (CPU model of the tiles) on the 2-voxel shells in 128^3 with
// 256-row tiles: key order 1.65, 65536-row windows with taps in index order 1.36, corner-first
// 1.28, 262144-row windows 1.18 (the wide conv measured 6 % faster than with 65536), Gray rank
// 1.166 (2 x 30k-voxel shells in 64^3: 1.344 -> 1.324); on the 1-voxel 512^3 shell with 32-row
// tiles: 1.13 (65536), 1.049 (262144), 1.044 (Gray rank).

#include <utility>

#include "tsc_internal.h"

namespace tsc {
namespace {

constexpr int kOrdThreads = 1024;
constexpr int kOrdItems = 16;
constexpr int kOrdTile = kOrdThreads * kOrdItems;  // 16384 rows per tile
constexpr int kOrdTilesPerWin = 16;                // 262144 rows per window
constexpr int kOrdWaves = kOrdThreads / 64;
constexpr int kOrdDigitBits = 9;
constexpr int kOrdBins = 1 << kOrdDigitBits;
constexpr int kOrdMaskBits = 26;
constexpr int kOrdPasses = (kOrdMaskBits + kOrdDigitBits - 1) / kOrdDigitBits;
// Significance of the taps in the sort key, most significant first: the 8 corners, the 12 edges,
// then the 6 faces (tap 13 is always present).  Corner neighbors are the rarest on surfaces, so
// grouping rows by them first keeps a 256-row tile's union of taps smallest (measured on the 2-
// voxel shells: processed/valid taps 1.28 instead of 1.36 with taps in index order).
__device__ __constant__ const int kMaskTap[kOrdMaskBits] = {0, 2,  6,  8,  18, 20, 24, 26, 1,
                                                            3, 5,  7,  9,  11, 15, 17, 19, 21,
                                                            23, 25, 4, 10, 12, 14, 16, 22};

__device__ __forceinline__ int block_excl_scan(int v, int* wsum, int nw) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(incl, off, 64);
    if (lane >= off) incl += t;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  int pre = incl - v;
  for (int ww = 0; ww < w && ww < nw; ++ww) pre += wsum[ww];
  __syncthreads();
  return pre;
}

__device__ __forceinline__ int digit(uint32_t k, int shift) {
  return (int)((k >> shift) & (uint32_t)(kOrdBins - 1));
}

__global__ void __launch_bounds__(kOrdThreads)
    ord_mask_kernel(const int32_t* __restrict__ nbr, const int32_t* __restrict__ perm,
                    int64_t n, uint32_t* __restrict__ keys, int32_t* __restrict__ vals,
                    int* __restrict__ counts) {
  __shared__ int hist[kOrdBins];
  const int tid = threadIdx.x;
  for (int d = tid; d < kOrdBins; d += kOrdThreads) hist[d] = 0;
  __syncthreads();
  const int64_t t0 = (int64_t)blockIdx.x * kOrdTile;
#pragma unroll 4
  for (int j = 0; j < kOrdItems; ++j) {
    const int64_t i = t0 + j * kOrdThreads + tid;
    if (i < n) {
      const int32_t r = perm ? perm[i] : (int32_t)i;
      const int32_t* nr = nbr + (int64_t)r * 27;
      uint32_t m = 0;
#pragma unroll
      for (int k = 0; k < kOrdMaskBits; ++k) m = (m << 1) | (uint32_t)(nr[kMaskTap[k]] >= 0);
      // Sort by the mask's position in the reflected binary (Gray) sequence: neighbors in that
      // sequence differ in one tap, where numeric neighbors can differ in many low taps.
      m ^= m >> 1;
      m ^= m >> 2;
      m ^= m >> 4;
      m ^= m >> 8;
      m ^= m >> 16;
      keys[i] = m;
      vals[i] = r;
      atomicAdd(&hist[digit(m, 0)], 1);
    }
  }
  __syncthreads();
  for (int d = tid; d < kOrdBins; d += kOrdThreads) counts[blockIdx.x * kOrdBins + d] = hist[d];
}

__global__ void __launch_bounds__(kOrdThreads)
    ord_hist_kernel(const uint32_t* __restrict__ keys, int64_t n, int shift,
                    int* __restrict__ counts) {
  __shared__ int hist[kOrdBins];
  const int tid = threadIdx.x;
  for (int d = tid; d < kOrdBins; d += kOrdThreads) hist[d] = 0;
  __syncthreads();
  const int64_t t0 = (int64_t)blockIdx.x * kOrdTile;
#pragma unroll 4
  for (int j = 0; j < kOrdItems; ++j) {
    const int64_t i = t0 + j * kOrdThreads + tid;
    if (i < n) atomicAdd(&hist[digit(keys[i], shift)], 1);
  }
  __syncthreads();
  for (int d = tid; d < kOrdBins; d += kOrdThreads) counts[blockIdx.x * kOrdBins + d] = hist[d];
}

// One block per window, thread = digit: offs[t][d] = (elements of smaller digits in the window)
// + (digit d in the window's earlier tiles).
__global__ void __launch_bounds__(kOrdBins)
    ord_scan_kernel(const int* __restrict__ counts, int ntiles, int* __restrict__ offs) {
  __shared__ int wsum[kOrdBins / 64];
  const int d = threadIdx.x;
  const int tb = blockIdx.x * kOrdTilesPerWin;
  const int nt = min(kOrdTilesPerWin, ntiles - tb);
  int c[kOrdTilesPerWin], tot = 0;
#pragma unroll
  for (int t = 0; t < kOrdTilesPerWin; ++t) {
    c[t] = t < nt ? counts[(tb + t) * kOrdBins + d] : 0;
    tot += c[t];
  }
  int run = block_excl_scan(tot, wsum, kOrdBins / 64);
#pragma unroll
  for (int t = 0; t < kOrdTilesPerWin; ++t) {
    if (t < nt) offs[(tb + t) * kOrdBins + d] = run;
    run += c[t];
  }
}

// Stable scatter of one tile.  Wave w ranks the contiguous run [w*ipw*64, (w+1)*ipw*64) of the
// tile item by item (lanes = consecutive elements), so element order = (wave, item, lane).
__global__ void __launch_bounds__(kOrdThreads)
    ord_scatter_kernel(const uint32_t* __restrict__ ksrc, const int32_t* __restrict__ vsrc,
                       int64_t n, int shift, int dbits, const int* __restrict__ offs,
                       uint32_t* __restrict__ kdst, int32_t* __restrict__ vdst) {
  __shared__ int wcnt[kOrdWaves][kOrdBins];
  __shared__ int start[kOrdBins];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * kOrdTile;
  const int64_t win0 = (int64_t)(blockIdx.x / kOrdTilesPerWin) * kOrdTilesPerWin * kOrdTile;
  const int size = (int)((n - t0) < kOrdTile ? (n - t0) : kOrdTile);
  for (int i = tid; i < kOrdWaves * kOrdBins; i += kOrdThreads) (&wcnt[0][0])[i] = 0;
  for (int d = tid; d < kOrdBins; d += kOrdThreads) start[d] = offs[blockIdx.x * kOrdBins + d];
  __syncthreads();
  const int ipw = ((size + 63) / 64 + kOrdWaves - 1) / kOrdWaves;
  const int wfirst = w * ipw * 64;
  const int wlimit = min(size, wfirst + ipw * 64);
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int mask = (1 << dbits) - 1;
  uint32_t kk[kOrdItems];
  int32_t vv[kOrdItems];
  int lr[kOrdItems];
#pragma unroll
  for (int j = 0; j < kOrdItems; ++j) {
    const int e = wfirst + j * 64 + lane;
    const bool valid = e < wlimit;
    kk[j] = valid ? ksrc[t0 + e] : 0u;
    vv[j] = valid ? vsrc[t0 + e] : 0;
  }
#pragma unroll
  for (int j = 0; j < kOrdItems; ++j) {
    lr[j] = 0;
    if (j >= ipw) continue;  // uniform
    const bool valid = wfirst + j * 64 + lane < wlimit;
    const int d = (int)((kk[j] >> shift) & (uint32_t)mask);
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < dbits; ++b) {
      const bool bit = (d >> b) & 1;
      const uint64_t mb = __ballot(valid && bit);
      peers &= bit ? mb : ~mb;
    }
    if (valid) {
      const int before = __popcll(peers & lt_mask);
      const int c = wcnt[w][d];
      lr[j] = c + before;
      if (before == 0) wcnt[w][d] = c + __popcll(peers);
    }
  }
  __syncthreads();
  if (tid < kOrdBins) {  // per digit: exclusive offsets of the waves
    int run = 0;
#pragma unroll
    for (int ww = 0; ww < kOrdWaves; ++ww) {
      const int c = wcnt[ww][tid];
      wcnt[ww][tid] = run;
      run += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kOrdItems; ++j) {
    const int e = wfirst + j * 64 + lane;
    if (j < ipw && e < wlimit) {
      const int d = (int)((kk[j] >> shift) & (uint32_t)mask);
      const int64_t pos = win0 + start[d] + wcnt[w][d] + lr[j];
      if (kdst) kdst[pos] = kk[j];
      vdst[pos] = vv[j];
    }
  }
}

}  // namespace

int conv_order_launch(tsc_ctx* ctx, const int32_t* nbr, const int32_t* perm, int64_t N,
                      int32_t* order) {
  if (N == 0) return TSC_OK;
  const int ntiles = (int)((N + kOrdTile - 1) / kOrdTile);
  const int nwin = (ntiles + kOrdTilesPerWin - 1) / kOrdTilesPerWin;
  const size_t need = 2 * align_up((size_t)N * 4, 256) + 2 * align_up((size_t)N * 4, 256) +
                      2 * align_up((size_t)ntiles * kOrdBins * 4, 256);
  void* ws;
  int st = workspace(ctx, need, &ws);
  if (st) return st;
  Carve cv(ws);
  uint32_t* kA = cv.take<uint32_t>(N);
  uint32_t* kB = cv.take<uint32_t>(N);
  int32_t* vA = cv.take<int32_t>(N);
  int32_t* vB = cv.take<int32_t>(N);
  int* counts = cv.take<int>((int64_t)ntiles * kOrdBins);
  int* offs = cv.take<int>((int64_t)ntiles * kOrdBins);
  hipStream_t s = ctx->stream;
  ProfScope p(ctx, "conv_order");
  ord_mask_kernel<<<ntiles, kOrdThreads, 0, s>>>(nbr, perm, N, kA, vA, counts);
  uint32_t *kc = kA, *kn = kB;
  int32_t *vc = vA, *vn = vB;
  for (int pass = 0; pass < kOrdPasses; ++pass) {
    const int shift = pass * kOrdDigitBits;
    const int dbits = kOrdMaskBits - shift < kOrdDigitBits ? kOrdMaskBits - shift : kOrdDigitBits;
    const bool last = pass == kOrdPasses - 1;
    if (pass > 0) ord_hist_kernel<<<ntiles, kOrdThreads, 0, s>>>(kc, N, shift, counts);
    ord_scan_kernel<<<nwin, kOrdBins, 0, s>>>(counts, ntiles, offs);
    ord_scatter_kernel<<<ntiles, kOrdThreads, 0, s>>>(kc, vc, N, shift, dbits, offs,
                                                      last ? nullptr : kn,
                                                      last ? order : vn);
    std::swap(kc, kn);
    std::swap(vc, vn);
  }
  return check_hip(hipGetLastError(), "conv_order launch");
}

}  // namespace tsc
