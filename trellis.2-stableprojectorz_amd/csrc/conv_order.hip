// Row order for the conv kernels: rows sorted by their set of present neighbors.
//
// The conv kernels process output rows in tiles (32 or 128 consecutive entries of `order`) and
// skip a tap only when no row of the tile has that neighbor.  In key order a tile of a thin
// shell touches nearly all 27 taps although each row has ~9-17 neighbors, so most tap work is
// multiplication by absent (zero) rows.  This kernel sorts rows inside windows of kOrdWin
// consecutive key-sorted rows (spatially compact, so gathers stay local) by their 26-bit mask of
// present neighbors (tap 0 in the top bit; tap 13, the row itself, is always present): numeric
// order puts masks that share their leading taps next to each other, so a tile's union of taps
// stays close to one row's.  One block per window: the masks and window positions (uint16) sit
// in LDS and three stable LSD passes of <= 9 bits rank them with wave ballots (peer mask per
// digit, popcount of lower peers + the wave's running count, cross-wave offsets per digit).
// Measured utilisation (valid taps / processed taps) on the thin shells: key order 0.37 (1-voxel
// shell, 32-row tiles) and 0.61 (2-voxel shells, 128-row tiles); sorted windows 0.81 and 0.72.

#include "tsc_internal.h"

namespace tsc {
namespace {

constexpr int kOrdThreads = 1024;
constexpr int kOrdItems = 16;
constexpr int kOrdWin = kOrdThreads * kOrdItems;  // 16384 rows per window
constexpr int kOrdWaves = kOrdThreads / 64;
constexpr int kOrdDigitBits = 9;
constexpr int kOrdBins = 1 << kOrdDigitBits;
constexpr int kOrdMaskBits = 26;

__device__ __forceinline__ int block_excl_scan_1024(int v, int* wsum) {
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
  for (int ww = 0; ww < w; ++ww) pre += wsum[ww];
  __syncthreads();
  return pre;
}

__global__ void __launch_bounds__(kOrdThreads)
    conv_order_kernel(const int32_t* __restrict__ nbr, const int32_t* __restrict__ perm,
                      int64_t n, int32_t* __restrict__ order) {
  __shared__ uint32_t skey[kOrdWin];
  __shared__ uint16_t spos[kOrdWin];
  __shared__ int wcnt[kOrdWaves][kOrdBins];
  __shared__ int run[kOrdBins];
  __shared__ int wsum[kOrdWaves];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t w0 = (int64_t)blockIdx.x * kOrdWin;
  const int size = (int)((n - w0) < kOrdWin ? (n - w0) : kOrdWin);
  for (int i = tid; i < size; i += kOrdThreads) {
    const int32_t r = perm ? perm[w0 + i] : (int32_t)(w0 + i);
    const int32_t* nr = nbr + (int64_t)r * 27;
    uint32_t m = 0;
#pragma unroll
    for (int v = 0; v < 27; ++v) {
      if (v == 13) continue;
      m = (m << 1) | (uint32_t)(nr[v] >= 0);
    }
    skey[i] = m;
    spos[i] = (uint16_t)i;
  }
  // Wave w ranks the contiguous run [w*ipw*64, (w+1)*ipw*64) of the window.
  const int ipw = ((size + 63) / 64 + kOrdWaves - 1) / kOrdWaves;
  const int wfirst = w * ipw * 64;
  const int wlimit = min(size, wfirst + ipw * 64);
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  constexpr int passes = (kOrdMaskBits + kOrdDigitBits - 1) / kOrdDigitBits;
  for (int p = 0; p < passes; ++p) {
    const int shift = p * kOrdDigitBits;
    const int dbits = min(kOrdDigitBits, kOrdMaskBits - shift);
    const int mask = (1 << dbits) - 1;
    for (int i = tid; i < kOrdWaves * kOrdBins; i += kOrdThreads) (&wcnt[0][0])[i] = 0;
    __syncthreads();
    uint32_t kk[kOrdItems];
    uint16_t pp[kOrdItems];
    int lr[kOrdItems];
#pragma unroll
    for (int j = 0; j < kOrdItems; ++j) {
      const int e = wfirst + j * 64 + lane;
      const bool valid = e < wlimit;
      kk[j] = valid ? skey[e] : 0u;
      pp[j] = valid ? spos[e] : (uint16_t)0;
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
    // Per digit (thread t < kOrdBins): per-wave exclusive offsets and the digit total; then the
    // exclusive scan over digits gives each digit's start.
    int tot = 0;
    if (tid < kOrdBins) {
#pragma unroll
      for (int ww = 0; ww < kOrdWaves; ++ww) {
        const int c = wcnt[ww][tid];
        wcnt[ww][tid] = tot;
        tot += c;
      }
    }
    const int start = block_excl_scan_1024(tid < kOrdBins ? tot : 0, wsum);
    if (tid < kOrdBins) run[tid] = start;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kOrdItems; ++j) {
      const int e = wfirst + j * 64 + lane;
      if (j < ipw && e < wlimit) {
        const int d = (int)((kk[j] >> shift) & (uint32_t)mask);
        const int pos = run[d] + wcnt[w][d] + lr[j];
        skey[pos] = kk[j];
        spos[pos] = pp[j];
      }
    }
    __syncthreads();
  }
  for (int i = tid; i < size; i += kOrdThreads)
    order[w0 + i] = perm ? perm[w0 + spos[i]] : (int32_t)(w0 + spos[i]);
}

}  // namespace

int conv_order_launch(tsc_ctx* ctx, const int32_t* nbr, const int32_t* perm, int64_t N,
                      int32_t* order) {
  if (N == 0) return TSC_OK;
  ProfScope p(ctx, "conv_order");
  const unsigned grid = (unsigned)((N + kOrdWin - 1) / kOrdWin);
  conv_order_kernel<<<grid, kOrdThreads, 0, ctx->stream>>>(nbr, perm, N, order);
  return check_hip(hipGetLastError(), "conv_order launch");
}

}  // namespace tsc
