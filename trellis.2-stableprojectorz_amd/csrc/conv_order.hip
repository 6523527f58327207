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
// Stable LSD radix sort, three passes of <= 9 bits, over tiles of 4096 rows (64 per window):
//   rowmask  per row, reading the map in row order: the Gray rank of its mask
//   mask     key = rowmask[perm[i]], val = perm[i]; tile histogram of digit 0
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

#include <climits>
#include <utility>

#include "tsc_internal.h"

namespace tsc {
namespace {

constexpr int kOrdThreads = 1024;
// 4096-row tiles: 370 blocks per pass at 1.5 M rows and 60 at 243 k, against 93 / 15 with
// 16384-row tiles, which left most CUs idle (conv order 254 -> 209 us at 1.5 M rows, 187 ->
// 127 us at 243 k; 2048- and 8192-row tiles measured slower).
constexpr int kOrdItems = 4;
constexpr int kOrdTile = kOrdThreads * kOrdItems;  // 4096 rows per tile
constexpr int kOrdTilesPerWin = 64;                // 262144 rows per window
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

// Row masks in row order: each block copies the neighbor rows of 256 consecutive rows into LDS with
// coalesced loads (27 dwords per thread), then thread t forms row r0 + t's 26-bit mask and ranks
// it in the reflected binary (Gray) sequence, whose neighbors differ in one tap where numeric
// neighbors can differ in many low taps.  Reading the map in row order is ~2.5x faster than
// reading its 108-byte rows in key order (random addresses, two cache lines each).
constexpr int kRowThreads = 256;
__global__ void __launch_bounds__(kRowThreads)
    ord_rowmask_kernel(const int32_t* __restrict__ nbr, int64_t n, uint32_t* __restrict__ rowmask) {
  __shared__ int32_t s[kRowThreads * 27];
  const int tid = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.x * kRowThreads;
  const int rows = (int)(n - r0 < kRowThreads ? n - r0 : kRowThreads);
  const int32_t* src = nbr + r0 * 27;
  if (rows == kRowThreads) {
    int32_t v[27];
#pragma unroll
    for (int k = 0; k < 27; ++k) v[k] = src[k * kRowThreads + tid];
#pragma unroll
    for (int k = 0; k < 27; ++k) s[k * kRowThreads + tid] = v[k];
  } else {
    for (int w = tid; w < rows * 27; w += kRowThreads) s[w] = src[w];
  }
  __syncthreads();
  if (tid < rows) {
    const int32_t* nr = s + tid * 27;  // stride 27 words: conflict-free
    uint32_t m = 0;
#pragma unroll
    for (int k = 0; k < kOrdMaskBits; ++k) m = (m << 1) | (uint32_t)(nr[kMaskTap[k]] >= 0);
    m ^= m >> 1;
    m ^= m >> 2;
    m ^= m >> 4;
    m ^= m >> 8;
    m ^= m >> 16;
    rowmask[r0 + tid] = m;
  }
}

// Keys of the first sort pass: key = rank of row perm[i]'s mask, val = perm[i]; tile histogram of
// digit 0.
__global__ void __launch_bounds__(kOrdThreads)
    ord_mask_kernel(const uint32_t* __restrict__ rowmask, const int32_t* __restrict__ perm,
                    int64_t n, uint32_t* __restrict__ keys, int32_t* __restrict__ vals,
                    int* __restrict__ counts) {
  __shared__ int hist[kOrdBins];
  const int tid = threadIdx.x;
  for (int d = tid; d < kOrdBins; d += kOrdThreads) hist[d] = 0;
  __syncthreads();
  const int64_t t0 = (int64_t)blockIdx.x * kOrdTile;
  if (t0 + kOrdTile <= n) {
    int32_t r[kOrdItems];
#pragma unroll
    for (int j = 0; j < kOrdItems; ++j) {
      const int64_t i = t0 + j * kOrdThreads + tid;
      r[j] = perm ? perm[i] : (int32_t)i;
    }
    uint32_t m[kOrdItems];
#pragma unroll
    for (int j = 0; j < kOrdItems; ++j) m[j] = rowmask[r[j]];
#pragma unroll
    for (int j = 0; j < kOrdItems; ++j) {
      const int64_t i = t0 + j * kOrdThreads + tid;
      keys[i] = m[j];
      vals[i] = r[j];
      atomicAdd(&hist[digit(m[j], 0)], 1);
    }
  } else {
    for (int j = 0; j < kOrdItems; ++j) {
      const int64_t i = t0 + j * kOrdThreads + tid;
      if (i < n) {
        const int32_t r = perm ? perm[i] : (int32_t)i;
        const uint32_t m = rowmask[r];
        keys[i] = m;
        vals[i] = r;
        atomicAdd(&hist[digit(m, 0)], 1);
      }
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

// Greedy tile grouping inside chunks of kGrChunk rows of the mask-sorted order (one block per
// chunk).  The sort alone leaves tiles that straddle many short runs of distinct masks (on the
// 2-voxel shells ~16 k distinct masks for 64-243 k rows); this pass rebuilds each 256-row tile
// around one popular mask and the masks contained in it:
//   entries  the chunk's runs of equal masks, ordered by row count capped at 255 (descending),
//            then by the sort key; each keeps its next unused position and its remaining rows
//   tile     seed = the first entry with rows left; OR = its mask.  Repeat: take rows, in entry
//            order, from every entry whose mask lies inside OR, until the tile is full; if rows
//            are still missing, add to OR the entry mask that brings the fewest new taps (lowest
//            entry index on ties) and take again.  Every added mask brings at least one new tap,
//            so a tile completes after at most 26 growths.
// Chunks of consecutive sorted rows share their leading taps, so grouping inside a chunk loses
// little against one pool of all rows (processed / valid taps with 256-row tiles on the 2-voxel
// shells: sorted 1.166 / 1.324, chunks of 4096 1.112 / 1.227, of 8192 1.107 / 1.222, one pool
// 1.101 / 1.213; a block's passes run one after another, so 4096-row chunks halve the kernel's
// critical path for +0.5 % of taps; the count cap changes nothing measurable and makes the
// entry order an 8-bit stable counting sort).
// Thread t owns entries [t*E, t*E + E) in registers throughout the tile loop, so a pass over the
// entries is register work plus two block reductions.  The loops over a thread's entries stop
// after E steps (E is block-uniform, mostly 1): unrolled to kGrPerThread with only per-thread
// guards they cost every pass 8x the instructions (conv order 276 -> 253 us at 1.5 M voxels).
constexpr int kGrChunk = 4096;   // rows per chunk (and at most this many entries)
constexpr int kGrThreads = 512;
constexpr int kGrTile = 256;     // rows per tile of the 256-row conv kernels
constexpr int kGrPerThread = kGrChunk / kGrThreads;  // rows, and entries at most, per thread
static_assert(kOrdTilesPerWin * kOrdTile % kGrChunk == 0, "chunks never straddle a window");
static_assert(kGrChunk % kGrTile == 0, "chunks hold whole tiles");
static_assert(kGrTile <= kGrThreads, "one thread per tile slot");

// Entry state: mask (26 bits) | next position in the chunk << 26 | rows left << 40.  Positions
// and counts reach kGrChunk itself (a run that ends the chunk), so each field has 14 bits.
static_assert(kGrChunk < (1 << 14), "14-bit position and count fields");
__device__ __forceinline__ uint32_t gr_mask(uint64_t e) { return (uint32_t)(e & 0x3ffffffu); }
__device__ __forceinline__ int gr_pos(uint64_t e) { return (int)((e >> 26) & 0x3fffu); }
__device__ __forceinline__ int gr_left(uint64_t e) { return (int)(e >> 40); }
__device__ __forceinline__ uint64_t gr_make(uint32_t mask, int pos, int left) {
  return (uint64_t)mask | ((uint64_t)pos << 26) | ((uint64_t)left << 40);
}

// Inclusive wave64 scans on DPP lane moves (row_shr inside each 16-lane row, then row_bcast:15
// and row_bcast:31 across rows); lanes whose source is outside the row keep the identity.
template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp_mov(int old, int x) {
  return __builtin_amdgcn_update_dpp(old, x, CTRL, ROWS, 0xf, false);
}
__device__ __forceinline__ int wave_incl_add(int x) {
  x += dpp_mov<0x111, 0xf>(0, x);  // row_shr:1
  x += dpp_mov<0x112, 0xf>(0, x);  // row_shr:2
  x += dpp_mov<0x114, 0xf>(0, x);  // row_shr:4
  x += dpp_mov<0x118, 0xf>(0, x);  // row_shr:8
  x += dpp_mov<0x142, 0xa>(0, x);  // row_bcast:15 into rows 1 and 3
  x += dpp_mov<0x143, 0xc>(0, x);  // row_bcast:31 into rows 2 and 3
  return x;
}
__device__ __forceinline__ uint32_t umin32(uint32_t a, uint32_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint32_t wave_incl_umin(uint32_t x) {
  const int m = -1;  // identity: 0xffffffff
  x = umin32(x, (uint32_t)dpp_mov<0x111, 0xf>(m, (int)x));
  x = umin32(x, (uint32_t)dpp_mov<0x112, 0xf>(m, (int)x));
  x = umin32(x, (uint32_t)dpp_mov<0x114, 0xf>(m, (int)x));
  x = umin32(x, (uint32_t)dpp_mov<0x118, 0xf>(m, (int)x));
  x = umin32(x, (uint32_t)dpp_mov<0x142, 0xa>(m, (int)x));
  x = umin32(x, (uint32_t)dpp_mov<0x143, 0xc>(m, (int)x));
  return x;
}
__device__ __forceinline__ int wave_incl_max(int x) {  // x >= -1
  x = max(x, dpp_mov<0x111, 0xf>(-1, x));
  x = max(x, dpp_mov<0x112, 0xf>(-1, x));
  x = max(x, dpp_mov<0x114, 0xf>(-1, x));
  x = max(x, dpp_mov<0x118, 0xf>(-1, x));
  x = max(x, dpp_mov<0x142, 0xa>(-1, x));
  x = max(x, dpp_mov<0x143, 0xc>(-1, x));
  return x;
}

// Sort digit of entry e (runs in run order: head[e] = first position): 255 - min(rows, 255).
__device__ __forceinline__ int gr_digit(const int32_t* head, int e) {
  const int rows = head[e + 1] - head[e];
  return 255 - (rows < 255 ? rows : 255);
}

__global__ void __launch_bounds__(kGrThreads)
    ord_greedy_kernel(const uint32_t* __restrict__ keys, const int32_t* __restrict__ vals,
                      int64_t n, int32_t* __restrict__ order) {
  __shared__ int32_t head[kGrChunk + 1];  // run starts; later the tile's segment marks
  __shared__ int32_t idxa[kGrChunk];      // entry order (sort); later each output slot's source
  __shared__ int32_t buf[8 * kGrThreads + kGrChunk];  // sort counters | entry order; later masks
  __shared__ int wsum[kGrThreads / 64];
  __shared__ int wmax[kGrThreads / 64];
  __shared__ int wtot[2][kGrThreads / 64];        // per-pass wave sums (two buffers by parity)
  __shared__ uint32_t wbest[2][kGrThreads / 64];  // per-pass wave minima
  __shared__ uint32_t wseed[kGrThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t c0 = (int64_t)blockIdx.x * kGrChunk;
  const int nc = (int)(n - c0 < kGrChunk ? n - c0 : kGrChunk);

  // Runs of equal keys: thread t owns positions [t*P, t*P + P).
  int nd;
  {
    uint32_t hb = 0;  // bit j: position p0 + j starts a run
    const int p0 = tid * kGrPerThread;
    uint32_t prev = p0 > 0 && p0 <= nc ? keys[c0 + p0 - 1] : 0u;
#pragma unroll
    for (int j = 0; j < kGrPerThread; ++j) {
      const int i = p0 + j;
      const uint32_t k = i < nc ? keys[c0 + i] : 0u;
      hb |= (i < nc && (i == 0 || k != prev) ? 1u : 0u) << j;
      prev = k;
    }
    int e = block_excl_scan(__popc(hb), wsum, kGrThreads / 64);
    nd = 0;
#pragma unroll
    for (int ww = 0; ww < kGrThreads / 64; ++ww) nd += wsum[ww];
    for (uint32_t m = hb; m; m &= m - 1) head[e++] = p0 + __ffs(m) - 1;
    if (tid == 0) head[nd] = nc;
  }
  // Entries per thread: contiguous runs [ebeg, ebeg + ne).
  const int E = (nd + kGrThreads - 1) / kGrThreads;
  const int ebeg = tid * E;
  const int ne = max(0, min(nd - ebeg, E));
  for (int i = tid; i < nd; i += kGrThreads) idxa[i] = i;
  __syncthreads();
  // Stable LSD counting sort of the entries by gr_digit, three passes of 3 bits: per-thread digit
  // counts in a digit-major [8][kGrThreads] matrix, one block scan, stable placement; the passes
  // alternate between idxa and idxb and end in idxb.
  constexpr int kDig = 8, kCpt = kDig * kGrThreads / kGrThreads;  // counters per thread in the scan
  int32_t* const cnt = buf;  // [kDig][kGrThreads]
  int32_t* const idxb = buf + kDig * kGrThreads;
  static_assert(kDig == 8 && kGrChunk <= kDig * kGrThreads, "counters, order and masks fit buf");
  for (int pass = 0; pass < 3; ++pass) {
    const int32_t* src = (pass & 1) ? idxb : idxa;
    int32_t* dst = (pass & 1) ? idxa : idxb;
    const int sh = 3 * pass;
    // column tid of the counter matrix belongs to this thread alone
    for (int d = 0; d < kDig; ++d) cnt[d * kGrThreads + tid] = 0;
    for (int j = 0; j < ne; ++j)
      ++cnt[((gr_digit(head, src[ebeg + j]) >> sh) & (kDig - 1)) * kGrThreads + tid];
    __syncthreads();
    // exclusive scan of the counters in digit-major order: thread t scans [t*kCpt, t*kCpt + kCpt)
    int sum = 0;
    for (int q = 0; q < kCpt; ++q) sum += cnt[tid * kCpt + q];
    int pre = block_excl_scan(sum, wsum, kGrThreads / 64);
    for (int q = 0; q < kCpt; ++q) {
      const int c = cnt[tid * kCpt + q];
      cnt[tid * kCpt + q] = pre;
      pre += c;
    }
    __syncthreads();
    for (int j = 0; j < ne; ++j) {
      const int e = src[ebeg + j];
      dst[cnt[((gr_digit(head, e) >> sh) & (kDig - 1)) * kGrThreads + tid]++] = e;
    }
    __syncthreads();
  }
  // This thread's entries (sorted positions ebeg..ebeg+ne) into registers; masks to LDS.
  uint64_t my[kGrPerThread];
#pragma unroll
  for (int j = 0; j < kGrPerThread; ++j) {
    my[j] = 0;
    if (j < ne) {
      const int e = idxb[ebeg + j];
      const int a = head[e];
      const uint32_t rank = keys[c0 + a];
      my[j] = gr_make(rank ^ (rank >> 1), a, head[e + 1] - a);
    }
  }
  __syncthreads();
  uint32_t* const emask = (uint32_t*)buf;
#pragma unroll
  for (int j = 0; j < kGrPerThread; ++j)
    if (j < ne) emask[ebeg + j] = gr_mask(my[j]);
  // Segment marks over the chunk's output slots (the run starts are no longer needed): a taking
  // entry marks the first slot it fills with (its source position - that slot + kMarkOff); the
  // slots after it up to the next mark come from the same run.  The marks are resolved once for
  // the whole chunk after the tile loop (a tile's slot 0 is always marked), so a tile costs its
  // passes plus one seed reduction; resolving them per tile took two more block barriers per
  // tile (the kernel ran ~7 % longer).  The seed reduction's barrier orders this clear before
  // the first mark.
  int32_t* const mark = head;
  constexpr int kMarkOff = 1 << 16;
  for (int i = tid; i < nc; i += kGrThreads) mark[i] = 0;
  const int ntile = (nc + kGrTile - 1) / kGrTile;
  for (int t = 0; t < ntile; ++t) {
    const int rows = min(kGrTile, nc - t * kGrTile);
    const int base = t * kGrTile;
    // seed: the first entry with rows left
    uint32_t fa = ~0u;
#pragma unroll
    for (int j = 0; j < kGrPerThread; ++j) {
      if (j >= E) break;  // uniform: no thread owns more entries
      if (j < ne && gr_left(my[j]) > 0 && fa == ~0u) fa = (uint32_t)(ebeg + j);
    }
    fa = wave_incl_umin(fa);
    if (lane == 63) wseed[wid] = fa;
    __syncthreads();
#pragma unroll
    for (int ww = 0; ww < kGrThreads / 64; ++ww) fa = umin32(fa, wseed[ww]);
    uint32_t orm = emask[fa];  // rows remain, so an entry with rows exists
    int need = rows, fill = 0;
    for (int iter = 0;; ++iter) {
      if (iter >= 27) orm = ~0u;  // 26 growths fill OR; guard only
      // One block reduction per pass: the rows of the entries inside OR (to be taken, in entry
      // order) and, among the other entries with rows left, the one whose mask adds the fewest
      // taps (lowest index on ties) -- the growth if the tile is still short.  Taking touches
      // only entries inside OR, so the growth candidate stays valid after it.
      int sum = 0;
      uint32_t cand = ~0u;
#pragma unroll
      for (int j = 0; j < kGrPerThread; ++j) {
        if (j >= E) break;
        const int left = gr_left(my[j]);
        if (j < ne && left > 0) {
          const uint32_t out = gr_mask(my[j]) & ~orm;
          if (out == 0u) sum += left;
          else cand = umin32(cand, ((uint32_t)__popc(out) << 14) | (uint32_t)(ebeg + j));
        }
      }
      const int incl = wave_incl_add(sum);
      const uint32_t wmin = wave_incl_umin(cand);
      int* const wt = wtot[iter & 1];
      uint32_t* const wb = wbest[iter & 1];
      if (lane == 63) {
        wt[wid] = incl;
        wb[wid] = wmin;
      }
      __syncthreads();
      int o = incl - sum, tot = 0;
      uint32_t best = ~0u;
#pragma unroll
      for (int ww = 0; ww < kGrThreads / 64; ++ww) {
        const int v = wt[ww];
        tot += v;
        o += ww < wid ? v : 0;
        best = umin32(best, wb[ww]);
      }
#pragma unroll
      for (int j = 0; j < kGrPerThread; ++j) {
        if (j >= E) break;
        const int left = gr_left(my[j]);
        if (j < ne && left > 0 && (gr_mask(my[j]) & ~orm) == 0u && o < need) {
          const int take = min(left, need - o);
          const int pos = gr_pos(my[j]);
          mark[base + fill + o] = pos - (base + fill + o) + kMarkOff;
          my[j] = gr_make(gr_mask(my[j]), pos + take, left - take);
          o += left;
        }
      }
      const int got = min(tot, need);
      fill += got;
      need -= got;
      if (need == 0) break;
      orm |= best != ~0u ? emask[best & 0x3fffu] : ~0u;
    }
  }
  __syncthreads();  // marks of every thread
  // Slot r takes its source from the last mark at or before r: thread t scans its slots
  // [t*P, t*P + P), the last mark before them is an exclusive max scan over the threads.
  const int r0 = tid * kGrPerThread;
  int lastj[kGrPerThread];
  int last = -1;
#pragma unroll
  for (int j = 0; j < kGrPerThread; ++j) {
    if (r0 + j < nc && mark[r0 + j] != 0) last = r0 + j;
    lastj[j] = last;
  }
  const int incl = wave_incl_max(last);
  if (lane == 63) wmax[wid] = incl;
  __syncthreads();
  int before = __shfl_up(incl, 1, 64);
  if (lane == 0) before = -1;
  for (int ww = 0; ww < wid; ++ww) before = max(before, wmax[ww]);
#pragma unroll
  for (int j = 0; j < kGrPerThread; ++j) {
    const int r = r0 + j;
    if (r < nc) {
      const int l = lastj[j] >= 0 ? lastj[j] : before;
      order[c0 + r] = vals[c0 + r + mark[l] - kMarkOff];
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
                      2 * align_up((size_t)ntiles * kOrdBins * 4, 256) +
                      align_up((size_t)N * 4, 256);
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
  uint32_t* rowmask = cv.take<uint32_t>(N);
  hipStream_t s = ctx->stream;
  ProfScope p(ctx, "conv_order");
  ord_rowmask_kernel<<<(unsigned)((N + kRowThreads - 1) / kRowThreads), kRowThreads, 0, s>>>(
      nbr, N, rowmask);
  ord_mask_kernel<<<ntiles, kOrdThreads, 0, s>>>(rowmask, perm, N, kA, vA, counts);
  uint32_t *kc = kA, *kn = kB;
  int32_t *vc = vA, *vn = vB;
  for (int pass = 0; pass < kOrdPasses; ++pass) {
    const int shift = pass * kOrdDigitBits;
    const int dbits = kOrdMaskBits - shift < kOrdDigitBits ? kOrdMaskBits - shift : kOrdDigitBits;
    if (pass > 0) ord_hist_kernel<<<ntiles, kOrdThreads, 0, s>>>(kc, N, shift, counts);
    ord_scan_kernel<<<nwin, kOrdBins, 0, s>>>(counts, ntiles, offs);
    ord_scatter_kernel<<<ntiles, kOrdThreads, 0, s>>>(kc, vc, N, shift, dbits, offs, kn, vn);
    std::swap(kc, kn);
    std::swap(vc, vn);
  }
  ord_greedy_kernel<<<(unsigned)((N + kGrChunk - 1) / kGrChunk), kGrThreads, 0, s>>>(kc, vc, N,
                                                                                     order);
  return check_hip(hipGetLastError(), "conv_order launch");
}

}  // namespace tsc
