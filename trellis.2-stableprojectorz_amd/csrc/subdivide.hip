// Subdivision: every voxel becomes its 2x2x2 children at twice the resolution (the sparse
// decoder's upsample step, src/models/sparse_unet_vae_decoder.ts:155-175, where the TS port only
// doubles the spatial shape and keeps the coordinates).
//
//   parent row n = [b, x, y, z]  ->  child [b, 2x+dx, 2y+dy, 2z+dz],  c = dx*4 + dy*2 + dz,
//   feature row = the parent's row (copied); rows parent-major, children in increasing c.
//   With keep (one byte per parent, bit c = keep child c) only the kept children, same order.
//
// Tiles of 256 parents, one thread per parent for the coordinates.  Without keep a tile's
// output starts at 8 * 256 * tile; with keep, subdiv_count_kernel sums each tile's kept children
// and subdiv_scan_kernel turns the sums into tile offsets (and the total at [ntiles]).  Inside a
// tile an exclusive block scan of the per-parent counts gives each parent's first child row.
// Features are copied in 16-byte pieces (4- or 2-byte when the row size requires): consecutive
// threads take consecutive pieces of one parent row, load each piece once and store it to every
// kept child (non-temporal stores), so loads and stores are coalesced runs of whole rows.  Bound: HBM, bytes per parent
// = 16 + R (coords and row in) + k * (16 + R) (k kept children out), R = C * element size.

#include "tsc_internal.h"

namespace tsc {
namespace {

constexpr int kSubThreads = 256;  // parents per tile, threads per block

// Non-temporal store of a feature piece: child rows are written once and not read back here.
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
template <typename P>
__device__ __forceinline__ void store_nt(const P& v, P* dst) {
  if constexpr (sizeof(P) == 16)
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, v), (u32x4_t*)dst);
  else
    __builtin_nontemporal_store(v, dst);
}

__device__ __forceinline__ int block_excl_scan256(int v, int* wsum, int* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(incl, off, 64);
    if (lane >= off) incl += t;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  int pre = incl - v, tot = 0;
#pragma unroll
  for (int ww = 0; ww < kSubThreads / 64; ++ww) {
    if (ww < w) pre += wsum[ww];
    tot += wsum[ww];
  }
  __syncthreads();
  *total = tot;
  return pre;
}

__global__ void __launch_bounds__(kSubThreads)
    subdiv_count_kernel(const uint8_t* __restrict__ keep, int64_t n, int64_t* __restrict__ sums) {
  __shared__ int wsum[kSubThreads / 64];
  const int64_t p = (int64_t)blockIdx.x * kSubThreads + threadIdx.x;
  const int c = p < n ? __popc((uint32_t)keep[p]) : 0;
  int tot;
  block_excl_scan256(c, wsum, &tot);
  if (threadIdx.x == 0) sums[blockIdx.x] = tot;
}

// One block: exclusive scan of the tile sums in place, total at sums[ntiles].
__global__ void __launch_bounds__(1024)
    subdiv_scan_kernel(int64_t* __restrict__ sums, int64_t ntiles) {
  __shared__ int64_t wsum[16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int64_t carry = 0;
  for (int64_t base = 0; base < ntiles; base += 1024) {
    const int64_t i = base + tid;
    const int64_t v = i < ntiles ? sums[i] : 0;
    int64_t incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int64_t t = __shfl_up(incl, off, 64);
      if (lane >= off) incl += t;
    }
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    int64_t pre = incl - v, tot = 0;
#pragma unroll
    for (int ww = 0; ww < 16; ++ww) {
      if (ww < w) pre += wsum[ww];
      tot += wsum[ww];
    }
    __syncthreads();
    if (i < ntiles) sums[i] = carry + pre;
    carry += tot;
  }
  if (tid == 0) sums[ntiles] = carry;
}

template <typename P>  // feature piece: uint4, uint32_t or uint16_t
__global__ void __launch_bounds__(kSubThreads)
    subdivide_kernel(const int4* __restrict__ coords, int64_t n, const P* __restrict__ feats,
                     int32_t pieces, const uint8_t* __restrict__ keep,
                     const int64_t* __restrict__ tile_offs, int4* __restrict__ coords_out,
                     P* __restrict__ feats_out) {
  __shared__ int wsum[kSubThreads / 64];
  __shared__ int64_t s_first[kSubThreads];
  __shared__ uint32_t s_mask[kSubThreads];
  const int tid = threadIdx.x;
  const int64_t p0 = (int64_t)blockIdx.x * kSubThreads;
  const int64_t p = p0 + tid;
  const uint32_t mask = p < n ? (keep ? (uint32_t)keep[p] : 0xffu) : 0u;
  int tot;
  const int pre = block_excl_scan256(__popc(mask), wsum, &tot);
  const int64_t first = (keep ? tile_offs[blockIdx.x] : p0 * 8) + pre;
  s_first[tid] = first;
  s_mask[tid] = mask;
  if (mask) {
    const int4 c = coords[p];
    int r = 0;
#pragma unroll
    for (int ch = 0; ch < 8; ++ch) {
      if ((mask >> ch) & 1u) {
        coords_out[first + r] =
            make_int4(c.x, 2 * c.y + (ch >> 2), 2 * c.z + ((ch >> 1) & 1), 2 * c.w + (ch & 1));
        ++r;
      }
    }
  }
  if (!feats) return;
  __syncthreads();
  const int np = (int)((n - p0 < kSubThreads) ? n - p0 : kSubThreads);
  const int total = np * pieces;  // < 2^31: the host caps the row size
  for (int q = tid; q < total; q += kSubThreads) {
    const int lp = q / pieces;
    const int k = q - lp * pieces;
    const uint32_t m = s_mask[lp];
    if (!m) continue;
    const P v = feats[(p0 + lp) * pieces + k];
    const int64_t f = s_first[lp];
    int r = 0;
#pragma unroll
    for (int ch = 0; ch < 8; ++ch) {
      if ((m >> ch) & 1u) {
        store_nt(v, &feats_out[(f + r) * pieces + k]);
        ++r;
      }
    }
  }
}

}  // namespace

int subdivide_count_launch(tsc_ctx* ctx, const uint8_t* keep, int64_t N, int64_t* count_host) {
  if (N == 0) {
    *count_host = 0;
    return TSC_OK;
  }
  const int64_t ntiles = (N + kSubThreads - 1) / kSubThreads;
  void* ws;
  int st = workspace(ctx, align_up((size_t)(ntiles + 1) * 8, 256), &ws);
  if (st) return st;
  int64_t* sums = (int64_t*)ws;
  {
    ProfScope p(ctx, "subdiv_count");
    subdiv_count_kernel<<<(unsigned)ntiles, kSubThreads, 0, ctx->stream>>>(keep, N, sums);
    subdiv_scan_kernel<<<1, 1024, 0, ctx->stream>>>(sums, ntiles);
  }
  st = check_hip(hipGetLastError(), "subdivide count launch");
  if (st) return st;
  st = check_hip(hipMemcpyAsync(count_host, sums + ntiles, 8, hipMemcpyDeviceToHost, ctx->stream),
                 "subdivide count copy");
  if (st) return st;
  return check_hip(hipStreamSynchronize(ctx->stream), "subdivide count sync");
}

int subdivide_launch(tsc_ctx* ctx, const int32_t* coords, int64_t N, const void* feats,
                     int64_t row_bytes, const uint8_t* keep, int32_t* coords_out,
                     void* feats_out) {
  if (N == 0) return TSC_OK;
  const int64_t ntiles = (N + kSubThreads - 1) / kSubThreads;
  int64_t* offs = nullptr;
  if (keep) {
    void* ws;
    int st = workspace(ctx, align_up((size_t)(ntiles + 1) * 8, 256), &ws);
    if (st) return st;
    offs = (int64_t*)ws;
    ProfScope p(ctx, "subdiv_count");
    subdiv_count_kernel<<<(unsigned)ntiles, kSubThreads, 0, ctx->stream>>>(keep, N, offs);
    subdiv_scan_kernel<<<1, 1024, 0, ctx->stream>>>(offs, ntiles);
  }
  ProfScope p(ctx, "subdivide");
  const int4* c4 = (const int4*)coords;
  int4* o4 = (int4*)coords_out;
  if (!feats || row_bytes == 0) {
    subdivide_kernel<uint4><<<(unsigned)ntiles, kSubThreads, 0, ctx->stream>>>(
        c4, N, nullptr, 0, keep, offs, o4, nullptr);
  } else if (row_bytes % 16 == 0) {
    subdivide_kernel<uint4><<<(unsigned)ntiles, kSubThreads, 0, ctx->stream>>>(
        c4, N, (const uint4*)feats, (int32_t)(row_bytes / 16), keep, offs, o4, (uint4*)feats_out);
  } else if (row_bytes % 4 == 0) {
    subdivide_kernel<uint32_t><<<(unsigned)ntiles, kSubThreads, 0, ctx->stream>>>(
        c4, N, (const uint32_t*)feats, (int32_t)(row_bytes / 4), keep, offs, o4,
        (uint32_t*)feats_out);
  } else {
    subdivide_kernel<uint16_t><<<(unsigned)ntiles, kSubThreads, 0, ctx->stream>>>(
        c4, N, (const uint16_t*)feats, (int32_t)(row_bytes / 2), keep, offs, o4,
        (uint16_t*)feats_out);
  }
  return check_hip(hipGetLastError(), "subdivide launch");
}

}  // namespace tsc
