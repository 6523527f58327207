// Submanifold sparse conv3d as an implicit GEMM on gfx950 MFMA.
//
//   out[n, co] = bias[co] + sum_{v : nbr[n,v] >= 0} sum_ci feats[nbr[n,v], ci] * W[co, v, ci]
//
// (reference semantics: src/sparse/ops/conv3d_wgsl.ts:132-231, weight at co*27*Ci + v*Ci + ci,
// conv3d_wgsl.ts:197; accumulation here is always fp32.)
//
// GEMM view: M = voxel rows (in `order`), N = Co, K = 27 taps x Ci.  A block owns a BM x BN
// output tile.  It first stages the BM neighbor rows (BM x 27 int32) in LDS and ORs their
// valid-tap bits: taps that no row of the tile uses are skipped entirely.  The K loop then walks
// (tap, Ci-chunk) pairs; per chunk every thread issues 16-byte global loads for its share of the
// gathered A rows (feats[nbr[row,v]], zero when nbr < 0) and of the B rows (W[co, v, ci-chunk],
// K-contiguous), stores them into a double-buffered, XOR-swizzled LDS tile and the four waves run
// 32x32 MFMAs over it (v_mfma_f32_32x32x16_{bf16,f16}, v_mfma_f32_32x32x2_f32).  The next chunk's
// global loads are in flight while the current chunk is multiplied; one barrier per chunk.
//
// MFMA operand layout used (32x32 family): lane l supplies A[i = l%32][k in half l/32] and
// B[k in half l/32][j = l%32]; accumulator register r of lane l holds
// D[8*(r/4) + 4*(l/32) + r%4][l%32].  Any assignment of K indices to (lane half, element) is
// valid as long as A and B use the same one; here half h of micro-step s reads 16-byte LDS
// piece 2s+h of the row.

#include <string>
#include <type_traits>

#include "tsc_internal.h"

namespace tsc {
namespace {

typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef _Float16 f16x8_t __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef float f32x16_t __attribute__((__vector_size__(16 * sizeof(float))));

template <typename T>
__device__ __forceinline__ float to_f32(T v) { return (float)v; }
template <typename T>
__device__ __forceinline__ T from_f32(float v) { return (T)v; }

// One 16-byte A piece times one 16-byte B piece, accumulated into a 32x32 fp32 tile.
template <typename T>
__device__ __forceinline__ void mfma_piece(const uint4& a, const uint4& b, f32x16_t& acc);

template <>
__device__ __forceinline__ void mfma_piece<__bf16>(const uint4& a, const uint4& b, f32x16_t& acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), acc, 0, 0, 0);
}
template <>
__device__ __forceinline__ void mfma_piece<_Float16>(const uint4& a, const uint4& b,
                                                     f32x16_t& acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                               __builtin_bit_cast(f16x8_t, b), acc, 0, 0, 0);
}
template <>
__device__ __forceinline__ void mfma_piece<float>(const uint4& a, const uint4& b, f32x16_t& acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
}

// XOR swizzle of 16-byte pieces within an LDS row of PPR pieces, so that the 8 lanes that read
// one piece column from 8 consecutive rows hit 8 distinct bank groups.
template <int PPR>
__device__ __forceinline__ int swz(int row, int part) {
  constexpr int rows_per_128 = (PPR >= 8) ? 1 : 8 / PPR;
  return part ^ ((row / rows_per_128) % PPR);
}

constexpr int kTaps = 27;

template <typename T, int BM, int BN, int KB, int WM, int WN, int EPI>
struct ConvCfg {
  static constexpr int NT = 64 * WM * WN;
  static constexpr int PPR = KB / 16;              // 16-byte pieces per LDS row
  static constexpr int KC = KB / (int)sizeof(T);   // K elements per chunk
  static constexpr int EPP = 16 / (int)sizeof(T);  // elements per piece
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int FM = WTM / 32, FN = WTN / 32;
  static constexpr int MS = KB / 32;               // micro-steps per chunk
  static constexpr int A_PIECES = BM * PPR, B_PIECES = BN * PPR;
  static constexpr int AP = (A_PIECES + NT - 1) / NT, BP = (B_PIECES + NT - 1) / NT;
  static_assert(KB % 32 == 0 && KB <= 128, "chunk must be 32..128 bytes");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32x32");
};

template <typename T, int BM, int BN, int KB, int WM, int WN, int EPI>
__global__ void __launch_bounds__(64 * WM * WN)
    conv_mfma_kernel(const T* __restrict__ feats, const T* __restrict__ weight,
                     const T* __restrict__ bias, const int32_t* __restrict__ nbr,
                     const int32_t* __restrict__ order, int64_t N, int32_t Ci, int32_t Co,
                     int32_t m_tiles, int32_t n_tiles, int32_t per_xcd,
                     const T* __restrict__ residual, T* __restrict__ out) {
  using C = ConvCfg<T, BM, BN, KB, WM, WN, EPI>;
  __shared__ __attribute__((aligned(16))) unsigned char sA[2][BM * KB];
  __shared__ __attribute__((aligned(16))) unsigned char sB[2][BN * KB];
  __shared__ int32_t sNbr[BM * kTaps];
  __shared__ int32_t sRow[BM];
  __shared__ int32_t sTaps[kTaps];
  __shared__ uint32_t sMask;

  // XCD-aware tile order: hardware hands block b to XCD b % 8; give each XCD a contiguous run of
  // logical tiles, with the n-tiles of one m-tile adjacent, so gathered rows are reused in L2.
  const int bid = blockIdx.x;
  const int logical = (bid & 7) * per_xcd + (bid >> 3);
  if (logical >= m_tiles * n_tiles) return;
  const int m_tile = logical / n_tiles, n_tile = logical % n_tiles;
  const int64_t m0 = (int64_t)m_tile * BM;
  const int n0 = n_tile * BN;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid / WN, wn = wid % WN;

  if (tid == 0) sMask = 0u;
  for (int r = tid; r < BM; r += C::NT) {
    int64_t pos = m0 + r;
    sRow[r] = (pos < N) ? (order ? order[pos] : (int32_t)pos) : -1;
  }
  __syncthreads();
  uint32_t mymask = 0u;
  for (int j = tid; j < BM * kTaps; j += C::NT) {
    int r = j / kTaps, v = j - r * kTaps;
    int32_t row = sRow[r];
    int32_t s = (row >= 0) ? nbr[(int64_t)row * kTaps + v] : -1;
    sNbr[j] = s;
    if (s >= 0) mymask |= 1u << v;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mymask |= __shfl_xor(mymask, off, 64);
  if (lane == 0 && mymask) atomicOr(&sMask, mymask);
  __syncthreads();
  const uint32_t mask = sMask;
  const int ntaps = __popc(mask);
  if (tid == 0) {
    int k = 0;
    for (uint32_t m = mask; m; m &= m - 1) sTaps[k++] = __ffs(m) - 1;
  }
  __syncthreads();

  const int cpt = Ci / C::KC;  // chunks per tap
  const int nchunks = ntaps * cpt;

  f32x16_t acc[C::FM][C::FN];
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  uint4 ra[C::AP], rb[C::BP];

  auto load_chunk = [&](int c) {
    const int ti = c / cpt;
    const int ci0 = (c - ti * cpt) * C::KC;
    const int v = sTaps[ti];
#pragma unroll
    for (int j = 0; j < C::AP; ++j) {
      const int q = tid + j * C::NT;
      uint4 val = make_uint4(0u, 0u, 0u, 0u);
      if (C::A_PIECES % C::NT == 0 || q < C::A_PIECES) {
        const int r = q / C::PPR, part = q % C::PPR;
        const int32_t src = sNbr[r * kTaps + v];
        if (src >= 0)
          val = *(const uint4*)(feats + (int64_t)src * Ci + ci0 + part * C::EPP);
      }
      ra[j] = val;
    }
#pragma unroll
    for (int j = 0; j < C::BP; ++j) {
      const int q = tid + j * C::NT;
      uint4 val = make_uint4(0u, 0u, 0u, 0u);
      if (C::B_PIECES % C::NT == 0 || q < C::B_PIECES) {
        const int r = q / C::PPR, part = q % C::PPR;
        val = *(const uint4*)(weight + ((int64_t)(n0 + r) * kTaps + v) * Ci + ci0 + part * C::EPP);
      }
      rb[j] = val;
    }
  };
  auto store_chunk = [&](int buf) {
#pragma unroll
    for (int j = 0; j < C::AP; ++j) {
      const int q = tid + j * C::NT;
      if (C::A_PIECES % C::NT == 0 || q < C::A_PIECES) {
        const int r = q / C::PPR, part = q % C::PPR;
        *(uint4*)(&sA[buf][r * KB + swz<C::PPR>(r, part) * 16]) = ra[j];
      }
    }
#pragma unroll
    for (int j = 0; j < C::BP; ++j) {
      const int q = tid + j * C::NT;
      if (C::B_PIECES % C::NT == 0 || q < C::B_PIECES) {
        const int r = q / C::PPR, part = q % C::PPR;
        *(uint4*)(&sB[buf][r * KB + swz<C::PPR>(r, part) * 16]) = rb[j];
      }
    }
  };

  if (nchunks > 0) {
    load_chunk(0);
    store_chunk(0);
  }
  for (int c = 0; c < nchunks; ++c) {
    const int buf = c & 1;
    __syncthreads();
    if (c + 1 < nchunks) load_chunk(c + 1);
#pragma unroll
    for (int s = 0; s < C::MS; ++s) {
      const int part = 2 * s + (lane >> 5);
      uint4 a[C::FM], b[C::FN];
#pragma unroll
      for (int i = 0; i < C::FM; ++i) {
        const int r = wm * C::WTM + i * 32 + (lane & 31);
        a[i] = *(const uint4*)(&sA[buf][r * KB + swz<C::PPR>(r, part) * 16]);
      }
#pragma unroll
      for (int j = 0; j < C::FN; ++j) {
        const int r = wn * C::WTN + j * 32 + (lane & 31);
        b[j] = *(const uint4*)(&sB[buf][r * KB + swz<C::PPR>(r, part) * 16]);
      }
#pragma unroll
      for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j) mfma_piece<T>(a[i], b[j], acc[i][j]);
    }
    if (c + 1 < nchunks) store_chunk(buf ^ 1);
  }

  // Epilogue: bias (+ residual), round to T, scatter rows back to their original positions.
#pragma unroll
  for (int j = 0; j < C::FN; ++j) {
    const int co = n0 + wn * C::WTN + j * 32 + (lane & 31);
    const float bv = bias ? to_f32<T>(bias[co]) : 0.f;
#pragma unroll
    for (int i = 0; i < C::FM; ++i) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int rl = wm * C::WTM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int32_t row = sRow[rl];
        if (row >= 0) {
          float val = acc[i][j][e] + bv;
          const int64_t o = (int64_t)row * Co + co;
          if (EPI == TSC_EPI_BIAS_RESIDUAL) val += to_f32<T>(residual[o]);
          out[o] = from_f32<T>(val);
        }
      }
    }
  }
}

template <typename T, int BM, int BN, int KB, int WM, int WN, int EPI>
int launch_cfg(tsc_ctx* ctx, const ConvArgs& a) {
  const int32_t m_tiles = (int32_t)((a.N + BM - 1) / BM);
  const int32_t n_tiles = a.Co / BN;
  const int64_t total = (int64_t)m_tiles * n_tiles;
  const int32_t per_xcd = (int32_t)((total + 7) / 8);
  const unsigned grid = (unsigned)per_xcd * 8u;
  static const std::string name = std::string("conv_") +
      (sizeof(T) == 4 ? "f32" : std::is_same<T, __bf16>::value ? "bf16" : "f16") + "_" +
      std::to_string(BM) + "x" + std::to_string(BN) + "_k" + std::to_string(KB) +
      (EPI == TSC_EPI_BIAS_RESIDUAL ? "_res" : "");
  ProfScope p(ctx, name.c_str());
  conv_mfma_kernel<T, BM, BN, KB, WM, WN, EPI><<<grid, 64 * WM * WN, 0, ctx->stream>>>(
      (const T*)a.feats, (const T*)a.weight, (const T*)a.bias, a.nbr, a.order, a.N, a.Ci, a.Co,
      m_tiles, n_tiles, per_xcd, (const T*)a.residual, (T*)a.out);
  return check_hip(hipGetLastError(), "conv launch");
}

// Largest chunk (bytes per row) that divides the Ci row and is a multiple of 32 bytes.
inline int pick_kb(int row_bytes) {
  if (row_bytes % 128 == 0) return 128;
  if (row_bytes % 64 == 0) return 64;
  return 32;
}

template <typename T, int EPI>
int dispatch_tiles(tsc_ctx* ctx, const ConvArgs& a) {
  const int kb = pick_kb(a.Ci * (int)sizeof(T));
  if (a.Co % 128 == 0 && a.Co >= 128) {
    // Wide channels: 128x128 tile, 2x2 waves of 64x64.
    if (kb == 128) return launch_cfg<T, 128, 128, 128, 2, 2, EPI>(ctx, a);
    if (kb == 64) return launch_cfg<T, 128, 128, 64, 2, 2, EPI>(ctx, a);
    return launch_cfg<T, 128, 128, 32, 2, 2, EPI>(ctx, a);
  }
  if (a.Co % 64 == 0) {
    // Narrow channels: 128 rows x 64 cols, 4 waves of 32 rows.
    if (kb == 128) return launch_cfg<T, 128, 64, 128, 4, 1, EPI>(ctx, a);
    if (kb == 64) return launch_cfg<T, 128, 64, 64, 4, 1, EPI>(ctx, a);
    return launch_cfg<T, 128, 64, 32, 4, 1, EPI>(ctx, a);
  }
  // Co % 32 == 0
  if (kb == 128) return launch_cfg<T, 128, 32, 128, 4, 1, EPI>(ctx, a);
  if (kb == 64) return launch_cfg<T, 128, 32, 64, 4, 1, EPI>(ctx, a);
  return launch_cfg<T, 128, 32, 32, 4, 1, EPI>(ctx, a);
}

template <typename T>
int dispatch_epi(tsc_ctx* ctx, const ConvArgs& a) {
  if (a.epilogue == TSC_EPI_BIAS_RESIDUAL) return dispatch_tiles<T, TSC_EPI_BIAS_RESIDUAL>(ctx, a);
  return dispatch_tiles<T, TSC_EPI_BIAS>(ctx, a);
}

}  // namespace

int conv_launch(tsc_ctx* ctx, const ConvArgs& a) {
  if (a.N == 0) return TSC_OK;
  switch (a.dtype) {
    case TSC_F32: return dispatch_epi<float>(ctx, a);
    case TSC_F16: return dispatch_epi<_Float16>(ctx, a);
    case TSC_BF16: return dispatch_epi<__bf16>(ctx, a);
  }
  return fail(TSC_ERR_INVALID, "conv: unknown dtype %d", a.dtype);
}

}  // namespace tsc
