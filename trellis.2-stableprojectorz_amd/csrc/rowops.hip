// Row / elementwise ops of the sparse ResBlock, fp32 math on fp32/fp16/bf16 storage.
//
//   layernorm : per row of C: mean, biased variance (divide by C), inv = 1/sqrt(var+eps),
//               y = (x-mean)*inv*gamma + beta          (src/dense/ops/layer_norm.ts:34-65)
//               optionally followed by SiLU in the same pass (one read, one write per element)
//   silu      : y = x * 1/(1+exp(-x))                   (src/dense/ops/silu.ts:25-29)
//   add       : y = a + b                               (src/dense/ops/elementwise.ts:33-40)
//
// LayerNorm runs one wave64 per row: each lane owns C/64 strided 16-byte vectors, the row is
// read from HBM once and kept in registers (C <= 64 lanes * MAXV vectors * elements per vector),
// mean and variance come from two wave reductions over those registers, and the normalised row
// is written once.  Rows of at most 32 vectors share a wave (one lane group per row, the same
// bits); longer or unaligned rows take a three-pass strided kernel.

#include <type_traits>

#include "rownorm.h"
#include "tsc_internal.h"

namespace tsc {
namespace {

template <typename T>
struct Vec;  // 16-byte vector of T
template <>
struct Vec<float> {
  static constexpr int n = 4;
};
template <>
struct Vec<_Float16> {
  static constexpr int n = 8;
};
template <>
struct Vec<__bf16> {
  static constexpr int n = 8;
};

template <typename T>
__device__ __forceinline__ void unpack(const uint4& u, float* f) {
  const T* p = (const T*)&u;
#pragma unroll
  for (int i = 0; i < Vec<T>::n; ++i) f[i] = (float)p[i];
}
template <typename T>
__device__ __forceinline__ uint4 pack(const float* f) {
  uint4 u;
  T* p = (T*)&u;
#pragma unroll
  for (int i = 0; i < Vec<T>::n; ++i) p[i] = (T)f[i];
  return u;
}

__device__ __forceinline__ float wave_sum(float v) { return rn_wave_sum(v); }
__device__ __forceinline__ float silu_f(float x) { return rn_silu(x); }

// MAXV = max 16-byte vectors per lane (row length <= 64 * MAXV * Vec<T>::n).
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

template <typename T, int MAXV>
__global__ void __launch_bounds__(256)
    layernorm_kernel(const T* x, int64_t N, int32_t C, const T* __restrict__ gamma,
                     const T* __restrict__ beta, float eps, int32_t apply_silu, T* y) {
  constexpr int VN = Vec<T>::n;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  const int nvec = C / VN;
  const uint4* xr = (const uint4*)(x + row * C);
  float v[MAXV][VN];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < MAXV; ++k) {
    const int vi = lane + 64 * k;
    if (vi < nvec) {
      unpack<T>(xr[vi], v[k]);
#pragma unroll
      for (int e = 0; e < VN; ++e) s += v[k][e];
    }
  }
  const float mean = wave_sum(s) / (float)C;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < MAXV; ++k) {
    const int vi = lane + 64 * k;
    if (vi < nvec) {
#pragma unroll
      for (int e = 0; e < VN; ++e) {
        const float d = v[k][e] - mean;
        q += d * d;
      }
    }
  }
  const float var = wave_sum(q) / (float)C;
  const float inv = 1.0f / sqrtf(var + eps);
  uint4* yr = (uint4*)(y + row * C);
#pragma unroll
  for (int k = 0; k < MAXV; ++k) {
    const int vi = lane + 64 * k;
    if (vi < nvec) {
      float g[VN], b[VN];
      if (gamma) unpack<T>(((const uint4*)gamma)[vi], g);
      else
#pragma unroll
        for (int e = 0; e < VN; ++e) g[e] = 1.f;
      if (beta) unpack<T>(((const uint4*)beta)[vi], b);
      else
#pragma unroll
        for (int e = 0; e < VN; ++e) b[e] = 0.f;
      float o[VN];
#pragma unroll
      for (int e = 0; e < VN; ++e) {
        float t = (v[k][e] - mean) * inv * g[e] + b[e];
        o[e] = apply_silu ? silu_f(t) : t;
      }
      // non-temporal: the normalised rows are read back only by the next layer's kernel
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, pack<T>(o)), (u32x4_t*)&yr[vi]);
    }
  }
}

// Rows of at most 32 16-byte vectors: 64 / LPR rows per wave, LPR lanes per row (LPR = the power
// of two >= the row's vector count), reduced over the lane group.  Lane i of a group holds the
// row's vector i, as lane i of a wave does in layernorm_kernel, and the group butterfly gives the
// same bits as the wave butterfly there (the wave's wider steps add only zeros), so the result
// is bit-identical to one row per wave without idling the lanes past the row's vectors.
template <typename T, int LPR>
__global__ void __launch_bounds__(256)
    layernorm_rows_kernel(const T* x, int64_t N, int32_t C, const T* __restrict__ gamma,
                          const T* __restrict__ beta, float eps, int32_t apply_silu, T* y) {
  constexpr int VN = Vec<T>::n, RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, vi = lane % LPR;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW;
  if (row0 >= N) return;  // uniform per wave
  const int64_t row = row0 + lane / LPR;
  const int nvec = C / VN;
  const bool live = row < N && vi < nvec;
  float v[VN];
  if (live) {
    unpack<T>(((const uint4*)(x + row * C))[vi], v);
  } else {
#pragma unroll
    for (int e = 0; e < VN; ++e) v[e] = 0.f;
  }
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < VN; ++e) s += v[e];
  const float mean = rn_group_sum<LPR>(s) / (float)C;
  float q = 0.f;
  if (vi < nvec) {
#pragma unroll
    for (int e = 0; e < VN; ++e) {
      const float d = v[e] - mean;
      q += d * d;
    }
  }
  const float var = rn_group_sum<LPR>(q) / (float)C;
  const float inv = 1.0f / sqrtf(var + eps);
  if (!live) return;
  float g[VN], b[VN];
  if (gamma) unpack<T>(((const uint4*)gamma)[vi], g);
  else
#pragma unroll
    for (int e = 0; e < VN; ++e) g[e] = 1.f;
  if (beta) unpack<T>(((const uint4*)beta)[vi], b);
  else
#pragma unroll
    for (int e = 0; e < VN; ++e) b[e] = 0.f;
  float o[VN];
#pragma unroll
  for (int e = 0; e < VN; ++e) {
    const float t = (v[e] - mean) * inv * g[e] + b[e];
    o[e] = apply_silu ? silu_f(t) : t;
  }
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, pack<T>(o)),
                              (u32x4_t*)(y + row * C) + vi);
}

// Generic-length fallback (any C): one wave per row, three strided passes over global memory.
template <typename T>
__global__ void __launch_bounds__(256)
    layernorm_any_kernel(const T* x, int64_t N, int32_t C, const T* __restrict__ gamma,
                         const T* __restrict__ beta, float eps, int32_t apply_silu,
                         T* y) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  const T* xr = x + row * C;
  float s = 0.f;
  for (int c = lane; c < C; c += 64) s += (float)xr[c];
  const float mean = wave_sum(s) / (float)C;
  float q = 0.f;
  for (int c = lane; c < C; c += 64) {
    const float d = (float)xr[c] - mean;
    q += d * d;
  }
  const float var = wave_sum(q) / (float)C;
  const float inv = 1.0f / sqrtf(var + eps);
  T* yr = y + row * C;
  // x and y may alias: every lane reads element c before writing it, and no lane touches
  // another lane's elements.
  for (int c = lane; c < C; c += 64) {
    const float g = gamma ? (float)gamma[c] : 1.f;
    const float b = beta ? (float)beta[c] : 0.f;
    float t = ((float)xr[c] - mean) * inv * g + b;
    yr[c] = (T)(apply_silu ? silu_f(t) : t);
  }
}

template <typename T>
__global__ void __launch_bounds__(256)
    silu_kernel(const T* x, int64_t n, T* y) {
  int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (; i < n; i += stride) y[i] = (T)silu_f((float)x[i]);
}

template <typename T>
__global__ void __launch_bounds__(256)
    add_kernel(const T* a, const T* __restrict__ b, int64_t n, T* y) {
  int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (; i < n; i += stride) y[i] = (T)((float)a[i] + (float)b[i]);
}

inline unsigned ew_grid(int64_t n) {
  int64_t b = (n + 255) / 256;
  if (b > 65536) b = 65536;
  return (unsigned)(b < 1 ? 1 : b);
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <typename T>
int ln_dispatch(tsc_ctx* ctx, const T* x, int64_t N, int32_t C, const T* g, const T* b, float eps,
                int32_t silu, T* y) {
  const unsigned grid = (unsigned)((N + 3) / 4);
  constexpr int VN = Vec<T>::n;
  const bool vec_ok = (C % VN == 0) && aligned16(x) && aligned16(y) && (!g || aligned16(g)) &&
                      (!b || aligned16(b));
  const int nvec = C / VN;
  ProfScope p(ctx, silu ? "layernorm_silu" : "layernorm");
  auto rows = [&](auto lpr) {
    constexpr int L = decltype(lpr)::value;
    const unsigned g2 = (unsigned)((N + 4 * (64 / L) - 1) / (4 * (64 / L)));
    layernorm_rows_kernel<T, L><<<g2, 256, 0, ctx->stream>>>(x, N, C, g, b, eps, silu, y);
  };
  if (vec_ok && nvec <= 1) rows(std::integral_constant<int, 1>());
  else if (vec_ok && nvec <= 2) rows(std::integral_constant<int, 2>());
  else if (vec_ok && nvec <= 4) rows(std::integral_constant<int, 4>());
  else if (vec_ok && nvec <= 8) rows(std::integral_constant<int, 8>());
  else if (vec_ok && nvec <= 16) rows(std::integral_constant<int, 16>());
  else if (vec_ok && nvec <= 32) rows(std::integral_constant<int, 32>());
  else if (vec_ok && nvec <= 64 * 2)
    layernorm_kernel<T, 2><<<grid, 256, 0, ctx->stream>>>(x, N, C, g, b, eps, silu, y);
  else if (vec_ok && nvec <= 64 * 8)
    layernorm_kernel<T, 8><<<grid, 256, 0, ctx->stream>>>(x, N, C, g, b, eps, silu, y);
  else
    layernorm_any_kernel<T><<<grid, 256, 0, ctx->stream>>>(x, N, C, g, b, eps, silu, y);
  return check_hip(hipGetLastError(), "layernorm launch");
}

}  // namespace

int layernorm_launch(tsc_ctx* ctx, int32_t dtype, const void* x, int64_t N, int32_t C,
                     const void* gamma, const void* beta, float eps, int32_t apply_silu, void* y) {
  if (N == 0) return TSC_OK;
  switch (dtype) {
    case TSC_F32:
      return ln_dispatch<float>(ctx, (const float*)x, N, C, (const float*)gamma,
                                (const float*)beta, eps, apply_silu, (float*)y);
    case TSC_F16:
      return ln_dispatch<_Float16>(ctx, (const _Float16*)x, N, C, (const _Float16*)gamma,
                                   (const _Float16*)beta, eps, apply_silu, (_Float16*)y);
    case TSC_BF16:
      return ln_dispatch<__bf16>(ctx, (const __bf16*)x, N, C, (const __bf16*)gamma,
                                 (const __bf16*)beta, eps, apply_silu, (__bf16*)y);
  }
  return fail(TSC_ERR_INVALID, "layernorm: unknown dtype %d", dtype);
}

int silu_launch(tsc_ctx* ctx, int32_t dtype, const void* x, int64_t n, void* y) {
  if (n == 0) return TSC_OK;
  ProfScope p(ctx, "silu");
  switch (dtype) {
    case TSC_F32: silu_kernel<float><<<ew_grid(n), 256, 0, ctx->stream>>>((const float*)x, n, (float*)y); break;
    case TSC_F16: silu_kernel<_Float16><<<ew_grid(n), 256, 0, ctx->stream>>>((const _Float16*)x, n, (_Float16*)y); break;
    case TSC_BF16: silu_kernel<__bf16><<<ew_grid(n), 256, 0, ctx->stream>>>((const __bf16*)x, n, (__bf16*)y); break;
    default: return fail(TSC_ERR_INVALID, "silu: unknown dtype %d", dtype);
  }
  return check_hip(hipGetLastError(), "silu launch");
}

int add_launch(tsc_ctx* ctx, int32_t dtype, const void* a, const void* b, int64_t n, void* y) {
  if (n == 0) return TSC_OK;
  ProfScope p(ctx, "add");
  switch (dtype) {
    case TSC_F32: add_kernel<float><<<ew_grid(n), 256, 0, ctx->stream>>>((const float*)a, (const float*)b, n, (float*)y); break;
    case TSC_F16: add_kernel<_Float16><<<ew_grid(n), 256, 0, ctx->stream>>>((const _Float16*)a, (const _Float16*)b, n, (_Float16*)y); break;
    case TSC_BF16: add_kernel<__bf16><<<ew_grid(n), 256, 0, ctx->stream>>>((const __bf16*)a, (const __bf16*)b, n, (__bf16*)y); break;
    default: return fail(TSC_ERR_INVALID, "add: unknown dtype %d", dtype);
  }
  return check_hip(hipGetLastError(), "add launch");
}

}  // namespace tsc
