// Varlen scaled-dot-product attention over packed sequences: the reference's sparseAttention
// (src/sparse/ops/attention.ts:24-79, which runs B > 1 as a per-sample CPU round trip) and its
// dense scaledDotProductAttention (src/dense/ops/attention.ts:36-110) for B = 1.
//
//   out[n, h, :] = softmax_k(q[n, h, :] . k[m, h, :] * scale) @ v[m, h, :]
//   n in [cu_q[b], cu_q[b+1]),  m in [cu_kv[b], cu_kv[b+1]),  rows (total, H, D) row-major.
//   A sample with no keys gives zeros (attention.ts:57).
//
// A bf16/f16 block = 8 waves = 256 queries of one (sequence, head) (an f32 block: 4 waves, 128);
// each wave owns 32 queries and walks the sequence's keys in blocks, with an online softmax
// (running max and sum per query).
// The scores are computed transposed, S^T = K Q^T (M = keys, N = queries), so that in the MFMA
// result layout each lane holds 16 keys of ONE query (lane l: query l % 32): the row max / sum
// need one cross-half exchange (lane l ^ 32) per step, and the output O^T = V^T P^T keeps the
// same "one query per lane" layout, so the rescale by exp(m_old - m_new) is lane-local.  P^T is
// used as the MFMA B operand straight from the score registers; the keys of each MFMA k-step are
// therefore the score layout's rows 8(j/4) + 4(l/32) + j%4, and V is staged transposed in LDS
// (V^T[d][key], 4-key units XOR-swizzled) so that each lane reads its two 4-key runs as 8 bytes.
//   bf16/f16: v_mfma_f32_32x32x16 (Q^T fragment kept in registers, K block in LDS row-major with
//             16-byte chunks XOR-swizzled by row), 64-key blocks, K/V double-buffered in LDS
//             and prefetched one block ahead through registers.
//   f32:      v_mfma_f32_32x32x2f32 (k-step = 2 dims / 2 keys; K and V row-major in LDS with
//             padded strides, no transpose needed), 32-key blocks.
// Bound: MFMA (4 * D flops per query-key pair) and the softmax's exp per pair.

#include "tsc_internal.h"

namespace tsc {
namespace {

typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef _Float16 f16x8_t __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef float f32x16_t __attribute__((__vector_size__(16 * sizeof(float))));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;   // f32 kernel: 4 waves
constexpr int kBQ = 128;        // f32 kernel: queries per block, 32 per wave
constexpr int kMmaThreads = 512;  // bf16/f16 kernel: 8 waves (2 per SIMD)
constexpr int kMmaBQ = 256;       // bf16/f16 kernel: queries per block, 32 per wave
constexpr float kLazy = 8.f;    // log2 headroom before the running max is raised

template <typename T>
struct Mma;
template <>
struct Mma<__bf16> {
  static __device__ __forceinline__ void run(const uint4& a, const uint4& b, f32x16_t& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {  // RNE, one cvt_pk
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
  }
  // acc + the two packed values (v_dot2 with (1, 1)): the softmax denominator is summed over the
  // same rounded P that the second product uses.
  static __device__ __forceinline__ float add2(uint32_t packed, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, packed),
                                          __builtin_bit_cast(bf16x2_t, 0x3f803f80u), acc, false);
  }
};
template <>
struct Mma<_Float16> {
  static __device__ __forceinline__ void run(const uint4& a, const uint4& b, f32x16_t& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                               __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, f16x2_t));
  }
  static __device__ __forceinline__ float add2(uint32_t packed, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, packed),
                                  __builtin_bit_cast(f16x2_t, 0x3c003c00u), acc, false);
  }
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Max / sum of a value and the one held by lane l ^ 32 (both halves of the wave hold the same
// query): v_permlane32_swap exchanges the wave halves in registers (no LDS round trip).
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Segment b's [begin, end) clamped into [0, total] (a malformed cu_seqlens cannot index outside).
__device__ __forceinline__ void segment(const int32_t* cu, int b, int64_t total, int* begin,
                                        int* len) {
  const int64_t s = min<int64_t>(max<int64_t>(cu[b], 0), total);
  const int64_t e = min<int64_t>(max<int64_t>(cu[b + 1], s), total);
  *begin = (int)s;
  *len = (int)(e - s);
}

// Block -> (q tile, head, sequence) so that each XCD (blocks are dealt to the 8 XCDs round robin)
// gets a contiguous run of q tiles: the blocks that stream one head's K and V share an L2.
// XCD r holds total/8 blocks, one more for r < total % 8; block lin = 8i + r is its i-th, so the
// map is a bijection of [0, total).
__device__ __forceinline__ void xcd_block(int* bx, int* bh, int* bb) {
  const int gx = gridDim.x, gy = gridDim.y;
  const int total = gx * gy * gridDim.z;
  const int lin = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const int r = lin % 8, base = total / 8, extra = total % 8;
  const int v = r * base + min(r, extra) + lin / 8;
  *bx = v % gx;
  *bh = (v / gx) % gy;
  *bb = v / (gx * gy);
}

// ---------------------------------------------------------------------------------- bf16 / f16
template <typename T, int D>
__global__ void __launch_bounds__(kMmaThreads)
    attn_mma_kernel(const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
                    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_kv,
                    int64_t total_q, int64_t total_kv, int32_t H, float scale_log2,
                    T* __restrict__ out) {
  constexpr int BK = 64;
  constexpr int DC = D / 8;                  // 16-byte chunks per row
  constexpr int KS = D / 16;                 // k-steps of S^T = K Q^T
  constexpr int MT = D / 32;                 // 32-dim tiles of O^T
  constexpr int KL = BK * DC / kMmaThreads;  // K chunks each thread stages per block
  constexpr int VT = BK / 2 * DC;            // threads staging V (2 keys x 8 dims each)
  constexpr int VU = BK / 4;                 // 4-key (8-byte) units per V^T row
  static_assert(KL >= 1 && VT <= kMmaThreads && (D == 64 || D == 128), "tile shape");
  __shared__ __attribute__((aligned(16))) uint4 ks[2][BK * DC];
  __shared__ __attribute__((aligned(16))) uint2 vt[2][D * VU];

  int bx, h, bb;
  xcd_block(&bx, &h, &bb);
  int q0, q_len, kv0, kv_len;
  segment(cu_q, bb, total_q, &q0, &q_len);
  segment(cu_kv, bb, total_kv, &kv0, &kv_len);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l32 = lane & 31, hf = lane >> 5;
  const int64_t rs = (int64_t)H * D;
  const T* kbase = k + (int64_t)kv0 * rs + (int64_t)h * D;
  const T* vbase = v + (int64_t)kv0 * rs + (int64_t)h * D;
  // LDS: 32 banks of 4 bytes; a b128 access is served 8 lanes at a time, b64 16, b32 32.
  // K chunk (row, c) lives at slot c ^ (row & 15) (D = 128) or c ^ (row & 7) (D = 64): the 8
  // lanes of one read step (rows r..r+7, one chunk column) and of one write step (one row, 8
  // chunks) each cover all 32 banks.  V^T unit u of row d lives at u ^ (d & 15): the 16 rows a
  // b64 read step touches get 16 distinct units, and rows d and d + 32 share the pattern, so the
  // reads of the two dim tiles pair into one ds_read2st64.  A b32 write step writes one row per
  // 32 lanes (all 32 banks).
  auto kslot = [](int row, int c) { return row * DC + (c ^ (row & (DC - 1))); };
  auto vslot = [](int d, int u) { return d * VU + (u ^ (d & 15)); };

  for (int qt = bx * kMmaBQ; qt < q_len; qt += gridDim.x * kMmaBQ) {
    const int qi = qt + w * 32 + l32;
    T* orow = out + (int64_t)(q0 + qi) * rs + (int64_t)h * D;
    if (kv_len == 0) {  // no keys: zeros (uniform over the block)
      if (qi < q_len)
        for (int c = hf; c < DC; c += 2) *(uint4*)(orow + 8 * c) = make_uint4(0, 0, 0, 0);
      continue;
    }
    uint4 qf[KS];  // Q^T fragment: lane (query l32, half hf) holds dims 16s + 8hf .. + 7
    {
      const T* qrow = q + (int64_t)(q0 + min(qi, q_len - 1)) * rs + (int64_t)h * D + 8 * hf;
#pragma unroll
      for (int s = 0; s < KS; ++s) qf[s] = *(const uint4*)(qrow + 16 * s);
    }
    uint4 kr[KL], vr[2];
    auto load = [&](int kb) {
#pragma unroll
      for (int i = 0; i < KL; ++i) {
        const int id = tid + kMmaThreads * i, row = id / DC, c = id % DC;
        kr[i] = kb + row < kv_len ? *(const uint4*)(kbase + (int64_t)(kb + row) * rs + 8 * c)
                                  : make_uint4(0, 0, 0, 0);
      }
      if (tid < VT) {  // 32 consecutive threads: the 32 key pairs of one 8-dim chunk
        const int kp = tid % 32, dv = tid / 32;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int key = kb + 2 * kp + i;
          vr[i] = key < kv_len ? *(const uint4*)(vbase + (int64_t)key * rs + 8 * dv)
                               : make_uint4(0, 0, 0, 0);
        }
      }
    };
    auto store = [&](int buf) {
#pragma unroll
      for (int i = 0; i < KL; ++i) {
        const int id = tid + kMmaThreads * i;
        ks[buf][kslot(id / DC, id % DC)] = kr[i];
      }
      if (tid < VT) {  // keys 2kp, 2kp+1 of dims 8dv..8dv+7 -> half (kp & 1) of unit kp / 2
        const int kp = tid % 32, dv = tid / 32;
        const uint32_t* a = (const uint32_t*)&vr[0];
        const uint32_t* b = (const uint32_t*)&vr[1];
        uint32_t* base = (uint32_t*)&vt[buf][0] + (kp & 1);
#pragma unroll
        for (int j = 0; j < 8; ++j)  // (a.lo, b.lo) or (a.hi, b.hi) of dword j / 2
          base[2 * vslot(8 * dv + j, kp >> 1)] =
              __builtin_amdgcn_perm(b[j >> 1], a[j >> 1], (j & 1) ? 0x07060302u : 0x05040100u);
      }
    };

    float m_use = -INFINITY, l_run = 0.f;
    f32x16_t o[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 16; ++j) o[mt][j] = 0.f;
    const int nblk = (kv_len + BK - 1) / BK;
    load(0);
    store(0);
    __syncthreads();
    for (int jb = 0; jb < nblk; ++jb) {
      const int buf = jb & 1, kb = jb * BK;
      const bool more = jb + 1 < nblk;
      if (more) load(kb + BK);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {  // two 32-key halves: S^T tile, softmax, P^T V
        f32x16_t s;
#pragma unroll
        for (int j = 0; j < 16; ++j) s[j] = 0.f;
#pragma unroll
        for (int st = 0; st < KS; ++st)
          Mma<T>::run(ks[buf][kslot(kt * 32 + l32, 2 * st + hf)], qf[st], s);
        const int k0 = kb + kt * 32;
        if (k0 + 32 > kv_len) {
#pragma unroll
          for (int j = 0; j < 16; ++j)
            if (k0 + 8 * (j >> 2) + 4 * hf + (j & 3) >= kv_len) s[j] = -INFINITY;
        }
        float mx = s[0];
#pragma unroll
        for (int j = 1; j < 16; ++j) mx = fmaxf(mx, s[j]);
        mx = pair_max(mx);  // -inf only for a fully masked half
        if (__builtin_amdgcn_ballot_w64(mx * scale_log2 > m_use * scale_log2 + kLazy)) {
          const float m_new = fmaxf(m_use, mx);
          const float alpha = fast_exp2((m_use - m_new) * scale_log2);  // 0 while m_use = -inf
          m_use = m_new;
          l_run *= alpha;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < 16; ++j) o[mt][j] *= alpha;
        }
        const float mc = m_use * scale_log2;
#pragma unroll
        for (int half = 0; half < 2; ++half) {  // k-step: keys 16 half + {4hf.., 8+4hf..}
          float p[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) p[i] = fast_exp2(fmaf(s[8 * half + i], scale_log2, -mc));
          const uint4 pf = make_uint4(Mma<T>::pack(p[0], p[1]), Mma<T>::pack(p[2], p[3]),
                                      Mma<T>::pack(p[4], p[5]), Mma<T>::pack(p[6], p[7]));
          l_run = Mma<T>::add2(pf.w, Mma<T>::add2(pf.z, Mma<T>::add2(pf.y, Mma<T>::add2(pf.x, l_run))));
          const int u = 8 * kt + 4 * half + hf;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const int d = 32 * mt + l32;
            const uint2 x = vt[buf][vslot(d, u)];
            const uint2 y = vt[buf][vslot(d, u + 2)];
            Mma<T>::run(make_uint4(x.x, x.y, y.x, y.y), pf, o[mt]);
          }
        }
      }
      if (more) store(buf ^ 1);
      __syncthreads();
    }
    l_run = pair_sum(l_run);
    const float inv = 1.f / l_run;
    if (qi < q_len) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *(uint2*)(orow + 32 * mt + 8 * g + 4 * hf) =
              make_uint2(Mma<T>::pack(o[mt][4 * g] * inv, o[mt][4 * g + 1] * inv),
                         Mma<T>::pack(o[mt][4 * g + 2] * inv, o[mt][4 * g + 3] * inv));
    }
  }
}

// ---------------------------------------------------------------------------------- f32
template <int D>
__global__ void __launch_bounds__(kThreads)
    attn_f32_kernel(const float* __restrict__ q, const float* __restrict__ k,
                    const float* __restrict__ v, const int32_t* __restrict__ cu_q,
                    const int32_t* __restrict__ cu_kv, int64_t total_q, int64_t total_kv,
                    int32_t H, float scale_log2, float* __restrict__ out) {
  constexpr int BK = 32;
  constexpr int KST = D + 2;  // K row stride: lanes (key, half) read 64 distinct banks
  constexpr int VST = D + 8;  // V row stride: rows 4 apart land 32 banks apart
  constexpr int MT = D / 32;
  constexpr int NC = BK * D / 4;               // float4 chunks per K (or V) block
  constexpr int CL = NC / kThreads;            // chunks each thread stages
  static_assert(CL >= 1 && (D == 64 || D == 128), "tile shape");
  __shared__ __attribute__((aligned(16))) float ks[2][BK * KST];
  __shared__ __attribute__((aligned(16))) float vs[2][BK * VST];

  int bx, h, bb;
  xcd_block(&bx, &h, &bb);
  int q0, q_len, kv0, kv_len;
  segment(cu_q, bb, total_q, &q0, &q_len);
  segment(cu_kv, bb, total_kv, &kv0, &kv_len);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l32 = lane & 31, hf = lane >> 5;
  const int64_t rs = (int64_t)H * D;
  const float* kbase = k + (int64_t)kv0 * rs + (int64_t)h * D;
  const float* vbase = v + (int64_t)kv0 * rs + (int64_t)h * D;

  for (int qt = bx * kBQ; qt < q_len; qt += gridDim.x * kBQ) {
    const int qi = qt + w * 32 + l32;
    float* orow = out + (int64_t)(q0 + qi) * rs + (int64_t)h * D;
    if (kv_len == 0) {
      if (qi < q_len)
        for (int c = hf; c < D / 4; c += 2) *(float4*)(orow + 4 * c) = make_float4(0, 0, 0, 0);
      continue;
    }
    float qf[D / 2];  // B operand of step st: dim 2st + hf of this lane's query
    {
      const float* qrow = q + (int64_t)(q0 + min(qi, q_len - 1)) * rs + (int64_t)h * D;
#pragma unroll
      for (int c = 0; c < D / 4; ++c) {
        const float4 x = *(const float4*)(qrow + 4 * c);
        qf[2 * c] = hf ? x.y : x.x;
        qf[2 * c + 1] = hf ? x.w : x.z;
      }
    }
    float4 kr[CL], vr[CL];
    auto load = [&](int kb) {
#pragma unroll
      for (int i = 0; i < CL; ++i) {
        const int id = tid + kThreads * i, row = id / (D / 4), c = id % (D / 4);
        const bool ok = kb + row < kv_len;
        const int64_t off = (int64_t)(kb + row) * rs + 4 * c;
        kr[i] = ok ? *(const float4*)(kbase + off) : make_float4(0, 0, 0, 0);
        vr[i] = ok ? *(const float4*)(vbase + off) : make_float4(0, 0, 0, 0);
      }
    };
    auto store = [&](int buf) {
#pragma unroll
      for (int i = 0; i < CL; ++i) {
        const int id = tid + kThreads * i, row = id / (D / 4), c = id % (D / 4);
        float2* kd = (float2*)&ks[buf][row * KST + 4 * c];
        kd[0] = make_float2(kr[i].x, kr[i].y);
        kd[1] = make_float2(kr[i].z, kr[i].w);
        *(float4*)&vs[buf][row * VST + 4 * c] = vr[i];
      }
    };

    float m_run = -INFINITY, l_run = 0.f;
    f32x16_t o[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 16; ++j) o[mt][j] = 0.f;
    const int nblk = (kv_len + BK - 1) / BK;
    load(0);
    store(0);
    __syncthreads();
    for (int jb = 0; jb < nblk; ++jb) {
      const int buf = jb & 1, kb = jb * BK;
      const bool more = jb + 1 < nblk;
      if (more) load(kb + BK);
      f32x16_t s0, s1;  // two accumulation chains over the dims
#pragma unroll
      for (int j = 0; j < 16; ++j) s0[j] = s1[j] = 0.f;
      const float* krow = &ks[buf][l32 * KST + hf];
#pragma unroll
      for (int st = 0; st < D / 2; st += 2) {
        s0 = __builtin_amdgcn_mfma_f32_32x32x2f32(krow[2 * st], qf[st], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(krow[2 * st + 2], qf[st + 1], s1, 0, 0, 0);
      }
      float s[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        s[j] = s0[j] + s1[j];
        if (kb + 8 * (j >> 2) + 4 * hf + (j & 3) >= kv_len) s[j] = -INFINITY;
      }
      float mx = m_run;
#pragma unroll
      for (int j = 0; j < 16; ++j) mx = fmaxf(mx, s[j]);
      mx = pair_max(mx);
      const float mc = mx * scale_log2;
      const float alpha = fast_exp2(m_run * scale_log2 - mc);
      m_run = mx;
      l_run *= alpha;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 16; ++j) o[mt][j] *= alpha;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        s[j] = fast_exp2(fmaf(s[j], scale_log2, -mc));
        l_run += s[j];
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float* vrow = &vs[buf][(8 * (j >> 2) + 4 * hf + (j & 3)) * VST + l32];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          o[mt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 * mt], s[j], o[mt], 0, 0, 0);
      }
      if (more) store(buf ^ 1);
      __syncthreads();
    }
    l_run = pair_sum(l_run);
    const float inv = 1.f / l_run;
    if (qi < q_len) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *(float4*)(orow + 32 * mt + 8 * g + 4 * hf) =
              make_float4(o[mt][4 * g] * inv, o[mt][4 * g + 1] * inv, o[mt][4 * g + 2] * inv,
                          o[mt][4 * g + 3] * inv);
    }
  }
}

template <typename T, int D>
void launch_mma(tsc_ctx* ctx, dim3 grid, const void* q, const void* k, const void* v,
                const int32_t* cu_q, const int32_t* cu_kv, int64_t tq, int64_t tkv, int32_t H,
                float sl2, void* out) {
  attn_mma_kernel<T, D><<<grid, kMmaThreads, 0, ctx->stream>>>(
      (const T*)q, (const T*)k, (const T*)v, cu_q, cu_kv, tq, tkv, H, sl2, (T*)out);
}

}  // namespace

int attention_launch(tsc_ctx* ctx, int32_t dtype, const void* q, const void* k, const void* v,
                     const int32_t* cu_q, const int32_t* cu_kv, int32_t B, int64_t total_q,
                     int64_t total_kv, int32_t H, int32_t D, float scale, int32_t max_seqlen_q,
                     void* out) {
  if (B == 0 || total_q == 0 || max_seqlen_q == 0) return TSC_OK;
  const float sl2 = scale * 1.4426950408889634f;  // scale * log2(e): softmax in base 2
  // q tiles beyond the grid's x extent are covered by the kernels' tile loops
  const int bq = dtype == TSC_F32 ? kBQ : kMmaBQ;
  const int64_t hb = (int64_t)H * B;  // the block index arithmetic is 32-bit
  if (hb > (int64_t)(INT32_MAX / 16))
    return fail(TSC_ERR_UNSUPPORTED, "attention: %lld (head, sequence) pairs", (long long)hb);
  const unsigned gx = (unsigned)std::min<int64_t>(
      std::min<int64_t>((max_seqlen_q + bq - 1) / bq, 65535), (INT32_MAX / 16) / hb);
  const dim3 grid(gx, (unsigned)H, (unsigned)B);
  ProfScope p(ctx, "attention");
  if (dtype == TSC_BF16) {
    if (D == 64) launch_mma<__bf16, 64>(ctx, grid, q, k, v, cu_q, cu_kv, total_q, total_kv, H, sl2, out);
    else launch_mma<__bf16, 128>(ctx, grid, q, k, v, cu_q, cu_kv, total_q, total_kv, H, sl2, out);
  } else if (dtype == TSC_F16) {
    if (D == 64) launch_mma<_Float16, 64>(ctx, grid, q, k, v, cu_q, cu_kv, total_q, total_kv, H, sl2, out);
    else launch_mma<_Float16, 128>(ctx, grid, q, k, v, cu_q, cu_kv, total_q, total_kv, H, sl2, out);
  } else if (D == 64) {
    attn_f32_kernel<64><<<grid, kThreads, 0, ctx->stream>>>(
        (const float*)q, (const float*)k, (const float*)v, cu_q, cu_kv, total_q, total_kv, H, sl2,
        (float*)out);
  } else {
    attn_f32_kernel<128><<<grid, kThreads, 0, ctx->stream>>>(
        (const float*)q, (const float*)k, (const float*)v, cu_q, cu_kv, total_q, total_kv, H, sl2,
        (float*)out);
  }
  return check_hip(hipGetLastError(), "attention launch");
}

}  // namespace tsc
