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
// (tap, Ci-chunk) pairs over XOR-swizzled LDS tiles of gathered A rows (feats[nbr[row,v]], zero
// when nbr < 0) and K-contiguous B rows (W[co, v, ci-chunk]); four waves run 32x32 MFMAs
// (v_mfma_f32_32x32x16_{bf16,f16}, v_mfma_f32_32x32x2_f32).  Two pipelines feed the tiles:
//   conv_mfma_kernel      rows longer than 64 bytes (wide channels, several chunks per tap):
//                         a 3-8 stage ring filled by direct-to-LDS loads (global_load_lds),
//                         per-tap source addresses kept in registers, fragments read with
//                         explicit LDS waits, one block of 4 waves per CU
//   conv_regstage_kernel  rows of at most 64 bytes (one chunk per tap): register-staged double
//                         buffer, one barrier per chunk, two blocks per CU
//
// MFMA operand layout used (32x32 family): lane l supplies A[i = l%32][k in half l/32] and
// B[k in half l/32][j = l%32]; accumulator register r of lane l holds
// D[8*(r/4) + 4*(l/32) + r%4][l%32].  Any assignment of K indices to (lane half, element) is
// valid as long as A and B use the same one; here half h of micro-step s reads 16-byte LDS
// piece 2s+h of the row.

#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "rownorm.h"
#include "tsc_internal.h"

namespace tsc {

// Schedule scratch of tsc_conv_fused_noalloc: one copy per device, alive until the process ends,
// shared by every call on that device (calls that overlap on one device race on it).  Host code
// must not pass `scratch` itself to a kernel: its host-side name is not the device address.  The
// device address comes from hipGetSymbolAddress, once per device (sched_scratch_ptr).
static __device__ __align__(256) int32_t scratch[kSchedScratchBytes / 4];

int sched_scratch_ptr(int device, void** out) {
  static std::mutex mu;
  static std::vector<void*> ptrs;
  std::lock_guard<std::mutex> lock(mu);
  if (device < 0) return fail(TSC_ERR_INVALID, "scratch: bad device %d", device);
  if ((size_t)device < ptrs.size() && ptrs[device]) {
    *out = ptrs[device];
    return TSC_OK;
  }
  int cur = -1;
  int st = check_hip(hipGetDevice(&cur), "scratch: hipGetDevice");
  if (st) return st;
  if (cur != device) return fail(TSC_ERR_INVALID, "scratch: device %d is not current", device);
  void* p = nullptr;
  st = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "scratch: hipGetSymbolAddress");
  if (st) return st;
  if (!p) return fail(TSC_ERR_HIP, "scratch: null symbol address");
  if ((size_t)device >= ptrs.size()) ptrs.resize((size_t)device + 1, nullptr);
  ptrs[device] = p;
  *out = p;
  return TSC_OK;
}

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

// XOR swizzle of 16-byte pieces within an LDS row of PPR pieces.  gfx950 LDS has 64 four-byte
// banks (256 bytes) and serves a ds_read_b128 16 lanes at a time; the MFMA fragment reads have 16
// consecutive lanes reading one logical piece of 16 consecutive rows.  Rows r and r' share bank
// groups when (r*PPR*16) mod 256 agrees, i.e. within each residue of r mod (16/PPR); XOR-ing the
// piece index with (r / (16/PPR)) mod PPR gives those rows distinct pieces -> conflict-free.
template <int PPR>
__device__ __forceinline__ int swz(int row, int part) {
  constexpr int rows_per_256 = 16 / PPR;
  return part ^ ((row / rows_per_256) % PPR);
}

// Zeros in device memory: the source of the gathered A pieces whose neighbor is absent (a
// direct-to-LDS load cannot be told to write zeros).  Rows of up to kZeroBytes bytes: a zero
// piece advances through it by the same Ci offset as a real feature row.
constexpr int kZeroBytes = 65536;
__device__ __attribute__((aligned(16))) uint4 g_zero[kZeroBytes / 16];

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// 32-bit LDS address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}
__device__ __forceinline__ u32x4 lds_read16(uint32_t addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
__device__ __forceinline__ int32_t lds_read_i32(const int32_t* p) {
  int32_t v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(lds_addr(p)));
  return v;
}
// Waits for every LDS read issued so far; pin() then ties a value read by asm to this point, so
// that its uses cannot be scheduled above the wait.
__device__ __forceinline__ void lds_wait_all() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
template <typename V>
__device__ __forceinline__ void pin(V& v) {
  asm volatile("" : "+v"(v));
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// global_load_lds_dwordx4: lane l copies 16 bytes from g to LDS at dst + 16*l (dst is
// wave-uniform).  The builtin only exists for the device; if it appears in a kernel body that the
// host pass also parses, clang silently drops the host-side launch stubs, so it lives here with a
// body compiled in the device pass only.
__device__ __forceinline__ void lds_dma16(const void* g, lds_ptr_t dst) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(g, dst, 16, 0, 0);
#endif
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  // gfx9 s_waitcnt immediate: vmcnt[3:0] | expcnt[6:4] (7 = no wait) | lgkmcnt[11:8] (15 = no
  // wait) | vmcnt[5:4] at [15:14].
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Block -> (row tile, column tile).  The hardware hands block b to XCD b % 8, and each XCD has
// its own L2.
//   * With a schedule (tile_map, built by tile_schedule_kernel): XCD x owns list x of row tiles,
//     longest first (-1: no tile), and computes every column tile of each: its i-th block takes
//     column tile i % n_tiles of list entry i / n_tiles.  The column tiles of one row tile run on
//     neighboring CUs at the same time, so the gathered rows are fetched into that XCD's L2 once
//     for all of them (measured 3-4 % faster than one column tile per XCD, whose weight slice
//     stays in L2 but whose rows are fetched by n_tiles XCDs).
//   * Without, when the column tiles divide 8: each XCD owns one column tile and a contiguous
//     range of row tiles, dealt from the end of the range (in the conv row order the late tiles
//     of each sort window use more taps).
//   * Otherwise each XCD gets a contiguous run of (row, column) tiles with the column tiles of one
//     row tile adjacent.
// per_xcd = blocks per XCD (grid = 8 * per_xcd).
__device__ __forceinline__ bool tile_of(int bid, int m_tiles, int n_tiles, int per_xcd,
                                        const int32_t* tile_map, int* m_tile, int* n_tile) {
  const int xcd = bid & 7, i = bid >> 3;
  if (tile_map) {
    *n_tile = i % n_tiles;
    *m_tile = tile_map[xcd * (per_xcd / n_tiles) + i / n_tiles];
    return *m_tile >= 0;
  }
  if (8 % n_tiles == 0) {
    *n_tile = xcd % n_tiles;
    *m_tile = (xcd / n_tiles) * per_xcd + (per_xcd - 1 - i);
    return *m_tile < m_tiles;
  }
  const int logical = xcd * per_xcd + i;
  *m_tile = logical / n_tiles;
  *n_tile = logical % n_tiles;
  return logical < m_tiles * n_tiles;
}

inline int32_t tile_grid_per_xcd(int32_t m_tiles, int32_t n_tiles) {
  if (8 % n_tiles == 0) {
    const int32_t groups = 8 / n_tiles;
    return (m_tiles + groups - 1) / groups;
  }
  return (int32_t)(((int64_t)m_tiles * n_tiles + 7) / 8);
}

constexpr int kTaps = 27;

// The tile's (row, tap) neighbor indices into LDS (sNbr[r*27 + v], -1 = absent) and the OR of
// the taps present, over this thread's entries j = tid + k*NT.  Every global load is issued
// before the first LDS write, from an address clamped to row 0 for rows past N (row 0 exists
// whenever a tile does): the loop it replaces stored each entry right after its own (skippable)
// load and so waited one global round trip per entry, ~14 in a row per 256-row tile.
template <int ENTRIES, int NT>
__device__ __forceinline__ uint32_t load_tile_nbr(const int32_t* __restrict__ nbr,
                                                  const int32_t* sRow, int32_t* sNbr, int tid) {
  constexpr int PER = (ENTRIES + NT - 1) / NT;
  int32_t sv[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int j = min(tid + k * NT, ENTRIES - 1);
    const int r = j / kTaps, v = j - r * kTaps;
    const int32_t row = sRow[r];
    sv[k] = nbr[(int64_t)(row >= 0 ? row : 0) * kTaps + v];
  }
  uint32_t mask = 0u;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int j = tid + k * NT;
    if (ENTRIES % NT == 0 || j < ENTRIES) {
      const int r = j / kTaps, v = j - r * kTaps;
      const int32_t e = sRow[r] >= 0 ? sv[k] : -1;
      sNbr[j] = e;
      if (e >= 0) mask |= 1u << v;
    }
  }
  return mask;
}

// Longest-first tile schedule.  A row tile's running time is about proportional to the taps it
// uses (the OR of its rows' neighbor masks); with a few rounds of tiles per CU, dealing them in
// row order leaves CUs idle at the end of the launch.  tile_cost_kernel counts each tile's taps;
// tile_schedule_kernel ranks the tiles by decreasing count (counting sort, ties in any order) and
// deals rank k to list g = k mod G on even rounds r = k / G and to G-1 - (k mod G) on odd ones
// (a serpentine), slot g*per + r.  Every list (one per XCD) gets a near-equal share of the work
// and starts with its longest tiles.  Slots past the tile count get -1.  The schedule only
// decides which block computes which tile: every tile's arithmetic is unchanged.
constexpr int kSchedThreads = 256;
static_assert(kSchedMaxTiles == (1 << 16), "schedule bound shared with the scratch size");

__global__ void __launch_bounds__(kSchedThreads)
    tile_cost_kernel(const int32_t* __restrict__ nbr, const int32_t* __restrict__ order, int64_t N,
                     int bm, int32_t* __restrict__ cost) {
  __shared__ uint32_t sMask;
  const int tid = threadIdx.x;
  const int64_t m0 = (int64_t)blockIdx.x * bm;
  if (tid == 0) sMask = 0u;
  __syncthreads();
  uint32_t mask = 0u;
  for (int r = tid; r < bm; r += kSchedThreads) {  // one 108-byte neighbor row per thread
    const int64_t pos = m0 + r;
    const int32_t row = pos < N ? (order ? order[pos] : (int32_t)pos) : -1;
    if (row >= 0) {
      const int32_t* nr = nbr + (int64_t)row * kTaps;
#pragma unroll
      for (int v = 0; v < kTaps; ++v) mask |= (uint32_t)(nr[v] >= 0) << v;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mask |= __shfl_xor(mask, off, 64);
  if ((tid & 63) == 0 && mask) atomicOr(&sMask, mask);
  __syncthreads();
  if (tid == 0) cost[blockIdx.x] = __popc(sMask);
}

__global__ void __launch_bounds__(kSchedThreads)
    tile_schedule_kernel(const int32_t* __restrict__ cost, int32_t m_tiles, int32_t lists,
                         int32_t per, int32_t* __restrict__ tile_map) {
  __shared__ int hist[kTaps + 1];
  __shared__ int next[kTaps + 1];
  const int tid = threadIdx.x;
  if (tid <= kTaps) hist[tid] = 0;
  __syncthreads();
  for (int t = tid; t < m_tiles; t += kSchedThreads) atomicAdd(&hist[cost[t]], 1);
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int c = kTaps; c >= 0; --c) {
      next[c] = run;
      run += hist[c];
    }
  }
  __syncthreads();
  auto slot_of = [&](int k) {
    const int r = k / lists, q = k - r * lists;
    const int g = (r & 1) ? lists - 1 - q : q;
    return g * per + r;
  };
  for (int t = tid; t < m_tiles; t += kSchedThreads) tile_map[slot_of(atomicAdd(&next[cost[t]], 1))] = t;
  for (int k = m_tiles + tid; k < lists * per; k += kSchedThreads) tile_map[slot_of(k)] = -1;
}

template <typename T, int BM, int BN, int KB, int STAGES, int WM, int WN>
struct ConvCfg {
  static constexpr int NT = 64 * WM * WN;
  static constexpr int WAVES = WM * WN;
  static constexpr int PPR = KB / 16;              // 16-byte pieces per LDS row
  static constexpr int KC = KB / (int)sizeof(T);   // K elements per chunk
  static constexpr int EPP = 16 / (int)sizeof(T);  // elements per piece
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int FM = WTM / 32, FN = WTN / 32;
  static constexpr int MS = KB / 32;               // micro-steps per chunk
  static constexpr int A_PIECES = BM * PPR, B_PIECES = BN * PPR;
  static constexpr int PIECES = A_PIECES + B_PIECES;  // per stage
  static constexpr int PPW = PIECES / WAVES;          // pieces per wave per stage
  static constexpr int IPW = (PPW + 63) / 64;         // load instructions per wave per stage
  static constexpr int STAGE_BYTES = PIECES * 16;
  static_assert(KB % 32 == 0 && KB <= 128, "chunk must be 32..128 bytes");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32x32");
  static_assert(PIECES % WAVES == 0, "every wave issues the same loads");
  static_assert(STAGES >= 2 && STAGES <= 8, "ring depth");
  static_assert(IPW * (STAGES - 2) < 64, "vmcnt range");
};

// Compiler-only memory barrier: keeps LDS accesses on their side of s_barrier without the
// s_waitcnt vmcnt(0) that a fence would add (that would drain the in-flight ring loads).
#define TSC_COMPILER_BARRIER() asm volatile("" ::: "memory")

// Submanifold conv tile kernel (see the file comment).  Pipeline per block:
//   prologue   output rows of the tile (via `order`), their 27 neighbor indices into LDS, OR of
//              valid-tap bits -> list of the taps any row of the tile uses
//   main loop  chunks = (used tap, Ci slice of KB bytes).  Chunk c is fetched straight into LDS
//              ring stage c % STAGES with global_load_lds_dwordx4 (gathered A rows, a zero block
//              for absent neighbors; K-contiguous weight rows for B), STAGES-1 chunks ahead.
//              Every wave issues the same IPW loads per chunk, so "chunk c has landed" is the
//              wave's own s_waitcnt vmcnt(IPW * chunks issued after c) followed by one
//              s_barrier.  All reads of the ring are inline asm, which the compiler's wait
//              insertion does not treat as reads of the DMA target, so it adds no vmcnt(0)
//              after the LDS-DMA loads.
//   epilogue   fp32 accumulators + bias (+ residual) rounded once to T, staged through a padded
//              LDS tile (the whole ring), written back as 16-byte runs of the scattered output
//              rows.
template <typename T, int BM, int BN, int KB, int STAGES, int WM, int WN, int EPI>
__global__ void __launch_bounds__(64 * WM * WN)
    conv_mfma_kernel(const T* __restrict__ feats, const T* __restrict__ weight,
                     const T* __restrict__ bias, const int32_t* __restrict__ nbr,
                     const int32_t* __restrict__ order, int64_t N, int32_t Ci, int32_t Co,
                     int32_t m_tiles, int32_t n_tiles, int32_t per_xcd,
                     const int32_t* __restrict__ tile_map, const T* residual, T* out,
                     const T* __restrict__ ln_g, const T* __restrict__ ln_b, float ln_eps) {
  using C = ConvCfg<T, BM, BN, KB, STAGES, WM, WN>;
  constexpr int SB = C::STAGE_BYTES;
  __shared__ __attribute__((aligned(16))) unsigned char ring_mem[STAGES * SB];
  __shared__ int32_t sNbr[BM * kTaps];
  __shared__ int32_t sRow[BM];
  __shared__ int32_t sTaps[kTaps];
  __shared__ uint32_t sMask;
  unsigned char* ring[STAGES];
#pragma unroll
  for (int s = 0; s < STAGES; ++s) ring[s] = ring_mem + s * SB;

  int m_tile, n_tile;
  if (!tile_of(blockIdx.x, m_tiles, n_tiles, per_xcd, tile_map, &m_tile, &n_tile)) return;
  const int64_t m0 = (int64_t)m_tile * BM;
  const int n0 = n_tile * BN;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid / WN, wn = wid % WN;

  if (tid == 0) sMask = 0u;
  for (int r = tid; r < BM; r += C::NT) {
    const int64_t pos = m0 + r;
    sRow[r] = (pos < N) ? (order ? order[pos] : (int32_t)pos) : -1;
  }
  __syncthreads();
  uint32_t mymask = load_tile_nbr<BM * kTaps, C::NT>(nbr, sRow, sNbr, tid);
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

  // Load-issue state.  Chunks are issued in order; whenever the stream enters a new tap, every
  // lane recomputes the byte address (at ci = 0, swizzle applied) of each piece it fetches:
  // the gathered feature row (or the zero block when the neighbor is absent) for A pieces, the
  // weight row W[co, v, :] for B pieces.  Within a tap a chunk only adds its Ci offset.
  const char* gsrc[C::IPW];
  int is_tap = -1, is_k = cpt - 1;
  auto advance = [&]() {
    if (++is_k == cpt) {
      is_k = 0;
      ++is_tap;
      int v = lds_read_i32(sTaps + is_tap);
      lds_wait_all();
      pin(v);
      int32_t src[C::IPW];
#pragma unroll
      for (int j = 0; j < C::IPW; ++j) {
        const int L = min(wid * C::PPW + j * 64 + lane, C::A_PIECES - 1);
        src[j] = lds_read_i32(sNbr + (L / C::PPR) * kTaps + v);
      }
      lds_wait_all();
#pragma unroll
      for (int j = 0; j < C::IPW; ++j) {
        pin(src[j]);
        const int L = wid * C::PPW + j * 64 + lane;
        const bool isA = L < C::A_PIECES;
        const int La = isA ? L : 0, Lb = isA ? 0 : min(L - C::A_PIECES, C::B_PIECES - 1);
        const int ra = La / C::PPR, rb = Lb / C::PPR;
        const char* ga = (src[j] >= 0)
            ? (const char*)(feats + (int64_t)src[j] * Ci + swz<C::PPR>(ra, La % C::PPR) * C::EPP)
            : (const char*)g_zero + swz<C::PPR>(ra, La % C::PPR) * 16;
        const char* gb = (const char*)(weight + ((int64_t)(n0 + rb) * kTaps + v) * Ci +
                                       swz<C::PPR>(rb, Lb % C::PPR) * C::EPP);
        gsrc[j] = isA ? ga : gb;
      }
    }
  };
  // Load instruction j of the current chunk (after advance()) into stage sbase.
  auto dma = [&](int j, unsigned char* sbase) {
    if (C::PPW % 64 == 0 || j * 64 + lane < C::PPW)
      lds_dma16(gsrc[j] + is_k * KB, (lds_ptr_t)(sbase + (wid * C::PPW + j * 64) * 16));
  };
  auto issue = [&](unsigned char* sbase) {
    advance();
#pragma unroll
    for (int j = 0; j < C::IPW; ++j) dma(j, sbase);
  };

  // MFMA over one stage.  Fragments are read with inline-asm ds_read_b128 and an explicit
  // lgkmcnt wait: the compiler sees no LDS read of the ring, so it adds no vmcnt wait for the
  // DMA loads still in flight into the other stages.
  // With nxt set, the next chunk's loads into stage nxt are spread over the micro-steps, each
  // group issued after that micro-step's MFMAs: the wave never stalls on a full load queue
  // ahead of its MFMAs (issuing all of a chunk's loads up front left the matrix pipe idle).
  auto compute = [&](const unsigned char* sA, unsigned char* nxt) {
    const uint32_t a0 = lds_addr(sA), b0 = a0 + C::A_PIECES * 16;
    if (nxt) advance();
    constexpr int JPS = (C::IPW + C::MS - 1) / C::MS;  // loads per micro-step
#pragma unroll
    for (int s = 0; s < C::MS; ++s) {
      const int part = 2 * s + (lane >> 5);
      u32x4 a[C::FM], b[C::FN];
#pragma unroll
      for (int i = 0; i < C::FM; ++i) {
        const int r = wm * C::WTM + i * 32 + (lane & 31);
        a[i] = lds_read16(a0 + r * KB + swz<C::PPR>(r, part) * 16);
      }
#pragma unroll
      for (int j = 0; j < C::FN; ++j) {
        const int r = wn * C::WTN + j * 32 + (lane & 31);
        b[j] = lds_read16(b0 + r * KB + swz<C::PPR>(r, part) * 16);
      }
      lds_wait_all();
#pragma unroll
      for (int i = 0; i < C::FM; ++i) pin(a[i]);
#pragma unroll
      for (int j = 0; j < C::FN; ++j) pin(b[j]);
#pragma unroll
      for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j)
          mfma_piece<T>(__builtin_bit_cast(uint4, a[i]), __builtin_bit_cast(uint4, b[j]),
                        acc[i][j]);
      if (nxt) {
#pragma unroll
        for (int j = s * JPS; j < (s + 1) * JPS; ++j)
          if (j < C::IPW) dma(j, nxt);
      }
    }
  };

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < nchunks) issue(ring[s]);
  for (int c0 = 0; c0 < nchunks; c0 += STAGES) {
#pragma unroll
    for (int s = 0; s < STAGES; ++s) {
      const int c = c0 + s;
      if (c < nchunks) {
        // Chunks issued so far: 0 .. min(nchunks, c + STAGES - 1) - 1; chunk c must be in LDS.
        const int later = min(nchunks - 1 - c, STAGES - 2);
        if (later >= STAGES - 2) wait_vmcnt<C::IPW * (STAGES - 2)>();
        else if (STAGES > 3 && later == 1) wait_vmcnt<C::IPW>();
        else if (STAGES > 4 && later == 2) wait_vmcnt<C::IPW * 2>();
        else if (STAGES > 5 && later == 3) wait_vmcnt<C::IPW * 3>();
        else if (STAGES > 6 && later == 4) wait_vmcnt<C::IPW * 4>();
        else if (STAGES > 7 && later == 5) wait_vmcnt<C::IPW * 5>();
        else wait_vmcnt<0>();
        // Every wave's part of chunk c has landed, and every wave is done reading stage
        // (c - 1) % STAGES (its MFMAs consumed those LDS reads), which is refilled next.
        TSC_COMPILER_BARRIER();
        __builtin_amdgcn_s_barrier();
        TSC_COMPILER_BARRIER();
        compute(ring[s], c + STAGES - 1 < nchunks ? ring[(s + STAGES - 1) % STAGES] : nullptr);
      }
    }
  }

  // Epilogue: bias (+ residual) in fp32, one rounding, staged through the ring (free now) in
  // passes of RPP rows for 16-byte stores of the scattered output rows.  With a residual the
  // staged values stay fp32 when 32 rows of them fit: the residual is then read in the same
  // 16-byte runs as the output (one coalesced load per run instead of one 2-byte load per
  // element), added, and rounded once.
  __syncthreads();
  constexpr int EB = STAGES * SB;  // staging bytes
  constexpr bool RES = EPI == TSC_EPI_BIAS_RESIDUAL;
  // LayerNorm + SiLU over whole rows (BN == Co): each staged row, rounded to T as the conv output
  // would be stored, is normalized with the row pass's arithmetic (rowops.hip): lane l < BN/8
  // sums its 8 consecutive columns in order, one wave butterfly per moment.
  constexpr bool LN = EPI == TSC_EPI_BIAS_LN_SILU;
  static_assert(!LN || (sizeof(T) == 2 && BN % 64 == 0 && BN <= 512), "LN epilogue shape");
  constexpr bool RES_IN_COPY = RES && (sizeof(T) == 4 || EB / (BN * 4) >= 32);
  using S = typename std::conditional<RES_IN_COPY, float, T>::type;  // staged element type
  constexpr int ROWB = BN * (int)sizeof(S);
  constexpr int LDE = EB / (ROWB + 16) >= 32 ? ROWB + 16 : ROWB;  // padded row stride if it fits
  constexpr int RFIT = EB / LDE;
  constexpr int RPP = RFIT >= BM ? BM : RFIT >= 128 && BM % 128 == 0 ? 128
                    : RFIT >= 64 && BM % 64 == 0 ? 64 : 32;  // rows per pass, dividing BM
  static_assert(RFIT >= 32 && BM % RPP == 0, "epilogue pass must hold 32-row blocks");
  constexpr int PIECES_PER_ROW = BN / C::EPP;  // 16-byte output pieces per row
  unsigned char* sE = ring_mem;
#pragma unroll
  for (int p0 = 0; p0 < BM; p0 += RPP) {
#pragma unroll
    for (int i = 0; i < C::FM; ++i) {
      const int rb = wm * C::WTM + i * 32;  // first row of this 32-row fragment block
      if (rb < p0 || rb >= p0 + RPP) continue;
#pragma unroll
      for (int j = 0; j < C::FN; ++j) {
        const int cl = wn * C::WTN + j * 32 + (lane & 31);
        const float bv = bias ? to_f32<T>(bias[n0 + cl]) : 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int rl = rb + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          float val = acc[i][j][e] + bv;
          if (RES && !RES_IN_COPY) {
            const int32_t row = sRow[rl];
            if (row >= 0) val += to_f32<T>(residual[(int64_t)row * Co + n0 + cl]);
          }
          S* dst = (S*)(sE + (rl - p0) * LDE + cl * (int)sizeof(S));
          if constexpr (std::is_same<S, float>::value) *dst = val;
          else *dst = from_f32<T>(val);
        }
      }
    }
    __syncthreads();
    if constexpr (LN) {
      constexpr int NV = BN / 8;  // 16-byte vectors per row
      const bool has = lane < NV;
      float g[8], bb[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        g[e] = (has && ln_g) ? to_f32<T>(ln_g[8 * lane + e]) : 1.f;
        bb[e] = (has && ln_b) ? to_f32<T>(ln_b[8 * lane + e]) : 0.f;
      }
      for (int r = wid; r < RPP; r += C::NT / 64) {
        const int32_t row = sRow[p0 + r];
        if (row < 0) continue;  // wave-uniform
        float v[8];
        float s = 0.f;
        if (has) {
          const uint4 u = *(const uint4*)(sE + r * LDE + lane * 16);
          const T* tv = (const T*)&u;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            v[e] = to_f32<T>(tv[e]);
            s += v[e];
          }
        }
        const float mean = rn_wave_sum(s) / (float)BN;
        float qs = 0.f;
        if (has) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float d = v[e] - mean;
            qs += d * d;
          }
        }
        const float var = rn_wave_sum(qs) / (float)BN;
        const float inv = 1.0f / sqrtf(var + ln_eps);
        if (has) {
          T y[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) y[e] = from_f32<T>(rn_silu((v[e] - mean) * inv * g[e] + bb[e]));
          *(uint4*)(out + (int64_t)row * Co + n0 + 8 * lane) = *(const uint4*)y;
        }
      }
      __syncthreads();
      continue;
    }
    for (int q = tid; q < RPP * PIECES_PER_ROW; q += C::NT) {
      const int r = q / PIECES_PER_ROW, pc = q - r * PIECES_PER_ROW;
      const int32_t row = sRow[p0 + r];
      if (row < 0) continue;
      T* dst = out + (int64_t)row * Co + n0 + pc * C::EPP;
      if constexpr (RES_IN_COPY) {
        // The residual run is read before the output run is written by the same thread, so the
        // output may alias the residual.
        const uint4 rr = *(const uint4*)(residual + (int64_t)row * Co + n0 + pc * C::EPP);
        const T* rt = (const T*)&rr;
        const float* sv = (const float*)(sE + r * LDE + pc * C::EPP * 4);
        T y[C::EPP];
#pragma unroll
        for (int k = 0; k < C::EPP; ++k) y[k] = from_f32<T>(sv[k] + to_f32<T>(rt[k]));
        *(uint4*)dst = *(const uint4*)y;
      } else {
        *(uint4*)dst = *(const uint4*)(sE + r * LDE + pc * 16);
      }
    }
    __syncthreads();
  }
}

// Register-staged variant for rows of at most 64 bytes (one K chunk per tap, e.g. 32 fp16
// channels): each thread loads its share of the next chunk into registers while the current
// chunk is multiplied, then stores it to a double-buffered LDS tile; one barrier per chunk.
// With a single chunk per tap there is no per-tap address reuse for the direct-to-LDS ring to
// exploit, and this shorter pipeline (two blocks per CU) keeps more rows in flight.
template <typename T, int BM, int BN, int KB, int WM, int WN, int EPI>
struct RegCfg {
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
    conv_regstage_kernel(const T* __restrict__ feats, const T* __restrict__ weight,
                     const T* __restrict__ bias, const int32_t* __restrict__ nbr,
                     const int32_t* __restrict__ order, int64_t N, int32_t Ci, int32_t Co,
                     int32_t m_tiles, int32_t n_tiles, int32_t per_xcd,
                     const T* __restrict__ residual, T* __restrict__ out) {
  using C = RegCfg<T, BM, BN, KB, WM, WN, EPI>;
  __shared__ __attribute__((aligned(16))) unsigned char sA[2][BM * KB];
  __shared__ __attribute__((aligned(16))) unsigned char sB[2][BN * KB];
  __shared__ int32_t sNbr[BM * kTaps];
  __shared__ int32_t sRow[BM];
  __shared__ int32_t sTaps[kTaps];
  __shared__ uint32_t sMask;

  int m_tile, n_tile;
  if (!tile_of(blockIdx.x, m_tiles, n_tiles, per_xcd, nullptr, &m_tile, &n_tile)) return;
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
  uint32_t mymask = load_tile_nbr<BM * kTaps, C::NT>(nbr, sRow, sNbr, tid);
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

  // Epilogue: bias (+ residual), round to T, scatter rows back to their original positions.  The
  // residual values are all loaded before the first store (rows past N read row 0 and are not
  // stored): loads under per-row branches would each wait for the one before.  Every output
  // element is read and written by the same lane, so the output may alias the residual.
#pragma unroll
  for (int j = 0; j < C::FN; ++j) {
    const int co = n0 + wn * C::WTN + j * 32 + (lane & 31);
    const float bv = bias ? to_f32<T>(bias[co]) : 0.f;
    float rv[C::FM][16];
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        rv[i][e] = 0.f;
        if (EPI == TSC_EPI_BIAS_RESIDUAL) {
          const int rl = wm * C::WTM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          const int32_t row = sRow[rl];
          rv[i][e] = to_f32<T>(residual[(int64_t)(row >= 0 ? row : 0) * Co + co]);
        }
      }
#pragma unroll
    for (int i = 0; i < C::FM; ++i) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int rl = wm * C::WTM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int32_t row = sRow[rl];
        if (row >= 0) {
          float val = acc[i][j][e] + bv;
          if (EPI == TSC_EPI_BIAS_RESIDUAL) val += rv[i][e];
          out[(int64_t)row * Co + co] = from_f32<T>(val);
        }
      }
    }
  }
}


template <typename T, int BM, int BN, int KB, int WM, int WN, int EPI>
int launch_reg(tsc_ctx* ctx, const ConvArgs& a) {
  const int32_t m_tiles = (int32_t)((a.N + BM - 1) / BM);
  const int32_t n_tiles = a.Co / BN;
  const int32_t per_xcd = tile_grid_per_xcd(m_tiles, n_tiles);
  const unsigned grid = (unsigned)per_xcd * 8u;
  static const std::string name = std::string("conv_regstage_kernel<") +
      (sizeof(T) == 4 ? "f32" : std::is_same<T, __bf16>::value ? "bf16" : "f16") + "," +
      std::to_string(BM) + "x" + std::to_string(BN) + ",k" + std::to_string(KB) +
      (EPI == TSC_EPI_BIAS_RESIDUAL ? ",res>" : ">");
  ProfScope p(ctx, name.c_str());
  conv_regstage_kernel<T, BM, BN, KB, WM, WN, EPI><<<grid, 64 * WM * WN, 0, ctx->stream>>>(
      (const T*)a.feats, (const T*)a.weight, (const T*)a.bias, a.nbr, a.order, a.N, a.Ci, a.Co,
      m_tiles, n_tiles, per_xcd, (const T*)a.residual, (T*)a.out);
  return check_hip(hipGetLastError(), "conv launch");
}

template <typename T, int BM, int BN, int KB, int WM, int WN, int EPI, int BPC = 2>
int launch_cfg(tsc_ctx* ctx, const ConvArgs& a) {
  // Ring stages: as many as fit beside the neighbor tile in 1/BPC of the 160 KB of LDS per CU
  // (BPC blocks share a CU, so one block's memory stalls overlap another's MFMAs); at most 8.
  constexpr int STAGE = (BM + BN) * KB;
  constexpr int FIXED = BM * kTaps * 4 + BM * 4 + 256;
  constexpr int FIT = (163840 / BPC - 512 - FIXED) / STAGE;
  constexpr int STAGES = FIT < 8 ? FIT : 8;
  static_assert(STAGES >= 2, "ring too shallow");
  const int32_t m_tiles = (int32_t)((a.N + BM - 1) / BM);
  const int32_t n_tiles = a.Co / BN;
  int32_t per_xcd = tile_grid_per_xcd(m_tiles, n_tiles);
  // Longest-first schedule for the 256-row tile (several rounds of long tiles per CU): one list
  // of row tiles per XCD, every column tile of a row tile on the same XCD.
  const int32_t* tile_map = nullptr;
  if (BM == 256 && m_tiles <= kSchedMaxTiles) {
    const int32_t lists = 8, per_list = (m_tiles + lists - 1) / lists;
    const size_t need = ((size_t)m_tiles + (size_t)lists * per_list) * 4;
    void* ws;
    tsc_sched_entry* entry = nullptr;
    if (a.sched_scratch) {  // the caller's fixed buffer (tsc_conv_fused_noalloc): built per call
      if (need > a.sched_scratch_bytes)
        return fail(TSC_ERR_INVALID, "conv: schedule needs %zu bytes of scratch, %zu available",
                    need, a.sched_scratch_bytes);
      ws = a.sched_scratch;
    } else {  // the context's cache: built by the first conv over this map and row order
      int st = sched_cached(ctx, a.nbr, a.order, a.N, BM, need, &entry);
      if (st) return st;
      ws = entry->buf;
    }
    int32_t* cost = (int32_t*)ws;
    int32_t* map = cost + m_tiles;
    if (!entry || !entry->valid) {
      {
        ProfScope p(ctx, "conv_tile_cost");
        tile_cost_kernel<<<m_tiles, kSchedThreads, 0, ctx->stream>>>(a.nbr, a.order, a.N, BM,
                                                                       cost);
      }
      {
        ProfScope p(ctx, "conv_tile_schedule");
        tile_schedule_kernel<<<1, kSchedThreads, 0, ctx->stream>>>(cost, m_tiles, lists,
                                                                     per_list, map);
      }
      int st = check_hip(hipGetLastError(), "conv tile schedule");
      if (st) return st;
      if (entry) entry->valid = true;
    }
    tile_map = map;
    per_xcd = per_list * n_tiles;
  }
  const unsigned grid = (unsigned)per_xcd * 8u;
  static const std::string name = std::string("conv_mfma_kernel<") +
      (sizeof(T) == 4 ? "f32" : std::is_same<T, __bf16>::value ? "bf16" : "f16") + "," +
      std::to_string(BM) + "x" + std::to_string(BN) + ",k" + std::to_string(KB) + ",s" +
      std::to_string(STAGES) +
      (EPI == TSC_EPI_BIAS_RESIDUAL ? ",res>" : EPI == TSC_EPI_BIAS_LN_SILU ? ",ln>" : ">");
  ProfScope p(ctx, name.c_str());
  conv_mfma_kernel<T, BM, BN, KB, STAGES, WM, WN, EPI><<<grid, 64 * WM * WN, 0, ctx->stream>>>(
      (const T*)a.feats, (const T*)a.weight, (const T*)a.bias, a.nbr, a.order, a.N, a.Ci, a.Co,
      m_tiles, n_tiles, per_xcd, tile_map, (const T*)a.residual, (T*)a.out,
      (const T*)a.ln_gamma, (const T*)a.ln_beta, a.ln_eps);
  return check_hip(hipGetLastError(), "conv launch");
}

// Narrow-channel kernel (Ci = 32: one 64-byte row per neighbor for 16-bit types, 128 bytes for
// fp32).  Every wave works alone on tiles of 32 output rows; there is no block barrier after the
// weights are staged.  fp32 keeps the same layout with two 16-byte pieces per lane and runs each
// tap as eight v_mfma_f32_16x16x4f32 steps (lane quarter q holds channels 8q..8q+7).  The
// design minimises distinct cache lines per memory instruction, which bounds the L1/TA rate of
// gather-heavy code:
//   rows      the 32 rows of the tile (entries of `order`); their 32 x 27 neighbor indices are
//             read with consecutive lanes on consecutive words of each 108-byte row and parked in
//             the wave's LDS slice as [tap][row]; an OR-reduction gives the tile's tap mask.
//   taps      only the tile's taps are visited; a ring of R slots holds the gathered feature
//             rows of the next R taps, 16 bytes per lane: in v_mfma_f32_16x16x32 B-operand order
//             lanes l, l+16, l+32, l+48 hold the four 16-byte pieces of row l%16, so one load
//             instruction fetches 16 whole rows (an absent neighbor reads the zero block).
//   MFMA      transposed product D[co][row] = W[co][k] * F[row][k]: A = weight fragment from LDS
//             (the (Co,27,Ci) tensor is staged once per block, 16-byte pieces XOR-swizzled per
//             row), B = the gathered rows.  Two 16-row blocks x Co/16 column blocks per tap.
//   epilogue  lane l owns row 16*rb + l%16 and co 16*cb + 4*(l/16) + {0..3}: bias (+ residual)
//             in fp32, one rounding, 8-byte stores.
// Tiles are dealt XCD-contiguously: XCD x owns tiles [x*tpx, (x+1)*tpx), so each XCD's L2 sees one
// spatial region of gathered rows.
constexpr int kNarrowSlots = 4;
typedef float f32x4_t __attribute__((__vector_size__(4 * sizeof(float))));

template <typename T>
__device__ __forceinline__ void mfma16_piece(const uint4& a, const uint4& b, f32x4_t& acc);
template <>
__device__ __forceinline__ void mfma16_piece<__bf16>(const uint4& a, const uint4& b,
                                                     f32x4_t& acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), acc, 0, 0, 0);
}
template <>
__device__ __forceinline__ void mfma16_piece<_Float16>(const uint4& a, const uint4& b,
                                                       f32x4_t& acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                               __builtin_bit_cast(f16x8_t, b), acc, 0, 0, 0);
}

// Eight v_mfma_f32_16x16x4f32 steps over the 8 fp32 values (two 16-byte pieces) of each operand.
__device__ __forceinline__ void mfma16_f32x8(const uint4 (&a)[2], const uint4 (&b)[2],
                                             f32x4_t& acc) {
  const uint32_t* av = (const uint32_t*)a;
  const uint32_t* bv = (const uint32_t*)b;
#pragma unroll
  for (int s = 0; s < 8; ++s)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(av[s]), __uint_as_float(bv[s]),
                                               acc, 0, 0, 0);
}

template <typename T, int CO, int EPI, int NT>
__global__ void __launch_bounds__(NT)
    conv_narrow_kernel(const T* __restrict__ feats, const T* __restrict__ weight,
                       const T* __restrict__ bias, const int32_t* __restrict__ nbr,
                       const int32_t* __restrict__ order, int64_t N, int32_t n_tiles,
                       int32_t tiles_per_xcd, const T* residual, T* out) {
  constexpr int CI = 32;
  constexpr int PL = sizeof(T) == 4 ? 2 : 1;  // 16-byte pieces per lane per row (fp32: 32 bytes)
  constexpr int PPR = 4 * PL;                 // 16-byte pieces per weight / feature row
  constexpr int CB = CO / 16;       // 16-column output blocks
  constexpr int NW = NT / 64;
  constexpr int R = kNarrowSlots;
  static_assert(CO % 16 == 0, "narrow kernel: Co multiple of 16");
  __shared__ uint4 sW[kTaps * CO * PPR];
  __shared__ int32_t sNb[NW][kTaps * 32];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int l16 = lane & 15, q = lane >> 4;

  // Stage W (Co,27,Ci): global piece g = (co*27 + v)*PPR + p  ->  LDS [(v*CO + co)*PPR + swz(p)].
  // fp32 rows are 128 bytes: piece p of row co sits at p ^ (co & 7), so the 8 lanes of one
  // 16-byte read step (8 consecutive co, one piece) cover all 32 banks.
  auto wslot = [](int co, int p) {
    if constexpr (sizeof(T) == 4) return p ^ (co & 7);
    else return swz<PPR>(co, p);
  };
  const uint4* wq = (const uint4*)weight;
  for (int g = tid; g < CO * kTaps * PPR; g += NT) {
    const int p = g % PPR, cv = g / PPR, v = cv % kTaps, co = cv / kTaps;
    sW[(v * CO + co) * PPR + wslot(co, p)] = wq[g];
  }
  __syncthreads();
  int32_t* const nbw = sNb[wid];

  const int xcd = blockIdx.x & 7;
  const int t_begin = xcd * tiles_per_xcd;
  const int t_end = min(n_tiles, t_begin + tiles_per_xcd);
  const int stride = (int)(gridDim.x >> 3) * NW;
  // Tiles are software-pipelined: while tile t computes, the neighbor indices of tile t+1 and
  // the row numbers of tile t+2 are in flight, so a tile starts without a dependent round trip.
  // Neighbor indices: iteration it reads rows 7*it .. 7*it+6, lane l < 63 taking taps
  // 3*(l%9) .. 3*(l%9)+2 of row 7*it + l/9 as one 12-byte load (five load instructions per tile;
  // the address unit's work per gather-heavy tile is what bounds this kernel).  They land in the
  // wave's LDS slice as [row][tap]: lane l writes words 3l .. 3l+2 of the 7-row block, stride 3
  // across lanes, conflict-free (odd row stride: the slot fills' 16-lane reads of one tap hit
  // distinct banks).
  constexpr int kNbrIters = (32 + 6) / 7;
  const int nr = lane / 9, nk = lane - nr * 9;  // nr = 7 for the idle lane 63
  auto load_row = [&](int t) -> int32_t {
    const int64_t pos = (int64_t)t * 32 + (lane & 31);
    return (t < t_end && pos < N) ? (order ? order[pos] : (int32_t)pos) : -1;
  };
  int32_t val[kNbrIters][3];
  auto load_nbr = [&](int32_t rows) {
#pragma unroll
    for (int it = 0; it < kNbrIters; ++it) {
      const int rr = it * 7 + nr;
      const int32_t row = __shfl(rows, rr & 31, 64);
      if (nr < 7 && rr < 32 && row >= 0) {
        const int32_t* src = nbr + (int64_t)row * kTaps + 3 * nk;
        val[it][0] = src[0];
        val[it][1] = src[1];
        val[it][2] = src[2];
      } else {
        val[it][0] = val[it][1] = val[it][2] = -1;
      }
    }
  };
  int tile = t_begin + (int)(blockIdx.x >> 3) * NW + wid;
  int32_t my_row = load_row(tile);
  int32_t row_next = load_row(tile + stride);
  load_nbr(my_row);
  for (; tile < t_end; tile += stride) {
#pragma unroll
    for (int it = 0; it < kNbrIters; ++it) {
      if (nr < 7 && it * 7 + nr < 32) {
        int32_t* dst = nbw + (it * 7 + nr) * kTaps + 3 * nk;
        dst[0] = val[it][0];
        dst[1] = val[it][1];
        dst[2] = val[it][2];
      }
    }
    load_nbr(row_next);
    const int32_t row_after = load_row(tile + 2 * stride);
    // Tap mask: lane l < 54 ORs tap l % 27 over rows [16*(l/27), 16*(l/27)+16).
    uint32_t mymask = 0;
    if (lane < 2 * kTaps) {
      const int v = lane % kTaps, r0 = (lane / kTaps) * 16;
      bool any = false;
#pragma unroll
      for (int r = 0; r < 16; ++r) any |= nbw[(r0 + r) * kTaps + v] >= 0;
      mymask = any ? 1u << v : 0u;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mymask |= __shfl_xor(mymask, off, 64);
    const uint32_t tmask = __builtin_amdgcn_readfirstlane(mymask);
    const int ntaps = __popc(tmask);

    f32x4_t acc[2][CB];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[rb][cb][e] = 0.f;

    // Slot ring: slot r holds tap vt[r] (-1 past the last tap: zero-block pieces, never used).
    uint32_t rem = tmask;
    int vt[R];
    uint4 fr[R][2][PL];
    // Loads are coalesced (lanes 4j..4j+3 read the four quarters of row 16*rb + j, one request
    // per row); the fragment the MFMA wants in lane t (row t%16, quarter t/16) is then fetched
    // from lane 4*(t%16) + t/16 with ds_bpermute right before use.
    auto fill = [&](int r) {
      const int v = rem ? __builtin_ctz(rem) : -1;
      rem &= rem - 1u;
      vt[r] = v;
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        const int32_t sidx = v >= 0 ? nbw[(rb * 16 + (lane >> 2)) * kTaps + v] : -1;
        const T* src = sidx >= 0 ? feats + (int64_t)sidx * CI + (lane & 3) * 8
                                 : (const T*)g_zero + (lane & 3) * 8;
#pragma unroll
        for (int h = 0; h < PL; ++h) fr[r][rb][h] = *(const uint4*)(src + h * (16 / sizeof(T)));
      }
    };
    const int src_lane = 4 * l16 + q;
    auto to_mfma = [&](const uint4& x) {
      uint4 y;
      y.x = __shfl(x.x, src_lane, 64);
      y.y = __shfl(x.y, src_lane, 64);
      y.z = __shfl(x.z, src_lane, 64);
      y.w = __shfl(x.w, src_lane, 64);
      return y;
    };
#pragma unroll
    for (int r = 0; r < R; ++r) fill(r);
    for (int t0 = 0; t0 < ntaps; t0 += R) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (t0 + r < ntaps) {
          const int v = vt[r];
          uint4 b0[PL], b1[PL];
#pragma unroll
          for (int h = 0; h < PL; ++h) {
            b0[h] = to_mfma(fr[r][0][h]);
            b1[h] = to_mfma(fr[r][1][h]);
          }
#pragma unroll
          for (int cb = 0; cb < CB; ++cb) {
            const int co = cb * 16 + l16;
            if constexpr (sizeof(T) == 4) {
              // k-step s of v_mfma_f32_16x16x4f32: lane (co / row, quarter q) holds ci 8q + s
              const uint4 wa[2] = {sW[(v * CO + co) * PPR + wslot(co, 2 * q)],
                                   sW[(v * CO + co) * PPR + wslot(co, 2 * q + 1)]};
              mfma16_f32x8(wa, b0, acc[0][cb]);
              mfma16_f32x8(wa, b1, acc[1][cb]);
            } else {
              const uint4 wa = sW[(v * CO + co) * PPR + wslot(co, q)];
              mfma16_piece<T>(wa, b0[0], acc[0][cb]);
              mfma16_piece<T>(wa, b1[0], acc[1][cb]);
            }
          }
        }
        fill(r);
      }
    }

    // Epilogue.  Bias and residual values are all loaded before the first store (rows past N
    // read row 0 and are not stored): loads under the per-row branches would each wait for the
    // one before.  Each output element is read and written by the same lane, so the output may
    // alias the residual.
    struct alignas(4 * sizeof(T)) V4 {
      T v[4];
    };
    int32_t rows[2];
    V4 bt[CB], rt[2][CB];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) rows[rb] = __shfl(my_row, rb * 16 + l16, 64);
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int c0 = cb * 16 + 4 * q;
      if (bias) bt[cb] = *(const V4*)(bias + c0);
      if (EPI == TSC_EPI_BIAS_RESIDUAL) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
          rt[rb][cb] = *(const V4*)(residual + (int64_t)(rows[rb] >= 0 ? rows[rb] : 0) * CO + c0);
      }
    }
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int32_t row = rows[rb];
      if (row < 0) continue;
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int c0 = cb * 16 + 4 * q;
        float x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = acc[rb][cb][i];
        if (bias) {
#pragma unroll
          for (int i = 0; i < 4; ++i) x[i] += to_f32<T>(bt[cb].v[i]);
        }
        if (EPI == TSC_EPI_BIAS_RESIDUAL) {
#pragma unroll
          for (int i = 0; i < 4; ++i) x[i] += to_f32<T>(rt[rb][cb].v[i]);
        }
        V4 y;
#pragma unroll
        for (int i = 0; i < 4; ++i) y.v[i] = from_f32<T>(x[i]);
        *(V4*)(out + (int64_t)row * CO + c0) = y;
      }
    }
    my_row = row_next;
    row_next = row_after;
  }
}

template <typename T, int CO, int EPI>
int launch_narrow(tsc_ctx* ctx, const ConvArgs& a) {
  // Block size: 8 waves (one block per CU) when the weights + per-wave neighbor slices fit.
  // Measured on the 1.5M-voxel shell: 8 waves beat 16 (fewer concurrent gathers thrash the
  // L1/L2 less) and 4 (too little memory-level parallelism).
  constexpr int kW = kTaps * CO * 4 * 16 * (sizeof(T) == 4 ? 2 : 1);
  constexpr int kPerWave = kTaps * 32 * 4;
  constexpr int NW = std::min(8, (163840 - 1024 - kW) / kPerWave);
  static_assert(NW >= 4, "narrow kernel: weights too large for LDS");
  constexpr int NT = NW * 64;
  const int32_t n_tiles = (int32_t)((a.N + 31) / 32);
  const int32_t tpx = (n_tiles + 7) / 8;
  int32_t blocks = std::min<int32_t>(256, (n_tiles + NW - 1) / NW);
  blocks = std::max<int32_t>(8, (blocks + 7) / 8 * 8);
  static const std::string name = std::string("conv_narrow_kernel<") +
      (std::is_same<T, __bf16>::value ? "bf16" : sizeof(T) == 4 ? "f32" : "f16") + ",32x" +
      std::to_string(CO) + (EPI == TSC_EPI_BIAS_RESIDUAL ? ",res>" : ">");
  ProfScope p(ctx, name.c_str());
  conv_narrow_kernel<T, CO, EPI, NT><<<blocks, NT, 0, ctx->stream>>>(
      (const T*)a.feats, (const T*)a.weight, (const T*)a.bias, a.nbr, a.order, a.N, n_tiles, tpx,
      (const T*)a.residual, (T*)a.out);
  return check_hip(hipGetLastError(), "conv launch");
}

// Any channel counts (the reference bounds-checks Ci and Co, conv3d_wgsl.ts:174-196, so it takes
// any shape): 64-row x 64-column tiles of four 32x32 waves, K in chunks of 32 bytes per row.
// Each chunk is loaded into registers in pieces of LW bytes (the widest width that divides the
// row and the buffers' alignment), with pieces past Ci or past Co replaced by zeros, then stored
// to a double-buffered LDS tile; zero pieces add exact zeros to the accumulators, so the K tail
// needs no special case.  The epilogue stores element by element, masking columns past Co.
// This is the path for shapes the tuned kernels do not take (row bytes not a multiple of 32,
// Co not a multiple of 32, or buffers that are not 16-byte aligned).
template <int LW> struct PieceOf;
template <> struct PieceOf<2> { typedef uint16_t type; };
template <> struct PieceOf<4> { typedef uint32_t type; };
template <> struct PieceOf<8> { typedef uint2 type; };
template <> struct PieceOf<16> { typedef uint4 type; };

constexpr int kGenBM = 64, kGenBN = 64, kGenKB = 32, kGenThreads = 256;

template <typename T, int LW, int EPI>
__global__ void __launch_bounds__(kGenThreads)
    conv_generic_kernel(const T* __restrict__ feats, const T* __restrict__ weight,
                        const T* __restrict__ bias, const int32_t* __restrict__ nbr,
                        const int32_t* __restrict__ order, int64_t N, int32_t Ci, int32_t Co,
                        int32_t m_tiles, int32_t n_tiles, int32_t per_xcd, const T* residual,
                        T* out) {
  typedef typename PieceOf<LW>::type P;
  constexpr int BM = kGenBM, BN = kGenBN, KB = kGenKB, NT = kGenThreads;
  constexpr int EPL = LW / (int)sizeof(T);  // elements per piece
  constexpr int KC = KB / (int)sizeof(T);   // elements per chunk
  constexpr int LPR = KB / LW;              // pieces per row per chunk
  constexpr int AL = BM * LPR / NT > 0 ? BM * LPR / NT : 1;
  constexpr int BL = BN * LPR / NT > 0 ? BN * LPR / NT : 1;
  static_assert((BM * LPR) % NT == 0 || BM * LPR < NT, "A pieces per thread");
  __shared__ __attribute__((aligned(16))) unsigned char sA[2][BM * KB];
  __shared__ __attribute__((aligned(16))) unsigned char sB[2][BN * KB];
  __shared__ int32_t sNbr[BM * kTaps];
  __shared__ int32_t sRow[BM];
  __shared__ int32_t sTaps[kTaps];
  __shared__ uint32_t sMask;

  int m_tile, n_tile;
  if (!tile_of(blockIdx.x, m_tiles, n_tiles, per_xcd, nullptr, &m_tile, &n_tile)) return;
  const int64_t m0 = (int64_t)m_tile * BM;
  const int n0 = n_tile * BN;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid >> 1, wn = wid & 1;  // 2 x 2 waves of 32 x 32

  if (tid == 0) sMask = 0u;
  for (int r = tid; r < BM; r += NT) {
    const int64_t pos = m0 + r;
    sRow[r] = (pos < N) ? (order ? order[pos] : (int32_t)pos) : -1;
  }
  __syncthreads();
  uint32_t mymask = load_tile_nbr<BM * kTaps, NT>(nbr, sRow, sNbr, tid);
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

  const int cpt = (Ci + KC - 1) / KC;  // chunks per tap, the last one zero-padded
  const int nchunks = ntaps * cpt;
  f32x16_t acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;

  P ra[AL], rb[BL];
  P zero;
  __builtin_memset(&zero, 0, sizeof(P));
  auto load_chunk = [&](int c) {
    const int ti = c / cpt;
    const int ci0 = (c - ti * cpt) * KC;
    const int v = sTaps[ti];
#pragma unroll
    for (int j = 0; j < AL; ++j) {
      const int q = tid + j * NT;
      P val = zero;
      if (q < BM * LPR) {
        const int r = q / LPR, ci = ci0 + (q % LPR) * EPL;
        const int32_t src = sNbr[r * kTaps + v];
        if (src >= 0 && ci < Ci) val = *(const P*)(feats + (int64_t)src * Ci + ci);
      }
      ra[j] = val;
    }
#pragma unroll
    for (int j = 0; j < BL; ++j) {
      const int q = tid + j * NT;
      P val = zero;
      if (q < BN * LPR) {
        const int r = q / LPR, ci = ci0 + (q % LPR) * EPL;
        if (n0 + r < Co && ci < Ci)
          val = *(const P*)(weight + ((int64_t)(n0 + r) * kTaps + v) * Ci + ci);
      }
      rb[j] = val;
    }
  };
  // Piece k of row r sits at byte k*LW of the row's 32 bytes; its 16-byte half is swizzled.
  auto lds_off = [](int r, int k) {
    const int byte = k * LW;
    return r * KB + swz<2>(r, byte >> 4) * 16 + (byte & 15);
  };
  auto store_chunk = [&](int buf) {
#pragma unroll
    for (int j = 0; j < AL; ++j) {
      const int q = tid + j * NT;
      if (q < BM * LPR) *(P*)(&sA[buf][lds_off(q / LPR, q % LPR)]) = ra[j];
    }
#pragma unroll
    for (int j = 0; j < BL; ++j) {
      const int q = tid + j * NT;
      if (q < BN * LPR) *(P*)(&sB[buf][lds_off(q / LPR, q % LPR)]) = rb[j];
    }
  };

  if (nchunks > 0) {
    load_chunk(0);
    store_chunk(0);
  }
  const int part = lane >> 5;
  const int ar = wm * 32 + (lane & 31), br = wn * 32 + (lane & 31);
  for (int c = 0; c < nchunks; ++c) {
    const int buf = c & 1;
    __syncthreads();
    if (c + 1 < nchunks) load_chunk(c + 1);
    const uint4 a = *(const uint4*)(&sA[buf][ar * KB + swz<2>(ar, part) * 16]);
    const uint4 b = *(const uint4*)(&sB[buf][br * KB + swz<2>(br, part) * 16]);
    mfma_piece<T>(a, b, acc);
    if (c + 1 < nchunks) store_chunk(buf ^ 1);
  }

  const int co = n0 + wn * 32 + (lane & 31);
  if (co >= Co) return;
  const float bv = bias ? to_f32<T>(bias[co]) : 0.f;
  // Residual values first, all loads before the first store (see conv_regstage_kernel).
  float rv[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    rv[e] = 0.f;
    if (EPI == TSC_EPI_BIAS_RESIDUAL) {
      const int32_t row = sRow[wm * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)];
      rv[e] = to_f32<T>(residual[(int64_t)(row >= 0 ? row : 0) * Co + co]);
    }
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int rl = wm * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
    const int32_t row = sRow[rl];
    if (row < 0) continue;
    float val = acc[e] + bv;
    if (EPI == TSC_EPI_BIAS_RESIDUAL) val += rv[e];
    out[(int64_t)row * Co + co] = from_f32<T>(val);
  }
}

template <typename T, int LW, int EPI>
int launch_generic(tsc_ctx* ctx, const ConvArgs& a) {
  const int32_t m_tiles = (int32_t)((a.N + kGenBM - 1) / kGenBM);
  const int32_t n_tiles = (a.Co + kGenBN - 1) / kGenBN;
  const int32_t per_xcd = tile_grid_per_xcd(m_tiles, n_tiles);
  static const std::string name = std::string("conv_generic_kernel<") +
      (sizeof(T) == 4 ? "f32" : std::is_same<T, __bf16>::value ? "bf16" : "f16") + ",p" +
      std::to_string(LW) + (EPI == TSC_EPI_BIAS_RESIDUAL ? ",res>" : ">");
  ProfScope p(ctx, name.c_str());
  conv_generic_kernel<T, LW, EPI><<<(unsigned)per_xcd * 8u, kGenThreads, 0, ctx->stream>>>(
      (const T*)a.feats, (const T*)a.weight, (const T*)a.bias, a.nbr, a.order, a.N, a.Ci, a.Co,
      m_tiles, n_tiles, per_xcd, (const T*)a.residual, (T*)a.out);
  return check_hip(hipGetLastError(), "conv launch");
}

template <typename T, int EPI>
int dispatch_generic(tsc_ctx* ctx, const ConvArgs& a) {
  // Widest piece that divides the row and the feats / weight addresses.
  const uintptr_t al = (uintptr_t)a.feats | (uintptr_t)a.weight;
  const int row = a.Ci * (int)sizeof(T);
  auto fits = [&](int w) { return row % w == 0 && al % w == 0; };
  if (fits(16)) return launch_generic<T, 16, EPI>(ctx, a);
  if (fits(8)) return launch_generic<T, 8, EPI>(ctx, a);
  if (sizeof(T) == 4 || fits(4)) return launch_generic<T, 4, EPI>(ctx, a);
  if constexpr (sizeof(T) == 2) return launch_generic<T, 2, EPI>(ctx, a);
  return fail(TSC_ERR_INVALID, "conv: misaligned feats / weight");
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
  if constexpr (sizeof(T) == 2) {
    // Narrow 16-bit rows: wave-level gather tiles (weights in LDS).
    if (a.Ci == 32 && a.Co == 32) return launch_narrow<T, 32, EPI>(ctx, a);
    if (a.Ci == 32 && a.Co == 64) return launch_narrow<T, 64, EPI>(ctx, a);
  } else {
    // fp32, Ci = Co = 32: the same wave tiles on v_mfma_f32_16x16x4f32 (the 32->64 weights do
    // not fit in LDS beside the neighbor slices).
    if (a.Ci == 32 && a.Co == 32) return launch_narrow<T, 32, EPI>(ctx, a);
  }
  if (a.Ci * (int)sizeof(T) <= 64) {
    // Other narrow input rows: one K chunk per tap -> register-staged double buffer.
    if (a.Co % 64 == 0) {
      if (kb == 64) return launch_reg<T, 128, 64, 64, 4, 1, EPI>(ctx, a);
      return launch_reg<T, 128, 64, 32, 4, 1, EPI>(ctx, a);
    }
    if (kb == 64) return launch_reg<T, 128, 32, 64, 4, 1, EPI>(ctx, a);
    return launch_reg<T, 128, 32, 32, 4, 1, EPI>(ctx, a);
  }
  // Ring path: chunks of at most 64 bytes, so that a ring of four stages plus the neighbor tile
  // fit in half of a CU's LDS (two resident blocks).  A 32-byte chunk stage is too small to
  // stage 32 epilogue rows of a 128-column half tile or a 64-column fp32 tile, so those shapes
  // take the next narrower tile.
  if constexpr (sizeof(T) < 4) {
    if (a.Co % 256 == 0 && kb >= 64) {
      // Widest channels: 256x256 tile, 2x4 waves of 128x64, one block per CU with a 4-stage
      // ring (128 flops per LDS/L2 byte, 0.75 fragment reads per MFMA).
      return launch_cfg<T, 256, 256, 64, 2, 4, EPI, 1>(ctx, a);
    }
    if (a.Co % 128 == 0 && kb >= 64) {
      // Wide channels: 128x128 tile, 2x2 waves of 64x64, two blocks per CU.
      return launch_cfg<T, 128, 128, 64, 2, 2, EPI>(ctx, a);
    }
    if (a.Co % 64 == 0) {
      // 128 rows x 64 cols, 4 waves of 32 rows.
      if (kb >= 64) return launch_cfg<T, 128, 64, 64, 4, 1, EPI>(ctx, a);
      return launch_cfg<T, 128, 64, 32, 4, 1, EPI>(ctx, a);
    }
  } else {
    // Small problems (fewer 128-row tiles than CUs, e.g. ~25k voxels): 64x64 tiles of four
    // 32x32 waves so every CU gets work.
    if (a.Co % 64 == 0 && kb >= 128 && ((a.N + 127) / 128) * (a.Co / 64) < 256)
      return launch_cfg<T, 64, 64, 128, 2, 2, EPI>(ctx, a);
    if (a.Co % 64 == 0 && kb >= 64) return launch_cfg<T, 128, 64, 64, 4, 1, EPI>(ctx, a);
  }
  // Co % 32 == 0
  if (kb >= 64) return launch_cfg<T, 128, 32, 64, 4, 1, EPI>(ctx, a);
  return launch_cfg<T, 128, 32, 32, 4, 1, EPI>(ctx, a);
}

// The ring configurations of dispatch_tiles whose column tile is the whole row (BN == Co), with
// the LayerNorm + SiLU epilogue; conv_fuses_ln admits exactly these shapes.
template <typename T>
int dispatch_ln(tsc_ctx* ctx, const ConvArgs& a) {
  if constexpr (sizeof(T) == 2) {
    const int kb = pick_kb(a.Ci * 2);
    if (a.Co == 256 && kb >= 64)
      return launch_cfg<T, 256, 256, 64, 2, 4, TSC_EPI_BIAS_LN_SILU, 1>(ctx, a);
    if (a.Co == 128 && kb >= 64) return launch_cfg<T, 128, 128, 64, 2, 2, TSC_EPI_BIAS_LN_SILU>(ctx, a);
    if (a.Co == 64) {
      if (kb >= 64) return launch_cfg<T, 128, 64, 64, 4, 1, TSC_EPI_BIAS_LN_SILU>(ctx, a);
      return launch_cfg<T, 128, 64, 32, 4, 1, TSC_EPI_BIAS_LN_SILU>(ctx, a);
    }
  }
  return fail(TSC_ERR_INVALID, "conv: no fused LayerNorm epilogue for Ci=%d Co=%d", a.Ci, a.Co);
}

template <typename T>
int dispatch_epi(tsc_ctx* ctx, const ConvArgs& a, bool tuned) {
  if (a.epilogue == TSC_EPI_BIAS_LN_SILU) return dispatch_ln<T>(ctx, a);
  if (a.epilogue == TSC_EPI_BIAS_RESIDUAL)
    return tuned ? dispatch_tiles<T, TSC_EPI_BIAS_RESIDUAL>(ctx, a)
                 : dispatch_generic<T, TSC_EPI_BIAS_RESIDUAL>(ctx, a);
  return tuned ? dispatch_tiles<T, TSC_EPI_BIAS>(ctx, a) : dispatch_generic<T, TSC_EPI_BIAS>(ctx, a);
}

}  // namespace

// Shapes and buffers the tuned kernels take: rows of a multiple of 32 bytes, Co a multiple of 32
// (whole MFMA column blocks), every buffer 16-byte aligned (16-byte row loads and stores).
bool conv_tuned_shape(const ConvArgs& a) {
  const int es = a.dtype == TSC_F32 ? 4 : 2;
  auto al16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  return (a.Ci * es) % 32 == 0 && a.Co % 32 == 0 && al16(a.feats) && al16(a.weight) &&
         al16(a.out) && (!a.bias || al16(a.bias)) &&
         (a.epilogue != TSC_EPI_BIAS_RESIDUAL || al16(a.residual));
}

bool conv_fuses_ln(const ConvArgs& a) {
  if (a.dtype == TSC_F32 || a.plan) return false;
  ConvArgs b = a;
  b.epilogue = TSC_EPI_BIAS;
  auto al16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  if (!conv_tuned_shape(b) || conv_gather_supported(b)) return false;
  if ((a.ln_gamma && !al16(a.ln_gamma)) || (a.ln_beta && !al16(a.ln_beta))) return false;
  // The ring path of dispatch_tiles (rows wider than 64 bytes, not the narrow kernels) with a
  // column tile equal to Co.
  if (a.Ci * 2 <= 64) return false;
  const int kb = pick_kb(a.Ci * 2);
  return (a.Co == 256 && kb >= 64) || (a.Co == 128 && kb >= 64) || a.Co == 64;
}

int conv_launch(tsc_ctx* ctx, const ConvArgs& a) {
  if (a.N == 0) return TSC_OK;
  const bool tuned = conv_tuned_shape(a);
  if (tuned && conv_gather_supported(a)) return conv_gather_launch(ctx, a);
  if (a.plan && !a.order) {  // other shapes: the plan's Morton row order
    ConvArgs b = a;
    b.order = (const int32_t*)((const char*)a.plan + plan_layout(a.N).rows);
    b.plan = nullptr;
    return conv_launch(ctx, b);
  }
  switch (a.dtype) {
    case TSC_F32: return dispatch_epi<float>(ctx, a, tuned);
    case TSC_F16: return dispatch_epi<_Float16>(ctx, a, tuned);
    case TSC_BF16: return dispatch_epi<__bf16>(ctx, a, tuned);
  }
  return fail(TSC_ERR_INVALID, "conv: unknown dtype %d", a.dtype);
}

}  // namespace tsc
