// Gather plan and the planned narrow conv (Ci = 32, 16-bit rows of 64 bytes).
//
// The direct narrow kernel gathers every (row, tap) neighbor row from global memory: ~9 gathers
// of 64 bytes per output row on a 1-voxel shell, most of them rows that other rows of the same
// tile gather too.  The plan removes that repetition:
//   * rows are processed in 64-row tiles in Morton (Z-curve) order of their coordinates, so a tile
//     is a compact patch of the surface;
//   * per tile, the distinct neighbor rows are listed once (~1.9 per output row instead of ~9 on
//     the 1-voxel 512^3 shell) and the conv gathers each of them once into the wave's LDS;
//   * a per-(row, tap) byte table gives the LDS slot of every neighbor (slot 0 = a zero row), so
//     the MFMA B fragments are read from LDS.
// The plan is built once per coordinate set (like the neighbor map it derives from) and reused
// by every narrow conv on that set.
//
// Plan buffer layout (all offsets 256-byte aligned, T = ceil(N/64) tiles):
//   rows   int32 [T*64]        row of each tile position in Morton order, -1 past N
//   count  int32 [T]           distinct neighbor rows of the tile (d <= 255), or -1 when the tile
//                              has more (it is then computed from the neighbor map directly)
//   rbm    uint32 [T*4]        taps present in any row of each 16-row block
//   list   int32 [T*256]       distinct rows of the tile, in slot order (slot s = list[s-1])
//   slots  uint8 [T][16][28][4] slot of (row 16*rb + i, tap v) at [i][v][rb]; 0 = absent
// Slot order: the tile's own rows first (row r -> slot r+1), then by first use in (tap, row)
// order, so the 16 rows of one (tap, row block) mostly sit in consecutive slots (distinct LDS
// banks for the fragment reads).

#include <climits>
#include <string>
#include <type_traits>

#include "tsc_internal.h"

namespace tsc {

PlanLayout plan_layout(int64_t N) {
  PlanLayout L;
  L.T = (N + kPlanRows - 1) / kPlanRows;
  size_t off = 0;
  L.rows = off;
  off = align_up(off + (size_t)L.T * kPlanRows * 4, 256);
  L.count = off;
  off = align_up(off + (size_t)L.T * 4, 256);
  L.rbm = off;
  off = align_up(off + (size_t)L.T * 16, 256);
  L.list = off;
  off = align_up(off + (size_t)L.T * kPlanSlots * 4, 256);
  L.slots = off;
  off = align_up(off + (size_t)L.T * kPlanTableBytes, 256);
  L.total = off;
  return L;
}

namespace {

typedef _Float16 f16x8_t __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x4_t __attribute__((__vector_size__(4 * sizeof(float))));

constexpr int kTaps = 27;
constexpr int kHash = 512;         // per-tile hash capacity (tiles past 255 rows overflow)
constexpr int kHashShift = 23;     // 32 - log2(kHash)
constexpr int kPrioWords = 56;     // 1792 priorities / 32
constexpr int kPlanWaves = 4;
constexpr int kTableQ = kPlanTableBytes / 16;  // 112 uint4 per tile table

// One wave per 64-row tile: distinct neighbor rows, their slots, the slot table and tap masks.
// sorted_rows and rows_out may be the same buffer (the launcher sorts in place): each lane reads
// its own entry before writing it, so neither is declared __restrict__.
__global__ void __launch_bounds__(64 * kPlanWaves)
    plan_tile_kernel(const int32_t* sorted_rows, const int32_t* __restrict__ nbr,
                     int64_t N, int64_t T, int32_t* rows_out,
                     int32_t* __restrict__ count_out, uint32_t* __restrict__ rbm_out,
                     int32_t* __restrict__ list_out, uint4* __restrict__ slots_out) {
  __shared__ __attribute__((aligned(16))) int32_t hkey[kPlanWaves][kHash];
  __shared__ __attribute__((aligned(16))) int32_t hval[kPlanWaves][kHash];  // min prio, then slot
  __shared__ uint32_t pbits[kPlanWaves][kPrioWords];
  __shared__ int32_t ppre[kPlanWaves][64];
  __shared__ uint4 table[kPlanWaves][kTableQ];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * kPlanWaves + w;
  if (t >= T) return;  // whole wave
  int32_t* const hk = hkey[w];
  int32_t* const hv = hval[w];
  for (int i = lane; i < kHash / 4; i += 64) {  // 16-byte stores
    ((int4*)hk)[i] = make_int4(-1, -1, -1, -1);
    ((int4*)hv)[i] = make_int4(INT_MAX, INT_MAX, INT_MAX, INT_MAX);
  }
  if (lane < kPrioWords) pbits[w][lane] = 0u;
  for (int i = lane; i < kTableQ; i += 64) table[w][i] = make_uint4(0, 0, 0, 0);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

  const int64_t pos = t * kPlanRows + lane;
  const int32_t row = pos < N ? sorted_rows[pos] : -1;
  rows_out[pos] = row;
  // Insert every present neighbor with priority: own row (tap 13) = its position in the tile,
  // else 64 + 64*tap + position.  Linear probing; an insert that finds the table full marks the
  // tile as overflowing (it has more distinct rows than a list holds anyway).
  // All 27 entries are loaded before the first insert, so the loads overlap.
  int32_t ev[kTaps];
#pragma unroll
  for (int v = 0; v < kTaps; ++v) ev[v] = row >= 0 ? nbr[(int64_t)row * kTaps + v] : -1;
  int hpos[kTaps];
  uint32_t present = 0;
  bool full = false;
#pragma unroll
  for (int v = 0; v < kTaps; ++v) {
    const int32_t e = ev[v];
    hpos[v] = -1;
    if (e >= 0) {
      present |= 1u << v;
      const int prio = v == 13 ? lane : 64 + 64 * v + lane;
      int h = (int)(((uint32_t)e * 2654435761u) >> kHashShift);
      bool ok = false;
      for (int probe = 0; probe < kHash; ++probe) {
        const int32_t old = atomicCAS(&hk[h], -1, e);
        if (old == -1 || old == e) {
          ok = true;
          break;
        }
        h = (h + 1) & (kHash - 1);
      }
      if (ok) {
        atomicMin(&hv[h], prio);
        hpos[v] = h;
      } else {
        full = true;
      }
    }
  }
  const bool overflow = __ballot(full) != 0;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  // Distinct count and the set of their (distinct) minimum priorities.
  int cnt = 0;
  for (int i = lane; i < kHash / 4; i += 64) {
    const int4 k4 = ((const int4*)hk)[i];
    const int4 v4 = ((const int4*)hv)[i];
    const int kk[4] = {k4.x, k4.y, k4.z, k4.w}, vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (kk[u] >= 0) {
        ++cnt;
        atomicOr(&pbits[w][vv[u] >> 5], 1u << (vv[u] & 31));
      }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off, 64);
  // Per-16-row tap masks.
  uint32_t m = present;
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) m |= __shfl_xor(m, off, 64);
  if ((lane & 15) == 0) rbm_out[t * 4 + (lane >> 4)] = m;
  if (overflow || cnt > kPlanSlots - 1) {
    if (lane == 0) count_out[t] = -1;
    return;
  }
  if (lane == 0) count_out[t] = cnt;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  // Exclusive prefix of the priority-bit popcounts (56 words, one per lane).
  const int pc = lane < kPrioWords ? __popc(pbits[w][lane]) : 0;
  int incl = pc;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  ppre[w][lane] = incl - pc;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  // Slot = 1 + rank of the row's minimum priority.
  int32_t* const list = list_out + t * kPlanSlots;
  for (int i = lane; i < kHash / 4; i += 64) {
    const int4 k4 = ((const int4*)hk)[i];
    int4 v4 = ((const int4*)hv)[i];
    int* const vv = (int*)&v4;
    const int kk[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (kk[u] >= 0) {
        const int p = vv[u];
        const int rank = ppre[w][p >> 5] + __popc(pbits[w][p >> 5] & ((1u << (p & 31)) - 1u));
        list[rank] = kk[u];
        vv[u] = rank + 1;
      }
    ((int4*)hv)[i] = v4;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  uint8_t* const tb = (uint8_t*)table[w];
  const int i16 = lane & 15, rb = lane >> 4;
#pragma unroll
  for (int v = 0; v < kTaps; ++v)
    if (hpos[v] >= 0) tb[(i16 * 28 + v) * 4 + rb] = (uint8_t)hv[hpos[v]];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  for (int i = lane; i < kTableQ; i += 64) slots_out[t * kTableQ + i] = table[w][i];
}

// ---- planned narrow conv -----------------------------------------------------------------------

template <typename T>
__device__ __forceinline__ void mfma16(const uint4& a, const uint4& b, f32x4_t& acc);
template <>
__device__ __forceinline__ void mfma16<_Float16>(const uint4& a, const uint4& b, f32x4_t& acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                               __builtin_bit_cast(f16x8_t, b), acc, 0, 0, 0);
}
template <>
__device__ __forceinline__ void mfma16<__bf16>(const uint4& a, const uint4& b, f32x4_t& acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), acc, 0, 0, 0);
}

constexpr int kGWaves = 7;   // waves per block (one block per CU: LDS-bound)
constexpr int kGStage = 208;  // LDS row slots per wave (slot 0 = zeros); tiles need d < 208
constexpr int kGChunks = kGStage / 16;

// Wave-level tile loop, one block per CU, blocks split between column halves for Co = 64
// (both halves of a tile run on one XCD, so the second gather of a row hits its L2).
//   stage   the tile's distinct rows -> LDS slots (row s at s*64, 16-byte piece p at
//           p ^ ((s >> 1) & 3): eight rows of consecutive slots read by one ds_read_b128 step
//           cover all 32 banks), its slot table -> LDS
//   MFMA    D[co][row] = W[co][k] * F[row][k] per (tap, 16-row block), v_mfma_f32_16x16x32,
//           A = weights from LDS (staged once per block), B = slot rows from LDS; taps in a
//           two-deep pipeline (fragments of tap k+1 in flight during the MFMAs of tap k)
//   overlap while tile t computes, tile t+1's rows and slot table are in flight and tile t+2's
//           list indices are loaded
// Tiles whose distinct rows exceed the staging (count -1 or >= kGStage) read their B fragments
// from global memory through the neighbor map instead.
template <typename T, int EPI>
__global__ void __launch_bounds__(64 * kGWaves)
    conv_gather_kernel(const T* __restrict__ feats, const T* __restrict__ weight,
                       const T* __restrict__ bias, const int32_t* __restrict__ nbr,
                       const int32_t* __restrict__ prow, const int32_t* __restrict__ pcount,
                       const uint32_t* __restrict__ prbm, const int32_t* __restrict__ plist,
                       const uint4* __restrict__ pslots, int64_t N, int32_t n_tiles,
                       int32_t tiles_per_xcd, int32_t co_total, int32_t halves,
                       const T* residual, T* out) {
  __shared__ uint4 sW[kTaps * 32 * 4];
  __shared__ uint4 sStage[kGWaves][kGStage * 4];
  __shared__ uint4 sTbl[kGWaves][kTableQ];
  __shared__ int32_t sTaken;  // tiles of the block's range handed out so far
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int l16 = lane & 15, q = lane >> 4;
  const int j = lane >> 2, p = lane & 3;
  const int xcd = blockIdx.x & 7;
  const int local = blockIdx.x >> 3;
  const int half = halves == 2 ? (local & 1) : 0;
  const int slot_in_half = halves == 2 ? (local >> 1) : local;
  const int blocks_in_half = (int)(gridDim.x >> 3) / halves;
  const int co0 = 32 * half;
  if (tid == 0) sTaken = 0;

  // Weights (Co,27,32) of this column half: row co, piece p -> [(v*32 + co)*4 + (p ^ ((co>>1)&3))].
  const uint4* wq = (const uint4*)weight;
  for (int g = tid; g < 32 * kTaps * 4; g += 64 * kGWaves) {
    const int pp = g & 3, v = (g >> 2) % kTaps, co = g / (kTaps * 4);
    sW[(v * 32 + co) * 4 + (pp ^ ((co >> 1) & 3))] = wq[((co0 + co) * kTaps + v) * 4 + pp];
  }
  if (lane < 4) sStage[wid][lane] = make_uint4(0, 0, 0, 0);
  float bv[2][4];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      bv[cb][i] = bias ? (float)bias[co0 + cb * 16 + 4 * q + i] : 0.f;
  __syncthreads();
  uint4* const st = sStage[wid];
  uint4* const tb = sTbl[wid];

  // Tiles are dealt at run time inside a block: the block owns a contiguous run of its XCD's tiles
  // (adjacent Morton tiles, so its gathers share L2 lines) and each wave takes the next tile of the
  // run from an LDS counter, so waves that drew short tiles take more and the block ends when its
  // work does, not when the wave with the longest fixed share does.  The counter read for the
  // tile after next is issued one tile ahead.  (A global counter per XCD measured 3x slower:
  // atomics on one address serialize.)
  const int xt_begin = xcd * tiles_per_xcd;
  const int xt_count = max(0, min(n_tiles, xt_begin + tiles_per_xcd) - xt_begin);
  const int per_block = (xt_count + blocks_in_half - 1) / blocks_in_half;
  const int t_begin = xt_begin + min(xt_count, slot_in_half * per_block);
  const int t_end = xt_begin + min(xt_count, (slot_in_half + 1) * per_block);
  // The counter's address goes through a zero the compiler cannot see through: with a uniform
  // address its atomic optimizer broadcasts the result at once (readfirstlane and a wait for
  // every LDS operation in flight).
  auto take_async = [&]() {  // counter value in lane 0, not yet waited for
    int32_t z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    int32_t v = 0;
    if (lane == 0) v = atomicAdd(&sTaken + z, 1);
    return v;
  };
  auto tile_of = [&](int32_t pending) { return t_begin + __builtin_amdgcn_readfirstlane(pending); };
  const int first = tile_of(take_async());
  if (first < t_end) {

  // Prefetch of a tile is straight-line code: per-lane loads whose addresses are clamped (never
  // skipped), so the compiler can count them exactly.  Loads under per-chunk branches made it
  // wait for every outstanding load before each dependent one (one vmcnt counts all loads in
  // order), which serialised a tile's ~20 index and row loads into one round trip each.
  //   meta  one load: lanes 0-3 the tile's four 16-row tap masks, lane 4 its distinct-row count
  //   idx   the list entries of slots 16c + j (always inside the tile's kPlanSlots entries)
  //   rows  row idx[c] piece p for slots below the count, else row 0 (valid, never staged)
  auto load_meta = [&](int t) {
    return lane < 4 ? (int32_t)prbm[t * 4 + lane] : pcount[t];
  };
  auto meta_count = [&](int32_t meta) {
    const int dd = __builtin_amdgcn_readlane(meta, 4);
    return dd < kGStage ? dd : -1;  // -1: not staged
  };
  typedef uint32_t xvec_t __attribute__((ext_vector_type(4 * kGChunks)));
  int32_t idx[kGChunks];
  xvec_t x = {};
  auto chunk_mask = [](int d) {
    return d > 0 ? __builtin_amdgcn_readfirstlane((1u << ((d + 15) >> 4)) - 1u) : 0u;
  };
  auto load_idx = [&](int t) {
    const int32_t* list = plist + (int64_t)t * kPlanSlots;
#pragma unroll
    for (int c = 0; c < kGChunks; ++c) idx[c] = list[16 * c + j];
  };
  auto gather = [&](int d) {
#pragma unroll
    for (int c = 0; c < kGChunks; ++c) {
      const int32_t r = idx[c];
      const bool ok = 16 * c + j < d && r >= 0 && r < N;
      const uint4 vv = ((const uint4*)(feats + (int64_t)(ok ? r : 0) * 32))[p];
      x[4 * c] = vv.x;
      x[4 * c + 1] = vv.y;
      x[4 * c + 2] = vv.z;
      x[4 * c + 3] = vv.w;
    }
  };
  auto load_tbl = [&](int t, uint4& ta, uint4& tb2) {
    const uint4* tq = pslots + (int64_t)t * kTableQ;
    ta = tq[lane];
    tb2 = tq[64 + (lane < kTableQ - 64 ? lane : 0)];
  };

  // Prologue: the first tile's rows gathered and its table loaded; the next tile's metadata and
  // indices.  A missing next tile repeats the current one (its loads stay in bounds, unused).
  int cur = first;
  int32_t meta = load_meta(cur);
  load_idx(cur);
  int d = meta_count(meta);
  uint32_t m[4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) m[rb] = (uint32_t)__builtin_amdgcn_readlane(meta, rb);
  gather(d);
  uint4 ta, tb2;
  load_tbl(cur, ta, tb2);
  int32_t row_n = prow[(int64_t)cur * kPlanRows + lane];
  int next = tile_of(take_async());
  int32_t pend = take_async();
  int nx = next < t_end ? next : cur;
  int32_t meta_n = load_meta(nx);
  load_idx(nx);

  for (;;) {
    // Stage tile `cur`: rows and slot table into the wave's LDS.
    __builtin_amdgcn_wave_barrier();
    const uint32_t cm = chunk_mask(d);
#pragma unroll
    for (int c = 0; c < kGChunks; ++c)
      if ((cm >> c) & 1u) {
        const int s = 1 + 16 * c + j;
        if (s < kGStage)
          st[s * 4 + (p ^ ((s >> 1) & 3))] = make_uint4(x[4 * c], x[4 * c + 1], x[4 * c + 2],
                                                        x[4 * c + 3]);
      }
    tb[lane] = ta;
    if (lane < kTableQ - 64) tb[64 + lane] = tb2;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t mc[4] = {m[0], m[1], m[2], m[3]};
    const bool staged = d >= 0;
    int32_t row_c = row_n < N ? row_n : -1;
    // Tile `next` (or `cur` again at the end): rows, table and row list go out now; the tile
    // after it gets its metadata and indices.
    const bool has_next = next < t_end;
    d = meta_count(meta_n);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) m[rb] = (uint32_t)__builtin_amdgcn_readlane(meta_n, rb);
    gather(d);
    load_tbl(nx, ta, tb2);
    row_n = prow[(int64_t)nx * kPlanRows + lane];
    const int nn = tile_of(pend);
    pend = take_async();
    const int nnx = nn < t_end ? nn : nx;
    meta_n = load_meta(nnx);
    load_idx(nnx);
    f32x4_t acc[4][2];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) acc[rb][cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const uint32_t tm = mc[0] | mc[1] | mc[2] | mc[3];
    auto rd_a = [&](int v, uint4 (&a)[2]) {
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const int co = 16 * cb + l16;
        a[cb] = sW[(v * 32 + co) * 4 + (q ^ ((co >> 1) & 3))];
      }
    };
    auto mm = [&](const uint4 (&b)[4], const uint4 (&a)[2]) {
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) mfma16<T>(a[cb], b[rb], acc[rb][cb]);
    };
    if (staged && tm) {
      // Every 16-row block of a used tap (absent rows read the zero slot).
      const uint32_t* tb32 = (const uint32_t*)tb + l16 * 28;
      auto rd = [&](int v, uint4 (&b)[4], uint4 (&a)[2]) {
        const uint32_t s4 = tb32[v];
        rd_a(v, a);
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
          const int s = (s4 >> (8 * rb)) & 0xff;
          b[rb] = st[s * 4 + (q ^ ((s >> 1) & 3))];
        }
      };
      uint32_t rem = tm;
      uint4 bA[4], aA[2], bB[4], aB[2];
      rd(__builtin_ctz(rem), bA, aA);
      rem &= rem - 1u;
      for (;;) {
        const bool hb = rem != 0;
        if (hb) rd(__builtin_ctz(rem), bB, aB);
        rem &= rem - 1u;
        mm(bA, aA);
        if (!hb) break;
        const bool ha = rem != 0;
        if (ha) rd(__builtin_ctz(rem), bA, aA);
        rem &= rem - 1u;
        mm(bB, aB);
        if (!ha) break;
      }
    } else if (tm) {
      // Tile with too many distinct rows: fragments straight from the neighbor map.
      uint32_t rem = tm;
      while (rem) {
        const int v = __builtin_ctz(rem);
        rem &= rem - 1u;
        uint4 a[2], b[4];
        rd_a(v, a);
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
          const int32_t r = __shfl(row_c, rb * 16 + l16, 64);
          const int32_t e = r >= 0 ? nbr[(int64_t)r * kTaps + v] : -1;
          const bool ok = e >= 0 && e < N;
          const uint4 bv4 = ((const uint4*)(feats + (int64_t)(ok ? e : 0) * 32))[q];
          b[rb] = ok ? bv4 : make_uint4(0u, 0u, 0u, 0u);
        }
        mm(b, a);
      }
    }

    // Epilogue: lane (l16, q) owns row 16*rb + l16, columns co0 + 16*cb + 4q .. +3.  Residual
    // values are all loaded before the first store (rows past N read row 0, not stored); each
    // element is read and written by the same lane, so the output may alias the residual.
    struct alignas(4 * sizeof(T)) V4 {
      T v[4];
    };
    int32_t rows[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) rows[rb] = __shfl(row_c, rb * 16 + l16, 64);
    V4 rt[4][2];
    if (EPI == TSC_EPI_BIAS_RESIDUAL) {
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
          rt[rb][cb] = *(const V4*)(residual + (int64_t)(rows[rb] >= 0 ? rows[rb] : 0) * co_total +
                                    co0 + cb * 16 + 4 * q);
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const int32_t row = rows[rb];
      if (row < 0) continue;
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const int c = co0 + cb * 16 + 4 * q;
        float xv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) xv[i] = acc[rb][cb][i] + bv[cb][i];
        if (EPI == TSC_EPI_BIAS_RESIDUAL) {
#pragma unroll
          for (int i = 0; i < 4; ++i) xv[i] += (float)rt[rb][cb].v[i];
        }
        V4 y;
#pragma unroll
        for (int i = 0; i < 4; ++i) y.v[i] = (T)xv[i];
        *(V4*)(out + (int64_t)row * co_total + c) = y;
      }
    }
    if (!has_next) break;
    cur = next;
    next = nn;
    nx = nnx;
  }
  }  // first < t_end
}

template <typename T, int EPI>
int launch_gather(tsc_ctx* ctx, const ConvArgs& a) {
  const PlanLayout L = plan_layout(a.N);
  const char* base = (const char*)a.plan;
  const int32_t n_tiles = (int32_t)L.T;
  const int32_t tpx = (n_tiles + 7) / 8;
  const int32_t halves = a.Co / 32;
  static const std::string name = std::string("conv_gather_kernel<") +
      (std::is_same<T, __bf16>::value ? "bf16" : "f16") +
      (EPI == TSC_EPI_BIAS_RESIDUAL ? ",res>" : ">");
  ProfScope ps(ctx, name.c_str());
  conv_gather_kernel<T, EPI><<<256, 64 * kGWaves, 0, ctx->stream>>>(
      (const T*)a.feats, (const T*)a.weight, (const T*)a.bias, a.nbr,
      (const int32_t*)(base + L.rows), (const int32_t*)(base + L.count),
      (const uint32_t*)(base + L.rbm), (const int32_t*)(base + L.list),
      (const uint4*)(base + L.slots), a.N, n_tiles, tpx, a.Co, halves, (const T*)a.residual,
      (T*)a.out);
  return check_hip(hipGetLastError(), "conv launch");
}

}  // namespace

bool conv_gather_supported(const ConvArgs& a) {
  auto al8 = [](const void* q) { return ((uintptr_t)q & 7) == 0; };
  return a.plan && a.Ci == 32 && (a.Co == 32 || a.Co == 64) &&
         (a.dtype == TSC_F16 || a.dtype == TSC_BF16) && a.N > 0 && a.N <= INT32_MAX - 64 &&
         al8(a.out) && (a.epilogue != TSC_EPI_BIAS_RESIDUAL || al8(a.residual));
}

int conv_gather_launch(tsc_ctx* ctx, const ConvArgs& a) {
  const bool res = a.epilogue == TSC_EPI_BIAS_RESIDUAL;
  if (a.dtype == TSC_F16)
    return res ? launch_gather<_Float16, TSC_EPI_BIAS_RESIDUAL>(ctx, a)
               : launch_gather<_Float16, TSC_EPI_BIAS>(ctx, a);
  return res ? launch_gather<__bf16, TSC_EPI_BIAS_RESIDUAL>(ctx, a)
             : launch_gather<__bf16, TSC_EPI_BIAS>(ctx, a);
}

int gather_plan_launch(tsc_ctx* ctx, const int32_t* coords, const int32_t* nbr, int64_t N,
                       int32_t B, int32_t X, int32_t Y, int32_t Z, void* plan) {
  if (N == 0) return TSC_OK;
  const PlanLayout L = plan_layout(N);
  auto bitlen = [](int64_t v) {
    int b = 0;
    while (b < 63 && (v >> b) != 0) ++b;
    return b;
  };
  // Coordinate bits above 21 are left out of the curve (the order stays a permutation).
  const int bits = std::min(21, bitlen(std::max(X, std::max(Y, Z)) - 1));
  const int total = 3 * bits + bitlen((int64_t)B - 1);
  // Keys wider than 64 bits drop their lowest Morton bits: a coarser curve, still a permutation.
  const int shift = total > 64 ? total - 64 : 0;
  const int nbits = std::max(1, std::min(64, total));
  char* base = (char*)plan;
  int32_t* rows = (int32_t*)(base + L.rows);
  ProfScope ps(ctx, "gather_plan");
  const int st = sort_rows_morton(ctx, coords, N, bits, shift, nbits, rows);
  if (st) return st;
  const unsigned blocks = (unsigned)((L.T + kPlanWaves - 1) / kPlanWaves);
  plan_tile_kernel<<<blocks, 64 * kPlanWaves, 0, ctx->stream>>>(
      rows, nbr, N, L.T, rows, (int32_t*)(base + L.count), (uint32_t*)(base + L.rbm),
      (int32_t*)(base + L.list), (uint4*)(base + L.slots));
  return check_hip(hipGetLastError(), "gather plan tiles");
}

}  // namespace tsc
