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
//                              has more (it is then computed from the neighbor map directly);
//                              a split tile (below) stores d | sA << 8 | aonly << 16 | 1 << 30
//   rbm    uint32 [T*4]        taps present in any row of each 16-row block
//   list   int32 [T*256]       distinct rows of the tile, in slot order (slot s = list[s-1])
//   slots  uint8 [T][16][28][4] slot of (row 16*rb + i, tap v) at [i][v][rb]; 0 = absent
// Slot order: the tile's own rows first (row r -> slot r+1), then by first use in (tap, row)
// order, so the 16 rows of one (tap, row block) mostly sit in consecutive slots (distinct LDS
// banks for the fragment reads).
// Split tiles: a tile with more distinct rows than the conv's staging holds (d >= kPlanStage),
// but whose two 32-row halves each need fewer (sA, sB < kPlanStage; a 4x4x4 block of a solid:
// 216 rows, 144 per half), orders its rows as (rows only the first half uses, rows both use,
// rows only the second half uses), each group in the order above.  The first half's rows are
// then slots 1..sA and the second half's slots aonly+1..d (aonly = rows of the first group);
// the second half's table entries are stored minus aonly, so each half stages its own rows
// at 1.. and the conv computes the tile as two passes of 32 rows.

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
constexpr int kOrderWords = 3 * kPrioWords;  // split tiles: (group, priority) sort keys
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
  __shared__ uint32_t pbits[kPlanWaves][kOrderWords];
  __shared__ int32_t ppre[kPlanWaves][kOrderWords];
  __shared__ uint32_t hgrp[kPlanWaves][kHash / 16];  // 2 bits per hash entry: halves using it
  __shared__ int32_t hdum[kPlanWaves][64];            // per-lane target of absent taps' atomics
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
  for (int i = lane; i < kOrderWords; i += 64) pbits[w][i] = 0u;
  if (lane < kHash / 16) hgrp[w][lane] = 0u;
  hdum[w][lane] = -2;
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
  // All 27 entries are loaded before the first insert, so the loads overlap, and unconditionally
  // (rows past N read row 0's, then -1): loads each under a `row >= 0` test ran 3x slower.
  int32_t ev[kTaps];
  const int32_t* nr = nbr + (int64_t)(row >= 0 ? row : 0) * kTaps;
#pragma unroll
  for (int v = 0; v < kTaps; ++v) ev[v] = nr[v];
#pragma unroll
  for (int v = 0; v < kTaps; ++v) ev[v] = row >= 0 ? ev[v] : -1;
  // Hash inserts: every present tap's CAS at its home slot is issued before the first result is
  // used (absent taps aim at the lane's own dummy word, which never holds -1), then the few that
  // met another key probe on one by one; the priorities likewise go out in one batch.
  int hpos[kTaps];
  uint32_t present = 0;
  bool full = false;
  int32_t old[kTaps];
#pragma unroll
  for (int v = 0; v < kTaps; ++v) {
    hpos[v] = (int)(((uint32_t)ev[v] * 2654435761u) >> kHashShift);
    if (ev[v] >= 0) present |= 1u << v;
  }
#pragma unroll
  for (int v = 0; v < kTaps; ++v)
    old[v] = atomicCAS(ev[v] >= 0 ? &hk[hpos[v]] : &hdum[w][lane], -1, ev[v]);
#pragma unroll
  for (int v = 0; v < kTaps; ++v) {
    if (ev[v] >= 0 && old[v] != -1 && old[v] != ev[v]) {
      int h = hpos[v];
      bool ok = false;
      for (int probe = 1; probe < kHash; ++probe) {
        h = (h + 1) & (kHash - 1);
        const int32_t o = atomicCAS(&hk[h], -1, ev[v]);
        if (o == -1 || o == ev[v]) {
          ok = true;
          break;
        }
      }
      hpos[v] = ok ? h : -1;
      full = full || !ok;
    }
    if (ev[v] < 0) hpos[v] = -1;
  }
#pragma unroll
  for (int v = 0; v < kTaps; ++v)
    atomicMin(hpos[v] >= 0 ? &hv[hpos[v]] : &hdum[w][lane], v == 13 ? lane : 64 + 64 * v + lane);
  const bool overflow = __ballot(full) != 0;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  // Distinct count; for a tile over the staging also the rows each half uses (split decision).
  int cnt = 0;
  for (int i = lane; i < kHash / 4; i += 64) {
    const int4 k4 = ((const int4*)hk)[i];
    cnt += (k4.x >= 0) + (k4.y >= 0) + (k4.z >= 0) + (k4.w >= 0);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off, 64);
  int ca = 0, cb = 0;
  if (cnt >= kPlanStage && cnt <= kPlanSlots - 1 && !overflow) {  // wave-uniform
#pragma unroll
    for (int v = 0; v < kTaps; ++v)
      if (hpos[v] >= 0) atomicOr(&hgrp[w][hpos[v] >> 4], (lane < 32 ? 1u : 2u) << (2 * (hpos[v] & 15)));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    for (int i = lane; i < kHash; i += 64) {
      if (hk[i] >= 0) {
        const uint32_t g = (hgrp[w][i >> 4] >> (2 * (i & 15))) & 3u;
        ca += g & 1u;
        cb += g >> 1;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      ca += __shfl_xor(ca, off, 64);
      cb += __shfl_xor(cb, off, 64);
    }
  }
  // Per-16-row tap masks.
  uint32_t m = present;
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) m |= __shfl_xor(m, off, 64);
  if ((lane & 15) == 0) rbm_out[t * 4 + (lane >> 4)] = m;
  if (overflow || cnt > kPlanSlots - 1) {
    if (lane == 0) count_out[t] = -1;
    return;
  }
  const bool split = cnt >= kPlanStage && ca < kPlanStage && cb < kPlanStage;
  const int aonly = cnt - cb;  // rows only the first half uses
  if (lane == 0)
    count_out[t] = split ? (cnt | ca << 8 | aonly << 16 | 1 << 30) : cnt;
  // Sort key of every distinct row: its minimum priority, for split tiles offset by its group.
  for (int i = lane; i < kHash / 4; i += 64) {
    const int4 k4 = ((const int4*)hk)[i];
    const int4 v4 = ((const int4*)hv)[i];
    const int kk[4] = {k4.x, k4.y, k4.z, k4.w}, vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (kk[u] >= 0) {
        const int h = 4 * i + u;
        const uint32_t g = (hgrp[w][h >> 4] >> (2 * (h & 15))) & 3u;
        const int key = vv[u] + (split ? (g == 1u ? 0 : g == 3u ? 1 : 2) * kPrioWords * 32 : 0);
        atomicOr(&pbits[w][key >> 5], 1u << (key & 31));
      }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  // Exclusive prefix of the key-bit popcounts (168 words, three consecutive ones per lane).
  int pc[3], loc = 0;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    pc[k] = lane < kPrioWords ? __popc(pbits[w][3 * lane + k]) : 0;
    loc += pc[k];
  }
  int incl = loc;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  if (lane < kPrioWords) {
    int base = incl - loc;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      ppre[w][3 * lane + k] = base;
      base += pc[k];
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  // Slot = 1 + rank of the row's sort key.
  int32_t* const list = list_out + t * kPlanSlots;
  for (int i = lane; i < kHash / 4; i += 64) {
    const int4 k4 = ((const int4*)hk)[i];
    int4 v4 = ((const int4*)hv)[i];
    int* const vv = (int*)&v4;
    const int kk[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (kk[u] >= 0) {
        const int h = 4 * i + u;
        const uint32_t g = (hgrp[w][h >> 4] >> (2 * (h & 15))) & 3u;
        const int p = vv[u] + (split ? (g == 1u ? 0 : g == 3u ? 1 : 2) * kPrioWords * 32 : 0);
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
  const int slot_base = split && lane >= 32 ? aonly : 0;  // second half of a split tile
#pragma unroll
  for (int v = 0; v < kTaps; ++v)
    if (hpos[v] >= 0) tb[(i16 * 28 + v) * 4 + rb] = (uint8_t)(hv[hpos[v]] - slot_base);
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
constexpr int kGStage = kPlanStage;  // LDS row slots per wave (slot 0 = zeros)
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
// Split tiles (the plan's count says which) run as two units of the same pipeline, one per
// 32-row half: the first stages slots 1..sA, the second the list from entry aonly on, with the
// other half's table bytes masked to slot 0 (its rows add zero products, as absent taps do) and
// the taps of the half's row blocks.  Each row still sums its taps in tap order, so the result
// is the same bits as a one-pass tile.  Tiles whose distinct rows exceed the staging otherwise
// (count -1, or >= kGStage without a split) read their B fragments from global memory through
// the neighbor map instead.
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
  // The lane's 16-byte store in an output row: columns co0 + 16*(q & 1) + 8*(q >> 1) .. +7
  // (the epilogue's column exchange), rows reached by one 32 x 32 -> 64-bit multiply-add.
  const uint32_t row_bytes = (uint32_t)co_total * (uint32_t)sizeof(T);
  T* const out_lane = out + co0 + 16 * (q & 1) + 8 * (q >> 1);
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
  //   idx   the list entries of slots off + 16c + j (unclamped, see load_idx)
  //   rows  row idx[c] piece p for slots below the count, else row 0 (valid, never staged)
  auto load_meta = [&](int t) {
    return lane < 4 ? (int32_t)prbm[t * 4 + lane] : pcount[t];
  };
  // A unit of work: a whole tile, or one half of a split tile (second = the second half).
  struct Unit {
    int g;           // rows to stage (-1: the tile reads through the neighbor map)
    uint32_t pmask;  // table bytes (row blocks) of this unit
    uint32_t taps;   // taps any of its row blocks uses
    bool first;      // first half of a split tile: the second half follows, no epilogue yet
    bool second;     // second half: accumulators carried over from the first
  };
  auto decode = [&](int32_t meta, bool second) {
    const int dd = __builtin_amdgcn_readlane(meta, 4);
    uint32_t mk[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) mk[rb] = (uint32_t)__builtin_amdgcn_readlane(meta, rb);
    Unit u{dd >= 0 && dd < kGStage ? dd : -1, 0xffffffffu, mk[0] | mk[1] | mk[2] | mk[3], false,
           false};
    if (dd >= 0 && (dd & (1 << 30))) {
      if (!second) {
        u = Unit{(dd >> 8) & 0xff, 0x0000ffffu, mk[0] | mk[1], true, false};
      } else {
        u = Unit{(dd & 0xff) - ((dd >> 16) & 0xff), 0xffff0000u, mk[2] | mk[3], false, true};
      }
    }
    return u;
  };
  auto second_offset = [&](int32_t meta) {  // list entry of the second half's first slot
    return (__builtin_amdgcn_readlane(meta, 4) >> 16) & 0xff;
  };
  typedef uint32_t xvec_t __attribute__((ext_vector_type(4 * kGChunks)));
  int32_t idx[kGChunks];
  xvec_t x = {};
  auto chunk_mask = [](int d) {
    return d > 0 ? __builtin_amdgcn_readfirstlane((1u << ((d + 15) >> 4)) - 1u) : 0u;
  };
  // Entries off + 16c + j at immediate offsets, unclamped: gather() uses only those below the
  // unit's count (all inside the tile's list); the others may read the next tile's list or, for
  // the last tile, the slot tables that follow the lists in the plan buffer (off <= 255, so at
  // most 16 * kGChunks - 1 entries past its end).
  static_assert((16 * kGChunks - 1) * 4 <= kPlanTableBytes, "reads past the last list stay in the plan");
  auto load_idx = [&](int t, int off) {
    const int32_t* list = plist + (int64_t)t * kPlanSlots + off + j;
#pragma unroll
    for (int c = 0; c < kGChunks; ++c) idx[c] = list[16 * c];
  };
  // Rows are 64 bytes and N < 2^31 here, so one unsigned compare covers 0 <= r < N; the row is
  // selected as 32 bits before the 64-bit address (left to itself the compiler selected both
  // halves of the shifted address: 8 instead of 5 VALU instructions per chunk).
  const uint32_t n32 = (uint32_t)N;
  const char* const fpiece = (const char*)feats + 16 * p;
  auto gather = [&](int d) {
#pragma unroll
    for (int c = 0; c < kGChunks; ++c) {
      const int32_t r = idx[c];
      uint32_t rr = (uint32_t)r < n32 && 16 * c + j < d ? (uint32_t)r : 0u;
      asm("" : "+v"(rr));
      const uint4 vv = *(const uint4*)(fpiece + (uint64_t)rr * 64u);
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

  // Prologue: the first unit's rows gathered and its table loaded; the next unit's metadata and
  // indices.  A missing next tile repeats the current one (its loads stay in bounds, unused).
  // `pend` always holds the counter take for the next new tile; the second half of a split tile
  // follows its first half without one.
  int cur = first;
  int32_t meta = load_meta(cur);
  load_idx(cur, 0);
  Unit uc = decode(meta, false);
  gather(uc.g);
  uint4 ta, tb2;
  load_tbl(cur, ta, tb2);
  // Rows of the four 16-row blocks as the epilogue needs them (row 16*rb + l16 in lane (l16, q)),
  // loaded with the tile's other prefetches rather than broadcast through LDS afterwards.
  auto load_rows = [&](int t, int32_t (&r4)[4]) {
    const int32_t* pr = prow + (int64_t)t * kPlanRows + l16;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) r4[rb] = pr[16 * rb];
  };
  int32_t rows_n[4];
  load_rows(cur, rows_n);
  int32_t pend = take_async();
  int next;
  bool next_second = uc.first;
  if (next_second) {
    next = cur;
  } else {
    next = tile_of(pend);
    pend = take_async();
  }
  int nx = next < t_end ? next : cur;
  int32_t meta_n = load_meta(nx);
  load_idx(nx, next_second ? second_offset(meta) : 0);
  f32x4_t acc[4][2];

  for (;;) {
    // Stage tile `cur`: rows and slot table into the wave's LDS.
    __builtin_amdgcn_wave_barrier();
    const uint32_t cm = chunk_mask(uc.g);
#pragma unroll
    for (int c = 0; c < kGChunks; ++c)
      if ((cm >> c) & 1u) {
        const int s = 1 + 16 * c + j;
        if (s < kGStage)
          st[s * 4 + (p ^ ((s >> 1) & 3))] = make_uint4(x[4 * c], x[4 * c + 1], x[4 * c + 2],
                                                        x[4 * c + 3]);
      }
    // The unit's row blocks only: the other half of a split tile reads slot 0.
    const uint32_t pm = uc.pmask;
    tb[lane] = make_uint4(ta.x & pm, ta.y & pm, ta.z & pm, ta.w & pm);
    if (lane < kTableQ - 64) tb[64 + lane] = make_uint4(tb2.x & pm, tb2.y & pm, tb2.z & pm, tb2.w & pm);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const Unit u = uc;
    const bool staged = u.g >= 0;
    int32_t rows[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) rows[rb] = rows_n[rb] < N ? rows_n[rb] : -1;
    // Unit `next` (or `cur` again at the end): rows, table and row list go out now; the unit
    // after it gets its metadata and indices.
    const bool has_next = next < t_end;
    uc = decode(meta_n, next_second);
    gather(uc.g);
    load_tbl(nx, ta, tb2);
    load_rows(nx, rows_n);
    int nn;
    const bool nn_second = uc.first;
    if (nn_second) {
      nn = next;
    } else {
      nn = tile_of(pend);
      pend = take_async();
    }
    const int nnx = nn < t_end ? nn : nx;
    const int nn_off = nn_second ? second_offset(meta_n) : 0;
    meta_n = load_meta(nnx);
    load_idx(nnx, nn_off);
    if (!u.second) {
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) acc[rb][cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    const uint32_t tm = u.taps;
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
      const uint32_t q4 = (uint32_t)q * 0x01010101u;
      auto rd = [&](int v, uint4 (&b)[4], uint4 (&a)[2]) {
        const uint32_t s4 = tb32[v];
        rd_a(v, a);
        // The four slots' swizzled piece indices at once: byte rb of x4 = q ^ ((s_rb >> 1) & 3)
        // (20 instead of 23 VALU instructions per tap; 1.5-2.5 % faster on 32->32).
        const uint32_t x4 = ((s4 >> 1) & 0x03030303u) ^ q4;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
          const uint32_t s = (s4 >> (8 * rb)) & 0xffu;
          const uint32_t x = (x4 >> (8 * rb)) & 0xffu;
          b[rb] = st[s * 4 + x];
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
          const int32_t r = rows[rb];
          const int32_t e = r >= 0 ? nbr[(int64_t)r * kTaps + v] : -1;
          const bool ok = e >= 0 && e < N;
          const uint4 bv4 = ((const uint4*)(feats + (int64_t)(ok ? e : 0) * 32))[q];
          b[rb] = ok ? bv4 : make_uint4(0u, 0u, 0u, 0u);
        }
        mm(b, a);
      }
    }

    // Epilogue (after the second half of a split tile): lane (l16, q) holds row 16*rb + l16,
    // columns co0 + 16*cb + 4q .. +3.  Residual values are all loaded before the first store
    // (rows past N read row 0, not stored); every stored element is computed from the residual
    // element at the same address, so the output may alias the residual.
    struct alignas(4 * sizeof(T)) V4 {
      T v[4];
    };
    if (!u.first) {
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
      uint32_t pk[2][2];  // [cb]: the lane's four converted columns, two per dword
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        float xv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) xv[i] = acc[rb][cb][i] + bv[cb][i];
        if (EPI == TSC_EPI_BIAS_RESIDUAL) {
#pragma unroll
          for (int i = 0; i < 4; ++i) xv[i] += (float)rt[rb][cb].v[i];
        }
        // Pairs as 2-vectors: one v_cvt_pk_{f16,bf16}_f32 each (round to nearest even, as the
        // scalar conversion; built element by element the compiler emitted two converts and an OR).
        typedef T t2 __attribute__((ext_vector_type(2)));
        const t2 lo = {(T)xv[0], (T)xv[1]}, hi = {(T)xv[2], (T)xv[3]};
        pk[cb][0] = __builtin_bit_cast(uint32_t, lo);
        pk[cb][1] = __builtin_bit_cast(uint32_t, hi);
      }
      // v_permlane16_swap trades the odd 16-lane rows of its first operand (cb 0) with the even
      // rows of its second (cb 1), between lanes of one l16 and so of one output row: afterwards
      // q0 holds columns 0-7, q1 16-23, q2 8-15, q3 24-31, and one 16-byte store per lane writes
      // the row's 64 bytes (two 8-byte stores per half-row block measured ~5 % slower at Co 64).
      const auto s0 = __builtin_amdgcn_permlane16_swap(pk[0][0], pk[1][0], false, false);
      const auto s1 = __builtin_amdgcn_permlane16_swap(pk[0][1], pk[1][1], false, false);
      const int32_t row = rows[rb];
      if (row >= 0)
        *(uint4*)((char*)out_lane + (uint64_t)(uint32_t)row * row_bytes) =
            make_uint4(s0[0], s1[0], s0[1], s1[1]);
    }
    }  // !u.first
    if (!has_next) break;
    cur = next;
    next = nn;
    next_second = nn_second;
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
  auto al16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  return a.plan && a.Ci == 32 && (a.Co == 32 || a.Co == 64) &&
         (a.dtype == TSC_F16 || a.dtype == TSC_BF16) && a.N > 0 && a.N <= INT32_MAX - 64 &&
         al16(a.out) && (a.epilogue != TSC_EPI_BIAS_RESIDUAL || al8(a.residual));
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
  ProfScope pt(ctx, "plan_tiles");
  plan_tile_kernel<<<blocks, 64 * kPlanWaves, 0, ctx->stream>>>(
      rows, nbr, N, L.T, rows, (int32_t*)(base + L.count), (uint32_t*)(base + L.rbm),
      (int32_t*)(base + L.list), (uint4*)(base + L.slots));
  return check_hip(hipGetLastError(), "gather plan tiles");
}

}  // namespace tsc
