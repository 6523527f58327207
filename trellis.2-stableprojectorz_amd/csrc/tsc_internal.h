// Internal declarations shared by the translation units of libtrellis_sparse.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include <string>
#include <vector>

#include "../../include/tsc.h"

// One kernel launch bracketed by events (recorded only while profiling is on).
struct tsc_prof_rec {
  const char* name;
  hipEvent_t start, stop;
};
struct tsc_prof_agg {
  std::string name;
  double total_ms;
  int64_t launches;
};

// A longest-first tile schedule of the 256-row conv tiles (conv.hip) kept for reuse.  It depends
// only on the neighbor map, the row order, N and the tile height, so every conv over one
// coordinate set (the eight convs of a ResBlock chain) builds it once.  Keyed by the buffers'
// addresses: an entry is dropped when tsc_map_build or tsc_map_conv_order writes to, or tsc_free
// releases, one of them.  Whatever a stale entry holds, it is a permutation of the same tiles, so
// it can only change which block computes a tile, never a result.
struct tsc_sched_entry {
  const int32_t* nbr = nullptr;
  const int32_t* order = nullptr;
  int64_t N = -1;
  int32_t bm = 0;
  bool valid = false;   // schedule written (launched) for this key
  void* buf = nullptr;  // device: cost per tile, then the XCD lists
  size_t bytes = 0;
  uint64_t used = 0;    // last use, for replacement
};

struct tsc_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  // Growable device workspace (stream-ordered users; grown only after a stream sync).
  void* ws = nullptr;
  size_t ws_bytes = 0;
  // Cached conv tile schedules (a conv may run while `ws` holds the intermediate rows of a
  // ResBlock, so they live in buffers of their own).
  std::vector<tsc_sched_entry> sched;
  uint64_t sched_tick = 0;
  // hipBLASLt handle (created on the first linear layer) and its workspace.
  void* blaslt = nullptr;
  void* ws_blas = nullptr;
  size_t ws_blas_bytes = 0;
  void* blas_algos = nullptr;  // tuned algorithm per linear shape (linear.hip)
  // Pinned host chunks (and their last copies' events) of the safetensors reader.
  void* st_pin[2] = {nullptr, nullptr};
  hipEvent_t st_ev[2] = {nullptr, nullptr};
  bool st_pending[2] = {false, false};
  int st_next = 0;  // chunk the next load starts with
  // Device address of this device's static schedule scratch, looked up by the first
  // tsc_conv_fused_noalloc call on this context.
  void* sched_scratch = nullptr;
  bool profile = false;
  std::vector<tsc_prof_rec> prof;      // pending launches
  std::vector<tsc_prof_agg> prof_agg;  // aggregated by tsc_profile_collect
};

namespace tsc {

// Thread-local error string; returns `code` so call sites can `return fail(...)`.
int fail(int code, const char* fmt, ...);
int check_hip(hipError_t e, const char* what);

// Ensures ctx->ws holds at least `bytes`; returns TSC_OK or an error status.
int workspace(tsc_ctx* ctx, size_t bytes, void** out);
// The same for ctx->ws_blas.
int blas_workspace(tsc_ctx* ctx, size_t bytes, void** out);
// The cached tile schedule of (nbr, order, N, bm).  On a hit *entry->valid is true and
// entry->buf holds it; on a miss the least recently used entry (at most kSchedCacheEntries) is
// re-keyed with valid = false and its buffer grown to `bytes`; the caller launches the schedule
// kernels into it and then sets valid.
constexpr int kSchedCacheEntries = 4;
int sched_cached(tsc_ctx* ctx, const int32_t* nbr, const int32_t* order, int64_t N, int32_t bm,
                 size_t bytes, tsc_sched_entry** entry);
// Drops the cached schedules whose neighbor map or row order is the buffer at p.
void sched_forget(tsc_ctx* ctx, const void* p);

void prof_clear(tsc_ctx* ctx);

// Records start/stop events on the context stream around one launch when profiling is on.
struct ProfScope {
  tsc_ctx* ctx;
  tsc_prof_rec rec;
  bool on;
  ProfScope(tsc_ctx* c, const char* name) : ctx(c), rec{name, nullptr, nullptr}, on(c->profile) {
    if (on && (hipEventCreate(&rec.start) != hipSuccess || hipEventCreate(&rec.stop) != hipSuccess ||
               hipEventRecord(rec.start, ctx->stream) != hipSuccess))
      on = false;
  }
  ~ProfScope() {
    if (on && hipEventRecord(rec.stop, ctx->stream) == hipSuccess) ctx->prof.push_back(rec);
  }
};

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Bump allocator over a workspace region (256-byte aligned slices).
struct Carve {
  char* base;
  size_t off;
  explicit Carve(void* b) : base((char*)b), off(0) {}
  template <typename T>
  T* take(size_t count) {
    T* p = (T*)(base + off);
    off = align_up(off + count * sizeof(T), 256);
    return p;
  }
};

// ---- launchers implemented in map_build.hip ----
int map_build_bitmap(tsc_ctx* ctx, const int32_t* coords, int64_t N, int32_t B, int32_t X,
                     int32_t Y, int32_t Z, const int32_t dil[3], void* keys_out, int32_t* perm_out,
                     int32_t* nbr_out, uint32_t* status_dev);
int map_build_radix(tsc_ctx* ctx, const int32_t* coords, int64_t N, int32_t B, int32_t X,
                    int32_t Y, int32_t Z, const int32_t dil[3], void* keys_out, int32_t* perm_out,
                    int32_t* nbr_out, uint32_t* status_dev);
// Rows 0..N-1 sorted by the (batch, Z-curve) key of their coordinates over the low `bits` bits of
// x, y, z (z lowest), the lowest `shift` bits dropped, nbits = key width (<= 64); the radix sort
// of map_build_radix with a Morton key.  Writes rows_out[0..N).
int sort_rows_morton(tsc_ctx* ctx, const int32_t* coords, int64_t N, int bits, int shift,
                     int nbits, int32_t* rows_out);

// The store pattern of the radix path's fill alone (a measurement kernel): row rows[i] (i when
// rows is null) of the (N,27) int32 table `out` written as the fill writes it; rows outside
// [0, N) are skipped.
int map_write_floor_launch(tsc_ctx* ctx, const int32_t* rows, int64_t N, int32_t* out);

// ---- launcher implemented in conv_order.hip ----
int conv_order_launch(tsc_ctx* ctx, const int32_t* nbr, const int32_t* perm, int64_t N,
                      int32_t* order);

// ---- launchers implemented in conv.hip ----
struct ConvArgs {
  int32_t dtype;
  const void* feats;
  const void* weight;
  const void* bias;      // may be null
  const int32_t* nbr;
  const int32_t* order;  // may be null
  int64_t N;
  int32_t Ci, Co;
  int32_t epilogue;      // TSC_EPI_BIAS, TSC_EPI_BIAS_RESIDUAL, or TSC_EPI_BIAS_LN_SILU when
                         // conv_fuses_ln (else LN runs as a row pass by the caller)
  const void* residual;  // for TSC_EPI_BIAS_RESIDUAL
  void* out;
  const void* plan = nullptr;  // gather plan (conv_gather.hip) or null
  // Device buffer for the 256-row tile schedule instead of the context's growable workspace
  // (tsc_conv_fused_noalloc), and its size in bytes.
  void* sched_scratch = nullptr;
  size_t sched_scratch_bytes = 0;
  // LayerNorm + SiLU inside the conv epilogue (epilogue TSC_EPI_BIAS_LN_SILU, only where
  // conv_fuses_ln says so): gamma / beta (Co, NULL = 1 / 0) and eps.
  const void* ln_gamma = nullptr;
  const void* ln_beta = nullptr;
  float ln_eps = 0.f;
};
// Row tiles the longest-first schedule handles (beyond it tiles run in row order), and the
// schedule's largest scratch: a cost per tile plus 8 lists of ceil(tiles / 8) slots.
constexpr int kSchedMaxTiles = 1 << 16;
constexpr size_t kSchedScratchBytes = (size_t)2 * kSchedMaxTiles * 4;
// Rows a tsc_conv_fused_noalloc call may have: every 256-row tile fits the schedule.
constexpr int64_t kNoallocMaxRows = (int64_t)kSchedMaxTiles * 256;
// The static schedule scratch of this device (conv.hip), found once per device by
// hipGetSymbolAddress with that device current; null with an error status on failure.
int sched_scratch_ptr(int device, void** out);
int conv_launch(tsc_ctx* ctx, const ConvArgs& a);
// True when the tuned kernels take this shape and these buffers (else the generic kernel runs).
bool conv_tuned_shape(const ConvArgs& a);
// True when the kernel conv_launch picks for `a` owns whole output rows and can apply
// LayerNorm + SiLU in its epilogue (16-bit wide rows with Co of 64, 128 or 256, 16-byte aligned
// gamma / beta); callers then pass epilogue TSC_EPI_BIAS_LN_SILU instead of a row pass.
bool conv_fuses_ln(const ConvArgs& a);

// ---- gather plan + planned narrow conv (conv_gather.hip) ----
constexpr int kPlanRows = 64;                   // rows per plan tile
constexpr int kPlanSlots = 256;                 // distinct-row list capacity per tile
constexpr int kPlanStage = 208;                 // LDS row slots per wave of the planned conv
                                                // (slot 0 = zeros): staged tiles and halves
                                                // have fewer distinct rows
constexpr int kPlanTableBytes = 16 * 28 * 4;    // slot table per tile: [16][28 taps][4 blocks]
struct PlanLayout {
  int64_t T;                                    // tiles
  size_t rows, count, rbm, list, slots, total;  // byte offsets in the plan buffer, and its size
};
PlanLayout plan_layout(int64_t N);
int gather_plan_launch(tsc_ctx* ctx, const int32_t* coords, const int32_t* nbr, int64_t N,
                       int32_t B, int32_t X, int32_t Y, int32_t Z, void* plan);
bool conv_gather_supported(const ConvArgs& a);
int conv_gather_launch(tsc_ctx* ctx, const ConvArgs& a);

// ---- launchers implemented in subdivide.hip ----
int subdivide_count_launch(tsc_ctx* ctx, const uint8_t* keep, int64_t N, int64_t* count_host);
int subdivide_launch(tsc_ctx* ctx, const int32_t* coords, int64_t N, const void* feats,
                     int64_t row_bytes, const uint8_t* keep, int32_t* coords_out,
                     void* feats_out);

// ---- implemented in linear.hip ----
int linear_launch(tsc_ctx* ctx, int32_t dtype, const void* x, int64_t N, int32_t Cin,
                  const void* weight, const void* bias, const void* residual, int32_t Cout,
                  void* out);
void blas_destroy(tsc_ctx* ctx);

// ---- implemented in safetensors.hip ----
int st_open(const char* path, tsc_st** out);
void st_close(tsc_st* f);
void st_counts(const tsc_st* f, int64_t* tensors, int64_t* metadata, int64_t* data_offset);
int st_name(const tsc_st* f, int64_t i, char* buf, int32_t len);
int st_metadata(const tsc_st* f, int64_t i, char* key, int32_t key_len, char* value,
                int32_t value_len);
int st_info(const tsc_st* f, const char* name, int32_t* dtype, int32_t* ndim, int64_t* shape,
            int32_t max_dims, int64_t* offsets);
int st_load(tsc_ctx* ctx, const tsc_st* f, const char* name, int32_t out_dtype, void* dst);
void st_release(tsc_ctx* ctx);

// ---- implemented in attention.hip ----
int attention_launch(tsc_ctx* ctx, int32_t dtype, const void* q, const void* k, const void* v,
                     const int32_t* cu_q, const int32_t* cu_kv, int32_t B, int64_t total_q,
                     int64_t total_kv, int32_t H, int32_t D, float scale, int32_t max_seqlen_q,
                     void* out);

// ---- launchers implemented in rowops.hip ----
int layernorm_launch(tsc_ctx* ctx, int32_t dtype, const void* x, int64_t N, int32_t C,
                     const void* gamma, const void* beta, float eps, int32_t apply_silu, void* y);
int silu_launch(tsc_ctx* ctx, int32_t dtype, const void* x, int64_t numel, void* y);
int add_launch(tsc_ctx* ctx, int32_t dtype, const void* a, const void* b, int64_t numel, void* y);

}  // namespace tsc
