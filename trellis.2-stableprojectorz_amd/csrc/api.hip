// C ABI of libtrellis_sparse.so: argument validation, contexts, workspace, error reporting.
// Validation mirrors what the reference checks before dispatch (src/sparse/ops/conv3d.ts:41-49:
// GPU input, Ci = weight.shape[4], Co = weight.shape[0]) and adds the checks a C ABI needs
// (null pointers, alignment, size limits), so bad input becomes a status code, never a fault.

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>

#include "tsc_internal.h"

namespace tsc {

static thread_local char g_err[512];

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return TSC_OK;
  return fail(TSC_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

namespace {
// Grows a stream-ordered device buffer to at least `bytes` (with 25 % headroom, at least 1 MiB).
int grow_buffer(tsc_ctx* ctx, void** buf, size_t* cap, size_t bytes, const char* what,
                void** out) {
  if (bytes <= *cap) {
    *out = *buf;
    return TSC_OK;
  }
  // Growing: earlier enqueued work may still use the old block.
  int st = check_hip(hipStreamSynchronize(ctx->stream), "workspace sync");
  if (st) return st;
  if (*buf) {
    st = check_hip(hipFree(*buf), "workspace free");
    *buf = nullptr;
    *cap = 0;
    if (st) return st;
  }
  size_t want = std::max(bytes + bytes / 4, (size_t)(1u << 20));
  void* p = nullptr;
  if (hipMalloc(&p, want) != hipSuccess) {
    (void)hipGetLastError();
    return fail(TSC_ERR_OOM, "%s: cannot allocate %zu bytes", what, want);
  }
  *buf = p;
  *cap = want;
  *out = p;
  return TSC_OK;
}
}  // namespace

int workspace(tsc_ctx* ctx, size_t bytes, void** out) {
  return grow_buffer(ctx, &ctx->ws, &ctx->ws_bytes, bytes, "workspace", out);
}

int sched_cached(tsc_ctx* ctx, const int32_t* nbr, const int32_t* order, int64_t N, int32_t bm,
                 size_t bytes, tsc_sched_entry** entry) {
  const uint64_t now = ++ctx->sched_tick;
  for (auto& e : ctx->sched)
    if (e.valid && e.nbr == nbr && e.order == order && e.N == N && e.bm == bm && e.bytes >= bytes) {
      e.used = now;
      *entry = &e;
      return TSC_OK;
    }
  if ((int)ctx->sched.size() < kSchedCacheEntries) ctx->sched.emplace_back();
  tsc_sched_entry* victim = &ctx->sched[0];
  for (auto& e : ctx->sched)
    if (e.used < victim->used) victim = &e;
  victim->valid = false;
  void* buf;
  const int st = grow_buffer(ctx, &victim->buf, &victim->bytes, bytes, "schedule workspace", &buf);
  if (st) return st;
  victim->nbr = nbr;
  victim->order = order;
  victim->N = N;
  victim->bm = bm;
  victim->used = now;
  *entry = victim;
  return TSC_OK;
}

void sched_forget(tsc_ctx* ctx, const void* p) {
  if (!p) return;
  for (auto& e : ctx->sched)
    if ((const void*)e.nbr == p || (const void*)e.order == p) e.valid = false;
}

int blas_workspace(tsc_ctx* ctx, size_t bytes, void** out) {
  return grow_buffer(ctx, &ctx->ws_blas, &ctx->ws_blas_bytes, bytes, "hipBLASLt workspace", out);
}

void prof_clear(tsc_ctx* ctx) {
  for (auto& r : ctx->prof) {
    (void)hipEventDestroy(r.start);
    (void)hipEventDestroy(r.stop);
  }
  ctx->prof.clear();
}

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// True when the byte ranges [a, a + na) and [b, b + nb) share a byte.
static bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return na && nb && x < y + nb && y < x + na;
}

static int elem_size(int32_t dtype) {
  switch (dtype) {
    case TSC_F32: return 4;
    case TSC_F16: return 2;
    case TSC_BF16: return 2;
  }
  return 0;
}

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

static int check_ctx(tsc_ctx* ctx) {
  if (!ctx) return fail(TSC_ERR_INVALID, "null context");
  return TSC_OK;
}

static int validate_conv(tsc_ctx* ctx, int32_t dtype, const void* feats, const void* weight,
                         const void* bias, const int32_t* nbr, int64_t N, int32_t Ci, int32_t Co,
                         void* out) {
  int st = check_ctx(ctx);
  if (st) return st;
  const int es = elem_size(dtype);
  if (!es) return fail(TSC_ERR_INVALID, "conv: unknown dtype %d", dtype);
  if (N < 0 || N > INT32_MAX) return fail(TSC_ERR_INVALID, "conv: N=%lld out of range", (long long)N);
  if (Ci <= 0 || Co <= 0) return fail(TSC_ERR_INVALID, "conv: Ci=%d Co=%d must be positive", Ci, Co);
  if ((int64_t)Ci * es > 65536)
    return fail(TSC_ERR_UNSUPPORTED, "conv: Ci*elem_size=%lld bytes exceeds 65536",
                (long long)Ci * es);
  if (Co > 65536) return fail(TSC_ERR_UNSUPPORTED, "conv: Co=%d exceeds 65536", Co);
  if (N == 0) return TSC_OK;
  if (!feats || !weight || !nbr || !out) return fail(TSC_ERR_INVALID, "conv: null buffer");
  // Element alignment is all any kernel needs; 16-byte aligned buffers (and channel counts in
  // whole 32-byte rows / 32-column blocks) select the tuned kernels.
  if (!aligned(feats, es) || !aligned(weight, es) || !aligned(out, es) ||
      (bias && !aligned(bias, es)) || !aligned(nbr, 4))
    return fail(TSC_ERR_INVALID, "conv: feats, weight, bias and out must be aligned to their "
                                 "element size, nbr to 4 bytes");
  return TSC_OK;
}

static int validate_residual(int32_t dtype, const void* residual) {
  if (!residual) return fail(TSC_ERR_INVALID, "conv: residual epilogue needs a residual buffer");
  if (!aligned(residual, elem_size(dtype)))
    return fail(TSC_ERR_INVALID, "conv: residual must be aligned to its element size");
  return TSC_OK;
}

}  // namespace tsc

using namespace tsc;

extern "C" {

int tsc_version(void) { return TSC_VERSION; }

const char* tsc_last_error(void) { return g_err; }

int tsc_ctx_create(int device, void* stream, tsc_ctx** out) {
  g_err[0] = 0;
  if (!out) return fail(TSC_ERR_INVALID, "ctx_create: null out");
  *out = nullptr;
  int ndev = 0;
  int st = check_hip(hipGetDeviceCount(&ndev), "hipGetDeviceCount");
  if (st) return st;
  if (device < 0 || device >= ndev)
    return fail(TSC_ERR_INVALID, "ctx_create: device %d not in [0,%d)", device, ndev);
  tsc_ctx* c = new tsc_ctx();
  c->device = device;
  c->ws = nullptr;
  c->ws_bytes = 0;
  c->stream = (hipStream_t)stream;  // NULL = the HIP null stream
  *out = c;
  return TSC_OK;
}

int tsc_ctx_destroy(tsc_ctx* ctx) {
  g_err[0] = 0;
  if (!ctx) return TSC_OK;
  DeviceGuard g(ctx->device);
  int st = check_hip(hipStreamSynchronize(ctx->stream), "ctx_destroy sync");
  if (ctx->ws) (void)hipFree(ctx->ws);
  for (auto& e : ctx->sched)
    if (e.buf) (void)hipFree(e.buf);
  blas_destroy(ctx);
  if (ctx->ws_blas) (void)hipFree(ctx->ws_blas);
  st_release(ctx);
  prof_clear(ctx);
  delete ctx;
  return st;
}

int tsc_ctx_set_stream(tsc_ctx* ctx, void* stream) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  DeviceGuard g(ctx->device);
  // Work already queued on the old stream may use the workspace: order the new stream after it.
  if ((hipStream_t)stream != ctx->stream) {
    st = check_hip(hipStreamSynchronize(ctx->stream), "set_stream sync");
    if (st) return st;
  }
  ctx->stream = (hipStream_t)stream;
  return TSC_OK;
}

void* tsc_ctx_stream(tsc_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int tsc_sync(tsc_ctx* ctx) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  DeviceGuard g(ctx->device);
  return check_hip(hipStreamSynchronize(ctx->stream), "tsc_sync");
}

int tsc_malloc(tsc_ctx* ctx, size_t bytes, void** out) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (!out) return fail(TSC_ERR_INVALID, "malloc: null out");
  DeviceGuard g(ctx->device);
  if (hipMalloc(out, bytes ? bytes : 1) != hipSuccess) {
    (void)hipGetLastError();
    *out = nullptr;
    return fail(TSC_ERR_OOM, "malloc: cannot allocate %zu bytes", bytes);
  }
  return TSC_OK;
}

int tsc_free(tsc_ctx* ctx, void* ptr) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (!ptr) return TSC_OK;
  DeviceGuard g(ctx->device);
  st = check_hip(hipStreamSynchronize(ctx->stream), "free sync");
  if (st) return st;
  sched_forget(ctx, ptr);
  return check_hip(hipFree(ptr), "hipFree");
}

int tsc_memcpy_h2d(tsc_ctx* ctx, void* dst, const void* src, size_t bytes) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (!bytes) return TSC_OK;
  if (!dst || !src) return fail(TSC_ERR_INVALID, "memcpy_h2d: null pointer");
  DeviceGuard g(ctx->device);
  st = check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "memcpy_h2d");
  if (st) return st;
  return check_hip(hipStreamSynchronize(ctx->stream), "memcpy_h2d sync");
}

int tsc_memcpy_d2h(tsc_ctx* ctx, void* dst, const void* src, size_t bytes) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (!bytes) return TSC_OK;
  if (!dst || !src) return fail(TSC_ERR_INVALID, "memcpy_d2h: null pointer");
  DeviceGuard g(ctx->device);
  st = check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "memcpy_d2h");
  if (st) return st;
  return check_hip(hipStreamSynchronize(ctx->stream), "memcpy_d2h sync");
}

int tsc_memset_zero(tsc_ctx* ctx, void* dst, size_t bytes) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (!bytes) return TSC_OK;
  if (!dst) return fail(TSC_ERR_INVALID, "memset_zero: null pointer");
  DeviceGuard g(ctx->device);
  return check_hip(hipMemsetAsync(dst, 0, bytes, ctx->stream), "memset_zero");
}

int tsc_map_key_bytes(int32_t B, int32_t X, int32_t Y, int32_t Z) {
  if (B <= 0 || X <= 0 || Y <= 0 || Z <= 0) return 0;
  const int64_t cells = (int64_t)B * X * Y * Z;
  return cells < (int64_t(1) << 31) ? 4 : 8;
}

int tsc_map_build(tsc_ctx* ctx, const int32_t* coords, int64_t N, int32_t B, int32_t X, int32_t Y,
                  int32_t Z, const int32_t kernel[3], const int32_t dilation[3], int32_t method,
                  void* keys_out, int32_t* perm_out, int32_t* nbr_out, uint32_t* status_dev) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (!kernel || !dilation) return fail(TSC_ERR_INVALID, "map_build: null kernel/dilation");
  if (kernel[0] != 3 || kernel[1] != 3 || kernel[2] != 3)
    return fail(TSC_ERR_UNSUPPORTED, "map_build: kernel %dx%dx%d unsupported (3x3x3 only)",
                kernel[0], kernel[1], kernel[2]);
  if (dilation[0] < 1 || dilation[1] < 1 || dilation[2] < 1)
    return fail(TSC_ERR_INVALID, "map_build: dilation must be >= 1");
  if (N < 0 || N > INT32_MAX) return fail(TSC_ERR_INVALID, "map_build: N=%lld out of range", (long long)N);
  if (B <= 0 || X <= 0 || Y <= 0 || Z <= 0)
    return fail(TSC_ERR_INVALID, "map_build: grid %dx%dx%dx%d must be positive", B, X, Y, Z);
  if ((__int128)B * X * Y * Z > ((__int128)1 << 62))
    return fail(TSC_ERR_UNSUPPORTED, "map_build: grid %dx%dx%dx%d has more than 2^62 cells", B,
                X, Y, Z);
  if (!status_dev) return fail(TSC_ERR_INVALID, "map_build: null status");
  if (N > 0 && (!coords || !nbr_out)) return fail(TSC_ERR_INVALID, "map_build: null coords/nbr");
  if (coords && !aligned(coords, 16))
    return fail(TSC_ERR_INVALID, "map_build: coords must be 16-byte aligned");
  const int kb = tsc_map_key_bytes(B, X, Y, Z);
  if (keys_out && !aligned(keys_out, kb)) return fail(TSC_ERR_INVALID, "map_build: misaligned keys");
  if (method < TSC_MAP_AUTO || method > TSC_MAP_RADIX)
    return fail(TSC_ERR_INVALID, "map_build: unknown method %d", method);
  const int64_t cells = (int64_t)B * X * Y * Z;
  // The bitmap path streams cells/8 bytes of bitmap three times and scatters with device
  // atomics; the radix path (bucket partition + per-bucket LDS sort + LDS-window fill) has one
  // or two more launches but no grid-sized pass.  Measured on MI355X: equal within ~2 us up to
  // 2^21 cells, radix ahead beyond (1.9x at 1.5M voxels in 512^3).
  const int64_t kMaxBitmapCells = int64_t(1) << 32;  // 512 MB bitmap
  if (method == TSC_MAP_AUTO) method = cells <= (int64_t(1) << 21) ? TSC_MAP_BITMAP : TSC_MAP_RADIX;
  if (method == TSC_MAP_BITMAP && cells > kMaxBitmapCells)
    return fail(TSC_ERR_UNSUPPORTED, "map_build: grid of %lld cells too large for the bitmap path",
                (long long)cells);
  DeviceGuard g(ctx->device);
  sched_forget(ctx, nbr_out);
  if (method == TSC_MAP_RADIX)
    return map_build_radix(ctx, coords, N, B, X, Y, Z, dilation, keys_out, perm_out, nbr_out,
                           status_dev);
  return map_build_bitmap(ctx, coords, N, B, X, Y, Z, dilation, keys_out, perm_out, nbr_out,
                          status_dev);
}

int tsc_map_write_floor(tsc_ctx* ctx, const int32_t* rows, int64_t N, int32_t* out) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (N < 0 || N > INT32_MAX)
    return fail(TSC_ERR_INVALID, "map_write_floor: N=%lld out of range", (long long)N);
  if (N > 0 && !out) return fail(TSC_ERR_INVALID, "map_write_floor: null out");
  if (!aligned(out, 4) || !aligned(rows, 4))
    return fail(TSC_ERR_INVALID, "map_write_floor: rows and out must be 4-byte aligned");
  DeviceGuard g(ctx->device);
  sched_forget(ctx, out);
  return tsc::map_write_floor_launch(ctx, rows, N, out);
}

int tsc_map_conv_order(tsc_ctx* ctx, const int32_t* nbr, const int32_t* perm, int64_t N,
                       int32_t* order_out) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (N < 0 || N > INT32_MAX)
    return fail(TSC_ERR_INVALID, "map_conv_order: N=%lld out of range", (long long)N);
  if (N > 0 && (!nbr || !order_out)) return fail(TSC_ERR_INVALID, "map_conv_order: null nbr/order");
  DeviceGuard g(ctx->device);
  sched_forget(ctx, order_out);
  return tsc::conv_order_launch(ctx, nbr, perm, N, order_out);
}

int64_t tsc_map_gather_plan_bytes(int64_t N) {
  if (N < 0 || N > INT32_MAX - 64) return -1;
  return (int64_t)tsc::plan_layout(N).total;
}

int tsc_map_gather_plan(tsc_ctx* ctx, const int32_t* coords, const int32_t* nbr, int64_t N,
                        int32_t B, int32_t X, int32_t Y, int32_t Z, void* plan) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (N < 0 || N > INT32_MAX - 64)
    return fail(TSC_ERR_INVALID, "map_gather_plan: N=%lld out of range", (long long)N);
  if (B <= 0 || X <= 0 || Y <= 0 || Z <= 0)
    return fail(TSC_ERR_INVALID, "map_gather_plan: grid %dx%dx%dx%d must be positive", B, X, Y, Z);
  if (N > 0 && (!coords || !nbr || !plan))
    return fail(TSC_ERR_INVALID, "map_gather_plan: null coords/nbr/plan");
  if (coords && !aligned(coords, 16))
    return fail(TSC_ERR_INVALID, "map_gather_plan: coords must be 16-byte aligned");
  if (plan && !aligned(plan, 256))
    return fail(TSC_ERR_INVALID, "map_gather_plan: plan must be 256-byte aligned");
  DeviceGuard g(ctx->device);
  return tsc::gather_plan_launch(ctx, coords, nbr, N, B, X, Y, Z, plan);
}

namespace {
// The conv's epilogue for a requested TSC_EPI_BIAS_LN_SILU: inside the conv when its kernel owns
// whole rows (conv_fuses_ln), else bias only, with the caller running the LayerNorm row pass.
// Returns true when the caller still has to run that pass.
bool set_ln_epilogue(ConvArgs& a, int32_t epilogue, const void* ln_gamma, const void* ln_beta,
                     float eps) {
  if (epilogue != TSC_EPI_BIAS_LN_SILU) return false;
  a.ln_gamma = ln_gamma;
  a.ln_beta = ln_beta;
  a.ln_eps = eps;
  a.epilogue = TSC_EPI_BIAS_LN_SILU;
  if (conv_fuses_ln(a)) return false;
  a.epilogue = TSC_EPI_BIAS;
  return true;
}
}  // namespace

int tsc_conv_planned(tsc_ctx* ctx, int32_t dtype, const void* feats, const void* weight,
                     const void* bias, const int32_t* nbr, const void* plan, int64_t N,
                     int32_t Ci, int32_t Co, int32_t epilogue, const void* residual,
                     const void* ln_gamma, const void* ln_beta, float eps, void* out) {
  g_err[0] = 0;
  int st = validate_conv(ctx, dtype, feats, weight, bias, nbr, N, Ci, Co, out);
  if (st) return st;
  if (epilogue < TSC_EPI_BIAS || epilogue > TSC_EPI_BIAS_LN_SILU)
    return fail(TSC_ERR_INVALID, "conv: unknown epilogue %d", epilogue);
  if (epilogue == TSC_EPI_BIAS_RESIDUAL && N > 0 && (st = validate_residual(dtype, residual)))
    return st;
  if (N > 0 && !plan) return fail(TSC_ERR_INVALID, "conv_planned: null plan");
  if (plan && !aligned(plan, 256))
    return fail(TSC_ERR_INVALID, "conv_planned: plan must be 256-byte aligned");
  if (N == 0) return TSC_OK;
  if (N > INT32_MAX - 64)
    return fail(TSC_ERR_INVALID, "conv_planned: N=%lld out of range", (long long)N);
  DeviceGuard g(ctx->device);
  ConvArgs a{dtype, feats, weight, bias, nbr, nullptr, N, Ci, Co,
             epilogue == TSC_EPI_BIAS_RESIDUAL ? TSC_EPI_BIAS_RESIDUAL : TSC_EPI_BIAS,
             residual, out, plan};
  const bool ln_pass = set_ln_epilogue(a, epilogue, ln_gamma, ln_beta, eps);
  st = conv_launch(ctx, a);
  if (st || !ln_pass) return st;
  return layernorm_launch(ctx, dtype, out, N, Co, ln_gamma, ln_beta, eps, 1, out);
}

int tsc_conv(tsc_ctx* ctx, int32_t dtype, const void* feats, const void* weight, const void* bias,
             const int32_t* nbr, const int32_t* order, int64_t N, int32_t Ci, int32_t Co,
             void* out) {
  return tsc_conv_fused(ctx, dtype, feats, weight, bias, nbr, order, N, Ci, Co, TSC_EPI_BIAS,
                        nullptr, nullptr, nullptr, 0.f, out);
}

int tsc_conv_fused(tsc_ctx* ctx, int32_t dtype, const void* feats, const void* weight,
                   const void* bias, const int32_t* nbr, const int32_t* order, int64_t N,
                   int32_t Ci, int32_t Co, int32_t epilogue, const void* residual,
                   const void* ln_gamma, const void* ln_beta, float eps, void* out) {
  g_err[0] = 0;
  int st = validate_conv(ctx, dtype, feats, weight, bias, nbr, N, Ci, Co, out);
  if (st) return st;
  if (epilogue < TSC_EPI_BIAS || epilogue > TSC_EPI_BIAS_LN_SILU)
    return fail(TSC_ERR_INVALID, "conv: unknown epilogue %d", epilogue);
  if (epilogue == TSC_EPI_BIAS_RESIDUAL && N > 0 && (st = validate_residual(dtype, residual)))
    return st;
  if (N == 0) return TSC_OK;
  DeviceGuard g(ctx->device);
  ConvArgs a{dtype, feats, weight, bias, nbr, order, N, Ci, Co,
             epilogue == TSC_EPI_BIAS_RESIDUAL ? TSC_EPI_BIAS_RESIDUAL : TSC_EPI_BIAS,
             residual, out};
  const bool ln_pass = set_ln_epilogue(a, epilogue, ln_gamma, ln_beta, eps);
  st = conv_launch(ctx, a);
  if (st || !ln_pass) return st;
  return layernorm_launch(ctx, dtype, out, N, Co, ln_gamma, ln_beta, eps, 1, out);
}

int tsc_conv_fused_noalloc(tsc_ctx* ctx, int32_t dtype, const void* feats, const void* weight,
                           const void* bias, const int32_t* nbr, const int32_t* order, int64_t N,
                           int32_t Ci, int32_t Co, int32_t epilogue, const void* residual,
                           const void* ln_gamma, const void* ln_beta, float eps, void* out) {
  g_err[0] = 0;
  int st = validate_conv(ctx, dtype, feats, weight, bias, nbr, N, Ci, Co, out);
  if (st) return st;
  if (epilogue < TSC_EPI_BIAS || epilogue > TSC_EPI_BIAS_LN_SILU)
    return fail(TSC_ERR_INVALID, "conv: unknown epilogue %d", epilogue);
  if (epilogue == TSC_EPI_BIAS_RESIDUAL && N > 0 && (st = validate_residual(dtype, residual)))
    return st;
  if (N > kNoallocMaxRows)
    return fail(TSC_ERR_INVALID, "conv_noalloc: N=%lld exceeds the static scratch limit of %lld "
                                 "rows", (long long)N, (long long)kNoallocMaxRows);
  if (N == 0) return TSC_OK;
  DeviceGuard g(ctx->device);
  // This device's static scratch: looked up (hipGetSymbolAddress, once per device, cached) by the
  // first call on the context, with the device current.
  if (!ctx->sched_scratch && (st = sched_scratch_ptr(ctx->device, &ctx->sched_scratch))) return st;
  // Per-kernel profiling records events (an allocation): off for this call.
  const bool prof = ctx->profile;
  ctx->profile = false;
  ConvArgs a{dtype, feats, weight, bias, nbr, order, N, Ci, Co,
             epilogue == TSC_EPI_BIAS_RESIDUAL ? TSC_EPI_BIAS_RESIDUAL : TSC_EPI_BIAS,
             residual, out};
  a.sched_scratch = ctx->sched_scratch;
  a.sched_scratch_bytes = kSchedScratchBytes;
  const bool ln_pass = set_ln_epilogue(a, epilogue, ln_gamma, ln_beta, eps);
  st = conv_launch(ctx, a);
  if (!st && ln_pass)
    st = layernorm_launch(ctx, dtype, out, N, Co, ln_gamma, ln_beta, eps, 1, out);
  ctx->profile = prof;
  return st;
}

int tsc_layernorm(tsc_ctx* ctx, int32_t dtype, const void* x, int64_t N, int32_t C,
                  const void* gamma, const void* beta, float eps, int32_t apply_silu, void* y) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (!elem_size(dtype)) return fail(TSC_ERR_INVALID, "layernorm: unknown dtype %d", dtype);
  if (N < 0 || C <= 0) return fail(TSC_ERR_INVALID, "layernorm: bad shape N=%lld C=%d", (long long)N, C);
  if (N > 0 && (!x || !y)) return fail(TSC_ERR_INVALID, "layernorm: null buffer");
  if (!(eps >= 0.f)) return fail(TSC_ERR_INVALID, "layernorm: eps must be >= 0");
  DeviceGuard g(ctx->device);
  return layernorm_launch(ctx, dtype, x, N, C, gamma, beta, eps, apply_silu, y);
}

int tsc_silu(tsc_ctx* ctx, int32_t dtype, const void* x, int64_t numel, void* y) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (!elem_size(dtype)) return fail(TSC_ERR_INVALID, "silu: unknown dtype %d", dtype);
  if (numel < 0) return fail(TSC_ERR_INVALID, "silu: negative size");
  if (numel > 0 && (!x || !y)) return fail(TSC_ERR_INVALID, "silu: null buffer");
  DeviceGuard g(ctx->device);
  return silu_launch(ctx, dtype, x, numel, y);
}

int tsc_add(tsc_ctx* ctx, int32_t dtype, const void* a, const void* b, int64_t numel, void* y) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (!elem_size(dtype)) return fail(TSC_ERR_INVALID, "add: unknown dtype %d", dtype);
  if (numel < 0) return fail(TSC_ERR_INVALID, "add: negative size");
  if (numel > 0 && (!a || !b || !y)) return fail(TSC_ERR_INVALID, "add: null buffer");
  DeviceGuard g(ctx->device);
  return add_launch(ctx, dtype, a, b, numel, y);
}

int tsc_resblock(tsc_ctx* ctx, int32_t dtype, const void* x, const int32_t* nbr,
                 const int32_t* order, int64_t N, int32_t C, const void* w1, const void* b1,
                 const void* ln_gamma, const void* ln_beta, float eps, const void* w2,
                 const void* b2, void* out) {
  g_err[0] = 0;
  int st = validate_conv(ctx, dtype, x, w1, b1, nbr, N, C, C, out);
  if (st) return st;
  if (N == 0) return TSC_OK;
  if (!w2) return fail(TSC_ERR_INVALID, "resblock: null w2");
  const int es = elem_size(dtype);
  if (!aligned(w2, es) || (b2 && !aligned(b2, es)) || (ln_gamma && !aligned(ln_gamma, es)) ||
      (ln_beta && !aligned(ln_beta, es)))
    return fail(TSC_ERR_INVALID, "resblock: w2, b2, ln_gamma and ln_beta must be aligned to "
                                 "their element size");
  const size_t rows_bytes = (size_t)N * C * es;
  if (overlaps(x, rows_bytes, out, rows_bytes))
    return fail(TSC_ERR_INVALID, "resblock: out must not overlap x");
  DeviceGuard g(ctx->device);
  void* h;
  st = workspace(ctx, (size_t)N * C * elem_size(dtype), &h);
  if (st) return st;
  // h = silu(LN(conv1(x) + b1));  out = x + conv2(h) + b2
  ConvArgs a1{dtype, x, w1, b1, nbr, order, N, C, C, TSC_EPI_BIAS, nullptr, h};
  const bool ln_pass = set_ln_epilogue(a1, TSC_EPI_BIAS_LN_SILU, ln_gamma, ln_beta, eps);
  st = conv_launch(ctx, a1);
  if (st) return st;
  if (ln_pass) st = layernorm_launch(ctx, dtype, h, N, C, ln_gamma, ln_beta, eps, 1, h);
  if (st) return st;
  ConvArgs a2{dtype, h, w2, b2, nbr, order, N, C, C, TSC_EPI_BIAS_RESIDUAL, x, out};
  return conv_launch(ctx, a2);
}

int tsc_linear(tsc_ctx* ctx, int32_t dtype, const void* x, int64_t N, int32_t Cin,
               const void* weight, const void* bias, const void* residual, int32_t Cout, void* out) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (!elem_size(dtype)) return fail(TSC_ERR_INVALID, "linear: unknown dtype %d", dtype);
  if (N < 0 || Cin <= 0 || Cout <= 0)
    return fail(TSC_ERR_INVALID, "linear: bad shape N=%lld Cin=%d Cout=%d", (long long)N, Cin, Cout);
  if (N > 0 && (!x || !weight || !out)) return fail(TSC_ERR_INVALID, "linear: null buffer");
  const size_t es = (size_t)elem_size(dtype);
  const size_t out_bytes = (size_t)N * Cout * es;
  if (overlaps(x, (size_t)N * Cin * es, out, out_bytes))
    return fail(TSC_ERR_INVALID, "linear: out must not overlap x");
  if (residual && residual != out && overlaps(residual, out_bytes, out, out_bytes))
    return fail(TSC_ERR_INVALID, "linear: residual must be out itself or not overlap it");
  DeviceGuard g(ctx->device);
  return linear_launch(ctx, dtype, x, N, Cin, weight, bias, residual, Cout, out);
}

int tsc_subdivide_count(tsc_ctx* ctx, const uint8_t* keep, int64_t N, int64_t* count) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (N < 0 || !count) return fail(TSC_ERR_INVALID, "subdivide_count: bad arguments");
  if (N > 0 && !keep) return fail(TSC_ERR_INVALID, "subdivide_count: null keep mask");
  DeviceGuard g(ctx->device);
  return subdivide_count_launch(ctx, keep, N, count);
}

int tsc_subdivide(tsc_ctx* ctx, const int32_t* coords, int64_t N, int32_t dtype, const void* feats,
                  int32_t C, const uint8_t* keep, int32_t* coords_out, void* feats_out) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (N < 0) return fail(TSC_ERR_INVALID, "subdivide: negative N");
  if (N == 0) return TSC_OK;
  if (!coords || !coords_out) return fail(TSC_ERR_INVALID, "subdivide: null coordinate buffer");
  if (!aligned(coords, 16) || !aligned(coords_out, 16))
    return fail(TSC_ERR_INVALID, "subdivide: coordinate buffers must be 16-byte aligned");
  int64_t row_bytes = 0;
  if (feats) {
    if (!elem_size(dtype)) return fail(TSC_ERR_INVALID, "subdivide: unknown dtype %d", dtype);
    if (C <= 0) return fail(TSC_ERR_INVALID, "subdivide: C must be positive, got %d", C);
    if (!feats_out) return fail(TSC_ERR_INVALID, "subdivide: null feats_out");
    row_bytes = (int64_t)C * elem_size(dtype);
    if (row_bytes > (int64_t)1 << 20)
      return fail(TSC_ERR_UNSUPPORTED, "subdivide: feature rows above 1 MiB (C=%d)", C);
    const size_t piece = row_bytes % 16 == 0 ? 16 : row_bytes % 4 == 0 ? 4 : 2;
    if (!aligned(feats, piece) || !aligned(feats_out, piece))
      return fail(TSC_ERR_INVALID, "subdivide: feature buffers must be %zu-byte aligned", piece);
  }
  DeviceGuard g(ctx->device);
  return subdivide_launch(ctx, coords, N, feats, row_bytes, keep, coords_out, feats_out);
}

int tsc_attention(tsc_ctx* ctx, int32_t dtype, const void* q, const void* k, const void* v,
                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_kv, int32_t B,
                  int64_t total_q, int64_t total_kv, int32_t num_heads, int32_t head_dim,
                  float scale, int32_t max_seqlen_q, void* out) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (!elem_size(dtype)) return fail(TSC_ERR_INVALID, "attention: unknown dtype %d", dtype);
  if (head_dim != 64 && head_dim != 128)
    return fail(TSC_ERR_UNSUPPORTED, "attention: head_dim %d (64 and 128 are supported)", head_dim);
  if (B < 0 || num_heads <= 0 || num_heads > 65535 || B > 65535 || total_q < 0 || total_kv < 0 ||
      max_seqlen_q < 0 || total_q > INT32_MAX || total_kv > INT32_MAX)
    return fail(TSC_ERR_INVALID, "attention: bad sizes B=%d H=%d total_q=%lld total_kv=%lld", B,
                num_heads, (long long)total_q, (long long)total_kv);
  if (B == 0 || total_q == 0) return TSC_OK;
  if (!q || !out || !cu_seqlens_q || !cu_seqlens_kv || (total_kv > 0 && (!k || !v)))
    return fail(TSC_ERR_INVALID, "attention: null buffer");
  if (!aligned(q, 16) || !aligned(out, 16) || (total_kv > 0 && (!aligned(k, 16) || !aligned(v, 16))))
    return fail(TSC_ERR_INVALID, "attention: q, k, v and out must be 16-byte aligned");
  if (out == q || out == k || out == v) return fail(TSC_ERR_INVALID, "attention: out aliases an input");
  if (!(scale > 0.f)) scale = 1.f / sqrtf((float)head_dim);
  DeviceGuard g(ctx->device);
  return attention_launch(ctx, dtype, q, total_kv > 0 ? k : q, total_kv > 0 ? v : q, cu_seqlens_q,
                          cu_seqlens_kv, B, total_q, total_kv, num_heads, head_dim, scale,
                          max_seqlen_q, out);
}

int tsc_st_open(const char* path, tsc_st** out) {
  g_err[0] = 0;
  if (!path || !out) return fail(TSC_ERR_INVALID, "st_open: null argument");
  *out = nullptr;
  return st_open(path, out);
}

int tsc_st_close(tsc_st* f) {
  g_err[0] = 0;
  if (f) st_close(f);
  return TSC_OK;
}

int tsc_st_counts(tsc_st* f, int64_t* tensors, int64_t* metadata, int64_t* data_offset) {
  g_err[0] = 0;
  if (!f) return fail(TSC_ERR_INVALID, "st_counts: null file");
  st_counts(f, tensors, metadata, data_offset);
  return TSC_OK;
}

int tsc_st_name(tsc_st* f, int64_t index, char* name, int32_t name_len) {
  g_err[0] = 0;
  if (!f) return fail(TSC_ERR_INVALID, "st_name: null file");
  return st_name(f, index, name, name_len);
}

int tsc_st_metadata(tsc_st* f, int64_t index, char* key, int32_t key_len, char* value,
                    int32_t value_len) {
  g_err[0] = 0;
  if (!f) return fail(TSC_ERR_INVALID, "st_metadata: null file");
  return st_metadata(f, index, key, key_len, value, value_len);
}

int tsc_st_info(tsc_st* f, const char* name, int32_t* dtype, int32_t* ndim, int64_t* shape,
                int32_t max_dims, int64_t* offsets) {
  g_err[0] = 0;
  if (!f || !name) return fail(TSC_ERR_INVALID, "st_info: null argument");
  return st_info(f, name, dtype, ndim, shape, max_dims, offsets);
}

int tsc_st_load(tsc_ctx* ctx, tsc_st* f, const char* name, int32_t out_dtype, void* dst) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (!f || !name) return fail(TSC_ERR_INVALID, "st_load: null argument");
  DeviceGuard g(ctx->device);
  return st_load(ctx, f, name, out_dtype, dst);
}

int tsc_profile_enable(tsc_ctx* ctx, int on) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  ctx->profile = on != 0;
  return TSC_OK;
}

int tsc_profile_collect(tsc_ctx* ctx, int* count) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  DeviceGuard g(ctx->device);
  st = check_hip(hipStreamSynchronize(ctx->stream), "profile sync");
  if (st) return st;
  for (auto& r : ctx->prof) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess) continue;
    tsc_prof_agg* a = nullptr;
    for (auto& e : ctx->prof_agg)
      if (e.name == r.name) a = &e;
    if (!a) {
      ctx->prof_agg.push_back({r.name, 0.0, 0});
      a = &ctx->prof_agg.back();
    }
    a->total_ms += ms;
    a->launches += 1;
  }
  prof_clear(ctx);
  if (count) *count = (int)ctx->prof_agg.size();
  return TSC_OK;
}

int tsc_profile_entry(tsc_ctx* ctx, int index, char* name, int name_len, double* total_ms,
                      int64_t* launches) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  if (index < 0 || index >= (int)ctx->prof_agg.size())
    return fail(TSC_ERR_INVALID, "profile_entry: index %d out of range", index);
  const tsc_prof_agg& e = ctx->prof_agg[index];
  if (name && name_len > 0) snprintf(name, (size_t)name_len, "%s", e.name.c_str());
  if (total_ms) *total_ms = e.total_ms;
  if (launches) *launches = e.launches;
  return TSC_OK;
}

int tsc_profile_reset(tsc_ctx* ctx) {
  g_err[0] = 0;
  int st = check_ctx(ctx);
  if (st) return st;
  DeviceGuard g(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  prof_clear(ctx);
  ctx->prof_agg.clear();
  return TSC_OK;
}

}  // extern "C"
