// Per-voxel linear layer: out (N,Cout) = x (N,Cin) * W^T + bias (+ residual), W in the
// nn.Linear layout (Cout, Cin).  A plain dense GEMM, so it goes to hipBLASLt (fp32 accumulate),
// with the bias as the library's bias epilogue and the residual as its C matrix (beta = 1): one
// launch writes the block's skip-connected output.  Used by the sparse ConvNeXt block
// (src/models/sparse_unet_vae_decoder.ts:48-78: LN -> Linear -> LN -> SiLU -> Linear + skip) and
// SparseLinear (src/sparse/ops/linear.ts:9-29, where the TS port multiplies by W untransposed).
//
// hipBLASLt is column-major: the row-major (N,Cout) output is the column-major (Cout,N) matrix
// D = op(A) * B with A = W read as (Cin,Cout) column-major and transposed, B = x read as (Cin,N).

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <tuple>

#include "tsc_internal.h"

namespace tsc {
namespace {

constexpr size_t kBlasWorkspace = (size_t)64 << 20;
constexpr int kTuneCandidates = 16;          // heuristic results timed per new shape
constexpr size_t kTuneScratch = (size_t)512 << 20;  // largest tuning output (fewer rows above)

// Fastest algorithm per (dtype, rows timed, Cin, Cout, bias, residual), chosen once per context
// by timing the heuristic's candidates (the library's first pick is up to ~20 % slower on some
// of the ConvNeXt shapes).
using AlgoKey = std::tuple<int32_t, int64_t, int32_t, int32_t, bool, bool>;
using AlgoCache = std::map<AlgoKey, hipblasLtMatmulAlgo_t>;

hipDataType blas_type(int32_t dtype) {
  switch (dtype) {
    case TSC_F16: return HIP_R_16F;
    case TSC_BF16: return HIP_R_16BF;
    default: return HIP_R_32F;
  }
}

int blas_check(hipblasStatus_t s, const char* what) {
  if (s == HIPBLAS_STATUS_SUCCESS) return TSC_OK;
  return fail(TSC_ERR_HIP, "hipBLASLt %s failed (status %d)", what, (int)s);
}

// Destroys the descriptors of one call whatever path returns.
struct BlasCall {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulPreference_t pref = nullptr;
  ~BlasCall() {
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    if (lc) hipblasLtMatrixLayoutDestroy(lc);
    if (lb) hipblasLtMatrixLayoutDestroy(lb);
    if (la) hipblasLtMatrixLayoutDestroy(la);
    if (desc) hipblasLtMatmulDescDestroy(desc);
  }
};

}  // namespace

void blas_destroy(tsc_ctx* ctx) {
  if (ctx->blaslt) hipblasLtDestroy((hipblasLtHandle_t)ctx->blaslt);
  ctx->blaslt = nullptr;
  delete (AlgoCache*)ctx->blas_algos;
  ctx->blas_algos = nullptr;
}

int linear_launch(tsc_ctx* ctx, int32_t dtype, const void* x, int64_t N, int32_t Cin,
                  const void* weight, const void* bias, const void* residual, int32_t Cout,
                  void* out) {
  if (N == 0) return TSC_OK;
  int st;
  if (!ctx->blaslt) {
    hipblasLtHandle_t h;
    st = blas_check(hipblasLtCreate(&h), "create");
    if (st) return st;
    ctx->blaslt = h;
  }
  void* ws;
  st = blas_workspace(ctx, kBlasWorkspace, &ws);
  if (st) return st;
  const hipDataType t = blas_type(dtype);
  BlasCall c;
  st = blas_check(hipblasLtMatmulDescCreate(&c.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F), "desc");
  if (st) return st;
  const int32_t opT = HIPBLAS_OP_T, opN = HIPBLAS_OP_N;
  st = blas_check(hipblasLtMatmulDescSetAttribute(c.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opT,
                                                  sizeof(opT)), "transA");
  if (st) return st;
  st = blas_check(hipblasLtMatmulDescSetAttribute(c.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opN,
                                                  sizeof(opN)), "transB");
  if (st) return st;
  if (bias) {
    const uint32_t epi = HIPBLASLT_EPILOGUE_BIAS;
    const int32_t bt = t;
    st = blas_check(hipblasLtMatmulDescSetAttribute(c.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi,
                                                    sizeof(epi)), "epilogue");
    if (st) return st;
    st = blas_check(hipblasLtMatmulDescSetAttribute(c.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER,
                                                    &bias, sizeof(bias)), "bias");
    if (st) return st;
    st = blas_check(hipblasLtMatmulDescSetAttribute(c.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE,
                                                    &bt, sizeof(bt)), "bias type");
    if (st) return st;
  }
  st = blas_check(hipblasLtMatrixLayoutCreate(&c.la, t, Cin, Cout, Cin), "layout A");
  if (st) return st;
  st = blas_check(hipblasLtMatrixLayoutCreate(&c.lb, t, Cin, N, Cin), "layout B");
  if (st) return st;
  st = blas_check(hipblasLtMatrixLayoutCreate(&c.lc, t, Cout, N, Cout), "layout C/D");
  if (st) return st;
  st = blas_check(hipblasLtMatmulPreferenceCreate(&c.pref), "preference");
  if (st) return st;
  const uint64_t wsb = kBlasWorkspace;
  st = blas_check(hipblasLtMatmulPreferenceSetAttribute(
                      c.pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof(wsb)),
                  "workspace preference");
  if (st) return st;
  const float alpha = 1.f, beta = residual ? 1.f : 0.f;
  const hipblasLtHandle_t lt = (hipblasLtHandle_t)ctx->blaslt;
  if (!ctx->blas_algos) ctx->blas_algos = new AlgoCache();
  AlgoCache& cache = *(AlgoCache*)ctx->blas_algos;
  // Tuning runs write a scratch output (an in-place residual is never accumulated twice), on at
  // most kTuneScratch bytes of rows.
  const size_t esz = dtype == TSC_F32 ? 4 : 2;
  const int64_t nt = std::min<int64_t>(N, std::max<int64_t>(1, (int64_t)(kTuneScratch / (esz * Cout))));
  const AlgoKey key{dtype, nt, Cin, Cout, bias != nullptr, residual != nullptr};
  auto it = cache.find(key);
  if (it == cache.end()) {
    BlasCall tc;  // layouts of the tuning problem (nt rows)
    st = blas_check(hipblasLtMatrixLayoutCreate(&tc.lb, t, Cin, nt, Cin), "layout B (tune)");
    if (st) return st;
    st = blas_check(hipblasLtMatrixLayoutCreate(&tc.lc, t, Cout, nt, Cout), "layout C/D (tune)");
    if (st) return st;
    hipblasLtMatmulHeuristicResult_t res[kTuneCandidates];
    int found = 0;
    st = blas_check(hipblasLtMatmulAlgoGetHeuristic(lt, c.desc, c.la, tc.lb, tc.lc, tc.lc, c.pref,
                                                    kTuneCandidates, res, &found),
                    "heuristic");
    if (st) return st;
    if (found < 1)
      return fail(TSC_ERR_UNSUPPORTED, "linear: no hipBLASLt algorithm for %dx%d", Cin, Cout);
    int best = 0;
    if (found > 1) {
      void* scratch;
      st = workspace(ctx, (size_t)nt * Cout * esz, &scratch);
      if (st) return st;
      hipEvent_t e0, e1;
      st = check_hip(hipEventCreate(&e0), "linear tune event");
      if (st) return st;
      st = check_hip(hipEventCreate(&e1), "linear tune event");
      if (st) {
        (void)hipEventDestroy(e0);
        return st;
      }
      float best_ms = 0.f;
      bool have = false;
      for (int i = 0; i < found; ++i) {
        const void* cin = residual ? residual : scratch;
        auto run = [&] {
          return hipblasLtMatmul(lt, c.desc, &alpha, weight, c.la, x, tc.lb, &beta, cin, tc.lc,
                                 scratch, tc.lc, &res[i].algo, ws, kBlasWorkspace, ctx->stream);
        };
        if (run() != HIPBLAS_STATUS_SUCCESS) continue;  // warm-up; unusable candidates drop out
        (void)hipEventRecord(e0, ctx->stream);
        bool ok = run() == HIPBLAS_STATUS_SUCCESS && run() == HIPBLAS_STATUS_SUCCESS;
        (void)hipEventRecord(e1, ctx->stream);
        float ms = 0.f;
        ok = ok && hipEventSynchronize(e1) == hipSuccess &&
             hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
        if (ok && (!have || ms < best_ms)) {
          best_ms = ms;
          best = i;
          have = true;
        }
      }
      (void)hipEventDestroy(e0);
      (void)hipEventDestroy(e1);
      (void)hipGetLastError();
    }
    it = cache.emplace(key, res[best].algo).first;
  }
  ProfScope p(ctx, "linear");
  if (hipblasLtMatmul(lt, c.desc, &alpha, weight, c.la, x, c.lb, &beta, residual ? residual : out,
                      c.lc, out, c.lc, &it->second, ws, kBlasWorkspace,
                      ctx->stream) == HIPBLAS_STATUS_SUCCESS)
    return TSC_OK;
  // The algorithm was timed on fewer rows and does not take this many: the library's pick.
  (void)hipGetLastError();
  hipblasLtMatmulHeuristicResult_t res;
  int found = 0;
  st = blas_check(hipblasLtMatmulAlgoGetHeuristic(lt, c.desc, c.la, c.lb, c.lc, c.lc, c.pref, 1,
                                                  &res, &found),
                  "heuristic");
  if (st) return st;
  if (found < 1) return fail(TSC_ERR_UNSUPPORTED, "linear: no hipBLASLt algorithm for %dx%d", Cin, Cout);
  return blas_check(hipblasLtMatmul(lt, c.desc, &alpha, weight, c.la, x, c.lb, &beta,
                                    residual ? residual : out, c.lc, out, c.lc, &res.algo, ws,
                                    kBlasWorkspace, ctx->stream),
                    "matmul");
}

}  // namespace tsc
