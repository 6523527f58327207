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

#include "tsc_internal.h"

namespace tsc {
namespace {

constexpr size_t kBlasWorkspace = (size_t)64 << 20;

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
  hipblasLtMatmulHeuristicResult_t res;
  int found = 0;
  st = blas_check(hipblasLtMatmulAlgoGetHeuristic((hipblasLtHandle_t)ctx->blaslt, c.desc, c.la,
                                                  c.lb, c.lc, c.lc, c.pref, 1, &res, &found),
                  "heuristic");
  if (st) return st;
  if (found < 1) return fail(TSC_ERR_UNSUPPORTED, "linear: no hipBLASLt algorithm for %dx%d", Cin, Cout);
  const float alpha = 1.f, beta = residual ? 1.f : 0.f;
  ProfScope p(ctx, "linear");
  return blas_check(hipblasLtMatmul((hipblasLtHandle_t)ctx->blaslt, c.desc, &alpha, weight, c.la, x,
                                    c.lb, &beta, residual ? residual : out, c.lc, out, c.lc,
                                    &res.algo, ws, kBlasWorkspace, ctx->stream),
                    "matmul");
}

}  // namespace tsc
