// BF16-weight prefill products on hipBLASLt, the ROCm library's GEMM
// kernels for gfx950: with the weights already bf16 the product is a plain
// bf16 x bf16 -> fp32 GEMM, which the library runs near twice as fast as
// the hand-written matrix-core kernel at the 3B prefill shapes (measured
// 1.1-1.3 PFLOP/s against 0.57). The epilogues stay hand-written kernels.
#include <hipblaslt/hipblaslt.h>

#include <cstdint>
#include <vector>

#include "kernels.h"

namespace {

struct Plan {
  int64_t m, n, k, lda, ldy;
  bool acc;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t ws = 0;
  bool ok = false;
};

}  // namespace

struct BlasLt {
  hipblasLtHandle_t h = nullptr;
  void *ws = nullptr;
  std::vector<Plan> plans;
};

namespace {

constexpr size_t kWorkspace = (size_t)64 << 20;

void destroy_plan(Plan &p) {
  if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
  if (p.lb) hipblasLtMatrixLayoutDestroy(p.lb);
  if (p.lc) hipblasLtMatrixLayoutDestroy(p.lc);
  if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
}

// The library is column-major: y (row-major [M][N], row stride ldy) is the
// column-major N x M matrix D = op(A) * B with A = W (row-major [N][K] is
// column-major K x N, transposed) and B = X (column-major K x M).
bool make_plan(BlasLt &b, Plan &p) {
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, p.k, p.n, p.lda) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16BF, p.k, p.m, p.k) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_32F, p.n, p.m, p.ldy) != HIPBLAS_STATUS_SUCCESS)
    return false;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return false;
  const uint64_t cap = kWorkspace;
  hipblasLtMatmulHeuristicResult_t res[1];
  int got = 0;
  const bool found =
      hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &cap, sizeof(cap)) ==
          HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatmulAlgoGetHeuristic(b.h, p.desc, p.la, p.lb, p.lc, p.lc, pref, 1, res, &got) ==
          HIPBLAS_STATUS_SUCCESS &&
      got > 0 && res[0].state == HIPBLAS_STATUS_SUCCESS && res[0].workspaceSize <= kWorkspace;
  hipblasLtMatmulPreferenceDestroy(pref);
  if (!found) return false;
  p.algo = res[0].algo;
  p.ws = res[0].workspaceSize;
  return true;
}

}  // namespace

BlasLt *blaslt_create() {
  BlasLt *b = new BlasLt;
  if (hipblasLtCreate(&b->h) != HIPBLAS_STATUS_SUCCESS || hipMalloc(&b->ws, kWorkspace) != hipSuccess) {
    blaslt_destroy(b);
    return nullptr;
  }
  return b;
}

void blaslt_destroy(BlasLt *b) {
  if (!b) return;
  for (Plan &p : b->plans) destroy_plan(p);
  if (b->ws) hipFree(b->ws);
  if (b->h) hipblasLtDestroy(b->h);
  delete b;
}

namespace {

// The cached plan of a shape (made on first use; null where the library
// has none).
Plan *find_plan(BlasLt *b, const MatDesc &w, int m, int ldy, bool accumulate) {
  if (!b || w.fmt != FMT_BF16 || m < 1 || w.vstride % 2 || ldy < w.rows) return nullptr;
  const int64_t n = w.rows, k = w.cols, lda = w.vstride / 2;
  for (Plan &q : b->plans)
    if (q.m == m && q.n == n && q.k == k && q.lda == lda && q.ldy == ldy && q.acc == accumulate) return q.ok ? &q : nullptr;
  Plan q;
  q.m = m, q.n = n, q.k = k, q.lda = lda, q.ldy = ldy, q.acc = accumulate;
  q.ok = make_plan(*b, q);
  b->plans.push_back(q);
  return q.ok ? &b->plans.back() : nullptr;
}

}  // namespace

bool blaslt_bf16_ready(BlasLt *b, const MatDesc &w, int m, int ldy) { return find_plan(b, w, m, ldy, false) != nullptr; }

hipError_t blaslt_bf16_product(BlasLt *b, const MatDesc &w, const uint16_t *x, int m, float *y, int ldy,
                               bool accumulate, hipStream_t st) {
  Plan *p = find_plan(b, w, m, ldy, accumulate);
  if (!p) return hipErrorNotSupported;
  const float alpha = 1.f, beta = accumulate ? 1.f : 0.f;
  const hipblasStatus_t s = hipblasLtMatmul(b->h, p->desc, &alpha, w.vals, p->la, x, p->lb, &beta, y, p->lc, y,
                                            p->lc, &p->algo, b->ws, p->ws, st);
  return s == HIPBLAS_STATUS_SUCCESS ? hipSuccess : hipErrorLaunchFailure;
}
