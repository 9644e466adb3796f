// exl3_dense.cpp -- dense GEMMs through hipBLASLt (see exl3_dense.h).
#include "exl3_dense.h"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>
#include <utility>

namespace exl3 {
namespace {

constexpr size_t kWorkspaceBytes = (size_t)32 << 20;

hipDataType dt_of(int t) {
  return t == DENSE_F16 ? HIP_R_16F : t == DENSE_BF16 ? HIP_R_16BF : HIP_R_32F;
}

using ShapeKey = std::tuple<int, int, int64_t, int64_t, int64_t, int64_t>;

struct Plan {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

struct StreamBlas {
  std::mutex mu;
  hipblasLtHandle_t h = nullptr;
  void *ws = nullptr;
  std::map<ShapeKey, Plan> plans;
};

std::mutex g_mu;
std::map<std::pair<int, hipStream_t>, StreamBlas> g_blas;

StreamBlas *blas_for(hipStream_t s) {
  int dev = 0;
  (void)hipGetDevice(&dev);
  std::lock_guard<std::mutex> g(g_mu);
  return &g_blas[{dev, s}];
}

// Column-major view of the row-major product: Y^T [n, rows] = W^T [n, k] *
// X^T [k, rows], W^T with leading dimension ldw.
hipError_t plan_for(StreamBlas *sb, const ShapeKey &key, Plan **out) {
  auto it = sb->plans.find(key);
  if (it != sb->plans.end()) {
    *out = &it->second;
    return hipSuccess;
  }
  const auto [xdt, ydt, rows, k, n, ldw] = key;
  Plan p;
  bool okay = hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) ==
              HIPBLAS_STATUS_SUCCESS;
  const hipblasOperation_t tn = HIPBLAS_OP_N;
  okay = okay && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &tn,
                                                 sizeof(tn)) == HIPBLAS_STATUS_SUCCESS;
  okay = okay && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tn,
                                                 sizeof(tn)) == HIPBLAS_STATUS_SUCCESS;
  okay = okay && hipblasLtMatrixLayoutCreate(&p.a, dt_of(xdt), (uint64_t)n, (uint64_t)k, ldw) ==
                     HIPBLAS_STATUS_SUCCESS;
  okay = okay && hipblasLtMatrixLayoutCreate(&p.b, dt_of(xdt), (uint64_t)k, (uint64_t)rows, k) ==
                     HIPBLAS_STATUS_SUCCESS;
  okay = okay && hipblasLtMatrixLayoutCreate(&p.d, dt_of(ydt), (uint64_t)n, (uint64_t)rows, n) ==
                     HIPBLAS_STATUS_SUCCESS;
  hipblasLtMatmulPreference_t pref = nullptr;
  okay = okay && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
  const uint64_t wsb = kWorkspaceBytes;
  okay = okay && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                       &wsb, sizeof(wsb)) == HIPBLAS_STATUS_SUCCESS;
  hipblasLtMatmulHeuristicResult_t res[1];
  int found = 0;
  okay = okay && hipblasLtMatmulAlgoGetHeuristic(sb->h, p.op, p.a, p.b, p.d, p.d, pref, 1, res,
                                                 &found) == HIPBLAS_STATUS_SUCCESS;
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  if (!okay || found < 1) {
    if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
    if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
    if (p.d) hipblasLtMatrixLayoutDestroy(p.d);
    if (p.op) hipblasLtMatmulDescDestroy(p.op);
    return hipErrorNotSupported;
  }
  p.algo = res[0].algo;
  *out = &sb->plans.emplace(key, p).first->second;
  return hipSuccess;
}

}  // namespace

hipError_t dense_gemm(const void *x, int xdt, const void *w, int64_t ldw, void *y, int ydt,
                      int64_t rows, int64_t k, int64_t n, hipStream_t s) {
  if (rows <= 0 || k <= 0 || n <= 0 || ldw < n) return hipErrorInvalidValue;
  StreamBlas *sb = blas_for(s);
  std::lock_guard<std::mutex> g(sb->mu);
  if (sb->h == nullptr) {
    if (hipblasLtCreate(&sb->h) != HIPBLAS_STATUS_SUCCESS) {
      sb->h = nullptr;
      return hipErrorNotInitialized;
    }
  }
  if (sb->ws == nullptr) {
    const hipError_t e = hipMalloc(&sb->ws, kWorkspaceBytes);
    if (e != hipSuccess) {
      sb->ws = nullptr;
      return e;
    }
  }
  Plan *p = nullptr;
  const hipError_t e = plan_for(sb, ShapeKey{xdt, ydt, rows, k, n, ldw}, &p);
  if (e != hipSuccess) return e;
  const float alpha = 1.0f, beta = 0.0f;
  const hipblasStatus_t st = hipblasLtMatmul(sb->h, p->op, &alpha, w, p->a, x, p->b, &beta, y, p->d,
                                             y, p->d, &p->algo, sb->ws, kWorkspaceBytes, s);
  return st == HIPBLAS_STATUS_SUCCESS ? hipSuccess : hipErrorLaunchFailure;
}

}  // namespace exl3
