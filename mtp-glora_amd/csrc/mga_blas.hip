// Plain GEMMs through hipBLASLt (bf16, fp16 or fp32 operands), in row-major terms.
//
//   D[M, N] = op(A)[M, K] * op(B)[K, N] (+ D when accumulate), fp32 compute,
//   op(A) = A ([M, K], row stride lda) or A^T (A stored [K, M]),
//   op(B) = B ([K, N], row stride ldb) or B^T (B stored [N, K]).
//
// hipBLASLt is column-major: a row-major [M, N] matrix with row stride ld is
// the column-major [N, M] matrix with leading dimension ld, so the row-major
// product is issued as D^T = op(B)^T op(A)^T with the operands swapped.
// One handle per device, created on first use; the heuristic's algorithm is
// cached per (device, shape, transposes, strides, accumulate).
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "mga_internal.hpp"

namespace mga {

namespace {

struct AlgoKey {
  int dev, dtype;
  bool ta, tb, acc;
  int64_t m, n, k, lda, ldb, ldd;
  bool operator<(const AlgoKey &o) const {
    return std::tie(dev, dtype, ta, tb, acc, m, n, k, lda, ldb, ldd) <
           std::tie(o.dev, o.dtype, o.ta, o.tb, o.acc, o.m, o.n, o.k, o.lda, o.ldb, o.ldd);
  }
};

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, ld = nullptr;
  hipblasLtMatmulAlgo_t algo;
  size_t ws = 0;
};

std::mutex g_mu;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<AlgoKey, Plan> g_plans;

const char *status_name(hipblasStatus_t s) {
  switch (s) {
    case HIPBLAS_STATUS_SUCCESS: return "success";
    case HIPBLAS_STATUS_NOT_INITIALIZED: return "not initialized";
    case HIPBLAS_STATUS_ALLOC_FAILED: return "alloc failed";
    case HIPBLAS_STATUS_INVALID_VALUE: return "invalid value";
    case HIPBLAS_STATUS_NOT_SUPPORTED: return "not supported";
    case HIPBLAS_STATUS_EXECUTION_FAILED: return "execution failed";
    default: return "error";
  }
}

}  // namespace

int gemm(int dtype, bool ta, bool tb, int64_t M, int64_t N, int64_t K, const void *A, int64_t lda, const void *B,
         int64_t ldb, bool accumulate, void *D, int64_t ldd, void *workspace, size_t ws_bytes, hipStream_t stream,
         const char **err) {
  *err = nullptr;
  const hipDataType dt = dtype == kDtF16 ? HIP_R_16F : (dtype == kDtF32 ? HIP_R_32F : HIP_R_16BF);
  if (M == 0 || N == 0) return 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    *err = "hipGetDevice failed";
    return -1;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  hipblasStatus_t st;
  auto h = g_handles.find(dev);
  if (h == g_handles.end()) {
    hipblasLtHandle_t hd;
    if ((st = hipblasLtCreate(&hd)) != HIPBLAS_STATUS_SUCCESS) {
      *err = status_name(st);
      return -1;
    }
    h = g_handles.emplace(dev, hd).first;
  }
  const AlgoKey key{dev, dtype, ta, tb, accumulate, M, N, K, lda, ldb, ldd};
  auto it = g_plans.find(key);
  if (it == g_plans.end()) {
    Plan p;
    // column-major D^T [N, M] = opA'(B) [N, K] * opB'(A) [K, M]
    hipblasOperation_t opa = tb ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    hipblasOperation_t opb = ta ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    if ((st = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F)) != HIPBLAS_STATUS_SUCCESS ||
        (st = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opa, sizeof(opa))) !=
            HIPBLAS_STATUS_SUCCESS ||
        (st = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opb, sizeof(opb))) !=
            HIPBLAS_STATUS_SUCCESS) {
      *err = status_name(st);
      return -1;
    }
    // stored (column-major) shapes of the swapped operands
    const uint64_t a_rows = tb ? K : N, a_cols = tb ? N : K;   // B buffer
    const uint64_t b_rows = ta ? M : K, b_cols = ta ? K : M;   // A buffer
    if ((st = hipblasLtMatrixLayoutCreate(&p.la, dt, a_rows, a_cols, ldb)) != HIPBLAS_STATUS_SUCCESS ||
        (st = hipblasLtMatrixLayoutCreate(&p.lb, dt, b_rows, b_cols, lda)) != HIPBLAS_STATUS_SUCCESS ||
        (st = hipblasLtMatrixLayoutCreate(&p.ld, dt, N, M, ldd)) != HIPBLAS_STATUS_SUCCESS) {
      *err = status_name(st);
      return -1;
    }
    hipblasLtMatmulPreference_t pref;
    uint64_t max_ws = ws_bytes;
    hipblasLtMatmulPreferenceCreate(&pref);
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &max_ws, sizeof(max_ws));
    hipblasLtMatmulHeuristicResult_t res[1];
    int found = 0;
    st = hipblasLtMatmulAlgoGetHeuristic(h->second, p.desc, p.la, p.lb, p.ld, p.ld, pref, 1, res, &found);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS || found == 0) {
      *err = st != HIPBLAS_STATUS_SUCCESS ? status_name(st) : "no hipBLASLt algorithm for this GEMM";
      return -1;
    }
    p.algo = res[0].algo;
    p.ws = res[0].workspaceSize;
    it = g_plans.emplace(key, p).first;
  }
  const Plan &p = it->second;
  if (p.ws > ws_bytes) {
    *err = "GEMM workspace too small";
    return -1;
  }
  const float alpha = 1.f, beta = accumulate ? 1.f : 0.f;
  st = hipblasLtMatmul(h->second, p.desc, &alpha, B, p.la, A, p.lb, &beta, D, p.ld, D, p.ld, &p.algo, workspace,
                       ws_bytes, stream);
  if (st != HIPBLAS_STATUS_SUCCESS) {
    *err = status_name(st);
    return -1;
  }
  return 0;
}

int gemm_bf16(bool ta, bool tb, int64_t M, int64_t N, int64_t K, const void *A, int64_t lda, const void *B,
              int64_t ldb, bool accumulate, void *D, int64_t ldd, void *workspace, size_t ws_bytes,
              hipStream_t stream, const char **err) {
  return gemm(kDtBf16, ta, tb, M, N, K, A, lda, B, ldb, accumulate, D, ldd, workspace, ws_bytes, stream, err);
}

}  // namespace mga
