// The same plain fp16 GEMMs as csrc/blas.hip through hipBLASLt, whose Tensile solutions for the
// step's shapes are in places faster than rocBLAS's (gate|up forward and backward by 8-9 %, the
// o projection by 8 %, timed on MI355X), and whose bias epilogue adds the qkv bias before the
// single rounding without a separate fill of the output.
//
// Row-major interface as qlora_gemm: C[M, N] = alpha A[M, K] op(B) (+ bias[N]) + beta C, op = 0:
// B [N, K], op = 1: B [K, N]; hipBLASLt is column-major, so the call is m = N, n = M with B as
// its first operand. A solution is named by the index hipBLASLt stores in the first four bytes
// of its algorithm (the index its own extension API reports); solution 0 is the heuristic's first
// choice. Only algorithms hipBLASLt's heuristic returns for the exact problem are ever run: a
// plan per problem (descriptors and the heuristic's answer, cached) is looked up, and a solution
// missing from it is refused with an error instead of being forced onto the problem. The
// heuristic's full list costs tens of milliseconds of host time per new problem, its first
// choice much less, so a plan holds only the first choice until a listed solution is asked for.
//
// hipBLASLt status codes are returned as 200000 + status.
#include "common.h"

#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

namespace qlora {
namespace lt {

constexpr int kStatusBase = 200000;
constexpr int kMaxDevices = 64;
constexpr int kMaxAlgos = 256;
constexpr size_t kMaxPlans = 1024;  // the cache is cleared when it grows past this

int status(hipblasStatus_t s) { return s == HIPBLAS_STATUS_SUCCESS ? 0 : kStatusBase + (int)s; }

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  std::vector<hipblasLtMatmulHeuristicResult_t> algos;
  bool complete = false;  // algos is the heuristic's whole list (else at most its first choice)
  ~Plan() {
    if (a) hipblasLtMatrixLayoutDestroy(a);
    if (b) hipblasLtMatrixLayoutDestroy(b);
    if (c) hipblasLtMatrixLayoutDestroy(c);
    if (desc) hipblasLtMatmulDescDestroy(desc);
  }
};

using Key = std::tuple<int, int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int,
                       int64_t>;  // device, op, M, N, K, lda, ldb, ldc, bias, workspace

std::mutex g_mu;
hipblasLtHandle_t g_handle[kMaxDevices] = {};
std::map<Key, Plan*> g_plans;

int solution_of(const hipblasLtMatmulAlgo_t& algo) {
  int idx;
  std::memcpy(&idx, algo.data, sizeof(idx));
  return idx;
}

// The heuristic's answer for the plan's problem: its first choice, or (all) its whole list.
int query(hipblasLtHandle_t handle, Plan* p, int64_t ws_bytes, bool all) {
  hipblasLtMatmulPreference_t pref = nullptr;
  int rc = status(hipblasLtMatmulPreferenceCreate(&pref));
  if (rc != 0) return rc;
  const uint64_t wsb = (uint64_t)ws_bytes;
  rc = status(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                    &wsb, sizeof(wsb)));
  std::vector<hipblasLtMatmulHeuristicResult_t> got(all ? kMaxAlgos : 1);
  int n = 0;
  if (rc == 0)
    rc = status(hipblasLtMatmulAlgoGetHeuristic(handle, p->desc, p->a, p->b, p->c, p->c, pref,
                                                (int)got.size(), got.data(), &n));
  hipblasLtMatmulPreferenceDestroy(pref);
  if (rc != 0) return rc;
  got.resize(n > 0 ? std::min<size_t>(n, got.size()) : 0);
  p->algos.clear();
  for (auto& r : got)
    if (r.state == HIPBLAS_STATUS_SUCCESS && r.workspaceSize <= (size_t)ws_bytes)
      p->algos.push_back(r);
  p->complete = all;
  return 0;
}

// The plan of this problem on the current device, built on first use (with the heuristic's
// whole list when `all`). Call with g_mu held.
int plan_for(int32_t op, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
             bool bias, int64_t ws_bytes, bool all, hipblasLtHandle_t* handle, Plan** out) {
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev)) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
  if (g_handle[dev] == nullptr) {
    if (int rc = status(hipblasLtCreate(&g_handle[dev]))) {
      g_handle[dev] = nullptr;
      return rc;
    }
  }
  *handle = g_handle[dev];
  const Key key{dev, op, M, N, K, lda, ldb, ldc, bias ? 1 : 0, ws_bytes};
  auto it = g_plans.find(key);
  if (it != g_plans.end()) {
    if (all && !it->second->complete) {
      if (int rc = query(*handle, it->second, ws_bytes, true)) return rc;
    }
    *out = it->second;
    return 0;
  }
  if (g_plans.size() >= kMaxPlans) {
    for (auto& kv : g_plans) delete kv.second;
    g_plans.clear();
  }
  Plan* p = new Plan();
  int rc = 0;
  const hipblasOperation_t ta = op == 0 ? HIPBLAS_OP_T : HIPBLAS_OP_N, tb = HIPBLAS_OP_N;
  do {
    if ((rc = status(hipblasLtMatmulDescCreate(&p->desc, HIPBLAS_COMPUTE_32F, HIP_R_32F)))) break;
    if ((rc = status(hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta,
                                                     sizeof(ta)))))
      break;
    if ((rc = status(hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb,
                                                     sizeof(tb)))))
      break;
    if (bias) {
      const hipblasLtEpilogue_t epi = HIPBLASLT_EPILOGUE_BIAS;
      const int32_t bt = HIP_R_16F;
      if ((rc = status(hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_EPILOGUE,
                                                       &epi, sizeof(epi)))))
        break;
      if ((rc = status(hipblasLtMatmulDescSetAttribute(
               p->desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)))))
        break;
    }
    // column-major: A := our B (stored K x N for op T, N x K for op N), B := our A (K x M),
    // C = D := our C (N x M)
    if ((rc = status(op == 0 ? hipblasLtMatrixLayoutCreate(&p->a, HIP_R_16F, K, N, ldb)
                             : hipblasLtMatrixLayoutCreate(&p->a, HIP_R_16F, N, K, ldb))))
      break;
    if ((rc = status(hipblasLtMatrixLayoutCreate(&p->b, HIP_R_16F, K, M, lda)))) break;
    if ((rc = status(hipblasLtMatrixLayoutCreate(&p->c, HIP_R_16F, N, M, ldc)))) break;
    rc = query(*handle, p, ws_bytes, all);
  } while (false);
  if (rc != 0) {
    delete p;
    return rc;
  }
  g_plans[key] = p;
  *out = p;
  return 0;
}

int check(int32_t op, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
          int64_t ws_bytes) {
  QLORA_CHECK_ARG(op == 0 || op == 1);
  QLORA_CHECK_ARG(M > 0 && N > 0 && K > 0 && ws_bytes >= 0);
  QLORA_CHECK_ARG(lda >= K && ldb >= (op == 0 ? K : N) && ldc >= N);
  return 0;
}

}  // namespace lt
}  // namespace qlora

using namespace qlora::lt;

// The solution indices hipBLASLt's heuristic offers for this problem (bias: with the bias
// epilogue; workspace limit ws_bytes): up to cap into list, the number into *count.
QLORA_API int qlora_gemmlt_solutions(int32_t op, int64_t M, int64_t N, int64_t K, int64_t lda,
                                     int64_t ldb, int64_t ldc, int32_t bias, int64_t ws_bytes,
                                     int32_t* list, int32_t cap, int32_t* count) {
  if (int rc = check(op, M, N, K, lda, ldb, ldc, ws_bytes)) return rc;
  QLORA_CHECK_ARG(count && cap >= 0 && (cap == 0 || list));
  std::lock_guard<std::mutex> lock(g_mu);
  hipblasLtHandle_t h;
  Plan* p;
  if (int rc = plan_for(op, M, N, K, lda, ldb, ldc, bias != 0, ws_bytes, true, &h, &p)) return rc;
  *count = (int32_t)p->algos.size();
  for (int i = 0; i < cap && i < (int)p->algos.size(); ++i) list[i] = solution_of(p->algos[i].algo);
  return 0;
}

// C = alpha A op(B) (+ bias) + beta C with hipBLASLt solution `solution` (0: the heuristic's first
// choice; else one it lists for this exact problem; otherwise hipErrorInvalidValue and nothing
// runs).
QLORA_API int qlora_gemmlt(int32_t op, int64_t M, int64_t N, int64_t K, const void* A,
                           int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
                           const void* bias, float alpha, float beta, int32_t solution,
                           void* workspace, int64_t ws_bytes, void* stream) {
  if (int rc = check(op, M, N, K, lda, ldb, ldc, ws_bytes)) return rc;
  QLORA_CHECK_ARG(A && B && C && (ws_bytes == 0 || workspace));
  std::lock_guard<std::mutex> lock(g_mu);
  hipblasLtHandle_t h;
  Plan* p;
  if (int rc = plan_for(op, M, N, K, lda, ldb, ldc, bias != nullptr, ws_bytes, solution != 0, &h,
                        &p))
    return rc;
  const hipblasLtMatmulHeuristicResult_t* r = nullptr;
  if (solution == 0) {
    if (!p->algos.empty()) r = &p->algos[0];
  } else {
    for (auto& x : p->algos)
      if (solution_of(x.algo) == solution) {
        r = &x;
        break;
      }
  }
  QLORA_CHECK_ARG(r != nullptr);
  if (bias != nullptr) {
    if (int rc = status(hipblasLtMatmulDescSetAttribute(
            p->desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias))))
      return rc;
  }
  return status(hipblasLtMatmul(h, p->desc, &alpha, B, p->a, A, p->b, &beta, C, p->c, C, p->c,
                                &r->algo, workspace, (size_t)ws_bytes, (hipStream_t)stream));
}
