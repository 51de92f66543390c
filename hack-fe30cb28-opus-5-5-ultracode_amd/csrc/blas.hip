// Plain fp16 GEMMs of the step (the frozen projections, forward and backward, after the NF4
// dequant) through rocBLAS's Tensile kernels with an explicitly chosen solution.
//
// The reference runs these as torch matmuls (engine.py:1067-1071, 1160-1185), which pick a
// kernel from a size heuristic. For the step's shapes (a few thousand tokens against 1.5k-18k
// wide weights) the heuristic's choice runs at 0.6-1.0 PFLOP/s while other solutions of the same
// library reach 0.9-1.3; the caller times the candidates once per weight shape and passes the
// winner's index. Solution 0 is rocBLAS's own choice.
//
// Row-major interface, C[M, N] = alpha A[M, K] op(B) + beta C with op = 0: B [N, K] (C = A B^T,
// a forward projection y = x W^T) or op = 1: B [K, N] (C = A B, the input gradient dX = dY W).
// rocBLAS is column-major: the row-major C is the column-major C^T = op(B)^T A^T, so the call
// is m = N, n = M, k = K with B as its first operand.
//
// rocBLAS status codes are returned as kStatusBase + status, so they do not collide with HIP
// error codes; qlora_error_string names both.
#include "common.h"

#define ROCBLAS_BETA_FEATURES_API  // rocblas_gemm_ex_get_solutions
#include <rocblas/rocblas.h>

#include <mutex>

namespace qlora {
namespace blas {

constexpr int kStatusBase = 100000;
constexpr int kMaxDevices = 64;

std::mutex g_mu;
rocblas_handle g_handle[kMaxDevices] = {};

int status(rocblas_status s) { return s == rocblas_status_success ? 0 : kStatusBase + (int)s; }

// The calling thread's current device's handle, created on first use.
int handle_for(rocblas_handle* out) {
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_handle[dev] == nullptr) {
    const int rc = status(rocblas_create_handle(&g_handle[dev]));
    if (rc != 0) {
      g_handle[dev] = nullptr;
      return rc;
    }
  }
  *out = g_handle[dev];
  return 0;
}

struct Problem {
  rocblas_operation ta;
  rocblas_int m, n, k, lda, ldb, ldc;
};

int make_problem(int32_t op, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                 int64_t ldc, Problem* p) {
  QLORA_CHECK_ARG(op == 0 || op == 1);
  QLORA_CHECK_ARG(M > 0 && N > 0 && K > 0);
  QLORA_CHECK_ARG(lda >= K && ldb >= (op == 0 ? K : N) && ldc >= N);
  const int64_t lim = (int64_t)0x7fffffff;
  QLORA_CHECK_ARG(M <= lim && N <= lim && K <= lim && lda <= lim && ldb <= lim && ldc <= lim);
  p->ta = op == 0 ? rocblas_operation_transpose : rocblas_operation_none;
  p->m = (rocblas_int)N;
  p->n = (rocblas_int)M;
  p->k = (rocblas_int)K;
  p->lda = (rocblas_int)ldb;  // rocBLAS's first operand is B
  p->ldb = (rocblas_int)lda;
  p->ldc = (rocblas_int)ldc;
  return 0;
}

}  // namespace blas
}  // namespace qlora

using namespace qlora::blas;

QLORA_API int qlora_gemm(int32_t op, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                         const void* B, int64_t ldb, void* C, int64_t ldc, float alpha,
                         float beta, int32_t solution, void* stream) {
  Problem p;
  int rc = make_problem(op, M, N, K, lda, ldb, ldc, &p);
  if (rc != 0) return rc;
  QLORA_CHECK_ARG(A && B && C && solution >= 0);
  rocblas_handle h;
  if ((rc = handle_for(&h)) != 0) return rc;
  if ((rc = status(rocblas_set_stream(h, (hipStream_t)stream))) != 0) return rc;
  return status(rocblas_gemm_ex(
      h, p.ta, rocblas_operation_none, p.m, p.n, p.k, &alpha, B, rocblas_datatype_f16_r, p.lda, A,
      rocblas_datatype_f16_r, p.ldb, &beta, C, rocblas_datatype_f16_r, p.ldc, C,
      rocblas_datatype_f16_r, p.ldc, rocblas_datatype_f32_r,
      solution > 0 ? rocblas_gemm_algo_solution_index : rocblas_gemm_algo_standard, solution,
      rocblas_gemm_flags_none));
}

// The solution indices rocBLAS can run for this problem: up to `cap` of them into `list`, the
// total count into *count.
QLORA_API int qlora_gemm_solutions(int32_t op, int64_t M, int64_t N, int64_t K, const void* A,
                                   int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
                                   int32_t* list, int32_t cap, int32_t* count) {
  Problem p;
  int rc = make_problem(op, M, N, K, lda, ldb, ldc, &p);
  if (rc != 0) return rc;
  QLORA_CHECK_ARG(A && B && C && count && cap >= 0 && (cap == 0 || list));
  rocblas_handle h;
  if ((rc = handle_for(&h)) != 0) return rc;
  const float alpha = 1.f, beta = 0.f;
  rocblas_int size = 0;
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wdeprecated-declarations"
  rc = status(rocblas_gemm_ex_get_solutions(
      h, p.ta, rocblas_operation_none, p.m, p.n, p.k, &alpha, B, rocblas_datatype_f16_r, p.lda,
      A, rocblas_datatype_f16_r, p.ldb, &beta, C, rocblas_datatype_f16_r, p.ldc, C,
      rocblas_datatype_f16_r, p.ldc, rocblas_datatype_f32_r, rocblas_gemm_algo_solution_index,
      rocblas_gemm_flags_none, nullptr, &size));
  if (rc != 0) return rc;
  *count = size;
  if (cap == 0 || size == 0) return 0;
  rocblas_int n = size < cap ? size : cap;
  rc = status(rocblas_gemm_ex_get_solutions(
      h, p.ta, rocblas_operation_none, p.m, p.n, p.k, &alpha, B, rocblas_datatype_f16_r, p.lda,
      A, rocblas_datatype_f16_r, p.ldb, &beta, C, rocblas_datatype_f16_r, p.ldc, C,
      rocblas_datatype_f16_r, p.ldc, rocblas_datatype_f32_r, rocblas_gemm_algo_solution_index,
      rocblas_gemm_flags_none, list, &n));
#pragma clang diagnostic pop
  return rc;
}
