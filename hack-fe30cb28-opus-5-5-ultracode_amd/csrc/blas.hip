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
// Split-K (qlora_gemm_splitk): the reduction is cut into `splits` equal slices computed as one
// strided-batched GEMM with fp32 outputs [splits][M][N] (a workspace), then summed in a fixed
// order and rounded once to fp16 (plus an optional bias) by splitk_reduce_kernel - for the
// products whose output is too small to fill the GPU with tiles (long K, narrow N: the
// gate|up input gradient, the lm_head's).
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

namespace qlora {
namespace blas {

// out[m][n] = fp16(sum_j work[j][m][n] (+ bias[n])), four columns per thread (N % 4 == 0).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ work,
                                                            int splits, int64_t M, int64_t N,
                                                            uint16_t* out, int64_t ldc,
                                                            const uint16_t* bias) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= M * N) return;
  const int64_t m = i / N, n = i % N;
  float4 acc = *reinterpret_cast<const float4*>(work + i);
  for (int j = 1; j < splits; ++j) {
    const float4 w = *reinterpret_cast<const float4*>(work + (int64_t)j * M * N + i);
    acc.x += w.x;
    acc.y += w.y;
    acc.z += w.z;
    acc.w += w.w;
  }
  if (bias != nullptr) {
    acc.x += h2f_bits(bias[n]);
    acc.y += h2f_bits(bias[n + 1]);
    acc.z += h2f_bits(bias[n + 2]);
    acc.w += h2f_bits(bias[n + 3]);
  }
  uint2 r;
  r.x = pack2h(acc.x, acc.y);
  r.y = pack2h(acc.z, acc.w);
  *reinterpret_cast<uint2*>(out + m * ldc + n) = r;
}

// out_f32[m][n] = resid[m][n] + f32(fp16(sum_j work[j][m][n])): the split-K sum rounded to fp16
// (the product's own rounding) and added to the fp32 residual stream, as resid_add_kernel adds
// an fp16 product.
__global__ __launch_bounds__(256) void splitk_reduce_resid_kernel(const float* __restrict__ work,
                                                                  int splits, int64_t M,
                                                                  int64_t N,
                                                                  const float* __restrict__ resid,
                                                                  int64_t ldr, float* out,
                                                                  int64_t ldo) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= M * N) return;
  const int64_t m = i / N, n = i % N;
  float4 acc = *reinterpret_cast<const float4*>(work + i);
  for (int j = 1; j < splits; ++j) {
    const float4 w = *reinterpret_cast<const float4*>(work + (int64_t)j * M * N + i);
    acc.x += w.x;
    acc.y += w.y;
    acc.z += w.z;
    acc.w += w.w;
  }
  const float4 r = *reinterpret_cast<const float4*>(resid + m * ldr + n);
  *reinterpret_cast<float4*>(out + m * ldo + n) =
      make_float4(r.x + h2f(f2h(acc.x)), r.y + h2f(f2h(acc.y)), r.z + h2f(f2h(acc.z)),
                  r.w + h2f(f2h(acc.w)));
}

struct Split {
  Problem p;
  rocblas_int kc;                 // K per slice
  rocblas_stride sa, sb, sc;      // rocBLAS strides of its A (our B), B (our A) and C
};

int make_split(int32_t op, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
               int32_t splits, Split* sp) {
  int rc = make_problem(op, M, N, K, lda, ldb, N, &sp->p);
  if (rc != 0) return rc;
  QLORA_CHECK_ARG(splits >= 2 && splits <= 64 && K % (8 * splits) == 0 && N % 4 == 0);
  QLORA_CHECK_ARG(M * N * (int64_t)splits < (1ll << 40));
  const int64_t kc = K / splits;
  sp->kc = (rocblas_int)kc;
  sp->p.k = (rocblas_int)kc;
  sp->sa = op == 0 ? kc : kc * ldb;  // B [N, K]: column slices; B [K, N]: row slices
  sp->sb = kc;                       // A [M, K]: column slices
  sp->sc = M * N;                    // fp32 [M, N] per slice, ld N
  return 0;
}

}  // namespace blas
}  // namespace qlora

// fp16 C[M, N] (ld ldc) = fp16(A op(B) (+ bias)) with the reduction cut into `splits` slices:
// fp32 partial products into work [splits][M][N] (one strided-batched rocBLAS call, solution as
// in qlora_gemm but of the batched fp32-output problem), then one fixed-order sum and rounding.
// Requires K % (8 splits) == 0, N % 4 == 0, work_elems >= splits M N.
namespace {

// The strided-batched fp32-output GEMM of a split: work[j] = A[:, slice j] op(B)[slice j, :].
int splitk_partials(const qlora::blas::Split& sp, int64_t N, const void* A, const void* B,
                    float* work, int32_t splits, int32_t solution, hipStream_t st) {
  using namespace qlora::blas;
  rocblas_handle h;
  int rc;
  if ((rc = handle_for(&h)) != 0) return rc;
  if ((rc = status(rocblas_set_stream(h, st))) != 0) return rc;
  const float alpha = 1.f, beta = 0.f;
  const Problem& p = sp.p;
  return status(rocblas_gemm_strided_batched_ex(
      h, p.ta, rocblas_operation_none, p.m, p.n, p.k, &alpha, B, rocblas_datatype_f16_r, p.lda,
      sp.sa, A, rocblas_datatype_f16_r, p.ldb, sp.sb, &beta, work, rocblas_datatype_f32_r,
      (rocblas_int)N, sp.sc, work, rocblas_datatype_f32_r, (rocblas_int)N, sp.sc, splits,
      rocblas_datatype_f32_r,
      solution > 0 ? rocblas_gemm_algo_solution_index : rocblas_gemm_algo_standard, solution,
      rocblas_gemm_flags_none));
}

}  // namespace

// fp16 C[M, N] (ld ldc) = fp16(A op(B) (+ bias)) with the reduction cut into `splits` slices:
// fp32 partial products into work [splits][M][N] (one strided-batched rocBLAS call, solution as
// in qlora_gemm but of the batched fp32-output problem), then one fixed-order sum and rounding.
// Requires K % (8 splits) == 0, N % 4 == 0, work_elems >= splits M N.
QLORA_API int qlora_gemm_splitk(int32_t op, int64_t M, int64_t N, int64_t K, const void* A,
                                int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
                                const void* bias, int32_t splits, float* work,
                                int64_t work_elems, int32_t solution, void* stream) {
  Split sp;
  int rc = make_split(op, M, N, K, lda, ldb, splits, &sp);
  if (rc != 0) return rc;
  QLORA_CHECK_ARG(A && B && C && work && solution >= 0 && ldc >= N);
  QLORA_CHECK_ARG(work_elems >= M * N * (int64_t)splits);
  QLORA_CHECK_ARG(((uintptr_t)C & 7) == 0 && ldc % 4 == 0 && ((uintptr_t)work & 15) == 0);
  hipStream_t st = (hipStream_t)stream;
  if ((rc = splitk_partials(sp, N, A, B, work, splits, solution, st)) != 0) return rc;
  const int64_t quads = M * N / 4;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)qlora_cdiv(quads, 256)), dim3(256), 0,
                     st, work, splits, M, N, static_cast<uint16_t*>(C), ldc,
                     static_cast<const uint16_t*>(bias));
  return qlora_launch_status();
}

// The same product added to an fp32 residual: out[M, N] (fp32, ld ldo) = resid (fp32, ld ldr) +
// f32(fp16(A op(B))), the sum of the slices rounded once to fp16 and added (out may be resid).
// Requires as qlora_gemm_splitk, and ldr, ldo % 4 == 0, resid and out 16-byte aligned.
QLORA_API int qlora_gemm_splitk_resid(int32_t op, int64_t M, int64_t N, int64_t K, const void* A,
                                      int64_t lda, const void* B, int64_t ldb,
                                      const float* resid, int64_t ldr, float* out, int64_t ldo,
                                      int32_t splits, float* work, int64_t work_elems,
                                      int32_t solution, void* stream) {
  Split sp;
  int rc = make_split(op, M, N, K, lda, ldb, splits, &sp);
  if (rc != 0) return rc;
  QLORA_CHECK_ARG(A && B && resid && out && work && solution >= 0 && ldr >= N && ldo >= N);
  QLORA_CHECK_ARG(work_elems >= M * N * (int64_t)splits);
  QLORA_CHECK_ARG(ldr % 4 == 0 && ldo % 4 == 0 && ((uintptr_t)resid & 15) == 0 &&
                  ((uintptr_t)out & 15) == 0 && ((uintptr_t)work & 15) == 0);
  hipStream_t st = (hipStream_t)stream;
  if ((rc = splitk_partials(sp, N, A, B, work, splits, solution, st)) != 0) return rc;
  const int64_t quads = M * N / 4;
  hipLaunchKernelGGL(splitk_reduce_resid_kernel, dim3((unsigned)qlora_cdiv(quads, 256)),
                     dim3(256), 0, st, work, splits, M, N, resid, ldr, out, ldo);
  return qlora_launch_status();
}

// The solution indices of the strided-batched fp32-output problem of qlora_gemm_splitk.
QLORA_API int qlora_gemm_splitk_solutions(int32_t op, int64_t M, int64_t N, int64_t K,
                                          const void* A, int64_t lda, const void* B, int64_t ldb,
                                          float* work, int32_t splits, int32_t* list, int32_t cap,
                                          int32_t* count) {
  Split sp;
  int rc = make_split(op, M, N, K, lda, ldb, splits, &sp);
  if (rc != 0) return rc;
  QLORA_CHECK_ARG(A && B && work && count && cap >= 0 && (cap == 0 || list));
  rocblas_handle h;
  if ((rc = handle_for(&h)) != 0) return rc;
  const float alpha = 1.f, beta = 0.f;
  const Problem& p = sp.p;
  rocblas_int size = 0;
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wdeprecated-declarations"
  for (int pass = 0; pass < 2; ++pass) {
    rocblas_int* arr = pass == 0 ? nullptr : list;
    rocblas_int n = pass == 0 ? 0 : (size < cap ? size : cap);
    rocblas_int* sz = pass == 0 ? &size : &n;
    rc = status(rocblas_gemm_strided_batched_ex_get_solutions(
        h, p.ta, rocblas_operation_none, p.m, p.n, p.k, &alpha, B, rocblas_datatype_f16_r,
        p.lda, sp.sa, A, rocblas_datatype_f16_r, p.ldb, sp.sb, &beta, work,
        rocblas_datatype_f32_r, (rocblas_int)N, sp.sc, work, rocblas_datatype_f32_r,
        (rocblas_int)N, sp.sc, splits, rocblas_datatype_f32_r, rocblas_gemm_algo_solution_index,
        rocblas_gemm_flags_none, arr, sz));
    if (rc != 0) return rc;
    if (pass == 0) {
      *count = size;
      if (cap == 0 || size == 0) return 0;
    }
  }
#pragma clang diagnostic pop
  return 0;
}
