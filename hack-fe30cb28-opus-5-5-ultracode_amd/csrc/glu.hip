// SwiGLU over the fused [gate | up] projection output, and its backward written in place.
// Reference: glu_fwd_kernel kernels.py:312-321 (_glu_fwd engine.py:1012-1017) and
// glu_bwd_kernel kernels.py:324-336 (_glu_bwd engine.py:1020-1023).
//   m  = fp16( g * sigmoid(g) * u )                               g, u = gu[:, :I], gu[:, I:]
//   gu <- [ fp16(dm * u * s * (1 + g (1 - s))) | fp16(dm * g * s) ]   s = sigmoid(g)
// HBM-bound elementwise: 8 columns per thread (16-byte loads and stores) when I % 8 == 0. The
// sigmoid is 1 / (1 + 2^(-g log2 e)) with the hardware exp2 and reciprocal (v_exp_f32,
// v_rcp_f32, about 1 ulp each in fp32, ahead of the fp16 rounding); with the correctly rounded
// expf and an IEEE division per element, and a 64-bit division for each thread's row, the
// forward issued about 280 instructions per 48 bytes and was bound by them, not by HBM.
#include "common.h"

namespace qlora {

template <int W>
struct VecH;
template <>
struct VecH<8> {
  using T = uint4;
  static __device__ __forceinline__ void unpack(const T w, float (&v)[8]) {
    v[0] = lo_h(w.x); v[1] = hi_h(w.x); v[2] = lo_h(w.y); v[3] = hi_h(w.y);
    v[4] = lo_h(w.z); v[5] = hi_h(w.z); v[6] = lo_h(w.w); v[7] = hi_h(w.w);
  }
  static __device__ __forceinline__ T pack(const float (&v)[8]) {
    return make_uint4(pack2h(v[0], v[1]), pack2h(v[2], v[3]), pack2h(v[4], v[5]),
                      pack2h(v[6], v[7]));
  }
};
template <>
struct VecH<1> {
  using T = uint16_t;
  static __device__ __forceinline__ void unpack(const T w, float (&v)[1]) { v[0] = h2f_bits(w); }
  static __device__ __forceinline__ T pack(const float (&v)[1]) { return f2h_bits(v[0]); }
};

// The thread's row and first column: 32-bit division while the thread count fits (SMALL).
template <bool SMALL>
__device__ __forceinline__ void row_col(int64_t gid, int64_t per_row, int W, int64_t& row,
                                        int64_t& col) {
  if constexpr (SMALL) {
    const uint32_t g = (uint32_t)gid, pr = (uint32_t)per_row, r = g / pr;
    row = r;
    col = (int64_t)(g - r * pr) * W;
  } else {
    row = gid / per_row;
    col = (gid - row * per_row) * W;
  }
}

template <int W, bool SMALL>
__global__ __launch_bounds__(256) void glu_fwd_kernel(const uint16_t* gu, uint16_t* m,
                                                      int64_t n, int64_t I) {
  using V = VecH<W>;
  using T = typename V::T;
  const int64_t per_row = I / W;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n * per_row) return;
  int64_t row, col;
  row_col<SMALL>(gid, per_row, W, row, col);
  const uint16_t* src = gu + row * 2 * I + col;
  float g[W], u[W], o[W];
  V::unpack(*reinterpret_cast<const T*>(src), g);
  V::unpack(*reinterpret_cast<const T*>(src + I), u);
#pragma unroll
  for (int i = 0; i < W; ++i) o[i] = g[i] * sigmoid_fast(g[i]) * u[i];
  *reinterpret_cast<T*>(m + row * I + col) = V::pack(o);
}

template <int W, bool SMALL>
__global__ __launch_bounds__(256) void glu_bwd_kernel(const uint16_t* dm, uint16_t* gu,
                                                      int64_t n, int64_t I) {
  using V = VecH<W>;
  using T = typename V::T;
  const int64_t per_row = I / W;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n * per_row) return;
  int64_t row, col;
  row_col<SMALL>(gid, per_row, W, row, col);
  uint16_t* src = gu + row * 2 * I + col;
  float g[W], u[W], d[W], og[W], ou[W];
  V::unpack(*reinterpret_cast<const T*>(src), g);
  V::unpack(*reinterpret_cast<const T*>(src + I), u);
  V::unpack(*reinterpret_cast<const T*>(dm + row * I + col), d);
#pragma unroll
  for (int i = 0; i < W; ++i) {
    const float s = sigmoid_fast(g[i]);
    og[i] = d[i] * u[i] * s * (1.0f + g[i] * (1.0f - s));
    ou[i] = d[i] * g[i] * s;
  }
  *reinterpret_cast<T*>(src) = V::pack(og);
  *reinterpret_cast<T*>(src + I) = V::pack(ou);
}

}  // namespace qlora

using namespace qlora;

namespace {
bool al(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }
}

QLORA_API int qlora_glu_fwd(const void* gu, void* m, int64_t n, int64_t I, void* stream) {
  QLORA_CHECK_ARG(n >= 0 && I > 0);
  if (n == 0) return 0;
  QLORA_CHECK_ARG(gu && m);
  const bool v8 = I % 8 == 0 && al(gu, 16) && al(m, 16);
  const int W = v8 ? 8 : 1;
  const int64_t total = n * (I / W);
  QLORA_CHECK_ARG(qlora_cdiv(total, 256) < (1ll << 32));
  const dim3 grid((unsigned)qlora_cdiv(total, 256));
  const bool small = qlora_cdiv(total, 256) * 256 <= (int64_t)UINT32_MAX;
  const uint16_t* src = static_cast<const uint16_t*>(gu);
  uint16_t* dst = static_cast<uint16_t*>(m);
  hipStream_t s = (hipStream_t)stream;
  if (v8 && small) hipLaunchKernelGGL((glu_fwd_kernel<8, true>), grid, dim3(256), 0, s, src, dst, n, I);
  else if (v8) hipLaunchKernelGGL((glu_fwd_kernel<8, false>), grid, dim3(256), 0, s, src, dst, n, I);
  else if (small) hipLaunchKernelGGL((glu_fwd_kernel<1, true>), grid, dim3(256), 0, s, src, dst, n, I);
  else hipLaunchKernelGGL((glu_fwd_kernel<1, false>), grid, dim3(256), 0, s, src, dst, n, I);
  return qlora_launch_status();
}

QLORA_API int qlora_glu_bwd(const void* dm, void* gu, int64_t n, int64_t I, void* stream) {
  QLORA_CHECK_ARG(n >= 0 && I > 0);
  if (n == 0) return 0;
  QLORA_CHECK_ARG(gu && dm);
  const bool v8 = I % 8 == 0 && al(gu, 16) && al(dm, 16);
  const int W = v8 ? 8 : 1;
  const int64_t total = n * (I / W);
  QLORA_CHECK_ARG(qlora_cdiv(total, 256) < (1ll << 32));
  const dim3 grid((unsigned)qlora_cdiv(total, 256));
  const bool small = qlora_cdiv(total, 256) * 256 <= (int64_t)UINT32_MAX;
  const uint16_t* d = static_cast<const uint16_t*>(dm);
  uint16_t* x = static_cast<uint16_t*>(gu);
  hipStream_t s = (hipStream_t)stream;
  if (v8 && small) hipLaunchKernelGGL((glu_bwd_kernel<8, true>), grid, dim3(256), 0, s, d, x, n, I);
  else if (v8) hipLaunchKernelGGL((glu_bwd_kernel<8, false>), grid, dim3(256), 0, s, d, x, n, I);
  else if (small) hipLaunchKernelGGL((glu_bwd_kernel<1, true>), grid, dim3(256), 0, s, d, x, n, I);
  else hipLaunchKernelGGL((glu_bwd_kernel<1, false>), grid, dim3(256), 0, s, d, x, n, I);
  return qlora_launch_status();
}

// out = a + fp32(d): the residual add after a projection whose fp16 output d is added to the fp32
// residual stream (engine.py:1048-1051, h3 = h2 + d). 4 elements per thread.
__global__ __launch_bounds__(256) void resid_add_kernel(const float* a, const uint16_t* d,
                                                        float* out, int64_t n4) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  const float4 x = reinterpret_cast<const float4*>(a)[i];
  const uint2 y = reinterpret_cast<const uint2*>(d)[i];
  reinterpret_cast<float4*>(out)[i] =
      make_float4(x.x + lo_h(y.x), x.y + hi_h(y.x), x.z + lo_h(y.y), x.w + hi_h(y.y));
}

QLORA_API int qlora_resid_add(const float* a, const void* d, float* out, int64_t numel,
                              void* stream) {
  QLORA_CHECK_ARG(numel >= 0);
  if (numel == 0) return 0;
  QLORA_CHECK_ARG(a && d && out && numel % 4 == 0);
  QLORA_CHECK_ARG(((uintptr_t)a & 15) == 0 && ((uintptr_t)out & 15) == 0 &&
                  ((uintptr_t)d & 7) == 0);
  const int64_t n4 = numel / 4;
  hipLaunchKernelGGL(resid_add_kernel, dim3((unsigned)qlora_cdiv(n4, 256)), dim3(256), 0,
                     (hipStream_t)stream, a, static_cast<const uint16_t*>(d), out, n4);
  return qlora_launch_status();
}
