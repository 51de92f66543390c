// RMSNorm forward with the residual add and the two LoRA-dropout inputs, RMSNorm backward that
// merges the LoRA-dropout gradients, and the keep-mask test hook.
// Reference: rms_fwd_kernel kernels.py:145-175 (_rms_fwd engine.py:947-966), rms_bwd_kernel
// kernels.py:178-205 (_rms_bwd engine.py:969-981), torch_dropout_keep_kernel kernels.py:129-135.
//
// One 64-lane wavefront per row, four rows per workgroup: the row lives in registers (each lane
// holds NV chunks of W consecutive columns), the sums are wavefront reductions (no LDS, no
// barrier). HBM-bound: per row of H columns the forward moves 4H (x) [+2H delta +4H xsum] + 2H
// (y) + 2H (yq) + 2H (yv) bytes and the backward 2H (dy) + 2H (tq) + 2H (tv) + 4H (x) [+4H dres]
// + 4H (dx). The masks are regenerated from (seed, counter) in both directions, never stored.
#include "philox.h"

namespace qlora {

constexpr int kRowsPerBlock = 4;

struct RmsFwdArgs {
  const float* x;
  const uint16_t* delta;  // fp16 [n, H] or null
  const void* w;          // [H], fp32 or fp16
  float* xsum;            // fp32 [n, H] (written when delta)
  uint16_t* y;            // fp16 [n, H] or null
  uint16_t* yq;           // fp16 [n, H] or null
  uint16_t* yv;           // fp16 [n, H] or null
  float* rstd;            // fp32 [n]
  const int64_t* tok;     // padded-batch index of each row (dropout) or null
  int64_t n, H;
  float eps, keep_scale;
  uint64_t ctr_q, ctr_v;
  DropParams drop;
  int w_half;
};

struct RmsBwdArgs {
  const uint16_t* dy;  // fp16, row stride dy_stride
  const uint16_t* tq;  // fp16 [n, H] or null
  const uint16_t* tv;  // fp16 [n, H] or null
  const float* x;
  const float* rstd;
  const void* w;
  const float* dres;  // fp32 [n, H] or null
  float* dx;
  uint16_t* dx16;     // fp16 copy of dx [n, H] or null (the next product's fp16 operand)
  const int64_t* tok;
  int64_t n, H, dy_stride;
  float keep_scale, grad_scale;
  uint64_t ctr_q, ctr_v;
  DropParams drop;
  int w_half;
};

template <int W>
__device__ __forceinline__ void load_f32(const float* p, float (&v)[W]) {
  if constexpr (W == 4) {
    const float4 t = *reinterpret_cast<const float4*>(p);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  } else {
    v[0] = *p;
  }
}
template <int W>
__device__ __forceinline__ void store_f32(float* p, const float (&v)[W]) {
  if constexpr (W == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    *p = v[0];
  }
}
template <int W>
__device__ __forceinline__ void load_h(const uint16_t* p, float (&v)[W]) {
  if constexpr (W == 4) {
    const uint2 t = *reinterpret_cast<const uint2*>(p);
    v[0] = lo_h(t.x); v[1] = hi_h(t.x); v[2] = lo_h(t.y); v[3] = hi_h(t.y);
  } else {
    v[0] = h2f_bits(*p);
  }
}
template <int W>
__device__ __forceinline__ void store_h(uint16_t* p, const float (&v)[W]) {
  if constexpr (W == 4) {
    *reinterpret_cast<uint2*>(p) = make_uint2(pack2h(v[0], v[1]), pack2h(v[2], v[3]));
  } else {
    *p = f2h_bits(v[0]);
  }
}
template <int W>
__device__ __forceinline__ void load_w(const void* w, int w_half, int64_t col, float (&v)[W]) {
  if (w_half)
    load_h<W>(static_cast<const uint16_t*>(w) + col, v);
  else
    load_f32<W>(static_cast<const float*>(w) + col, v);
}
// keep bits of W consecutive elements starting at e0 (4 | e0 when W == 4)
template <int W>
__device__ __forceinline__ uint32_t keep_bits(const DropParams& d, uint64_t e0) {
  if constexpr (W == 4) return drop_keep4(d, e0);
  else return (uint32_t)drop_keep(d, e0);
}

template <int W, int NV>
__global__ __launch_bounds__(kWave* kRowsPerBlock) void rms_fwd_kernel(RmsFwdArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= a.n) return;
  const int64_t base = row * a.H;
  const int64_t chunks = a.H / W;
  float x[NV][W];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = lane + (int64_t)i * kWave;
#pragma unroll
    for (int k = 0; k < W; ++k) x[i][k] = 0.f;
    if (c < chunks) {
      load_f32<W>(a.x + base + c * W, x[i]);
      if (a.delta) {
        float d[W];
        load_h<W>(a.delta + base + c * W, d);
#pragma unroll
        for (int k = 0; k < W; ++k) x[i][k] += d[k];
        store_f32<W>(a.xsum + base + c * W, x[i]);
      }
#pragma unroll
      for (int k = 0; k < W; ++k) ss += x[i][k] * x[i][k];
    }
  }
  ss = wave_sum(ss);
  const float rstd = 1.0f / sqrtf(ss / (float)a.H + a.eps);
  if (lane == 0) a.rstd[row] = rstd;
  const uint64_t tok_e = a.tok ? (uint64_t)a.tok[row] * (uint64_t)a.H : 0;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = lane + (int64_t)i * kWave;
    if (c >= chunks) continue;
    float wv[W], y[W];
    load_w<W>(a.w, a.w_half, c * W, wv);
#pragma unroll
    for (int k = 0; k < W; ++k) y[k] = wv[k] * (x[i][k] * rstd);
    if (a.y) store_h<W>(a.y + base + c * W, y);
    const uint64_t e0 = tok_e + (uint64_t)(c * W);
    if (a.yq) {
      DropParams d = a.drop;
      d.ctr = a.ctr_q;
      const uint32_t keep = keep_bits<W>(d, e0);
      float o[W];
#pragma unroll
      for (int k = 0; k < W; ++k) o[k] = (keep >> k) & 1 ? y[k] * a.keep_scale : 0.f;
      store_h<W>(a.yq + base + c * W, o);
    }
    if (a.yv) {
      DropParams d = a.drop;
      d.ctr = a.ctr_v;
      const uint32_t keep = keep_bits<W>(d, e0);
      float o[W];
#pragma unroll
      for (int k = 0; k < W; ++k) o[k] = (keep >> k) & 1 ? y[k] * a.keep_scale : 0.f;
      store_h<W>(a.yv + base + c * W, o);
    }
  }
}

template <int W, int NV>
__global__ __launch_bounds__(kWave* kRowsPerBlock) void rms_bwd_kernel(RmsBwdArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= a.n) return;
  const int64_t base = row * a.H;
  const int64_t chunks = a.H / W;
  const float rstd = a.rstd[row];
  const uint64_t tok_e = a.tok ? (uint64_t)a.tok[row] * (uint64_t)a.H : 0;
  float g[NV][W], xh[NV][W];
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = lane + (int64_t)i * kWave;
#pragma unroll
    for (int k = 0; k < W; ++k) g[i][k] = xh[i][k] = 0.f;
    if (c >= chunks) continue;
    float dy[W];
    load_h<W>(a.dy + row * a.dy_stride + c * W, dy);
    const uint64_t e0 = tok_e + (uint64_t)(c * W);
    if (a.tq) {
      DropParams d = a.drop;
      d.ctr = a.ctr_q;
      const uint32_t keep = keep_bits<W>(d, e0);
      float t[W];
      load_h<W>(a.tq + base + c * W, t);
#pragma unroll
      for (int k = 0; k < W; ++k) dy[k] += (keep >> k) & 1 ? t[k] * a.keep_scale : 0.f;
    }
    if (a.tv) {
      DropParams d = a.drop;
      d.ctr = a.ctr_v;
      const uint32_t keep = keep_bits<W>(d, e0);
      float t[W];
      load_h<W>(a.tv + base + c * W, t);
#pragma unroll
      for (int k = 0; k < W; ++k) dy[k] += (keep >> k) & 1 ? t[k] * a.keep_scale : 0.f;
    }
    float wv[W], xv[W];
    load_w<W>(a.w, a.w_half, c * W, wv);
    load_f32<W>(a.x + base + c * W, xv);
#pragma unroll
    for (int k = 0; k < W; ++k) {
      g[i][k] = dy[k] * wv[k];
      xh[i][k] = xv[k] * rstd;
      dot += g[i][k] * xh[i][k];
    }
  }
  dot = wave_sum(dot);
  const float mean = dot / (float)a.H;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = lane + (int64_t)i * kWave;
    if (c >= chunks) continue;
    float dx[W];
#pragma unroll
    for (int k = 0; k < W; ++k) dx[k] = rstd * (g[i][k] - xh[i][k] * mean) * a.grad_scale;
    if (a.dres) {
      float r[W];
      load_f32<W>(a.dres + base + c * W, r);
#pragma unroll
      for (int k = 0; k < W; ++k) dx[k] += r[k];
    }
    store_f32<W>(a.dx + base + c * W, dx);
    if (a.dx16) {
#pragma unroll
      for (int k = 0; k < W; ++k) a.dx16[base + c * W + k] = f2h_bits(dx[k]);
    }
  }
}

__global__ void dropout_keep_kernel(int8_t* out, int64_t nelem, DropParams d) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // group of 4 elements
  const int64_t e0 = q * 4;
  if (e0 >= nelem) return;
  const uint32_t bits = drop_keep4(d, (uint64_t)e0);
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (e0 + k < nelem) out[e0 + k] = (int8_t)((bits >> k) & 1);
}

}  // namespace qlora

using namespace qlora;

namespace {

template <int W, int NV>
struct FwdK {
  static void launch(dim3 g, hipStream_t s, const RmsFwdArgs& a) {
    hipLaunchKernelGGL((rms_fwd_kernel<W, NV>), g, dim3(kWave * kRowsPerBlock), 0, s, a);
  }
};
template <int W, int NV>
struct BwdK {
  static void launch(dim3 g, hipStream_t s, const RmsBwdArgs& a) {
    hipLaunchKernelGGL((rms_bwd_kernel<W, NV>), g, dim3(kWave * kRowsPerBlock), 0, s, a);
  }
};

// Smallest register-resident chunk count NV >= need among the compiled variants; 0 if none.
int pick_nv(int64_t need) {
  static const int kNV[] = {1, 2, 3, 4, 5, 6, 7, 8, 12, 16};
  for (int v : kNV)
    if (v >= need) return v;
  return 0;
}

template <template <int, int> class K, int W, class Args>
void launch_nv(int nv, dim3 g, hipStream_t s, const Args& a) {
  switch (nv) {
    case 1: K<W, 1>::launch(g, s, a); break;
    case 2: K<W, 2>::launch(g, s, a); break;
    case 3: K<W, 3>::launch(g, s, a); break;
    case 4: K<W, 4>::launch(g, s, a); break;
    case 5: K<W, 5>::launch(g, s, a); break;
    case 6: K<W, 6>::launch(g, s, a); break;
    case 7: K<W, 7>::launch(g, s, a); break;
    case 8: K<W, 8>::launch(g, s, a); break;
    case 12: K<W, 12>::launch(g, s, a); break;
    default: K<W, 16>::launch(g, s, a); break;
  }
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

DropParams make_drop(int64_t seed, int64_t G, float p_keep, int32_t vec) {
  DropParams d;
  d.seed = (uint64_t)seed;
  d.ctr = 0;
  d.G = (uint64_t)(G > 0 ? G : 1);
  d.p_keep = p_keep;
  d.vec = vec;
  return d;
}

}  // namespace

QLORA_API int qlora_rms_fwd(const float* x, const void* delta, const void* w, int32_t w_half,
                            float* xsum, void* y, void* yq, void* yv, float* rstd,
                            const int64_t* tok, int64_t n, int64_t H, float eps, float p_keep,
                            float keep_scale, int64_t seed, int64_t ctr_q, int64_t ctr_v,
                            int64_t G, int32_t has_delta, int32_t write_y, int32_t drop_q,
                            int32_t drop_v, int32_t vec, void* stream) {
  QLORA_CHECK_ARG(n >= 0 && H > 0);
  if (n == 0) return 0;
  QLORA_CHECK_ARG(x && w && rstd);
  QLORA_CHECK_ARG(!has_delta || (delta && xsum));
  QLORA_CHECK_ARG(!write_y || y);
  QLORA_CHECK_ARG(!drop_q || yq);
  QLORA_CHECK_ARG(!drop_v || yv);
  QLORA_CHECK_ARG(!(drop_q || drop_v) || (tok && (vec == 4 || vec == 8) && G > 0));
  RmsFwdArgs a{x, has_delta ? static_cast<const uint16_t*>(delta) : nullptr, w,
               has_delta ? xsum : nullptr, write_y ? static_cast<uint16_t*>(y) : nullptr,
               drop_q ? static_cast<uint16_t*>(yq) : nullptr,
               drop_v ? static_cast<uint16_t*>(yv) : nullptr, rstd,
               (drop_q || drop_v) ? tok : nullptr, n, H, eps, keep_scale, (uint64_t)ctr_q,
               (uint64_t)ctr_v, make_drop(seed, G, p_keep, vec), w_half};
  const bool v4 = H % 4 == 0 && aligned(x, 16) && aligned(w, w_half ? 8 : 16) &&
                  (!a.delta || aligned(delta, 8)) && (!a.xsum || aligned(xsum, 16)) &&
                  (!a.y || aligned(y, 8)) && (!a.yq || aligned(yq, 8)) &&
                  (!a.yv || aligned(yv, 8));
  const int W = v4 ? 4 : 1;
  const int nv = pick_nv(qlora_cdiv(H / W, kWave));
  QLORA_CHECK_ARG(nv > 0);
  const dim3 grid((unsigned)qlora_cdiv(n, kRowsPerBlock));
  if (v4) launch_nv<FwdK, 4>(nv, grid, (hipStream_t)stream, a);
  else launch_nv<FwdK, 1>(nv, grid, (hipStream_t)stream, a);
  return qlora_launch_status();
}

QLORA_API int qlora_rms_bwd(const void* dy, const void* tq, const void* tv, const float* x,
                            const float* rstd, const void* w, int32_t w_half, const float* dres,
                            float* dx, void* dx16, const int64_t* tok, int64_t n, int64_t H,
                            int64_t dy_stride, float p_keep, float keep_scale, int64_t seed,
                            int64_t ctr_q, int64_t ctr_v, int64_t G, float grad_scale,
                            int32_t drop_q, int32_t drop_v, int32_t has_res, int32_t vec,
                            void* stream) {
  QLORA_CHECK_ARG(n >= 0 && H > 0);
  if (n == 0) return 0;
  QLORA_CHECK_ARG(dy && x && rstd && w && dx && dy_stride >= H);
  QLORA_CHECK_ARG(!drop_q || tq);
  QLORA_CHECK_ARG(!drop_v || tv);
  QLORA_CHECK_ARG(!has_res || dres);
  QLORA_CHECK_ARG(!(drop_q || drop_v) || (tok && (vec == 4 || vec == 8) && G > 0));
  RmsBwdArgs a{static_cast<const uint16_t*>(dy), drop_q ? static_cast<const uint16_t*>(tq)
                                                        : nullptr,
               drop_v ? static_cast<const uint16_t*>(tv) : nullptr, x, rstd, w,
               has_res ? dres : nullptr, dx, static_cast<uint16_t*>(dx16),
               (drop_q || drop_v) ? tok : nullptr, n, H,
               dy_stride, keep_scale, grad_scale, (uint64_t)ctr_q, (uint64_t)ctr_v,
               make_drop(seed, G, p_keep, vec), w_half};
  const bool v4 = H % 4 == 0 && dy_stride % 4 == 0 && aligned(dy, 8) && aligned(x, 16) &&
                  aligned(w, w_half ? 8 : 16) && aligned(dx, 16) &&
                  (!a.tq || aligned(tq, 8)) && (!a.tv || aligned(tv, 8)) &&
                  (!a.dres || aligned(dres, 16));
  const int W = v4 ? 4 : 1;
  const int nv = pick_nv(qlora_cdiv(H / W, kWave));
  QLORA_CHECK_ARG(nv > 0);
  const dim3 grid((unsigned)qlora_cdiv(n, kRowsPerBlock));
  if (v4) launch_nv<BwdK, 4>(nv, grid, (hipStream_t)stream, a);
  else launch_nv<BwdK, 1>(nv, grid, (hipStream_t)stream, a);
  return qlora_launch_status();
}

QLORA_API int qlora_dropout_keep(int8_t* out, int64_t nelem, int64_t seed, int64_t ctr,
                                 int64_t G, float p_keep, int32_t vec, void* stream) {
  QLORA_CHECK_ARG(nelem >= 0);
  if (nelem == 0) return 0;
  QLORA_CHECK_ARG(out && G > 0 && (vec == 4 || vec == 8));
  DropParams d = make_drop(seed, G, p_keep, vec);
  d.ctr = (uint64_t)ctr;
  const int64_t quads = qlora_cdiv(nelem, 4);
  hipLaunchKernelGGL(dropout_keep_kernel, dim3((unsigned)qlora_cdiv(quads, 256)), dim3(256), 0,
                     (hipStream_t)stream, out, nelem, d);
  return qlora_launch_status();
}
