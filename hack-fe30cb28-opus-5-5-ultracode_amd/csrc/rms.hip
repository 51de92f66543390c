// RMSNorm forward with the residual add and the two LoRA-dropout inputs, RMSNorm backward that
// merges the LoRA-dropout gradients, and the keep-mask test hook.
// Reference: rms_fwd_kernel kernels.py:145-175 (_rms_fwd engine.py:947-966), rms_bwd_kernel
// kernels.py:178-205 (_rms_bwd engine.py:969-981), torch_dropout_keep_kernel kernels.py:129-135.
//
// One 64-lane wavefront per row, four rows per workgroup: the row lives in registers (each lane
// holds NV chunks of W consecutive columns), the sums are wavefront reductions (no LDS, no
// barrier). HBM-bound: per row of H columns the forward moves 4H (x) [+2H delta +4H xsum] + 2H
// (y) + 2H (yq) + 2H (yv) bytes and the backward 2H (dy) + 2H (tq) + 2H (tv) + 4H (x) [+4H dres]
// + 4H (dx). The masks come from (seed, counter); the forward may also store them as bits
// (keep: u8 [n][2][ceil(H / 4)], bit k of byte j of mask m = element 4 j + k kept, m = 0 for
// q, 1 for v) for the backward to read instead of drawing them again.
#include "philox.h"

#include <type_traits>

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
  uint8_t* keep;          // u8 [n][2][ceil(H / 4)] keep bits (written when dropping) or null
  const int64_t* ctr_base = nullptr;  // device int64 added to ctr_q / ctr_v, or null
  const uint8_t* keep_in = nullptr;   // keep bits an earlier pass stored: read, not drawn
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
  const uint8_t* keep;  // keep bits stored by the forward, or null: draw them again
  const int64_t* ctr_base = nullptr;  // device int64 added to ctr_q / ctr_v, or null
  // fp16 [n, H] or null: the forward's input was x + f32(xdelta) and its rstd is formed here
  // again (the forward's order of operations, the same bits), rstd then not read
  const uint16_t* xdelta = nullptr;
  float eps = 0.f;
  // fp32 [nparts, n, H] or null: dy = fp16(the parts summed in order), the split-K product's
  // slices (its reduce folded in here); dy is then not read
  const float* dy_parts = nullptr;
  int nparts = 0;
};

// The counter of a mask: the launch's argument plus, when the caller keeps the step's first
// counter on the device (a captured step replayed with fresh masks), that base.
__device__ __forceinline__ uint64_t mask_ctr(uint64_t ctr, const int64_t* base) {
  return base ? ctr + (uint64_t)*base : ctr;
}

// Bytes of one mask of one row in the keep-bit layout.
__host__ __device__ __forceinline__ int64_t keep_row_bytes(int64_t H) { return (H + 3) / 4; }

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
    uint8_t* kr = W == 4 && a.keep ? a.keep + row * 2 * keep_row_bytes(a.H) + c : nullptr;
    // mask m's bits of these W elements from the stored bits (bit k of byte j: element 4 j + k)
    auto stored = [&](int m) -> uint32_t {
      const uint8_t* b = a.keep_in + (row * 2 + m) * keep_row_bytes(a.H);
      return W == 4 ? (uint32_t)b[c] : ((uint32_t)b[(c * W) >> 2] >> ((c * W) & 3)) & 1u;
    };
    if (a.yq) {
      DropParams d = a.drop;
      d.ctr = mask_ctr(a.ctr_q, a.ctr_base);
      const uint32_t keep = a.keep_in ? stored(0) : keep_bits<W>(d, e0);
      float o[W];
#pragma unroll
      for (int k = 0; k < W; ++k) o[k] = (keep >> k) & 1 ? y[k] * a.keep_scale : 0.f;
      store_h<W>(a.yq + base + c * W, o);
      if (kr) kr[0] = (uint8_t)keep;
    }
    if (a.yv) {
      DropParams d = a.drop;
      d.ctr = mask_ctr(a.ctr_v, a.ctr_base);
      const uint32_t keep = a.keep_in ? stored(1) : keep_bits<W>(d, e0);
      float o[W];
#pragma unroll
      for (int k = 0; k < W; ++k) o[k] = (keep >> k) & 1 ? y[k] * a.keep_scale : 0.f;
      store_h<W>(a.yv + base + c * W, o);
      if (kr) kr[keep_row_bytes(a.H)] = (uint8_t)keep;
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
  float xs[NV][W];  // with xdelta: the forward's input x + delta, and rstd formed from it
  float rstd;
  if (a.xdelta) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t c = lane + (int64_t)i * kWave;
#pragma unroll
      for (int k = 0; k < W; ++k) xs[i][k] = 0.f;
      if (c < chunks) {
        float d[W];
        load_f32<W>(a.x + base + c * W, xs[i]);
        load_h<W>(a.xdelta + base + c * W, d);
#pragma unroll
        for (int k = 0; k < W; ++k) xs[i][k] += d[k];
#pragma unroll
        for (int k = 0; k < W; ++k) ss += xs[i][k] * xs[i][k];
      }
    }
    ss = wave_sum(ss);
    rstd = 1.0f / sqrtf(ss / (float)a.H + a.eps);
  } else {
    rstd = a.rstd[row];
  }
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
    if (a.dy_parts) {  // fp16 of the K slices summed in slice order (the reduce's)
      load_f32<W>(a.dy_parts + base + c * W, dy);
      for (int kp = 1; kp < a.nparts; ++kp) {
        float t[W];
        load_f32<W>(a.dy_parts + (int64_t)kp * a.n * a.H + base + c * W, t);
#pragma unroll
        for (int k = 0; k < W; ++k) dy[k] += t[k];
      }
#pragma unroll
      for (int k = 0; k < W; ++k) dy[k] = h2f_bits(f2h_bits(dy[k]));
    } else {
      load_h<W>(a.dy + row * a.dy_stride + c * W, dy);
    }
    const uint64_t e0 = tok_e + (uint64_t)(c * W);
    const uint8_t* kr = W == 4 && a.keep ? a.keep + row * 2 * keep_row_bytes(a.H) + c : nullptr;
    if (a.tq) {
      DropParams d = a.drop;
      d.ctr = mask_ctr(a.ctr_q, a.ctr_base);
      const uint32_t keep = kr ? kr[0] : keep_bits<W>(d, e0);
      float t[W];
      load_h<W>(a.tq + base + c * W, t);
#pragma unroll
      for (int k = 0; k < W; ++k) dy[k] += (keep >> k) & 1 ? t[k] * a.keep_scale : 0.f;
    }
    if (a.tv) {
      DropParams d = a.drop;
      d.ctr = mask_ctr(a.ctr_v, a.ctr_base);
      const uint32_t keep = kr ? kr[keep_row_bytes(a.H)] : keep_bits<W>(d, e0);
      float t[W];
      load_h<W>(a.tv + base + c * W, t);
#pragma unroll
      for (int k = 0; k < W; ++k) dy[k] += (keep >> k) & 1 ? t[k] * a.keep_scale : 0.f;
    }
    float wv[W], xv[W];
    load_w<W>(a.w, a.w_half, c * W, wv);
    if (a.xdelta) {
#pragma unroll
      for (int k = 0; k < W; ++k) xv[k] = xs[i][k];
    } else {
      load_f32<W>(a.x + base + c * W, xv);
    }
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

// ---- rows of H = 256 NV columns: every lane holds NV chunks of 4 (no bounds tests), and all
// of a row's loads are issued before the first use of any of them (a load whose result feeds
// the next instruction, or one behind a per-lane branch, makes the wavefront wait for it
// before issuing the next: the generic kernels above pay a full memory round trip per chunk).
// Dropout element indices (token * H + column) are below 2^32 (checked on the host).
__device__ __forceinline__ float4 h4(uint2 t) {
  return make_float4(lo_h(t.x), hi_h(t.x), lo_h(t.y), hi_h(t.y));
}
__device__ __forceinline__ uint2 pack4(float a, float b, float c, float d) {
  return make_uint2(pack2h(a, b), pack2h(c, d));
}
__device__ __forceinline__ float comp(const float4& v, int k) {
  return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}

// weights of the lane's NV chunks as fp32 (fp32 or fp16 storage)
template <int NV>
__device__ __forceinline__ void load_w4(const void* w, int w_half, int lane, float4 (&wv)[NV]) {
  if (w_half) {
    uint2 t[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i)
      t[i] = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(w) + 4 * (lane + 64 * i));
#pragma unroll
    for (int i = 0; i < NV; ++i) wv[i] = h4(t[i]);
  } else {
#pragma unroll
    for (int i = 0; i < NV; ++i)
      wv[i] = *reinterpret_cast<const float4*>(static_cast<const float*>(w) + 4 * (lane + 64 * i));
  }
}

template <int NV, bool DELTA, bool DROP>
__global__ __launch_bounds__(kWave* kRowsPerBlock) void rms_fwd4_kernel(RmsFwdArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  // wave-uniform row: its token index and rstd go through scalar loads, which the vector
  // loads' counter does not hold up
  const int64_t row =
      (int64_t)blockIdx.x * kRowsPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= a.n) return;
  const int64_t base = row * a.H;
  const uint32_t tok_e = DROP ? (uint32_t)a.tok[row] * (uint32_t)a.H : 0u;
  float4 x[NV];
  uint2 dr[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t off = base + 4 * (lane + 64 * i);
    x[i] = *reinterpret_cast<const float4*>(a.x + off);
    if constexpr (DELTA) dr[i] = *reinterpret_cast<const uint2*>(a.delta + off);
  }
  float4 wv[NV];
  load_w4<NV>(a.w, a.w_half, lane, wv);
  uint32_t kq[NV], kv[NV];
  if (DROP && a.keep_in) {  // the masks an earlier pass stored as bits (a recompute)
    const int64_t kb = a.H / 4;
    const uint8_t* kr = a.keep_in + row * 2 * kb;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      kq[i] = a.yq ? (uint32_t)kr[lane + 64 * i] : 0u;
      kv[i] = a.yv ? (uint32_t)kr[kb + lane + 64 * i] : 0u;
    }
  } else if constexpr (DROP) {  // the masks, while the loads are in flight (p = 0: all kept)
    const uint32_t G32 = (uint32_t)a.drop.G;
    const int vs = a.drop.vec == 8 ? 3 : 2;
    const bool all = a.drop.p_keep >= 1.0f;
    DropParams dq = a.drop, dv = a.drop;
    dq.ctr = mask_ctr(a.ctr_q, a.ctr_base);
    dv.ctr = mask_ctr(a.ctr_v, a.ctr_base);
    // element groups of the lane's NV quads, g0 + step i: one division for both masks and
    // every quad (a launch over at least one row has G >= 256 NV > step (NV - 1) threads, so
    // the thread index wraps at most once; the loop also takes any smaller G)
    const uint32_t e_first = tok_e + 4u * (uint32_t)lane;
    const uint32_t g0 = e_first >> vs, step = 64u >> (vs - 2);
    const uint32_t sub = (e_first & ((1u << vs) - 1)) >> 2;
    uint32_t it = g0 / G32, th = g0 - it * G32;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      kq[i] = !a.yq ? 0u : all ? 0xFu : drop_keep4_at(dq, it, th, vs, sub);
      kv[i] = !a.yv ? 0u : all ? 0xFu : drop_keep4_at(dv, it, th, vs, sub);
      th += step;
      while (th >= G32) {
        th -= G32;
        ++it;
      }
    }
    if (a.keep) {
      const int64_t kb = a.H / 4;
      uint8_t* kr = a.keep + row * 2 * kb;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        if (a.yq) kr[lane + 64 * i] = (uint8_t)kq[i];
        if (a.yv) kr[kb + lane + 64 * i] = (uint8_t)kv[i];
      }
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if constexpr (DELTA) {
      const float4 d = h4(dr[i]);
      x[i].x += d.x;
      x[i].y += d.y;
      x[i].z += d.z;
      x[i].w += d.w;
      *reinterpret_cast<float4*>(a.xsum + base + 4 * (lane + 64 * i)) = x[i];
    }
    ss += x[i].x * x[i].x;  // the generic kernel's order of additions
    ss += x[i].y * x[i].y;
    ss += x[i].z * x[i].z;
    ss += x[i].w * x[i].w;
  }
  ss = wave_sum(ss);
  const float rstd = 1.0f / sqrtf(ss / (float)a.H + a.eps);
  if (lane == 0) a.rstd[row] = rstd;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t off = base + 4 * (lane + 64 * i);
    const float4 y = make_float4(wv[i].x * (x[i].x * rstd), wv[i].y * (x[i].y * rstd),
                                 wv[i].z * (x[i].z * rstd), wv[i].w * (x[i].w * rstd));
    if (a.y) *reinterpret_cast<uint2*>(a.y + off) = pack4(y.x, y.y, y.z, y.w);
    if constexpr (DROP) {
      uint16_t* outs[2] = {a.yq, a.yv};
      const uint32_t keeps[2] = {kq[i], kv[i]};
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (outs[t] == nullptr) continue;
        const uint32_t keep = keeps[t];
        float o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = (keep >> k) & 1 ? comp(y, k) * a.keep_scale : 0.f;
        *reinterpret_cast<uint2*>(outs[t] + off) = pack4(o[0], o[1], o[2], o[3]);
      }
    }
  }
}

template <int NV, bool DROP, bool RES, bool XD = false, bool PARTS = false>
__global__ __launch_bounds__(kWave* kRowsPerBlock) void rms_bwd4_kernel(RmsBwdArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row =  // wave-uniform, as the forward
      (int64_t)blockIdx.x * kRowsPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= a.n) return;
  const int64_t base = row * a.H;
  const uint32_t tok_e = DROP && !a.keep ? (uint32_t)a.tok[row] * (uint32_t)a.H : 0u;
  uint2 dyr[NV], tqr[NV], tvr[NV], xdr[NV];
  float4 x[NV], r[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t col = 4 * (lane + 64 * i);
    if constexpr (!PARTS) dyr[i] = *reinterpret_cast<const uint2*>(a.dy + row * a.dy_stride + col);
    x[i] = *reinterpret_cast<const float4*>(a.x + base + col);
    if constexpr (XD) xdr[i] = *reinterpret_cast<const uint2*>(a.xdelta + base + col);
    if constexpr (DROP) {
      tqr[i] = *reinterpret_cast<const uint2*>(a.tq + base + col);
      tvr[i] = *reinterpret_cast<const uint2*>(a.tv + base + col);
    }
    if constexpr (RES) r[i] = *reinterpret_cast<const float4*>(a.dres + base + col);
  }
  if constexpr (PARTS) {  // dy = fp16 of the K slices summed in slice order (the reduce's)
    float4 ps[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i)
      ps[i] = *reinterpret_cast<const float4*>(a.dy_parts + base + 4 * (lane + 64 * i));
    for (int k = 1; k < a.nparts; ++k) {
      const float* pk = a.dy_parts + (int64_t)k * a.n * a.H + base;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const float4 t = *reinterpret_cast<const float4*>(pk + 4 * (lane + 64 * i));
        ps[i].x += t.x; ps[i].y += t.y; ps[i].z += t.z; ps[i].w += t.w;
      }
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) dyr[i] = pack4(ps[i].x, ps[i].y, ps[i].z, ps[i].w);
  }
  float4 wv[NV];
  load_w4<NV>(a.w, a.w_half, lane, wv);
  float rstd;
  if constexpr (XD) {  // the forward's x += delta and rstd, in its order of operations
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const float4 d = h4(xdr[i]);
      x[i].x += d.x;
      x[i].y += d.y;
      x[i].z += d.z;
      x[i].w += d.w;
      ss += x[i].x * x[i].x;
      ss += x[i].y * x[i].y;
      ss += x[i].z * x[i].z;
      ss += x[i].w * x[i].w;
    }
    ss = wave_sum(ss);
    rstd = 1.0f / sqrtf(ss / (float)a.H + a.eps);
  } else {
    rstd = a.rstd[row];
  }
  uint32_t kq[NV], kv[NV];
  if (DROP && a.keep) {  // the forward's masks
    const int64_t kb = a.H / 4;
    const uint8_t* kr = a.keep + row * 2 * kb;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      kq[i] = kr[lane + 64 * i];
      kv[i] = kr[kb + lane + 64 * i];
    }
  } else if constexpr (DROP) {  // the masks, while the loads are in flight (p = 0: all kept)
    const uint32_t G32 = (uint32_t)a.drop.G;
    const int vs = a.drop.vec == 8 ? 3 : 2;
    const bool all = a.drop.p_keep >= 1.0f;
    DropParams dq = a.drop, dv = a.drop;
    dq.ctr = mask_ctr(a.ctr_q, a.ctr_base);
    dv.ctr = mask_ctr(a.ctr_v, a.ctr_base);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t e0 = tok_e + 4u * (uint32_t)(lane + 64 * i);
      kq[i] = all ? 0xFu : drop_keep4_u32(dq, e0, G32, vs);
      kv[i] = all ? 0xFu : drop_keep4_u32(dv, e0, G32, vs);
    }
  }
  float g[NV][4], xh[NV][4];
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const float4 dy = h4(dyr[i]);
    float d[4] = {dy.x, dy.y, dy.z, dy.w};
    if constexpr (DROP) {
      const float4 q = h4(tqr[i]), v = h4(tvr[i]);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        d[k] += (kq[i] >> k) & 1 ? comp(q, k) * a.keep_scale : 0.f;
        d[k] += (kv[i] >> k) & 1 ? comp(v, k) * a.keep_scale : 0.f;
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      g[i][k] = d[k] * comp(wv[i], k);
      xh[i][k] = comp(x[i], k) * rstd;
      dot += g[i][k] * xh[i][k];
    }
  }
  dot = wave_sum(dot);
  const float mean = dot / (float)a.H;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t off = base + 4 * (lane + 64 * i);
    float dx[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      dx[k] = rstd * (g[i][k] - xh[i][k] * mean) * a.grad_scale;
      if constexpr (RES) dx[k] += comp(r[i], k);
    }
    *reinterpret_cast<float4*>(a.dx + off) = make_float4(dx[0], dx[1], dx[2], dx[3]);
    if (a.dx16) *reinterpret_cast<uint2*>(a.dx16 + off) = pack4(dx[0], dx[1], dx[2], dx[3]);
  }
}

// Keep bits of the rows [n, H] in the keep-bit layout, element by element (the forward's
// one-column path, which holds single elements per lane). One thread per byte of each mask.
__global__ void rms_keep_bits_kernel(uint8_t* keep, const int64_t* tok, int64_t n, int64_t H,
                                     DropParams d, uint64_t ctr_q, uint64_t ctr_v,
                                     const int64_t* ctr_base, int has_q, int has_v) {
  const int64_t kb = keep_row_bytes(H);
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (row, mask, byte)
  if (i >= n * 2 * kb) return;
  const int64_t row = i / (2 * kb), m = (i / kb) % 2, j = i % kb;
  if (!(m == 0 ? has_q : has_v)) return;
  d.ctr = mask_ctr(m == 0 ? ctr_q : ctr_v, ctr_base);
  const uint64_t e = (uint64_t)tok[row] * (uint64_t)H + 4 * j;
  uint32_t bits = 0;
  for (int k = 0; k < 4 && 4 * j + k < H; ++k) bits |= (uint32_t)drop_keep(d, e + k) << k;
  keep[i] = (uint8_t)bits;
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

// The fast kernels' NV (H = 256 NV); 0: use the generic kernels.
int fast_nv(int64_t H) {
  if (H % 256) return 0;
  const int64_t nv = H / 256;
  return (nv <= 8 || nv == 12 || nv == 14 || nv == 16) ? (int)nv : 0;
}

template <int NV>
void fwd4_launch(dim3 g, hipStream_t s, const RmsFwdArgs& a, bool delta, bool drop) {
  const dim3 b(kWave * kRowsPerBlock);
  if (delta && drop) hipLaunchKernelGGL((rms_fwd4_kernel<NV, true, true>), g, b, 0, s, a);
  else if (delta) hipLaunchKernelGGL((rms_fwd4_kernel<NV, true, false>), g, b, 0, s, a);
  else if (drop) hipLaunchKernelGGL((rms_fwd4_kernel<NV, false, true>), g, b, 0, s, a);
  else hipLaunchKernelGGL((rms_fwd4_kernel<NV, false, false>), g, b, 0, s, a);
}
template <int NV>
void bwd4_launch(dim3 g, hipStream_t s, const RmsBwdArgs& a, bool drop, bool res) {
  const dim3 b(kWave * kRowsPerBlock);
  // dy from split-K slices (the post-attention norm's backward: no dropout)
  if (a.dy_parts && !drop) {
    if (a.xdelta && res)
      hipLaunchKernelGGL((rms_bwd4_kernel<NV, false, true, true, true>), g, b, 0, s, a);
    else if (a.xdelta)
      hipLaunchKernelGGL((rms_bwd4_kernel<NV, false, false, true, true>), g, b, 0, s, a);
    else if (res)
      hipLaunchKernelGGL((rms_bwd4_kernel<NV, false, true, false, true>), g, b, 0, s, a);
    else
      hipLaunchKernelGGL((rms_bwd4_kernel<NV, false, false, false, true>), g, b, 0, s, a);
    return;
  }
  // the input x + xdelta (the post-attention norm's backward after a recompute)
  if (a.xdelta && !drop && res)
    hipLaunchKernelGGL((rms_bwd4_kernel<NV, false, true, true>), g, b, 0, s, a);
  else if (a.xdelta && !drop)
    hipLaunchKernelGGL((rms_bwd4_kernel<NV, false, false, true>), g, b, 0, s, a);
  else if (a.xdelta && res)
    hipLaunchKernelGGL((rms_bwd4_kernel<NV, true, true, true>), g, b, 0, s, a);
  else if (a.xdelta)
    hipLaunchKernelGGL((rms_bwd4_kernel<NV, true, false, true>), g, b, 0, s, a);
  else if (drop && res) hipLaunchKernelGGL((rms_bwd4_kernel<NV, true, true>), g, b, 0, s, a);
  else if (drop) hipLaunchKernelGGL((rms_bwd4_kernel<NV, true, false>), g, b, 0, s, a);
  else if (res) hipLaunchKernelGGL((rms_bwd4_kernel<NV, false, true>), g, b, 0, s, a);
  else hipLaunchKernelGGL((rms_bwd4_kernel<NV, false, false>), g, b, 0, s, a);
}

template <class F>
void by_nv(int nv, F&& f) {
  switch (nv) {
    case 1: f(std::integral_constant<int, 1>()); break;
    case 2: f(std::integral_constant<int, 2>()); break;
    case 3: f(std::integral_constant<int, 3>()); break;
    case 4: f(std::integral_constant<int, 4>()); break;
    case 5: f(std::integral_constant<int, 5>()); break;
    case 6: f(std::integral_constant<int, 6>()); break;
    case 7: f(std::integral_constant<int, 7>()); break;
    case 8: f(std::integral_constant<int, 8>()); break;
    case 12: f(std::integral_constant<int, 12>()); break;
    case 14: f(std::integral_constant<int, 14>()); break;
    default: f(std::integral_constant<int, 16>()); break;
  }
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

// The smallest Philox word r whose uniform 2^-32 + r 2^-32 (fp32, as the kernels and rocRAND's
// uniform map form it) is not below p_keep: the words below it are kept. The map is
// non-decreasing in r (the conversion rounds to nearest, the product is exact), so a binary
// search over [0, 2^32) finds it. 0 keeps nothing (p_keep <= 2^-32, or NaN); p_keep >= 1 keeps
// every word through the kernels' own test.
uint32_t keep_below(float p_keep) {
  const float inv = 0x1p-32f;
  auto u = [inv](uint64_t r) { return inv + (float)(uint32_t)r * inv; };
  if (!(p_keep > u(0))) return 0u;
  if (p_keep >= 1.0f) return 0xFFFFFFFFu;
  uint64_t lo = 0, hi = 0xFFFFFFFFull;  // u(lo) < p_keep <= u(hi) = 1
  while (hi - lo > 1) {
    const uint64_t mid = (lo + hi) / 2;
    (u(mid) < p_keep ? lo : hi) = mid;
  }
  return (uint32_t)hi;
}

DropParams make_drop(int64_t seed, int64_t G, float p_keep, int32_t vec) {
  DropParams d;
  d.seed = (uint64_t)seed;
  d.ctr = 0;
  d.G = (uint64_t)(G > 0 ? G : 1);
  d.p_keep = p_keep;
  d.vec = vec;
  d.keep_below = keep_below(p_keep);
  return d;
}

}  // namespace

QLORA_API int qlora_dropout_keep_below(float p_keep, uint32_t* out) {
  QLORA_CHECK_ARG(out);
  *out = keep_below(p_keep);
  return 0;
}

QLORA_API int qlora_rms_fwd(const float* x, const void* delta, const void* w, int32_t w_half,
                            float* xsum, void* y, void* yq, void* yv, float* rstd,
                            const int64_t* tok, int64_t n, int64_t H, float eps, float p_keep,
                            float keep_scale, int64_t seed, int64_t ctr_q, int64_t ctr_v,
                            int64_t G, int32_t has_delta, int32_t write_y, int32_t drop_q,
                            int32_t drop_v, int32_t vec, uint8_t* keep,
                            const uint8_t* keep_in, const int64_t* ctr_base, void* stream) {
  QLORA_CHECK_ARG(n >= 0 && H > 0);
  if (n == 0) return 0;
  QLORA_CHECK_ARG(x && w && rstd);
  QLORA_CHECK_ARG(!(keep && keep_in) && (!keep_in || drop_q || drop_v));
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
  a.keep = drop_q || drop_v ? keep : nullptr;
  a.keep_in = keep_in;
  a.ctr_base = ctr_base;
  const bool v4 = H % 4 == 0 && aligned(x, 16) && aligned(w, w_half ? 8 : 16) &&
                  (!a.delta || aligned(delta, 8)) && (!a.xsum || aligned(xsum, 16)) &&
                  (!a.y || aligned(y, 8)) && (!a.yq || aligned(yq, 8)) &&
                  (!a.yv || aligned(yv, 8));
  const int W = v4 ? 4 : 1;
  const int nv = pick_nv(qlora_cdiv(H / W, kWave));
  QLORA_CHECK_ARG(nv > 0);
  const dim3 grid((unsigned)qlora_cdiv(n, kRowsPerBlock));
  const int fnv = v4 ? fast_nv(H) : 0;
  if (fnv > 0) {
    const bool delta = a.delta != nullptr, drop = a.yq != nullptr || a.yv != nullptr;
    by_nv(fnv, [&](auto k) { fwd4_launch<decltype(k)::value>(grid, (hipStream_t)stream, a,
                                                                delta, drop); });
  } else if (v4) {
    launch_nv<FwdK, 4>(nv, grid, (hipStream_t)stream, a);
  } else {
    launch_nv<FwdK, 1>(nv, grid, (hipStream_t)stream, a);
    if (a.keep) {  // the one-column kernel holds single elements: the bits in a pass of their own
      if (int rc = qlora_launch_status()) return rc;
      const int64_t total = n * 2 * keep_row_bytes(H);
      QLORA_CHECK_ARG(qlora_cdiv(total, 256) < (1ll << 31));
      hipLaunchKernelGGL(rms_keep_bits_kernel, dim3((unsigned)qlora_cdiv(total, 256)), dim3(256),
                         0, (hipStream_t)stream, a.keep, tok, n, H, a.drop, a.ctr_q, a.ctr_v,
                         a.ctr_base, drop_q ? 1 : 0, drop_v ? 1 : 0);
    }
  }
  return qlora_launch_status();
}

QLORA_API int qlora_rms_bwd(const void* dy, const void* tq, const void* tv, const float* x,
                            const float* rstd, const void* w, int32_t w_half, const float* dres,
                            float* dx, void* dx16, const int64_t* tok, int64_t n, int64_t H,
                            int64_t dy_stride, float p_keep, float keep_scale, int64_t seed,
                            int64_t ctr_q, int64_t ctr_v, int64_t G, float grad_scale,
                            int32_t drop_q, int32_t drop_v, int32_t has_res, int32_t vec,
                            const uint8_t* keep, const int64_t* ctr_base, const void* xdelta,
                            float eps, const float* dy_parts, int32_t nparts, void* stream) {
  QLORA_CHECK_ARG(n >= 0 && H > 0);
  if (n == 0) return 0;
  QLORA_CHECK_ARG((dy || dy_parts) && x && (rstd || xdelta) && w && dx && dy_stride >= H);
  QLORA_CHECK_ARG(!dy_parts || (nparts >= 1 && nparts <= 16 && !drop_q && !drop_v));
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
  a.keep = drop_q || drop_v ? keep : nullptr;  // the one-column kernel draws the masks again
  a.ctr_base = ctr_base;
  a.xdelta = static_cast<const uint16_t*>(xdelta);
  a.eps = eps;
  a.dy_parts = dy_parts;
  a.nparts = dy_parts ? nparts : 0;
  const bool v4 = H % 4 == 0 && dy_stride % 4 == 0 && (dy_parts ? aligned(dy_parts, 16)
                                                                 : aligned(dy, 8)) &&
                  aligned(x, 16) &&
                  (!xdelta || aligned(xdelta, 8)) &&
                  aligned(w, w_half ? 8 : 16) && aligned(dx, 16) &&
                  (!a.tq || aligned(tq, 8)) && (!a.tv || aligned(tv, 8)) &&
                  (!a.dres || aligned(dres, 16));
  const int W = v4 ? 4 : 1;
  const int nv = pick_nv(qlora_cdiv(H / W, kWave));
  QLORA_CHECK_ARG(nv > 0);
  const dim3 grid((unsigned)qlora_cdiv(n, kRowsPerBlock));
  // the fast kernel takes both LoRA inputs or neither (the step's two cases)
  const int fnv = v4 && (a.tq != nullptr) == (a.tv != nullptr) ? fast_nv(H) : 0;
  if (fnv > 0) {
    const bool drop = a.tq != nullptr, res = a.dres != nullptr;
    by_nv(fnv, [&](auto k) { bwd4_launch<decltype(k)::value>(grid, (hipStream_t)stream, a,
                                                                drop, res); });
  } else if (v4) {
    launch_nv<BwdK, 4>(nv, grid, (hipStream_t)stream, a);
  } else {
    launch_nv<BwdK, 1>(nv, grid, (hipStream_t)stream, a);
  }
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
