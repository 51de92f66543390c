// qkv split + LoRA deltas + rotary embedding over packed variable-length tokens, and its inverse.
// Reference: qkv_rope_fwd_kernel kernels.py:212-264 (_rope_fwd engine.py:984-997) and
// qkv_rope_bwd_kernel kernels.py:267-306 (_rope_bwd engine.py:1000-1009).
//
// Rotate-half RoPE over the two halves of each head (Qwen2):
//   out[:D/2] = x1 cos - x2 sin,  out[D/2:] = x2 cos + x1 sin,   cos/sin = table[pos, 0:D/2]
// with pos restarting at every sequence of the packed batch. One work item is 8 columns of
// one half-head pair (two 16-byte loads, two 16-byte stores per output copy).
//
// k and v come out with `kv_heads_out` heads: HKV (grouped-query layout) or HQ (each kv head
// repeated HQ/HKV times, as repeat_kv does: kv head j at heads j*G .. j*G+G-1).
#include "common.h"

namespace qlora {

struct RopeFwdArgs {
  const uint16_t* qkv;  // fp16 [n, (HQ + 2 HKV) D]
  const uint16_t* lq;   // fp16 [n, HQ D] or null
  const uint16_t* lv;   // fp16 [n, HKV D] or null
  const float* cos;     // fp32 [positions, D/2]
  const float* sin;
  const int32_t* pos;   // int32 [n], each < positions
  uint16_t* q;          // fp16 [n, HQ, D]
  uint16_t* k;          // fp16 [n, KH, D]
  uint16_t* v;          // fp16 [n, KH, D]
  int64_t n, positions;
  int HQ, HKV, D, KH;
  float lora_scale;
};

struct RopeBwdArgs {
  const uint16_t* dq;  // fp16 [n, HQ, D]
  const uint16_t* dk;  // fp16 [n, KH, D]
  const uint16_t* dv;  // fp16 [n, KH, D]
  const float* cos;
  const float* sin;
  const int32_t* pos;
  uint16_t* dqkv;      // fp16 [n, (HQ + 2 HKV) D]
  int64_t n, positions;
  int HQ, HKV, D, KH;
};

__device__ __forceinline__ void unpack8(const uint4 w, float (&v)[8]) {
  v[0] = lo_h(w.x); v[1] = hi_h(w.x); v[2] = lo_h(w.y); v[3] = hi_h(w.y);
  v[4] = lo_h(w.z); v[5] = hi_h(w.z); v[6] = lo_h(w.w); v[7] = hi_h(w.w);
}
__device__ __forceinline__ uint4 pack8(const float (&v)[8]) {
  return make_uint4(pack2h(v[0], v[1]), pack2h(v[2], v[3]), pack2h(v[4], v[5]),
                    pack2h(v[6], v[7]));
}
__device__ __forceinline__ uint4 ld16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void st16(uint16_t* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }
// cos/sin of position p (8 columns from d0); a position outside the table gives NaN instead of
// an out-of-bounds read (the address is clamped, the values replaced after the load).
__device__ __forceinline__ void ld_table(const float* tab, int64_t p, int64_t positions,
                                         int half, int d0, float (&v)[8]) {
  const bool ok = p >= 0 && p < positions;
  const int64_t pc = ok ? p : 0;
  const float4 a = reinterpret_cast<const float4*>(tab + pc * half + d0)[0];
  const float4 b = reinterpret_cast<const float4*>(tab + pc * half + d0)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  if (!ok) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __builtin_nanf("");
  }
}

// Work items are head-major: item = (head n + token) * per_head + chunk, so a wavefront's items
// are one head of consecutive tokens (the q / k / v branches are uniform but at head
// boundaries) and each token-head's 8-column chunks are consecutive threads (128 contiguous
// bytes per half-head). The position is loaded first and the data right after it, so the table
// loads that need the position wait for that one load only: two memory round trips per item.
__device__ __forceinline__ void item_of(uint32_t gid, uint32_t n, int per_head, int& head,
                                        int64_t& tok, int& d0) {
  const uint32_t per = n * (uint32_t)per_head, h = gid / per, rem = gid - h * per;
  head = (int)h;
  tok = rem / (uint32_t)per_head;
  d0 = (int)(rem - (uint32_t)tok * (uint32_t)per_head) * 8;
}

__global__ __launch_bounds__(256) void rope_fwd_kernel(RopeFwdArgs a) {
  const int half = a.D / 2, per_head = half / 8;
  const int heads = a.HQ + 2 * a.HKV;
  const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (uint32_t)a.n * (uint32_t)(heads * per_head)) return;
  int head, d0;
  int64_t tok;
  item_of(gid, (uint32_t)a.n, per_head, head, tok, d0);
  const int p = a.pos[tok];
  const int C = heads * a.D;
  const uint16_t* src = a.qkv + tok * C + (int64_t)head * a.D + d0;
  const uint4 w1 = ld16(src), w2 = ld16(src + half);
  const bool is_q = head < a.HQ, is_v = head >= a.HQ + a.HKV;
  const int hv = head - a.HQ - a.HKV;
  // the LoRA delta of a q or v head (a k head, or an absent delta: none)
  const uint16_t* l = is_q ? a.lq : is_v ? a.lv : nullptr;
  uint4 m1 = make_uint4(0u, 0u, 0u, 0u), m2 = m1;
  if (l != nullptr) {
    l += is_q ? tok * ((int64_t)a.HQ * a.D) + (int64_t)head * a.D + d0
              : tok * ((int64_t)a.HKV * a.D) + (int64_t)hv * a.D + d0;
    m1 = ld16(l);
    m2 = ld16(l + half);
  }
  float x1[8], x2[8];
  unpack8(w1, x1);
  unpack8(w2, x2);
  if (l != nullptr) {
    float l1[8], l2[8];
    unpack8(m1, l1);
    unpack8(m2, l2);
#pragma unroll
    for (int i = 0; i < 8; ++i) { x1[i] += l1[i] * a.lora_scale; x2[i] += l2[i] * a.lora_scale; }
  }
  if (is_v) {  // v: no rotation
    const uint4 o1 = pack8(x1), o2 = pack8(x2);
    const int rep = a.KH / a.HKV;
    for (int r = 0; r < rep; ++r) {
      uint16_t* dst = a.v + tok * ((int64_t)a.KH * a.D) + (int64_t)(hv * rep + r) * a.D + d0;
      st16(dst, o1);
      st16(dst + half, o2);
    }
    return;
  }
  float c[8], s[8], o1[8], o2[8];
  ld_table(a.cos, p, a.positions, half, d0, c);
  ld_table(a.sin, p, a.positions, half, d0, s);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    o1[i] = x1[i] * c[i] - x2[i] * s[i];
    o2[i] = x2[i] * c[i] + x1[i] * s[i];
  }
  const uint4 p1 = pack8(o1), p2 = pack8(o2);
  if (is_q) {
    uint16_t* dst = a.q + tok * ((int64_t)a.HQ * a.D) + (int64_t)head * a.D + d0;
    st16(dst, p1);
    st16(dst + half, p2);
  } else {
    const int hk = head - a.HQ;
    const int rep = a.KH / a.HKV;
    for (int r = 0; r < rep; ++r) {
      uint16_t* dst = a.k + tok * ((int64_t)a.KH * a.D) + (int64_t)(hk * rep + r) * a.D + d0;
      st16(dst, p1);
      st16(dst + half, p2);
    }
  }
}

__global__ __launch_bounds__(256) void rope_bwd_kernel(RopeBwdArgs a) {
  const int half = a.D / 2, per_head = half / 8;
  const int heads = a.HQ + 2 * a.HKV;
  const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (uint32_t)a.n * (uint32_t)(heads * per_head)) return;
  int head, d0;
  int64_t tok;
  item_of(gid, (uint32_t)a.n, per_head, head, tok, d0);
  const int p = a.pos[tok];
  const int C = heads * a.D;
  uint16_t* out = a.dqkv + tok * C + (int64_t)head * a.D + d0;
  float g1[8], g2[8];
  const bool is_q = head < a.HQ, is_v = head >= a.HQ + a.HKV;
  if (is_q) {
    const uint16_t* src = a.dq + tok * ((int64_t)a.HQ * a.D) + (int64_t)head * a.D + d0;
    const uint4 w1 = ld16(src), w2 = ld16(src + half);
    unpack8(w1, g1);
    unpack8(w2, g2);
  } else {
    const int hk = is_v ? head - a.HQ - a.HKV : head - a.HQ;
    const uint16_t* base = (is_v ? a.dv : a.dk) + tok * ((int64_t)a.KH * a.D);
    const int rep = a.KH / a.HKV;
#pragma unroll
    for (int i = 0; i < 8; ++i) g1[i] = g2[i] = 0.f;
    // sum of the grouped-query replicas, fp32, in order; up to 8 replicas' loads are issued
    // before the first sum (one round trip, not one per replica)
    constexpr int kMaxRep = 8;
    uint4 w[kMaxRep][2];
#pragma unroll
    for (int r = 0; r < kMaxRep; ++r)
      if (r < rep) {
        const uint16_t* src = base + (int64_t)(hk * rep + r) * a.D + d0;
        w[r][0] = ld16(src);
        w[r][1] = ld16(src + half);
      }
#pragma unroll
    for (int r = 0; r < kMaxRep; ++r)
      if (r < rep) {
        float t1[8], t2[8];
        unpack8(w[r][0], t1);
        unpack8(w[r][1], t2);
#pragma unroll
        for (int i = 0; i < 8; ++i) { g1[i] += t1[i]; g2[i] += t2[i]; }
      }
    for (int r = kMaxRep; r < rep; ++r) {
      const uint16_t* src = base + (int64_t)(hk * rep + r) * a.D + d0;
      float t1[8], t2[8];
      unpack8(ld16(src), t1);
      unpack8(ld16(src + half), t2);
#pragma unroll
      for (int i = 0; i < 8; ++i) { g1[i] += t1[i]; g2[i] += t2[i]; }
    }
    if (is_v) {
      st16(out, pack8(g1));
      st16(out + half, pack8(g2));
      return;
    }
  }
  float c[8], s[8], o1[8], o2[8];
  ld_table(a.cos, p, a.positions, half, d0, c);
  ld_table(a.sin, p, a.positions, half, d0, s);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    o1[i] = g1[i] * c[i] + g2[i] * s[i];
    o2[i] = g2[i] * c[i] - g1[i] * s[i];
  }
  st16(out, pack8(o1));
  st16(out + half, pack8(o2));
}

}  // namespace qlora

using namespace qlora;

namespace {
bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }
}

QLORA_API int qlora_rope_fwd(const void* qkv, const void* lq, const void* lv, const float* cos,
                             const float* sin, int64_t positions, const int32_t* pos, void* q,
                             void* k, void* v, int64_t n, int32_t HQ, int32_t HKV, int32_t D,
                             int32_t kv_heads_out, float lora_scale, void* stream) {
  QLORA_CHECK_ARG(n >= 0);
  if (n == 0) return 0;
  QLORA_CHECK_ARG(qkv && cos && sin && pos && q && k && v && positions > 0);
  QLORA_CHECK_ARG(HQ > 0 && HKV > 0 && HQ % HKV == 0 && D > 0 && D % 16 == 0);
  QLORA_CHECK_ARG(kv_heads_out == HKV || kv_heads_out == HQ);
  QLORA_CHECK_ARG(al16(qkv) && al16(q) && al16(k) && al16(v) && al16(cos) && al16(sin));
  QLORA_CHECK_ARG((!lq || al16(lq)) && (!lv || al16(lv)));
  RopeFwdArgs a{static_cast<const uint16_t*>(qkv), static_cast<const uint16_t*>(lq),
                static_cast<const uint16_t*>(lv), cos, sin, pos, static_cast<uint16_t*>(q),
                static_cast<uint16_t*>(k), static_cast<uint16_t*>(v), n, positions, HQ, HKV,
                D, kv_heads_out, lora_scale};
  const int64_t total = n * (int64_t)(HQ + 2 * HKV) * (D / 16);
  QLORA_CHECK_ARG(qlora_cdiv(total, 256) * 256 <= (int64_t)UINT32_MAX);  // 32-bit item index
  hipLaunchKernelGGL(rope_fwd_kernel, dim3((unsigned)qlora_cdiv(total, 256)), dim3(256), 0,
                     (hipStream_t)stream, a);
  return qlora_launch_status();
}

QLORA_API int qlora_rope_bwd(const void* dq, const void* dk, const void* dv, const float* cos,
                             const float* sin, int64_t positions, const int32_t* pos, void* dqkv,
                             int64_t n,
                             int32_t HQ, int32_t HKV, int32_t D, int32_t kv_heads_in,
                             void* stream) {
  QLORA_CHECK_ARG(n >= 0);
  if (n == 0) return 0;
  QLORA_CHECK_ARG(dq && dk && dv && cos && sin && pos && dqkv && positions > 0);
  QLORA_CHECK_ARG(HQ > 0 && HKV > 0 && HQ % HKV == 0 && D > 0 && D % 16 == 0);
  QLORA_CHECK_ARG(kv_heads_in == HKV || kv_heads_in == HQ);
  QLORA_CHECK_ARG(al16(dq) && al16(dk) && al16(dv) && al16(dqkv) && al16(cos) && al16(sin));
  RopeBwdArgs a{static_cast<const uint16_t*>(dq), static_cast<const uint16_t*>(dk),
                static_cast<const uint16_t*>(dv), cos, sin, pos, static_cast<uint16_t*>(dqkv),
                n, positions, HQ, HKV, D, kv_heads_in};
  const int64_t total = n * (int64_t)(HQ + 2 * HKV) * (D / 16);
  QLORA_CHECK_ARG(qlora_cdiv(total, 256) * 256 <= (int64_t)UINT32_MAX);  // 32-bit item index
  hipLaunchKernelGGL(rope_bwd_kernel, dim3((unsigned)qlora_cdiv(total, 256)), dim3(256), 0,
                     (hipStream_t)stream, a);
  return qlora_launch_status();
}
