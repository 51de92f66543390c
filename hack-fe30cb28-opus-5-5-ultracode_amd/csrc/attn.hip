// Causal attention over the packed variable-length sequences of a step (flash attention: online
// softmax, no [L, L] matrix in memory), grouped-query heads, forward and backward, on gfx950
// MFMA (v_mfma_f32_32x32x16_f16: fp16 operands, fp32 accumulation).
// Reference: _attn_fwd / _attn_bwd engine.py:857-869 (PyTorch's memory-efficient attention in
// its cu_seqlens form, causal, dropout 0, scale = D^-1/2) fed with k/v repeated to the q heads by
// _expand_kv engine.py:655-660. Here k/v are read in their grouped layout [n, KH, D]: q head h
// uses kv head h / (HQ / KH).
//
// Layout of the work. A wavefront owns 32 queries of one q head (forward, dQ) or 32 keys of one
// q head (dK/dV). MFMA register layout for C[32x32] = A[32x16] B[16x32]: lane l supplies
// A[l % 32][8(l / 32) .. +7] and B[8(l / 32) .. +7][l % 32]; register r of lane l receives
// C[8(r / 4) + 4(l / 32) + r % 4][l % 32].
//  * forward / dQ compute S^T = K Q^T, so lane l holds one query (l % 32) and 16 of the keys of
//    each 32-key tile; the online-softmax state (running max, sum) is a per-lane scalar (lanes l
//    and l ^ 32 share a query and combine their maxima with one shuffle), and O^T = V^T P^T
//    keeps the lane <-> query ownership, so rescaling O is a per-lane multiply.
//  * dK/dV compute S = Q K^T (lane <-> key), dV^T = dO^T P and dK^T = Q^T dS.
// A product that contracts over tokens needs a token-contiguous operand: V^T (forward), K^T
// (dQ), Q^T and dO^T (dK/dV) are transposed while being staged into LDS. The P/dS operand comes
// straight from the accumulator registers, whose rows within each 16-row group are in the
// order 0-3, 8-11, 4-7, 12-15 for the lower/upper half-wave; the transposed tiles store their
// tokens in that same slot order (perm16: swap rows 4-7 with 8-11), so no register shuffles
// are needed.
// LDS tiles are XOR-swizzled by 16-byte chunk so that the operand reads (32 rows, same chunk)
// and the staging writes are spread over the banks.
//
// One workgroup = the q heads that share a kv head (forward, dQ), which share the staged K/V
// tiles; dK/dV: one wavefront per (32-key block, q head). dK/dV come out per q head
// ([n, HQ, D]); the caller sums each group (the RoPE backward does, as the reference sums the
// repeated kv heads). The log-sum-exp of the forward (natural log, fp32 [HQ, n]) and
// delta = rowsum(dO * O) (fp32 [HQ, n], written by the dQ kernel) feed the dK/dV kernel.
#include "common.h"

namespace qlora {
namespace attn {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTok = 32;   // queries (forward, dQ) or keys (dK/dV) per wavefront
constexpr int kKB = 64;    // keys per staged block (forward, dQ)
constexpr int kMaxGroup = 6;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct Args {
  const uint16_t* q;     // fp16 [n, HQ, D]
  const uint16_t* k;     // fp16 [n, KH, D]
  const uint16_t* v;     // fp16 [n, KH, D]
  const uint16_t* o;     // fp16 [n, HQ, D] (forward output; read by the backward)
  const uint16_t* dout;  // fp16 [n, HQ, D]
  uint16_t* out;         // forward: o; dQ: dq [n, HQ, D]
  uint16_t* dk;          // fp16 [n, HQ, D]
  uint16_t* dv;          // fp16 [n, HQ, D]
  float* lse;            // fp32 [HQ, n] natural-log log-sum-exp of each query's scores
  float* delta;          // fp32 [HQ, n]
  const int32_t* cu;     // int32 [nseq + 1]
  int64_t n;
  int HQ, KH;
  float scale;
};

__device__ __forceinline__ f32x16 mfma(half8_t a, half8_t b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Token order of the transposed tiles within each aligned group of 16 (self-inverse).
__device__ __forceinline__ int perm16(int s) {
  return s ^ ((((s >> 2) ^ (s >> 3)) & 1) * 12);
}

// [rows][D] tile, 16-byte chunk c of row r at chunk c ^ (r mod D/8).
template <int D>
__device__ __forceinline__ int rm_off(int row, int chunk) {
  return row * D + ((chunk ^ (row & (D / 8 - 1))) << 3);
}
// [D][S] transposed tile (S = 64 or 32 token slots).
template <int S>
__device__ __forceinline__ int tr_off(int d, int slot) {
  const int sw = S == 64 ? ((d ^ (d >> 3)) & 7) : ((d >> 2) & 3);
  return d * S + (((slot >> 3) ^ sw) << 3) + (slot & 7);
}

template <int D>
__device__ __forceinline__ half8_t ld_rm(const uint16_t* t, int row, int chunk) {
  return *reinterpret_cast<const half8_t*>(t + rm_off<D>(row, chunk));
}
template <int S>
__device__ __forceinline__ half8_t ld_tr(const uint16_t* t, int d, int chunk) {
  return *reinterpret_cast<const half8_t*>(t + tr_off<S>(d, 8 * chunk));
}
__device__ __forceinline__ half8_t ld_g(const uint16_t* p) {
  return *reinterpret_cast<const half8_t*>(p);
}

// rows [0, rows) of a token-major matrix (row stride `stride` elements) into a [rows][D] tile;
// rows >= valid are zero.
template <int D>
__device__ __forceinline__ void stage_rows(uint16_t* tile, const uint16_t* base, int64_t stride,
                                           int rows, int valid, int tid, int nthr) {
  constexpr int CPR = D / 8;
  for (int id = tid; id < rows * CPR; id += nthr) {
    const int r = id / CPR, c = id % CPR;
    uint4 x = make_uint4(0, 0, 0, 0);
    if (r < valid) x = *reinterpret_cast<const uint4*>(base + (int64_t)r * stride + c * 8);
    *reinterpret_cast<uint4*>(tile + rm_off<D>(r, c)) = x;
  }
}

__device__ __forceinline__ uint32_t half_of(const uint4& x, int i) {
  const uint32_t w = i < 2 ? (i == 0 ? x.x : x.y) : (i == 2 ? x.z : x.w);
  return w;
}

// rows [0, S) of a token-major matrix into the transposed [D][S] tile, token t at slot
// (t & ~15) | perm16(t & 15); rows >= valid are zero. A work item is a pair of rows x 8 columns.
template <int D, int S>
__device__ __forceinline__ void stage_tr(uint16_t* tile, const uint16_t* base, int64_t stride,
                                         int valid, int tid, int nthr) {
  constexpr int CPR = D / 8;
  for (int id = tid; id < (S / 2) * CPR; id += nthr) {
    const int c = id % CPR, j = id / CPR;
    const int r0 = 2 * j;
    uint4 a = make_uint4(0, 0, 0, 0), b = make_uint4(0, 0, 0, 0);
    if (r0 < valid) a = *reinterpret_cast<const uint4*>(base + (int64_t)r0 * stride + c * 8);
    if (r0 + 1 < valid)
      b = *reinterpret_cast<const uint4*>(base + (int64_t)(r0 + 1) * stride + c * 8);
    const int slot = (r0 & ~15) | perm16(r0 & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t wa = half_of(a, i), wb = half_of(b, i);
      *reinterpret_cast<uint32_t*>(tile + tr_off<S>(8 * c + 2 * i, slot)) =
          (wa & 0xFFFFu) | (wb << 16);
      *reinterpret_cast<uint32_t*>(tile + tr_off<S>(8 * c + 2 * i + 1, slot)) =
          (wa >> 16) | (wb & 0xFFFF0000u);
    }
  }
}

// 8 accumulator values (registers 8 * half .. + 7 of acc) as an fp16 B operand.
__device__ __forceinline__ half8_t to_b(const f32x16& acc, int half) {
  half8_t r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (_Float16)acc[8 * half + i];
  return r;
}

// Row (query or key) index within the 32 x 32 tile of register r for this lane.
__device__ __forceinline__ int acc_row(int r, int lane) {
  return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}

// Stores 32 x D values of one token (lane & 31) held as D/32 accumulators (d in the rows).
template <int D>
__device__ __forceinline__ void store_token_row(uint16_t* row, const f32x16 (&acc)[D / 32],
                                                float mul, int lane) {
#pragma unroll
  for (int u = 0; u < D / 32; ++u)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * u + 8 * j + 4 * (lane >> 5);
      *reinterpret_cast<uint2*>(row + d) =
          make_uint2(pack2h(acc[u][4 * j] * mul, acc[u][4 * j + 1] * mul),
                     pack2h(acc[u][4 * j + 2] * mul, acc[u][4 * j + 3] * mul));
    }
}

// ------------------------------------------------------------------------------------------------
// Forward: O = softmax(scale Q K^T + causal mask) V per sequence, and the log-sum-exp.
// grid (nseq * KH, ceil(max_len / 32)), block 64 * (HQ / KH).
// ------------------------------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(64 * kMaxGroup) void attn_fwd_kernel(Args a) {
  constexpr int KC = D / 16, DT = D / 32;
  __shared__ __align__(16) uint16_t ks[kKB * D];
  __shared__ __align__(16) uint16_t vt[D * kKB];
  const int G = blockDim.x / 64;
  const int seq = blockIdx.x / a.KH, kvh = blockIdx.x % a.KH;
  const int q0 = (gridDim.y - 1 - blockIdx.y) * kTok;  // longest rows first
  const int start = a.cu[seq], L = a.cu[seq + 1] - start;
  if (q0 >= L) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int h = kvh * G + (tid >> 6);
  const int qi = q0 + (lane & 31);
  const bool qok = qi < L;
  const int64_t qs = (int64_t)a.HQ * D, kvs = (int64_t)a.KH * D;

  half8_t qr[KC];
#pragma unroll
  for (int kk = 0; kk < KC; ++kk) qr[kk] = half8_t{};
  if (qok) {
    const uint16_t* p = a.q + (int64_t)(start + qi) * qs + h * D + 8 * (lane >> 5);
#pragma unroll
    for (int kk = 0; kk < KC; ++kk) qr[kk] = ld_g(p + 16 * kk);
  }
  f32x16 o[DT];
#pragma unroll
  for (int u = 0; u < DT; ++u) o[u] = f32x16{};
  float m = -__builtin_inff(), lsum = 0.f;
  const float c = a.scale * kLog2e;
  const int kend = min(q0 + kTok, L);
  const int nkb = (kend + kKB - 1) / kKB;
  const uint16_t* kbase = a.k + (int64_t)start * kvs + kvh * D;
  const uint16_t* vbase = a.v + (int64_t)start * kvs + kvh * D;

  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * kKB;
    const int valid = min(kKB, L - k0);
    __syncthreads();
    stage_rows<D>(ks, kbase + (int64_t)k0 * kvs, kvs, kKB, valid, tid, blockDim.x);
    stage_tr<D, kKB>(vt, vbase + (int64_t)k0 * kvs, kvs, valid, tid, blockDim.x);
    __syncthreads();
    f32x16 s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      s[t] = f32x16{};
#pragma unroll
      for (int kk = 0; kk < KC; ++kk)
        s[t] = mfma(ld_rm<D>(ks, 32 * t + (lane & 31), 2 * kk + (lane >> 5)), qr[kk], s[t]);
    }
    const bool mask = k0 + kKB - 1 > q0 || k0 + kKB > L;
    float mx = -__builtin_inff();
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = s[t][r] * c;
        if (mask) {
          const int key = k0 + 32 * t + acc_row(r, lane);
          if (key > qi || key >= L) x = -__builtin_inff();
        }
        s[t][r] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mnew = fmaxf(m, mx);
    const float alpha = exp2f(m - mnew);
    m = mnew;
    float ps = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = exp2f(s[t][r] - mnew);
        s[t][r] = p;
        ps += p;
      }
    lsum = lsum * alpha + ps;
#pragma unroll
    for (int u = 0; u < DT; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[u][r] *= alpha;
    half8_t pb[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) pb[kk] = to_b(s[kk >> 1], kk & 1);
#pragma unroll
    for (int u = 0; u < DT; ++u)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        o[u] = mfma(ld_tr<kKB>(vt, 32 * u + (lane & 31), 2 * kk + (lane >> 5)), pb[kk], o[u]);
  }
  const float ltot = lsum + __shfl_xor(lsum, 32, 64);
  if (qok) {
    store_token_row<D>(a.out + (int64_t)(start + qi) * qs + h * D, o, 1.0f / ltot, lane);
    if (lane < 32) a.lse[(int64_t)h * a.n + start + qi] = (m + log2f(ltot)) * kLn2;
  }
}

// ------------------------------------------------------------------------------------------------
// Backward, dQ (and delta = rowsum(dO * O)): per 32 queries of a q head, over the key blocks
// up to the diagonal: S^T = K Q^T, P = exp(S - lse), dP^T = V dO^T, dS = P (dP - delta),
// dQ^T += K^T dS^T. grid and block as the forward.
// ------------------------------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(64 * kMaxGroup) void attn_dq_kernel(Args a) {
  constexpr int KC = D / 16, DT = D / 32;
  __shared__ __align__(16) uint16_t ks[kKB * D];
  __shared__ __align__(16) uint16_t vs[kKB * D];
  __shared__ __align__(16) uint16_t kt[D * kKB];
  const int G = blockDim.x / 64;
  const int seq = blockIdx.x / a.KH, kvh = blockIdx.x % a.KH;
  const int q0 = (gridDim.y - 1 - blockIdx.y) * kTok;
  const int start = a.cu[seq], L = a.cu[seq + 1] - start;
  if (q0 >= L) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int h = kvh * G + (tid >> 6);
  const int qi = q0 + (lane & 31);
  const bool qok = qi < L;
  const int64_t qs = (int64_t)a.HQ * D, kvs = (int64_t)a.KH * D;

  half8_t qr[KC], dr[KC];
#pragma unroll
  for (int kk = 0; kk < KC; ++kk) qr[kk] = dr[kk] = half8_t{};
  float dpart = 0.f, lse2 = __builtin_inff();  // out-of-range queries: P = 0
  if (qok) {
    const int64_t off = (int64_t)(start + qi) * qs + h * D + 8 * (lane >> 5);
#pragma unroll
    for (int kk = 0; kk < KC; ++kk) {
      qr[kk] = ld_g(a.q + off + 16 * kk);
      dr[kk] = ld_g(a.dout + off + 16 * kk);
      const half8_t ov = ld_g(a.o + off + 16 * kk);
#pragma unroll
      for (int i = 0; i < 8; ++i) dpart += (float)dr[kk][i] * (float)ov[i];
    }
    lse2 = a.lse[(int64_t)h * a.n + start + qi] * kLog2e;
  }
  const float delta = dpart + __shfl_xor(dpart, 32, 64);
  if (qok && lane < 32) a.delta[(int64_t)h * a.n + start + qi] = delta;

  f32x16 dq[DT];
#pragma unroll
  for (int u = 0; u < DT; ++u) dq[u] = f32x16{};
  const float c = a.scale * kLog2e;
  const int kend = min(q0 + kTok, L);
  const int nkb = (kend + kKB - 1) / kKB;
  const uint16_t* kbase = a.k + (int64_t)start * kvs + kvh * D;
  const uint16_t* vbase = a.v + (int64_t)start * kvs + kvh * D;

  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * kKB;
    const int valid = min(kKB, L - k0);
    __syncthreads();
    stage_rows<D>(ks, kbase + (int64_t)k0 * kvs, kvs, kKB, valid, tid, blockDim.x);
    stage_rows<D>(vs, vbase + (int64_t)k0 * kvs, kvs, kKB, valid, tid, blockDim.x);
    stage_tr<D, kKB>(kt, kbase + (int64_t)k0 * kvs, kvs, valid, tid, blockDim.x);
    __syncthreads();
    f32x16 s[2], dp[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      s[t] = f32x16{};
      dp[t] = f32x16{};
#pragma unroll
      for (int kk = 0; kk < KC; ++kk) {
        const int row = 32 * t + (lane & 31), ch = 2 * kk + (lane >> 5);
        s[t] = mfma(ld_rm<D>(ks, row, ch), qr[kk], s[t]);
        dp[t] = mfma(ld_rm<D>(vs, row, ch), dr[kk], dp[t]);
      }
    }
    const bool mask = k0 + kKB - 1 > q0 || k0 + kKB > L;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = exp2f(s[t][r] * c - lse2);
        if (mask) {
          const int key = k0 + 32 * t + acc_row(r, lane);
          if (key > qi || key >= L) p = 0.f;
        }
        s[t][r] = p * (dp[t][r] - delta);
      }
    half8_t sb[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) sb[kk] = to_b(s[kk >> 1], kk & 1);
#pragma unroll
    for (int u = 0; u < DT; ++u)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        dq[u] = mfma(ld_tr<kKB>(kt, 32 * u + (lane & 31), 2 * kk + (lane >> 5)), sb[kk], dq[u]);
  }
  if (qok) store_token_row<D>(a.out + (int64_t)(start + qi) * qs + h * D, dq, a.scale, lane);
}

// ------------------------------------------------------------------------------------------------
// Backward, dK and dV of one q head: per 32 keys, over the query blocks from the diagonal to the
// end of the sequence: S = Q K^T, P = exp(S - lse), dP = dO V^T, dS = P (dP - delta),
// dV^T += dO^T P, dK^T += Q^T dS. grid (nseq * HQ, ceil(max_len / 32)), block 64.
// ------------------------------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(64) void attn_dkdv_kernel(Args a) {
  constexpr int KC = D / 16, DT = D / 32;
  __shared__ __align__(16) uint16_t qsm[kTok * D];
  __shared__ __align__(16) uint16_t qt[D * kTok];
  __shared__ __align__(16) uint16_t dsm[kTok * D];
  __shared__ __align__(16) uint16_t dt[D * kTok];
  const int seq = blockIdx.x / a.HQ, h = blockIdx.x % a.HQ;
  const int kvh = h / (a.HQ / a.KH);
  const int k0 = blockIdx.y * kTok;
  const int start = a.cu[seq], L = a.cu[seq + 1] - start;
  if (k0 >= L) return;
  const int lane = threadIdx.x;
  const int kj = k0 + (lane & 31);
  const bool kok = kj < L;
  const int64_t qs = (int64_t)a.HQ * D, kvs = (int64_t)a.KH * D;

  half8_t kr[KC], vr[KC];
#pragma unroll
  for (int kk = 0; kk < KC; ++kk) kr[kk] = vr[kk] = half8_t{};
  if (kok) {
    const int64_t off = (int64_t)(start + kj) * kvs + kvh * D + 8 * (lane >> 5);
#pragma unroll
    for (int kk = 0; kk < KC; ++kk) {
      kr[kk] = ld_g(a.k + off + 16 * kk);
      vr[kk] = ld_g(a.v + off + 16 * kk);
    }
  }
  f32x16 dk[DT], dv[DT];
#pragma unroll
  for (int u = 0; u < DT; ++u) dk[u] = dv[u] = f32x16{};
  const float c = a.scale * kLog2e;
  const uint16_t* qbase = a.q + (int64_t)start * qs + h * D;
  const uint16_t* dbase = a.dout + (int64_t)start * qs + h * D;
  const float* lse = a.lse + (int64_t)h * a.n + start;
  const float* dl = a.delta + (int64_t)h * a.n + start;

  for (int q0 = k0; q0 < L; q0 += kTok) {
    const int valid = min(kTok, L - q0);
    __syncthreads();
    stage_rows<D>(qsm, qbase + (int64_t)q0 * qs, qs, kTok, valid, lane, 64);
    stage_tr<D, kTok>(qt, qbase + (int64_t)q0 * qs, qs, valid, lane, 64);
    stage_rows<D>(dsm, dbase + (int64_t)q0 * qs, qs, kTok, valid, lane, 64);
    stage_tr<D, kTok>(dt, dbase + (int64_t)q0 * qs, qs, valid, lane, 64);
    __syncthreads();
    f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
    for (int kk = 0; kk < KC; ++kk) {
      const int row = lane & 31, ch = 2 * kk + (lane >> 5);
      s = mfma(ld_rm<D>(qsm, row, ch), kr[kk], s);
      dp = mfma(ld_rm<D>(dsm, row, ch), vr[kk], dp);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qq = q0 + acc_row(r, lane);
      float p = 0.f, d = 0.f;
      if (qq < L && kj <= qq) {
        p = exp2f(s[r] * c - lse[qq] * kLog2e);
        d = dl[qq];
      }
      s[r] = p;
      dp[r] = p * (dp[r] - d);
    }
    half8_t pb[2], sb[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      pb[kk] = to_b(s, kk);
      sb[kk] = to_b(dp, kk);
    }
#pragma unroll
    for (int u = 0; u < DT; ++u)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int d = 32 * u + (lane & 31), ch = 2 * kk + (lane >> 5);
        dv[u] = mfma(ld_tr<kTok>(dt, d, ch), pb[kk], dv[u]);
        dk[u] = mfma(ld_tr<kTok>(qt, d, ch), sb[kk], dk[u]);
      }
  }
  if (kok) {
    const int64_t off = (int64_t)(start + kj) * qs + h * D;
    store_token_row<D>(a.dk + off, dk, a.scale, lane);
    store_token_row<D>(a.dv + off, dv, 1.0f, lane);
  }
}

}  // namespace attn
}  // namespace qlora

using namespace qlora::attn;

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int check_common(int32_t nseq, int32_t max_len, int64_t n, int32_t HQ, int32_t KH, int32_t D) {
  QLORA_CHECK_ARG(nseq >= 0 && max_len >= 0 && n >= 0);
  QLORA_CHECK_ARG(D == 64 || D == 128);
  QLORA_CHECK_ARG(HQ > 0 && KH > 0 && HQ % KH == 0 && HQ / KH <= kMaxGroup);
  QLORA_CHECK_ARG((int64_t)nseq * HQ < (1ll << 31));
  return 0;
}

}  // namespace

// Forward. q [n, HQ, D], k/v [n, KH, D], out [n, HQ, D] fp16 contiguous; lse fp32 [HQ, n];
// cu_seqlens int32 [nseq + 1] on the device, non-decreasing from 0 to n, every length
// <= max_len (the kernel reads no token outside [cu[s], cu[s + 1]) for sequence s).
QLORA_API int qlora_attn_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                             const int32_t* cu_seqlens, int32_t nseq, int32_t max_len, int64_t n,
                             int32_t HQ, int32_t KH, int32_t D, float scale, void* stream) {
  if (int rc = check_common(nseq, max_len, n, HQ, KH, D)) return rc;
  if (n == 0 || nseq == 0 || max_len == 0) return 0;
  QLORA_CHECK_ARG(q && k && v && out && lse && cu_seqlens);
  QLORA_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out));
  Args a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.out = static_cast<uint16_t*>(out);
  a.lse = lse;
  a.cu = cu_seqlens;
  a.n = n;
  a.HQ = HQ;
  a.KH = KH;
  a.scale = scale;
  const dim3 grid((unsigned)(nseq * KH), (unsigned)qlora_cdiv(max_len, kTok));
  const dim3 block(64 * (HQ / KH));
  hipStream_t s = (hipStream_t)stream;
  if (D == 128) hipLaunchKernelGGL(attn_fwd_kernel<128>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(attn_fwd_kernel<64>, grid, block, 0, s, a);
  return qlora_launch_status();
}

// Backward. dout/out/q [n, HQ, D], k/v [n, KH, D] as in the forward, lse from it; delta: fp32
// workspace [HQ, n]; dq, dk, dv fp16 [n, HQ, D] (dk/dv per q head, not yet summed over the
// q heads of a kv head).
QLORA_API int qlora_attn_bwd(const void* dout, const void* q, const void* k, const void* v,
                             const void* out, const float* lse, float* delta, void* dq, void* dk,
                             void* dv, const int32_t* cu_seqlens, int32_t nseq, int32_t max_len,
                             int64_t n, int32_t HQ, int32_t KH, int32_t D, float scale,
                             void* stream) {
  if (int rc = check_common(nseq, max_len, n, HQ, KH, D)) return rc;
  if (n == 0 || nseq == 0 || max_len == 0) return 0;
  QLORA_CHECK_ARG(dout && q && k && v && out && lse && delta && dq && dk && dv && cu_seqlens);
  QLORA_CHECK_ARG(aligned16(dout) && aligned16(q) && aligned16(k) && aligned16(v) &&
                  aligned16(out) && aligned16(dq) && aligned16(dk) && aligned16(dv));
  Args a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.o = static_cast<const uint16_t*>(out);
  a.dout = static_cast<const uint16_t*>(dout);
  a.out = static_cast<uint16_t*>(dq);
  a.dk = static_cast<uint16_t*>(dk);
  a.dv = static_cast<uint16_t*>(dv);
  a.lse = const_cast<float*>(lse);
  a.delta = delta;
  a.cu = cu_seqlens;
  a.n = n;
  a.HQ = HQ;
  a.KH = KH;
  a.scale = scale;
  hipStream_t s = (hipStream_t)stream;
  const unsigned blocks = (unsigned)qlora_cdiv(max_len, kTok);
  const dim3 g1((unsigned)(nseq * KH), blocks), b1(64 * (HQ / KH));
  if (D == 128) hipLaunchKernelGGL(attn_dq_kernel<128>, g1, b1, 0, s, a);
  else hipLaunchKernelGGL(attn_dq_kernel<64>, g1, b1, 0, s, a);
  if (int rc = qlora_launch_status()) return rc;
  const dim3 g2((unsigned)(nseq * HQ), blocks), b2(64);
  if (D == 128) hipLaunchKernelGGL(attn_dkdv_kernel<128>, g2, b2, 0, s, a);
  else hipLaunchKernelGGL(attn_dkdv_kernel<64>, g2, b2, 0, s, a);
  return qlora_launch_status();
}
