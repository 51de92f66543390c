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
// A product that contracts over tokens needs a token-contiguous operand (V^T forward, K^T dQ,
// Q^T and dO^T dK/dV): the tiles are staged row-major with 16-byte stores and read transposed
// with ds_read_b64_tr_b16 (tr_operand). The P/dS operand comes straight from the accumulator
// registers, whose rows within each 16-row group are in the order 0-3, 8-11, 4-7, 12-15 for the
// lower/upper half-wave; tr_operand hands out the tokens in that same order, so no register
// shuffles are needed.
// LDS tiles are XOR-swizzled by 16-byte chunk so that the operand reads (32 rows, same chunk)
// and the staging writes are spread over the banks.
//
// One workgroup = the q heads that share a kv head (forward, dQ), which share the staged K/V
// tiles; dK/dV: four wavefronts on 128 consecutive keys of one q head, sharing the staged Q/dO.
// Global loads of the next tile are issued before the current tile's MFMAs (register
// prefetch), so their latency overlaps the arithmetic. dK/dV come out per q head
// ([n, HQ, D]); the caller sums each group (the RoPE backward does, as the reference sums the
// repeated kv heads). The log-sum-exp of the forward (natural log, fp32 [HQ, n]) and
// delta = rowsum(dO * O) (fp32 [HQ, n], written by attn_delta_kernel) feed the dQ and the dK/dV
// kernels, which run at the same time on two streams.
#include "common.h"

#include <mutex>

namespace qlora {
namespace attn {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTok = 32;   // queries (forward, dQ) or keys (dK/dV) per wavefront
constexpr int kKB = 64;    // keys per staged block (forward, dQ)
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
  float* part;           // split key range: fp32 partial O / dQ [nch][n][HQ][D]
  float2* part_ml;       // forward split: (running max (log2 units), sum) [nch][HQ][n]
  int64_t n;
  int HQ, KH;
  int chunk;             // key blocks per workgroup (0: the whole range in one workgroup)
  int ntiles;            // query (forward, dQ) or key (dK/dV) tiles per sequence and head
  float scale;
};

// The key range of a query tile with nkb key blocks may be cut into chunks of a.chunk blocks, one
// workgroup each (blockIdx.z = chunk), when a batch of few long sequences would otherwise leave
// most of the GPU idle while its longest tiles walk their keys. With one chunk the workgroup
// writes the result itself; otherwise each writes fp32 partials and attn_merge_kernel merges them
// in chunk order.
__device__ __forceinline__ int num_chunks(int nkb, int chunk) {
  return chunk > 0 ? (nkb + chunk - 1) / chunk : 1;
}

// 2^x by the hardware instruction (v_exp_f32): no denormal-range fix-up (results below 2^-126
// flush to zero, which a probability that small does not miss).
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f32x16 mfma(half8_t a, half8_t b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// [rows][D] tile, 16-byte chunk c of row r at chunk c ^ (r mod D/8).
template <int D>
__device__ __forceinline__ int rm_off(int row, int chunk) {
  return row * D + ((chunk ^ (row & (D / 8 - 1))) << 3);
}

// [rows][D] tile read transposed by ds_read_b64_tr_b16 (tr_operand): a half-wave reads 4
// consecutive rows (the first a multiple of 4) x 4 aligned chunks, which this swizzle spreads
// over distinct banks; 16-byte row stores (16 threads a row) stay conflict-free too.
template <int D>
__device__ __forceinline__ int tt_off(int row, int chunk) {
  const int j = D == 128 ? row : row >> 1;  // rows sharing the 64 banks: 1 (D = 128) or 2
  const int sw = D == 128 ? (((j & 3) << 2) | ((j >> 2) & 3)) : (((j & 1) << 2) | ((j >> 1) & 3));
  return row * D + ((chunk ^ sw) << 3);
}

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

// The MFMA A operand T[d][8 token slots] of a tt_off tile (T = the tile transposed): lane l
// supplies d = d0 + l % 32 and tokens k0 + 4 (l / 32) + {0..3, 8..11}, the slot order of an
// accumulator's rows (acc_row). ds_read_b64_tr_b16 gives lane i of each 16-lane group element
// i % 4 of the 4 halves read by lane 4 j + i / 4 of the group, as its element j; so lane p of the
// group reads row (first token) + p / 4, columns (group's first d) + 4 (p % 4) .. + 3.
template <int D>
__device__ __forceinline__ half8_t tr_operand(const uint16_t* t, int k0, int d0, int lane) {
  const int p = lane & 15;
  const int row = k0 + 4 * (lane >> 5) + (p >> 2);
  const int col = d0 + 16 * ((lane >> 4) & 1) + 4 * (p & 3);
  const int o0 = tt_off<D>(row, col >> 3) + (col & 7);
  const int o1 = tt_off<D>(row + 8, col >> 3) + (col & 7);
  const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(t + o0));
  const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(t + o1));
  return __builtin_bit_cast(half8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// A row operand (as ld_rm) of a tt_off tile: the swizzle maps 16 consecutive rows of one chunk
// to distinct banks too.
template <int D>
__device__ __forceinline__ half8_t ld_tt(const uint16_t* t, int row, int chunk) {
  return *reinterpret_cast<const half8_t*>(t + tt_off<D>(row, chunk));
}

template <int D>
__device__ __forceinline__ half8_t ld_rm(const uint16_t* t, int row, int chunk) {
  return *reinterpret_cast<const half8_t*>(t + rm_off<D>(row, chunk));
}
__device__ __forceinline__ half8_t ld_g(const uint16_t* p) {
  return *reinterpret_cast<const half8_t*>(p);
}

// Staging of token-major global rows into LDS tiles, split into a load phase (all of a thread's
// global loads issued back to back into registers, so their latencies overlap, and early enough
// to hide behind the previous tile's MFMAs) and a store phase into the tile. The loads are
// buffer loads over the sequence's rows of one head: rows past the sequence read zeros, so
// there is neither a clamp nor a select on the loaded value (which the compiler may turn into a
// branch around the load, whose join then waits for every load in flight).
//
// Offsets are bytes from the resource base: row r at r * stride_b, chunk c (8 halves) at 16 c.
//
// RowStage: rows [row0, row0 + ROWS) into a [ROWS][D] tile (swizzle rm_off, or tt_off for a
// tile read by tr_operand).
template <int D, int ROWS, int NT, bool TT = false>
struct RowStage {
  static constexpr int CPR = D / 8, TOTAL = ROWS * CPR, CNT = (TOTAL + NT - 1) / NT;
  uint4 r[CNT];
  __device__ __forceinline__ void load(rsrc_t src, int row0, int stride_b, int tid) {
#pragma unroll
    for (int i = 0; i < CNT; ++i) {
      const int id = tid + i * NT, row = id / CPR, c = id % CPR;  // id >= TOTAL: not stored
      r[i] = buf_load16(src, (uint32_t)((row0 + row) * stride_b + c * 16));
    }
  }
  __device__ __forceinline__ void store(uint16_t* tile, int tid) const {
#pragma unroll
    for (int i = 0; i < CNT; ++i) {
      const int id = tid + i * NT;
      if (id < TOTAL)
        *reinterpret_cast<uint4*>(tile + (TT ? tt_off<D>(id / CPR, id % CPR)
                                             : rm_off<D>(id / CPR, id % CPR))) = r[i];
    }
  }
};

__device__ __forceinline__ uint32_t word_of(const uint4& x, int i) {
  return i < 2 ? (i == 0 ? x.x : x.y) : (i == 2 ? x.z : x.w);
}

// A resource over rows [0, L) of one head of a token-major [*, stride] fp16 matrix starting at
// `base` (the sequence's first row, this head's first column).
__device__ __forceinline__ rsrc_t rows_rsrc(const uint16_t* base, int L, int64_t stride, int D) {
  return make_rsrc(base, L > 0 ? (uint32_t)(((int64_t)(L - 1) * stride + D) * 2) : 0u);
}

// One token's D/16 MFMA operands (chunks 2 kk + l/32 of row `row`) from a row resource.
template <int D>
__device__ __forceinline__ void load_token(rsrc_t src, int row, int stride_b, int lane,
                                           half8_t (&out)[D / 16]) {
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk)
    out[kk] = __builtin_bit_cast(
        half8_t, buf_load16(src, (uint32_t)(row * stride_b + (2 * kk + (lane >> 5)) * 16)));
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

// Stores 32 x D fp32 values of one token (lane & 31) held as D/32 accumulators (d in the rows).
template <int D>
__device__ __forceinline__ void store_token_row_f32(float* row, const f32x16 (&acc)[D / 32],
                                                    int lane) {
#pragma unroll
  for (int u = 0; u < D / 32; ++u)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = 32 * u + 8 * j + 4 * (lane >> 5);
      *reinterpret_cast<float4*>(row + d) =
          make_float4(acc[u][4 * j], acc[u][4 * j + 1], acc[u][4 * j + 2], acc[u][4 * j + 3]);
    }
}

// ------------------------------------------------------------------------------------------------
// Forward: O = softmax(scale Q K^T + causal mask) V per sequence, and the log-sum-exp.
// grid (ceil(max_len / 32) * nseq * KH, 1, chunks), block 64 * G (G = HQ / KH q heads, one per
// wavefront). Key blocks of 64 keys: block kb + 1 is loaded into registers while block kb is
// multiplied. The longest query tiles' key ranges set the kernel's time when the batch has few
// sequences (the rest of the GPU idles): cutting the range into chunks spreads one tile over
// several workgroups.
// ------------------------------------------------------------------------------------------------
template <int D, int G>
__global__ __launch_bounds__(64 * G) void attn_fwd_kernel(Args a) {
  constexpr int KC = D / 16, DT = D / 32, NT = 64 * G;
  __shared__ __align__(16) uint16_t ks[kKB * D];
  __shared__ __align__(16) uint16_t vs[kKB * D];
  // blockIdx.x = tile + ntiles (seq KH + kvh), the tile fastest: consecutive workgroups (which
  // the dispatcher deals to the 8 XCDs in turn) take tiles of the same sequence, so every XCD
  // gets a share of each; the longest rows first
  const int sh = blockIdx.x / a.ntiles;
  const int tile = a.ntiles - 1 - (int)(blockIdx.x - sh * a.ntiles);
  const int seq = sh / a.KH, kvh = sh % a.KH;
  const int q0 = tile * kTok;
  const int start = a.cu[seq], L = a.cu[seq + 1] - start;
  if (q0 >= L) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int h = kvh * G + __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int qi = q0 + (lane & 31);
  const int64_t qs = (int64_t)a.HQ * D, kvs = (int64_t)a.KH * D;
  const int kvs_b = (int)(kvs * 2);
  const int kend = min(q0 + kTok, L);
  const int nkb = (kend + kKB - 1) / kKB;
  const int nch = num_chunks(nkb, a.chunk), ch = blockIdx.z;
  if (ch >= nch) return;
  const int kb0 = ch * a.chunk, kb1 = nch == 1 ? nkb : min(nkb, kb0 + a.chunk);
  const rsrc_t ksrc = rows_rsrc(a.k + (int64_t)start * kvs + kvh * D, L, kvs, D);
  const rsrc_t vsrc = rows_rsrc(a.v + (int64_t)start * kvs + kvh * D, L, kvs, D);

  RowStage<D, kKB, NT> sk;
  RowStage<D, kKB, NT, true> sv;
  sk.load(ksrc, kb0 * kKB, kvs_b, tid);
  sv.load(vsrc, kb0 * kKB, kvs_b, tid);

  half8_t qr[KC];  // queries past the sequence read zeros (their rows are not stored)
  load_token<D>(rows_rsrc(a.q + (int64_t)start * qs + h * D, L, qs, D), qi, (int)(qs * 2), lane,
                qr);
  f32x16 o[DT];
#pragma unroll
  for (int u = 0; u < DT; ++u) o[u] = f32x16{};
  float m = -__builtin_inff(), lsum = 0.f;
  const float c = a.scale * kLog2e;
  const int lim = min(qi, L - 1);  // the last key this query attends to

  // one key block from the staged tiles (ks, vs)
  auto block = [&](int k0) {
    f32x16 s[2];
    s[0] = s[1] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < KC; ++kk) {
      const half8_t k0op = ld_rm<D>(ks, lane & 31, 2 * kk + (lane >> 5));
      const half8_t k1op = ld_rm<D>(ks, 32 + (lane & 31), 2 * kk + (lane >> 5));
      s[0] = mfma(k0op, qr[kk], s[0]);
      s[1] = mfma(k1op, qr[kk], s[1]);
    }
    if (k0 + kKB - 1 > q0) {  // a block on the diagonal (uniform): mask keys past the query
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          s[t][r] = k0 + 32 * t + acc_row(r, lane) > lim ? -__builtin_inff() : s[t][r];
    }
    // the state is in log2 units of the scaled scores: m = max(c s), p = 2^(c s - m)
    float mx = -__builtin_inff();
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[t][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mnew = fmaxf(m, mx * c);
    const float alpha = ex2(m - mnew);
    m = mnew;
    float ps = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = ex2(fmaf(s[t][r], c, -mnew));
        s[t][r] = p;
        ps += p;
      }
    lsum = lsum * alpha + ps;
    if (__any(alpha != 1.f)) {  // once the running maxima settle, most blocks skip this
#pragma unroll
      for (int u = 0; u < DT; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[u][r] *= alpha;
    }
    half8_t pb[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) pb[kk] = to_b(s[kk >> 1], kk & 1);
#pragma unroll
    for (int u = 0; u < DT; ++u) {
      half8_t vop[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) vop[kk] = tr_operand<D>(vs, 16 * kk, 32 * u, lane);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) o[u] = mfma(vop[kk], pb[kk], o[u]);
    }
  };

  for (int kb = kb0; kb < kb1; ++kb) {
    __syncthreads();
    sk.store(ks, tid);
    sv.store(vs, tid);
    __syncthreads();
    // the next block (past the sequence: zeros, not used)
    sk.load(ksrc, (kb + 1) * kKB, kvs_b, tid);
    sv.load(vsrc, (kb + 1) * kKB, kvs_b, tid);
    block(kb * kKB);
  }
  const float ltot = lsum + __shfl_xor(lsum, 32, 64);
  if (nch == 1) {
    if (qi < L) {
      store_token_row<D>(a.out + (int64_t)(start + qi) * qs + h * D, o, 1.0f / ltot, lane);
      if (lane < 32) a.lse[(int64_t)h * a.n + start + qi] = (m + log2f(ltot)) * kLn2;
    }
    return;
  }
  // Several chunks: this one's unnormalised partial and (m, l). Every chunk holds at least one
  // unmasked key of each query (the last one starts at or before the tile's first query: q0 is
  // a multiple of 32, blocks are 64 keys; the others precede it), so m is finite.
  if (qi < L) {
    store_token_row_f32<D>(a.part + (((int64_t)ch * a.n + start + qi) * a.HQ + h) * D, o, lane);
    if (lane < 32)
      a.part_ml[((int64_t)ch * a.HQ + h) * a.n + start + qi] = make_float2(m, ltot);
  }
}

// ------------------------------------------------------------------------------------------------
// Backward, delta = rowsum(dO * O) per (q head, token), fp32 [HQ, n], read by both the dQ and the
// dK/dV kernel (which may then run at the same time). Two threads per row: thread `half` sums
// the products of the 16-byte chunks 2 kk + half (kk = 0 .. D/16 - 1) in order, then the pair's
// two sums are added.
// ------------------------------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void attn_delta_kernel(const uint16_t* dout, const uint16_t* o,
                                                         float* delta, int64_t n, int HQ) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t p = t >> 1;  // h n + token
  const int half = (int)(t & 1);
  const bool ok = p < n * HQ;
  float s = 0.f;
  if (ok) {
    const int64_t h = p / n, tok = p - h * n;
    const uint4* dr = reinterpret_cast<const uint4*>(dout + (tok * HQ + h) * D);
    const uint4* orow = reinterpret_cast<const uint4*>(o + (tok * HQ + h) * D);
    uint4 x[D / 16], y[D / 16];
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      x[kk] = dr[2 * kk + half];
      y[kk] = orow[2 * kk + half];
    }
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t xa = word_of(x[kk], w), ya = word_of(y[kk], w);
        s += lo_h(xa) * lo_h(ya);
        s += hi_h(xa) * hi_h(ya);
      }
  }
  const float tot = s + __shfl_xor(s, 1, 64);
  if (ok && half == 0) delta[p] = tot;
}

// ------------------------------------------------------------------------------------------------
// Backward, dQ: per 32 queries of a q head, over 32-key blocks up to the diagonal: S^T = K Q^T,
// P = exp(S - lse), dP^T = V dO^T, dS = P (dP - delta), dQ^T += K^T dS^T. grid and block as the
// forward; block kb + 1 prefetched during block kb. OWN_DELTA: the kernel forms delta itself
// (lanes l and l ^ 32 sum the chunks of attn_delta_kernel's two threads, in its order) and the
// first chunk writes it for the dK/dV kernel that follows; else it reads attn_delta_kernel's.
// ------------------------------------------------------------------------------------------------
template <int D, int G, bool OWN_DELTA>
__global__ __launch_bounds__(64 * G) void attn_dq_kernel(Args a) {
  constexpr int KC = D / 16, DT = D / 32, NT = 64 * G, KB = kTok;
  __shared__ __align__(16) uint16_t ks[KB * D];  // tt_off: read by rows and transposed
  __shared__ __align__(16) uint16_t vs[KB * D];
  const int sh = blockIdx.x / a.ntiles;  // as the forward
  const int tile = a.ntiles - 1 - (int)(blockIdx.x - sh * a.ntiles);
  const int seq = sh / a.KH, kvh = sh % a.KH;
  const int q0 = tile * kTok;
  const int start = a.cu[seq], L = a.cu[seq + 1] - start;
  if (q0 >= L) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int h = kvh * G + __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int qi = q0 + (lane & 31);
  const int64_t qs = (int64_t)a.HQ * D, kvs = (int64_t)a.KH * D;
  const int qs_b = (int)(qs * 2), kvs_b = (int)(kvs * 2);
  const int kend = min(q0 + kTok, L);
  const int nkb = (kend + KB - 1) / KB;
  const int nch = num_chunks(nkb, a.chunk), ch = blockIdx.z;
  if (ch >= nch) return;
  const int kb0 = ch * a.chunk, kb1 = nch == 1 ? nkb : min(nkb, kb0 + a.chunk);
  const rsrc_t ksrc = rows_rsrc(a.k + (int64_t)start * kvs + kvh * D, L, kvs, D);
  const rsrc_t vsrc = rows_rsrc(a.v + (int64_t)start * kvs + kvh * D, L, kvs, D);

  RowStage<D, KB, NT, true> sk;  // K: one tile for S^T = K Q^T and K^T (tr_operand)
  RowStage<D, KB, NT> sv;
  sk.load(ksrc, kb0 * KB, kvs_b, tid);
  sv.load(vsrc, kb0 * KB, kvs_b, tid);

  // this query's q and dO (queries past the sequence read zeros; their dq is not stored), its
  // log-sum-exp and delta (attn_delta_kernel)
  const int64_t hoff = (int64_t)start * qs + h * D;
  half8_t qr[KC], dr[KC];
  load_token<D>(rows_rsrc(a.q + hoff, L, qs, D), qi, qs_b, lane, qr);
  load_token<D>(rows_rsrc(a.dout + hoff, L, qs, D), qi, qs_b, lane, dr);
  const float lse2 =
      buf_load_f32(make_rsrc(a.lse + (int64_t)h * a.n + start, (uint32_t)L * 4), qi * 4) *
      kLog2e;
  float delta;
  if constexpr (OWN_DELTA) {
    half8_t orow[KC];
    load_token<D>(rows_rsrc(a.o + hoff, L, qs, D), qi, qs_b, lane, orow);
    float dpart = 0.f;
#pragma unroll
    for (int kk = 0; kk < KC; ++kk)
#pragma unroll
      for (int i = 0; i < 8; ++i) dpart += (float)dr[kk][i] * (float)orow[kk][i];
    delta = dpart + __shfl_xor(dpart, 32, 64);
    if (ch == 0 && qi < L && lane < 32) a.delta[(int64_t)h * a.n + start + qi] = delta;
  } else {
    delta = buf_load_f32(make_rsrc(a.delta + (int64_t)h * a.n + start, (uint32_t)L * 4), qi * 4);
  }

  f32x16 dq[DT];
#pragma unroll
  for (int u = 0; u < DT; ++u) dq[u] = f32x16{};
  const float c = a.scale * kLog2e;
  const int lim = min(qi, L - 1);

  for (int kb = kb0; kb < kb1; ++kb) {
    const int k0 = kb * KB;
    __syncthreads();
    sk.store(ks, tid);
    sv.store(vs, tid);
    __syncthreads();
    sk.load(ksrc, k0 + KB, kvs_b, tid);
    sv.load(vsrc, k0 + KB, kvs_b, tid);
    f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
    for (int kk = 0; kk < KC; ++kk) {
      const int row = lane & 31, ch = 2 * kk + (lane >> 5);
      const half8_t kop = ld_tt<D>(ks, row, ch), vop = ld_rm<D>(vs, row, ch);
      s = mfma(kop, qr[kk], s);
      dp = mfma(vop, dr[kk], dp);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = ex2(fmaf(s[r], c, -lse2));
    if (k0 + KB - 1 > q0) {  // a block on the diagonal (uniform)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = k0 + acc_row(r, lane) > lim ? 0.f : s[r];
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] *= dp[r] - delta;
    half8_t sb[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) sb[kk] = to_b(s, kk);
#pragma unroll
    for (int u = 0; u < DT; ++u) {
      const half8_t t0 = tr_operand<D>(ks, 0, 32 * u, lane);
      const half8_t t1 = tr_operand<D>(ks, 16, 32 * u, lane);
      dq[u] = mfma(t0, sb[0], dq[u]);
      dq[u] = mfma(t1, sb[1], dq[u]);
    }
  }
  if (nch == 1) {
    if (qi < L) store_token_row<D>(a.out + (int64_t)(start + qi) * qs + h * D, dq, a.scale, lane);
    return;
  }
  // several chunks: this one's unscaled partial
  if (qi < L)
    store_token_row_f32<D>(a.part + (((int64_t)ch * a.n + start + qi) * a.HQ + h) * D, dq, lane);
}

// ------------------------------------------------------------------------------------------------
// Merge of the chunks' partials, in chunk order. Forward: M = max m_c, l = sum l_c 2^(m_c - M),
// O = sum o_c 2^(m_c - M) / l, lse = (M + log2 l) ln 2; dQ: dq = scale sum dq_c. One thread per
// 4 columns of a query row: all C chunk loads are issued before any use (chunks past the tile's
// count read the last one again and weigh 0). blockIdx.x = tile + ntiles (q head of the group +
// G (seq KH + kvh)), block 32 D/4; tiles of one chunk were written directly and are skipped.
// ------------------------------------------------------------------------------------------------
template <int D, int C, bool FWD>
__global__ __launch_bounds__(32 * D / 4) void attn_merge_kernel(Args a) {
  constexpr int D4 = D / 4, KBLK = FWD ? kKB : kTok;
  const int G = a.HQ / a.KH;
  const int rest = blockIdx.x / a.ntiles;
  const int tile = (int)(blockIdx.x - rest * a.ntiles);
  const int g = rest % G, sh = rest / G;
  const int seq = sh / a.KH, h = (sh % a.KH) * G + g;
  const int q0 = tile * kTok;
  const int start = a.cu[seq], L = a.cu[seq + 1] - start;
  if (q0 >= L) return;
  const int kend = min(q0 + kTok, L);
  const int nch = num_chunks((kend + KBLK - 1) / KBLK, a.chunk);
  const int qi = q0 + (int)(threadIdx.x / D4), d4 = (int)(threadIdx.x % D4);
  if (nch == 1 || qi >= L) return;
  const int64_t cstride = a.n * a.HQ * D, mstride = (int64_t)a.HQ * a.n;
  const float* src = a.part + ((int64_t)(start + qi) * a.HQ + h) * D + 4 * d4;
  float4 x[C];
  float w[C];
#pragma unroll
  for (int c = 0; c < C; ++c) x[c] = *reinterpret_cast<const float4*>(src + min(c, nch - 1) * cstride);
  float M = 0.f, l = 0.f;
  if constexpr (FWD) {
    const float2* ml = a.part_ml + (int64_t)h * a.n + start + qi;
    float2 y[C];
#pragma unroll
    for (int c = 0; c < C; ++c) y[c] = ml[min(c, nch - 1) * mstride];
    M = -__builtin_inff();
#pragma unroll
    for (int c = 0; c < C; ++c) M = fmaxf(M, y[c].x);  // repeats of the last chunk change nothing
#pragma unroll
    for (int c = 0; c < C; ++c) {
      w[c] = c < nch ? ex2(y[c].x - M) : 0.f;
      l += y[c].y * w[c];
    }
    const float inv = 1.0f / l;
#pragma unroll
    for (int c = 0; c < C; ++c) w[c] *= inv;
  } else {
#pragma unroll
    for (int c = 0; c < C; ++c) w[c] = c < nch ? a.scale : 0.f;
  }
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    acc.x += w[c] * x[c].x;
    acc.y += w[c] * x[c].y;
    acc.z += w[c] * x[c].z;
    acc.w += w[c] * x[c].w;
  }
  *reinterpret_cast<uint2*>(a.out + ((int64_t)(start + qi) * a.HQ + h) * D + 4 * d4) =
      make_uint2(pack2h(acc.x, acc.y), pack2h(acc.z, acc.w));
  if (FWD && d4 == 0) a.lse[(int64_t)h * a.n + start + qi] = (M + log2f(l)) * kLn2;
}

// ------------------------------------------------------------------------------------------------
// Backward, dK and dV of one q head: a workgroup of 4 wavefronts owns 128 consecutive keys (32
// per wavefront) and walks the 32-query blocks from its first key to the end of the sequence,
// staging each block's Q and dO (rows and transposed, plus lse and delta) once for the four
// wavefronts: S = Q K^T, P = exp(S - lse), dP = dO V^T, dS = P (dP - delta), dV^T += dO^T P,
// dK^T += Q^T dS. A wavefront skips query blocks that lie wholly before its keys.
// grid (nseq * HQ * ceil(max_len / 128)), block 256.
// ------------------------------------------------------------------------------------------------
constexpr int kKeyWaves = 4;

template <int D>
__global__ __launch_bounds__(64 * kKeyWaves) void attn_dkdv_kernel(Args a) {
  constexpr int KC = D / 16, DT = D / 32, NT = 64 * kKeyWaves;
  __shared__ __align__(16) uint16_t qsm[kTok * D];  // tt_off: read by rows and transposed
  __shared__ __align__(16) uint16_t dsm[kTok * D];
  __shared__ __align__(16) float lse_s[kTok];
  __shared__ __align__(16) float dl_s[kTok];
  // blockIdx.x = (seq HQ + h) + pairs key tile: the first key tiles of every sequence and head,
  // which walk the most queries, are dispatched first (with more workgroups than CUs, the
  // heaviest then do not wait for a free CU)
  const int pairs = (int)(gridDim.x / a.ntiles);
  const int kt = blockIdx.x / pairs, sh = (int)(blockIdx.x - kt * pairs);
  const int seq = sh / a.HQ, h = sh % a.HQ;
  const int kvh = h / (a.HQ / a.KH);
  const int kw0 = kt * kTok * kKeyWaves;
  const int start = a.cu[seq], L = a.cu[seq + 1] - start;
  if (kw0 >= L) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int k0 = kw0 + kTok * wave;
  const int kj = k0 + (lane & 31);
  const int64_t qs = (int64_t)a.HQ * D, kvs = (int64_t)a.KH * D;
  const int qs_b = (int)(qs * 2), kvs_b = (int)(kvs * 2);
  const int64_t hoff = (int64_t)start * qs + h * D;
  const rsrc_t qsrc = rows_rsrc(a.q + hoff, L, qs, D);
  const rsrc_t dsrc = rows_rsrc(a.dout + hoff, L, qs, D);
  const rsrc_t lsrc = make_rsrc(a.lse + (int64_t)h * a.n + start, (uint32_t)L * 4);
  const rsrc_t dlsrc = make_rsrc(a.delta + (int64_t)h * a.n + start, (uint32_t)L * 4);

  RowStage<D, kTok, NT, true> sq, sd;
  float lv = 0.f;  // threads 0..31: lse (log2) of query q0 + tid; 32..63: delta of q0 + tid - 32
  const float first = tid < kTok ? 1.f : 0.f;
  auto load = [&](int q0) {
    sq.load(qsrc, q0, qs_b, tid);
    sd.load(dsrc, q0, qs_b, tid);
    const uint32_t off = (uint32_t)(q0 + (tid & (kTok - 1))) * 4;
    const float xl = buf_load_f32(lsrc, off), xd = buf_load_f32(dlsrc, off);
    lv = fmaf(first, xl * kLog2e, (1.f - first) * xd);  // a blend, not a select of loads
  };
  load(kw0);

  half8_t kr[KC], vr[KC];  // keys past the sequence read zeros (their rows are not stored)
  {
    const int64_t koff = (int64_t)start * kvs + kvh * D;
    load_token<D>(rows_rsrc(a.k + koff, L, kvs, D), kj, kvs_b, lane, kr);
    load_token<D>(rows_rsrc(a.v + koff, L, kvs, D), kj, kvs_b, lane, vr);
  }
  f32x16 dk[DT], dv[DT];
#pragma unroll
  for (int u = 0; u < DT; ++u) dk[u] = dv[u] = f32x16{};
  const float c = a.scale * kLog2e;

  for (int q0 = kw0; q0 < L; q0 += kTok) {
    __syncthreads();
    sq.store(qsm, tid);
    sd.store(dsm, tid);
    if (tid < 2 * kTok) (tid < kTok ? lse_s : dl_s)[tid & (kTok - 1)] = lv;
    __syncthreads();
    load(q0 + kTok);  // the next block (past the sequence: zeros, not used)
    if (q0 + kTok <= k0 || k0 >= L) continue;  // every query of the block precedes these keys
    f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
    for (int kk = 0; kk < KC; ++kk) {
      const int row = lane & 31, ch = 2 * kk + (lane >> 5);
      const half8_t qop = ld_tt<D>(qsm, row, ch), dop = ld_tt<D>(dsm, row, ch);
      s = mfma(qop, kr[kk], s);
      dp = mfma(dop, vr[kk], dp);
    }
    // masks only where the block reaches the diagonal or the end of the sequence (uniform)
    const bool edge = q0 < k0 + kTok || q0 + kTok > L;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int qr0 = 8 * j + 4 * (lane >> 5);
      const float4 l4 = *reinterpret_cast<const float4*>(lse_s + qr0);
      const float4 d4 = *reinterpret_cast<const float4*>(dl_s + qr0);
      const float lq[4] = {l4.x, l4.y, l4.z, l4.w}, dq4[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * j + i;
        s[r] = ex2(fmaf(s[r], c, -lq[i]));
        if (edge) {
          const int qq = q0 + qr0 + i;
          s[r] = (qq < L && kj <= qq) ? s[r] : 0.f;
        }
        dp[r] = s[r] * (dp[r] - dq4[i]);
      }
    }
    half8_t pb[2], sb[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      pb[kk] = to_b(s, kk);
      sb[kk] = to_b(dp, kk);
    }
#pragma unroll
    for (int u = 0; u < DT; ++u) {
      const half8_t d0 = tr_operand<D>(dsm, 0, 32 * u, lane);
      const half8_t d1 = tr_operand<D>(dsm, 16, 32 * u, lane);
      const half8_t q0op = tr_operand<D>(qsm, 0, 32 * u, lane);
      const half8_t q1op = tr_operand<D>(qsm, 16, 32 * u, lane);
      dv[u] = mfma(d0, pb[0], dv[u]);
      dk[u] = mfma(q0op, sb[0], dk[u]);
      dv[u] = mfma(d1, pb[1], dv[u]);
      dk[u] = mfma(q1op, sb[1], dk[u]);
    }
  }
  if (kj < L) {
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
  QLORA_CHECK_ARG(HQ > 0 && KH > 0 && HQ % KH == 0);
  const int G = HQ / KH;
  QLORA_CHECK_ARG(G >= 1 && G <= 8);  // every Qwen2 size: 14/2, 12/2, 16/2, 28/4, 40/8, 64/8
  QLORA_CHECK_ARG((int64_t)nseq * HQ < (1ll << 31));
  // buffer offsets within one sequence's rows (plus the prefetch past its end) fit 32 bits
  QLORA_CHECK_ARG(((int64_t)max_len + 4 * kKB) * HQ * D * 2 < (1ll << 31));
  return 0;
}

// MODE: 0 forward, 1 dQ reading delta, 2 dQ forming delta
template <int D, int G, int MODE>
void launch_q(const Args& a, dim3 grid, hipStream_t s) {
  if constexpr (MODE == 1)
    hipLaunchKernelGGL((attn_dq_kernel<D, G, false>), grid, dim3(64 * G), 0, s, a);
  else if constexpr (MODE == 2)
    hipLaunchKernelGGL((attn_dq_kernel<D, G, true>), grid, dim3(64 * G), 0, s, a);
  else hipLaunchKernelGGL((attn_fwd_kernel<D, G>), grid, dim3(64 * G), 0, s, a);
}

template <int MODE, int D>
void launch_q_g(const Args& a, int G, dim3 grid, hipStream_t s) {
  switch (G) {
    case 1: launch_q<D, 1, MODE>(a, grid, s); break;
    case 2: launch_q<D, 2, MODE>(a, grid, s); break;
    case 3: launch_q<D, 3, MODE>(a, grid, s); break;
    case 4: launch_q<D, 4, MODE>(a, grid, s); break;
    case 5: launch_q<D, 5, MODE>(a, grid, s); break;
    case 6: launch_q<D, 6, MODE>(a, grid, s); break;
    case 7: launch_q<D, 7, MODE>(a, grid, s); break;
    default: launch_q<D, 8, MODE>(a, grid, s); break;
  }
}

template <int MODE>
void launch_q_any(const Args& a, int D, int G, dim3 grid, hipStream_t s) {
  if (D == 128) launch_q_g<MODE, 128>(a, G, grid, s);
  else launch_q_g<MODE, 64>(a, G, grid, s);
}

// Chunks of the split forms: chunk_keys a positive multiple of 64, at most kMaxChunks chunks.
constexpr int kMaxChunks = 16;
int split_chunks(int32_t max_len, int32_t chunk_keys, int64_t* nch) {
  QLORA_CHECK_ARG(chunk_keys >= kKB && chunk_keys % kKB == 0);
  *nch = qlora_cdiv(max_len, chunk_keys);
  QLORA_CHECK_ARG(*nch >= 1 && *nch <= kMaxChunks);
  return 0;
}

// Workgroups of one launch: tiles x (sequence, head) pairs, within the 32-bit grid.
int grid_of(int64_t tiles, int64_t pairs, unsigned* x) {
  QLORA_CHECK_ARG(tiles * pairs < (1ll << 31));
  *x = (unsigned)(tiles * pairs);
  return 0;
}

// The merge kernel for nch chunks (C: the next supported count at or above it).
template <bool FWD>
int launch_merge(const Args& a, int D, int64_t nseq, int64_t nch, hipStream_t s) {
  unsigned gx;
  if (int rc = grid_of(a.ntiles, nseq * a.HQ, &gx)) return rc;
#define QLORA_MERGE(DD, CC) \
  hipLaunchKernelGGL((attn_merge_kernel<DD, CC, FWD>), dim3(gx), dim3(32 * DD / 4), 0, s, a)
  if (D == 128) {
    if (nch <= 2) QLORA_MERGE(128, 2);
    else if (nch <= 4) QLORA_MERGE(128, 4);
    else if (nch <= 8) QLORA_MERGE(128, 8);
    else QLORA_MERGE(128, 16);
  } else {
    if (nch <= 2) QLORA_MERGE(64, 2);
    else if (nch <= 4) QLORA_MERGE(64, 4);
    else if (nch <= 8) QLORA_MERGE(64, 8);
    else QLORA_MERGE(64, 16);
  }
#undef QLORA_MERGE
  return qlora_launch_status();
}

int run_fwd(Args a, int32_t nseq, int32_t max_len, int D, int64_t nch, hipStream_t s) {
  a.ntiles = (int)qlora_cdiv(max_len, kTok);
  unsigned gx;
  if (int rc = grid_of(a.ntiles, (int64_t)nseq * a.KH, &gx)) return rc;
  launch_q_any<0>(a, D, a.HQ / a.KH, dim3(gx, 1, (unsigned)nch), s);
  if (int rc = qlora_launch_status()) return rc;
  return nch > 1 ? launch_merge<true>(a, D, nseq, nch, s) : 0;
}

// The second stream of each device on which the dK/dV kernel runs while the dQ kernel runs on
// the caller's stream (both only read what the delta kernel and the forward wrote): neither
// launch alone fills the GPU when the batch holds few sequences. Fork and join are event
// waits, so the caller's stream orders everything after the backward as before. Created on
// first use (default priority), kept for the process.
struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
std::mutex g_side_mu;
SideStream g_side[64];

int side_stream(SideStream** out) {
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev)) return (int)e;
  if (dev < 0 || dev >= 64) return (int)hipErrorInvalidDevice;
  SideStream& ss = g_side[dev];
  if (ss.stream == nullptr) {
    if (hipError_t e = hipStreamCreateWithFlags(&ss.stream, hipStreamNonBlocking)) return (int)e;
    if (hipError_t e = hipEventCreateWithFlags(&ss.fork, hipEventDisableTiming)) return (int)e;
    if (hipError_t e = hipEventCreateWithFlags(&ss.join, hipEventDisableTiming)) return (int)e;
  }
  *out = &ss;
  return 0;
}

// Concurrent dQ and dK/dV pay when the dQ launch is long but leaves most of the GPU idle (few
// long sequences: at most ~1.25 workgroups per CU of 256, key ranges of 512 and more); a full
// launch gains nothing from the second stream and pays the delta kernel and the fork.
bool bwd_concurrent(int32_t max_len, unsigned dq_groups) {
  return max_len >= 512 && dq_groups <= 320;
}

void launch_dkdv(const Args& b, int D, unsigned gkv, hipStream_t s) {
  if (D == 128)
    hipLaunchKernelGGL(attn_dkdv_kernel<128>, dim3(gkv), dim3(64 * kKeyWaves), 0, s, b);
  else
    hipLaunchKernelGGL(attn_dkdv_kernel<64>, dim3(gkv), dim3(64 * kKeyWaves), 0, s, b);
}

int run_bwd(Args a, int32_t nseq, int32_t max_len, int D, int64_t nch, hipStream_t s) {
  Args b = a;  // dK/dV
  b.ntiles = (int)qlora_cdiv(max_len, kTok * kKeyWaves);
  unsigned gkv;
  if (int rc = grid_of(b.ntiles, (int64_t)nseq * a.HQ, &gkv)) return rc;
  a.ntiles = (int)qlora_cdiv(max_len, kTok);
  const int W = a.HQ / a.KH;
  unsigned gx;
  if (int rc = grid_of(a.ntiles, (int64_t)nseq * a.KH, &gx)) return rc;
  if (!bwd_concurrent(max_len, gx * (unsigned)nch)) {  // dQ (writing delta), then dK/dV
    launch_q_any<2>(a, D, W, dim3(gx, 1, (unsigned)nch), s);
    if (int rc = qlora_launch_status()) return rc;
    if (nch > 1) {
      if (int rc = launch_merge<false>(a, D, nseq, nch, s)) return rc;
    }
    launch_dkdv(b, D, gkv, s);
    return qlora_launch_status();
  }
  const int64_t rows = a.n * a.HQ;
  QLORA_CHECK_ARG(qlora_cdiv(2 * rows, 256) < (1ll << 31));
  const dim3 dgrid((unsigned)qlora_cdiv(2 * rows, 256));
  if (D == 128)
    hipLaunchKernelGGL(attn_delta_kernel<128>, dgrid, dim3(256), 0, s, a.dout, a.o, a.delta,
                       a.n, a.HQ);
  else
    hipLaunchKernelGGL(attn_delta_kernel<64>, dgrid, dim3(256), 0, s, a.dout, a.o, a.delta, a.n,
                       a.HQ);
  if (int rc = qlora_launch_status()) return rc;

  std::lock_guard<std::mutex> lock(g_side_mu);
  SideStream* ss;
  if (int rc = side_stream(&ss)) return rc;
  if (hipError_t e = hipEventRecord(ss->fork, s)) return (int)e;
  if (hipError_t e = hipStreamWaitEvent(ss->stream, ss->fork, 0)) return (int)e;
  launch_dkdv(b, D, gkv, ss->stream);
  int rc = qlora_launch_status();
  if (rc == 0) {
    launch_q_any<1>(a, D, W, dim3(gx, 1, (unsigned)nch), s);
    rc = qlora_launch_status();
  }
  if (rc == 0 && nch > 1) rc = launch_merge<false>(a, D, nseq, nch, s);
  // join whatever was launched, also after an error
  if (hipError_t e = hipEventRecord(ss->join, ss->stream)) return rc ? rc : (int)e;
  if (hipError_t e = hipStreamWaitEvent(s, ss->join, 0)) return rc ? rc : (int)e;
  return rc;
}

Args make_args(const void* q, const void* k, const void* v, int64_t n, int32_t HQ, int32_t KH,
               float scale, const int32_t* cu) {
  Args a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.cu = cu;
  a.n = n;
  a.HQ = HQ;
  a.KH = KH;
  a.scale = scale;
  return a;
}

// The split's chunk count and fp32 workspace for these sizes (none when max_len fits one chunk).
int split_sizes(int32_t max_len, int64_t n, int32_t HQ, int32_t D, int32_t chunk_keys,
                int64_t* nch, int64_t* work) {
  if (int rc = split_chunks(max_len, chunk_keys, nch)) return rc;
  *work = *nch == 1 ? 0 : *nch * n * HQ * (int64_t)(D + 2);
  return 0;
}

}  // namespace

// fp32 workspace elements of qlora_attn_fwd_split / qlora_attn_bwd_split for these sizes and
// chunk_keys (keys per workgroup: a positive multiple of 64 with ceil(max_len / chunk_keys)
// <= 16); 0 when max_len fits one chunk. No reference counterpart: a work split of the same
// attention.
QLORA_API int qlora_attn_split_workspace(int32_t max_len, int64_t n, int32_t HQ, int32_t D,
                                         int32_t chunk_keys, int64_t* work_elems) {
  QLORA_CHECK_ARG(work_elems && max_len >= 0 && n >= 0 && HQ > 0 && (D == 64 || D == 128));
  *work_elems = 0;
  if (max_len == 0 || n == 0) return 0;
  int64_t nch;
  return split_sizes(max_len, n, HQ, D, chunk_keys, &nch, work_elems);
}

// qlora_attn_fwd with each query tile's key range cut into chunks of chunk_keys keys (0: not
// cut), one workgroup each, and a second kernel that merges the fp32 partials in chunk order.
// work: fp32, 16-byte aligned, of qlora_attn_split_workspace elements. Same reference call site
// as qlora_attn_fwd (engine.py:857-862).
QLORA_API int qlora_attn_fwd_split(const void* q, const void* k, const void* v, void* out,
                                   float* lse, const int32_t* cu_seqlens, int32_t nseq,
                                   int32_t max_len, int64_t n, int32_t HQ, int32_t KH, int32_t D,
                                   float scale, int32_t chunk_keys, float* work,
                                   int64_t work_elems, void* stream) {
  if (int rc = check_common(nseq, max_len, n, HQ, KH, D)) return rc;
  if (n == 0 || nseq == 0 || max_len == 0) return 0;
  int64_t nch = 1, need = 0;
  if (chunk_keys != 0) {
    if (int rc = split_sizes(max_len, n, HQ, D, chunk_keys, &nch, &need)) return rc;
  }
  QLORA_CHECK_ARG(q && k && v && out && lse && cu_seqlens);
  QLORA_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out));
  QLORA_CHECK_ARG(work_elems >= need && (nch == 1 || (work && aligned16(work))));
  Args a = make_args(q, k, v, n, HQ, KH, scale, cu_seqlens);
  a.out = static_cast<uint16_t*>(out);
  a.lse = lse;
  if (nch > 1) {
    a.chunk = chunk_keys / kKB;
    a.part = work;
    a.part_ml = reinterpret_cast<float2*>(work + nch * n * HQ * D);
  }
  return run_fwd(a, nseq, max_len, D, nch, (hipStream_t)stream);
}

// Forward. q [n, HQ, D], k/v [n, KH, D], out [n, HQ, D] fp16 contiguous; lse fp32 [HQ, n];
// cu_seqlens int32 [nseq + 1] on the device, non-decreasing from 0 to n, every length
// <= max_len (the kernel reads no token outside [cu[s], cu[s + 1]) for sequence s).
QLORA_API int qlora_attn_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                             const int32_t* cu_seqlens, int32_t nseq, int32_t max_len, int64_t n,
                             int32_t HQ, int32_t KH, int32_t D, float scale, void* stream) {
  return qlora_attn_fwd_split(q, k, v, out, lse, cu_seqlens, nseq, max_len, n, HQ, KH, D, scale,
                              0, nullptr, 0, stream);
}

// qlora_attn_bwd with the dQ kernel's key range cut into chunks of chunk_keys keys (0: not cut),
// one workgroup each, summed in chunk order by a second kernel; dK/dV as in qlora_attn_bwd. work
// as for qlora_attn_fwd_split. Same reference call site (engine.py:865-869).
QLORA_API int qlora_attn_bwd_split(const void* dout, const void* q, const void* k, const void* v,
                                   const void* out, const float* lse, float* delta, void* dq,
                                   void* dk, void* dv, const int32_t* cu_seqlens, int32_t nseq,
                                   int32_t max_len, int64_t n, int32_t HQ, int32_t KH, int32_t D,
                                   float scale, int32_t chunk_keys, float* work,
                                   int64_t work_elems, void* stream) {
  if (int rc = check_common(nseq, max_len, n, HQ, KH, D)) return rc;
  if (n == 0 || nseq == 0 || max_len == 0) return 0;
  int64_t nch = 1, need = 0;
  if (chunk_keys != 0) {
    if (int rc = split_sizes(max_len, n, HQ, D, chunk_keys, &nch, &need)) return rc;
  }
  QLORA_CHECK_ARG(dout && q && k && v && out && lse && delta && dq && dk && dv && cu_seqlens);
  QLORA_CHECK_ARG(aligned16(dout) && aligned16(q) && aligned16(k) && aligned16(v) &&
                  aligned16(out) && aligned16(dq) && aligned16(dk) && aligned16(dv));
  QLORA_CHECK_ARG(work_elems >= need && (nch == 1 || (work && aligned16(work))));
  Args a = make_args(q, k, v, n, HQ, KH, scale, cu_seqlens);
  a.o = static_cast<const uint16_t*>(out);
  a.dout = static_cast<const uint16_t*>(dout);
  a.out = static_cast<uint16_t*>(dq);
  a.dk = static_cast<uint16_t*>(dk);
  a.dv = static_cast<uint16_t*>(dv);
  a.lse = const_cast<float*>(lse);
  a.delta = delta;
  if (nch > 1) {
    a.chunk = chunk_keys / kTok;
    a.part = work;
  }
  return run_bwd(a, nseq, max_len, D, nch, (hipStream_t)stream);
}

// Backward. dout/out/q [n, HQ, D], k/v [n, KH, D] as in the forward, lse from it; delta: fp32
// workspace [HQ, n]; dq, dk, dv fp16 [n, HQ, D] (dk/dv per q head, not yet summed over the
// q heads of a kv head).
QLORA_API int qlora_attn_bwd(const void* dout, const void* q, const void* k, const void* v,
                             const void* out, const float* lse, float* delta, void* dq, void* dk,
                             void* dv, const int32_t* cu_seqlens, int32_t nseq, int32_t max_len,
                             int64_t n, int32_t HQ, int32_t KH, int32_t D, float scale,
                             void* stream) {
  return qlora_attn_bwd_split(dout, q, k, v, out, lse, delta, dq, dk, dv, cu_seqlens, nseq,
                              max_len, n, HQ, KH, D, scale, 0, nullptr, 0, stream);
}
