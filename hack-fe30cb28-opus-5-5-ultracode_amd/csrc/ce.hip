// Cross-entropy over the 151,936-word vocabulary from fp16 logits: whole rows, or piece by piece
// with the online state carried in memory, and the finish step that forms the hidden-state
// gradient. Reference: lm_head_ce_kernel kernels.py:344-388 (_ce engine.py:1026-1030),
// lm_head_piece_kernel kernels.py:401-450 (_ce_piece engine.py:1033-1038),
// lm_head_finish_kernel kernels.py:458-479 (_ce_finish engine.py:1041-1045).
//
// Per row the online state is (m = running max, s = sum e^(x-m), t = sum e^(x-m) x, best logit,
// its first index). lse = m + log s, entropy = lse - t/s, loss = lse - x_target, correct =
// (argmax == target), first maximum wins.
//
// One 256-thread workgroup per row. The row is consumed in blocks of kCeBlock = 4096 columns
// (16 per thread, two 16-byte loads): each thread folds its 16 values, the workgroup merges the
// 256 partial states (wavefront butterfly, then LDS across the four wavefronts) into the block's
// state, and every thread folds that into the running row state in block order. A piece of the
// vocabulary that starts on a multiple of kCeBlock therefore runs exactly the same operations on
// the same blocks as the whole-row kernel: piece-wise loss/entropy/accuracy equal the whole-row
// ones bit for bit. The target's logit is captured by the thread that reads it in the first
// pass; in the second pass every thread rewrites only columns it read itself, after the last
// merge barrier: the in-place gradient cannot race with a read of the row.
#include "common.h"

namespace qlora {

constexpr int kCeThreads = 256;
constexpr int kCeVec = 8;                          // fp16 per 16-byte load
constexpr int kCePerThread = 16;                   // columns per thread per block
constexpr int kCeBlock = kCeThreads * kCePerThread;  // 4096
constexpr float kNegInf = -__builtin_huge_valf();

struct Online {
  float m, s, t, best;
  int32_t idx;
};

__device__ __forceinline__ Online online_empty() {
  return {kNegInf, 0.f, 0.f, kNegInf, 0x7fffffff};
}

__device__ __forceinline__ float rescale(float m_old, float m_new) {
  return m_old == kNegInf ? 0.f : __expf(m_old - m_new);
}

// Merge of two partial states over disjoint columns; ties of the best logit go to the smaller
// column index, so the result does not depend on the operand order for the argmax.
__device__ __forceinline__ Online merge(const Online& a, const Online& b) {
  Online r;
  r.m = fmaxf(a.m, b.m);
  const float fa = rescale(a.m, r.m), fb = rescale(b.m, r.m);
  r.s = a.s * fa + b.s * fb;
  r.t = a.t * fa + b.t * fb;
  const bool take_b = b.best > a.best || (b.best == a.best && b.idx < a.idx);
  r.best = take_b ? b.best : a.best;
  r.idx = take_b ? b.idx : a.idx;
  return r;
}

// Running row state `row` followed by a later block `blk`: a later column only wins with a
// strictly larger logit (first maximum wins).
__device__ __forceinline__ Online advance(const Online& row, const Online& blk) {
  Online r;
  r.m = fmaxf(row.m, blk.m);
  const float fa = rescale(row.m, r.m), fb = rescale(blk.m, r.m);
  r.s = row.s * fa + blk.s * fb;
  r.t = row.t * fa + blk.t * fb;
  const bool take = blk.best > row.best;
  r.best = take ? blk.best : row.best;
  r.idx = take ? blk.idx : row.idx;
  return r;
}

__device__ __forceinline__ void unpack8(const uint4 w, float* x) {
  x[0] = lo_h(w.x); x[1] = hi_h(w.x); x[2] = lo_h(w.y); x[3] = hi_h(w.y);
  x[4] = lo_h(w.z); x[5] = hi_h(w.z); x[6] = lo_h(w.w); x[7] = hi_h(w.w);
}

// The thread's 16 columns of block starting at b0: two runs of 8 at b0 + 8 t and
// b0 + 2048 + 8 t (each wavefront load covers 1 KiB contiguous). Columns >= width are -inf.
template <bool VEC>
__device__ __forceinline__ void load_block(const uint16_t* row, int64_t b0, int64_t width,
                                           float (&x)[kCePerThread]) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t c = b0 + h * (kCeBlock / 2) + (int64_t)threadIdx.x * kCeVec;
    if constexpr (VEC) {
      if (c + kCeVec <= width) {
        unpack8(*reinterpret_cast<const uint4*>(row + c), x + h * kCeVec);
        continue;
      }
    }
#pragma unroll
    for (int i = 0; i < kCeVec; ++i)
      x[h * kCeVec + i] = c + i < width ? h2f_bits(row[c + i]) : kNegInf;
  }
}
// Column of value j of thread t's 16 in the block starting at b0.
__device__ __forceinline__ int64_t col_of(int64_t b0, int j, int t = threadIdx.x) {
  return b0 + (j / kCeVec) * (kCeBlock / 2) + (int64_t)t * kCeVec + (j % kCeVec);
}

// Fold thread t's 16 values (fresh state), in increasing column order.
__device__ __forceinline__ Online fold16(const float (&x)[kCePerThread], int64_t b0,
                                        int t = threadIdx.x) {
  float mx = x[0];
  int j_best = 0;
#pragma unroll
  for (int j = 1; j < kCePerThread; ++j)
    if (x[j] > mx) { mx = x[j]; j_best = j; }
  Online st;
  st.m = mx;
  st.best = mx;
  st.idx = mx == kNegInf ? 0x7fffffff : (int32_t)col_of(b0, j_best, t);
  float se = 0.f, te = 0.f;
  if (mx != kNegInf) {
#pragma unroll
    for (int j = 0; j < kCePerThread; ++j) {
      const float e = __expf(x[j] - mx);  // -inf columns give 0
      se += e;
      te += x[j] == kNegInf ? 0.f : e * x[j];
    }
  }
  st.s = se;
  st.t = te;
  return st;
}

// The wavefront's state from its lanes' states, identical in every lane: the maximum first (a
// butterfly of fmaxf, exact), each lane's sums rescaled to it once, then butterflies of fp32 adds
// (a + b and b + a are the same float, so both lanes of a pair, and in the end all 64, hold the
// same bits) and of the best logit with its first column. One exponential per lane, where
// merging the full states level by level takes two per level.
__device__ __forceinline__ Online wave_state(const Online& st) {
  float m = st.m;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
  const float f = rescale(st.m, m);
  float s = st.s * f, t = st.t * f, best = st.best;
  int32_t idx = st.idx;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    s += __shfl_xor(s, off, kWave);
    t += __shfl_xor(t, off, kWave);
    const float ob = __shfl_xor(best, off, kWave);
    const int32_t oi = __shfl_xor(idx, off, kWave);
    const bool take = ob > best || (ob == best && oi < idx);
    best = take ? ob : best;
    idx = take ? oi : idx;
  }
  return {m, s, t, best, idx};
}

// The block's state, identical in every thread. `buf` alternates between two LDS slots so one
// barrier per block suffices.
__device__ __forceinline__ Online block_state(Online st, Online (*part)[kCeThreads / kWave],
                                              int buf) {
  st = wave_state(st);
  if ((threadIdx.x & (kWave - 1)) == 0) part[buf][threadIdx.x / kWave] = st;
  __syncthreads();
  Online r = part[buf][0];
#pragma unroll
  for (int i = 1; i < kCeThreads / kWave; ++i) r = merge(r, part[buf][i]);
  return r;
}

// Online pass over columns [0, width) of `row`, starting from `st`; also the logit at column
// `local` (0 if outside), reduced over the workgroup. Ends after a barrier.
template <bool VEC>
__device__ __forceinline__ Online scan(const uint16_t* row, int64_t width, int64_t local,
                                       Online st, float& xt) {
  __shared__ Online part[2][kCeThreads / kWave];
  __shared__ float xt_part[kCeThreads / kWave];
  float mine = 0.f;
  float x[kCePerThread];
  int buf = 0;
  if (width > 0) load_block<VEC>(row, 0, width, x);
  for (int64_t b0 = 0; b0 < width; b0 += kCeBlock, buf ^= 1) {
    float cur[kCePerThread];
#pragma unroll
    for (int j = 0; j < kCePerThread; ++j) cur[j] = x[j];
    if (b0 + kCeBlock < width) load_block<VEC>(row, b0 + kCeBlock, width, x);  // prefetch
    if (local >= b0 && local < b0 + kCeBlock) {
#pragma unroll
      for (int j = 0; j < kCePerThread; ++j)
        if (col_of(b0, j) == local) mine = cur[j];
    }
    st = advance(st, block_state(fold16(cur, b0), part, buf));
  }
  mine = wave_sum(mine);
  if ((threadIdx.x & (kWave - 1)) == 0) xt_part[threadIdx.x / kWave] = mine;
  __syncthreads();
  xt = 0.f;
#pragma unroll
  for (int i = 0; i < kCeThreads / kWave; ++i) xt += xt_part[i];
  return st;
}

// Rewrite columns [0, width) of the row with f(x, col), each thread its own columns.
template <bool VEC, class F>
__device__ __forceinline__ void rewrite(uint16_t* row, int64_t width, F f) {
  for (int64_t b0 = 0; b0 < width; b0 += kCeBlock) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t c = b0 + h * (kCeBlock / 2) + (int64_t)threadIdx.x * kCeVec;
      if (VEC && c + kCeVec <= width) {
        float x[kCeVec];
        unpack8(*reinterpret_cast<const uint4*>(row + c), x);
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = pack2h(f(x[2 * i], c + 2 * i), f(x[2 * i + 1], c + 2 * i + 1));
        *reinterpret_cast<uint4*>(row + c) = make_uint4(o[0], o[1], o[2], o[3]);
      } else {
        for (int i = 0; i < kCeVec; ++i)
          if (c + i < width) row[c + i] = f2h_bits(f(h2f_bits(row[c + i]), c + i));
      }
    }
  }
}

template <bool VEC>
__global__ __launch_bounds__(kCeThreads) void ce_full_kernel(uint16_t* logits, int64_t ld,
                                                             const int64_t* target,
                                                             float* loss, float* entropy,
                                                             int32_t* correct, int64_t V,
                                                             int zero_unsupervised) {
  const int64_t r = blockIdx.x;
  uint16_t* row = logits + r * ld;
  const int64_t tgt = target[r];
  float xt;
  const Online st = scan<VEC>(row, V, tgt, online_empty(), xt);
  const float lse = st.m + logf(st.s);
  const bool valid = tgt >= 0;
  if (threadIdx.x == 0) {
    entropy[r] = lse - st.t / st.s;
    loss[r] = valid ? lse - xt : 0.f;
    correct[r] = (int32_t)(valid && (int64_t)st.idx == tgt);
  }
  if (valid)
    rewrite<VEC>(row, V, [&](float x, int64_t c) {
      return __expf(x - lse) - (c == tgt ? 1.f : 0.f);
    });
  else if (zero_unsupervised)
    rewrite<VEC>(row, V, [](float, int64_t) { return 0.f; });
}

// Whole rows with the row held in registers: one 1024-thread workgroup per row, four groups of
// 256 threads; group g holds blocks g, g + 4, ... of the row (NB blocks at most, 16 columns per
// thread each, the same columns a thread of ce_full_kernel reads in that block), so the row is
// read from memory once and written once (ce_full_kernel reads it twice). The arithmetic is
// ce_full_kernel's, in its order: each block's state from the same per-thread folds and the
// same wavefront butterfly and four-wave merge, then the blocks advanced in column order; the
// results are equal bit for bit. Requires V % 8 == 0, 16-byte aligned rows, V <= NB 4 kCeBlock.
constexpr int kRowGroups = 4;
constexpr int kRowThreads = kCeThreads * kRowGroups;

template <int NB>
__global__ __launch_bounds__(kRowThreads) void ce_rows_kernel(uint16_t* logits, int64_t ld,
                                                              const int64_t* target, float* loss,
                                                              float* entropy, int32_t* correct,
                                                              int64_t V, int zero_unsupervised) {
  __shared__ Online wpart[NB * kRowGroups][kCeThreads / kWave];
  __shared__ Online blk[NB * kRowGroups];
  __shared__ Online fin;
  __shared__ float xt_part[kRowThreads / kWave];
  const int64_t r = blockIdx.x;
  uint16_t* row = logits + r * ld;
  const rsrc_t src = make_rsrc(row, (uint32_t)(V * 2));
  const int tid = threadIdx.x, grp = tid / kCeThreads, t = tid % kCeThreads;
  const int nblocks = (int)((V + kCeBlock - 1) / kCeBlock);
  const int64_t tgt = target[r];
  // every load issued before any use; blocks past the row read zeros (masked below)
  uint4 raw[NB][2];
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t c = (int64_t)(grp + kRowGroups * j) * kCeBlock + h * (kCeBlock / 2) + t * kCeVec;
      raw[j][h] = buf_load16(src, (uint32_t)(c * 2));
    }
  float mine = 0.f;
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int b = grp + kRowGroups * j;
    if (b >= nblocks) break;  // uniform over the wavefront
    const int64_t b0 = (int64_t)b * kCeBlock;
    float x[kCePerThread];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      unpack8(raw[j][h], x + h * kCeVec);
      const int64_t c = b0 + h * (kCeBlock / 2) + t * kCeVec;
      if (c >= V) {  // V % 8 == 0: a run is wholly inside or outside the row
#pragma unroll
        for (int i = 0; i < kCeVec; ++i) x[h * kCeVec + i] = kNegInf;
      }
      if (tgt >= c && tgt < c + kCeVec) {
#pragma unroll
        for (int i = 0; i < kCeVec; ++i)
          if (c + i == tgt) mine = x[h * kCeVec + i];
      }
    }
    // the block's state as block_state forms it: wavefront butterfly, then the four waves
    const Online st = wave_state(fold16(x, b0, t));
    if ((t & (kWave - 1)) == 0) wpart[b][t / kWave] = st;
  }
  mine = wave_sum(mine);
  if ((tid & (kWave - 1)) == 0) xt_part[tid / kWave] = mine;
  __syncthreads();
  if (tid < nblocks) {
    Online bs = wpart[tid][0];
#pragma unroll
    for (int i = 1; i < kCeThreads / kWave; ++i) bs = merge(bs, wpart[tid][i]);
    blk[tid] = bs;
  }
  __syncthreads();
  if (tid == 0) {
    Online st = online_empty();
    for (int b = 0; b < nblocks; ++b) st = advance(st, blk[b]);
    fin = st;
  }
  __syncthreads();
  const Online st = fin;
  float xt = 0.f;
#pragma unroll
  for (int i = 0; i < kRowThreads / kWave; ++i) xt += xt_part[i];
  const float lse = st.m + logf(st.s);
  const bool valid = tgt >= 0;
  if (tid == 0) {
    entropy[r] = lse - st.t / st.s;
    loss[r] = valid ? lse - xt : 0.f;
    correct[r] = (int32_t)(valid && (int64_t)st.idx == tgt);
  }
  if (!valid && !zero_unsupervised) return;
  // in place: fp16(e^(x - lse) - onehot), or zeros; stores past the row are dropped
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int b = grp + kRowGroups * j;
    if (b >= nblocks) break;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t c = (int64_t)b * kCeBlock + h * (kCeBlock / 2) + t * kCeVec;
      float x[kCeVec];
      unpack8(raw[j][h], x);
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float g0 = valid ? __expf(x[2 * i] - lse) - (c + 2 * i == tgt ? 1.f : 0.f) : 0.f;
        const float g1 =
            valid ? __expf(x[2 * i + 1] - lse) - (c + 2 * i + 1 == tgt ? 1.f : 0.f) : 0.f;
        o[i] = pack2h(g0, g1);
      }
      buf_store16(src, (uint32_t)(c * 2), make_uint4(o[0], o[1], o[2], o[3]));
    }
  }
}

template <bool VEC>
__global__ __launch_bounds__(kCeThreads) void ce_piece_kernel(
    uint16_t* logits, int64_t ld, const uint16_t* w, const int64_t* target, float* state,
    int32_t* best_idx, float* xt_out, float* alpha, uint16_t* wt, int64_t v0, int64_t width,
    int64_t n_sup, int64_t H) {
  const int64_t r = blockIdx.x;
  uint16_t* row = logits + r * ld;
  const int64_t tgt = target[r];
  const int64_t local = tgt >= 0 ? tgt - v0 : -1;
  Online prev;
  prev.m = state[r * 4 + 0];
  prev.s = state[r * 4 + 1];
  prev.t = state[r * 4 + 2];
  prev.best = state[r * 4 + 3];
  prev.idx = best_idx[r];
  // the block indices of this piece are local; shift the running best index into it
  Online st = prev;
  st.idx = (int32_t)(prev.idx - v0);
  float xt;
  st = scan<VEC>(row, width, local, st, xt);
  st.idx = (int32_t)(st.idx + v0);
  const bool in_piece = local >= 0 && local < width;
  if (threadIdx.x == 0) {
    state[r * 4 + 0] = st.m;
    state[r * 4 + 1] = st.s;
    state[r * 4 + 2] = st.t;
    state[r * 4 + 3] = st.best;
    best_idx[r] = st.idx;
    if (in_piece) xt_out[r] = xt;
    if (r < n_sup) alpha[r] = rescale(prev.m, st.m);
  }
  if (in_piece && r < n_sup) {
    const uint16_t* src = w + local * H;
    for (int64_t h = threadIdx.x; h < H; h += kCeThreads) wt[r * H + h] = src[h];
  }
  if (r < n_sup) {
    const float m = st.m;
    rewrite<VEC>(row, width, [&](float x, int64_t) { return __expf(x - m); });
  }
}

// After the last piece: the logits of one piece (rows < n_sup, recomputed) overwritten with
// fp16(e^(x - lse) - onehot), lse from the finished row state. The expression is the whole-row
// kernel's, and a row's state after all pieces equals the whole-row state bit for bit, so the
// piece's gradient rows equal the columns [v0, v0 + width) of the whole-row gradient.
template <bool VEC>
__global__ __launch_bounds__(kCeThreads) void ce_grad_kernel(uint16_t* logits, int64_t ld,
                                                             const int64_t* target,
                                                             const float* state, int64_t v0,
                                                             int64_t width) {
  const int64_t r = blockIdx.x;
  uint16_t* row = logits + r * ld;
  const float lse = state[r * 4 + 0] + logf(state[r * 4 + 1]);
  const int64_t local = target[r] >= 0 ? target[r] - v0 : -1;
  rewrite<VEC>(row, width, [&](float x, int64_t c) {
    return __expf(x - lse) - (c == local ? 1.f : 0.f);
  });
}

__global__ __launch_bounds__(kCeThreads) void ce_finish_kernel(
    const float* state, const int32_t* best_idx, const float* xt, const int64_t* target,
    float* loss, float* entropy, int32_t* correct, const float* acc, const uint16_t* wt,
    uint16_t* dh, int64_t n_sup, int64_t H) {
  const int64_t r = blockIdx.x;
  const float m = state[r * 4 + 0], s = state[r * 4 + 1], t = state[r * 4 + 2];
  const float lse = m + logf(s);
  const int64_t tgt = target[r];
  const bool valid = tgt >= 0;
  if (threadIdx.x == 0) {
    entropy[r] = lse - t / s;
    loss[r] = valid ? lse - xt[r] : 0.f;
    correct[r] = (int32_t)(valid && (int64_t)best_idx[r] == tgt);
  }
  if (r < n_sup) {
    for (int64_t h = threadIdx.x; h < H; h += kCeThreads)
      dh[r * H + h] = f2h_bits(acc[r * H + h] / s - h2f_bits(wt[r * H + h]));
  }
}

}  // namespace qlora

using namespace qlora;

namespace {
bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }
}

QLORA_API int qlora_ce(void* logits, int64_t ld, const int64_t* target, float* loss,
                       float* entropy, int32_t* correct, int64_t rows, int64_t V,
                       int32_t zero_unsupervised, void* stream) {
  QLORA_CHECK_ARG(rows >= 0 && V > 0 && ld >= V);
  if (rows == 0) return 0;
  QLORA_CHECK_ARG(logits && target && loss && entropy && correct);
  QLORA_CHECK_ARG(V < (1ll << 31) - kCeBlock && rows < (1ll << 31));
  const bool vec = ld % 8 == 0 && al16(logits);
  const int64_t nb = (qlora_cdiv(V, kCeBlock) + kRowGroups - 1) / kRowGroups;
  if (vec && V % 8 == 0 && nb <= 12) {
    hipStream_t s = (hipStream_t)stream;
    uint16_t* lg = static_cast<uint16_t*>(logits);
    const dim3 g((unsigned)rows), b(kRowThreads);
#define QLORA_CE_ROWS(NB)                                                                        \
  hipLaunchKernelGGL(ce_rows_kernel<NB>, g, b, 0, s, lg, ld, target, loss, entropy, correct, V, \
                     zero_unsupervised)
    if (nb <= 2) QLORA_CE_ROWS(2);
    else if (nb <= 4) QLORA_CE_ROWS(4);
    else if (nb <= 6) QLORA_CE_ROWS(6);
    else if (nb <= 8) QLORA_CE_ROWS(8);
    else if (nb <= 10) QLORA_CE_ROWS(10);
    else QLORA_CE_ROWS(12);
#undef QLORA_CE_ROWS
  } else if (vec)
    hipLaunchKernelGGL(ce_full_kernel<true>, dim3((unsigned)rows), dim3(kCeThreads), 0,
                       (hipStream_t)stream, static_cast<uint16_t*>(logits), ld, target, loss,
                       entropy, correct, V, zero_unsupervised);
  else
    hipLaunchKernelGGL(ce_full_kernel<false>, dim3((unsigned)rows), dim3(kCeThreads), 0,
                       (hipStream_t)stream, static_cast<uint16_t*>(logits), ld, target, loss,
                       entropy, correct, V, zero_unsupervised);
  return qlora_launch_status();
}

QLORA_API int qlora_ce_piece(void* logits, int64_t ld, const void* w, const int64_t* target,
                             float* state, int32_t* best_idx, float* xt, float* alpha,
                             void* wt, int64_t v0, int64_t rows, int64_t width, int64_t n_sup,
                             int64_t H, void* stream) {
  QLORA_CHECK_ARG(rows >= 0 && width > 0 && ld >= width && H > 0 && n_sup >= 0);
  if (rows == 0) return 0;
  QLORA_CHECK_ARG(logits && w && target && state && best_idx && xt);
  QLORA_CHECK_ARG(n_sup == 0 || (alpha && wt));
  QLORA_CHECK_ARG(v0 >= 0 && v0 + width < (1ll << 31) - kCeBlock && rows < (1ll << 31));
  const bool vec = ld % 8 == 0 && al16(logits);
  if (vec)
    hipLaunchKernelGGL(ce_piece_kernel<true>, dim3((unsigned)rows), dim3(kCeThreads), 0,
                       (hipStream_t)stream, static_cast<uint16_t*>(logits), ld,
                       static_cast<const uint16_t*>(w), target, state, best_idx, xt, alpha,
                       static_cast<uint16_t*>(wt), v0, width, n_sup, H);
  else
    hipLaunchKernelGGL(ce_piece_kernel<false>, dim3((unsigned)rows), dim3(kCeThreads), 0,
                       (hipStream_t)stream, static_cast<uint16_t*>(logits), ld,
                       static_cast<const uint16_t*>(w), target, state, best_idx, xt, alpha,
                       static_cast<uint16_t*>(wt), v0, width, n_sup, H);
  return qlora_launch_status();
}

QLORA_API int qlora_ce_finish(const float* state, const int32_t* best_idx, const float* xt,
                              const int64_t* target, float* loss, float* entropy,
                              int32_t* correct, const float* acc, const void* wt, void* dh,
                              int64_t rows, int64_t n_sup, int64_t H, void* stream) {
  QLORA_CHECK_ARG(rows >= 0 && n_sup >= 0 && n_sup <= rows && H > 0);
  if (rows == 0) return 0;
  QLORA_CHECK_ARG(state && best_idx && xt && target && loss && entropy && correct);
  QLORA_CHECK_ARG(n_sup == 0 || (acc && wt && dh));
  hipLaunchKernelGGL(ce_finish_kernel, dim3((unsigned)rows), dim3(kCeThreads), 0,
                     (hipStream_t)stream, state, best_idx, xt, target, loss, entropy, correct,
                     acc, static_cast<const uint16_t*>(wt), static_cast<uint16_t*>(dh), n_sup, H);
  return qlora_launch_status();
}

// Gradient rows of one recomputed piece after the finish step (for the embedding gradient).
QLORA_API int qlora_ce_grad(void* logits, int64_t ld, const int64_t* target, const float* state,
                            int64_t v0, int64_t n_sup, int64_t width, void* stream) {
  QLORA_CHECK_ARG(n_sup >= 0 && width >= 0 && ld >= width && v0 >= 0);
  if (n_sup == 0 || width == 0) return 0;
  QLORA_CHECK_ARG(logits && target && state);
  const bool vec = ld % kCeVec == 0 && al16(logits);
  if (vec)
    hipLaunchKernelGGL(ce_grad_kernel<true>, dim3((unsigned)n_sup), dim3(kCeThreads), 0,
                       (hipStream_t)stream, static_cast<uint16_t*>(logits), ld, target, state,
                       v0, width);
  else
    hipLaunchKernelGGL(ce_grad_kernel<false>, dim3((unsigned)n_sup), dim3(kCeThreads), 0,
                       (hipStream_t)stream, static_cast<uint16_t*>(logits), ld, target, state,
                       v0, width);
  return qlora_launch_status();
}
