// Per-token parts of the LoRA forward and backward for the q and v adapters of a layer, one
// launch each, on gfx950 MFMA (v_mfma_f32_32x32x16_f16), for LoRA ranks r = 8, 16, 32, 64.
// Reference: engine.py:1088-1093 (forward: lora_A then lora_B on the dropped LoRA input) and
// engine.py:1319-1331 (backward). Both are two chained fp16 products through the rank-r
// bottleneck, each accumulated in fp32 and rounded once, as the reference's GEMMs:
//   forward:   x  = f16(a A^T)            [n, r]    (kept for the backward)
//              l  = f16(x B^T)            [n, N]    (added to the projection by the RoPE kernel)
//   backward:  dx = f16(f16(g B) * s)     [n, r]    (g: the adapter's columns of d[q|k|v])
//              t  = f16(dx A)             [n, H]    (the gradient reaching the LoRA input)
// The token reductions of the backward (dB = s g^T x, dA = dx^T a) are qlora_lora_grad, below.
//
// Generic form: phase 1 P = X W (X [n, K1] rows, W given as Wt [r, K1]), phase 2 Y = P V (V
// given as Vt [M2, r]). Every MFMA operand is then a 16-byte run along the contraction. The
// backward's Wt = B^T and Vt = A^T are the fp16 copies the caller keeps transposed.
//
// A workgroup owns 32 tokens of one adapter (blockIdx.y: 0 = q, 1 = v), eight wavefronts.
// Phase 1: 32 x 32 MFMA tiles over the rank columns, the 16-wide k-steps dealt round-robin to the
// wavefronts in chunks whose loads are all issued before the chunk's MFMAs; the eight partial
// tiles are summed in LDS and rounded. Phase 2 computes Y^T = Vt P^T, one MFMA per 32 output
// columns and 16 ranks (a lane holds columns of one token), over chunks of kChunkCols output
// columns: the wavefronts put their tiles into an LDS copy of the chunk's 32 rows, then the
// workgroup writes the rows with 16-byte stores, a wavefront per 1 KiB of a row (the MFMA layout
// itself would store 16-byte pieces of 32 different rows per instruction, which ran phase 2 at
// a third of the bandwidth). A workgroup takes a.cpw consecutive chunks (blockIdx.z: which
// group; each group's workgroup forms P itself, the first writes it): a workgroup's time is a
// chain of dependent steps, so a launch that would not fill the GPU gives each chunk its own
// workgroup (more, shorter chains), a full one keeps a row's chunks together (no second phase
// 1). The first chunk's Vt operands are loaded before phase 1, the next chunk's before the
// current one is stored.
#include "common.h"

#include <mutex>

namespace qlora {
namespace lora {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTok = 32;
constexpr int kWaves = 8;
constexpr int kChunk1 = 12;  // phase-1 k-steps per wavefront per chunk
constexpr int kChunkCols = 512;  // phase-2 output columns staged in LDS at a time
constexpr int kCUs = 256;        // compute units of an MI355X
constexpr int kTilesPerWave = kChunkCols / 32 / kWaves;  // phase-2 tiles per wavefront per chunk
constexpr int kStageLd = kChunkCols + 4;  // LDS row stride (halves): 8-byte writes of the 32
                                          // rows of a tile land on distinct banks

// The LoRA ranks the kernels take (template parameter R).
__host__ __device__ constexpr bool rank_ok(int r) { return r == 8 || r == 16 || r == 32 || r == 64; }

struct Job {
  const uint16_t* X;   // fp16 [n, ldx] (phase-1 rows)
  const uint16_t* Wt;  // fp16 [R, K1]
  uint16_t* P;         // fp16 [n, R]
  const uint16_t* Vt;  // fp16 [M2, R]
  uint16_t* Y;         // fp16 [n, M2] or null (no phase 2)
  int64_t ldx;
  int K1, M2;
};

struct Args {
  Job job[2];
  int64_t n;
  float s;
  int scale;  // 1: P = f16(f16(acc) * s), 0: P = f16(acc)
  int cpw;    // phase-2 column chunks per workgroup
};

__device__ __forceinline__ f32x16 mfma(half8_t a, half8_t b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half8_t ld8(const uint16_t* p) {
  return *reinterpret_cast<const half8_t*>(p);
}

// Rank R: phase 1 uses ceil(R / 32) MFMA column tiles (rank columns past R read duplicated rows
// of Wt and are dropped); phase 2 contracts over ceil(R / 16) k-steps of 16, the rank-R
// intermediate zero-padded to a multiple of 16 in LDS (the matching Vt columns then read
// duplicated, finite weights: 0 x finite adds exactly 0).
template <int R>
__global__ __launch_bounds__(64 * kWaves) void lora_rows_kernel(Args a) {
  constexpr int NT1 = (R + 31) / 32, KS2 = (R + 15) / 16, RP = 16 * KS2;
  constexpr int CH1 = NT1 == 1 ? kChunk1 : kChunk1 / 2;
  __shared__ float red[kWaves][kTok][R];
  __shared__ __align__(16) uint16_t ps[kTok][RP];
  __shared__ __align__(16) uint16_t stage[kTok][kStageLd];
  const Job& jb = a.job[blockIdx.y];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = lane & 31, half = lane >> 5;
  const int64_t t0 = (int64_t)blockIdx.x * kTok;
  const int64_t tok = t0 + row < a.n ? t0 + row : a.n - 1;  // rows past n: computed, not stored
  const bool two = jb.Y != nullptr;
  const int tiles = two ? jb.M2 / 32 : 0;
  constexpr int kTilesPerChunk = kChunkCols / 32;
  const int group = blockIdx.z, c_first = group * a.cpw * kTilesPerChunk;
  const int c_end = min(tiles, c_first + a.cpw * kTilesPerChunk);
  if (group > 0 && c_first >= tiles) return;  // uniform: this job has fewer chunks
  // phase-2 operands of this wavefront's tiles of the first chunk: Vt rows 32 c + l%32, ranks
  // 16 kk + 8(l/32)..+7 (past R: the row's first ranks again; tiles past the end: the last one)
  half8_t vop[kTilesPerWave][KS2];
  auto load_vop = [&](int c0) {
#pragma unroll
    for (int i = 0; i < kTilesPerWave; ++i) {
      const int c = min(c0 + kTilesPerWave * wave + i, max(tiles - 1, 0));
#pragma unroll
      for (int kk = 0; kk < KS2; ++kk) {
        const int r0 = min(16 * kk + 8 * half, R - 8);
        vop[i][kk] = two ? ld8(jb.Vt + (int64_t)(32 * c + row) * R + r0) : half8_t{};
      }
    }
  };
  load_vop(c_first);
  // phase 1: P[32 x R] = X[32 x K1] W[K1 x R]
  const uint16_t* xrow = jb.X + tok * jb.ldx + 8 * half;
  const uint16_t* wrow[NT1];
#pragma unroll
  for (int t = 0; t < NT1; ++t)
    wrow[t] = jb.Wt + (int64_t)((32 * t + row) & (R - 1)) * jb.K1 + 8 * half;
  const int steps = jb.K1 / 16;
  f32x16 acc[NT1];
#pragma unroll
  for (int t = 0; t < NT1; ++t) acc[t] = f32x16{};
  for (int k0 = wave; k0 < steps; k0 += kWaves * CH1) {
    half8_t xa[CH1], wb[CH1][NT1];
#pragma unroll
    for (int i = 0; i < CH1; ++i) {
      const int ks = min(k0 + kWaves * i, steps - 1);
      xa[i] = ld8(xrow + 16 * ks);
#pragma unroll
      for (int t = 0; t < NT1; ++t) wb[i][t] = ld8(wrow[t] + 16 * ks);
    }
    // keep every load of the chunk ahead of its MFMAs: left alone, the scheduler sinks each
    // load next to its MFMA and the wavefront waits out one memory round trip per k-step
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < CH1; ++i)
#pragma unroll
      for (int t = 0; t < NT1; ++t)
        acc[t] = mfma(xa[i], k0 + kWaves * i < steps ? wb[i][t] : half8_t{}, acc[t]);
  }
  // register r of lane l holds P[8(r/4) + 4(l/32) + r%4][32 t + l%32]
#pragma unroll
  for (int t = 0; t < NT1; ++t) {
    if (32 * t + row < R) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        red[wave][8 * (r >> 2) + 4 * half + (r & 3)][32 * t + row] = acc[t][r];
    }
  }
  __syncthreads();
  for (int idx = tid; idx < kTok * RP; idx += 64 * kWaves) {
    const int t = idx / RP, k = idx % RP;
    uint16_t b = 0;
    if (k < R) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) v += red[w][t][k];
      v = h2f(f2h(v));
      if (a.scale) v = h2f(f2h(v * a.s));
      b = f2h_bits(v);
      if (group == 0 && t0 + t < a.n) jb.P[(t0 + t) * R + k] = b;
    }
    ps[t][k] = b;
  }
  if (!two) return;  // uniform over the workgroup
  __syncthreads();
  // phase 2: Y^T[32 cols x 32 tok] = Vt[32 x R] P^T[R x 32]; B operand P[l%32][16 kk + 8(l/32)..]
  half8_t pb[KS2];
#pragma unroll
  for (int kk = 0; kk < KS2; ++kk) pb[kk] = ld8(&ps[row][16 * kk + 8 * half]);
  for (int c0 = c_first; c0 < c_end; c0 += kTilesPerChunk) {
    f32x16 ys[kTilesPerWave];
#pragma unroll
    for (int i = 0; i < kTilesPerWave; ++i) {
      ys[i] = f32x16{};
#pragma unroll
      for (int kk = 0; kk < KS2; ++kk) ys[i] = mfma(vop[i][kk], pb[kk], ys[i]);
    }
    if (c0 + kTilesPerChunk < c_end) load_vop(c0 + kTilesPerChunk);  // the next chunk's
    if (c0 != c_first) __syncthreads();  // the previous chunk's rows are out of the stage
#pragma unroll
    for (int i = 0; i < kTilesPerWave; ++i) {
      const int lt = kTilesPerWave * wave + i;  // tile within the chunk
      const f32x16& y = ys[i];
      // register r: Y[t0 + l%32][32 c + 8(r/4) + 4(l/32) + r%4]
      if (c0 + lt < tiles) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          uint2 w;
          w.x = pack2h(y[4 * j + 0], y[4 * j + 1]);
          w.y = pack2h(y[4 * j + 2], y[4 * j + 3]);
          *reinterpret_cast<uint2*>(&stage[row][32 * lt + 8 * j + 4 * half]) = w;
        }
      }
    }
    __syncthreads();
    // the chunk's rows: 16-byte units, consecutive threads along a row
    const int ccols = min(kChunkCols, 32 * (tiles - c0));
    const int units = ccols / 8;  // per row
    for (int u = tid; u < kTok * units; u += 64 * kWaves) {
      const int tr = u / units, cu = u - tr * units;
      if (t0 + tr >= a.n) continue;
      const uint2 lo = *reinterpret_cast<const uint2*>(&stage[tr][8 * cu]);
      const uint2 hi = *reinterpret_cast<const uint2*>(&stage[tr][8 * cu + 4]);
      *reinterpret_cast<uint4*>(jb.Y + (t0 + tr) * jb.M2 + 32 * c0 + 8 * cu) =
          make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
  }
}

bool aligned(const void* p, uintptr_t b) { return ((uintptr_t)p & (b - 1)) == 0; }

int launch(Args& a, int r, hipStream_t stream) {
  QLORA_CHECK_ARG(rank_ok(r));
  for (int i = 0; i < 2; ++i) {
    const Job& j = a.job[i];
    QLORA_CHECK_ARG(j.X && j.Wt && j.P && j.K1 > 0 && j.K1 % 16 == 0 && j.ldx >= j.K1);
    QLORA_CHECK_ARG(j.ldx % 8 == 0 && aligned(j.X, 16) && aligned(j.Wt, 16) && aligned(j.P, 2));
    QLORA_CHECK_ARG(j.Y == nullptr ||
                    (j.Vt && j.M2 > 0 && j.M2 % 32 == 0 && aligned(j.Vt, 16) && aligned(j.Y, 16)));
  }
  QLORA_CHECK_ARG(a.n < (1ll << 31) * kTok);
  int chunks = 1;  // phase-2 column chunks of the job with the most
  for (int i = 0; i < 2; ++i)
    if (a.job[i].Y != nullptr)
      chunks = (int)std::max<int64_t>(chunks, qlora_cdiv(a.job[i].M2, kChunkCols));
  // the chunks of a row go to separate workgroups while the workgroups that have work stay
  // within one per CU (256 on MI355X: a job with fewer chunks leaves its later groups empty,
  // and those return at once); a fuller launch keeps them together
  const int64_t rows = qlora_cdiv(a.n, kTok);
  auto working = [&](int g) {
    const int64_t per = qlora_cdiv(chunks, g);  // chunks per workgroup
    int64_t w = 0;
    for (int i = 0; i < 2; ++i)
      w += rows * qlora_cdiv(a.job[i].Y ? qlora_cdiv(a.job[i].M2, kChunkCols) : 1, per);
    return w;
  };
  int groups = chunks;
  while (groups > 1 && working(groups) > kCUs) --groups;
  a.cpw = (int)qlora_cdiv(chunks, groups);
  groups = (int)qlora_cdiv(chunks, a.cpw);
  const dim3 grid((unsigned)rows, 2, (unsigned)groups), block(64 * kWaves);
  switch (r) {
    case 8: hipLaunchKernelGGL(lora_rows_kernel<8>, grid, block, 0, stream, a); break;
    case 16: hipLaunchKernelGGL(lora_rows_kernel<16>, grid, block, 0, stream, a); break;
    case 32: hipLaunchKernelGGL(lora_rows_kernel<32>, grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL(lora_rows_kernel<64>, grid, block, 0, stream, a); break;
  }
  return qlora_launch_status();
}

// ------------------------------------------------------------------------------------------------
// Token reductions of the LoRA backward (engine.py:1327, 1329), all four in one pair of launches:
//   dB_a = s * sum_t g_a[t]^T x_a[t]     fp32 [N_a, 16]
//   dA_a =     sum_t dx_a[t]^T a_a[t]    fp32 [16, H]
// Generic job: out[c][k] = scale * sum_t W[t][c] Z[t][k] with W token-major (a wide fp16 matrix
// read along its rows, coalesced) and Z fp16 [n, 16]. Pass 1: a workgroup takes 128 columns of
// one job and a chunk of kGradChunk tokens, split in four quarters (one per wavefront). A thread
// owns two adjacent columns of its quarter: it issues the loads of all its token pairs at once
// (enough bytes in flight to cover the memory latency), then accumulates the 2 x 16 sums with
// v_dot2_f32_f16 (the pair (W[t][c], W[t+1][c]) against (Z[t][k], Z[t+1][k]), the latter
// staged in LDS and read as a broadcast). The quarters are added in LDS and the chunk's fp32
// partial sums go to a workspace [chunks][columns][16]. Pass 2 adds the chunks in a fixed order
// (the result does not depend on scheduling) and writes the outputs, transposed for dA.
// Products are exact in fp32; sums are fp32, as the reference's GEMMs accumulate.
// ------------------------------------------------------------------------------------------------
constexpr int kGradThreads = 256;
constexpr int kGradPairs = 64;                     // column pairs per workgroup (one wavefront)
constexpr int kGradCols = 2 * kGradPairs;          // columns per workgroup
constexpr int kGradQuarter = 64;                   // tokens per wavefront
constexpr int kGradChunk = 4 * kGradQuarter;       // tokens per workgroup
constexpr int kGradJobs = 4;

struct GradJob {
  const uint16_t* W;  // fp16, column c of token t at W[t * ldw + c]
  const uint16_t* Z;  // fp16 [n, 16]
  float* out;         // trans 0: out[c * 16 + k]; trans 1: out[k * ncols + c]
  int64_t ldw;
  int ncols, trans, col0;  // col0: the job's first column in the workspace (multiple of 128)
  float scale;
};

struct GradArgs {
  GradJob job[kGradJobs];
  float* part;
  int64_t n;
  int total_cols, nchunks;
};

__device__ __forceinline__ int grad_job(const GradArgs& a, int col) {
  int j = 0;
#pragma unroll
  for (int i = 1; i < kGradJobs; ++i) j = col >= a.job[i].col0 ? i : j;
  return j;
}

__device__ __forceinline__ uint32_t word_of4(const uint4& x, int i) {
  return i < 2 ? (i == 0 ? x.x : x.y) : (i == 2 ? x.z : x.w);
}

__device__ __forceinline__ float dot2u(uint32_t a, uint32_t b, float c) {
  typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b),
                                c, false);
}

// Rank R: every thread accumulates all R sums of its two columns (2 R fp32 registers); they are
// merged over the quarters in LDS in slices of S = min(R, 16) ranks.
template <int R>
__global__ __launch_bounds__(kGradThreads) void lora_grad_part_kernel(GradArgs a) {
  constexpr int S = R < 16 ? R : 16;
  constexpr int kQP = kGradQuarter / 2;  // token pairs per thread
  constexpr int kRow = 2 * S + 4;        // floats per column pair in the LDS sum (padded)
  __shared__ __align__(16) uint32_t zp[kGradChunk / 2][R];
  __shared__ __align__(16) float red[4][kGradPairs][kRow];
  const int tid = threadIdx.x, quarter = tid >> 6, cp = tid & 63;
  const int wg_col = blockIdx.x * kGradCols;
  const GradJob& jb = a.job[grad_job(a, wg_col)];
  const int64_t t0 = (int64_t)blockIdx.y * kGradChunk;
  const int nt = (int)min((int64_t)kGradChunk, a.n - t0);  // >= 1
  // this thread's loads first: its quarter's token pairs of columns c, c + 1 (rows past the
  // chunk read its last row and meet a zero Z below)
  const int c = wg_col - jb.col0 + 2 * cp;
  const bool col_ok = c < jb.ncols;
  const uint16_t* wp = jb.W + (col_ok ? c : 0);
  uint32_t w0[kQP], w1[kQP];
#pragma unroll
  for (int i = 0; i < kQP; ++i) {
    const int64_t ta = t0 + min(kGradQuarter * quarter + 2 * i, nt - 1);
    const int64_t tb = t0 + min(kGradQuarter * quarter + 2 * i + 1, nt - 1);
    w0[i] = *reinterpret_cast<const uint32_t*>(wp + ta * jb.ldw);
    w1[i] = *reinterpret_cast<const uint32_t*>(wp + tb * jb.ldw);
  }
  for (int i = tid; i < (kGradChunk / 2) * R; i += kGradThreads) {
    const int p = i / R, k = i % R;
    const int64_t ta = t0 + min(2 * p, nt - 1), tb = t0 + min(2 * p + 1, nt - 1);
    const uint32_t za = jb.Z[ta * R + k], zb = jb.Z[tb * R + k];
    zp[p][k] = (2 * p < nt ? za : 0u) | ((2 * p + 1 < nt ? zb : 0u) << 16);
  }
  __syncthreads();
  float acc0[R], acc1[R];
#pragma unroll
  for (int k = 0; k < R; ++k) acc0[k] = acc1[k] = 0.f;
#pragma unroll
  for (int i = 0; i < kQP; ++i) {
    const uint32_t pc0 = (w0[i] & 0xFFFFu) | (w1[i] << 16);  // column c, tokens t, t + 1
    const uint32_t pc1 = (w0[i] >> 16) | (w1[i] & 0xFFFF0000u);  // column c + 1
    const uint4* zq = reinterpret_cast<const uint4*>(zp[kQP * quarter + i]);
#pragma unroll
    for (int q = 0; q < R / 4; ++q) {
      const uint4 z = zq[q];
      acc0[4 * q + 0] = dot2u(pc0, z.x, acc0[4 * q + 0]);
      acc0[4 * q + 1] = dot2u(pc0, z.y, acc0[4 * q + 1]);
      acc0[4 * q + 2] = dot2u(pc0, z.z, acc0[4 * q + 2]);
      acc0[4 * q + 3] = dot2u(pc0, z.w, acc0[4 * q + 3]);
      acc1[4 * q + 0] = dot2u(pc1, z.x, acc1[4 * q + 0]);
      acc1[4 * q + 1] = dot2u(pc1, z.y, acc1[4 * q + 1]);
      acc1[4 * q + 2] = dot2u(pc1, z.z, acc1[4 * q + 2]);
      acc1[4 * q + 3] = dot2u(pc1, z.w, acc1[4 * q + 3]);
    }
  }
  const int pair = tid >> 2, sub = tid & 3;  // the final sums: 4 threads per column pair
  const bool pair_ok = wg_col - jb.col0 + 2 * pair < jb.ncols;
#pragma unroll
  for (int rs = 0; rs < R / S; ++rs) {
    if (rs > 0) __syncthreads();  // the previous slice's sums have been read
    float4* mine = reinterpret_cast<float4*>(red[quarter][cp]);
#pragma unroll
    for (int q = 0; q < S / 4; ++q) {
      const int k = rs * S + 4 * q;
      mine[q] = make_float4(acc0[k], acc0[k + 1], acc0[k + 2], acc0[k + 3]);
      mine[S / 4 + q] = make_float4(acc1[k], acc1[k + 1], acc1[k + 2], acc1[k + 3]);
    }
    __syncthreads();
    // the pair's 2 S sums as S / 2 float4: the first S / 4 of column c, the rest of c + 1
    if (pair_ok) {
      for (int f = sub; f < S / 2; f += 4) {
        float4 v = reinterpret_cast<const float4*>(red[0][pair])[f];
#pragma unroll
        for (int qq = 1; qq < 4; ++qq) {
          const float4 u = reinterpret_cast<const float4*>(red[qq][pair])[f];
          v.x += u.x;
          v.y += u.y;
          v.z += u.z;
          v.w += u.w;
        }
        const int col = wg_col + 2 * pair + (f >= S / 4 ? 1 : 0);
        const int k = rs * S + 4 * (f % (S / 4));
        *reinterpret_cast<float4*>(a.part + ((int64_t)blockIdx.y * a.total_cols + col) * R + k) =
            v;
      }
    }
  }
}

// MFMA form of the same pass (the same partial sums up to fp32 summation order), for jobs whose
// rows hold whole 16-byte chunks: the workgroup stages its 256 tokens x 128 columns of W in LDS
// with 16-byte row loads (16 chunks a row, chunk c of row t at c ^ 4 (t mod 4)) and Z^T
// [R][256] (rows padded by 16 bytes); wavefront w then forms out[32 w .. + 31][0 .. R) over the
// 16 token steps of 16 with v_mfma_f32_32x32x16_f16: A = W^T through ds_read_b64_tr_b16 (8
// consecutive tokens of one column per lane), B = Z from Z^T. The v_dot2 form spends most of its
// time in the 256 products per token pair and thread; this one in the loads.
constexpr int kZLd = kGradChunk + 8;  // Z^T row stride (halves)

__device__ __forceinline__ int wt_off(int row, int col) {
  return row * kGradCols + (((col >> 3) ^ ((row & 3) << 2)) << 3) + (col & 7);
}

// The MFMA A operand W^T[32 columns][8 tokens] of a wt_off tile: lane l supplies column
// c0 + l % 32 and tokens k0 + 8 (l / 32) .. + 7. ds_read_b64_tr_b16 gives lane i of each
// 16-lane group element i % 4 of the 4 halves read by lane 4 j + i / 4 of the group as its
// element j; so lane p of a group reads row (first token) + p / 4, columns (group's first) +
// 4 (p % 4) .. + 3, and two reads cover the 8 tokens.
__device__ __forceinline__ half8_t tr_cols(const uint16_t* t, int k0, int c0, int lane) {
  typedef short short4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) short4_t lds_short4_t;
  const int p = lane & 15;
  const int row = k0 + 8 * (lane >> 5) + (p >> 2);
  const int col = c0 + 16 * ((lane >> 4) & 1) + 4 * (p & 3);
  const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(t + wt_off(row, col)));
  const short4_t hi =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(t + wt_off(row + 4, col)));
  return __builtin_bit_cast(half8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

template <int R>
__global__ __launch_bounds__(kGradThreads) void lora_grad_mfma_kernel(GradArgs a) {
  constexpr int NTR = (R + 31) / 32;  // 32-rank tiles of the MFMA output
  constexpr int kLoads = kGradChunk * (kGradCols / 8) / kGradThreads;
  __shared__ __align__(16) uint16_t wt[kGradChunk * kGradCols];
  __shared__ __align__(16) uint16_t zt[R][kZLd];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wg_col = blockIdx.x * kGradCols;
  const GradJob& jb = a.job[grad_job(a, wg_col)];
  const int64_t t0 = (int64_t)blockIdx.y * kGradChunk;
  const int nt = (int)min((int64_t)kGradChunk, a.n - t0);  // >= 1
  const int cbase = wg_col - jb.col0;  // the tile's first column within the job
  // W: every load issued first (rows past the chunk read its last row and meet a zero Z^T;
  // columns past the job read its last chunk and are not written)
  uint4 wv[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int id = tid + i * kGradThreads, row = id >> 4, ch = id & 15;
    const int c = min(cbase + 8 * ch, jb.ncols - 8);
    wv[i] = *reinterpret_cast<const uint4*>(jb.W + (t0 + min(row, nt - 1)) * jb.ldw + c);
  }
  for (int i = tid; i < kGradChunk * (R / 8); i += kGradThreads) {
    const int t = i / (R / 8), kq = i % (R / 8);
    uint4 z = *reinterpret_cast<const uint4*>(jb.Z + (t0 + min(t, nt - 1)) * R + 8 * kq);
    if (t >= nt) z = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = word_of4(z, j);
      zt[8 * kq + 2 * j][t] = (uint16_t)(w & 0xFFFFu);
      zt[8 * kq + 2 * j + 1][t] = (uint16_t)(w >> 16);
    }
  }
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int id = tid + i * kGradThreads, row = id >> 4, ch = id & 15;
    *reinterpret_cast<uint4*>(wt + wt_off(row, 8 * ch)) = wv[i];
  }
  __syncthreads();
  f32x16 acc[NTR];
#pragma unroll
  for (int u = 0; u < NTR; ++u) acc[u] = f32x16{};
#pragma unroll 4
  for (int kk = 0; kk < kGradChunk / 16; ++kk) {
    const half8_t aop = tr_cols(wt, 16 * kk, 32 * wave, lane);
#pragma unroll
    for (int u = 0; u < NTR; ++u) {
      const int rank = 32 * u + (lane & 31);
      const half8_t bop = rank < R ? ld8(&zt[rank < R ? rank : 0][16 * kk + 8 * (lane >> 5)])
                                   : half8_t{};
      acc[u] = mfma(aop, bop, acc[u]);
    }
  }
  // register r of lane l: out[column 32 w + 8(r/4) + 4(l/32) + r%4][rank 32 u + l%32]
#pragma unroll
  for (int u = 0; u < NTR; ++u) {
    const int rank = 32 * u + (lane & 31);
    if (rank >= R) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = 32 * wave + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (cbase + m < jb.ncols)
        a.part[((int64_t)blockIdx.y * a.total_cols + wg_col + m) * R + rank] = acc[u][r];
    }
  }
}

template <int R>
__global__ __launch_bounds__(256) void lora_grad_reduce_kernel(GradArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)a.total_cols * R) return;
  const int col = (int)(i / R), k = (int)(i % R);
  const GradJob& jb = a.job[grad_job(a, col)];
  const int c = col - jb.col0;
  if (c >= jb.ncols) return;
  float v = 0.f;
#pragma unroll 8
  for (int ch = 0; ch < a.nchunks; ++ch) v += a.part[(int64_t)ch * a.total_cols * R + i];
  v *= jb.scale;
  jb.out[jb.trans ? (int64_t)k * jb.ncols + c : (int64_t)c * R + k] = v;
}

int64_t grad_pad(int64_t c) { return qlora_cdiv(c, kGradCols) * kGradCols; }

int64_t grad_workspace(int64_t n, int N_q, int N_v, int H, int r) {
  const int64_t cols = grad_pad(N_q) + grad_pad(N_v) + 2 * grad_pad(H);
  return qlora_cdiv(n, kGradChunk) * cols * r;
}

}  // namespace lora
}  // namespace qlora

using namespace qlora::lora;

QLORA_API int qlora_lora_fwd_rows(const void* a_q, const void* a_v, const void* A_q,
                                  const void* A_v, const void* B_q, const void* B_v, void* x_q,
                                  void* x_v, void* l_q, void* l_v, int64_t n, int32_t N_q,
                                  int32_t N_v, int32_t H, int32_t r, void* stream) {
  QLORA_CHECK_ARG(n >= 0 && N_q > 0 && N_v > 0 && H > 0);
  if (n == 0) return 0;
  QLORA_CHECK_ARG(rank_ok(r) && (l_q == nullptr) == (l_v == nullptr));
  Args a{};
  a.job[0] = Job{static_cast<const uint16_t*>(a_q), static_cast<const uint16_t*>(A_q),
                 static_cast<uint16_t*>(x_q), static_cast<const uint16_t*>(B_q),
                 static_cast<uint16_t*>(l_q), H, H, N_q};
  a.job[1] = Job{static_cast<const uint16_t*>(a_v), static_cast<const uint16_t*>(A_v),
                 static_cast<uint16_t*>(x_v), static_cast<const uint16_t*>(B_v),
                 static_cast<uint16_t*>(l_v), H, H, N_v};
  a.n = n;
  a.s = 1.f;
  a.scale = 0;
  return launch(a, r, (hipStream_t)stream);
}

QLORA_API int qlora_lora_bwd_rows(const void* g_q, const void* g_v, int64_t ldg,
                                  const void* Bt_q, const void* Bt_v, const void* At_q,
                                  const void* At_v, void* dx_q, void* dx_v, void* t_q, void* t_v,
                                  int64_t n, int32_t N_q, int32_t N_v, int32_t H, int32_t r,
                                  float s, void* stream) {
  QLORA_CHECK_ARG(n >= 0 && N_q > 0 && N_v > 0 && H > 0);
  if (n == 0) return 0;
  QLORA_CHECK_ARG(rank_ok(r) && (t_q == nullptr) == (t_v == nullptr));
  Args a{};
  a.job[0] = Job{static_cast<const uint16_t*>(g_q), static_cast<const uint16_t*>(Bt_q),
                 static_cast<uint16_t*>(dx_q), static_cast<const uint16_t*>(At_q),
                 static_cast<uint16_t*>(t_q), ldg, N_q, H};
  a.job[1] = Job{static_cast<const uint16_t*>(g_v), static_cast<const uint16_t*>(Bt_v),
                 static_cast<uint16_t*>(dx_v), static_cast<const uint16_t*>(At_v),
                 static_cast<uint16_t*>(t_v), ldg, N_v, H};
  a.n = n;
  a.s = s;
  a.scale = 1;
  return launch(a, r, (hipStream_t)stream);
}

// Workspace (fp32 elements) qlora_lora_grad needs for these sizes.
QLORA_API int qlora_lora_grad_workspace(int64_t n, int32_t N_q, int32_t N_v, int32_t H,
                                        int32_t r, int64_t* elems) {
  QLORA_CHECK_ARG(n >= 0 && N_q > 0 && N_v > 0 && H > 0 && rank_ok(r) && elems);
  *elems = grad_workspace(n, N_q, N_v, H, r);
  return 0;
}

// dB_a = s g_a^T x_a fp32 [N_a, r], dA_a = dx_a^T a_a fp32 [r, H] for a = q, v (zeros for n = 0).
QLORA_API int qlora_lora_grad(const void* g_q, const void* g_v, int64_t ldg, const void* x_q,
                              const void* x_v, const void* a_q, const void* a_v,
                              const void* dx_q, const void* dx_v, float* dB_q, float* dB_v,
                              float* dA_q, float* dA_v, int64_t n, int32_t N_q, int32_t N_v,
                              int32_t H, int32_t r, float s, float* work, int64_t work_elems,
                              void* stream) {
  QLORA_CHECK_ARG(n >= 0 && N_q > 0 && N_v > 0 && H > 0 && rank_ok(r));
  QLORA_CHECK_ARG(N_q % 2 == 0 && N_v % 2 == 0 && H % 2 == 0 && ldg % 2 == 0);
  QLORA_CHECK_ARG(ldg >= N_q && ldg >= N_v);
  QLORA_CHECK_ARG(dB_q && dB_v && dA_q && dA_v);
  QLORA_CHECK_ARG(work_elems >= grad_workspace(n, N_q, N_v, H, r) && (n == 0 || work));
  if (n > 0) {
    QLORA_CHECK_ARG(g_q && g_v && x_q && x_v && a_q && a_v && dx_q && dx_v);
    QLORA_CHECK_ARG(aligned(g_q, 4) && aligned(g_v, 4) && aligned(a_q, 4) && aligned(a_v, 4));
    QLORA_CHECK_ARG(aligned(work, 16));
  }
  GradArgs a{};
  int col = 0;
  const void* W[4] = {g_q, g_v, a_q, a_v};
  const void* Z[4] = {x_q, x_v, dx_q, dx_v};
  float* out[4] = {dB_q, dB_v, dA_q, dA_v};
  const int64_t ldw[4] = {ldg, ldg, H, H};
  const int nc[4] = {N_q, N_v, H, H};
  for (int j = 0; j < 4; ++j) {
    a.job[j] = GradJob{static_cast<const uint16_t*>(W[j]), static_cast<const uint16_t*>(Z[j]),
                       out[j], ldw[j], nc[j], j >= 2, col, j < 2 ? s : 1.f};
    col += (int)grad_pad(nc[j]);
  }
  a.part = work;
  a.n = n;
  a.total_cols = col;
  a.nchunks = (int)qlora_cdiv(n, kGradChunk);
  hipStream_t st = (hipStream_t)stream;
  const dim3 g1(col / kGradCols, a.nchunks), g2((unsigned)qlora_cdiv((int64_t)col * r, 256));
  // the MFMA pass needs whole 16-byte chunks in every row of every job
  bool mfma_ok = true;
  for (int j = 0; j < 4; ++j)
    mfma_ok = mfma_ok && aligned(W[j], 16) && aligned(Z[j], 16) && ldw[j] % 8 == 0 &&
              nc[j] % 8 == 0;
#define QLORA_GRAD(RR)                                                                     \
  do {                                                                                     \
    if (n > 0 && mfma_ok)                                                                  \
      hipLaunchKernelGGL(lora_grad_mfma_kernel<RR>, g1, dim3(kGradThreads), 0, st, a);     \
    else if (n > 0)                                                                        \
      hipLaunchKernelGGL(lora_grad_part_kernel<RR>, g1, dim3(kGradThreads), 0, st, a);     \
    hipLaunchKernelGGL(lora_grad_reduce_kernel<RR>, g2, dim3(256), 0, st, a);              \
  } while (0)
  switch (r) {
    case 8: QLORA_GRAD(8); break;
    case 16: QLORA_GRAD(16); break;
    case 32: QLORA_GRAD(32); break;
    default: QLORA_GRAD(64); break;
  }
#undef QLORA_GRAD
  return qlora_launch_status();
}

// ------------------------------------------------------------------------------------------------
// Allocation-free form of qlora_lora_grad, for callers that cannot allocate (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc): the pass-1 partial sums go to a
// file-scope device array instead of a caller workspace. Its address is taken once per device
// (hipGetSymbolAddress, that device current) on the first call there and kept; kernels get that
// address, never the array's name (a host-side stand-in). Every element pass 2 reads is written
// by pass 1 of the same call, so the array needs no clearing between calls; calls that overlap
// on one GPU (two streams) share the array and race.
// ------------------------------------------------------------------------------------------------
namespace {

constexpr int64_t kGradScratchElems = int64_t(4) << 20;  // fp32: 16 MiB per device
static __device__ __align__(256) float scratch[kGradScratchElems];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, or nullptr on a failed lookup.
float* scratch_on_current_device(int* rc) {
  int dev = 0;
  *rc = (int)hipGetDevice(&dev);
  if (*rc != 0) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *rc = (int)hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    *rc = (int)hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (*rc != 0) return nullptr;
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  return g_scratch_ptr[dev];
}

}  // namespace

// qlora_lora_grad without a workspace argument; QLORA_ERR_SCRATCH_TOO_SMALL when
// qlora_lora_grad_workspace(...) exceeds the static scratch (4 Mi fp32).
QLORA_API int qlora_lora_grad_noalloc(const void* g_q, const void* g_v, int64_t ldg,
                                      const void* x_q, const void* x_v, const void* a_q,
                                      const void* a_v, const void* dx_q, const void* dx_v,
                                      float* dB_q, float* dB_v, float* dA_q, float* dA_v,
                                      int64_t n, int32_t N_q, int32_t N_v, int32_t H, int32_t r,
                                      float s, void* stream) {
  QLORA_CHECK_ARG(n >= 0 && N_q > 0 && N_v > 0 && H > 0 && rank_ok(r));
  if (grad_workspace(n, N_q, N_v, H, r) > kGradScratchElems) return QLORA_ERR_SCRATCH_TOO_SMALL;
  int rc = 0;
  float* work = scratch_on_current_device(&rc);
  if (work == nullptr) return rc != 0 ? rc : (int)hipErrorInvalidValue;
  return qlora_lora_grad(g_q, g_v, ldg, x_q, x_v, a_q, a_v, dx_q, dx_v, dB_q, dB_v, dA_q, dA_v, n,
                         N_q, N_v, H, r, s, work, kGradScratchElems, stream);
}
