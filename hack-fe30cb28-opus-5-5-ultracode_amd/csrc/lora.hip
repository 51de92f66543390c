// Per-token parts of the LoRA forward and backward for the q and v adapters of a layer, one
// launch each, on gfx950 MFMA (v_mfma_f32_32x32x16_f16).
// Reference: engine.py:1088-1093 (forward: lora_A then lora_B on the dropped LoRA input) and
// engine.py:1319-1331 (backward). Both are two chained fp16 products through the rank-16
// bottleneck, each accumulated in fp32 and rounded once, as the reference's GEMMs:
//   forward:   x  = f16(a A^T)            [n, 16]   (kept for the backward)
//              l  = f16(x B^T)            [n, N]    (added to the projection by the RoPE kernel)
//   backward:  dx = f16(f16(g B) * s)     [n, 16]   (g: the adapter's columns of d[q|k|v])
//              t  = f16(dx A)             [n, H]    (the gradient reaching the LoRA input)
// The token reductions of the backward (dB = s g^T x, dA = dx^T a) stay GEMMs.
//
// Generic form: phase 1 P = X W (X [n, K1] rows, W given as Wt [16, K1]), phase 2 Y = P V (V
// given as Vt [M2, 16]). Every MFMA operand is then a 16-byte run along the contraction. The
// backward's Wt = B^T and Vt = A^T are the fp16 copies the caller keeps transposed.
//
// A workgroup owns 32 tokens of one adapter (blockIdx.y: 0 = q, 1 = v), eight wavefronts.
// Phase 1: a 32 x 32 MFMA tile (rank columns 16..31 ignored), the 16-wide k-steps dealt
// round-robin to the wavefronts in chunks whose loads are all issued before the chunk's MFMAs;
// the eight partial tiles are summed in LDS and rounded. Phase 2 computes Y^T = Vt P^T, one
// MFMA per 32 output columns, so that a lane holds four consecutive columns of one token and
// writes 8-byte runs; the first chunk of Vt operands is loaded before phase 1.
#include "common.h"

namespace qlora {
namespace lora {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kRank = 16;
constexpr int kTok = 32;
constexpr int kWaves = 8;
constexpr int kChunk1 = 6;  // phase-1 k-steps per wavefront per chunk
constexpr int kChunk2 = 6;  // phase-2 column tiles per wavefront per chunk

struct Job {
  const uint16_t* X;   // fp16 [n, ldx] (phase-1 rows)
  const uint16_t* Wt;  // fp16 [16, K1]
  uint16_t* P;         // fp16 [n, 16]
  const uint16_t* Vt;  // fp16 [M2, 16]
  uint16_t* Y;         // fp16 [n, M2] or null (no phase 2)
  int64_t ldx;
  int K1, M2;
};

struct Args {
  Job job[2];
  int64_t n;
  float s;
  int scale;  // 1: P = f16(f16(acc) * s), 0: P = f16(acc)
};

__device__ __forceinline__ f32x16 mfma(half8_t a, half8_t b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half8_t ld8(const uint16_t* p) {
  return *reinterpret_cast<const half8_t*>(p);
}

__global__ __launch_bounds__(64 * kWaves) void lora_rows_kernel(Args a) {
  __shared__ float red[kWaves][kTok][kRank];
  __shared__ __align__(16) uint16_t ps[kTok][kRank];
  const Job& jb = a.job[blockIdx.y];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = lane & 31, half = lane >> 5;
  const int64_t t0 = (int64_t)blockIdx.x * kTok;
  const int64_t tok = t0 + row < a.n ? t0 + row : a.n - 1;  // rows past n: computed, not stored
  const bool two = jb.Y != nullptr;
  const int tiles = two ? jb.M2 / 32 : 0;
  // phase-2 operands of the first chunk: Vt rows 32 c + l%32, ranks 8(l/32)..+7
  half8_t vop[kChunk2];
#pragma unroll
  for (int i = 0; i < kChunk2; ++i) {
    const int c = min(wave + kWaves * i, max(tiles - 1, 0));
    vop[i] = two ? ld8(jb.Vt + (int64_t)(32 * c + row) * kRank + 8 * half) : half8_t{};
  }
  // phase 1: P[32 x 16] = X[32 x K1] W[K1 x 16]
  const uint16_t* xrow = jb.X + tok * jb.ldx + 8 * half;
  const uint16_t* wrow = jb.Wt + (int64_t)(row & (kRank - 1)) * jb.K1 + 8 * half;
  const int steps = jb.K1 / 16;
  f32x16 acc = f32x16{};
  for (int k0 = wave; k0 < steps; k0 += kWaves * kChunk1) {
    half8_t xa[kChunk1], wb[kChunk1];
#pragma unroll
    for (int i = 0; i < kChunk1; ++i) {
      const int ks = min(k0 + kWaves * i, steps - 1);
      xa[i] = ld8(xrow + 16 * ks);
      wb[i] = ld8(wrow + 16 * ks);
    }
#pragma unroll
    for (int i = 0; i < kChunk1; ++i)
      acc = mfma(xa[i], k0 + kWaves * i < steps ? wb[i] : half8_t{}, acc);
  }
  // register r of lane l holds P[8(r/4) + 4(l/32) + r%4][l%32]
  if (row < kRank) {
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave][8 * (r >> 2) + 4 * half + (r & 3)][row] = acc[r];
  }
  __syncthreads();
  {
    const int t = tid / kRank, k = tid % kRank;  // 512 threads = 32 tokens x 16 ranks
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) v += red[w][t][k];
    v = h2f(f2h(v));
    if (a.scale) v = h2f(f2h(v * a.s));
    const uint16_t b = f2h_bits(v);
    ps[t][k] = b;
    if (t0 + t < a.n) jb.P[(t0 + t) * kRank + k] = b;
  }
  if (!two) return;  // uniform over the workgroup
  __syncthreads();
  // phase 2: Y^T[32 cols x 32 tok] = Vt[32 x 16] P^T[16 x 32]; B operand P[l%32][8(l/32)..+7]
  const half8_t pb = ld8(&ps[row][8 * half]);
  const bool store = t0 + row < a.n;
  uint16_t* yrow = jb.Y + (t0 + row) * jb.M2 + 4 * half;
  for (int c0 = wave; c0 < tiles; c0 += kWaves * kChunk2) {
    if (c0 != wave) {
#pragma unroll
      for (int i = 0; i < kChunk2; ++i) {
        const int c = min(c0 + kWaves * i, tiles - 1);
        vop[i] = ld8(jb.Vt + (int64_t)(32 * c + row) * kRank + 8 * half);
      }
    }
#pragma unroll
    for (int i = 0; i < kChunk2; ++i) {
      const int c = c0 + kWaves * i;
      const f32x16 y = mfma(vop[i], pb, f32x16{});
      // register r: Y[t0 + l%32][32 c + 8(r/4) + 4(l/32) + r%4]
      if (store && c < tiles) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          uint2 w;
          w.x = pack2h(y[4 * j + 0], y[4 * j + 1]);
          w.y = pack2h(y[4 * j + 2], y[4 * j + 3]);
          *reinterpret_cast<uint2*>(yrow + 32 * c + 8 * j) = w;
        }
      }
    }
  }
}

bool aligned(const void* p, uintptr_t b) { return ((uintptr_t)p & (b - 1)) == 0; }

int launch(Args& a, hipStream_t stream) {
  for (int i = 0; i < 2; ++i) {
    const Job& j = a.job[i];
    QLORA_CHECK_ARG(j.X && j.Wt && j.P && j.K1 > 0 && j.K1 % 16 == 0 && j.ldx >= j.K1);
    QLORA_CHECK_ARG(j.ldx % 8 == 0 && aligned(j.X, 16) && aligned(j.Wt, 16) && aligned(j.P, 2));
    QLORA_CHECK_ARG(j.Y == nullptr ||
                    (j.Vt && j.M2 > 0 && j.M2 % 32 == 0 && aligned(j.Vt, 16) && aligned(j.Y, 8)));
  }
  QLORA_CHECK_ARG(a.n < (1ll << 31) * kTok);
  hipLaunchKernelGGL(lora_rows_kernel, dim3((unsigned)qlora_cdiv(a.n, kTok), 2),
                     dim3(64 * kWaves), 0, stream, a);
  return qlora_launch_status();
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
  QLORA_CHECK_ARG(r == kRank && l_q && l_v);
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
  return launch(a, (hipStream_t)stream);
}

QLORA_API int qlora_lora_bwd_rows(const void* g_q, const void* g_v, int64_t ldg,
                                  const void* Bt_q, const void* Bt_v, const void* At_q,
                                  const void* At_v, void* dx_q, void* dx_v, void* t_q, void* t_v,
                                  int64_t n, int32_t N_q, int32_t N_v, int32_t H, int32_t r,
                                  float s, void* stream) {
  QLORA_CHECK_ARG(n >= 0 && N_q > 0 && N_v > 0 && H > 0);
  if (n == 0) return 0;
  QLORA_CHECK_ARG(r == kRank && (t_q == nullptr) == (t_v == nullptr));
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
  return launch(a, (hipStream_t)stream);
}
