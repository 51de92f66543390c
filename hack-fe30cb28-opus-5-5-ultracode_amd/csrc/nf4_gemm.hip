// NF4 dequantisation fused into fp16 MFMA GEMMs for the frozen projections of the step.
// Reference: the dequant kernel (kernels.py:68-105) followed by cuBLAS at engine.py:1082
// (qkv + bias), 1112 (o), 1163 (gate|up), 1179 (down) in forward and 1239, 1293, 1301, 1316
// (dY W) in backward.
//
//   NT (forward):  C[m, n] = sum_k A[m, k] W[n, k]      W = [N, K] NF4, K = reduction
//   NN (backward): C[m, n] = sum_k A[m, k] W[k, n]      W = [K, N] NF4, N = W's columns
//
// The W tile is decoded once per workgroup, straight from the bitsandbytes bytes (4-bit codes,
// double-quantised absmax) into LDS as fp16, with the same two roundings as the standalone
// dequant, so the fused product equals dequant-then-GEMM up to the fp32 summation order. The
// LDS B tile is always [n][k] with k contiguous (the MFMA B-operand layout): in NN each thread
// decodes an 8-row x 4-column block and packs each column's 8 values along the rows.
//
// Two tile shapes: 256 x 256 x 64 with 8 wavefronts (2 x 4, each a 128 x 64 block of
// v_mfma_f32_32x32x16_f16 accumulators; two wavefronts per SIMD, so one's NF4 decode (VALU)
// overlaps the other's MFMAs) for the wide projections, and 128 x 128 x 64 with 4 wavefronts
// (2 x 2 of 64 x 64) for the 1536/2048-wide ones, where 256-wide tiles would leave most of the
// 256 CUs idle. The 256-entry double-quant code and the 16 NF4 levels live in LDS; a thread's
// global loads for k-tile t + 1 (activations, packed nibbles, absmax bytes) are issued before
// the MFMAs of tile t and decoded into the other LDS buffer after them (double buffering, one
// barrier per k-tile). LDS rows hold 64 halves (eight 16-byte chunks); chunk c of row r sits
// at c ^ ((r ^ r >> 3) & 7), so the fragment reads (consecutive rows, same chunk) and the tile
// writes are free of bank conflicts. Workgroups are ordered so each XCD (blocks are dispatched
// round-robin over the 8 XCDs) sweeps a contiguous range of W tiles.
//
// Split-K: with splits > 1 each z-slice reduces a contiguous range of k-tiles into an fp32
// workspace [splits, M, N]; a second kernel sums the slices and applies the epilogue.
//
// Epilogues: fp16 store; + fp16 bias (qkv); fp32 residual add out = res + f32(fp16(acc))
// (h3 = h2 + d); SwiGLU m = fp16(silu(fp16 g) * fp16 u) with the gate and up rows of one output
// column in the same wavefront (gate|up forward without materialising [gate|up]).
#include "nf4.h"

namespace qlora {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;

enum { kEpiStore = 0, kEpiBias = 1, kEpiResid = 2, kEpiSwiglu = 3, kEpiPartial = 4 };

struct GemmArgs {
  const void* a;         // [M, Kr] fp16, or fp32 (a_f32: rounded to fp16 on load)
  int64_t lda;
  NF4Ref w;
  int64_t Kw;            // W's row length (columns)
  void* c;               // fp16 [M, ldc]; fp32 for kEpiResid; fp32 [splits, M, N] partials
  int64_t ldc;
  const uint16_t* bias;  // fp16 [N] (kEpiBias)
  const float* resid;    // fp32 [M, ldr] (kEpiResid)
  int64_t ldr;
  int64_t M, N, Kr;      // output rows, output columns, reduction length
  int64_t I;             // SwiGLU: first W row of the up projection
  int64_t kt_per_split;  // k-tiles per z-slice
};

__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * kBK + ((chunk ^ swz(row)) << 3);
}

__device__ __forceinline__ int64_t tile_order(int64_t b, int64_t total) {
  const int64_t full = total / 8 * 8;
  return b < full ? (b % 8) * (full / 8) + b / 8 : b;
}

// The raw inputs of one block scale, loaded with the tile; the scale itself is formed when the
// tile is decoded (the code2 lookup and the segment offset come from LDS, after the absmax byte
// has arrived). Every load is unconditional (pointers selected instead of branches), so the
// loads of a tile issue back to back instead of each waiting for the one before.
struct ScaleIn {
  uint32_t q;    // nested: absmax code
  float a2;      // nested: absmax2 of the block's group; plain: the fp32 absmax
  uint32_t seg;  // nested: segment of the block (stacked weights)
};

__device__ __forceinline__ ScaleIn scale_load(const NF4Ref& w, int64_t b) {
  ScaleIn s;
  const bool nested = w.nested;
  s.q = static_cast<const uint8_t*>(w.absmax)[nested ? b : 0];
  s.a2 = nested ? w.absmax2[b >> w.bs2_shift] : static_cast<const float*>(w.absmax)[b];
  s.seg = (uint32_t)((int)(b >= w.seg1) + (int)(b >= w.seg2));
  return s;
}

// fp32(fp32(code2[q] * absmax2) + offset), the product rounded before the add (bitsandbytes).
__device__ __forceinline__ float scale_of(const ScaleIn& s, int nested, const float* c2,
                                          const float* offs) {
  if (!nested) return s.a2;
  float prod = c2[s.q] * s.a2;
  fp32_barrier(prod);
  return prod + offs[s.seg];
}

template <int BM, int NT, bool A_F32>
struct ALoader {
  static constexpr int kPer = BM * kBK / 8 / NT;  // 16-byte chunks per thread
  uint4 v[kPer];
  __device__ __forceinline__ void load(const GemmArgs& g, int64_t m0, int64_t k0) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int id = threadIdx.x + NT * i;
      const int row = id >> 3, col = (id & 7) * 8;
      const int64_t m = m0 + row;
      const bool ok = m < g.M;
      const int64_t mc = ok ? m : g.M - 1;  // rows past M: load a valid row, then zero it
      uint4 x;
      if constexpr (A_F32) {
        const float* p = static_cast<const float*>(g.a) + mc * g.lda + k0 + col;
        const float4 lo = reinterpret_cast<const float4*>(p)[0];
        const float4 hi = reinterpret_cast<const float4*>(p)[1];
        x = make_uint4(pack2h(lo.x, lo.y), pack2h(lo.z, lo.w), pack2h(hi.x, hi.y),
                       pack2h(hi.z, hi.w));
      } else {
        x = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(g.a) + mc * g.lda +
                                            k0 + col);
      }
      v[i] = ok ? x : make_uint4(0, 0, 0, 0);
    }
  }
  __device__ __forceinline__ void store(uint16_t* s) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int id = threadIdx.x + NT * i;
      *reinterpret_cast<uint4*>(s + lds_off(id >> 3, id & 7)) = v[i];
    }
  }
};

// W row of LDS B row `n` in the NT orientation. SwiGLU: within each wavefront's WN rows, the
// first half are gate rows and the second half the up rows of the same output columns.
template <int BN, int WN, int EPI>
__device__ __forceinline__ int64_t nt_wrow(const GemmArgs& g, int64_t tile_n, int n) {
  if constexpr (EPI == kEpiSwiglu) {
    constexpr int HALF = WN / 2;
    const int64_t j = tile_n * (BN / 2) + (n / WN) * HALF + (n % HALF);
    return (n % WN) >= HALF ? g.I + j : j;
  } else {
    return tile_n * BN + n;
  }
}

// NT: B tile = W rows (BN) x 64 columns; a run = 32 columns of one row (16 bytes, one scale).
template <int BN, int WN, int NT, int EPI>
struct BLoaderNT {
  static constexpr int kPer = BN * kBK / 32 / NT;
  uint4 v[kPer];
  ScaleIn sc[kPer];
  __device__ __forceinline__ void load(const GemmArgs& g, int64_t tile_n, int64_t k0) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int id = threadIdx.x + NT * i;
      const int n = id % BN, part = id / BN;
      const int64_t e = nt_wrow<BN, WN, EPI>(g, tile_n, n) * g.Kw + k0 + 32 * part;
      v[i] = *reinterpret_cast<const uint4*>(g.w.packed + (e >> 1));
      sc[i] = scale_load(g.w, e >> g.w.bs1_shift);
    }
  }
  __device__ __forceinline__ void store(uint16_t* s, const GemmArgs& g, const float* lut,
                                        const float* c2, const float* offs) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int id = threadIdx.x + NT * i;
      const int n = id % BN, part = id / BN;
      const float scale = scale_of(sc[i], g.w.nested, c2, offs);
      *reinterpret_cast<uint4*>(s + lds_off(n, 4 * part + 0)) = nf4_decode_word(v[i].x, scale, lut);
      *reinterpret_cast<uint4*>(s + lds_off(n, 4 * part + 1)) = nf4_decode_word(v[i].y, scale, lut);
      *reinterpret_cast<uint4*>(s + lds_off(n, 4 * part + 2)) = nf4_decode_word(v[i].z, scale, lut);
      *reinterpret_cast<uint4*>(s + lds_off(n, 4 * part + 3)) = nf4_decode_word(v[i].w, scale, lut);
    }
  }
};

// NN: B tile = W rows k0..k0+63 x columns n0..n0+BN-1; thread t decodes rows 8g..8g+7 of a
// 4-column group (2 bytes per row, one scale per row) and writes each column's 8 values as one
// 16-byte chunk of the [n][k] tile. The eight scales' inputs are kept compact (absmax codes
// packed four to a register, segment numbers as 2-bit fields) to stay within two wavefronts'
// register budget per SIMD.
template <int BN, int NT>
struct BLoaderNN {
  static constexpr int CW = 8 * BN / NT;   // columns per thread: 4 or 8
  static constexpr int CHUNKS = BN / CW;   // column groups per row
  static_assert(CW == 4 || CW == 8, "8 rows x 4 or 8 columns per thread");
  static constexpr int VR = CW == 8 ? 8 : 4;  // registers of packed bytes
  uint32_t v[VR];  // CW == 4: row i's two bytes in half i & 1 of v[i / 2]; CW == 8: row i
  uint32_t q[2];   // nested: absmax code of row i in byte i & 3 of q[i / 4]
  float a2[8];     // nested: absmax2; plain: the fp32 absmax
  uint32_t seg;    // 2 bits per row
  __device__ __forceinline__ void load(const GemmArgs& g, int64_t n0, int64_t k0) {
    const int c = threadIdx.x % CHUNKS, gr = threadIdx.x / CHUNKS;
    seg = 0;
    uint32_t vv[8], qq[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t e = (k0 + 8 * gr + i) * g.Kw + n0 + CW * c;
      if constexpr (CW == 8) vv[i] = *reinterpret_cast<const uint32_t*>(g.w.packed + (e >> 1));
      else vv[i] = *reinterpret_cast<const uint16_t*>(g.w.packed + (e >> 1));
      const ScaleIn si = scale_load(g.w, e >> g.w.bs1_shift);
      qq[i] = si.q;
      a2[i] = si.a2;
      seg |= si.seg << (2 * i);
    }
#pragma unroll
    for (int i = 0; i < VR; ++i) v[i] = CW == 8 ? vv[i] : (vv[2 * i] | (vv[2 * i + 1] << 16));
#pragma unroll
    for (int i = 0; i < 2; ++i)
      q[i] = qq[4 * i] | (qq[4 * i + 1] << 8) | (qq[4 * i + 2] << 16) | (qq[4 * i + 3] << 24);
  }
  __device__ __forceinline__ void store(uint16_t* s, const GemmArgs& g, const float* lut,
                                        const float* c2, const float* offs) const {
    const int c = threadIdx.x % CHUNKS, gr = threadIdx.x / CHUNKS;
    uint32_t out[CW][4];  // column j, row pair p: fp16 pair (row 2p, row 2p + 1)
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      float x[2][CW];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int i = 2 * p + h;
        const float scale = scale_of(
            ScaleIn{(q[i >> 2] >> (8 * (i & 3))) & 0xFFu, a2[i], (seg >> (2 * i)) & 3u},
            g.w.nested, c2, offs);
        const uint32_t row = CW == 8 ? v[i] : ((v[i >> 1] >> (16 * (i & 1))) & 0xFFFFu);
#pragma unroll
        for (int k = 0; k < CW / 2; ++k) {
          const uint32_t byte = (row >> (8 * k)) & 0xFFu;
          float a = lut[byte >> 4] * scale;
          float b = lut[byte & 15u] * scale;
          fp32_barrier(a);  // fp16(fp32(level * scale)): two roundings
          fp32_barrier(b);
          x[h][2 * k] = a;
          x[h][2 * k + 1] = b;
        }
      }
#pragma unroll
      for (int j = 0; j < CW; ++j) out[j][p] = pack2h(x[0][j], x[1][j]);
    }
#pragma unroll
    for (int j = 0; j < CW; ++j)
      *reinterpret_cast<uint4*>(s + lds_off(CW * c + j, gr)) =
          make_uint4(out[j][0], out[j][1], out[j][2], out[j][3]);
  }
};

template <int BM, int BN>
struct GemmSmem {
  uint16_t a[2][BM * kBK];
  uint16_t b[2][BN * kBK];
  float lut[16];
  float c2[256];
  float offs[4];
};

template <int BM, int BN, int WGM, int WGN, bool NN, int EPI, bool A_F32>
__global__ __launch_bounds__(WGM * WGN * 64) void nf4_gemm_kernel(GemmArgs g) {
  constexpr int NT = WGM * WGN * 64;
  constexpr int WM = BM / WGM, WN = BN / WGN, FM = WM / 32, FN = WN / 32;
  __shared__ GemmSmem<BM, BN> sm;
  const int tid = threadIdx.x;
  if (tid < 16) sm.lut[tid] = g.w.standard ? kNF4Levels[tid] : g.w.code[tid];
  if (g.w.nested) {
    for (int i = tid; i < 256; i += NT) sm.c2[i] = g.w.code2[i];
    // segment offsets: one per stacked weight; an absent segment bound is INT64_MAX
    if (tid < 3) {
      const int nseg = 1 + (int)(g.w.seg1 != INT64_MAX) + (int)(g.w.seg2 != INT64_MAX);
      sm.offs[tid] = g.w.offsets[tid < nseg ? tid : 0];
    }
  }

  const int64_t m_tiles = (g.M + BM - 1) / BM;
  const int64_t t = tile_order(blockIdx.x, gridDim.x);
  const int64_t tile_m = t % m_tiles, tile_n = t / m_tiles;
  const int64_t m0 = tile_m * BM;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;

  ALoader<BM, NT, A_F32> la;
  BLoaderNT<BN, WN, NT, EPI> lbt;
  BLoaderNN<BN, NT> lbn;
  const int64_t kt0 = (int64_t)blockIdx.z * g.kt_per_split;
  int64_t kt1 = kt0 + g.kt_per_split;
  const int64_t ktiles_all = g.Kr / kBK;
  if (kt1 > ktiles_all) kt1 = ktiles_all;

  auto load_tile = [&](int64_t kt) {
    la.load(g, m0, kt * kBK);
    if constexpr (NN) lbn.load(g, tile_n * BN, kt * kBK);
    else lbt.load(g, tile_n, kt * kBK);
  };
  auto store_tile = [&](int buf) {
    la.store(sm.a[buf]);
    if constexpr (NN) lbn.store(sm.b[buf], g, sm.lut, sm.c2, sm.offs);
    else lbt.store(sm.b[buf], g, sm.lut, sm.c2, sm.offs);
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};

  if (kt0 < kt1) load_tile(kt0);
  __syncthreads();  // lut, c2, offs
  if (kt0 < kt1) store_tile(0);
  __syncthreads();

  const int frow = lane & 31, fchunk = lane >> 5;
  for (int64_t kt = kt0; kt < kt1; ++kt) {
    const int buf = (kt - kt0) & 1;
    const bool more = kt + 1 < kt1;
    if (more) load_tile(kt + 1);
    const uint16_t* sa = sm.a[buf];
    const uint16_t* sb = sm.b[buf];
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      half8_t af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const half8_t*>(
            sa + lds_off(wm * WM + i * 32 + frow, 2 * ks + fchunk));
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[j] = *reinterpret_cast<const half8_t*>(
            sb + lds_off(wn * WN + j * 32 + frow, 2 * ks + fchunk));
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (more) store_tile(buf ^ 1);
    __syncthreads();
  }

  // epilogue: register r of lane l in a 32x32 block holds row 8(r/4) + 4(l/32) + r%4, col l%32
  const int col_in = lane & 31;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t m = m0 + wm * WM + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      if (m >= g.M) continue;
      if constexpr (EPI == kEpiSwiglu) {
#pragma unroll
        for (int j = 0; j < FN / 2; ++j) {
          const int64_t n = tile_n * (BN / 2) + wn * (WN / 2) + j * 32 + col_in;
          const float gt = h2f(f2h(acc[i][j][r])), up = h2f(f2h(acc[i][j + FN / 2][r]));
          const float mval = gt * sigmoid_fast(gt) * up;  // as glu_fwd_kernel
          static_cast<uint16_t*>(g.c)[m * g.ldc + n] = f2h_bits(mval);
        }
      } else {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int64_t n = tile_n * BN + wn * WN + j * 32 + col_in;
          float v = acc[i][j][r];
          if constexpr (EPI == kEpiPartial) {
            static_cast<float*>(g.c)[((int64_t)blockIdx.z * g.M + m) * g.N + n] = v;
          } else if constexpr (EPI == kEpiResid) {
            static_cast<float*>(g.c)[m * g.ldc + n] = g.resid[m * g.ldr + n] + h2f(f2h(v));
          } else {
            if constexpr (EPI == kEpiBias) v += h2f_bits(g.bias[n]);
            static_cast<uint16_t*>(g.c)[m * g.ldc + n] = f2h_bits(v);
          }
        }
      }
    }
  }
}

// Sum of the split-K partials [splits, M, N] and the epilogue (store / bias / residual).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* ws, int splits,
                                                            int64_t M, int64_t N, int epi,
                                                            void* c, int64_t ldc,
                                                            const uint16_t* bias,
                                                            const float* resid, int64_t ldr) {
  const int64_t idx = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (idx >= M * N) return;
  const int64_t m = idx / N, n = idx - m * N;  // N % 4 == 0: four columns of one row
  float4 s = reinterpret_cast<const float4*>(ws + idx)[0];
  for (int k = 1; k < splits; ++k) {
    const float4 t = reinterpret_cast<const float4*>(ws + (int64_t)k * M * N + idx)[0];
    s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
  }
  float v[4] = {s.x, s.y, s.z, s.w};
  if (epi == kEpiResid) {
    float* out = static_cast<float*>(c) + m * ldc + n;
    const float* r = resid + m * ldr + n;
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = r[i] + h2f(f2h(v[i]));
  } else {
    uint16_t* out = static_cast<uint16_t*>(c) + m * ldc + n;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (epi == kEpiBias) v[i] += h2f_bits(bias[n + i]);
      out[i] = f2h_bits(v[i]);
    }
  }
}

}  // namespace qlora

using namespace qlora;

namespace {

template <int BM, int BN, int WGN, bool NN, int EPI, bool A_F32>
void launch_gemm(const GemmArgs& g, dim3 grid, hipStream_t s) {
  constexpr int WGM = 2;
  hipLaunchKernelGGL((nf4_gemm_kernel<BM, BN, WGM, WGN, NN, EPI, A_F32>), grid,
                     dim3(WGM * WGN * 64), 0, s, g);
}

template <int BM, int BN, int WGN, bool NN, int EPI>
void launch_a(const GemmArgs& g, dim3 grid, hipStream_t s, bool a_f32) {
  if (a_f32) launch_gemm<BM, BN, WGN, NN, EPI, true>(g, grid, s);
  else launch_gemm<BM, BN, WGN, NN, EPI, false>(g, grid, s);
}

template <int BM, int BN, int WGN, bool NN>
void launch_epi(const GemmArgs& g, dim3 grid, hipStream_t s, bool a_f32, int epi) {
  switch (epi) {
    case kEpiStore: launch_a<BM, BN, WGN, NN, kEpiStore>(g, grid, s, a_f32); break;
    case kEpiBias: launch_a<BM, BN, WGN, NN, kEpiBias>(g, grid, s, a_f32); break;
    case kEpiResid: launch_a<BM, BN, WGN, NN, kEpiResid>(g, grid, s, a_f32); break;
    case kEpiPartial: launch_a<BM, BN, WGN, NN, kEpiPartial>(g, grid, s, a_f32); break;
    default:
      if constexpr (!NN) launch_a<BM, BN, WGN, NN, kEpiSwiglu>(g, grid, s, a_f32);
      break;
  }
}

bool al(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

}  // namespace

// mode: 0 = NT (C = A W^T), 1 = NN (C = A W). epi: 0 store fp16, 1 + bias, 2 fp32 residual,
// 3 SwiGLU (NT only). a_f32: A is fp32 (rounded to fp16 on load). tile: 0 = 256 x 256
// (8 wavefronts), 1 = 128 x 128 (4 wavefronts), 2 = 256 x 256 (4 wavefronts of 128 x 128). splits > 1: split-K through `ws` (fp32, splits * M * N elements).
QLORA_API int qlora_nf4_gemm(const void* a, int64_t lda, int32_t a_f32, const void* packed,
                             const void* absmax, const float* code2, const float* absmax2,
                             const float* offsets, const float* code, int32_t nested,
                             int32_t standard, int32_t bs1, int32_t bs2, int64_t seg1,
                             int64_t seg2, int64_t w_rows, int64_t w_cols, void* c, int64_t ldc,
                             const void* bias, const float* resid, int64_t ldr, int64_t M,
                             int32_t mode, int32_t epi, int64_t swiglu_I, int32_t tile,
                             int32_t splits, float* ws, int64_t ws_elems, void* stream) {
  QLORA_CHECK_ARG(M >= 0 && w_rows > 0 && w_cols > 0);
  if (M == 0) return 0;
  QLORA_CHECK_ARG(a && packed && absmax && c && (mode == 0 || mode == 1));
  QLORA_CHECK_ARG(epi >= 0 && epi <= 3 && !(epi == 3 && mode != 0));
  QLORA_CHECK_ARG(tile >= 0 && tile <= 2);
  QLORA_CHECK_ARG(splits >= 1 && splits <= 16 && !(splits > 1 && epi == 3));
  QLORA_CHECK_ARG(bs1 >= 32 && (bs1 & (bs1 - 1)) == 0);
  QLORA_CHECK_ARG(!nested || (code2 && absmax2 && offsets && bs2 > 0 && (bs2 & (bs2 - 1)) == 0));
  QLORA_CHECK_ARG(standard || code);
  QLORA_CHECK_ARG(epi != 1 || bias);
  QLORA_CHECK_ARG(epi != 2 || (resid && ldr >= 0));
  const int BM = tile == 1 ? 128 : 256, BN = BM;
  int64_t N, Kr;
  if (mode == 0) {
    Kr = w_cols;
    N = epi == 3 ? swiglu_I : w_rows;
    QLORA_CHECK_ARG(epi != 3 || (swiglu_I % (BN / 2) == 0 && 2 * swiglu_I == w_rows));
    QLORA_CHECK_ARG(epi == 3 || w_rows % BN == 0);
    QLORA_CHECK_ARG(w_cols % kBK == 0);
  } else {
    Kr = w_rows;
    N = w_cols;
    QLORA_CHECK_ARG(w_cols % BN == 0 && w_rows % kBK == 0);
  }
  QLORA_CHECK_ARG(lda >= Kr && ldc >= N && (epi != 2 || ldr >= N));
  QLORA_CHECK_ARG(lda % 8 == 0 && al(a, 16) && al(packed, 16));
  QLORA_CHECK_ARG(splits == 1 || (ws && ws_elems >= (int64_t)splits * M * N && al(ws, 16)));
  const int64_t n_tiles = epi == 3 ? N / (BN / 2) : N / BN;
  const int64_t grid = qlora_cdiv(M, BM) * n_tiles;
  QLORA_CHECK_ARG(grid < (1ll << 31));
  const int64_t ktiles = Kr / kBK;
  GemmArgs g;
  g.a = a;
  g.lda = lda;
  g.w = NF4Ref{static_cast<const uint8_t*>(packed), absmax, code2, absmax2, offsets, code,
               seg1, seg2, __builtin_ctz(bs1), nested ? __builtin_ctz(bs2) : 0, nested,
               standard};
  g.Kw = w_cols;
  g.c = splits > 1 ? (void*)ws : c;
  g.ldc = ldc;
  g.bias = static_cast<const uint16_t*>(bias);
  g.resid = resid;
  g.ldr = ldr;
  g.M = M;
  g.N = N;
  g.Kr = Kr;
  g.I = swiglu_I;
  g.kt_per_split = qlora_cdiv(ktiles, splits);
  const int kepi = splits > 1 ? (int)kEpiPartial : epi;
  hipStream_t s = (hipStream_t)stream;
  const dim3 gdim((unsigned)grid, 1, (unsigned)splits);
  if (mode == 0) {
    if (tile == 0) launch_epi<256, 256, 4, false>(g, gdim, s, a_f32, kepi);
    else if (tile == 1) launch_epi<128, 128, 2, false>(g, gdim, s, a_f32, kepi);
    else launch_epi<256, 256, 2, false>(g, gdim, s, a_f32, kepi);
  } else {
    if (tile == 0) launch_epi<256, 256, 4, true>(g, gdim, s, a_f32, kepi);
    else if (tile == 1) launch_epi<128, 128, 2, true>(g, gdim, s, a_f32, kepi);
    else launch_epi<256, 256, 2, true>(g, gdim, s, a_f32, kepi);
  }
  int rc = qlora_launch_status();
  if (rc != 0 || splits == 1) return rc;
  QLORA_CHECK_ARG(N % 4 == 0 && ldc % 4 == 0 && (epi != 2 || ldr % 4 == 0));
  const int64_t quads = M * N / 4;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)qlora_cdiv(quads, 256)), dim3(256), 0,
                     s, ws, splits, M, N, epi, c, ldc, static_cast<const uint16_t*>(bias), resid,
                     ldr);
  return qlora_launch_status();
}
