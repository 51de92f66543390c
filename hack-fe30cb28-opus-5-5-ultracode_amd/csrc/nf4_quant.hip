// NF4 double quantisation on the GPU, in the storage format the path reads (a bitsandbytes
// Params4bit / QuantState: engine.py:77-101, hostload.py:66-79): the load-time step before the
// dequant kernel. Restates bitsandbytes 0.50.2's published quantiser (functional.quantize_4bit
// with compress_statistics=True: kQuantizeBlockwise with dQuantizeNF4, then quantize_blockwise of
// the centred absmax with dQuantize over the signed dynamic map).
//
// Per block of 64 consecutive elements (one 32-lane half of a wavefront, two elements a lane):
//   absmax = max |w| (fp32), normed = w * (1 / absmax) (0 for an all-zero block),
//   code   = NF4 decision tree: x > t_i for the 15 midpoints of neighbouring levels rounded to
//            fp32 (ties go to the lower level), packed two per byte, even element high.
// Double quantisation of the fp32 absmax a_b (n values):
//   offset = fp32(S / n), S = the sum of the a_b in fp64 over a binary tree of adjacent pairs
//            (the values zero-padded to a power of 1024; 1024 per workgroup, level by level);
//   per block of 256: v = a_b - offset (fp32), absmax2 = max |v|, code = dQuantize(v / absmax2)
//            over the sorted 256-entry code: a 7-step binary search, then the nearer of the last
//            pivots by fp32 midpoints (bitsandbytes' rule; its tie breaking included).
#include "common.h"

namespace qlora {
namespace nq {

constexpr int kBs1 = 64;
constexpr int kBs2 = 256;
constexpr int kSumChunk = 1024;  // absmax values summed per workgroup per level

// Midpoints of neighbouring NF4 levels (the levels of kernels.py:38-41), rounded to fp32.
#define QLORA_MID(a, b) ((float)(((double)(a) + (double)(b)) / 2.0))
__constant__ float kMid[15] = {
    QLORA_MID(-1.0f, -0.6961928009986877f),
    QLORA_MID(-0.6961928009986877f, -0.5250730514526367f),
    QLORA_MID(-0.5250730514526367f, -0.39491748809814453f),
    QLORA_MID(-0.39491748809814453f, -0.28444138169288635f),
    QLORA_MID(-0.28444138169288635f, -0.18477343022823334f),
    QLORA_MID(-0.18477343022823334f, -0.09105003625154495f),
    QLORA_MID(-0.09105003625154495f, 0.0f),
    QLORA_MID(0.0f, 0.07958029955625534f),
    QLORA_MID(0.07958029955625534f, 0.16093020141124725f),
    QLORA_MID(0.16093020141124725f, 0.24611230194568634f),
    QLORA_MID(0.24611230194568634f, 0.33791524171829224f),
    QLORA_MID(0.33791524171829224f, 0.44070982933044434f),
    QLORA_MID(0.44070982933044434f, 0.5626170039176941f),
    QLORA_MID(0.5626170039176941f, 0.7229568362236023f),
    QLORA_MID(0.7229568362236023f, 1.0f),
};
#undef QLORA_MID

// The tree's leaf for x: the number of midpoints below x (the thresholds are sorted, so the
// branch taken at each node is the same comparison); NaN compares false everywhere: code 0.
__device__ __forceinline__ uint32_t nf4_code(float x) {
  uint32_t c = 0;
#pragma unroll
  for (int i = 0; i < 15; ++i) c += x > kMid[i] ? 1u : 0u;
  return c;
}

template <bool F32>
__global__ __launch_bounds__(256) void nf4_quant_kernel(const void* w, uint8_t* packed,
                                                        float* absmax, int64_t n_blocks) {
  const int64_t blk = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  if (blk >= n_blocks) return;  // uniform over each 32-lane half
  const int j = threadIdx.x & 31;
  const int64_t e = blk * kBs1 + 2 * j;
  float x0, x1;
  if constexpr (F32) {
    const float2 v = *reinterpret_cast<const float2*>(static_cast<const float*>(w) + e);
    x0 = v.x;
    x1 = v.y;
  } else {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(w) + e);
    x0 = lo_h(v);
    x1 = hi_h(v);
  }
  float m = fmaxf(fabsf(x0), fabsf(x1));
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
  const float inv = m > 0.f ? 1.0f / m : 0.f;
  const uint32_t c0 = nf4_code(x0 * inv), c1 = nf4_code(x1 * inv);
  packed[e >> 1] = (uint8_t)((c0 << 4) | c1);
  if (j == 0) absmax[blk] = m;
}

// One level of the offset's sum: out[c] = tree sum of in[1024 c .. 1024 c + 1023] (zeros past
// n), in fp64, adjacent pairs first. `in_f32`: the level's input is the fp32 absmax.
__global__ __launch_bounds__(256) void tree_sum_kernel(const float* in32, const double* in64,
                                                       int64_t n, double* out) {
  __shared__ double part[4];
  const int64_t base = (int64_t)blockIdx.x * kSumChunk + 4 * threadIdx.x;
  double v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t k = base + i;
    v[i] = k < n ? (in32 ? (double)in32[k] : in64[k]) : 0.0;
  }
  double s = (v[0] + v[1]) + (v[2] + v[3]);
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) s = s + __shfl_xor(s, off, kWave);
  if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = s;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = (part[0] + part[1]) + (part[2] + part[3]);
}

// bitsandbytes' dQuantize (deterministic): 7 halving steps from pivot 127 over the sorted code,
// then the nearer of the last pivot and its bracketing pivot by an fp32 midpoint.
__device__ __forceinline__ uint32_t dquantize(const float* code, float x) {
  int pivot = 127, upper_pivot = 255, lower_pivot = 0;
  float lower = -1.0f, upper = 1.0f;
  float val = code[pivot];
  for (int i = 64; i > 0; i >>= 1) {
    if (x > val) {
      lower_pivot = pivot;
      lower = val;
      pivot += i;
    } else {
      upper_pivot = pivot;
      upper = val;
      pivot -= i;
    }
    val = code[pivot];
  }
  if (upper_pivot == 255) upper = code[upper_pivot];
  if (lower_pivot == 0) lower = code[lower_pivot];
  if (x > val) {
    const float mid = (upper + val) * 0.5f;
    return x > mid ? upper_pivot : pivot;
  }
  const float mid = (lower + val) * 0.5f;
  return x < mid ? lower_pivot : pivot;
}

// Per block of 256 absmax values: offset from the sum, absmax2, the 8-bit codes.
__global__ __launch_bounds__(kBs2) void absmax_quant_kernel(const float* absmax, int64_t n,
                                                            const double* total,
                                                            const float* code2, uint8_t* q,
                                                            float* absmax2, float* offset_out) {
  __shared__ float code[256];
  __shared__ float wmax[kBs2 / kWave];
  code[threadIdx.x] = code2[threadIdx.x];
  const float offset = (float)(*total / (double)n);
  if (blockIdx.x == 0 && threadIdx.x == 0) *offset_out = offset;
  const int64_t i = (int64_t)blockIdx.x * kBs2 + threadIdx.x;
  const float v = i < n ? absmax[i] - offset : 0.f;
  float m = fabsf(v);
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
  if ((threadIdx.x & (kWave - 1)) == 0) wmax[threadIdx.x / kWave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const float inv = m > 0.f ? 1.0f / m : 0.f;
  if (i < n) q[i] = (uint8_t)dquantize(code, v * inv);
  if (threadIdx.x == 0) absmax2[blockIdx.x] = m;
}

}  // namespace nq
}  // namespace qlora

using namespace qlora::nq;

// NF4 quantisation of a weight of n_blocks x 64 elements (fp16, or fp32 if w_f32), row-major
// flat: packed u8 [n_blocks * 32] (element i in byte i/2, high nibble for even i), absmax f32
// [n_blocks]. w 8-byte aligned (fp32) or 4-byte aligned (fp16). The step before the path: the
// bytes bitsandbytes' quantize_4bit stores in a Params4bit (engine.py:77-101).
QLORA_API int qlora_nf4_quantize(const void* w, int32_t w_f32, int64_t n_blocks, void* packed,
                                 float* absmax, void* stream) {
  QLORA_CHECK_ARG(n_blocks >= 0);
  if (n_blocks == 0) return 0;
  QLORA_CHECK_ARG(w && packed && absmax);
  QLORA_CHECK_ARG(((uintptr_t)w & (w_f32 ? 7 : 3)) == 0);
  QLORA_CHECK_ARG(qlora_cdiv(n_blocks, 8) < (1ll << 31));
  const dim3 grid((unsigned)qlora_cdiv(n_blocks, 8));
  if (w_f32)
    hipLaunchKernelGGL(nf4_quant_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, w,
                       static_cast<uint8_t*>(packed), absmax, n_blocks);
  else
    hipLaunchKernelGGL(nf4_quant_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, w,
                       static_cast<uint8_t*>(packed), absmax, n_blocks);
  return qlora_launch_status();
}

// fp64 workspace elements of qlora_nf4_quantize_stats for n absmax values.
QLORA_API int qlora_nf4_quantize_stats_workspace(int64_t n, int64_t* elems) {
  QLORA_CHECK_ARG(elems && n >= 0);
  int64_t total = 0;
  for (int64_t m = n; m > 1;) {
    m = qlora_cdiv(m, kSumChunk);
    total += m;
  }
  *elems = total + 1;
  return 0;
}

// Double quantisation of n fp32 absmax values (blocks of 256): q u8 [n] codes into code2 (the
// sorted signed dynamic map, f32 [256]), absmax2 f32 [ceil(n / 256)], offset f32 [1]; work:
// fp64 of qlora_nf4_quantize_stats_workspace elements. The QuantState's absmax / state2 /
// offset of a compress_statistics quantisation (engine.py:78-101).
QLORA_API int qlora_nf4_quantize_stats(const float* absmax, int64_t n, const float* code2,
                                       double* work, int64_t work_elems, uint8_t* q,
                                       float* absmax2, float* offset, void* stream) {
  QLORA_CHECK_ARG(n >= 0);
  if (n == 0) return 0;
  int64_t need;
  qlora_nf4_quantize_stats_workspace(n, &need);
  QLORA_CHECK_ARG(absmax && code2 && work && q && absmax2 && offset && work_elems >= need);
  QLORA_CHECK_ARG(qlora_cdiv(n, kBs2) < (1ll << 31));
  hipStream_t s = (hipStream_t)stream;
  // levels of the sum: n -> ceil(n / 1024) -> ... -> 1 (at least one level)
  const float* in32 = absmax;
  const double* in64 = nullptr;
  int64_t m = n;
  double* out = work;
  do {
    const int64_t groups = qlora_cdiv(m, kSumChunk);
    hipLaunchKernelGGL(tree_sum_kernel, dim3((unsigned)groups), dim3(256), 0, s, in32, in64, m,
                       out);
    if (int rc = qlora_launch_status()) return rc;
    in32 = nullptr;
    in64 = out;
    out += groups;
    m = groups;
  } while (m > 1);
  hipLaunchKernelGGL(absmax_quant_kernel, dim3((unsigned)qlora_cdiv(n, kBs2)), dim3(kBs2), 0, s,
                     absmax, n, in64, code2, q, absmax2, offset);
  return qlora_launch_status();
}
