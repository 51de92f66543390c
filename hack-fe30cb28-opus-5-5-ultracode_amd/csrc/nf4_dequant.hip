// Standalone NF4 -> fp16 dequantisation (reference: nf4_dequant_kernel, kernels.py:68-105;
// launched by NF4Weight.dequant_into / NF4Group.dequant_into, engine.py:103-157).
//
// HBM-bound: per 8 output values one 32-bit word of nibbles is read and 16 bytes are written.
// Each thread handles WPT words spaced a workgroup apart, so every load and every 16-byte store
// instruction of a wavefront covers one contiguous span (256 B in, 1 KiB out). The 16 levels
// sit in LDS; the per-block scale comes from the (L1/L2-resident) absmax tables.
#include "nf4.h"

namespace qlora {

constexpr int kDequantThreads = 256;
constexpr int kDequantWPT = 4;

__global__ __launch_bounds__(kDequantThreads) void nf4_dequant_kernel(NF4Ref w, uint4* out,
                                                                       int64_t n_words) {
  __shared__ float lut[16];
  if (threadIdx.x < 16)
    lut[threadIdx.x] = w.standard ? kNF4Levels[threadIdx.x] : w.code[threadIdx.x];
  __syncthreads();
  const uint32_t* words = reinterpret_cast<const uint32_t*>(w.packed);
  const int64_t base = (int64_t)blockIdx.x * (kDequantThreads * kDequantWPT) + threadIdx.x;
  uint32_t v[kDequantWPT];
#pragma unroll
  for (int i = 0; i < kDequantWPT; ++i) {
    const int64_t idx = base + i * kDequantThreads;
    v[i] = idx < n_words ? __builtin_nontemporal_load(words + idx) : 0u;
  }
#pragma unroll
  for (int i = 0; i < kDequantWPT; ++i) {
    const int64_t idx = base + i * kDequantThreads;
    if (idx < n_words) {
      const float scale = nf4_block_scale(w, idx >> (w.bs1_shift - 3));
      out[idx] = nf4_decode_word(v[i], scale, lut);
    }
  }
}

}  // namespace qlora

using namespace qlora;

QLORA_API int qlora_nf4_dequant(const void* packed, const void* absmax, const float* code2,
                                const float* absmax2, const float* offsets, const float* code,
                                void* out, int64_t n_blocks, int32_t nested, int32_t standard,
                                int32_t bs1, int32_t bs2, int64_t seg1, int64_t seg2,
                                void* stream) {
  QLORA_CHECK_ARG(n_blocks >= 0);
  if (n_blocks == 0) return 0;
  QLORA_CHECK_ARG(packed && absmax && out);
  QLORA_CHECK_ARG(bs1 >= 8 && (bs1 & (bs1 - 1)) == 0);
  QLORA_CHECK_ARG(!nested || (code2 && absmax2 && offsets && bs2 > 0 && (bs2 & (bs2 - 1)) == 0));
  QLORA_CHECK_ARG(standard || code);
  QLORA_CHECK_ARG(((uintptr_t)packed & 3) == 0 && ((uintptr_t)out & 15) == 0);
  NF4Ref w{static_cast<const uint8_t*>(packed), absmax, code2, absmax2, offsets, code,
           seg1, seg2, __builtin_ctz(bs1), nested ? __builtin_ctz(bs2) : 0, nested, standard};
  const int64_t n_words = n_blocks * (bs1 / 8);
  const int64_t grid = qlora_cdiv(n_words, (int64_t)kDequantThreads * kDequantWPT);
  QLORA_CHECK_ARG(grid < (1ll << 31));
  hipLaunchKernelGGL(nf4_dequant_kernel, dim3((unsigned)grid), dim3(kDequantThreads), 0,
                     (hipStream_t)stream, w, static_cast<uint4*>(out), n_words);
  return qlora_launch_status();
}
