// NF4 (bitsandbytes 4-bit NormalFloat) decode shared by the standalone dequant kernel and the
// fused dequant-GEMM B-operand loaders (reference: kernels.py:34-105, engine.py:74-157).
//
// Element i of a row-major [N, K] weight is nibble (i & 1 ? low : high) of byte i / 2. Its scale
// is that of block b = i / BS1:
//   nested:  fp32(fp32(code2[absmax_q[b]] * absmax2[b / BS2]) + offset[segment(b)])
//   plain:   absmax_f32[b]
// and its value fp16_rne(fp32(level[code] * scale)). The multiply and the add are separate IEEE
// operations (never fused): bitsandbytes rounds the product before adding the offset.
#pragma once

#include "common.h"

namespace qlora {

struct NF4Ref {
  const uint8_t* packed;    // numel / 2 bytes
  const void* absmax;       // uint8 [blocks] (nested) or fp32 [blocks]
  const float* code2;       // fp32 [256] (nested)
  const float* absmax2;     // fp32 [ceil(blocks / bs2)] (nested)
  const float* offsets;     // fp32 [segments] (nested)
  const float* code;        // fp32 [16] levels (used when !standard)
  int64_t seg1, seg2;       // first block of the 2nd / 3rd stacked weight
  int bs1_shift, bs2_shift;  // log2 of the block sizes (powers of two, as in bitsandbytes)
  int nested, standard;
};

// The 16 NF4 levels (QLoRA's NormalFloat4 code; kernels.py:38-41), fp32.
__device__ __constant__ static const float kNF4Levels[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

// Pins an fp32 value in a register: the compiler may otherwise fold a rounded fp32 product into
// the following add (FMA) or into the fp16 conversion (v_fma_mix*_f16, one rounding instead of
// two). Emits no instruction.
__device__ __forceinline__ void fp32_barrier(float& v) { __asm__ volatile("" : "+v"(v)); }

// fp32 scale of quantization block b: the product rounded to fp32, then the add.
__device__ __forceinline__ float nf4_block_scale(const NF4Ref& w, int64_t b) {
  if (w.nested) {
    const uint8_t q = static_cast<const uint8_t*>(w.absmax)[b];
    float prod = w.code2[q] * w.absmax2[b >> w.bs2_shift];
    fp32_barrier(prod);
    const int seg = (int)(b >= w.seg1) + (int)(b >= w.seg2);
    return prod + w.offsets[seg];
  }
  return static_cast<const float*>(w.absmax)[b];
}

// Eight fp16 values (as four packed fp16 pairs) from one 32-bit word of packed nibbles (bytes
// in memory order: element 2k is the high nibble of byte k). `lut` holds the 16 levels.
__device__ __forceinline__ uint4 nf4_decode_word(uint32_t word, float scale, const float* lut) {
  uint32_t out[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t byte = (word >> (8 * k)) & 0xFFu;
    float a = lut[byte >> 4] * scale;
    float b = lut[byte & 15u] * scale;
    fp32_barrier(a);  // fp16(fp32(level * scale)): two roundings, as the reference
    fp32_barrier(b);
    out[k] = pack2h(a, b);
  }
  return make_uint4(out[0], out[1], out[2], out[3]);
}

}  // namespace qlora
