// Shared helpers for the gfx950 kernels of the QLoRA training step.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define QLORA_API extern "C" __attribute__((visibility("default")))

// Error convention of every entry point: 0 on success, a hipError_t otherwise. Arguments that a
// kernel cannot take are rejected before anything is launched.
#define QLORA_CHECK_ARG(cond)                          \
  do {                                                 \
    if (!(cond)) return (int)hipErrorInvalidValue;     \
  } while (0)

static inline int qlora_launch_status() { return (int)hipGetLastError(); }

// Returned by an allocation-free entry point whose problem needs more than its static scratch.
#define QLORA_ERR_SCRATCH_TOO_SMALL 300001

static inline int64_t qlora_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

namespace qlora {

constexpr int kWave = 64;

// ---- fp16 <-> fp32 (round to nearest even, as the reference's `.to(tl.float16)`) -------------
__device__ __forceinline__ float h2f(__half h) { return __half2float(h); }
__device__ __forceinline__ __half f2h(float f) { return __float2half_rn(f); }

__device__ __forceinline__ float h2f_bits(uint16_t b) {
  return __half2float(__ushort_as_half(b));
}
__device__ __forceinline__ uint16_t f2h_bits(float f) {
  return __half_as_ushort(__float2half_rn(f));
}
// two fp32 -> packed pair of fp16 bits (low half = a)
__device__ __forceinline__ uint32_t pack2h(float a, float b) {
  return (uint32_t)f2h_bits(a) | ((uint32_t)f2h_bits(b) << 16);
}
// SwiGLU's sigmoid, 1 / (1 + 2^(-g log2 e)) with the hardware exp2 and reciprocal (v_exp_f32,
// v_rcp_f32, about 1 ulp each in fp32): g -> -inf gives 1 / inf = 0, g -> +inf gives 1, NaN stays
// NaN. Every kernel that forms silu(g) uses this one, so their fp16 results agree bit for bit.
__device__ __forceinline__ float sigmoid_fast(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}

__device__ __forceinline__ float lo_h(uint32_t w) { return h2f_bits((uint16_t)(w & 0xFFFFu)); }
__device__ __forceinline__ float hi_h(uint32_t w) { return h2f_bits((uint16_t)(w >> 16)); }

// ---- wavefront reductions (64 lanes) ----------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// ---- buffer loads ------------------------------------------------------------------------------
// A wave-uniform resource over [base, base + bytes): loads at offsets past the end return zeros
// (the hardware range check), so tile loads need neither clamped indices nor selects - and a
// select of a loaded value is what the compiler may turn into a branch around the load, whose
// join then waits for every load in flight.
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float buf_load_f32(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
// A vector store through the resource: bytes past its end are dropped by the range check.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void buf_store16(rsrc_t r, uint32_t off, uint4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, off, 0, 0);
}

}  // namespace qlora
