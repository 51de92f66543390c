// LoRA-dropout keep masks: the mask PyTorch-ROCm's vectorized dropout kernel draws, computed
// from the generator's (seed, offset) instead of stored (reference: kernels.py:108-126,
// engine.py:767-805).
//
// Element e of a dropout call over a contiguous tensor is handled by thread (e / VEC) mod G of
// the G-thread launch; that thread's j-th uniform4 draw, j = ((e / VEC) div G) * VEC/4 +
// (e mod VEC) / 4, is Philox4x32-10 (Random123) with key = seed and counter
// (ctr + j, thread) -- the layout rocrand_init(seed, subsequence = thread, offset = 4 ctr) gives
// -- and the element takes output word e mod 4, mapped to (0, 1] as 2^-32 + r * 2^-32 in fp32.
// Kept iff that value < 1 - p. The map is non-decreasing in r, so the test is r < keep_below,
// the smallest word whose value is not below 1 - p, found once on the host (rms.hip).
#pragma once

#include "common.h"

namespace qlora {

struct DropParams {
  uint64_t seed;    // generator seed (int64 bits as uint64)
  uint64_t ctr;     // generator offset / 4
  uint64_t G;       // threads of the dropout launch
  float p_keep;     // 1 - p
  int vec;          // elements per vector load (4 or 8)
  uint32_t keep_below;  // word r is kept iff r < keep_below (p_keep < 1)
};

__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint32_t k0, uint32_t k1) {
  constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
  constexpr uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
  // each round's two 32 x 32 -> 64-bit products as one v_mad_u64_u32 apiece (high and low
  // words together), not a mul_hi and a mul_lo; each three-way XOR as one v_bitop3_b32
  // (truth table 0x96 = a ^ b ^ c) instead of two v_xor_b32
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)M0 * c.x, p1 = (uint64_t)M1 * c.z;
    c = make_uint4(__builtin_amdgcn_bitop3_b32((uint32_t)(p1 >> 32), c.y, k0, 0x96),
                   (uint32_t)p1,
                   __builtin_amdgcn_bitop3_b32((uint32_t)(p0 >> 32), c.w, k1, 0x96),
                   (uint32_t)p0);
    k0 += W0;
    k1 += W1;
  }
  return c;
}

// 2^-32 + r * 2^-32 < p_keep as an integer compare; p_keep >= 1 (p = 0) keeps everything:
// PyTorch's dropout returns its input unchanged then.
__device__ __forceinline__ bool keep_word(uint32_t r, const DropParams& d) {
  return r < d.keep_below || d.p_keep >= 1.0f;
}

// The Philox words of the aligned group of four elements that holds element e (4 | e0).
__device__ __forceinline__ uint4 drop_words(const DropParams& d, uint64_t e0) {
  uint64_t g = e0 / (uint64_t)d.vec;
  uint64_t thread, it;
  if ((g >> 32) == 0 && (d.G >> 32) == 0) {
    const uint32_t g32 = (uint32_t)g, G32 = (uint32_t)d.G;
    it = g32 / G32;
    thread = g32 - (uint32_t)it * G32;
  } else {
    it = g / d.G;
    thread = g - it * d.G;
  }
  const uint64_t j = it * (uint64_t)(d.vec >> 2) + (e0 % (uint64_t)d.vec) / 4;
  const uint64_t c = d.ctr + j;
  return philox4x32_10(make_uint4((uint32_t)c, (uint32_t)(c >> 32), (uint32_t)thread,
                                  (uint32_t)(thread >> 32)),
                       (uint32_t)d.seed, (uint32_t)(d.seed >> 32));
}

__device__ __forceinline__ bool drop_keep(const DropParams& d, uint64_t e) {
  const uint4 w = drop_words(d, e & ~(uint64_t)3);
  const uint32_t comp = (uint32_t)(e & 3);
  const uint32_t r = comp == 0 ? w.x : comp == 1 ? w.y : comp == 2 ? w.z : w.w;
  return keep_word(r, d);
}

// Keep bits (bit i = element e0 + i) of four consecutive elements starting at e0, 4 | e0.
__device__ __forceinline__ uint32_t drop_keep4(const DropParams& d, uint64_t e0) {
  const uint4 w = drop_words(d, e0);
  return (uint32_t)keep_word(w.x, d) | ((uint32_t)keep_word(w.y, d) << 1) |
         ((uint32_t)keep_word(w.z, d) << 2) | ((uint32_t)keep_word(w.w, d) << 3);
}

// Keep bits of the quad whose element group has launch thread `thread` and round `it` of that
// thread (vec = 1 << vec_shift; sub = the quad's place within its vector), the body of
// drop_keep4_u32 once the group's division is done.
__device__ __forceinline__ uint32_t drop_keep4_at(const DropParams& d, uint32_t it,
                                                  uint32_t thread, int vec_shift, uint32_t sub) {
  const uint64_t c = d.ctr + (uint64_t)it * (uint32_t)(1 << (vec_shift - 2)) + sub;
  const uint4 w = philox4x32_10(make_uint4((uint32_t)c, (uint32_t)(c >> 32), thread, 0u),
                                (uint32_t)d.seed, (uint32_t)(d.seed >> 32));
  const uint32_t T = d.keep_below;
  return (uint32_t)(w.x < T) | ((uint32_t)(w.y < T) << 1) | ((uint32_t)(w.z < T) << 2) |
         ((uint32_t)(w.w < T) << 3);
}

// drop_keep4 for element indices below 2^32 with vec = 1 << vec_shift: 32-bit index arithmetic
// (a shift and one 32-bit division instead of the 64-bit divisions of drop_words). The caller
// handles p_keep >= 1 (every bit set).
__device__ __forceinline__ uint32_t drop_keep4_u32(const DropParams& d, uint32_t e0,
                                                   uint32_t G32, int vec_shift) {
  const uint32_t g = e0 >> vec_shift;
  const uint32_t it = g / G32, thread = g - it * G32;
  return drop_keep4_at(d, it, thread, vec_shift, (e0 & ((1u << vec_shift) - 1)) >> 2);
}

}  // namespace qlora
