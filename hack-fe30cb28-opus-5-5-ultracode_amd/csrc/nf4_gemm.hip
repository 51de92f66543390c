// fp16 MFMA GEMMs of the step, with the B operand either fp16 in memory or NF4 decoded inside the
// kernel. Reference: the dequant kernel (kernels.py:68-105) followed by cuBLAS at engine.py:1082
// (qkv + bias), 1112 (o), 1163 (gate|up), 1179 (down) in forward and 1239, 1293, 1301, 1316
// (dY W) in backward, and the lm_head products (engine.py:1376-1381).
//
//   NT (forward):  C[m, n] = sum_k A[m, k] B[n, k]      B = W [N, K], K = reduction
//   NN (backward): C[m, n] = sum_k A[m, k] B[k, n]      B = W [K, N], N = W's columns
//
// One workgroup = 4 wavefronts on a 256 x 256 output tile; each wavefront owns a 128 x 128
// block as 4 x 4 v_mfma_f32_32x32x16_f16 accumulators (256 accumulation registers, one
// wavefront per SIMD). Two main loops share the tile, the MFMA order and the epilogues: the NF4
// one (nf4_gemm_kernel, k-tiles of 32, four LDS stages, described below) and the fp16-B one
// (hgemm_kernel, k-tiles of 64, two stages: every DMA lane group then fetches whole 128-byte
// lines, which the L1 serves at twice the rate of 64-byte halves; described at the kernel). On gfx950 a 128 x 128 wavefront block is what keeps the operand reads
// below the MFMA time: per 16-wide k-step a wavefront reads 2 x 128 x 16 fp16 from LDS for 16
// MFMAs; smaller blocks make the kernel LDS-bound.
//
// Operand staging (NF4 kernel). The A tile goes from global memory straight into LDS
// (global_load_lds_dwordx4: a wavefront instruction writes 1 KB of consecutive LDS, lane l at
// 16 l), four stages, the loads of k-tile t + 3 issued in the middle of k-tile t and spread
// over its MFMAs. The LDS layout is swizzled through the choice of which global 16-byte chunk a
// lane fetches: in a K-contiguous tile [rows][32] (A; B in NT) chunk c of row r sits in slot
// c ^ ((r >> 2) & 3), so a fragment read covers all banks; in an N-contiguous tile [32][256] (B
// in NN; the decoded NF4 B is written the same way) chunk c of row k sits in slot
// c ^ ((k & 3) << 2), the pattern under which ds_read_b64_tr_b16 (4 rows x 16 columns per 16
// lanes) is conflict-free. Every stage is its own
// __shared__ array and the loop is unrolled by four, so the compiler can tell which buffer a
// read touches (an LDS read is otherwise held behind every outstanding LDS DMA); the waits are
// explicit: one vmcnt + lgkmcnt(0) and one s_barrier per k-tile.
//
// NF4 B. A thread decodes 32 values (half of a 64-value block) per k-tile (NT: one W row of the
// tile; NN: a quarter of one W row). Their codes (16 bytes) and the block's fp32 scale arrive by
// DMA too, five k-tiles ahead, into small LDS stages of their own; the scale is formed once per
// weight by nf4_block_scales_kernel (the double-quant chain code2[q] * absmax2 + offset, as the
// standalone dequant forms it), since the weights are frozen. With every operand arriving
// through LDS, no loaded register is live across the loop's back edge, where the compiler
// would otherwise drain the memory queue. The half-block of k-tile t + 2 is decoded while the
// MFMAs of k-tile t run, into its B stage. Decode: the block's 16 possible values
// fp16(fp32(level * scale)) (16 products, 8 v_cvt_pk_f16_f32: the standalone dequant's two
// roundings) are split into a low-byte and a high-byte plane of 16 bytes each; each value is
// then looked up by its code with v_perm_b32 (two 8-byte halves of a plane, merged by the code's
// bit 3): about 4 VALU instructions per value and no LDS lookup table. The result equals
// dequant-then-GEMM bit for bit in the B operand.
//
// Epilogues: fp16 store; + fp16 bias (qkv); fp32 residual out = res + f32(fp16(acc)) (down);
// SwiGLU m = fp16(silu(fp16 g) * fp16 u) (gate|up: each wavefront's first two 32-column blocks
// are gate rows, the last two the up rows of the same output columns); fp32 partial sums for
// split-K ([splits, M, N], summed in a fixed order by splitk_reduce_kernel). All but the
// partials stage the fp16 product through LDS from transposed accumulators (four consecutive
// columns per lane) and leave as whole 16-byte row pieces (the residual form: 32-byte fp32
// pieces, the residual's loaded in batches ahead of the stores).
//
// Work order: workgroup ids are dealt to the 8 XCDs in turn; tile_order gives each XCD a
// contiguous range of tiles (the M tiles of a few N tiles), so an XCD's L2 holds the B tiles it
// reads and the A tiles are shared through the MALL. fp16 B in one slice: when at most 64 tiles
// are left past the last full round of the 256 CUs, the same launch runs them as K slices
// (tail_plan; fp32 partials in the caller's workspace, tail_reduce_kernel sums them in slice
// order with the epilogue), so the last round is short instead of a whole tile long.
#include "nf4.h"

#include <hip/hip_ext.h>

#include <type_traits>

namespace qlora {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kBM = 256, kBN = 256, kBK = 32, kStages = 4, kThreads = 256;
constexpr int kTile = 256 * kBK;  // halves per operand stage (16 KB)

enum { kEpiStore = 0, kEpiBias = 1, kEpiResid = 2, kEpiSwiglu = 3, kEpiPartial = 4,
       kEpiSwigluKeep = 5, kEpiF32 = 6 };

// The SwiGLU forms: 3 writes m = fp16(silu(g) u) only, 5 also the fp16 [g | u] product (a
// recomputing layer keeps it for its backward instead of multiplying again).
constexpr bool swiglu_epi(int epi) { return epi == kEpiSwiglu || epi == kEpiSwigluKeep; }
enum { kBHalf = 0, kBNF4 = 1 };

// Epilogues that leave through LDS from transposed accumulators (every one but the fp32 forms:
// the split-K partials and kEpiF32): the fp16 product staged, then whole 16-byte row pieces (the
// residual form reads and writes fp32 row pieces of the same columns).
constexpr bool staged_epi(int epi) { return epi != kEpiPartial && epi != kEpiF32; }

// kEpiF32: out fp32 = alpha acc + (resid ? (row_scale ? row_scale[m] : 1) resid[m, n] : 0),
// unrounded (the accumulations of the LM head over vocabulary pieces). The K-sliced last round
// is not used with it (its reduce applies the fp16 epilogues).
constexpr bool tail_epi(int epi) { return epi != kEpiF32; }

struct GemmArgs {
  const uint16_t* a;     // A [M, Kr] fp16 (transposed-A mode: stored [Kr, M], lda >= M)
  int64_t lda;
  const uint16_t* b;     // fp16 B: NT [N rows, Kr], NN [Kr rows, N]
  int64_t ldb;
  // NF4 B: W [rows, Kw] (NT: rows = N, Kw = Kr; NN: rows = Kr, Kw = N), 64-value blocks
  const uint8_t* w_packed;  // codes, two per byte (element 2j in the high nibble of byte j)
  const float* w_scales;    // fp32 scale of each block
  const float* w_code;      // the 16 levels, or null for the NF4 table
  int w_tiled;              // NT: codes and scales in the tile-major order (qlora_nf4_gemm)
  int64_t Kw;
  void* c;               // fp16 [M, ldc]; fp32 for kEpiResid; fp32 [splits, M, N] partials
  int64_t ldc;
  const uint16_t* bias;  // fp16 [N] (kEpiBias)
  const float* resid;    // fp32 [M, ldr] (kEpiResid)
  int64_t ldr;
  int64_t M, N, Kr;      // output rows, output columns, reduction length
  int64_t I;             // SwiGLU: first W row of the up projection
  int kt_per_split;      // k-tiles per z-slice
  int m_tiles;
  int tiles;             // tiles of one K slice (m_tiles x the N tiles)
  // fp16 B, one slice: the last round's few tiles split along K (0: none). Workgroups
  // main_tiles .. main_tiles + tail tiles x tail_splits - 1 each form one K slice of one of the
  // last tiles (kt_per_tail k-tiles) into tail_ws ([tile][slice][256][256] fp32), summed in
  // slice order by tail_reduce_kernel with the epilogue.
  int main_tiles, tail_splits, kt_per_tail;
  float* tail_ws;
  int bm, bn;            // output tile (fp16 B: 256 x 256 or 128 x 128)
  uint16_t* gu;          // kEpiSwigluKeep: fp16 [M, 2 I] product [g | u] (ld ldgu)
  int64_t ldgu;
  float alpha;              // kEpiF32: scale of the product
  const float* row_scale;   // kEpiF32: fp32 [M] scale of each resid row, or null (1)
};

// ---- swizzled LDS offsets (in halves) ---------------------------------------------------------
__device__ __forceinline__ int kmaj_off(int row, int chunk) {  // [rows][32]
  return row * 32 + ((chunk ^ ((row >> 2) & 3)) << 3);
}
__device__ __forceinline__ int nmaj_off(int row, int chunk) {  // [32][256]
  return row * 256 + ((chunk ^ ((row & 3) << 2)) << 3);
}

// Workgroup b of `total` -> tile index: XCD x (= b % 8) takes the contiguous range
// [x total/8, (x+1) total/8) of tiles.
__device__ __forceinline__ int tile_order(int b, int total) {
  const int full = total / 8 * 8;
  return b < full ? (b % 8) * (full / 8) + b / 8 : b;
}

// The workgroup's (M tile, N tile, K slice), in scalar registers: the values are the same for
// every lane, and held in VGPRs across the main loop they cost registers the loop needs. The
// grid is one-dimensional, the K slices included (slice-major, then N tile, then M tile), so
// the XCD order above gives each XCD a run of tiles of one K slice: its L2 then holds the few
// A and B blocks of that K range which its workgroups share.
__device__ __forceinline__ void tile_of(int m_tiles, int tiles, int total, int64_t& tile_m,
                                        int64_t& tile_n, int& slice) {
  int t = tile_order(blockIdx.x, total);  // the grid is below 2^31 (host check)
  slice = __builtin_amdgcn_readfirstlane(t / tiles);
  t -= slice * tiles;
  tile_m = __builtin_amdgcn_readfirstlane(t % m_tiles);
  tile_n = __builtin_amdgcn_readfirstlane(t / m_tiles);
}

// ---- global -> LDS (DMA) ----------------------------------------------------------------------
// Lane byte offsets of a tile's DMA relative to a wave-uniform base (the tile's first element),
// computed once: the loads then take the scalar-base + 32-bit vector-offset form and advance by
// moving the base.
//
// K-contiguous tile (256 rows x 32 halves): wavefront w loads rows 64w .. 64w+63, sixteen rows
// per instruction.
struct DmaK {
  uint32_t off[4];
  // row_of(r): the row (relative to the base) that tile row r holds
  template <typename RowOf>
  __device__ __forceinline__ void init(int64_t ld, RowOf row_of, int wave, int lane) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 64 * wave + 16 * j + (lane >> 2);
      const int c = (lane & 3) ^ ((r >> 2) & 3);
      off[j] = (uint32_t)((row_of(r) * ld + 8 * c) * 2);
    }
  }
  // base: the tile's element (row0, k0)
  __device__ __forceinline__ void issue(const uint16_t* base, uint16_t* dst, int wave) const {
    const char* b = reinterpret_cast<const char*>(base);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_global_load_lds(b + off[j], (lds_void_t*)(dst + (64 * wave + 16 * j) * 32),
                                       16, 0, 0);
  }
};

// N-contiguous tile (32 rows x 256 halves): wavefront w loads rows 8w .. 8w+7, two rows per
// instruction.
struct DmaN {
  uint32_t off[4];
  __device__ __forceinline__ void init(int64_t ld, int wave, int lane) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 8 * wave + 2 * j + (lane >> 5);
      const int c = (lane & 31) ^ ((r & 3) << 2);
      off[j] = (uint32_t)((r * ld + 8 * c) * 2);
    }
  }
  __device__ __forceinline__ void issue(const uint16_t* base, uint16_t* dst, int wave) const {
    const char* b = reinterpret_cast<const char*>(base);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_global_load_lds(b + off[j], (lds_void_t*)(dst + (8 * wave + 2 * j) * 256),
                                       16, 0, 0);
  }
};

// ---- NF4 block decode -------------------------------------------------------------------------
// NF4 B by DMA: the codes of a thread's half-block of a k-tile (16 bytes, 32 values) and its
// block's fp32 scale go into slot `tid` of a codes stage and a scales stage (wavefront w's lanes
// fill slots 64 w .. 64 w + 63, the same wavefront's threads read them). `code_off`: the
// half-block's first byte in the codes, `scale_idx`: its block's scale.
__device__ __forceinline__ void nf4_issue(const GemmArgs& g, int64_t code_off, int64_t scale_idx,
                                          uint8_t* codes, float* scales, int wave) {
  __builtin_amdgcn_global_load_lds(g.w_packed + code_off, (lds_void_t*)(codes + 1024 * wave), 16,
                                   0, 0);
  __builtin_amdgcn_global_load_lds(g.w_scales + scale_idx, (lds_void_t*)(scales + 64 * wave), 4,
                                   0, 0);
}

// The block's 16 values fp16(fp32(level[c] * scale)) as byte planes: lo[p] holds the low bytes
// of values 4p .. 4p+3, hi[p] their high bytes.
struct NF4Planes {
  uint32_t lo[4], hi[4];
};

__device__ __forceinline__ NF4Planes nf4_planes(float scale, const float* lv) {
  uint32_t d[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // the fp32 product, then one RNE rounding to fp16: the library is built without the
    // v_fma_mix instructions, which would round the product to fp16 once (and an empty asm
    // pinning the product would also keep the scheduler from spreading the decode over the
    // MFMAs)
    const float p0 = lv[2 * i] * scale, p1 = lv[2 * i + 1] * scale;
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    d[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){p0, p1}, h2));
  }
  NF4Planes t;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    t.lo[p] = __builtin_amdgcn_perm(d[2 * p + 1], d[2 * p], 0x06040200u);
    t.hi[p] = __builtin_amdgcn_perm(d[2 * p + 1], d[2 * p], 0x07050301u);
  }
  return t;
}

// Four values from four codes (one per byte of `n`, 0..15): two packed fp16 pairs.
__device__ __forceinline__ uint2 nf4_lookup4(const NF4Planes& t, uint32_t n) {
  const uint32_t s = n & 0x07070707u;
  const uint32_t sel = ((n >> 1) & 0x04040404u) | 0x03020100u;  // byte i: i, or 4 + i if >= 8
  const uint32_t lo = __builtin_amdgcn_perm(__builtin_amdgcn_perm(t.lo[3], t.lo[2], s),
                                            __builtin_amdgcn_perm(t.lo[1], t.lo[0], s), sel);
  const uint32_t hi = __builtin_amdgcn_perm(__builtin_amdgcn_perm(t.hi[3], t.hi[2], s),
                                            __builtin_amdgcn_perm(t.hi[1], t.hi[0], s), sel);
  return make_uint2(__builtin_amdgcn_perm(hi, lo, 0x05010400u),
                    __builtin_amdgcn_perm(hi, lo, 0x07030602u));
}

// Eight values (16 bytes, memory order) from one 32-bit word of codes: element 2k is the high
// nibble of byte k.
__device__ __forceinline__ uint4 nf4_decode8(const NF4Planes& t, uint32_t wd) {
  const uint32_t lo4 = wd & 0x0F0F0F0Fu, hi4 = (wd >> 4) & 0x0F0F0F0Fu;
  const uint2 a = nf4_lookup4(t, __builtin_amdgcn_perm(hi4, lo4, 0x01050004u));
  const uint2 b = nf4_lookup4(t, __builtin_amdgcn_perm(hi4, lo4, 0x03070206u));
  return make_uint4(a.x, a.y, b.x, b.y);
}

// W row of LDS B row `n` (NT) of a tile BN rows wide. SwiGLU: within each wavefront's BN/2 rows
// the first BN/4 are gate rows and the last BN/4 the up rows of the same BN/4 output columns.
template <int EPI, int BN = kBN>
__device__ __forceinline__ int64_t nt_wrow(const GemmArgs& g, int64_t tile_n, int n) {
  if constexpr (swiglu_epi(EPI)) {
    constexpr int WC = BN / 2, HC = BN / 4;
    const int64_t j = tile_n * (BN / 2) + (n / WC) * HC + (n % HC);
    return (n % WC) >= HC ? g.I + j : j;
  } else {
    return tile_n * BN + n;
  }
}

// ---- the kernel -------------------------------------------------------------------------------
// The operand fragments of one 16-wide k-step: 4 A blocks (rows) and 4 B blocks (columns) of
// 32, 8 halves a lane.
template <int FM, int FN>
struct FragsT {
  half8_t a[FM], b[FN];
};
typedef FragsT<4, 4> Frags;

template <bool NN>
__device__ __forceinline__ void read_frags(Frags& f, const uint16_t* sa, const uint16_t* sb,
                                           int s, int wm, int wn, int lane) {
  const int frow = lane & 31, fhalf = lane >> 5;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    f.a[i] = *reinterpret_cast<const half8_t*>(
        sa + kmaj_off(wm * 128 + 32 * i + frow, 2 * s + fhalf));
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (!NN) {
      f.b[j] = *reinterpret_cast<const half8_t*>(
          sb + kmaj_off(wn * 128 + 32 * j + frow, 2 * s + fhalf));
    } else {
      // ds_read_b64_tr_b16: lane p of a 16-lane group reads row k + p / 4, columns
      // c0 + 4 (p % 4) .. + 3; lane i of the group receives column c0 + i of rows k .. k+3
      const int p = lane & 15;
      const int col = wn * 128 + 32 * j + 16 * ((lane >> 4) & 1) + 4 * (p & 3);
      const int k = 16 * s + 8 * fhalf + (p >> 2);
      const int o0 = nmaj_off(k, col >> 3) + (col & 7);
      const int o1 = nmaj_off(k + 4, col >> 3) + (col & 7);
      const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(sb + o0));
      const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(sb + o1));
      f.b[j] = __builtin_bit_cast(half8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  }
}

// T: the accumulators hold the transposed blocks (B fragments as the MFMA's first operand), so
// register r of lane l in block (i, j) is row 32 i + l % 32, column 32 j + 8 (r / 4) + 4 (l / 32)
// + r % 4: four consecutive output columns per lane, stored as one 8-byte LDS write. Otherwise
// register r is row 32 i + 8 (r / 4) + 4 (l / 32) + r % 4, column 32 j + l % 32.
template <bool T, int FM, int FN>
__device__ __forceinline__ void mfma_step(f32x16 (&acc)[FM][FN], const FragsT<FM, FN>& f) {
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
      acc[i][j] = T ? __builtin_amdgcn_mfma_f32_32x32x16_f16(f.b[j], f.a[i], acc[i][j], 0, 0, 0)
                    : __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
}

// Scheduling of one k-step: the reads of the next k-step's fragments between this k-step's 16
// MFMAs (one read per MFMA), `VMEM` global loads (the prefetch DMA) one per MFMA from the
// first, and `VALU` VALU instructions (the NF4 decode, the DMA addresses) after each MFMA.
// Spreading the DMA over the MFMAs keeps the four wavefronts, which leave the k-tile's barrier
// together, from queueing all their loads at the texture unit at once (measured: 6 % of the
// gate|up GEMM's time).
// FM x FN MFMA blocks a k-step: MF = FM FN MFMAs, FM + FN fragment reads (NN: B's take two
// transposed reads each); reads and loads dealt over the MFMAs as evenly as they go.
template <bool NN, int VALU, int VMEM, int FM = 4, int FN = 4, bool TA = false>
__device__ __forceinline__ void sched_step() {
  constexpr int MF = FM * FN, reads = (TA ? 2 : 1) * FM + (NN ? 2 : 1) * FN;
#pragma unroll
  for (int i = 0; i < MF; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    constexpr int rq = reads / MF, rr = reads % MF;
    if (i < rr) __builtin_amdgcn_sched_group_barrier(0x100, rq + 1, 0);  // DS read
    else if (rq > 0) __builtin_amdgcn_sched_group_barrier(0x100, rq, 0);
    constexpr int vq = VMEM / MF, vr = VMEM % MF;
    if (i < vr) __builtin_amdgcn_sched_group_barrier(0x020, vq + 1, 0);  // VMEM read
    else if (vq > 0) __builtin_amdgcn_sched_group_barrier(0x020, vq, 0);
    if constexpr (VALU > 0) __builtin_amdgcn_sched_group_barrier(0x002, VALU, 0);  // VALU
  }
}

// Half `part` (0, 1) of the decode of one half-block (32 values, codes `v`) with scale `sc` into
// the B stage: part 0 forms the byte planes (unless the planes of the block's other half are
// still in `t`: FRESH false) and words 0-1, part 1 words 2-3. NT: LDS row `row`, chunks 0-3;
// NN: row `row`, chunks chunk0 .. chunk0+3.
template <bool NN, bool FRESH = true>
__device__ __forceinline__ void nf4_decode_part(const uint4& v, float sc, NF4Planes& t,
                                                uint16_t* sb, int row, int chunk0,
                                                const float* lv, int part) {
  const uint32_t wds[4] = {v.x, v.y, v.z, v.w};
  if (part == 0 && FRESH) t = nf4_planes(sc, lv);
#pragma unroll
  for (int c = 2 * part; c < 2 * part + 2; ++c) {
    const int off = NN ? nmaj_off(row, chunk0 + c) : kmaj_off(row, c);
    *reinterpret_cast<uint4*>(sb + off) = nf4_decode8(t, wds[c]);
  }
}

// s_waitcnt with vmcnt(VM) and lgkmcnt(0), then s_barrier: this thread's LDS stores and all
// but its VM most recent vector-memory loads are done, and so are every other thread's.
template <int VM>
__device__ __forceinline__ void sync_tile() {
  static_assert(VM >= 0 && VM < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4));
  __builtin_amdgcn_s_barrier();
}

// Epilogue 5 of a BM x BN tile (registers and LDS areas as store_tile): the product [g | u]
// first, staged as a plain store would and written to gate column n and up column I + n of g.gu;
// while those stores issue (they stall when every CU of a round writes at once), the SwiGLU of
// the same accumulators is formed, one group of four values a lane per 16-byte store, and kept
// packed in registers; then m is staged in the same LDS area and stored. The values are those of
// epilogue 3 and of a plain store of the product, bit for bit.
template <int BM, int BN>
__device__ __forceinline__ void store_swiglu_keep(const GemmArgs& g,
                                                  f32x16 (&acc)[BM / 64][BN / 64], uint16_t* lo,
                                                  uint16_t* hi, int64_t m0, int64_t tile_n,
                                                  int lane, int wave) {
  constexpr int FM = BM / 64, FN = BN / 64, WR = BM / 2, WC = BN / 2, kHalf = WR / 2;
  constexpr int kCh2 = WC / 8, kRows2 = 64 / kCh2, kIt = WR / kRows2;
  constexpr int kGroups = FM * 4 * (FN / 2), kPer = kGroups / kIt;
  static_assert(kGroups % kIt == 0, "whole groups of SwiGLU values per store");
  const int wm = wave >> 1, wn = wave & 1, col_in = lane & 31, c4 = 4 * (lane >> 5);
  auto stage2 = [&](int row, int chunk) {
    return (row % kHalf) * WC + ((chunk ^ (row & (kCh2 - 1))) << 3);
  };
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int row = i * 32 + col_in;
    uint16_t* base = i < FM / 2 ? lo : hi;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = j * 32 + 8 * q + c4;
        *reinterpret_cast<uint2*>(base + stage2(row, col >> 3) + c4) =
            make_uint2(pack2h(acc[i][j][4 * q], acc[i][j][4 * q + 1]),
                       pack2h(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]));
      }
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wavefront's own LDS stores
  const int64_t g_base = tile_n * (BN / 2) + wn * (WC / 2);
  auto gu_piece = [&](int k) {
    const int row = k * kRows2 + lane / kCh2, chunk = lane % kCh2;
    return *reinterpret_cast<const uint4*>((row < kHalf ? lo : hi) + stage2(row, chunk));
  };
  uint2 mv[kGroups];  // group (i, q, j): four m values of row 32 i + l % 32, packed
  uint4 v = gu_piece(0);
#pragma unroll
  for (int k = 0; k < kIt; ++k) {
    uint4 vn;
    if (k + 1 < kIt) vn = gu_piece(k + 1);
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int gi = k * kPer + u, i = gi / (4 * (FN / 2)), q = (gi / (FN / 2)) % 4,
                j = gi % (FN / 2);
      float m[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float gt = h2f(f2h(acc[i][j][4 * q + e]));
        const float up = h2f(f2h(acc[i][j + FN / 2][4 * q + e]));
        m[e] = gt * sigmoid_fast(gt) * up;  // as glu_fwd_kernel
      }
      mv[gi] = make_uint2(pack2h(m[0], m[1]), pack2h(m[2], m[3]));
      // formed here, between this store and the next (else the compiler sinks the arithmetic
      // below the loop, where nothing overlaps it)
      asm volatile("" : "+v"(mv[gi].x), "+v"(mv[gi].y));
    }
    const int row = k * kRows2 + lane / kCh2, col = (lane % kCh2) * 8;
    const int64_t mm = m0 + wm * WR + row;
    const int64_t n = g_base + (col % (WC / 2)) + (col >= WC / 2 ? g.I : 0);
    if (mm < g.M) *reinterpret_cast<uint4*>(g.gu + mm * g.ldgu + n) = v;
    v = vn;
    __builtin_amdgcn_sched_barrier(0);
  }
  // m, fp16 [rows][WC / 2] per wavefront, through the same LDS area (its reads are complete:
  // their values have been stored)
  constexpr int kCols = WC / 2, kChunks = kCols / 8, kRowsPer = 64 / kChunks;
  auto stage_off = [&](int row, int chunk) {
    return (row % kHalf) * kCols + ((chunk ^ (row & (kChunks - 1))) << 3);
  };
  __builtin_amdgcn_s_waitcnt(0xC07F);
#pragma unroll
  for (int gi = 0; gi < kGroups; ++gi) {
    const int i = gi / (4 * (FN / 2)), q = (gi / (FN / 2)) % 4, j = gi % (FN / 2);
    const int row = i * 32 + col_in, col = j * 32 + 8 * q + c4;
    *reinterpret_cast<uint2*>((i < FM / 2 ? lo : hi) + stage_off(row, col >> 3) + c4) = mv[gi];
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);
  const int64_t n_base = tile_n * (BN / 2) + wn * (WC / 2);
#pragma unroll
  for (int k = 0; k < WR / kRowsPer; ++k) {
    const int row = k * kRowsPer + lane / kChunks, chunk = lane % kChunks;
    const uint4 w = *reinterpret_cast<const uint4*>((row < kHalf ? lo : hi) +
                                                     stage_off(row, chunk));
    const int64_t mm = m0 + wm * WR + row, n = n_base + chunk * 8;
    if (mm < g.M && n < g.N)
      *reinterpret_cast<uint4*>(static_cast<uint16_t*>(g.c) + mm * g.ldc + n) = w;
  }
}

// The epilogue of a BM x BN tile from the accumulators of mfma_step (4 wavefronts, each on a
// WR x WC block, WR = BM / 2, WC = BN / 2; register layouts as mfma_step): fp16 outputs are
// staged through LDS (`lo`: the wavefront's rows 0 .. WR/2 - 1, `hi`: the rest, [WR/2][columns]
// each, free for this wavefront's use) and leave as whole 16-byte row pieces (the fp32 residual
// output as 32-byte pieces); split-K partials are stored from the registers.
template <int EPI, int BM = kBM, int BN = kBN>
__device__ __forceinline__ void store_tile(const GemmArgs& g, f32x16 (&acc)[BM / 64][BN / 64],
                                           uint16_t* lo, uint16_t* hi, int64_t m0,
                                           int64_t tile_n, int lane, int wave, int slice = 0) {
  constexpr int FM = BM / 64, FN = BN / 64, WR = BM / 2, WC = BN / 2;
  constexpr bool kT = staged_epi(EPI);
  const int wm = wave >> 1, wn = wave & 1;
  const int col_in = lane & 31;
  if constexpr (EPI == kEpiSwigluKeep) {
    store_swiglu_keep<BM, BN>(g, acc, lo, hi, m0, tile_n, lane, wave);
  } else if constexpr (kT) {
    // each wavefront writes its block to LDS as fp16 (8-byte LDS stores of four columns,
    // 16-byte chunks XOR-swizzled by row so the 32 rows of a store spread over the banks), then
    // stores whole rows to memory with 16-byte stores
    constexpr int kCols = swiglu_epi(EPI) ? WC / 2 : WC;  // output columns of a wavefront
    constexpr int kChunks = kCols / 8;
    constexpr int kHalf = WR / 2;  // rows staged in `lo`
    auto stage_off = [&](int row, int chunk) {
      return (row % kHalf) * kCols + ((chunk ^ (row & (kChunks - 1))) << 3);
    };
    const int c4 = 4 * (lane >> 5);  // first of the lane's four columns in an 8-column group
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int row = i * 32 + col_in;
      uint16_t* base = i < FM / 2 ? lo : hi;
#pragma unroll
      for (int q = 0; q < 4; ++q) {  // 8-column group q of each 32-column block
        if constexpr (swiglu_epi(EPI)) {
#pragma unroll
          for (int j = 0; j < FN / 2; ++j) {
            const int col = j * 32 + 8 * q + c4;
            float m[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float gt = h2f(f2h(acc[i][j][4 * q + e]));
              const float up = h2f(f2h(acc[i][j + FN / 2][4 * q + e]));
              m[e] = gt * sigmoid_fast(gt) * up;  // as glu_fwd_kernel
            }
            *reinterpret_cast<uint2*>(base + stage_off(row, col >> 3) + c4) =
                make_uint2(pack2h(m[0], m[1]), pack2h(m[2], m[3]));
          }
        } else {
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            const int col = j * 32 + 8 * q + c4;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              v[e] = acc[i][j][4 * q + e];
              if constexpr (EPI == kEpiBias) {
                const int64_t n = tile_n * BN + wn * WC + col + e;
                v[e] += h2f_bits(g.bias[n < g.N ? n : g.N - 1]);
              }
            }
            *reinterpret_cast<uint2*>(base + stage_off(row, col >> 3) + c4) =
                make_uint2(pack2h(v[0], v[1]), pack2h(v[2], v[3]));
          }
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wavefront's own LDS stores
    constexpr int kRowsPer = 64 / kChunks;  // rows per 16-byte store instruction
    const int64_t n_base = swiglu_epi(EPI) ? tile_n * (BN / 2) + wn * (WC / 2)
                                           : tile_n * BN + wn * WC;
    if constexpr (EPI == kEpiResid) {
      // out = resid + f32(fp16 product), eight columns a lane: the residual row pieces of a
      // batch of rows are loaded before any output is stored (out may be resid itself; each
      // element is read before it is written), so their latencies overlap
      constexpr int kIters = WR / kRowsPer, kBatch = kIters < 4 ? kIters : 4;
#pragma unroll
      for (int k0 = 0; k0 < kIters; k0 += kBatch) {
        uint4 v[kBatch];
        float4 r0[kBatch], r1[kBatch];
        int64_t mo[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
          const int row = (k0 + b) * kRowsPer + lane / kChunks, chunk = lane % kChunks;
          v[b] = *reinterpret_cast<const uint4*>((row < kHalf ? lo : hi) + stage_off(row, chunk));
          const int64_t m = m0 + wm * WR + row, n = n_base + chunk * 8;
          mo[b] = (m < g.M && n < g.N) ? m : -1;
          if (mo[b] >= 0) {
            const float4* rp = reinterpret_cast<const float4*>(g.resid + m * g.ldr + n);
            r0[b] = rp[0];
            r1[b] = rp[1];
          }
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
          if (mo[b] < 0) continue;
          const int64_t n = n_base + (lane % kChunks) * 8;
          float4* op = reinterpret_cast<float4*>(static_cast<float*>(g.c) + mo[b] * g.ldc + n);
          op[0] = make_float4(r0[b].x + lo_h(v[b].x), r0[b].y + hi_h(v[b].x),
                              r0[b].z + lo_h(v[b].y), r0[b].w + hi_h(v[b].y));
          op[1] = make_float4(r1[b].x + lo_h(v[b].z), r1[b].y + hi_h(v[b].z),
                              r1[b].z + lo_h(v[b].w), r1[b].w + hi_h(v[b].w));
        }
      }
      return;
    }
#pragma unroll
    for (int k = 0; k < WR / kRowsPer; ++k) {
      const int row = k * kRowsPer + lane / kChunks, chunk = lane % kChunks;
      const uint4 v = *reinterpret_cast<const uint4*>((row < kHalf ? lo : hi) +
                                                       stage_off(row, chunk));
      const int64_t m = m0 + wm * WR + row, n = n_base + chunk * 8;
      if (m < g.M && n < g.N)
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(g.c) + m * g.ldc + n) = v;
    }
  } else if constexpr (EPI == kEpiF32) {
    // fp32 out = alpha acc (+ row-scaled resid), from the registers: each store instruction
    // writes 32 consecutive columns of two rows; each element's resid is read by the thread
    // that writes it (out may be resid itself)
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + wm * WR + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (m >= g.M) continue;
        const float rs = g.resid == nullptr ? 0.0f : g.row_scale == nullptr ? 1.0f
                                                                              : g.row_scale[m];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int64_t n = tile_n * BN + wn * WC + j * 32 + col_in;
          if (n >= g.N) continue;
          float v = g.alpha * acc[i][j][r];
          if (g.resid != nullptr) v += rs * g.resid[m * g.ldr + n];
          static_cast<float*>(g.c)[m * g.ldc + n] = v;
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + wm * WR + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (m >= g.M) continue;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int64_t n = tile_n * BN + wn * WC + j * 32 + col_in;
          if (n >= g.N) continue;
          static_cast<float*>(g.c)[((int64_t)slice * g.M + m) * g.N + n] = acc[i][j][r];
        }
      }
    }
  }
}

template <bool NN, int EPI>
__global__ __launch_bounds__(kThreads, 1) void nf4_gemm_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint16_t sA0[kTile];
  __shared__ __attribute__((aligned(1024))) uint16_t sA1[kTile];
  __shared__ __attribute__((aligned(1024))) uint16_t sA2[kTile];
  __shared__ __attribute__((aligned(1024))) uint16_t sA3[kTile];
  __shared__ __attribute__((aligned(1024))) uint16_t sB0[kTile];
  __shared__ __attribute__((aligned(1024))) uint16_t sB1[kTile];
  __shared__ __attribute__((aligned(1024))) uint16_t sB2[kTile];
  __shared__ __attribute__((aligned(1024))) uint16_t sB3[kTile];
  // NF4 codes and scales, stage u % 4 for k-tile u (unused with an fp16 B)
  __shared__ __attribute__((aligned(1024))) uint8_t sC0[kThreads * 16];
  __shared__ __attribute__((aligned(1024))) uint8_t sC1[kThreads * 16];
  __shared__ __attribute__((aligned(1024))) uint8_t sC2[kThreads * 16];
  __shared__ __attribute__((aligned(1024))) uint8_t sC3[kThreads * 16];
  __shared__ __attribute__((aligned(1024))) float sS0[kThreads];
  __shared__ __attribute__((aligned(1024))) float sS1[kThreads];
  __shared__ __attribute__((aligned(1024))) float sS2[kThreads];
  __shared__ __attribute__((aligned(1024))) float sS3[kThreads];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  int64_t tile_m, tile_n;
  int slice;
  tile_of(g.m_tiles, g.tiles, gridDim.x, tile_m, tile_n, slice);
  const int64_t m0 = tile_m * kBM;
  const int64_t kt0 = (int64_t)slice * g.kt_per_split;
  int64_t kt1 = kt0 + g.kt_per_split;
  if (kt1 > g.Kr / kBK) kt1 = g.Kr / kBK;  // k-tile counts are multiples of 4 (host check)
  const int64_t kt_last = kt1 - 1;

  DmaK dma_a;
  const int64_t a_rows = g.M - m0;  // rows past M re-read the last row
  dma_a.init(g.lda, [&](int r) -> int64_t { return r < a_rows ? r : a_rows - 1; }, wave, lane);
  const uint16_t* a_base = g.a + m0 * g.lda;  // + k0 per k-tile
  // NF4: levels in registers; this thread's half-block of k-tile kt (decoded into row b_row
  // from chunk b_chunk0; NT: row tid; NN: row tid / 8, chunks 4 (tid % 8) ..) has its codes at
  // byte c_base + kt c_step and its scale at s_base + (kt >> s_shift) s_step. Row-major codes
  // (bitsandbytes' order): NT one W row, 16 bytes a k-tile, a scale per two k-tiles; NN a
  // quarter of a W row, 32 rows down a k-tile. Tile-major codes (NT): each k-tile's 256 rows
  // of a tile are 4 KB in a row and their scales 1 KB, so one DMA instruction reads 1 KB in a
  // row instead of 16 bytes from each of 64 W rows.
  float lv[16];
  int64_t c_base = 0, c_step = 0, s_base = 0, s_step = 0;
  int s_shift = 0;
  int b_row = 0, b_chunk0 = 0;
  {
#pragma unroll
    for (int i = 0; i < 16; ++i) lv[i] = g.w_code ? g.w_code[i] : kNF4Levels[i];
    if constexpr (!NN) {
      b_row = tid;
      s_shift = 1;
      if (g.w_tiled) {
        const int64_t kt_all = g.Kr / kBK;
        c_base = (tile_n * kt_all * kThreads + tid) * 16;
        c_step = kThreads * 16;
        s_base = tile_n * (kt_all / 2) * kThreads + tid;
        s_step = kThreads;
      } else {
        const int64_t e_base = nt_wrow<EPI>(g, tile_n, tid) * g.Kw;
        c_base = e_base >> 1;
        c_step = kBK / 2;
        s_base = e_base >> 6;
        s_step = 1;
      }
    } else {
      b_row = tid >> 3;
      b_chunk0 = 4 * (tid & 7);
      const int64_t e_base = (int64_t)b_row * g.Kw + tile_n * kBN + 32 * (tid & 7);
      c_base = e_base >> 1;
      c_step = (int64_t)kBK * g.Kw / 2;
      s_base = e_base >> 6;
      s_step = (int64_t)kBK * g.Kw / 64;
    }
  }
  // vector-memory instructions one k-tile issues (the A DMA, codes and scales)
  constexpr int kVmPerTile = 4 + 2;

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  auto clamp_kt = [&](int64_t kt) { return kt < kt1 ? kt : kt_last; };
  auto issue_tile = [&](int64_t kt, uint16_t* sa, uint16_t* sb) {
    kt = clamp_kt(kt);
    dma_a.issue(a_base + kt * kBK, sa, wave);
  };

  // prologue: k-tiles kt0 .. kt0+2 into stages 0-2. NF4: the codes and scales of kt0 .. kt0+3
  // into their stages; kt0 and kt0+1 decoded into B stages 0 and 1, kt0+2's read into
  // registers (decoded during kt0), then kt0+4's DMA into stage 0.
  issue_tile(kt0, sA0, sB0);
  issue_tile(kt0 + 1, sA1, sB1);
  issue_tile(kt0 + 2, sA2, sB2);
  NF4Planes planes;
  uint4 cx{}, cy{};  // codes of the half-block decoded at the even / odd k-tiles of a trip
  float sx = 0.0f, sy = 0.0f;
  auto nf4_at = [&](int64_t kt, uint8_t* codes, float* scales) {
    kt = clamp_kt(kt);
    nf4_issue(g, c_base + kt * c_step, s_base + (kt >> s_shift) * s_step, codes, scales, wave);
  };
  {
    nf4_at(kt0, sC0, sS0);
    nf4_at(kt0 + 1, sC1, sS1);
    nf4_at(kt0 + 2, sC2, sS2);
    nf4_at(kt0 + 3, sC3, sS3);
    __builtin_amdgcn_s_waitcnt(0);  // (each thread reads the slots its own wavefront filled)
    const uint4 c0 = *reinterpret_cast<const uint4*>(sC0 + 16 * tid);
    const uint4 c1 = *reinterpret_cast<const uint4*>(sC1 + 16 * tid);
    const float s0 = sS0[tid], s1 = sS1[tid];
    cx = *reinterpret_cast<const uint4*>(sC2 + 16 * tid);
    sx = sS2[tid];
    nf4_decode_part<NN>(c0, s0, planes, sB0, b_row, b_chunk0, lv, 0);
    nf4_decode_part<NN>(c0, s0, planes, sB0, b_row, b_chunk0, lv, 1);
    nf4_decode_part<NN>(c1, s1, planes, sB1, b_row, b_chunk0, lv, 0);
    nf4_decode_part<NN>(c1, s1, planes, sB1, b_row, b_chunk0, lv, 1);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): stage 0 read before its next DMA
    nf4_at(kt0 + 4, sC0, sS0);
  }
  sync_tile<0>();

  // Software pipeline over four LDS stages, unrolled by four so every buffer is static (k-tile
  // t on stage t % 4). After the barrier in the middle of k-tile t the DMA of t + 3 goes into
  // the stage k-tile t - 1 used. NF4: k-tile t decodes t + 2 into its B stage across both
  // k-steps (done by the barrier that ends t + 1) from codes read into registers during t - 1;
  // after its barrier it issues the DMA of t + 5's codes and scales (stage (t + 1) % 4, read
  // during t - 2) and reads t + 3's, which that barrier made complete: everything a k-tile
  // issues has landed by the barrier of the k-tile after next. Every memory operand reaches the
  // kernel through LDS, so the compiler's waits on loaded registers never drain the queue. Each
  // k-step's 16 MFMAs run while the next k-step's fragments are read; the second k-step reads
  // the first fragments of t + 1 after the barrier that makes t + 1 visible (the wait leaves
  // the loads of t + 2 in flight). Past the last k-tile the prefetches re-read it into stages
  // no longer read: a trip has no branch.
  constexpr int kValu = 5;
  // fp16 outputs leave through LDS from transposed accumulators (mfma_step)
  constexpr bool kT = staged_epi(EPI);
  Frags f0, f1;
  read_frags<NN>(f0, sA0, sB0, 0, wm, wn, lane);
  // NT: a 64-value block spans k-tiles 2j and 2j + 1 of one W row (the rows start on a block:
  // Kr % 128 == 0), so the odd k-tile's decode reuses the even one's byte planes (`fresh`
  // false); the k-tile decoded is t + 2, even for the first and third of a trip's four
  auto k_tile = [&](int64_t t, uint16_t* sa, uint16_t* sb, uint16_t* sa_next, uint16_t* sb_next,
                    uint16_t* sa_pre, uint16_t* sb_pre, uint16_t* sb_dec, uint8_t* c_load,
                    float* s_load, const uint8_t* c_read, const float* s_read,
                    const uint4& c_dec, const float& s_dec, uint4& c_next, float& s_next,
                    auto fresh) {
    __builtin_amdgcn_sched_barrier(0);
    read_frags<NN>(f1, sa, sb, 1, wm, wn, lane);
    nf4_decode_part<NN, NN || decltype(fresh)::value>(c_dec, s_dec, planes, sb_dec, b_row,
                                                      b_chunk0, lv, 0);
    mfma_step<kT>(acc, f0);
    sched_step<NN, kValu, 0>();
    __builtin_amdgcn_sched_barrier(0);
    sync_tile<kVmPerTile>();  // k-tile t + 1 landed; t + 2 may still be in flight
    // the DMA of t + 3 into the stage t - 1 used (every wavefront's reads of it ended before
    // the barrier), spread over this k-step's MFMAs
    issue_tile(t + 3, sa_pre, sb_pre);
    nf4_at(t + 5, c_load, s_load);
    read_frags<NN>(f0, sa_next, sb_next, 0, wm, wn, lane);
    nf4_decode_part<NN>(c_dec, s_dec, planes, sb_dec, b_row, b_chunk0, lv, 1);
    c_next = *reinterpret_cast<const uint4*>(c_read + 16 * tid);
    s_next = s_read[tid];
    mfma_step<kT>(acc, f1);
    sched_step<NN, kValu, kVmPerTile>();
    __builtin_amdgcn_sched_barrier(0);
  };
  for (int64_t t = kt0; t < kt1; t += 4) {
    const std::true_type even;
    const std::false_type odd;
    k_tile(t, sA0, sB0, sA1, sB1, sA3, sB3, sB2, sC1, sS1, sC3, sS3, cx, sx, cy, sy, even);
    k_tile(t + 1, sA1, sB1, sA2, sB2, sA0, sB0, sB3, sC2, sS2, sC0, sS0, cy, sy, cx, sx, odd);
    k_tile(t + 2, sA2, sB2, sA3, sB3, sA1, sB1, sB0, sC3, sS3, sC1, sS1, cx, sx, cy, sy, even);
    k_tile(t + 3, sA3, sB3, sA0, sB0, sA2, sB2, sB1, sC0, sS0, sC2, sS2, cy, sy, cx, sx, odd);
  }
  // the prefetches past the end: nothing left in flight; fp16 outputs go through the LDS
  // stages, free once every wavefront is done with them
  __builtin_amdgcn_s_waitcnt(0);
  if constexpr (kT) __builtin_amdgcn_s_barrier();
  store_tile<EPI>(g, acc, wave == 0 ? sA0 : wave == 1 ? sA2 : wave == 2 ? sB0 : sB2,
                  wave == 0 ? sA1 : wave == 1 ? sA3 : wave == 2 ? sB1 : sB3, m0, tile_n, lane,
                  wave, slice);
}


// ---- fp16 B: 64-wide k-tiles ------------------------------------------------------------------
// The vector L1 serves whole 128-byte lines at about twice the rate of 64-byte halves (measured
// on MI355X: ~56 against ~29 bytes per clock per CU for global_load_lds_dwordx4 from L2): with
// 64-wide k-tiles every K-contiguous row piece a DMA lane group fetches is a whole line. Two
// stages per operand; the loop runs one k-tile ahead, each k-tile's DMA instructions spread over
// three k-steps of the one before.
//
// Two tile shapes share the code: 256 x 256 (4 wavefronts of 128 x 128, one workgroup per CU,
// 128 KB of LDS) for the wide products, and 128 x 128 (4 wavefronts of 64 x 64, 64 KB of LDS, so
// two workgroups share a CU and cover each other's waits) for the narrow ones (N = 1536 - 2048
// at a few thousand tokens: 60 tiles of 256 x 256 for 256 CUs, 240 of 128 x 128). A 64 x 64
// wavefront block reads twice the LDS bytes per MFMA of a 128 x 128 one.
constexpr int kBK64 = 64;
constexpr int kTile64 = 256 * kBK64;  // halves per operand stage of a 256 x 256 tile (32 KB)

// [rows][64]: chunk c of row r in slot c ^ ((r >> 1) & 7). A 16-lane group of a fragment read
// takes 16 consecutive rows of one chunk: two rows per 256-byte bank cycle, eight slots.
__device__ __forceinline__ int kmaj64_off(int row, int chunk) {
  return row * 64 + ((chunk ^ ((row >> 1) & 7)) << 3);
}

// [64][BN] (N-contiguous): chunk c of row k in slot c ^ ((k & 3) << 2), the pattern under which
// ds_read_b64_tr_b16 (4 rows x 16 columns per 16 lanes) is conflict-free for either width.
template <int BN>
__device__ __forceinline__ int nmaj_off_w(int row, int chunk) {
  return row * BN + ((chunk ^ ((row & 3) << 2)) << 3);
}

// K-contiguous tile (ROWS rows x 64 halves): wavefront w loads rows w ROWS/4 .. (w+1) ROWS/4 - 1,
// eight whole 128-byte rows per instruction (ROWS / 32 instructions a wavefront).
template <int ROWS>
struct DmaKT {
  static constexpr int N = ROWS / 32;
  uint32_t off[N];
  template <typename RowOf>
  __device__ __forceinline__ void init(int64_t ld, RowOf row_of, int wave, int lane) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int r = (ROWS / 4) * wave + 8 * j + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      off[j] = (uint32_t)((row_of(r) * ld + 8 * c) * 2);
    }
  }
  __device__ __forceinline__ void issue(const uint16_t* base, uint16_t* dst, int wave,
                                        int j) const {
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const char*>(base) + off[j],
                                     (lds_void_t*)(dst + ((ROWS / 4) * wave + 8 * j) * 64), 16,
                                     0, 0);
  }
};

// N-contiguous tile (64 rows x BN halves, nmaj_off_w): wavefront w loads rows 16w .. 16w+15,
// 1 KB (2048 / BN rows) per instruction (BN / 32 instructions a wavefront).
template <int BN>
struct DmaNT {
  static constexpr int RPI = 512 / BN, N = 16 / RPI, LPR = BN / 8;
  uint32_t off[N];
  __device__ __forceinline__ void init(int64_t ld, int wave, int lane) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int r = 16 * wave + RPI * j + lane / LPR;
      const int c = (lane % LPR) ^ ((r & 3) << 2);
      off[j] = (uint32_t)((r * ld + 8 * c) * 2);
    }
  }
  __device__ __forceinline__ void issue(const uint16_t* base, uint16_t* dst, int wave,
                                        int j) const {
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const char*>(base) + off[j],
                                     (lds_void_t*)(dst + (16 * wave + RPI * j) * BN), 16, 0, 0);
  }
};

// One MFMA operand fragment (32 rows or columns x 16 k, lane l: index l % 32, k 8 (l / 32) ..
// + 7) of k-step s from an N-contiguous stage [64][W] (nmaj_off_w): ds_read_b64_tr_b16, where lane
// p of a 16-lane group reads row k + p / 4, columns c0 + 4 (p % 4) .. + 3, and lane i of the
// group receives column c0 + i of rows k .. k+3; c: the fragment's first column in the stage.
template <int W>
__device__ __forceinline__ half8_t read_frag_tr(const uint16_t* st, int c, int s, int lane) {
  const int p = lane & 15, fhalf = lane >> 5;
  const int col = c + 16 * ((lane >> 4) & 1) + 4 * (p & 3);
  const int k = 16 * s + 8 * fhalf + (p >> 2);
  const int o0 = nmaj_off_w<W>(k, col >> 3) + (col & 7);
  const int o1 = nmaj_off_w<W>(k + 4, col >> 3) + (col & 7);
  const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(st + o0));
  const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(st + o1));
  return __builtin_bit_cast(half8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// The fragments of k-step s = 0..3 of a 64-wide stage: FM A blocks of 32 rows, FN B blocks of 32
// columns (the wavefront's block: rows wm BM/2 .., columns wn BN/2 ..). TA: the A stage is
// M-contiguous [64][BM] (A stored transposed), read as B is in NN.
template <bool NN, int BM, int BN, bool TA = false>
__device__ __forceinline__ void read_frags64(FragsT<BM / 64, BN / 64>& f, const uint16_t* sa,
                                             const uint16_t* sb, int s, int wm, int wn,
                                             int lane) {
  constexpr int FM = BM / 64, FN = BN / 64;
  const int frow = lane & 31, fhalf = lane >> 5;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    if constexpr (TA)
      f.a[i] = read_frag_tr<BM>(sa, wm * (BM / 2) + 32 * i, s, lane);
    else
      f.a[i] = *reinterpret_cast<const half8_t*>(
          sa + kmaj64_off(wm * (BM / 2) + 32 * i + frow, 2 * s + fhalf));
  }
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    if constexpr (!NN)
      f.b[j] = *reinterpret_cast<const half8_t*>(
          sb + kmaj64_off(wn * (BN / 2) + 32 * j + frow, 2 * s + fhalf));
    else
      f.b[j] = read_frag_tr<BN>(sb, wn * (BN / 2) + 32 * j, s, lane);
  }
}

// Tail split, slice partials: the tile's accumulators as fp32 [BM rows][BN B columns] (B column:
// the tile's n (SwiGLU: its gate and up rows) as the wavefront blocks hold them:
// wn BN/2 + 32 j + column within the MFMA block). T: transposed accumulators (mfma_step).
template <bool T, int BM, int BN>
__device__ __forceinline__ void store_tail_part(float* p, const f32x16 (&acc)[BM / 64][BN / 64],
                                                int lane, int wave) {
  constexpr int FM = BM / 64, FN = BN / 64;
  const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      if constexpr (T) {  // register 4 q + e: row i 32 + l % 32, column 8 q + 4 (l / 32) + e
        float* row = p + (wm * (BM / 2) + i * 32 + (lane & 31)) * BN + wn * (BN / 2) + j * 32 +
                     4 * (lane >> 5);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<float4*>(row + 8 * q) =
              make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                          acc[i][j][4 * q + 3]);
      } else {  // register r: row i 32 + 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32
#pragma unroll
        for (int r = 0; r < 16; ++r)
          p[(wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * BN +
            wn * (BN / 2) + j * 32 + (lane & 31)] = acc[i][j][r];
      }
    }
}

// The GEMM with an fp16 B in memory (qlora_gemm16): for 256 x 256 tiles the same wavefront blocks,
// MFMA order and epilogues as nf4_gemm_kernel, so the results are the same bits as that
// kernel's for the same B values; every tile shape accumulates each output's k-steps of 16 in
// order, so either shape gives the same bits in one slice.
// One tile (TAIL: one K slice of a tail tile, its partial sums to g.tail_ws + tail_u tiles;
// otherwise tail_u is the tile's K slice, for split-K partials) over k-tiles kt0 .. kt1 - 1
// through the LDS stages sA0/sA1/sB0/sB1. The tail form is a
// separate instantiation so that the main tiles' register allocation stays that of the plain
// epilogue.
template <bool NN, bool TA, int EPI, bool TAIL, int BM, int BN, int STAGES>
__device__ __forceinline__ void hgemm_tile(const GemmArgs& g, int64_t tile_m, int64_t tile_n,
                                           int64_t kt0, int64_t kt1, int tail_u, uint16_t* sA0,
                                           uint16_t* sA1, uint16_t* sB0, uint16_t* sB1,
                                           uint16_t* sA2, uint16_t* sA3, uint16_t* sB2,
                                           uint16_t* sB3) {
  static_assert(BM == BN && (BM == 256 || BM == 128), "square 256 or 128 tiles");
  static_assert(STAGES == 2 || (STAGES == 4 && BM == 128), "four stages fit 128 x 128 tiles");
  constexpr int FM = BM / 64, FN = BN / 64;
  // DMA instructions a wavefront issues per k-tile (A and B alternate), and how they are dealt:
  // kSA during k-step 3 of the k-tile two before, kSB during k-step 0 of the one before, the rest
  // during its k-step 1
  constexpr int kQ = BM / 32 + BN / 32, kSA = kQ * 6 / 16, kSB = kQ * 5 / 16;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  // k-tile counts are multiples of STAGES (host check)
  if (kt1 > g.Kr / kBK64) kt1 = g.Kr / kBK64;
  const int64_t m0 = tile_m * BM;
  const int64_t kt_last = kt1 - 1;

  DmaKT<BM> dma_a;
  DmaNT<BM> dma_at;  // TA: A stored [K, M], the tile's BM columns of 64 rows a k-tile
  const uint16_t* a_base;
  int64_t a_step;
  if constexpr (TA) {
    dma_at.init(g.lda, wave, lane);  // M % BM == 0 (host check): whole tiles only
    a_base = g.a + m0;
    a_step = (int64_t)kBK64 * g.lda;
  } else {
    const int64_t a_rows = g.M - m0;  // rows past M re-read the last row
    dma_a.init(g.lda, [&](int r) -> int64_t { return r < a_rows ? r : a_rows - 1; }, wave, lane);
    a_base = g.a + m0 * g.lda;
    a_step = kBK64;
  }
  DmaKT<BN> dma_bk;
  DmaNT<BN> dma_bn;
  const uint16_t* b_base;
  int64_t b_step;
  if constexpr (NN) {
    dma_bn.init(g.ldb, wave, lane);
    b_base = g.b + tile_n * BN;
    b_step = (int64_t)kBK64 * g.ldb;
  } else {
    // rows past N (a last, partial tile: the lm_head's 151,936) re-read row N - 1
    dma_bk.init(g.ldb, [&](int r) -> int64_t {
      const int64_t row = nt_wrow<EPI, BN>(g, tile_n, r);
      return (swiglu_epi(EPI) || row < g.N) ? row : g.N - 1;
    }, wave, lane);
    b_base = g.b;
    b_step = kBK64;
  }

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};

  // DMA instructions q0 .. q1 - 1 of k-tile kt (q even: A row group q / 2, odd: B's); past the
  // last k-tile the last one is re-read into a stage no longer read
  auto issue_part = [&](int64_t kt, uint16_t* sa, uint16_t* sb, int q0, int q1) {
    kt = kt < kt1 ? kt : kt_last;
#pragma unroll
    for (int q = q0; q < q1; ++q) {
      if ((q & 1) == 0) {
        if constexpr (TA) dma_at.issue(a_base + kt * a_step, sa, wave, q >> 1);
        else dma_a.issue(a_base + kt * a_step, sa, wave, q >> 1);
      } else if constexpr (NN) dma_bn.issue(b_base + kt * b_step, sb, wave, q >> 1);
      else dma_bk.issue(b_base + kt * b_step, sb, wave, q >> 1);
    }
  };

  constexpr bool kT = staged_epi(EPI);
  FragsT<FM, FN> f0, f1;
  if constexpr (STAGES == 2) {
    issue_part(kt0, sA0, sB0, 0, kQ);
    issue_part(kt0 + 1, sA1, sB1, 0, kSA);
    sync_tile<kSA>();  // k-tile kt0 landed
    read_frags64<NN, BM, BN, TA>(f0, sA0, sB0, 0, wm, wn, lane);
    // k-tile t on stage t % 2, its four k-steps each reading the next one's fragments while its
    // MFMAs run. k-steps 0 and 1 finish the DMA of t + 1 into the other stage. After k-step 2
    // every wavefront has read this stage and t + 1 has landed (the barrier): k-step 3 reads
    // t + 1's first fragments and starts the DMA of t + 2 into this stage.
    auto k_tile = [&](int64_t t, uint16_t* sa, uint16_t* sb, uint16_t* sa_n, uint16_t* sb_n) {
      __builtin_amdgcn_sched_barrier(0);
      issue_part(t + 1, sa_n, sb_n, kSA, kSA + kSB);
      read_frags64<NN, BM, BN, TA>(f1, sa, sb, 1, wm, wn, lane);
      mfma_step<kT>(acc, f0);
      sched_step<NN, 0, kSB, FM, FN, TA>();
      __builtin_amdgcn_sched_barrier(0);
      issue_part(t + 1, sa_n, sb_n, kSA + kSB, kQ);
      read_frags64<NN, BM, BN, TA>(f0, sa, sb, 2, wm, wn, lane);
      mfma_step<kT>(acc, f1);
      sched_step<NN, 0, kQ - kSA - kSB, FM, FN, TA>();
      __builtin_amdgcn_sched_barrier(0);
      read_frags64<NN, BM, BN, TA>(f1, sa, sb, 3, wm, wn, lane);
      mfma_step<kT>(acc, f0);
      sched_step<NN, 0, 0, FM, FN, TA>();
      __builtin_amdgcn_sched_barrier(0);
      sync_tile<0>();
      issue_part(t + 2, sa, sb, 0, kSA);
      read_frags64<NN, BM, BN, TA>(f0, sa_n, sb_n, 0, wm, wn, lane);
      mfma_step<kT>(acc, f1);
      sched_step<NN, 0, kSA, FM, FN, TA>();
      __builtin_amdgcn_sched_barrier(0);
    };
    for (int64_t t = kt0; t < kt1; t += 2) {
      k_tile(t, sA0, sB0, sA1, sB1);
      k_tile(t + 1, sA1, sB1, sA0, sB0);
    }
  } else {
    // Four stages, k-tile t on stage t % 4: the DMA of t + 3 goes into the stage t - 1 used
    // (free since the barrier that ended t - 1's reads), spread over k-steps 0-2 of t, so a
    // k-tile's loads have about eleven k-steps to land; the barrier after k-step 2 waits for
    // t + 1 only (t + 2 and t + 3 stay in flight).
    constexpr int q1 = (kQ + 2) / 3, q2 = 2 * q1;
    issue_part(kt0, sA0, sB0, 0, kQ);
    issue_part(kt0 + 1, sA1, sB1, 0, kQ);
    issue_part(kt0 + 2, sA2, sB2, 0, kQ);
    sync_tile<2 * kQ>();  // k-tile kt0 landed
    read_frags64<NN, BM, BN, TA>(f0, sA0, sB0, 0, wm, wn, lane);
    auto k_tile = [&](int64_t t, uint16_t* sa, uint16_t* sb, uint16_t* sa_n, uint16_t* sb_n,
                      uint16_t* sa_p, uint16_t* sb_p) {
      __builtin_amdgcn_sched_barrier(0);
      issue_part(t + 3, sa_p, sb_p, 0, q1);
      read_frags64<NN, BM, BN, TA>(f1, sa, sb, 1, wm, wn, lane);
      mfma_step<kT>(acc, f0);
      sched_step<NN, 0, q1, FM, FN, TA>();
      __builtin_amdgcn_sched_barrier(0);
      issue_part(t + 3, sa_p, sb_p, q1, q2);
      read_frags64<NN, BM, BN, TA>(f0, sa, sb, 2, wm, wn, lane);
      mfma_step<kT>(acc, f1);
      sched_step<NN, 0, q2 - q1, FM, FN, TA>();
      __builtin_amdgcn_sched_barrier(0);
      issue_part(t + 3, sa_p, sb_p, q2, kQ);
      read_frags64<NN, BM, BN, TA>(f1, sa, sb, 3, wm, wn, lane);
      mfma_step<kT>(acc, f0);
      sched_step<NN, 0, kQ - q2, FM, FN, TA>();
      __builtin_amdgcn_sched_barrier(0);
      sync_tile<2 * kQ>();  // t + 1 landed; t + 2, t + 3 may be in flight
      read_frags64<NN, BM, BN, TA>(f0, sa_n, sb_n, 0, wm, wn, lane);
      mfma_step<kT>(acc, f1);
      sched_step<NN, 0, 0, FM, FN, TA>();
      __builtin_amdgcn_sched_barrier(0);
    };
    for (int64_t t = kt0; t < kt1; t += 4) {
      k_tile(t, sA0, sB0, sA1, sB1, sA3, sB3);
      k_tile(t + 1, sA1, sB1, sA2, sB2, sA0, sB0);
      k_tile(t + 2, sA2, sB2, sA3, sB3, sA1, sB1);
      k_tile(t + 3, sA3, sB3, sA0, sB0, sA2, sB2);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  if constexpr (TAIL) {
    store_tail_part<kT, BM, BN>(g.tail_ws + (int64_t)tail_u * BM * BN, acc, lane, wave);
  } else {
    if constexpr (kT) __builtin_amdgcn_s_barrier();
    // each wavefront stages its fp16 block in one of the four operand stages
    uint16_t* st = wave == 0 ? sA0 : wave == 1 ? sA1 : wave == 2 ? sB0 : sB1;
    store_tile<EPI, BM, BN>(g, acc, st, st + (BM / 4) * (BN / 2), m0, tile_n, lane, wave,
                            tail_u);
  }
}

// STAGES: 2 (either tile; 128 x 128 tiles then leave room for a second workgroup per CU) or 4
// (128 x 128 only, 128 KB: one workgroup per CU, loads issued three k-tiles ahead).
template <bool NN, int EPI, int BM, int STAGES, bool TA = false>
__global__ __launch_bounds__(kThreads, (BM == 128 && STAGES == 2) ? 2 : 1) void hgemm_kernel(
    GemmArgs g) {
  constexpr int kX = STAGES == 4 ? BM * kBK64 : 8;  // stages 2-3 (unused with two stages)
  __shared__ __attribute__((aligned(1024))) uint16_t sA0[BM * kBK64];
  __shared__ __attribute__((aligned(1024))) uint16_t sA1[BM * kBK64];
  __shared__ __attribute__((aligned(1024))) uint16_t sB0[BM * kBK64];
  __shared__ __attribute__((aligned(1024))) uint16_t sB1[BM * kBK64];
  __shared__ __attribute__((aligned(1024))) uint16_t sA2[kX];
  __shared__ __attribute__((aligned(1024))) uint16_t sA3[kX];
  __shared__ __attribute__((aligned(1024))) uint16_t sB2[kX];
  __shared__ __attribute__((aligned(1024))) uint16_t sB3[kX];
  // past the main tiles: one K slice of one of the last round's tiles (tail split)
  const int tail_u = g.tail_splits > 0 ? (int)blockIdx.x - g.main_tiles : -1;
  if (tail_u >= 0) {
    const int t = g.main_tiles + tail_u / g.tail_splits;
    const int64_t kt0 =
        (int64_t)__builtin_amdgcn_readfirstlane(tail_u % g.tail_splits) * g.kt_per_tail;
    hgemm_tile<NN, TA, EPI, true, BM, BM, STAGES>(
        g, __builtin_amdgcn_readfirstlane(t % g.m_tiles),
        __builtin_amdgcn_readfirstlane(t / g.m_tiles), kt0, kt0 + g.kt_per_tail, tail_u, sA0,
        sA1, sB0, sB1, sA2, sA3, sB2, sB3);
    return;
  }
  int64_t tile_m, tile_n;
  int slice;
  tile_of(g.m_tiles, g.tiles, g.tail_splits > 0 ? g.main_tiles : (int)gridDim.x, tile_m, tile_n,
          slice);
  const int64_t kt0 = (int64_t)slice * g.kt_per_split;
  hgemm_tile<NN, TA, EPI, false, BM, BM, STAGES>(g, tile_m, tile_n, kt0, kt0 + g.kt_per_split,
                                                 slice, sA0, sA1, sB0, sB1, sA2, sA3, sB2, sB3);
}

// Tail split: the slices of each tail tile summed in slice order, then the epilogue (fp16 store,
// bias, fp32 residual, SwiGLU), four outputs per thread. Tile g.bm x g.bn.
__global__ __launch_bounds__(256) void tail_reduce_kernel(GemmArgs g, int epi, int tiles) {
  const bool sw = swiglu_epi(epi);
  const int BM = g.bm, BN = g.bn, WC = BN / 2;
  const int per_tile = sw ? BM * (BN / 8) : BM * (BN / 4);  // threads per tile
  const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= (int64_t)tiles * per_tile) return;
  const int u = (int)(id / per_tile), w = (int)(id - (int64_t)u * per_tile);
  const int t = g.main_tiles + u;
  const int64_t tile_m = t % g.m_tiles, tile_n = t / g.m_tiles;
  const int64_t slice = (int64_t)BM * BN;
  const float* part = g.tail_ws + (int64_t)u * g.tail_splits * slice;
  const int S = g.tail_splits;
  if (sw) {
    // four of the tile's BN / 2 output columns; a wavefront block's first WC / 2 B columns are
    // gate rows, its last WC / 2 the matching up rows
    const int row = w / (BN / 8), oc = (w % (BN / 8)) * 4;
    const int lc = (oc / (WC / 2)) * WC + oc % (WC / 2);  // gate; up: + WC / 2
    float4 gs = *reinterpret_cast<const float4*>(part + row * BN + lc);
    float4 us = *reinterpret_cast<const float4*>(part + row * BN + lc + WC / 2);
    for (int k = 1; k < S; ++k) {
      const float4 a = *reinterpret_cast<const float4*>(part + k * slice + row * BN + lc);
      const float4 b = *reinterpret_cast<const float4*>(part + k * slice + row * BN + lc +
                                                        WC / 2);
      gs.x += a.x; gs.y += a.y; gs.z += a.z; gs.w += a.w;
      us.x += b.x; us.y += b.y; us.z += b.z; us.w += b.w;
    }
    const int64_t m = tile_m * BM + row, n = tile_n * (BN / 2) + oc;
    if (m >= g.M) return;
    const float gv[4] = {gs.x, gs.y, gs.z, gs.w}, uv[4] = {us.x, us.y, us.z, us.w};
    if (epi == kEpiSwigluKeep) {  // the product [g | u] itself
      *reinterpret_cast<uint2*>(g.gu + m * g.ldgu + n) =
          make_uint2(pack2h(gv[0], gv[1]), pack2h(gv[2], gv[3]));
      *reinterpret_cast<uint2*>(g.gu + m * g.ldgu + g.I + n) =
          make_uint2(pack2h(uv[0], uv[1]), pack2h(uv[2], uv[3]));
    }
    float mv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float gt = h2f(f2h(gv[e])), up = h2f(f2h(uv[e]));
      mv[e] = gt * sigmoid_fast(gt) * up;  // as store_tile
    }
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(g.c) + m * g.ldc + n) =
        make_uint2(pack2h(mv[0], mv[1]), pack2h(mv[2], mv[3]));
    return;
  }
  const int row = w / (BN / 4), lc = (w % (BN / 4)) * 4;
  float4 v4 = *reinterpret_cast<const float4*>(part + row * BN + lc);
  for (int k = 1; k < S; ++k) {
    const float4 a = *reinterpret_cast<const float4*>(part + k * slice + row * BN + lc);
    v4.x += a.x; v4.y += a.y; v4.z += a.z; v4.w += a.w;
  }
  const int64_t m = tile_m * BM + row, n = tile_n * BN + lc;
  if (m >= g.M || n >= g.N) return;  // N % 8 == 0: the four columns lie on one side
  float v[4] = {v4.x, v4.y, v4.z, v4.w};
  if (epi == kEpiResid) {
    float* out = static_cast<float*>(g.c) + m * g.ldc + n;
    const float* r = g.resid + m * g.ldr + n;
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = r[e] + h2f(f2h(v[e]));
    return;
  }
  if (epi == kEpiBias)
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] += h2f_bits(g.bias[n + e]);
  *reinterpret_cast<uint2*>(static_cast<uint16_t*>(g.c) + m * g.ldc + n) =
      make_uint2(pack2h(v[0], v[1]), pack2h(v[2], v[3]));
}

// Sum of the split-K partials [splits, M, N] and the epilogue (store / bias / residual / fp32
// with alpha and a row-scaled residual).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* ws, int splits,
                                                            int64_t M, int64_t N, int epi,
                                                            void* c, int64_t ldc,
                                                            const uint16_t* bias,
                                                            const float* resid, int64_t ldr,
                                                            float alpha,
                                                            const float* row_scale) {
  const int64_t idx = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (idx >= M * N) return;
  const int64_t m = idx / N, n = idx - m * N;  // N % 4 == 0: four columns of one row
  float4 s = reinterpret_cast<const float4*>(ws + idx)[0];
  for (int k = 1; k < splits; ++k) {
    const float4 t = reinterpret_cast<const float4*>(ws + (int64_t)k * M * N + idx)[0];
    s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
  }
  float v[4] = {s.x, s.y, s.z, s.w};
  if (epi == kEpiF32) {  // as store_tile's kEpiF32 (out may be resid)
    float* out = static_cast<float*>(c) + m * ldc + n;
    const float rs = resid == nullptr ? 0.0f : row_scale == nullptr ? 1.0f : row_scale[m];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float o = alpha * v[i];
      if (resid != nullptr) o += rs * resid[m * ldr + n + i];
      out[i] = o;
    }
  } else if (epi == kEpiResid) {
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

// kernel selector: BSRC kBNF4 -> nf4_gemm_kernel, kBHalf -> hgemm_kernel. start/stop (may be
// null): events the dispatch records at the kernel's own start and end (hipExtLaunchKernelGGL)
template <int BSRC, bool NN, int EPI, int BM, int ST, bool TA = false>
void launch_one(const GemmArgs& g, dim3 grid, hipStream_t s, hipEvent_t start, hipEvent_t stop) {
  auto kernel = [] {
    if constexpr (BSRC == kBNF4) return nf4_gemm_kernel<NN, EPI>;
    else return hgemm_kernel<NN, EPI, BM, ST, TA>;
  }();
  if (start != nullptr || stop != nullptr)
    hipExtLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, s, start, stop, 0, g);
  else
    hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, s, g);
}

template <bool NN, int BSRC, int BM, int ST>
void launch_epi(const GemmArgs& g, dim3 grid, hipStream_t s, int epi, hipEvent_t start,
                hipEvent_t stop) {
  switch (epi) {
    case kEpiStore: launch_one<BSRC, NN, kEpiStore, BM, ST>(g, grid, s, start, stop); break;
    case kEpiBias: launch_one<BSRC, NN, kEpiBias, BM, ST>(g, grid, s, start, stop); break;
    case kEpiResid: launch_one<BSRC, NN, kEpiResid, BM, ST>(g, grid, s, start, stop); break;
    case kEpiPartial: launch_one<BSRC, NN, kEpiPartial, BM, ST>(g, grid, s, start, stop); break;
    case kEpiF32:
      if constexpr (NN && BSRC == kBHalf) launch_one<BSRC, NN, kEpiF32, BM, ST>(g, grid, s, start, stop);
      break;
    default:
      if constexpr (!NN) {
        if (epi == kEpiSwigluKeep) launch_one<BSRC, NN, kEpiSwigluKeep, BM, ST>(g, grid, s, start, stop);
        else launch_one<BSRC, NN, kEpiSwiglu, BM, ST>(g, grid, s, start, stop);
      }
      break;
  }
}

// Transposed A (B as in NN): the fp32 epilogue and its split-K partials only.
template <int BM, int ST>
void launch_ta(const GemmArgs& g, dim3 grid, hipStream_t s, int epi, hipEvent_t start,
               hipEvent_t stop) {
  if (epi == kEpiF32) launch_one<kBHalf, true, kEpiF32, BM, ST, true>(g, grid, s, start, stop);
  else launch_one<kBHalf, true, kEpiPartial, BM, ST, true>(g, grid, s, start, stop);
}

// The kernel for (B source, mode, tile, stages) with the epilogue epi (mode 2: transposed A).
void launch_any(const GemmArgs& g, int bsrc, int mode, int tile, int stages, dim3 grid,
                hipStream_t s, int epi, hipEvent_t start, hipEvent_t stop) {
  if (mode == 2) {
    if (tile == 128 && stages == 4) launch_ta<128, 4>(g, grid, s, epi, start, stop);
    else if (tile == 128) launch_ta<128, 2>(g, grid, s, epi, start, stop);
    else launch_ta<256, 2>(g, grid, s, epi, start, stop);
    return;
  }
  if (bsrc == kBNF4) {
    if (mode == 0) launch_epi<false, kBNF4, 256, 2>(g, grid, s, epi, start, stop);
    else launch_epi<true, kBNF4, 256, 2>(g, grid, s, epi, start, stop);
  } else if (tile == 128 && stages == 4) {
    if (mode == 0) launch_epi<false, kBHalf, 128, 4>(g, grid, s, epi, start, stop);
    else launch_epi<true, kBHalf, 128, 4>(g, grid, s, epi, start, stop);
  } else if (tile == 128) {
    if (mode == 0) launch_epi<false, kBHalf, 128, 2>(g, grid, s, epi, start, stop);
    else launch_epi<true, kBHalf, 128, 2>(g, grid, s, epi, start, stop);
  } else {
    if (mode == 0) launch_epi<false, kBHalf, 256, 2>(g, grid, s, epi, start, stop);
    else launch_epi<true, kBHalf, 256, 2>(g, grid, s, epi, start, stop);
  }
}

bool al(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

constexpr int kCUs = 256;  // compute units of an MI355X

// Workgroups resident at once for a tile shape: 256 x 256 tiles take a CU each (128 KB of
// LDS), 128 x 128 tiles two per CU with two stages (64 KB each), one with four (128 KB).
int64_t slots_of(int tile, int stages) { return tile == 128 && stages == 2 ? 2 * kCUs : kCUs; }

// Tail split of an fp16-B product in one slice: when the tiles past the GPU's last full round
// of tiles fill at most half a round they would take a whole round; as K slices (tail_splits
// of them per tile, kt_per_tail k-tiles each, an even count, no empty slice) they fill about
// one round of short workgroups instead. Returns the fp32 workspace elements it needs, 0 when
// it does not apply.
int64_t tail_plan(int64_t m_tiles, int64_t n_tiles, int64_t ktiles, int tile, int stages,
                  int* main_tiles, int* splits, int* kt_per) {
  const int64_t slots = slots_of(tile, stages);
  const int64_t tiles = m_tiles * n_tiles, full = tiles / slots * slots, r = tiles - full;
  if (full == 0 || r == 0 || r > slots / 2) return 0;
  for (int sp = 16; sp >= 2; --sp) {
    const int64_t per = qlora_cdiv(qlora_cdiv(ktiles, sp), stages) * stages;
    if (r * sp > slots || per * (sp - 1) >= ktiles) continue;
    *main_tiles = (int)full;
    *splits = sp;
    *kt_per = (int)per;
    return r * sp * tile * tile;
  }
  return 0;
}

int64_t n_tiles_of(int64_t N, int epi, int tile) {
  return swiglu_epi(epi) ? N / (tile / 2) : qlora_cdiv(N, tile);
}

// The tile shape, stage count and K split of qlora_gemm16 with tile 0 / splits 0: the cheapest
// variant under a fixed cost model, so a problem always runs the same kernels and gives the same
// bits (no timing at run time). A launch runs in rounds (as many workgroups as the GPU holds at
// once: 256 tiles of 256 x 256, 512 of 128 x 128 with two stages, 256 with four); its cost is
//   a rounds + b (the k elements its rounds walk) + c (MB of fp32 partials) + d (a reduce),
// the constants (us) least-squares fits of every variant over the step's nine products and the
// lm_head's at 1,024 - 4,096 tokens on MI355X (HIP graphs, warm caches; median error 5-8 %).
// Candidates: 256 x 256 tiles in 1-8 K slices (7 or 8 fill the GPU when a long reduction has
// 32-36 output tiles), 128 x 128 tiles in 1, 2 or 4 (up to K = 12,288: beyond that the
// measurements favoured 256 x 256 tiles, whose loads per flop are half).
struct PlanCoef {
  int tile, stages;
  double a, b, c, d;
};
constexpr PlanCoef kPlanCoef[] = {{256, 2, 9.74, 0.01998, 0.1219, 7.50},
                                  {128, 4, 4.62, 0.00788, 0.1462, 5.29},
                                  {128, 2, 6.31, 0.01262, 0.1125, 6.45}};

// The model's cost (us) of one variant, or a negative value when it cannot run the problem.
double plan_cost(int64_t M, int64_t N, int64_t K, int mode, int epi, const PlanCoef& v,
                 int splits) {
  const int tile = v.tile, stages = v.stages;
  const int64_t kt = K / kBK64;
  if (kt % stages != 0 || (mode != 0 && N % tile != 0) || (mode == 2 && M % tile != 0))
    return -1.0;
  if (swiglu_epi(epi) && (splits > 1 || N % (tile / 2) != 0)) return -1.0;
  const int64_t per = qlora_cdiv(qlora_cdiv(kt, splits), stages) * stages;
  if (per * (splits - 1) >= kt) return -1.0;  // an empty slice
  const int64_t m_tiles = qlora_cdiv(M, tile), tiles = m_tiles * n_tiles_of(N, epi, tile);
  const int64_t slots = slots_of(tile, stages);
  if (splits > 1) {
    const double rounds = (double)qlora_cdiv(tiles * splits, slots);
    return v.a * rounds + v.b * rounds * (double)(per * kBK64) +
           v.c * 8.0 * splits * (double)M * (double)N / 1e6 + v.d;
  }
  const int64_t full = tiles / slots, r = tiles - full * slots;
  double rounds = (double)full, kwalk = (double)full * (double)K, part = 0.0, red = 0.0;
  if (r > 0) {
    int main_t, ts, ktp;
    rounds += 1.0;
    if (tail_epi(epi) &&
        tail_plan(m_tiles, tiles / m_tiles, kt, tile, stages, &main_t, &ts, &ktp) > 0) {
      kwalk += (double)ktp * kBK64;
      part = 8.0 * (double)(r * ts) * tile * tile / 1e6;
      red = 1.0;
    } else {
      kwalk += (double)K;
    }
  }
  return v.a * rounds + v.b * kwalk + v.c * part + v.d * red;
}

// A product in one slice on 256 x 256 tiles whose last round of tiles would run part-full can
// instead run its whole rounds on 256 x 256 tiles, over the leading output columns that fill
// them (whole N tiles), and the remaining columns as a second launch on 128 x 128 tiles (which
// fill a round four times as finely and need no partials or reduce, where the K-sliced last
// round writes and sums fp32 slices). Returns the columns of the first launch (0 when the split
// does not apply) and, through cost, the model's cost of both launches (the same constants,
// plus kGap us for the second launch's start).
constexpr double kGap = 1.5;
int64_t rest_split(int64_t M, int64_t N, int64_t K, int mode, int epi, const PlanCoef& v128,
                   double* cost) {
  const PlanCoef& v256 = kPlanCoef[0];
  const int64_t kt = K / kBK64;
  if (epi == kEpiF32 || mode == 2 || kt % 2 != 0 || kt % v128.stages != 0 || K > 12288)
    return 0;
  const int cols = swiglu_epi(epi) ? 128 : 256;  // output columns of a 256 x 256 tile
  if (swiglu_epi(epi) ? N % 128 != 0 : (mode != 0 && N % 256 != 0)) return 0;
  const int64_t m_tiles = qlora_cdiv(M, 256), n_tiles = n_tiles_of(N, epi, 256);
  const int64_t rounds = m_tiles * n_tiles / kCUs;
  const int64_t n_main = rounds * kCUs / m_tiles;  // whole N tiles in the full rounds
  if (rounds == 0 || n_main == 0 || n_main >= n_tiles) return 0;
  const int64_t n_rest = N - n_main * cols;
  const int64_t t128 = qlora_cdiv(M, 128) * n_tiles_of(n_rest, epi, 128);
  const double r128 = (double)qlora_cdiv(t128, slots_of(128, v128.stages));
  *cost = v256.a * rounds + v256.b * rounds * (double)K + v128.a * r128 +
          v128.b * r128 * (double)K + kGap;
  return n_main * cols;
}

void auto_plan(int64_t M, int64_t N, int64_t K, int mode, int epi, int* tile, int* stages,
               int* splits, int* rest = nullptr, int64_t* n_first = nullptr) {
  double best = -1.0;
  *tile = 256;
  *stages = 2;
  *splits = 1;
  if (rest != nullptr) *rest = 0;
  if (n_first != nullptr) *n_first = 0;
  // first pass: 128 x 128 tiles up to K = 12,288 only; second (when none of the first's can run
  // the problem: an NN product whose N is not a multiple of 256), every variant
  for (int pass = 0; pass < 2 && best < 0.0; ++pass) {
    for (const PlanCoef& v : kPlanCoef) {
      if (pass == 0 && v.tile == 128 && K > 12288) continue;
      for (int sp = 1; sp <= (v.tile == 256 ? 8 : 4); ++sp) {
        if (v.tile == 128 && sp == 3) continue;
        const double c = plan_cost(M, N, K, mode, epi, v, sp);
        if (c >= 0.0 && (best < 0.0 || c < best)) {
          best = c;
          *tile = v.tile;
          *stages = v.stages;
          *splits = sp;
        }
      }
    }
  }
  if (rest == nullptr || best < 0.0) return;
  for (int vi = 1; vi <= 2; ++vi) {
    double c = -1.0;
    const int64_t nf = rest_split(M, N, K, mode, epi, kPlanCoef[vi], &c);
    if (nf > 0 && c < best) {
      best = c;
      *tile = 256;
      *stages = 2;
      *splits = 1;
      *rest = kPlanCoef[vi].stages;
      *n_first = nf;
    }
  }
}

// Shared launch path: shapes and workspace checked, then the tile grid (and the split-K reduce).
// tile: 256 or 128 (fp16 B; the NF4 kernel's is 256). start/stop (may be null): recorded at the
// start of the tile grid and the end of the last kernel.
int run_gemm(GemmArgs& g, int bsrc, int mode, int epi, int splits, float* ws, int64_t ws_elems,
             hipStream_t s, hipEvent_t start = nullptr, hipEvent_t stop = nullptr,
             int tile = 256, int stages = 2, bool parts_only = false) {
  QLORA_CHECK_ARG((tile == 256 && stages == 2) ||
                  (tile == 128 && bsrc == kBHalf && (stages == 2 || stages == 4)));
  g.bm = g.bn = tile;
  const int64_t n_tiles = n_tiles_of(g.N, epi, tile);
  g.m_tiles = (int)qlora_cdiv(g.M, tile);
  const int64_t grid = (int64_t)g.m_tiles * n_tiles;
  QLORA_CHECK_ARG(grid < (1ll << 31));
  g.tiles = (int)grid;
  // fp16 outputs leave in 16-byte row pieces
  QLORA_CHECK_ARG(epi == kEpiResid || epi == kEpiF32 || splits > 1 ||
                  (g.ldc % 8 == 0 && al(g.c, 16)));
  // the fp32 residual form reads and writes 32-byte row pieces
  QLORA_CHECK_ARG(epi != kEpiResid || splits > 1 ||
                  (g.ldc % 4 == 0 && g.ldr % 4 == 0 && al(g.c, 16) && al(g.resid, 16)));
  QLORA_CHECK_ARG(splits == 1 || (ws && ws_elems >= (int64_t)splits * g.M * g.N && al(ws, 16)));
  // NF4 B: k-tiles of 32, four per loop trip; fp16 B: k-tiles of 64, two per trip (the split
  // boundaries fall on the same multiples of 128 either way)
  const int bk = bsrc == kBNF4 ? kBK : kBK64, per_trip = bsrc == kBNF4 ? kStages : stages;
  const int64_t ktiles = g.Kr / bk;
  QLORA_CHECK_ARG(ktiles % per_trip == 0);
  g.kt_per_split = (int)(qlora_cdiv(qlora_cdiv(ktiles, splits), per_trip) * per_trip);
  QLORA_CHECK_ARG((int64_t)g.kt_per_split * (splits - 1) < ktiles);  // no empty slice
  int main_t = 0, tail_s = 0, kt_tail = 0;
  const int64_t tail_need =
      bsrc == kBHalf && splits == 1 && ws != nullptr && tail_epi(epi)
          ? tail_plan(g.m_tiles, n_tiles, ktiles, tile, stages, &main_t, &tail_s, &kt_tail)
          : 0;
  if (tail_need > 0 && ws_elems >= tail_need && al(ws, 16)) {
    g.main_tiles = main_t;
    g.tail_splits = tail_s;
    g.kt_per_tail = kt_tail;
    g.tail_ws = ws;
    const int64_t r = grid - main_t;
    const dim3 tg((unsigned)(main_t + r * tail_s));
    launch_any(g, bsrc, mode, tile, stages, tg, s, epi, start, nullptr);
    if (int rc = qlora_launch_status()) return rc;
    const int64_t threads = r * (swiglu_epi(epi) ? tile * (tile / 8) : tile * (tile / 4));
    const dim3 rg((unsigned)qlora_cdiv(threads, 256));
    if (stop != nullptr)
      hipExtLaunchKernelGGL(tail_reduce_kernel, rg, dim3(256), 0, s, nullptr, stop, 0, g, epi,
                            (int)r);
    else
      hipLaunchKernelGGL(tail_reduce_kernel, rg, dim3(256), 0, s, g, epi, (int)r);
    return qlora_launch_status();
  }
  const int kepi = splits > 1 ? (int)kEpiPartial : epi;
  void* out = g.c;
  if (splits > 1) g.c = ws;
  QLORA_CHECK_ARG(grid * splits < (1ll << 31));
  const dim3 gdim((unsigned)(grid * splits));
  launch_any(g, bsrc, mode, tile, stages, gdim, s, kepi, start, splits > 1 ? nullptr : stop);
  int rc = qlora_launch_status();
  if (rc != 0 || splits == 1 || parts_only) return rc;
  QLORA_CHECK_ARG(g.N % 4 == 0 && g.ldc % 4 == 0 && (epi != kEpiResid || g.ldr % 4 == 0));
  const int64_t quads = g.M * g.N / 4;
  const dim3 rgrid((unsigned)qlora_cdiv(quads, 256));
  if (stop != nullptr)
    hipExtLaunchKernelGGL(splitk_reduce_kernel, rgrid, dim3(256), 0, s, nullptr, stop, 0, ws,
                          splits, g.M, g.N, epi, out, g.ldc, g.bias, g.resid, g.ldr, g.alpha,
                          g.row_scale);
  else
    hipLaunchKernelGGL(splitk_reduce_kernel, rgrid, dim3(256), 0, s, ws, splits, g.M, g.N, epi,
                       out, g.ldc, g.bias, g.resid, g.ldr, g.alpha, g.row_scale);
  return qlora_launch_status();
}

// Output columns and reduction length of a problem, from the weight's shape and the mode.
int shape_of(int mode, int epi, int64_t w_rows, int64_t w_cols, int64_t swiglu_I, int64_t* N,
             int64_t* Kr) {
  if (mode == 0) {
    *Kr = w_cols;
    *N = epi == kEpiSwiglu ? swiglu_I : w_rows;
    QLORA_CHECK_ARG(epi != kEpiSwiglu || (swiglu_I % 128 == 0 && 2 * swiglu_I == w_rows));
    QLORA_CHECK_ARG(epi == kEpiSwiglu || w_rows % kBN == 0);
  } else {
    *Kr = w_rows;
    *N = w_cols;
    QLORA_CHECK_ARG(w_cols % kBN == 0);
  }
  QLORA_CHECK_ARG(*Kr % (kStages * kBK) == 0);
  return 0;
}

}  // namespace

// The fp32 scale of each 64-value block of an NF4 weight, as the dequant forms it (nf4.h:
// nf4_block_scale): the GEMM's B loader reads one word per block instead of the double-quant
// chain (absmax code -> code2 -> times absmax2 -> plus offset). Weights are frozen, so the host
// computes these once per weight.
__global__ __launch_bounds__(256) void nf4_block_scales_kernel(NF4Ref w, int64_t blocks,
                                                               float* out) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b < blocks) out[b] = nf4_block_scale(w, b);
}

QLORA_API int qlora_nf4_block_scales(const void* absmax, const float* code2,
                                     const float* absmax2, const float* offsets, int32_t nested,
                                     int32_t bs2, int64_t seg1, int64_t seg2, int64_t blocks,
                                     float* out, void* stream) {
  QLORA_CHECK_ARG(blocks >= 0);
  if (blocks == 0) return 0;
  QLORA_CHECK_ARG(absmax && out);
  QLORA_CHECK_ARG(!nested || (code2 && absmax2 && offsets && bs2 > 0 && (bs2 & (bs2 - 1)) == 0));
  const NF4Ref w{nullptr, absmax, code2, absmax2, offsets, nullptr, seg1, seg2, 6,
                 nested ? __builtin_ctz(bs2) : 0, nested, 1};
  hipLaunchKernelGGL(nf4_block_scales_kernel, dim3((unsigned)qlora_cdiv(blocks, 256)), dim3(256),
                     0, (hipStream_t)stream, w, blocks, out);
  return qlora_launch_status();
}

// NF4-decode GEMM. W [w_rows, w_cols]: `packed` codes, `scales` the fp32 scale of each 64-value
// block (qlora_nf4_block_scales), `code` the 16 levels or null for the NF4 table; tiled = 1
// (NT only): both in the tile-major order (each 32-column k-tile of each 256-row tile, its rows
// in the order the kernel's tile holds them, contiguous). mode: 0 = NT (C = A W^T), 1 = NN
// (C = A W). epi: 0 store fp16, 1 + bias, 2 fp32 residual, 3 SwiGLU (NT only). splits > 1:
// split-K through `ws` (fp32, splits M N).
QLORA_API int qlora_nf4_gemm(const void* a, int64_t lda, const void* packed, const float* scales,
                             const float* code, int32_t bs1, int32_t tiled, int64_t w_rows,
                             int64_t w_cols, void* c, int64_t ldc, const void* bias,
                             const float* resid, int64_t ldr, int64_t M, int32_t mode,
                             int32_t epi, int64_t swiglu_I, int32_t splits, float* ws,
                             int64_t ws_elems, void* stream) {
  QLORA_CHECK_ARG(M >= 0 && w_rows > 0 && w_cols > 0);
  if (M == 0) return 0;
  QLORA_CHECK_ARG(a && packed && scales && c && (mode == 0 || mode == 1));
  QLORA_CHECK_ARG(epi >= 0 && epi <= 3 && !(epi == 3 && mode != 0));
  QLORA_CHECK_ARG(splits >= 1 && splits <= 16 && !(splits > 1 && epi == 3));
  QLORA_CHECK_ARG(bs1 == 64);  // a thread's 32 values of a k-tile lie in one block
  QLORA_CHECK_ARG(tiled == 0 || (tiled == 1 && mode == 0));
  QLORA_CHECK_ARG(epi != 1 || bias);
  QLORA_CHECK_ARG(epi != 2 || (resid && ldr >= 0));
  int64_t N, Kr;
  int rc = shape_of(mode, epi, w_rows, w_cols, swiglu_I, &N, &Kr);
  if (rc) return rc;
  QLORA_CHECK_ARG(lda >= Kr && ldc >= N && (epi != 2 || ldr >= N));
  QLORA_CHECK_ARG(lda % 8 == 0 && al(a, 16) && al(packed, 16) && al(scales, 4));
  QLORA_CHECK_ARG(256 * lda * 2 < (1ll << 32));  // 32-bit DMA offsets within an A tile
  GemmArgs g{};
  g.a = static_cast<const uint16_t*>(a);
  g.lda = lda;
  g.w_packed = static_cast<const uint8_t*>(packed);
  g.w_scales = scales;
  g.w_code = code;
  g.w_tiled = tiled;
  g.Kw = w_cols;
  g.c = c;
  g.ldc = ldc;
  g.bias = static_cast<const uint16_t*>(bias);
  g.resid = resid;
  g.ldr = ldr;
  g.M = M;
  g.N = N;
  g.Kr = Kr;
  g.I = swiglu_I;
  return run_gemm(g, kBNF4, mode, epi, splits, ws, ws_elems, (hipStream_t)stream);
}

// The GEMM with an fp16 B in memory: NT B [N, K] (ldb), NN B [K, N] (ldb), on tile x tile
// output tiles (256 or 128). The timed form also records start/stop (hipEvent_t with timing,
// or null) at the start of the tile grid and the end of the last kernel.
QLORA_API int qlora_gemm16_timed(const void* a, int64_t lda, const void* b, int64_t ldb,
                                 int64_t M, int64_t N, int64_t K, int32_t mode, void* c,
                                 int64_t ldc, const void* bias, const float* resid, int64_t ldr,
                                 int32_t epi, int64_t swiglu_I, void* gu, int64_t ldgu,
                                 int32_t tile, int32_t stages, int32_t splits, float* ws,
                                 int64_t ws_elems, void* stream, void* start, void* stop) {
  QLORA_CHECK_ARG(M >= 0 && N > 0 && K > 0);
  if (M == 0) return 0;
  QLORA_CHECK_ARG(a && b && c && (mode == 0 || mode == 1));
  QLORA_CHECK_ARG((tile == 0) == (splits == 0));
  QLORA_CHECK_ARG(epi >= 0 && epi <= 5 && epi != kEpiPartial && !(swiglu_epi(epi) && mode != 0));
  int rest = 0;
  int64_t n_first = 0;
  if (tile == 0) auto_plan(M, N, K, mode, epi, &tile, &stages, &splits, &rest, &n_first);
  QLORA_CHECK_ARG((tile == 256 && stages == 2) || (tile == 128 && (stages == 2 || stages == 4)));
  QLORA_CHECK_ARG(splits >= 1 && splits <= 16 && !(splits > 1 && swiglu_epi(epi)));
  // the split-K reduce writes four columns a thread
  QLORA_CHECK_ARG(splits == 1 || (N % 4 == 0 && ldc % 4 == 0 && (epi != 2 || ldr % 4 == 0)));
  QLORA_CHECK_ARG(epi != 1 || bias);
  QLORA_CHECK_ARG(epi != 2 || (resid && ldr >= N));
  // the kept product [g | u]: [M, 2 N] fp16, 16-byte rows
  QLORA_CHECK_ARG(epi != kEpiSwigluKeep || (gu && ldgu >= 2 * N && ldgu % 8 == 0 && al(gu, 16)));
  QLORA_CHECK_ARG(K % (kStages * kBK) == 0 && (K / kBK64) % stages == 0);
  if (swiglu_epi(epi)) QLORA_CHECK_ARG(N % (tile / 2) == 0);  // N = I (output columns)
  else QLORA_CHECK_ARG(mode == 0 ? N % 8 == 0 : N % tile == 0);  // NT: a partial last tile
  QLORA_CHECK_ARG(lda >= K && lda % 8 == 0 && al(a, 16) && al(b, 16) && ldb % 8 == 0);
  QLORA_CHECK_ARG(mode == 0 ? ldb >= K : ldb >= N);
  QLORA_CHECK_ARG(ldc >= N);
  // the DMA addresses rows by 32-bit byte offsets: from B's start (NT), from a tile (A, NN B)
  if (mode == 0) QLORA_CHECK_ARG((swiglu_epi(epi) ? 2 * N : N) * ldb * 2 < (1ll << 32));
  QLORA_CHECK_ARG((int64_t)tile * lda * 2 < (1ll << 32) && 64 * ldb * 2 < (1ll << 32));
  GemmArgs g{};
  g.a = static_cast<const uint16_t*>(a);
  g.lda = lda;
  g.b = static_cast<const uint16_t*>(b);
  g.ldb = ldb;
  g.c = c;
  g.ldc = ldc;
  g.bias = static_cast<const uint16_t*>(bias);
  g.resid = resid;
  g.ldr = ldr;
  g.M = M;
  g.N = N;
  g.Kr = K;
  g.I = swiglu_I;
  g.gu = static_cast<uint16_t*>(gu);
  g.ldgu = ldgu;
  if (rest > 0) {
    // the leading n_first output columns on 256 x 256 tiles in whole rounds, the rest on
    // 128 x 128 tiles (NT: W rows n_first.., SwiGLU's up rows I + n_first..; NN: B's columns)
    GemmArgs g2 = g;
    g.N = n_first;
    if (int rc = run_gemm(g, kBHalf, mode, epi, 1, nullptr, 0, (hipStream_t)stream,
                          static_cast<hipEvent_t>(start), nullptr, 256, 2))
      return rc;
    g2.N = N - n_first;
    g2.b += mode == 0 ? n_first * ldb : n_first;
    g2.c = static_cast<char*>(c) + n_first * (epi == kEpiResid ? 4 : 2);
    if (g2.bias) g2.bias += n_first;
    if (g2.resid) g2.resid += n_first;
    if (g2.gu) g2.gu += n_first;
    return run_gemm(g2, kBHalf, mode, epi, 1, nullptr, 0, (hipStream_t)stream, nullptr,
                    static_cast<hipEvent_t>(stop), 128, rest);
  }
  return run_gemm(g, kBHalf, mode, epi, splits, ws, ws_elems, (hipStream_t)stream,
                  static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop), tile, stages);
}

QLORA_API int qlora_gemm16(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M,
                           int64_t N, int64_t K, int32_t mode, void* c, int64_t ldc,
                           const void* bias, const float* resid, int64_t ldr, int32_t epi,
                           int64_t swiglu_I, void* gu, int64_t ldgu, int32_t tile,
                           int32_t stages, int32_t splits, float* ws, int64_t ws_elems,
                           void* stream) {
  return qlora_gemm16_timed(a, lda, b, ldb, M, N, K, mode, c, ldc, bias, resid, ldr, epi,
                            swiglu_I, gu, ldgu, tile, stages, splits, ws, ws_elems, stream,
                            nullptr, nullptr);
}

// The K slices of a split-K product left unsummed: ws [splits, M, N] fp32, slice k the sum over
// its k-tiles, for a consumer that sums them itself in slice order (qlora_rms_bwd dy_parts).
QLORA_API int qlora_gemm16_parts(const void* a, int64_t lda, const void* b, int64_t ldb,
                                 int64_t M, int64_t N, int64_t K, int32_t mode, int32_t tile,
                                 int32_t stages, int32_t splits, float* ws, int64_t ws_elems,
                                 void* stream) {
  QLORA_CHECK_ARG(M > 0 && N > 0 && K > 0 && a && b && ws && (mode == 0 || mode == 1));
  QLORA_CHECK_ARG((tile == 256 && stages == 2) || (tile == 128 && (stages == 2 || stages == 4)));
  QLORA_CHECK_ARG(splits >= 2 && splits <= 16);
  QLORA_CHECK_ARG(K % (kStages * kBK) == 0 && (K / kBK64) % stages == 0);
  QLORA_CHECK_ARG(mode == 0 ? N % 8 == 0 : N % tile == 0);
  QLORA_CHECK_ARG(lda >= K && lda % 8 == 0 && al(a, 16) && al(b, 16) && ldb % 8 == 0);
  QLORA_CHECK_ARG(mode == 0 ? ldb >= K : ldb >= N);
  if (mode == 0) QLORA_CHECK_ARG(N * ldb * 2 < (1ll << 32));
  QLORA_CHECK_ARG((int64_t)tile * lda * 2 < (1ll << 32) && 64 * ldb * 2 < (1ll << 32));
  GemmArgs g{};
  g.a = static_cast<const uint16_t*>(a);
  g.lda = lda;
  g.b = static_cast<const uint16_t*>(b);
  g.ldb = ldb;
  g.c = ws;
  g.ldc = N;
  g.M = M;
  g.N = N;
  g.Kr = K;
  return run_gemm(g, kBHalf, mode, kEpiStore, splits, ws, ws_elems, (hipStream_t)stream,
                  nullptr, nullptr, tile, stages, true);
}

// The fp32-output GEMM: c = alpha A op(B) (+ row-scaled resid), mode 1 A [M, K] x B [K, N],
// mode 2 A^T: A stored [K, M] (lda >= M), B [K, N].
QLORA_API int qlora_gemm16_f32(const void* a, int64_t lda, const void* b, int64_t ldb,
                               int64_t M, int64_t N, int64_t K, int32_t mode, float* c,
                               int64_t ldc, float alpha, const float* row_scale,
                               const float* resid, int64_t ldr, int32_t tile, int32_t stages,
                               int32_t splits, float* ws, int64_t ws_elems, void* stream) {
  QLORA_CHECK_ARG(M >= 0 && N > 0 && K > 0);
  if (M == 0) return 0;
  QLORA_CHECK_ARG(a && b && c && (mode == 1 || mode == 2) && (tile == 0) == (splits == 0));
  QLORA_CHECK_ARG(row_scale == nullptr || resid != nullptr);
  if (tile == 0) auto_plan(M, N, K, mode, kEpiF32, &tile, &stages, &splits);
  QLORA_CHECK_ARG((tile == 256 && stages == 2) || (tile == 128 && (stages == 2 || stages == 4)));
  QLORA_CHECK_ARG(splits >= 1 && splits <= 16);
  QLORA_CHECK_ARG(K % (kStages * kBK) == 0 && (K / kBK64) % stages == 0 && N % tile == 0);
  QLORA_CHECK_ARG(mode == 1 ? lda >= K : (lda >= M && M % tile == 0));
  QLORA_CHECK_ARG(lda % 8 == 0 && al(a, 16) && al(b, 16) && ldb % 8 == 0 && ldb >= N);
  QLORA_CHECK_ARG(ldc >= N && (resid == nullptr || ldr >= N));
  QLORA_CHECK_ARG(splits == 1 || ldc % 4 == 0);
  // 32-bit DMA byte offsets within a tile: A's rows (mode 1) or 64 k-rows (mode 2), B's k-rows
  QLORA_CHECK_ARG((int64_t)(mode == 1 ? tile : 64) * lda * 2 < (1ll << 32) &&
                  64 * ldb * 2 < (1ll << 32));
  GemmArgs g{};
  g.a = static_cast<const uint16_t*>(a);
  g.lda = lda;
  g.b = static_cast<const uint16_t*>(b);
  g.ldb = ldb;
  g.c = c;
  g.ldc = ldc;
  g.resid = resid;
  g.ldr = ldr;
  g.M = M;
  g.N = N;
  g.Kr = K;
  g.alpha = alpha;
  g.row_scale = row_scale;
  return run_gemm(g, kBHalf, mode, kEpiF32, splits, ws, ws_elems, (hipStream_t)stream, nullptr,
                  nullptr, tile, stages);
}

// fp32 workspace elements of a qlora_gemm16 / qlora_gemm16_f32 (epi 6) problem: the split-K
// partials, or with one slice the tail split's (0 when the last round needs none).
QLORA_API int qlora_gemm16_workspace(int64_t M, int64_t N, int64_t K, int32_t mode, int32_t epi,
                                     int32_t tile, int32_t stages, int32_t splits,
                                     int64_t* elems) {
  QLORA_CHECK_ARG(elems && M >= 0 && N > 0 && K > 0 && splits >= 0 && epi >= 0 && epi <= 6 &&
                  epi != kEpiPartial);
  QLORA_CHECK_ARG((tile == 0) == (splits == 0) && mode >= 0 && mode <= 2);
  QLORA_CHECK_ARG((mode == 2) <= (epi == kEpiF32) && (epi == kEpiF32) <= (mode != 0));
  *elems = 0;
  if (M == 0) return 0;
  int rest = 0;
  int64_t n_first = 0;
  if (tile == 0) auto_plan(M, N, K, mode, epi, &tile, &stages, &splits, &rest, &n_first);
  if (rest > 0) return 0;
  QLORA_CHECK_ARG((tile == 256 && stages == 2) || (tile == 128 && (stages == 2 || stages == 4)));
  if (splits > 1) {
    *elems = (int64_t)splits * M * N;
    return 0;
  }
  if (M == 0 || K % (kStages * kBK) != 0 || !tail_epi(epi)) return 0;
  int main_t, tail_s, kt_tail;
  *elems = tail_plan(qlora_cdiv(M, tile), n_tiles_of(N, epi, tile), K / kBK64, tile, stages,
                     &main_t, &tail_s, &kt_tail);
  return 0;
}

// The plan of qlora_gemm16 with tile 0 and splits 0 in full: the first launch's (tile, stages,
// splits) and, when the remaining output columns run as a second launch on 128 x 128 tiles, that
// launch's stage count (rest, else 0) and the first launch's output columns (n_first).
QLORA_API int qlora_gemm16_plan_split(int64_t M, int64_t N, int64_t K, int32_t mode, int32_t epi,
                                      int32_t* tile, int32_t* stages, int32_t* splits,
                                      int32_t* rest, int64_t* n_first) {
  QLORA_CHECK_ARG(tile && stages && splits && rest && n_first && M >= 0 && N > 0 && K > 0);
  QLORA_CHECK_ARG(mode >= 0 && mode <= 1 && epi >= 0 && epi <= 5 && epi != kEpiPartial);
  int t, st, sp, r;
  int64_t nf;
  auto_plan(M, N, K, mode, epi, &t, &st, &sp, &r, &nf);
  *tile = t;
  *stages = st;
  *splits = sp;
  *rest = r;
  *n_first = nf;
  return 0;
}

// The (tile, stages, splits) qlora_gemm16 runs with tile 0 and splits 0 (its first launch's).
QLORA_API int qlora_gemm16_plan(int64_t M, int64_t N, int64_t K, int32_t mode, int32_t epi,
                                int32_t* tile, int32_t* stages, int32_t* splits) {
  QLORA_CHECK_ARG(tile && stages && splits && M >= 0 && N > 0 && K > 0);
  QLORA_CHECK_ARG(mode >= 0 && mode <= 2 && epi >= 0 && epi <= 6 && epi != kEpiPartial);
  QLORA_CHECK_ARG((mode == 2) <= (epi == kEpiF32) && (epi == kEpiF32) <= (mode != 0));
  int t, st, sp, r;
  int64_t nf;
  auto_plan(M, N, K, mode, epi, &t, &st, &sp, epi == kEpiF32 ? nullptr : &r, &nf);
  *tile = t;
  *stages = st;
  *splits = sp;
  return 0;
}
