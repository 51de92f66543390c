// Standalone NF4 -> fp16 dequantisation (reference: nf4_dequant_kernel, kernels.py:68-105;
// launched by NF4Weight.dequant_into / NF4Group.dequant_into, engine.py:103-157, and by
// dequant(), engine.py:683-694, for several weights at once).
//
// HBM-bound: per 8 output values one 32-bit word of nibbles is read and 16 bytes are written.
// One launch covers up to kMaxJobs weights (a layer's qkv, o, gate|up and down: 23 MB read and
// 94 MB written; or the weights of eight layers at once), so the launch cost and the tail of one
// weight overlap the next.
// Each thread handles kWPT words spaced a workgroup apart: every load and every 16-byte store instruction of a wavefront covers one contiguous
// span (256 B in, 1 KiB out). All loads are unconditional (indices clamped, results masked), so
// a thread's loads issue back to back. The 16 levels and the 256-entry double-quant code sit in
// LDS; the per-block absmax byte and absmax2 are shared by the 8 consecutive lanes of a block.
#include "nf4.h"

#include <hip/hip_ext.h>

namespace qlora {

constexpr int kDequantThreads = 256;
constexpr int kMaxJobs = 32;  // the batch stays within the 4 KiB of kernel arguments

struct DequantJob {
  NF4Ref w;
  uint4* out;
  int64_t n_words;
};

struct DequantBatch {
  DequantJob job[kMaxJobs];
  int32_t first_tile[kMaxJobs + 1];  // workgroup ranges of the jobs (< 2^31)
  int count;
};
static_assert(sizeof(DequantBatch) <= 4096, "kernel arguments");

// kWPT words per thread: 8 for large launches, fewer when that would leave CUs without work.
template <int kWPT>
__global__ __launch_bounds__(kDequantThreads) void nf4_dequant_kernel(DequantBatch b) {
  constexpr int kTileWords = kDequantThreads * kWPT;
  __shared__ float lut[16];
  __shared__ float c2[256];
  __shared__ float offs[3];
  // the job of this workgroup: the number of later jobs' first tiles at or before it. A count
  // over fixed offsets: its scalar loads issue together (a search would chain one round trip per
  // step before the first data load). Entries past count hold the total, which no tile reaches;
  int j = 0;
#pragma unroll
  for (int i = 1; i < kMaxJobs; ++i) j += (int)blockIdx.x >= b.first_tile[i] ? 1 : 0;
  const DequantJob job = b.job[j];  // by value: its fields are loaded once
  const NF4Ref& w = job.w;
  const int t = threadIdx.x;
  // the words and their block scales' inputs first (their latency then overlaps the table fill)
  const uint32_t* words = reinterpret_cast<const uint32_t*>(w.packed);
  const int64_t base = ((int64_t)blockIdx.x - b.first_tile[j]) * kTileWords + t;
  const int64_t last = job.n_words - 1;
  const int wshift = w.bs1_shift - 3;  // words per block = bs1 / 8
  uint32_t v[kWPT], q[kWPT];
  float a2[kWPT];
#pragma unroll
  for (int i = 0; i < kWPT; ++i) {
    int64_t idx = base + i * kDequantThreads;
    idx = idx < last ? idx : last;
    v[i] = __builtin_nontemporal_load(words + idx);
    const int64_t blk = idx >> wshift;
    if (w.nested) {
      q[i] = static_cast<const uint8_t*>(w.absmax)[blk];
      a2[i] = w.absmax2[blk >> w.bs2_shift];
    } else {
      q[i] = 0;
      a2[i] = static_cast<const float*>(w.absmax)[blk];
    }
  }
  if (t < 16) lut[t] = w.standard ? kNF4Levels[t] : w.code[t];
  if (w.nested) {
    c2[t] = w.code2[t];  // 256 threads, 256 entries
    if (t < 3) {
      const int nseg = 1 + (int)(w.seg1 != INT64_MAX) + (int)(w.seg2 != INT64_MAX);
      offs[t] = w.offsets[t < nseg ? t : 0];
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kWPT; ++i) {
    const int64_t idx = base + i * kDequantThreads;
    float scale = a2[i];
    if (w.nested) {
      const int64_t blk = idx >> wshift;
      float prod = c2[q[i]] * a2[i];  // rounded before the offset is added (bitsandbytes)
      fp32_barrier(prod);
      scale = prod + offs[(int)(blk >= w.seg1) + (int)(blk >= w.seg2)];
    }
    const uint4 r = nf4_decode_word(v[i], scale, lut);
    if (idx <= last) job.out[idx] = r;
  }
}

}  // namespace qlora

using namespace qlora;

namespace {

int make_job(DequantJob& job, const void* packed, const void* absmax, const float* code2,
             const float* absmax2, const float* offsets, const float* code, void* out,
             int64_t n_blocks, int32_t nested, int32_t standard, int32_t bs1, int32_t bs2,
             int64_t seg1, int64_t seg2) {
  QLORA_CHECK_ARG(n_blocks >= 0);
  job = DequantJob{};
  if (n_blocks == 0) return 0;  // nothing to read or write: no other argument is looked at
  QLORA_CHECK_ARG(packed && absmax && out);
  QLORA_CHECK_ARG(bs1 >= 8 && (bs1 & (bs1 - 1)) == 0);
  QLORA_CHECK_ARG(!nested || (code2 && absmax2 && offsets && bs2 > 0 && (bs2 & (bs2 - 1)) == 0));
  QLORA_CHECK_ARG(standard || code);
  QLORA_CHECK_ARG(((uintptr_t)packed & 3) == 0 && ((uintptr_t)out & 15) == 0);
  job.w = NF4Ref{static_cast<const uint8_t*>(packed), absmax, code2, absmax2, offsets, code,
                 seg1, seg2, __builtin_ctz(bs1), nested ? __builtin_ctz(bs2) : 0, nested,
                 standard};
  job.out = static_cast<uint4*>(out);
  job.n_words = n_blocks * (bs1 / 8);
  return 0;
}

// start/stop (may be null): events recorded by the dispatch itself at the kernel's start and end
// (hipExtLaunchKernelGGL), i.e. the kernel's own duration without the launch gap.
template <int kWPT>
int launch_wpt(DequantBatch& b, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  constexpr int64_t kTileWords = kDequantThreads * kWPT;
  int64_t tiles = 0;
  for (int i = 0; i < b.count; ++i) tiles += qlora_cdiv(b.job[i].n_words, kTileWords);
  QLORA_CHECK_ARG(tiles < (1ll << 31));
  tiles = 0;
  for (int i = 0; i < b.count; ++i) {
    b.first_tile[i] = (int32_t)tiles;
    tiles += qlora_cdiv(b.job[i].n_words, kTileWords);
  }
  for (int i = b.count; i <= kMaxJobs; ++i) b.first_tile[i] = (int32_t)tiles;
  if (start != nullptr || stop != nullptr)
    hipExtLaunchKernelGGL(nf4_dequant_kernel<kWPT>, dim3((unsigned)tiles),
                          dim3(kDequantThreads), 0, stream, start, stop, 0, b);
  else
    hipLaunchKernelGGL(nf4_dequant_kernel<kWPT>, dim3((unsigned)tiles), dim3(kDequantThreads),
                       0, stream, b);
  return qlora_launch_status();
}

int launch(DequantBatch& b, hipStream_t stream, hipEvent_t start = nullptr,
           hipEvent_t stop = nullptr) {
  // drop empty jobs, then lay the workgroups of the rest end to end
  int k = 0;
  int64_t words = 0;
  for (int i = 0; i < b.count; ++i)
    if (b.job[i].n_words > 0) {
      words += b.job[i].n_words;
      b.job[k++] = b.job[i];
    }
  b.count = k;
  if (k == 0) return 0;
  // at least ~2048 workgroups (8 per CU) when the launch is big enough for that
  constexpr int64_t kTarget = 2048 * kDequantThreads;
  if (words >= 8 * kTarget) return launch_wpt<8>(b, stream, start, stop);
  if (words >= 4 * kTarget) return launch_wpt<4>(b, stream, start, stop);
  if (words >= 2 * kTarget) return launch_wpt<2>(b, stream, start, stop);
  return launch_wpt<1>(b, stream, start, stop);
}

}  // namespace

QLORA_API int qlora_nf4_dequant(const void* packed, const void* absmax, const float* code2,
                                const float* absmax2, const float* offsets, const float* code,
                                void* out, int64_t n_blocks, int32_t nested, int32_t standard,
                                int32_t bs1, int32_t bs2, int64_t seg1, int64_t seg2,
                                void* stream) {
  DequantBatch b{};
  b.count = 1;
  if (int rc = make_job(b.job[0], packed, absmax, code2, absmax2, offsets, code, out, n_blocks,
                        nested, standard, bs1, bs2, seg1, seg2))
    return rc;
  return launch(b, (hipStream_t)stream);
}

// Up to 32 weights in one launch (a layer's four, or those of eight layers): argument arrays of
// length `count`, entry i as in qlora_nf4_dequant.
// qlora_nf4_dequant_many that also records two events at the kernel's own start and end (the
// dispatch timestamps rocprof reads), for callers that time the kernel without its launch gap.
// start/stop: hipEvent_t created with timing, or null. No reference counterpart (measurement).
QLORA_API int qlora_nf4_dequant_many_timed(int32_t count, const void* const* packed,
                                           const void* const* absmax, const float* const* code2,
                                           const float* const* absmax2,
                                           const float* const* offsets, const float* const* code,
                                           void* const* out, const int64_t* n_blocks,
                                           const int32_t* nested, const int32_t* standard,
                                           const int32_t* bs1, const int32_t* bs2,
                                           const int64_t* seg1, const int64_t* seg2,
                                           void* stream, void* start, void* stop);

QLORA_API int qlora_nf4_dequant_many(int32_t count, const void* const* packed,
                                     const void* const* absmax, const float* const* code2,
                                     const float* const* absmax2, const float* const* offsets,
                                     const float* const* code, void* const* out,
                                     const int64_t* n_blocks, const int32_t* nested,
                                     const int32_t* standard, const int32_t* bs1,
                                     const int32_t* bs2, const int64_t* seg1,
                                     const int64_t* seg2, void* stream) {
  return qlora_nf4_dequant_many_timed(count, packed, absmax, code2, absmax2, offsets, code, out,
                                      n_blocks, nested, standard, bs1, bs2, seg1, seg2, stream,
                                      nullptr, nullptr);
}

QLORA_API int qlora_nf4_dequant_many_timed(int32_t count, const void* const* packed,
                                           const void* const* absmax, const float* const* code2,
                                           const float* const* absmax2,
                                           const float* const* offsets, const float* const* code,
                                           void* const* out, const int64_t* n_blocks,
                                           const int32_t* nested, const int32_t* standard,
                                           const int32_t* bs1, const int32_t* bs2,
                                           const int64_t* seg1, const int64_t* seg2,
                                           void* stream, void* start, void* stop) {
  QLORA_CHECK_ARG(count >= 0 && count <= kMaxJobs);
  QLORA_CHECK_ARG(count == 0 || (packed && absmax && code2 && absmax2 && offsets && code &&
                                 out && n_blocks && nested && standard && bs1 && bs2 && seg1 &&
                                 seg2));
  DequantBatch b{};
  b.count = count;
  for (int i = 0; i < count; ++i)
    if (int rc = make_job(b.job[i], packed[i], absmax[i], code2[i], absmax2[i], offsets[i],
                          code[i], out[i], n_blocks[i], nested[i], standard[i], bs1[i], bs2[i],
                          seg1[i], seg2[i]))
      return rc;
  return launch(b, (hipStream_t)stream, static_cast<hipEvent_t>(start),
                static_cast<hipEvent_t>(stop));
}
