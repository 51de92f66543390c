/*
 * C-ABI of the MI355X (gfx950) QLoRA training-step kernels: libqlora_amd.so.
 *
 * Every entry point takes raw device pointers, sizes and scalars, launches on the given HIP
 * stream (hipStream_t passed as void*; NULL = the default stream) and returns 0 on success or a
 * hipError_t (hipErrorInvalidValue = 1 for arguments a kernel cannot take; checked before any
 * launch). Kernels allocate nothing: callers pass every output and workspace. The library keeps
 * this process-wide state, each created on first use per device and kept until the process ends:
 *   - one second stream and two events per device (csrc/attn.hip), on which the attention
 *     backward runs dK/dV beside dQ; it is forked from and joined back into the caller's stream
 *     inside the call, so the call is ordered on the caller's stream as any other;
 *   - the 16 MiB static device array of qlora_lora_grad_noalloc (csrc/lora.hip), one per device
 *     for the life of the process, and its address per device.
 * Entry points are callable from any thread; the state above is created under a lock.
 * n == 0 (rows, tokens, blocks) is a no-op that returns 0, as the reference skips such launches.
 *
 * Dtypes: "f16" = IEEE half as 16-bit words, "f32" = float, "i64"/"i32" = int64_t/int32_t.
 * All tensors are contiguous row-major unless a leading dimension is given.
 *
 * Each entry point replaces one Triton kernel launch of the reference (Magurin/hack-fe30cb28 -
 * solution/kernels.py), called through the Python wrappers of solution/engine.py; the citation
 * is given as kernel (file:line) <- wrapper (file:line).
 */
#ifndef QLORA_AMD_H
#define QLORA_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Library version of this ABI (1). */
int qlora_abi_version(void);
/* hipGetErrorString of a returned code. */
const char* qlora_error_string(int code);

/*
 * NF4 -> fp16 dequantisation, bit-exact with bitsandbytes' dequantize_4bit.
 * Replaces nf4_dequant_kernel (kernels.py:68-105) <- NF4Weight.dequant_into
 * (engine.py:103-109), NF4Group.dequant_into (engine.py:148-157), dequant (engine.py:683-694).
 *   packed   u8 [n_blocks*bs1/2], element i = high nibble of byte i/2 for even i, low for odd
 *   absmax   nested: u8 [n_blocks] codes into code2; else f32 [n_blocks]
 *   code2    f32 [256]; absmax2 f32 [ceil(n_blocks/bs2)]; offsets f32 [1..3] (nested only)
 *   code     f32 [16] levels, read only when standard == 0 (else the NF4 table)
 *   out      f16 [n_blocks*bs1]
 *   seg1/2   first block of the 2nd/3rd weight stacked back to back (INT64_MAX if none): they
 *            select offsets[1] / offsets[2]
 * Requires bs1 >= 8 and bs1, bs2 powers of two; packed 4-byte and out 16-byte aligned.
 */
int qlora_nf4_dequant(const void* packed, const void* absmax, const float* code2,
                      const float* absmax2, const float* offsets, const float* code, void* out,
                      int64_t n_blocks, int32_t nested, int32_t standard, int32_t bs1,
                      int32_t bs2, int64_t seg1, int64_t seg2, void* stream);

/*
 * NF4 quantisation on the GPU in bitsandbytes' Params4bit layout (the load-time step before the
 * path: the bytes engine.py:77-101 reads; restates bitsandbytes 0.50.2 quantize_4bit): per block
 * of 64 elements of w (fp16, or fp32 if w_f32; n_blocks x 64, row-major flat) absmax f32 =
 * max |w| and code = the NF4 decision tree on fp32 midpoints of w * (1 / absmax), two codes a byte
 * (even element high) in packed u8 [n_blocks * 32]. w 4-byte (fp16) / 8-byte (fp32) aligned.
 */
int qlora_nf4_quantize(const void* w, int32_t w_f32, int64_t n_blocks, void* packed,
                       float* absmax, void* stream);
/*
 * Its double quantisation (compress_statistics): offset = fp32(fp64 tree sum of the n absmax /
 * n), then per 256 values absmax2 = max |a - offset| and q u8 = bitsandbytes' dQuantize of
 * (a - offset) / absmax2 over code2 (its signed dynamic map, f32 [256], sorted). work: fp64 of
 * qlora_nf4_quantize_stats_workspace elements; absmax2 f32 [ceil(n / 256)], offset f32 [1].
 */
int qlora_nf4_quantize_stats_workspace(int64_t n, int64_t* elems);
int qlora_nf4_quantize_stats(const float* absmax, int64_t n, const float* code2, double* work,
                             int64_t work_elems, uint8_t* q, float* absmax2, float* offset,
                             void* stream);

/*
 * Keep mask (i8 0/1) of elements 0..nelem of one PyTorch dropout call whose Philox state is
 * (seed, offset = 4*ctr) over G threads, vec elements per thread load (4 fp32, 8 fp16).
 * Replaces torch_dropout_keep_kernel (kernels.py:129-135), the test hook of
 * test_kernels.py:52-60.
 */
int qlora_dropout_keep(int8_t* out, int64_t nelem, int64_t seed, int64_t ctr, int64_t G,
                       float p_keep, int32_t vec, void* stream);

/*
 * Host only (no GPU call): the keep threshold every dropout kernel of the library uses, the
 * smallest Philox word whose uniform 2^-32 + r 2^-32 (fp32) is not below p_keep; words below
 * it are kept (the compare of _torch_dropout_keep, kernels.py:108-126, made an integer one).
 */
int qlora_dropout_keep_below(float p_keep, uint32_t* out);

/*
 * RMSNorm forward over n rows of H: [x += f32(delta); xsum = x], rstd = 1/sqrt(mean(x^2)+eps),
 * y = w * (x * rstd) -> f16, and the LoRA inputs yq / yv = f16(keep ? y * keep_scale : 0) with
 * the keep masks of two dropout calls (counters ctr_q, ctr_v) at padded-batch elements
 * tok[row]*H + col (below 2^32). Replaces rms_fwd_kernel (kernels.py:145-175) <- _rms_fwd
 * (engine.py:947-966).
 *   x f32 [n,H]; delta f16 [n,H]; w [H] (f32, or f16 if w_half); xsum f32 [n,H];
 *   y, yq, yv f16 [n,H]; rstd f32 [n]; tok i64 [n]
 *   keep (may be null) u8 [n][2][ceil(H/4)]: with dropout, the masks stored as bits (bit k of
 *   byte j of mask m = element 4j+k kept; m = 0 for yq, 1 for yv) for qlora_rms_bwd to read
 *   instead of drawing them again (no reference counterpart: the reference draws them twice).
 *   keep_in (may be null; not with keep) u8 [n][2][ceil(H/4)]: with dropout, the masks read
 *   from bits an earlier call over the same rows stored (a recompute), not drawn (no reference
 *   counterpart).
 *   ctr_base (may be null) i64 [1] on the device: added to ctr_q and ctr_v (a step captured in
 *   a HIP graph passes its counters relative to the step's first, kept there; no reference
 *   counterpart).
 */
int qlora_rms_fwd(const float* x, const void* delta, const void* w, int32_t w_half, float* xsum,
                  void* y, void* yq, void* yv, float* rstd, const int64_t* tok, int64_t n,
                  int64_t H, float eps, float p_keep, float keep_scale, int64_t seed,
                  int64_t ctr_q, int64_t ctr_v, int64_t G, int32_t has_delta, int32_t write_y,
                  int32_t drop_q, int32_t drop_v, int32_t vec, uint8_t* keep,
                  const uint8_t* keep_in, const int64_t* ctr_base, void* stream);

/*
 * RMSNorm backward: g = w * (dy + keep_q * tq * keep_scale + keep_v * tv * keep_scale),
 * dx = [dres +] grad_scale * rstd * (g - xhat * mean(g * xhat)), xhat = x * rstd.
 * Replaces rms_bwd_kernel (kernels.py:178-205) <- _rms_bwd (engine.py:969-981).
 *   dy f16 [n, dy_stride]; tq, tv f16 [n,H]; x f32 [n,H]; rstd f32 [n]; dres, dx f32 [n,H];
 *   dx16 (optional, may be null) f16 [n,H] = fp16(dx), the operand of the next dY W product
 *   (engine.py:1238 and 1301 round the gradient to fp16 before it).
 *   keep (may be null) u8 [n][2][ceil(H/4)]: the masks qlora_rms_fwd stored for these rows
 *   (same tok, seed, counters and drop_q/drop_v); null: drawn again from (seed, ctr_q, ctr_v).
 *   ctr_base (may be null): as qlora_rms_fwd's.
 *   xdelta (may be null) f16 [n,H]: the forward normed x + f32(xdelta) (qlora_rms_fwd with
 *   delta); the kernel forms that sum and rstd = 1/sqrt(mean(x^2)+eps) again in the forward's
 *   order of operations (the same bits) and does not read rstd (may then be null). No reference
 *   counterpart: a recompute's post-attention norm folded into its backward.
 *   dy_parts (may be null; not with dropout) f32 [nparts, n, H]: dy = fp16 of the parts summed
 *   in order (the K slices of qlora_gemm16_parts: the split-K reduce folded in, the same bits);
 *   dy is then not read (may be null). No reference counterpart.
 */
int qlora_rms_bwd(const void* dy, const void* tq, const void* tv, const float* x,
                  const float* rstd, const void* w, int32_t w_half, const float* dres, float* dx,
                  void* dx16, const int64_t* tok, int64_t n, int64_t H, int64_t dy_stride,
                  float p_keep, float keep_scale, int64_t seed, int64_t ctr_q, int64_t ctr_v,
                  int64_t G, float grad_scale, int32_t drop_q, int32_t drop_v, int32_t has_res,
                  int32_t vec, const uint8_t* keep, const int64_t* ctr_base, const void* xdelta,
                  float eps, const float* dy_parts, int32_t nparts, void* stream);

/*
 * qkv split + LoRA deltas + rotate-half RoPE. q = f16(rope(qkv_q + s*lq)),
 * k = f16(rope(qkv_k)), v = f16(qkv_v + s*lv); cos/sin f32 [positions, D/2] at pos[t].
 * k, v are written with kv_heads_out heads: HKV, or HQ (each kv head repeated HQ/HKV times).
 * A position outside [0, positions) yields NaN for that token (no out-of-bounds table read).
 * Replaces qkv_rope_fwd_kernel (kernels.py:212-264) <- _rope_fwd (engine.py:984-997).
 *   qkv f16 [n,(HQ+2HKV)*D]; lq f16 [n,HQ*D] or NULL; lv f16 [n,HKV*D] or NULL; pos i32 [n]
 *   q f16 [n,HQ,D]; k, v f16 [n,kv_heads_out,D]. Requires D % 16 == 0, 16-byte alignment.
 */
int qlora_rope_fwd(const void* qkv, const void* lq, const void* lv, const float* cos,
                   const float* sin, int64_t positions, const int32_t* pos, void* q, void* k,
                   void* v, int64_t n, int32_t HQ, int32_t HKV, int32_t D, int32_t kv_heads_out,
                   float lora_scale, void* stream);

/*
 * Inverse: dqkv = [rope^-1(dq) | rope^-1(sum_g dk) | sum_g dv] f16 [n,(HQ+2HKV)*D], where
 * dk, dv have kv_heads_in heads (HQ: summed over each kv head's replicas in fp32).
 * Replaces qkv_rope_bwd_kernel (kernels.py:267-306) <- _rope_bwd (engine.py:1000-1009).
 */
int qlora_rope_bwd(const void* dq, const void* dk, const void* dv, const float* cos,
                   const float* sin, int64_t positions, const int32_t* pos, void* dqkv,
                   int64_t n, int32_t HQ, int32_t HKV, int32_t D, int32_t kv_heads_in,
                   void* stream);

/*
 * SwiGLU: m = f16(silu(g) * u), gu = [g | u] f16 [n, 2I], m f16 [n, I].
 * Replaces glu_fwd_kernel (kernels.py:312-321) <- _glu_fwd (engine.py:1012-1017).
 */
int qlora_glu_fwd(const void* gu, void* m, int64_t n, int64_t I, void* stream);

/*
 * SwiGLU backward in place: gu <- [dm*u*s*(1+g(1-s)) | dm*g*s], s = sigmoid(g).
 * Replaces glu_bwd_kernel (kernels.py:324-336) <- _glu_bwd (engine.py:1020-1023).
 */
int qlora_glu_bwd(const void* dm, void* gu, int64_t n, int64_t I, void* stream);

/*
 * Cross-entropy over whole rows of f16 logits [rows, V] (leading dimension ld), in place:
 * loss (f32, 0 if target < 0), entropy (f32), correct (i32, argmax == target, first max wins);
 * rows with a target get f16(softmax - onehot) written over their logits, the others zeros if
 * zero_unsupervised. Replaces lm_head_ce_kernel (kernels.py:344-388) <- _ce
 * (engine.py:1026-1030).
 */
int qlora_ce(void* logits, int64_t ld, const int64_t* target, float* loss, float* entropy,
             int32_t* correct, int64_t rows, int64_t V, int32_t zero_unsupervised,
             void* stream);

/*
 * One vocabulary piece [v0, v0+width) of the online cross-entropy: updates state f32 [rows,4]
 * (max, sum exp, sum exp*x, best), best_idx i32 [rows], xt f32 [rows] (target logit if in the
 * piece); for rows < n_sup writes alpha f32 [n_sup] = exp(m_old - m_new) and overwrites their
 * logits with f16(exp(x - m_new)); copies w[target - v0] (f16 [width, H]) into wt f16 [n_sup,H].
 * Replaces lm_head_piece_kernel (kernels.py:401-450) <- _ce_piece (engine.py:1033-1038).
 */
int qlora_ce_piece(void* logits, int64_t ld, const void* w, const int64_t* target, float* state,
                   int32_t* best_idx, float* xt, float* alpha, void* wt, int64_t v0,
                   int64_t rows, int64_t width, int64_t n_sup, int64_t H, void* stream);

/*
 * After the last piece: loss, entropy, correct as qlora_ce; dh f16 [n_sup,H] = acc/s - wt.
 * Replaces lm_head_finish_kernel (kernels.py:458-479) <- _ce_finish (engine.py:1041-1045).
 */
int qlora_ce_finish(const float* state, const int32_t* best_idx, const float* xt,
                    const int64_t* target, float* loss, float* entropy, int32_t* correct,
                    const float* acc, const void* wt, void* dh, int64_t rows, int64_t n_sup,
                    int64_t H, void* stream);

/*
 * Embedding-gradient pass of the chunked head (no reference counterpart: the reference's
 * embedding is frozen; BASELINE config 4 asks for dE): after qlora_ce_finish, the recomputed
 * logits of one piece, rows < n_sup (f16, row stride ld, columns [v0, v0 + width) of the
 * vocabulary) are overwritten in place with f16(e^(x - lse) - onehot(target)), lse = m + log s
 * from the finished state f32 [rows, 4]. Equal bit for bit to the same columns of qlora_ce's
 * in-place gradient.
 */
int qlora_ce_grad(void* logits, int64_t ld, const int64_t* target, const float* state,
                  int64_t v0, int64_t n_sup, int64_t width, void* stream);

/*
 * Up to 32 weights in one launch (a layer's qkv, o, gate|up and down, or the weights of eight
 * layers): arrays of `count` entries, entry i exactly the arguments of one qlora_nf4_dequant
 * call (pointer arrays and value arrays live in host memory; the pointers they hold are device
 * pointers). Replaces the per-weight launches of dequant() (engine.py:683-694) for whole layers.
 */
int qlora_nf4_dequant_many(int32_t count, const void* const* packed, const void* const* absmax,
                           const float* const* code2, const float* const* absmax2,
                           const float* const* offsets, const float* const* code,
                           void* const* out, const int64_t* n_blocks, const int32_t* nested,
                           const int32_t* standard, const int32_t* bs1, const int32_t* bs2,
                           const int64_t* seg1, const int64_t* seg2, void* stream);

/*
 * qlora_nf4_dequant_many that also records start/stop (hipEvent_t created with timing, or null)
 * at the kernel's own start and end (the dispatch's timestamps, as a profiler reads them, without
 * the launch gap an event pair around the call also measures). No reference counterpart: the
 * bench's per-launch timing of the step's dequant.
 */
int qlora_nf4_dequant_many_timed(int32_t count, const void* const* packed,
                                 const void* const* absmax, const float* const* code2,
                                 const float* const* absmax2, const float* const* offsets,
                                 const float* const* code, void* const* out,
                                 const int64_t* n_blocks, const int32_t* nested,
                                 const int32_t* standard, const int32_t* bs1, const int32_t* bs2,
                                 const int64_t* seg1, const int64_t* seg2, void* stream,
                                 void* start, void* stop);

/*
 * The fp32 scale of each of `blocks` 64-value NF4 blocks (nested: fp32(fp32(code2[absmax[b]] *
 * absmax2[b / bs2]) + offsets[segment(b)]), the segments as qlora_nf4_dequant's; plain: the fp32
 * absmax copied) into out [blocks]: the scale operand of qlora_nf4_gemm, bit-identical to the
 * scale qlora_nf4_dequant applies. The weights are frozen, so a caller forms it once per weight.
 * Replaces the absmax dequantisation of the reference's dequant (kernels.py:68-105,
 * engine.py:74-157), done once instead of per use.
 */
int qlora_nf4_block_scales(const void* absmax, const float* code2, const float* absmax2,
                           const float* offsets, int32_t nested, int32_t bs2, int64_t seg1,
                           int64_t seg2, int64_t blocks, float* out, void* stream);

/*
 * NF4 dequantisation fused into an fp16 MFMA GEMM (fp32 accumulation) with a frozen NF4 weight
 * W [w_rows, w_cols]: `packed` codes as qlora_nf4_dequant's, `scales` fp32 [w_rows*w_cols/64]
 * (qlora_nf4_block_scales), `code` the 16 levels (null: the NF4 table); 256 x 256 output tiles,
 * the NF4 blocks decoded into LDS inside the kernel. tiled = 1 (mode 0 only): codes and scales
 * rearranged once into the tile-major order, element (tile t, row r, k) at codes byte
 * ((t * w_cols/32 + k/32) * 256 + r) * 16 + (k%32)/2 and scale ((t * w_cols/64 + k/64) * 256 + r),
 * where tile row r is W row 256 t + r (epi 3: W row j or I + j, j = 128 t + 64 (r/128) +
 * r%64, the up row when r%128 >= 64); a DMA instruction then reads 1 KB in a row:
 *   mode 0 (NT): C[M, w_rows] = A[M, w_cols] W^T      mode 1 (NN): C[M, w_cols] = A[M, w_rows] W
 *   A f16 [M, lda].
 *   epi 0: C f16 = f16(acc);  epi 1: C f16 = f16(acc + bias[n]) (bias f16);
 *   epi 2: C f32 = resid[m, n] + f32(f16(acc)) (may alias resid);
 *   epi 3 (mode 0, SwiGLU): W = [gate; up] with gate rows [0, I) and up rows [I, 2I);
 *          C f16 [M, I] = f16(silu(f16 g) * f16 u), I = swiglu_I.
 *   splits > 1: split-K, the partial sums go through the caller's fp32 workspace ws
 *         (>= splits*M*N elements) and a reduce kernel applies the epilogue (not with epi 3).
 * The decoded weight values are bit-identical to qlora_nf4_dequant's.
 * Replaces dequant (engine.py:683-694) + the cuBLAS products at engine.py:1082 (qkv + bias),
 * 1112 (o), 1135-1165 (gate|up), 1179 (down), 1239, 1293, 1301, 1316 (dY W) and the
 * SwiGLU (kernels.py:312-321) and residual add (engine.py:1048-1051) that follow them.
 * Requires: M >= 0; bs1 == 64; mode 0: w_rows % 256 == 0 (epi 3: I % 128 == 0),
 * w_cols % 128 == 0; mode 1: w_cols % 256 == 0, w_rows % 128 == 0; lda % 8 == 0; A and packed
 * 16-byte aligned, scales 4-byte aligned; splits <= 16.
 */
int qlora_nf4_gemm(const void* a, int64_t lda, const void* packed, const float* scales,
                   const float* code, int32_t bs1, int32_t tiled, int64_t w_rows, int64_t w_cols,
                   void* c, int64_t ldc, const void* bias, const float* resid, int64_t ldr,
                   int64_t M, int32_t mode, int32_t epi, int64_t swiglu_I, int32_t splits,
                   float* ws, int64_t ws_elems, void* stream);

/*
 * The same GEMM with an fp16 B operand in memory (the dequantized projections; the lm_head):
 *   mode 0 (NT): C[M, N] = A[M, K] B^T, B [N, K] (ldb);  mode 1 (NN): C = A B, B [K, N] (ldb).
 * Output tiles of tile x tile: tile 256 (one workgroup of four 128 x 128 wavefront blocks per
 * CU) or 128 (four 64 x 64 wavefront blocks, two workgroups per CU: four times the tiles, for
 * the narrow products - N = 1536 or 2048 at a few thousand tokens). In one slice both tile
 * shapes give the same bits (each output sums its k-steps of 16 in order). stages: 2 (either
 * tile) or 4 (128 x 128 tiles only: 128 KB of LDS, one workgroup per CU, each k-tile's loads
 * issued three k-tiles ahead).
 * epi as qlora_nf4_gemm (epi 3: B = [gate; up] rows, N = I), and
 *   5 (NT, one slice): the SwiGLU of epi 3 and the product [g | u] itself, fp16 [M, 2 N] into
 *     gu (ldgu, 16-byte rows; gate column n and up column N + n), the same values a plain
 *     store of the product gives: a recomputing layer keeps it for its backward (the
 *     reference's step keeps [gate | up] rather than multiplying again: engine.py:1204-1213,
 *     430-445). gu is read for epi 5 only (else null).
 * splits > 1: split-K, fp32 partials in ws (>= splits*M*N elements), summed in a fixed order by
 * a reduce kernel that applies the epilogue (not with the SwiGLU forms). With splits == 1 a
 * 16-byte aligned ws of at least qlora_gemm16_workspace's elements lets the few tiles of a
 * last, nearly empty round of the GPU run as K slices (partials in ws, summed in slice order,
 * then the epilogue; the slice count follows the tile count and the GPU's workgroup slots: 256
 * tiles of 256, 512 of 128); a null or smaller ws runs them whole (results then differ in the
 * fp32 summation order of those tiles only).
 * tile 0 with splits 0 (and any stages): the plan of qlora_gemm16_plan_split; when it splits the
 * output columns, the first n_first run as whole rounds of 256 x 256 tiles and the rest as a
 * second launch on 128 x 128 tiles, on the same stream (the same bits as one launch of whole
 * 256 x 256 tiles without the K-sliced last round).
 * Replaces the cuBLAS products of the frozen projections after dequant (engine.py:1082, 1112,
 * 1163, 1179, 1239, 1293, 1301, 1316) and of the lm_head (engine.py:1376-1381).
 * Requires: K % (64 stages) == 0 and K % 128 == 0; mode 1: N % tile == 0; mode 0: N % 8 == 0
 * (epi 3, 5: N % (tile / 2) == 0); lda, ldb % 8 == 0; A, B 16-byte aligned.
 */
int qlora_gemm16(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M, int64_t N,
                 int64_t K, int32_t mode, void* c, int64_t ldc, const void* bias,
                 const float* resid, int64_t ldr, int32_t epi, int64_t swiglu_I, void* gu,
                 int64_t ldgu, int32_t tile, int32_t stages, int32_t splits, float* ws,
                 int64_t ws_elems, void* stream);

/*
 * The split-K form of qlora_gemm16 (epilogue 0) without its reduce: ws (16-byte aligned, at
 * least splits*M*N elements) receives the fp32 K slices [splits, M, N], slice k the sum over its
 * k-tiles, for a consumer that sums them in slice order itself (qlora_rms_bwd's dy_parts: the
 * gate|up input gradient, engine.py:1293, feeding the post-attention norm's backward). tile,
 * stages as qlora_gemm16 (splits >= 2). No reference counterpart (the reduce moved into the
 * consumer).
 */
int qlora_gemm16_parts(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M,
                       int64_t N, int64_t K, int32_t mode, int32_t tile, int32_t stages,
                       int32_t splits, float* ws, int64_t ws_elems, void* stream);

/*
 * qlora_gemm16 that also records start/stop (hipEvent_t created with timing, or null) at the
 * start of its tile grid and the end of its last kernel (the split-K or K-sliced-tail reduce),
 * the dispatches' own timestamps. No reference counterpart: the bench's per-launch timing of
 * the step's own MFMA GEMM.
 */
int qlora_gemm16_timed(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M,
                       int64_t N, int64_t K, int32_t mode, void* c, int64_t ldc,
                       const void* bias, const float* resid, int64_t ldr, int32_t epi,
                       int64_t swiglu_I, void* gu, int64_t ldgu, int32_t tile, int32_t stages,
                       int32_t splits, float* ws, int64_t ws_elems, void* stream, void* start,
                       void* stop);

/*
 * The package GEMM with an unrounded fp32 output (the LM head over vocabulary pieces):
 *   c[M, N] (f32, ldc) = alpha A op(B) + (resid ? rs[m] resid[m, n] : 0),
 *   rs = row_scale (f32 [M]) or 1 when null; resid (f32, ldr) may be c itself;
 *   mode 1: A [M, K] (lda >= K), B [K, N];  mode 2: A^T, A stored [K, M] (lda >= M), B [K, N].
 * tile, stages, splits, ws as qlora_gemm16 (no K-sliced last round: ws is for split-K only;
 * tile 0 / splits 0: the plan of qlora_gemm16_plan with epi 6).
 * Replaces the fp32 products of the reference's streamed head, acc = acc * alpha + P E_piece
 * (engine.py:1498-1547), the whole-row head's dh = G E, and the embedding gradient dE = G^T h
 * (the BASELINE config-4 extra: the reference freezes the embedding).
 * Requires: K % (64 stages) == 0 and K % 128 == 0; N % tile == 0; mode 2: M % tile == 0;
 * lda, ldb % 8 == 0; A, B 16-byte aligned; row_scale only with resid.
 */
int qlora_gemm16_f32(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M,
                     int64_t N, int64_t K, int32_t mode, float* c, int64_t ldc, float alpha,
                     const float* row_scale, const float* resid, int64_t ldr, int32_t tile,
                     int32_t stages, int32_t splits, float* ws, int64_t ws_elems, void* stream);

/*
 * fp32 workspace elements (*elems) qlora_gemm16 (epi 0-5, modes 0-1) or qlora_gemm16_f32
 * (epi 6, modes 1-2) uses for this problem, mode, tile and stage count: splits * M * N with
 * splits > 1; with one slice the K-sliced last round's partials (fp16 epilogues only), 0 when
 * that does not apply (tile 0 / splits 0: the automatic plan's). N as qlora_gemm16's (epi 3,
 * 5: I). No reference counterpart (sizes the caller's workspace).
 */
int qlora_gemm16_workspace(int64_t M, int64_t N, int64_t K, int32_t mode, int32_t epi,
                           int32_t tile, int32_t stages, int32_t splits, int64_t* elems);

/*
 * The tile, stage count and K split qlora_gemm16 (or, with epi 6, qlora_gemm16_f32) runs when
 * given tile 0 and splits 0: a fixed rule on (M, N, K, mode, epi), so a problem always runs the
 * same kernels and gives the same bits (no timing). No reference counterpart.
 */
int qlora_gemm16_plan(int64_t M, int64_t N, int64_t K, int32_t mode, int32_t epi, int32_t* tile,
                      int32_t* stages, int32_t* splits);

/*
 * The plan of qlora_gemm16 (epi 0-5, modes 0-1) with tile 0 and splits 0 in full: the first
 * launch's tile, stages and splits, and rest > 0 when the output columns past n_first run as a
 * second launch on 128 x 128 tiles with rest stages (else rest = n_first = 0). The split applies
 * to a product in one slice whose last round of 256 x 256 tiles would run part-full: its whole
 * rounds take the leading whole N tiles, and the remaining columns fill a round four times as
 * finely, without the K-sliced last round's fp32 partials and reduce; chosen by the same fixed
 * cost model. No reference counterpart.
 */
int qlora_gemm16_plan_split(int64_t M, int64_t N, int64_t K, int32_t mode, int32_t epi,
                            int32_t* tile, int32_t* stages, int32_t* splits, int32_t* rest,
                            int64_t* n_first);

/*
 * out = a + fp32(d) over numel elements (a, out f32; d f16; numel % 4 == 0; out may alias a):
 * the residual add after the down projection, h3 = h2 + d (engine.py:1048-1051, 1179).
 */
int qlora_resid_add(const float* a, const void* d, float* out, int64_t numel, void* stream);

/*
 * The LoRA forward of a layer's q and v adapters in one launch (engine.py:1088-1093):
 *   x_a = f16(a_a A_a^T)   f16 [n, r] (kept for the backward)
 *   l_a = f16(x_a B_a^T)   f16 [n, N_a] (added to the projection output by qlora_rope_fwd)
 * a_a f16 [n, H] (the dropped LoRA inputs of qlora_rms_fwd); A_a f16 [r, H]; B_a f16 [N_a, r].
 * l_q and l_v both null: x only (a backward that recomputes the LoRA inputs for its gradients,
 * its q and v kept from the forward).
 * Requires r in {8, 16, 32, 64}, H % 16 == 0, N_a % 32 == 0; a_a, A_a, B_a, l_a 16-byte
 * aligned.
 * No reference counterpart as one launch: the reference makes four fp16 products.
 */
int qlora_lora_fwd_rows(const void* a_q, const void* a_v, const void* A_q, const void* A_v,
                        const void* B_q, const void* B_v, void* x_q, void* x_v, void* l_q,
                        void* l_v, int64_t n, int32_t N_q, int32_t N_v, int32_t H, int32_t r,
                        void* stream);

/*
 * Per-token part of the LoRA backward of a layer's q and v adapters in one launch:
 *   dx_a = f16(f16(g_a B_a) * s)   f16 [n, r]        t_a = f16(dx_a A_a)   f16 [n, H]
 * g_q / g_v: the adapters' columns of the fused d[q|k|v] gradient (f16, row stride ldg);
 * Bt_a = B_a^T f16 [r, N_a]; At_a = A_a^T f16 [H, r] (the transposed adapter weights);
 * t_q/t_v may both be null (then not computed). Replaces `dx_lo = (g @ b_w) * s` and
 * `dx_lo @ a_w` (engine.py:1326-1330) for both adapters; the token reductions dB and dA are
 * qlora_lora_grad. Requires r in {8, 16, 32, 64}, N_a % 16 == 0, H % 32 == 0, ldg % 8 == 0;
 * g_a, Bt_a, At_a, t_a 16-byte aligned.
 */
int qlora_lora_bwd_rows(const void* g_q, const void* g_v, int64_t ldg, const void* Bt_q,
                        const void* Bt_v, const void* At_q, const void* At_v, void* dx_q,
                        void* dx_v, void* t_q, void* t_v, int64_t n, int32_t N_q, int32_t N_v,
                        int32_t H, int32_t r, float s, void* stream);

/*
 * Token reductions of the LoRA backward of a layer's q and v adapters (engine.py:1327, 1329):
 *   dB_a = s * g_a^T x_a   fp32 [N_a, r]        dA_a = dx_a^T a_a   fp32 [r, H]
 * g_q / g_v as in qlora_lora_bwd_rows (row stride ldg); x_a f16 [n, r] (qlora_lora_fwd_rows);
 * a_a f16 [n, H] (the dropped LoRA inputs); dx_a f16 [n, r] (qlora_lora_bwd_rows). fp32 sums
 * of exact products, reduced in a fixed order (deterministic); the reference rounds dB and dA
 * to fp16 before its `.float()`, these keep fp32. work: fp32 workspace of at least the
 * qlora_lora_grad_workspace size. n = 0 writes zeros. Requires r in {8, 16, 32, 64}; N_a, H,
 * ldg even.
 */
int qlora_lora_grad_workspace(int64_t n, int32_t N_q, int32_t N_v, int32_t H, int32_t r,
                              int64_t* elems);
int qlora_lora_grad(const void* g_q, const void* g_v, int64_t ldg, const void* x_q,
                    const void* x_v, const void* a_q, const void* a_v, const void* dx_q,
                    const void* dx_v, float* dB_q, float* dB_v, float* dA_q, float* dA_v,
                    int64_t n, int32_t N_q, int32_t N_v, int32_t H, int32_t r, float s,
                    float* work, int64_t work_elems, void* stream);

/*
 * qlora_lora_grad without a workspace argument: the partial sums go to a static device array of
 * the library (4 Mi fp32 = 16 MiB per GPU, held from the first call on that GPU until the
 * process ends). No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc);
 * it calls no hipMalloc/hipFree. Returns QLORA_ERR_SCRATCH_TOO_SMALL (300001) when
 * qlora_lora_grad_workspace(n, N_q, N_v, H, r) exceeds 4 Mi elements (e.g. more than 13,568
 * tokens at N_q = H = 1536, N_v = 256, r = 16). Calls that overlap on one GPU share the array
 * and race; the array needs no clearing between calls.
 */
int qlora_lora_grad_noalloc(const void* g_q, const void* g_v, int64_t ldg, const void* x_q,
                            const void* x_v, const void* a_q, const void* a_v, const void* dx_q,
                            const void* dx_v, float* dB_q, float* dB_v, float* dA_q,
                            float* dA_v, int64_t n, int32_t N_q, int32_t N_v, int32_t H,
                            int32_t r, float s, void* stream);

/*
 * Causal attention within each packed sequence (flash attention, online softmax), grouped-query
 * heads, fp16 operands and fp32 accumulation/softmax.
 *   q [n, HQ, D], k/v [n, KH, D] (q head h reads kv head h / (HQ/KH)), out [n, HQ, D] fp16,
 *   lse fp32 [HQ, n] (natural-log log-sum-exp of each query's scaled scores),
 *   cu_seqlens int32 [nseq + 1] on the device (0 = cu[0] <= ... <= cu[nseq] = n, every
 *   length <= max_len), scale = softmax scale (D^-1/2).
 * Replaces _attn_fwd engine.py:857-862 (aten._efficient_attention_forward with cu_seqlens,
 * causal) and the k/v repeat of _expand_kv engine.py:655-660.
 * Requires D in {64, 128}, HQ % KH == 0, HQ / KH <= 8, 16-byte aligned tensors.
 */
int qlora_attn_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                   const int32_t* cu_seqlens, int32_t nseq, int32_t max_len, int64_t n,
                   int32_t HQ, int32_t KH, int32_t D, float scale, void* stream);

/*
 * Its backward: dq [n, HQ, D]; dk, dv [n, HQ, D] per q head (the caller sums the HQ/KH heads
 * of each kv head, as the reference's backward through the repeated k/v does); delta is an
 * fp32 [HQ, n] workspace (rowsum(dout * out)). Replaces _attn_bwd engine.py:865-869
 * (aten._efficient_attention_backward). When the dQ launch would leave most of the GPU idle (few
 * long sequences) the dK/dV kernel runs on a second stream of the library's, forked from and
 * joined back into `stream` by events: work queued on `stream` afterwards sees every result.
 */
int qlora_attn_bwd(const void* dout, const void* q, const void* k, const void* v,
                   const void* out, const float* lse, float* delta, void* dq, void* dk, void* dv,
                   const int32_t* cu_seqlens, int32_t nseq, int32_t max_len, int64_t n,
                   int32_t HQ, int32_t KH, int32_t D, float scale, void* stream);

/*
 * Work-split forms of the two calls above (same results up to fp32 summation order): the key
 * range of each 32-query tile (forward, dQ) is cut into chunks of chunk_keys keys (a positive
 * multiple of 64, at most 16 chunks for max_len; 0: not cut), one workgroup each, and a second
 * kernel merges the fp32 partials in chunk order. A batch of few long sequences otherwise leaves
 * most of the GPU idle while its longest tiles walk their keys. work: fp32, 16-byte aligned, of
 * the elements qlora_attn_split_workspace returns (0 when max_len fits one chunk). Same
 * reference call sites (engine.py:857-869).
 */
int qlora_attn_split_workspace(int32_t max_len, int64_t n, int32_t HQ, int32_t D,
                               int32_t chunk_keys, int64_t* work_elems);
int qlora_attn_fwd_split(const void* q, const void* k, const void* v, void* out, float* lse,
                         const int32_t* cu_seqlens, int32_t nseq, int32_t max_len, int64_t n,
                         int32_t HQ, int32_t KH, int32_t D, float scale, int32_t chunk_keys,
                         float* work, int64_t work_elems, void* stream);
int qlora_attn_bwd_split(const void* dout, const void* q, const void* k, const void* v,
                         const void* out, const float* lse, float* delta, void* dq, void* dk,
                         void* dv, const int32_t* cu_seqlens, int32_t nseq, int32_t max_len,
                         int64_t n, int32_t HQ, int32_t KH, int32_t D, float scale,
                         int32_t chunk_keys, float* work, int64_t work_elems, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QLORA_AMD_H */
