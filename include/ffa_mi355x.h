/*
 * ffa_mi355x.h -- C ABI of the MI355X (gfx950) quantized-K pruned decode path.
 *
 * Plain pointers and sizes only.  Every pointer is a device pointer owned by
 * the caller; the library never allocates or frees device memory and never
 * synchronises the stream.  All calls are asynchronous on `stream`
 * (a hipStream_t passed as void*).  Return value: 0 on success, otherwise a
 * negative FFA_E_* code; ffa_last_error() then returns a message
 * (thread-local, valid until the next call on the same thread).
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   ffa_q2fp8_decode          ffa-q2fp8/attn_kernel/attn_kernel_v1210_fused_bsz_q2fp8.py:283-304
 *                             (stage-1 launch :283-291 + stage-2 launch :299-304 of
 *                              attn_forward_decode_quantized :191-309)
 *   ffa_q2fp8_decode_stage1   the stage-1 launch alone (:283-297, kernel
 *                             attn_forward_stage1_fused_threshold_qbits :10-139)
 *   ffa_q2fp8_decode_stage2   the stage-2 launch alone (:299-304, kernel
 *                             attn_forward_stage2_masked :142-171)
 *   ffa_q2fp8_decode with     ffa-q2fp8-meanv/attn_kernel/attn_kernel_v1210_meanv_bsz_q2fp8.py
 *     v_mean set              (the mean-V variant: stage 1 :10-153, stage 2 :156-202)
 *   ffa_v_mean                the same file :332 (v.mean(dim=1, dtype=float32).to(v.dtype))
 *   ffa_q2_quantize_channel   ffa-q2fp8/run_attn_bench_q2.py:78-105
 *                             (quantize_k_2bit_fp8_residual; same as
 *                              ffa-q2fp8/fused_kproj_rope_q2fp8.py:40-68)
 *   ffa_kproj_rope_q2_channel ffa-q2fp8/fused_kproj_rope_q2fp8.py:492-542
 *                             (the two Triton launches of kproj_rope_quantize_triton)
 *   ffa_q2_append_channel     no reference counterpart (the reference's incremental-quantization
 *                             TODO, ffa-q2fp8/OPTIMIZATION_NOTES.md:23-26): append to the
 *                             reference-layout cache with its existing per-channel scale / zero
 *   ffa_q2_quantize_g32_append no reference counterpart: g32 quantize + paged append of
 *                             given K rows (the paged g32 cache layout)
 *   ffa_q2_paged_dequant      ffa-fp8fp8/e2e/fp8fp8_cache.py:60-69, 84-89 (_refresh_fp_cache:
 *                             the cache's keys dequantized for exact attention), for the
 *                             paged g32 cache
 *   ffa_kproj_rope_q2_append  no reference counterpart: decode-time append of
 *                             K-proj + RoPE + g32 quantize into the paged cache
 *                             (incremental quantisation is a TODO in the reference,
 *                              ffa-q2fp8/OPTIMIZATION_NOTES.md:23-26)
 *   ffa_kproj_rope            F.linear + apply_rope of every reference producer, e.g.
 *                             ffa-fp8fp8/fused_kproj_rope_fp8fp8.py:80-88,
 *                             ffa-nvfp4fp8/fused_kproj_rope_nvfp4fp8.py:131-139,
 *                             ffa-nf4fp8/fused_kproj_rope_nf4fp8.py:428-436
 *   ffa_fp8fp8_quantize       ffa-fp8fp8/fused_kproj_rope_fp8fp8.py:58-64
 *                             (quantize_k_fp8_fp8_residual)
 *   ffa_fp8_scaled_quantize   no reference counterpart: fp8 K with one fp16 scale per
 *                             token and KV head (read by ffa_kfmt_decode)
 *   ffa_nvfp4_quantize        ffa-nvfp4fp8/fused_kproj_rope_nvfp4fp8.py:62-114
 *                             (encode_k_nvfp4_fp8_residual)
 *   ffa_nvfp4_g16_append,     no reference counterpart: paged nvfp4 / nf4 layouts
 *   ffa_nf4_g64_append        (per-token group scales), quantize + append
 *   ffa_nf4_quantize          ffa-nf4fp8/fused_kproj_rope_nf4fp8.py:72-96
 *                             (encode_k_nf4_fp8_residual; the Triton producer
 *                              kproj_rope_nf4_triton :440-558 is ffa_kproj_rope + this)
 */
#ifndef FFA_MI355X_H
#define FFA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element type codes */
enum {
  FFA_DT_F16 = 0,
  FFA_DT_BF16 = 1,
  FFA_DT_F32 = 2,
  FFA_DT_FP8_E4M3 = 3, /* OCP float8_e4m3fn */
  FFA_DT_FP8_E5M2 = 4, /* OCP float8_e5m2 */
  FFA_DT_NONE = 5      /* no residual */
};

/* KV-cache layouts */
enum {
  /* reference layout (attn_kernel_v1210_fused_bsz_q2fp8.py:192-197):
     k_q [B,T,HKV,32] u8, k_residual [B,T,HKV,128], v [B,T,HKV,128],
     per-channel k_scale/k_zero [B,HKV,128] */
  FFA_LAYOUT_CONTIG = 0,
  /* paged layout, 64-token pages from a pool of P pages:
     k_q        [P, HKV, 4 groups, 64 tokens, 8 bytes]   (group-major codes)
     k_scale    [P, HKV, 4 groups, 64 slots] fp16        (g32 mode)
     k_zero     [P, HKV, 4 groups, 64 slots] fp16        (g32 mode)
                token t of a page sits in slot 16*(t/16) + 4*(t%4) + (t/4)%4
     k_residual [P, HKV, 64 tokens, 128] fp8
     v          [P, HKV, 128, 64 tokens]                 (V^T pages)
     block_table[b, i] = pool page holding tokens [64i, 64i+64) of sequence b */
  FFA_LAYOUT_PAGED = 1
};

/* scale/zero modes */
enum {
  FFA_SCALE_CHANNEL = 0, /* one scale/zero per (b, hkv, d) over all tokens (reference) */
  FFA_SCALE_G32 = 1      /* one fp16 scale/zero per token per 32-wide group along d */
};

enum {
  FFA_OK = 0,
  FFA_E_INVALID = -1,     /* argument/shape error */
  FFA_E_UNSUPPORTED = -2, /* valid request this build does not implement */
  FFA_E_LAUNCH = -3       /* HIP launch error */
};

/*
 * Arguments of one pruned decode step.  Shapes use B sequences, HQ query
 * heads, HKV KV heads (G = HQ/HKV <= 16, the reference's 16-row tile,
 * attn_kernel_v1210_fused_bsz_q2fp8.py:19, 40-41), head dim D = DV = 128,
 * SBS a power of two >= 16 and BS a multiple of SBS.
 *
 * Scratch (caller-owned, see ffa_q2fp8_decode_nparts): one partial per query
 * row and 512-token span,
 *   m_buf, l_buf [B, HQ, nparts] f32; o_buf [B, HQ, nparts, 128] f32;
 *   mask [B, HKV, ntbs] i8 (1 = block kept, written for every block).
 * Two launches on `stream`: score + prune + exact pass, then the log-sum-exp
 * merge.  A group of more than 4 query rows or a prune block longer than 512
 * tokens (SBS > 512) needs every row's block maxima before any block is
 * decided: stage 1 is then two launches (maxima, then decide + exact pass) and
 * needs piece_max [B, HQ, npieces] f32 with npieces >= ffa_q2fp8_decode_pieces()
 * and threshold_out (or threshold_in).  Calls that share scratch must be
 * ordered on one stream.
 */
typedef struct ffa_q2fp8_decode_args {
  const void *q; /* [B, HQ, 128], dtype q_dtype */
  int q_dtype;
  const uint8_t *k_q;
  const void *k_scale;
  const void *k_zero;
  int scale_dtype; /* F16/BF16/F32 for CHANNEL mode, F16 for G32 */
  int scale_mode;
  const uint8_t *k_residual; /* may be NULL when res_dtype == FFA_DT_NONE */
  int res_dtype;             /* FP8_E4M3, FP8_E5M2 or NONE */
  const void *v;
  int v_dtype; /* F16 or BF16 */
  int layout;
  const int32_t *block_table; /* [B, bt_stride] (paged only), bt_stride >= ceil(T/64) */
  int bt_stride;
  const int32_t *seq_lens; /* [B] or NULL (all sequences have length T); clamped to [0, T] */
  int B, T, HQ, HKV;
  float scale;                /* softmax scale (1/sqrt(D) by default) */
  int BS, SBS;                /* threshold block size / prune block size */
  float delta;                /* threshold margin in log2-scaled units */
  const float *threshold_in;  /* [B, HQ] or NULL (probe windows are used) */
  float *threshold_out;       /* [B, HQ] or NULL */
  void *out;                  /* [B, HQ, 128], dtype out_dtype */
  int out_dtype;
  float *m_buf, *l_buf, *o_buf;
  int nparts;
  int8_t *mask;
  int ntbs;
  int num_pages; /* paged: pages P of every pool (> 0); block-table entries outside [0, P) read page 0 */
  float *piece_max; /* two-pass decodes only (else NULL): [B, HQ, npieces] f32 */
  int npieces;
  /* Mean-V fallback (ffa-q2fp8-meanv/attn_kernel/attn_kernel_v1210_meanv_bsz_q2fp8.py:109-119,
   * 156-202): with v_mean non-NULL a pruned block that holds tokens keeps its softmax mass on the
   * coarse (2-bit) scores, with v_mean as its value:
   *   out = (sum_kept 2^s v + sum_pruned 2^s_coarse * v_mean) / (sum_kept 2^s + sum_pruned 2^s_coarse).
   * NULL: pruned blocks are dropped (the q2fp8 decode).  approx_m / approx_l: scratch for the pruned
   * mass per query row and partial slot. */
  const void *v_mean; /* [B, HKV, 128], dtype v_mean_dtype (F16 / BF16 / F32), e.g. from ffa_v_mean */
  int v_mean_dtype;
  float *approx_m, *approx_l; /* with v_mean: [B, HQ, nparts] f32 each */
  /* CHANNEL mode with BF16 / F32 k_scale and k_zero: non-zero when the caller knows that every
   * value of both is exactly representable in fp16 (bf16 scales within fp16's range, the usual
   * case).  The decode then dequantizes as for fp16 scales (one packed fp16 FMA per pair of
   * channels, the same k_hat as the reference's fp16(fp32(fp32(c * s) + z)) for such values);
   * 0 keeps the fp32 arithmetic, correct for any values.  A non-zero flag on values fp16 does not
   * hold rounds them to fp16 first.  No counterpart in the reference, which always computes in fp32
   * (attn_kernel_v1210_fused_bsz_q2fp8.py:52-53, 93). */
  int scale_exact_f16;
} ffa_q2fp8_decode_args;

/* Number of partial slots per query row the scratch buffers must hold for max length T. */
int ffa_q2fp8_decode_nparts(int T, int BS, int SBS);
/* Pieces per query row of the two-pass scratch piece_max (prune blocks when SBS <= 512, else
 * 512-token spans), or 0 when the decode runs in one pass (G <= 4 and SBS <= 512).  Same rule
 * for ffa_kfmt_decode. */
int ffa_q2fp8_decode_pieces(int HQ, int HKV, int T, int BS, int SBS);

/* Both stages back to back on `stream`.  A stage-1 grid of more than 2^31 - 1 workgroups
 * (ceil(T / 512) x HKV * ceil(G / 4) x B), or of more than 65535 workgroup spans per sequence
 * (T above 32M tokens), returns FFA_E_UNSUPPORTED before any launch; the same holds for
 * ffa_kfmt_decode. */
int ffa_q2fp8_decode(const ffa_q2fp8_decode_args *args, void *stream);

/*
 * Mean over each sequence's tokens of V, the mean-V fallback's v_mean (replaces
 * `v.mean(dim=1, dtype=torch.float32).to(v.dtype)`, ffa-q2fp8-meanv/attn_kernel/
 * attn_kernel_v1210_meanv_bsz_q2fp8.py:332): fp32 sums, one rounding to out_dtype.
 *   layout CONTIG: v [B, T, HKV, 128]; PAGED: V^T pages [P, HKV, 128, 64] through block_table
 *   (entries outside [0, num_pages) read page 0, as in the decode).  seq_lens [B] or NULL (length T).
 *   out [B, HKV, 128] (0 for an empty sequence); partial: f32 scratch [B, HKV, nsplit, 128] with
 *   nsplit >= ffa_v_mean_nsplit(T).
 */
int ffa_v_mean_nsplit(int T);
int ffa_v_mean(const void *v, int v_dtype, int layout, const int32_t *block_table, int bt_stride, int num_pages,
               const int32_t *seq_lens, int B, int T, int HKV, float *partial, int nsplit, void *out, int out_dtype,
               void *stream);

/*
 * ffa_q2fp8_decode without any caller scratch and without allocating: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The caller passes inputs and `out` as for
 * ffa_q2fp8_decode; m_buf, l_buf, o_buf, nparts, piece_max, npieces, approx_m and approx_l are
 * ignored; mask (with ntbs) and threshold_out are written when given, else kept in the scratch.
 * The scratch is a static device array of FFA_NOALLOC_SCRATCH_BYTES per GPU, held until the
 * process ends; a shape whose scratch (partials 520 B per query row and 512-token span, 8 B more
 * with v_mean, plus mask, thresholds and the two-pass maxima) exceeds it returns FFA_E_UNSUPPORTED
 * before any launch.  Calls that overlap on
 * one GPU share the array and race: order them on one stream.
 */
#define FFA_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int ffa_q2fp8_decode_noalloc(const ffa_q2fp8_decode_args *args, void *stream);

/* Stage 1: coarse scores, threshold, prune (mask, threshold_out) and the exact pass over
 * kept blocks, writing the partials m_buf/l_buf/o_buf. */
int ffa_q2fp8_decode_stage1(const ffa_q2fp8_decode_args *args, void *stream);
/* Stage 2: log-sum-exp merge of the partials into `out` (same arguments as stage 1). */
int ffa_q2fp8_decode_stage2(const ffa_q2fp8_decode_args *args, void *stream);

/*
 * Reference quantizer (per-channel scale/zero over T, tau = k_dtype):
 *   k [B,T,HKV,D] -> k_q [B,T,HKV,ceil(D/4)] u8, scale/zero [B,HKV,D] (k_dtype),
 *   residual [B,T,HKV,D] fp8 (res_dtype).  Needs scratch f32 minmax
 *   [2, B, nsplit, HKV*D] with nsplit = ffa_q2_quantize_nsplit(T).
 */
int ffa_q2_quantize_nsplit(int T);
int ffa_q2_quantize_channel(const void *k, int k_dtype, int B, int T, int HKV, int D, uint8_t *k_q,
                            void *scale, void *zero, uint8_t *residual, int res_dtype, float *minmax,
                            void *stream);

/*
 * Append to the reference-layout cache (no reference counterpart: incremental quantization is
 * a TODO there, ffa-q2fp8/OPTIMIZATION_NOTES.md:23-26).  New tokens k_new [B, Tn, HKV, D]
 * (k_dtype) are quantized with the cache's existing per-channel scale / zero [B, HKV, D]
 * (k_dtype, as ffa_q2_quantize_channel wrote them) by the same per-element ops, so values
 * outside [zero, zero + 3 scale] take code 0 or 3 and the fp8 residual carries the rest; token n
 * of sequence b goes to position pos[b] + n of k_q [B, T_cap, HKV, ceil(D/4)] and residual
 * [B, T_cap, HKV, D]; positions outside [0, T_cap) are not written.  V is a plain copy (not here).
 */
int ffa_q2_append_channel(const void *k_new, int k_dtype, int B, int Tn, int HKV, int D, const int32_t *pos, int T_cap,
                          const void *scale, const void *zero, uint8_t *k_q, uint8_t *residual, int res_dtype,
                          void *stream);

/*
 * Fused K projection + RoPE + per-channel q2 quantize (reference producer).
 *   h [B,T,H] (bf16/fp16), w_k [HKV*D, H] (same dtype), bias [HKV*D] or NULL,
 *   cos/sin [T, D] (cs_dtype = F32 or the h dtype).  The RoPE output dtype is
 *   the promotion of h and cos dtypes (reference type promotion).
 *   Outputs as ffa_q2_quantize_channel; k_scratch [B,T,HKV,D] of the
 *   promoted dtype receives the rotated K.
 */
int ffa_kproj_rope_q2_channel(const void *h, const void *w_k, const void *bias, int h_dtype, const void *cos,
                              const void *sin, int cs_dtype, int B, int T, int H, int HKV, int D,
                              void *k_scratch, uint8_t *k_q, void *scale, void *zero, uint8_t *residual,
                              int res_dtype, float *minmax, void *stream);

/*
 * Fused K projection + RoPE + g32 quantize + append into the paged cache.
 *   h [B, Tn, H]; token n of sequence b goes to position pos[b] + n.
 *   cos/sin [B, Tn, D] f32 (per-token rows).  v_new [B, Tn, HKV, 128] (v_dtype)
 *   or NULL.  Writes codes/scale/zero/residual/V^T into the paged pools of num_pages
 *   pages.  Every append entry point writes nothing for a token whose position lies
 *   outside its block-table row (bt_stride columns) or whose page id is outside
 *   [0, num_pages); callers check positions on the host beforehand.
 */
int ffa_kproj_rope_q2_append(const void *h, const void *w_k, const void *bias, int h_dtype, const float *cos,
                             const float *sin, int B, int Tn, int H, int HKV, const int32_t *pos,
                             const int32_t *block_table, int bt_stride, int num_pages, uint8_t *k_q_pages,
                             void *scale_pages, void *zero_pages, uint8_t *res_pages, int res_dtype,
                             const void *v_new, void *v_pages, int v_dtype, void *stream);

/*
 * g32 quantize + append of given K rows into the paged cache (no projection):
 *   k [B, Tn, HKV, 128] (F16/BF16/F32); token n of sequence b goes to
 *   position pos[b] + n.  Same quantization rules as ffa_kproj_rope_q2_append.
 *   v_new [B, Tn, HKV, 128] (2-byte dtype of the V pool) or NULL.
 */
int ffa_q2_quantize_g32_append(const void *k, int k_dtype, int B, int Tn, int HKV, const int32_t *pos,
                               const int32_t *block_table, int bt_stride, int num_pages, uint8_t *k_q_pages,
                               void *scale_pages, void *zero_pages, uint8_t *res_pages, int res_dtype,
                               const void *v_new, void *v_pages, void *stream);

/*
 * Paged g32 cache -> contiguous K and V [B, T, HKV, 128] in out_dtype (F16/BF16/F32), the keys
 * dequantized as k = c * scale + zero + residual (fp32, one rounding to out_dtype) and V copied
 * from the V^T pages (v_dtype F16/BF16).  T is a multiple of 64; tokens at or past seq_lens[b]
 * (seq_lens may be NULL: every sequence holds T tokens) are written as zeros.  Block-table
 * entries outside [0, num_pages) read page 0.  Feeds exact attention over the cache (prefill,
 * chunked prefill, and decode steps that do not prune).
 */
int ffa_q2_paged_dequant(const uint8_t *k_q_pages, const void *scale_pages, const void *zero_pages,
                         const uint8_t *res_pages, int res_dtype, const void *v_pages, int v_dtype,
                         const int32_t *block_table, int bt_stride, int num_pages, const int32_t *seq_lens,
                         int B, int T, int HKV, void *k_out, void *v_out, int out_dtype, void *stream);

/*
 * K projection + RoPE without quantization (the first half of every producer):
 *   k_out [B, T, HKV, D] in the promoted dtype of h and cos (F32 when cs_dtype is F32,
 *   else h_dtype); same arithmetic as ffa_kproj_rope_q2_channel's k_scratch.
 */
int ffa_kproj_rope(const void *h, const void *w_k, const void *bias, int h_dtype, const void *cos, const void *sin,
                   int cs_dtype, int B, int T, int H, int HKV, int D, void *k_out, void *stream);

/*
 * Quantizers of the other K formats (reference layouts), bit-exact with the reference's
 * torch op sequences; k has dtype k_dtype (F16/BF16/F32), contiguous.
 *   fp8fp8: n elements -> base, residual (fp8_dtype FP8_E4M3/E5M2), same shape as k.
 *   nvfp4:  k [B, T, HKV, D] -> k_packed [B, T, HKV, ceil(D/2)] (low nibble first),
 *           scale [B, ceil(T/page_size), HKV] (k_dtype), residual [B, T, HKV, D] fp8.
 *   nf4:    k [B, T, HKV, D] -> k_packed [B, T, HKV, ceil(D/2)], scale [B, HKV, D]
 *           (k_dtype), residual; scratch absmax f32 [B, nsplit, HKV*D] with
 *           nsplit = ffa_nf4_quantize_nsplit(T).
 */
int ffa_fp8fp8_quantize(const void *k, int k_dtype, size_t n, uint8_t *base, uint8_t *residual, int fp8_dtype,
                        void *stream);
/* Per-token-scaled fp8 (no reference counterpart; the K layout ffa_kfmt_decode reads with
 * FFA_KSCALE_TOKEN): k [rows, D] (k_dtype) -> base [rows, D] fp8, scale [rows] fp16,
 * residual [rows, D] fp8; per row s = fp16(max(amax |k|, 1e-6) / fmax) with fmax 448 (e4m3)
 * or 57344 (e5m2), base = fp8(k / s), residual = fp8(k - base * s). */
int ffa_fp8_scaled_quantize(const void *k, int k_dtype, size_t rows, int D, uint8_t *base, void *scale,
                            uint8_t *residual, int fp8_dtype, void *stream);
int ffa_nvfp4_quantize(const void *k, int k_dtype, int B, int T, int HKV, int D, int page_size, uint8_t *k_packed,
                       void *scale, uint8_t *residual, int res_dtype, void *stream);
int ffa_nf4_quantize_nsplit(int T);

/*
 * Paged nvfp4-g16 / nf4-g64 modes (no reference counterpart): quantize K rows
 * k [B, Tn, HKV, 128] (F16/BF16/F32) and append them, with v_new [B, Tn, HKV, 128] (the
 * V pool's 2-byte dtype) or NULL, at positions pos[b] + n of the pages block_table[b, :].
 *   nvfp4-g16: per 16 channels s = e4m3(min(amax / 6, 448)), code = nearest e2m1 level of
 *              k / s by the midpoint rule (ties up), residual = fp8(k - level * s).
 *   nf4-g64:   per 64 channels s = fp16(max(amax, 1e-6)), code = nearest NF4 level of
 *              clamp(k / s, -1, 1) (ties down), residual = fp8(k - codebook[code] * s).
 * Pools as described at ffa_kfmt_decode.
 */
int ffa_nvfp4_g16_append(const void *k, int k_dtype, int B, int Tn, int HKV, const int32_t *pos,
                         const int32_t *block_table, int bt_stride, int num_pages, uint8_t *k_pages,
                         uint8_t *scale_pages, uint8_t *res_pages, int res_dtype, const void *v_new, void *v_pages,
                         void *stream);
int ffa_nf4_g64_append(const void *k, int k_dtype, int B, int Tn, int HKV, const int32_t *pos,
                       const int32_t *block_table, int bt_stride, int num_pages, uint8_t *k_pages, void *scale_pages,
                       uint8_t *res_pages, int res_dtype, const void *v_new, void *v_pages, void *stream);
int ffa_nf4_quantize(const void *k, int k_dtype, int B, int T, int HKV, int D, uint8_t *k_packed, void *scale,
                     uint8_t *residual, int res_dtype, float *absmax, void *stream);

/*
 * Pruned decode for the other K formats of the reference (contiguous [B, T, HKV, row]
 * layouts as in the reference), same prune / refine / merge as ffa_q2fp8_decode:
 *   FFA_KFMT_FP8_E4M3/E5M2 + FFA_KSCALE_NONE   fp8 base, k_hat = fp16(base)
 *       (ffa-fp8fp8/attn_kernel/attn_kernel_v1210_fused_bsz_fp8fp8.py:10-177, launches :263-309)
 *   FFA_KFMT_FP8_E4M3/E5M2 + FFA_KSCALE_TOKEN  k_hat = fp16(base * scale[b, t, h]) (per-token scales;
 *       no reference counterpart)
 *   FFA_KFMT_NVFP4 + FFA_KSCALE_BLOCK          packed e2m1 nibbles (low nibble first) times
 *       scale[b, t / BS, h] ([B, ceil(T/BS), HKV])
 *       (ffa-nvfp4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nvfp4fp8.py:24-210, launches :316-363)
 *   FFA_KFMT_NF4 + FFA_KSCALE_CHANNEL          NF4 codebook times scale[b, h, d] ([B, HKV, 128])
 *       (ffa-nf4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nf4fp8.py:41-199, launches :300-326)
 *   FFA_KFMT_NVFP4 + FFA_KSCALE_G16 / FFA_KFMT_NF4 + FFA_KSCALE_G64, layout FFA_LAYOUT_PAGED
 *       (no reference counterpart): 64-token pages through block_table
 *       [B, bt_stride]: k [P, HKV, 64, 64] packed nibbles, k_scale [P, HKV, 64, 8] e4m3 (G16) or
 *       [P, HKV, 64, 2] fp16 (G64), residual [P, HKV, 64, 128] fp8, v [P, HKV, 128, 64] (V^T pages);
 *       k_hat = fp16(value * scale of the channel's group).  Written by ffa_nvfp4_g16_append /
 *       ffa_nf4_g64_append.
 * Contiguous layout: k is [B, T, HKV, 128] fp8 bytes or [B, T, HKV, 64] packed nibbles; residual
 * [B, T, HKV, 128] fp8; v [B, T, HKV, 128].  Scratch as ffa_q2fp8_decode (nparts from
 * ffa_q2fp8_decode_nparts).
 */
enum { FFA_KFMT_FP8_E4M3 = 0, FFA_KFMT_FP8_E5M2 = 1, FFA_KFMT_NVFP4 = 2, FFA_KFMT_NF4 = 3 };
enum {
  FFA_KSCALE_NONE = 0,
  FFA_KSCALE_TOKEN = 1,
  FFA_KSCALE_BLOCK = 2,
  FFA_KSCALE_CHANNEL = 3,
  FFA_KSCALE_G16 = 4, /* paged nvfp4: one e4m3 scale per 16 channels of each token */
  FFA_KSCALE_G64 = 5  /* paged nf4: one fp16 scale per 64 channels of each token */
};

typedef struct ffa_kfmt_decode_args {
  const void *q; /* [B, HQ, 128] */
  int q_dtype;
  const uint8_t *k;
  int k_format;
  const void *k_scale; /* NULL with FFA_KSCALE_NONE */
  int scale_dtype;     /* F16/BF16/F32 */
  int scale_kind;
  const uint8_t *k_residual; /* may be NULL when res_dtype == FFA_DT_NONE */
  int res_dtype;
  const void *v;
  int v_dtype;
  const int32_t *seq_lens; /* [B] or NULL; clamped to [0, T] */
  int B, T, HQ, HKV;
  float scale;
  int BS, SBS;
  float delta;
  const float *threshold_in;
  float *threshold_out;
  void *out;
  int out_dtype;
  float *m_buf, *l_buf, *o_buf;
  int nparts;
  int8_t *mask;
  int ntbs;
  int layout;                 /* FFA_LAYOUT_CONTIG or FFA_LAYOUT_PAGED */
  const int32_t *block_table; /* [B, bt_stride] (paged only), bt_stride >= ceil(T/64) */
  int bt_stride;
  int num_pages; /* paged: pages P of every pool (> 0); block-table entries outside [0, P) read page 0 */
  float *piece_max; /* two-pass decodes only (G > 4 or SBS > 512), as in ffa_q2fp8_decode_args */
  int npieces;
} ffa_kfmt_decode_args;

int ffa_kfmt_decode(const ffa_kfmt_decode_args *args, void *stream);

const char *ffa_last_error(void);
const char *ffa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FFA_MI355X_H */
