// Shared definitions of the decode kernels (q2fp8 and the other K formats): parameters,
// workgroup shape, operand conversions and the stage-2 merge kernel.
#pragma once

#include "ffa_common.h"

#include <type_traits>

namespace ffa {

constexpr int kD = 128;
constexpr int kPage = 64;
constexpr int kWaves = 4;
constexpr int kPPW = 2;                      // 64-token chunks (pages) per wave
constexpr int kChunksPerWG = kWaves * kPPW;  // 512 tokens per workgroup
constexpr int kMinSpan = 2;                  // smallest span (chunks per workgroup) of a small grid
constexpr int kSmallSpanTokens = 8192;       // sequences up to this many tokens get slots for it
// LDS row pitch (bytes) of a V tile staged row-major for the transposing reads (vt_operand_lds,
// 8-byte aligned rows): whole tile (128 columns) 256 + 16; half a tile (64 columns) 128 + 8,
// which keeps the q2 reference-layout decoder within two workgroups per CU (80.6 KB of LDS)
constexpr int kVRow = 272;
constexpr int kVRowHalf = 136;

struct DecodeParams {
  const void *q;
  const uint8_t *kq;
  const void *ks;
  const void *kz;
  const uint8_t *kr;
  const void *v;
  const int32_t *bt;
  const int32_t *seq_lens;
  const float *th_in;
  float *th_out;
  void *out;
  float *m_buf, *l_buf, *o_buf;
  int8_t *mask;
  int q_dtype, s_dtype, out_dtype;
  int bt_stride;
  int num_pages;  // paged: pages in each pool; block-table entries outside [0, num_pages) read page 0
  int B, T, HQ, HKV, G;
  float scale;
  int BS, SBS;
  float delta;
  int nparts, ntbs;
  int nwg;  // decode workgroups per (sequence, KV head)
  // GQA groups of more than 4 query rows and prune blocks longer than a workgroup's 512 tokens
  // run as two passes of the same kernel over "units" of at most 4 query rows of one KV head
  // (grid y = HKV * nq):
  //   pass 0  one pass: each workgroup decides its blocks from its own scores (G <= 4, SBS <= 512)
  //   pass 1  scores only: the coarse maximum of every prune block (SBS <= 512) or 512-token span
  //           (SBS > 512) per query row goes to pmax [B, HQ, npieces], the thresholds to th_out
  //   pass 2  every block is decided from all G rows' maxima and thresholds (the group prune of
  //           the single pass), then the exact pass and partials as in pass 0
  int nq;        // units (quads of query rows) per KV head, ceil(G / 4)
  int pass;      // 0, 1 or 2
  float *pmax;   // pass 1 / 2 scratch, [B, HQ, npieces] f32
  int npieces;   // NTBS (SBS <= 512) or nparts (SBS > 512)
  // mean-V fallback (q2fp8 decode only; null = pruned blocks are dropped): stage 1 also writes,
  // per query row and partial slot, the maximum am and the sum al = sum 2^(s - am) of the coarse
  // scores s of the slot's pruned tokens; the merge gives that mass the value v_mean.
  const void *v_mean;  // [B, HKV, 128], dtype vm_dtype
  int vm_dtype;
  float *am_buf, *al_buf;  // [B, HQ, nparts] f32
  // 64-token chunks per workgroup (one partial slot each): kChunksPerWG, or 4 / 2 when a small grid
  // would leave CUs idle (the other-format decoder, one pass, SBS <= 64); each wave then owns one
  // chunk, and waves past the span only help with the operands, the probe and the merge
  int span;
};

// chunks per decode workgroup of a launch (0 in the struct means the default span)
__device__ __forceinline__ int decode_span(const DecodeParams &p) { return p.span > 0 ? p.span : kChunksPerWG; }

// The (KV head, query rows) unit of a decode workgroup: grid y = hkv * nq + quad, rows
// 4 quad .. 4 quad + Gu - 1 of the GQA group (query heads row0 ..).
struct DecodeUnit {
  int hkv, quad, Gu, row0;
};
__device__ __forceinline__ DecodeUnit decode_unit(const DecodeParams &p, int y) {
  DecodeUnit u;
  u.hkv = p.nq == 1 ? y : y / p.nq;
  u.quad = y - u.hkv * p.nq;
  u.Gu = min(4, p.G - 4 * u.quad);
  u.row0 = u.hkv * p.G + 4 * u.quad;
  return u;
}

// x / d for x >= 0 and d a power of two (SBS, spans of 64-token chunks): one shift.  A division by a
// runtime value is a sequence of dependent scalar and vector instructions, which at the head of a
// workgroup's chain costs it time (the position arithmetic of a rotated grid order cost config 2
// 0.2 us per step).
__device__ __forceinline__ int div_pow2(int x, int d) { return x >> __builtin_ctz((unsigned)d); }
// x / BS for x >= 0: a shift when BS is a power of two (the usual case), else the division
__device__ __forceinline__ int div_bs(const DecodeParams &p, int x) {
  return (p.BS & (p.BS - 1)) == 0 ? div_pow2(x, p.BS) : x / p.BS;
}

// Workgroup coordinates (span cg, unit y, sequence b) of a decode workgroup.  Dispatch is
// round-robin over the 8 XCDs in linear workgroup order (x fastest).  The grid is (span, unit,
// sequence), or, for the builds that place the unit fastest, (unit, span, sequence), launched so
// by the host: with 8 or 16 units per sequence the spans of a (sequence, KV head) then land on one
// XCD, whose L2 still holds their partials when the merge workgroups of those rows, placed on the
// same XCD (merge_partials), read them in the next kernel (config 2's step 12.78 -> 12.40 us).  The
// layouts whose code lines hold several KV heads (the per-channel q2 rows, the 4-bit formats'
// contiguous rows) keep the span fastest, so that the workgroups of one span's heads share each
// line through one XCD's L2 (the unit first took the reference-layout config 2 from 16.1 to 17.9
// us), and so does the other-format large-batch build (configs 3 and 4).  No division: the order
// is the grid's own (the position arithmetic of a rotated order cost config 2 0.2 us).
struct GridPos {
  int cg, y, b;
};
template <bool kUnitFastest>
__device__ __forceinline__ GridPos grid_pos() {
  if constexpr (kUnitFastest) return GridPos{(int)blockIdx.y, (int)blockIdx.x, (int)blockIdx.z};
  else return GridPos{(int)blockIdx.x, (int)blockIdx.y, (int)blockIdx.z};
}

// Pass 2: whether each prune block of the workgroup's span survives, from the coarse maxima pass 1
// wrote for every query row of the group: kept iff some row r has !(max over the block's pieces of
// pmax[r] < th[r]) -- the single pass's "prune iff every row is below its threshold".  s_keep[blk]
// (blk < 512 / SBS, or 0 when SBS > 512) must be zero beforehand and is read after a barrier.
// Spans past the sequence end (SBS > 512) are left out, as pass 1 wrote nothing for them.
__device__ __forceinline__ void decide_blocks(const DecodeParams &p, int b, int hkv, int cw, int Tb, int *s_keep) {
  const int G = p.G, SBS = p.SBS;
  const int span_tok = 8 * 64;  // tokens of one workgroup span
  const int nblk = SBS <= span_tok ? div_pow2(span_tok, SBS) : 1;
  const int per = SBS <= span_tok ? 1 : div_pow2(SBS, span_tok);  // pieces per block
  const int piece0 = div_pow2(cw * 64, SBS) * per;                  // first piece of block 0
  const float *thr = p.th_in != nullptr ? p.th_in : p.th_out;
  for (int idx = threadIdx.x; idx < nblk * G; idx += blockDim.x) {
    const int blk = idx / G, r = idx - blk * G;
    const size_t row = (size_t)b * p.HQ + hkv * G + r;
    float mx = -INFINITY;
    for (int s = 0; s < per; ++s) {
      const int piece = piece0 + blk * per + s;
      if (piece >= p.npieces || (per > 1 && piece * span_tok >= Tb)) break;
      const float v = p.pmax[row * p.npieces + piece];
      mx = s == 0 ? v : fmaxf(mx, v);
    }
    if (!(mx < thr[row])) atomicOr(&s_keep[blk], 1);
  }
}

// Survivor ballot of one 64-token chunk (first chunk of the workgroup cw, this chunk c): in pass 2
// each lane votes its 16 tokens' block decision from s_keep, otherwise its row's block maximum
// against the row's threshold (strict <; rows outside the unit do not vote).
__device__ __forceinline__ uint64_t chunk_ballot(const DecodeParams &p, bool row_ok, float mb, float th,
                                                 const int *s_keep, int cw, int c, int kc) {
  if (p.pass == 2) {
    const int rel = (c - cw) * 64 + 16 * kc;  // lane's first token relative to the span
    const int blk = p.SBS <= 512 ? div_pow2(rel, p.SBS) : 0;
    return __ballot(row_ok && s_keep[blk] != 0);
  }
  return __ballot(row_ok && !(mb < th));
}

// Pass 1: the coarse maximum of the prune block holding the lane's tokens (SBS <= 512), or of
// the whole span (SBS > 512), for the lane's query row; one lane per block and row writes.
// mb[j] is the chunk's block maximum after the cross-lane / cross-wave reductions.
__device__ __forceinline__ void write_piece_max(const DecodeParams &p, size_t row, int c0, int cg, int wv, int kc,
                                                const float *mb) {
  const int SBS = p.SBS;
  float *dst = p.pmax + row * p.npieces;
  if (SBS <= 64) {
    const bool first = SBS == 16 || (SBS == 32 ? (kc & 1) == 0 : kc == 0);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int jb = div_pow2((c0 + j) * 64 + 16 * kc, SBS);
      if (first && jb < p.npieces) dst[jb] = mb[j];
    }
  } else if (SBS <= 512) {
    const int wpb = max(SBS >> 7, 1);  // waves per block
    const int jb = div_pow2(c0 * 64, SBS);
    if (kc == 0 && (wv & (wpb - 1)) == 0 && jb < p.npieces) dst[jb] = mb[0];
  } else if (kc == 0 && wv == 0 && cg < p.npieces) {
    dst[cg] = mb[0];
  }
}

enum { kContig = 0, kPaged = 1 };

// ---------------------------------------------------------------------------
// Page-internal order of the paged pools (one (page, KV head) block each).  The
// decode reads every block with 16-byte-per-lane loads; lane L = 16 kc + mrow of an
// instruction reads the L-th 16-byte piece of one contiguous 1 KB (or 256 B) block, so
// each load instruction covers whole cache lines.  t = token in the page (0..63).
// ---------------------------------------------------------------------------
// residual [64 tokens][128 ch] fp8 -> [8 blocks (tau, h)][64 lanes (kc, mrow)][16 B]:
// tile tau = t & 3 holds tokens 4 mrow + tau, lane kc its channels 32 kc + 16 h + (0..15)
__host__ __device__ constexpr uint32_t res_off(int t, int c) {
  return (uint32_t)((((t & 3) * 2 + ((c >> 4) & 1)) * 64 + (c >> 5) * 16 + (t >> 2)) * 16 + (c & 15));
}
// V^T [128 columns][64 tokens] bf16 -> [16 blocks (nu, kap)][64 lanes (kc, n)][8 tokens]:
// element index of column c, token t (the P.V B operand of lane (n, kc), K-chunk kap)
__host__ __device__ constexpr uint32_t vt_off(int c, int t) {
  return (uint32_t)((((c >> 4) * 2 + ((t >> 3) & 1)) * 64 + (t >> 4) * 16 + (c & 15)) * 8 + (t & 7));
}
// q2 codes [4 groups][64 tokens][8 B] -> [2 blocks h][64 lanes (g, mrow)][2 tokens][8 B]:
// byte offset of the 8 code bytes of group g, token t (tokens 4 mrow + 2h, + 1 per lane)
__host__ __device__ constexpr uint32_t codes_off(int g, int t) {
  return (uint32_t)(((((t >> 1) & 1) * 64 + g * 16 + (t >> 2)) * 2 + (t & 1)) * 8);
}
// g32 scale / zero [4 groups][64 slots] f16 -> [2 h][4 groups][4 kc][8 slots]: element
// index of slot s of group g (a token's slot is scale_pos(t))
__host__ __device__ constexpr uint32_t gscale_off(int g, int s) {
  return (uint32_t)(((((s >> 3) & 1) * 4 + g) * 4 + (s >> 4)) * 8 + (s & 7));
}
// 4-bit codes [64 tokens][64 B] -> [4 blocks tau][64 lanes (kc, mrow)][16 B]: byte offset
// of byte b (channels 2b, 2b + 1) of token t
__host__ __device__ constexpr uint32_t k4_off(int t, int b) {
  return (uint32_t)(((t & 3) * 64 + (b >> 4) * 16 + (t >> 2)) * 16 + (b & 15));
}
// Pool page of position P of sequence b for the append kernels, or -1 (nothing is written) when
// P lies outside the block table's row or the table names a page outside [0, num_pages).
__device__ __forceinline__ int append_page(const int32_t *bt, int bt_stride, int num_pages, int b, int P) {
  if (P < 0 || (P >> 6) >= bt_stride) return -1;
  const int page = bt[(size_t)b * bt_stride + (P >> 6)];
  return (unsigned)page < (unsigned)num_pages ? page : -1;
}
// A decode workgroup whose 512 tokens all lie past its sequence's end (ragged batches) writes
// its survivor-mask bytes (all 0) and nothing else: the merge reads no partial slot past the
// sequence end, and the threshold is written by the sequence's first workgroup.
__device__ __forceinline__ void write_empty_mask(int8_t *mask_row, int cg, int SBS, int ntbs, int span = kChunksPerWG) {
  if (SBS > span * kPage) {  // a block of several spans: its first span writes its byte
    const int jb = div_pow2(cg * span * kPage, SBS);
    if (threadIdx.x == 0 && ((cg * span * kPage) & (SBS - 1)) == 0 && jb < ntbs) mask_row[jb] = 0;
    return;
  }
  const int nblk = div_pow2(span * kPage, SBS);
  for (int t = threadIdx.x; t < nblk; t += blockDim.x) {
    const int jb = cg * nblk + t;
    if (jb < ntbs) mask_row[jb] = 0;
  }
}
// 2^x on the hardware exponential (v_exp_f32, about 1 ulp).  The arguments are differences of
// log2-scaled scores, x <= 0; a result below 2^-126, which exp2f would return as a denormal after
// a range fix-up (five more instructions), is 0 here: far below the fp16 P operand's 2^-24 and the
// fp32 sums' resolution.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// exp2 softmax partial of one 64-token chunk in the exact pass.  Each lane holds the refined raw
// scores R[k] of 16 tokens of one query row (token 16 kc + k; the row's 64 tokens lie in the four
// lanes l, l ^ 16, l ^ 32, l ^ 48); its tokens k < nact are active (valid, in a kept prune block, a
// row of the group).  P[k] = 2^(s_k - m) for active tokens and 0 otherwise, with s = R * cs1 *
// log2(e) and m the row's maximum over active tokens; lsum = sum of P over the row.  When every lane
// of the wave has all 16 active (a full page of a kept block) a copy without the masks runs, so that
// no per-token compare or select sits on the exact pass's chain.
template <bool SPLIT = true>
__device__ __forceinline__ void chunk_softmax(const float *R, float cs1, int nact, float *P, float &mrow_max,
                                              float &lsum) {
  mrow_max = -INFINITY;
  lsum = 0.f;
  auto body = [&](auto FULL) {
    constexpr bool kFull = decltype(FULL)::value;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      P[k] = (R[k] * cs1) * kLog2e;
      mrow_max = (kFull || k < nact) ? fmaxf(mrow_max, P[k]) : mrow_max;
    }
    mrow_max = xor_max(mrow_max, 16);
    mrow_max = xor_max(mrow_max, 32);
#pragma unroll
    for (int k = 0; k < 16; ++k) {  // a row without an active token never reads its -inf maximum
      P[k] = (kFull || k < nact) ? exp2_hw(P[k] - mrow_max) : 0.f;
      lsum += P[k];
    }
  };
  if (SPLIT && __builtin_amdgcn_ballot_w64(nact == 16) == __builtin_amdgcn_read_exec())
    body(std::true_type());
  else
    body(std::false_type());
  lsum = xor_sum(lsum, 16);
  lsum = xor_sum(lsum, 32);
}

// AND masks of a lane's V^T words (P.V B operand, K-chunk kap: tokens 16 kc + 8 kap + (0..7), two
// per word) that keep only the first nvs tokens of a partial page: the pool slots past the sequence
// end are not data (they may hold NaN patterns, which a zero P would not cancel)
__device__ __forceinline__ void partial_page_masks(int kc, int nvs, u32x4 *keepw) {
#pragma unroll
  for (int kap = 0; kap < 2; ++kap)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int tk = 16 * kc + 8 * kap + 2 * e;
      keepw[kap][e] = (tk < nvs ? 0x0000ffffu : 0u) | (tk + 1 < nvs ? 0xffff0000u : 0u);
    }
}

// per-channel scales (fp16: dequantized by packed fp16 FMAs, exact), g32 scales, and per-channel
// scales of other dtypes (fp32 / bf16: dequantized in fp32 as the reference does)
enum { kChannel = 0, kG32 = 1, kChannelF32 = 2 };
enum { kResNone = 0, kResE4M3 = 1, kResE5M2 = 2 };
enum { kVF16 = 0, kVBF16 = 1 };

// 8 fp8 residual bytes -> 8 fp16 (exact)
template <int RES>
__device__ __forceinline__ f16x8 fp8x8_to_f16x8(uint32_t lo, uint32_t hi) {
  u32x4 r;
  if constexpr (RES == kResE5M2) {
    // e5m2 is the high byte of the fp16 with the same value
    r[0] = __builtin_amdgcn_perm(lo, lo, 0x010c000cu);
    r[1] = __builtin_amdgcn_perm(lo, lo, 0x030c020cu);
    r[2] = __builtin_amdgcn_perm(hi, hi, 0x010c000cu);
    r[3] = __builtin_amdgcn_perm(hi, hi, 0x030c020cu);
  } else {
    f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, false);
    f16x2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, true);
    f16x2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, false);
    f16x2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, true);
    r[0] = __builtin_bit_cast(uint32_t, a);
    r[1] = __builtin_bit_cast(uint32_t, b);
    r[2] = __builtin_bit_cast(uint32_t, c);
    r[3] = __builtin_bit_cast(uint32_t, d);
  }
  return __builtin_bit_cast(f16x8, r);
}

// The same 8 residual bytes in the element order of the reference-layout score operands: channel
// pairs (0,2) (4,6) (1,3) (5,7)
template <int RES>
__device__ __forceinline__ f16x8 fp8x8_to_f16x8_perm(uint32_t lo, uint32_t hi) {
  u32x4 r;
  if constexpr (RES == kResE5M2) {
    r[0] = __builtin_amdgcn_perm(lo, lo, 0x020c000cu);
    r[1] = __builtin_amdgcn_perm(hi, hi, 0x020c000cu);
    r[2] = __builtin_amdgcn_perm(lo, lo, 0x030c010cu);
    r[3] = __builtin_amdgcn_perm(hi, hi, 0x030c010cu);
  } else {
    const uint32_t x = __builtin_amdgcn_perm(lo, lo, 0x03010200u);  // bytes 0, 2, 1, 3
    const uint32_t y = __builtin_amdgcn_perm(hi, hi, 0x03010200u);
    r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, false));
    r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(y, 1.0f, false));
    r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, true));
    r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(y, 1.0f, true));
  }
  return __builtin_bit_cast(f16x8, r);
}

// B operand of a P.V MFMA from a V tile staged row-major in LDS (token rows of `pitch` bytes):
// lane (kc, n) needs V[16 kc + 8 kap + e][16 nl + n], e = 0..7, i.e. a column of the tile.
// ds_read_b64_tr_b16 (gfx950) transposes inside each 16-lane group: lane i receives element i % 4
// of the 4-element rows addressed by lanes i / 4 + 4 e' (e' = 0..3).  So lane n addresses token
// 16 kc + 8 kap + n / 4 (+ 4 for the second read) at column 16 nl + 4 (n % 4), and receives its
// column's tokens e = 0..3 (then 4..7); two reads per operand instead of eight 2-byte reads.
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 vt_operand_lds(const uint8_t *st, int pitch, int nl, int kap, int kc, int n) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const uint32_t off = (uint32_t)((16 * kc + 8 * kap + (n >> 2)) * pitch + (16 * nl + 4 * (n & 3)) * 2);
  const auto *p0 = (const lds_s16x4 *)((__attribute__((address_space(3))) const uint8_t *)st + off);
  const auto *p1 = (const lds_s16x4 *)((__attribute__((address_space(3))) const uint8_t *)st + off + 4 * pitch);
  const u32x2 a = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)p0));
  const u32x2 b = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)p1));
  return u32x4{a[0], a[1], b[0], b[1]};
}

// P.V runs on fp16 operands whatever V's storage type, as the reference's decode kernels cast
// both p and v to fp16 before the product (attn_kernel_v1210_fused_bsz_q2fp8.py:130-131 and the
// same lines of the fp8fp8 / nvfp4fp8 / nf4fp8 kernels): fp16 P keeps 11 significant bits, and
// bf16 V is rounded to fp16 (round to nearest even) in registers.
template <int VT>
struct VTraits;
template <>
struct VTraits<kVF16> {
  typedef f16x8 vec;
  __device__ static __forceinline__ f32x4 mfma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack2(float x, float y) {
    return pk_f16_bits(x, y);
  }
  // 8 stored V elements (4 words) -> the B operand
  __device__ static __forceinline__ vec operand(u32x4 w) { return __builtin_bit_cast(vec, w); }
};
template <>
struct VTraits<kVBF16> : VTraits<kVF16> {
  __device__ static __forceinline__ vec operand(u32x4 w) {
    u32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = __uint_as_float(w[e] << 16), hi = __uint_as_float(w[e] & 0xffff0000u);
      r[e] = pk_f16_bits(lo, hi);
    }
    return __builtin_bit_cast(vec, r);
  }
};

// 16 consecutive elements of a float tensor (dtype 0=f16, 1=bf16, 2=f32): four raw 16-byte
// loads whatever the dtype (16-bit data uses the first two), conversion afterwards.
struct Raw16 {
  uint4 v[4];
};
// 16 elements of element size es (2 or 4 bytes) at byte offset off of a resource of `bytes`
// bytes.  All four loads are issued whatever the dtype: for 16-bit dtypes the upper two read at
// `bytes`, past the resource (zeros, no memory access), and are OR-ed into the lower two.  Every
// load then has a use on every dtype path, so the compiler neither moves the f32-only loads into
// that path, behind loads issued later, nor counts them among the outstanding loads of the other
// paths: the waits for the window stay exact and do not wait for the cache loads behind it.
__device__ __forceinline__ void raw16_load(Raw16 &r, brsrc rs, uint32_t off, uint32_t es, uint32_t bytes) {
  r.v[0] = bload16(rs, off);
  r.v[1] = bload16(rs, off + 16);
  r.v[2] = bload16(rs, es == 4 ? off + 32 : bytes);
  r.v[3] = bload16(rs, es == 4 ? off + 48 : bytes);
}
__device__ __forceinline__ void raw16_to_f32(const Raw16 &r, int dt, float *out) {
  if (dt == 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[4 * i + 0] = __uint_as_float(r.v[i].x);
      out[4 * i + 1] = __uint_as_float(r.v[i].y);
      out[4 * i + 2] = __uint_as_float(r.v[i].z);
      out[4 * i + 3] = __uint_as_float(r.v[i].w);
    }
  } else if (dt == 1) {  // one uniform branch per dtype, not a select per element
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      // r.v[i + 2] is zero for 16-bit dtypes (see raw16_load)
      const uint32_t w[4] = {r.v[i].x | r.v[i + 2].x, r.v[i].y | r.v[i + 2].y, r.v[i].z | r.v[i + 2].z,
                             r.v[i].w | r.v[i + 2].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        out[8 * i + 2 * k] = __uint_as_float(w[k] << 16);
        out[8 * i + 2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      // r.v[i + 2] is zero for 16-bit dtypes (see raw16_load)
      const uint32_t w[4] = {r.v[i].x | r.v[i + 2].x, r.v[i].y | r.v[i + 2].y, r.v[i].z | r.v[i + 2].z,
                             r.v[i].w | r.v[i + 2].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        out[8 * i + 2 * k] = f16_bits_to_f32(w[k] & 0xffffu);
        out[8 * i + 2 * k + 1] = f16_bits_to_f32(w[k] >> 16);
      }
    }
  }
}

__device__ __forceinline__ uint32_t f16x2_bits(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ f16x2 bits_f16x2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }

__device__ __forceinline__ f16x8 add_f16x8(f16x8 a, f16x8 b) { return a + b; }

// stage 2: log-sum-exp merge of the per-workgroup partials (defined in q2fp8_decode.hip):
// launches the merge kernel suited to the batch on stream st
hipError_t launch_merge(const DecodeParams &p, hipStream_t st);
// CUs of the current device (queried once per device; 0 when the query fails)
int device_cus();

}  // namespace ffa
