// q2fp8 pruned decode attention for gfx950 (MI355X).
//
// Semantics follow ffa-q2fp8/attn_kernel/attn_kernel_v1210_fused_bsz_q2fp8.py
// (stage 1 :10-139, stage 2 :142-171): coarse scores from 2-bit K, a
// threshold from two 16-token probe windows (incl. the "(NTB-1)*16" window of
// :70-73), group prune ("prune iff every query row of the GQA group is below
// its threshold", :99-102), refined scores with the fp8 residual for kept
// blocks, exp2 partial softmax and P.V, and a log-sum-exp merge.
//
// Design (one workgroup = 4 waves = 4 consecutive 64-token chunks of one
// (sequence, KV head); a chunk is one page in the paged layout):
//   * score pass: v_mfma_f32_16x16x32_f16 with the 2-bit codes as the A
//     operand.  A code c sitting at bit 2p of a 16-bit lane half is the fp16
//     subnormal c * 2^(2p-24); the matching q element is pre-divided by 4^p,
//     so unpacking is one AND per two codes.  Rows of the MFMA are tokens,
//     columns are (group j, query row i): the B operand holds q_i only on the
//     channels of group j, so the four 32-channel groups come out separately
//     and their per-token g32 scale/zero are applied in the epilogue
//     (q.(c*s+z) = s*(q.c) + z*sum(q)).
//   * prune: block max per row -> compare with the threshold -> wave ballot.
//   * exact pass (kept chunks only): refined score = coarse score + q.r with
//     r the fp8 residual (another f16 MFMA), exp2 softmax, P.V with a bf16/f16
//     MFMA reading V^T pages (16-byte loads) or V staged through LDS for the
//     contiguous reference layout.
//   * the 8 chunk partials (m, l, o) of a workgroup are merged in LDS into one
//     partial per 512 tokens; a second kernel merges those with one batch of
//     loads (back to back in a HIP graph).  Merging in the last-arriving
//     workgroup of each (sequence, KV head) instead was measured slower: the
//     release needs an L2 write-back per workgroup (__threadfence), or, with
//     device-scope stores and loads, the arrival atomic and the device-scope
//     loads of one workgroup take longer than the kernel boundary plus a
//     128-workgroup merge launch.
//   * the q operands of the MFMAs are built once per workgroup (one per wave)
//     and shared through LDS.
//   * each wave owns two consecutive chunks; the grid is 1-D with the
//     workgroup index along the sequence fastest, so consecutive workgroups of
//     one (sequence, KV head) go to different XCDs and its kept chunks'
//     residual/V traffic spreads over every XCD's memory path.
#include "decode_common.h"
#include "ffa_mi355x.h"

#include <stdio.h>

#include <mutex>
#include <type_traits>

// Timeline build (compiled with -DFFA_TIMELINE, never in the library that ffa_mi355x.build makes):
// each wave records s_memrealtime (the 100 MHz constant clock) at the points STAMP marks and, at
// its end, 16 words per wave into the buffer ffa_debug_set_timeline sets: stamps 0-12, then the
// kept chunks it refined, the workgroup's kept chunks, and (XCC_ID << 32 | HW_ID).  The stamps are
// SMEM reads that share lgkmcnt with LDS, so they shift what they measure by a little.
#ifdef FFA_TIMELINE
__device__ unsigned long long *g_timeline = nullptr;
#define FFA_STAMP(i) (st_[i] = __builtin_amdgcn_s_memrealtime())
#else
#define FFA_STAMP(i) ((void)0)
#endif

namespace ffa {

// A-operand words of the score MFMAs from 16 packed codes (one 32-bit word).
// s = 0: codes (q, q+8) at bits (2q, 16+2q) -> value c * 4^q * 2^-24
// s = 1: same for codes (4+q, 12+q) after a shift by 8.
__device__ __forceinline__ f16x8 codes_to_f16x8(uint32_t w, int s) {
  const uint32_t y = s ? (w >> 8) : w;
  u32x4 r;
  r[0] = y & 0x00030003u;
  r[1] = y & 0x000c000cu;
  r[2] = y & 0x00300030u;
  r[3] = y & 0x00c000c0u;
  return __builtin_bit_cast(f16x8, r);
}

// Reference-layout dequantization of 16 channels (one 32-bit code word, code i at bits 2i) into
// the A operands of two score MFMAs, for fp16 scale / zero: k_hat = fp16(c * s + z) with one
// rounding.  The reference computes fp16(fp32(fp32(c * s) + z)) with s and z in fp32
// (attn_kernel_v1210_fused_bsz_q2fp8.py:50-53, 93).  For fp16 s and z, c * s (at most 13
// significant bits) is exact in fp32, and the two results differ only where the fp32 sum drops a
// zero point below 2^-23 of c * s and c * s lies on an fp16 rounding midpoint (checked against
// every finite fp16 z and c = 1..3 over a stride of the fp16 scales: no difference with
// |z| >= 2^-23 c s).  Other
// scale dtypes take dequant8_channel_f32.  A code zero-extended to a
// nibble is the e2m1 value c/2, so the hardware fp4 conversion with scale 2 yields c exactly, two
// codes per instruction: masking with 0x33 leaves codes 4k and 4k+2 in the nibbles of byte k.
// Element order inside each 8 channels: kChanPerm pairs (0,2) (4,6) (1,3) (5,7); the q operand,
// the (s, z) pairs sp / zp (4 per operand) and the residual follow the same order.
__device__ __forceinline__ void dequant16_channel(uint32_t w, const uint32_t *sp, const uint32_t *zp, f16x8 &k0,
                                                  f16x8 &k1) {
  const uint32_t e = w & 0x33333333u;         // byte k: codes 4k, 4k + 2
  const uint32_t o = (w >> 2) & 0x33333333u;  // byte k: codes 4k + 1, 4k + 3
  const f16x2 c[8] = {__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(e, 2.0f, 0), __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(e, 2.0f, 1),
                      __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(o, 2.0f, 0), __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(o, 2.0f, 1),
                      __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(e, 2.0f, 2), __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(e, 2.0f, 3),
                      __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(o, 2.0f, 2), __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(o, 2.0f, 3)};
  u32x4 r0, r1;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    r0[q] = f16x2_bits(__builtin_elementwise_fma(c[q], bits_f16x2(sp[q]), bits_f16x2(zp[q])));
    r1[q] = f16x2_bits(__builtin_elementwise_fma(c[4 + q], bits_f16x2(sp[4 + q]), bits_f16x2(zp[4 + q])));
  }
  k0 = __builtin_bit_cast(f16x8, r0);
  k1 = __builtin_bit_cast(f16x8, r1);
}
// channel (within 8) of each element of a reference-layout score operand
__host__ __device__ constexpr int kChanPerm(int e) { return (e & 1) * 2 + ((e >> 1) & 1) * 4 + (e >> 2); }

// The same dequantization for fp32 scale / zero (and bf16, whose values fp16 cannot always
// hold): k_hat = fp16(fp32(fp32(c * s) + z)), two fp32 roundings and one fp16 rounding, as the
// reference computes it (attn_kernel_v1210_fused_bsz_q2fp8.py:52-53, 93).  One operand (8
// channels) at a time: HALF = 0 takes codes 0-7 of the word (bytes 0, 1), HALF = 1 codes 8-15.
// sz holds the operand's (s, z) in element order: [0], [1] = s of elements 0-3, 4-7; [2], [3] = z.
template <int HALF>
__device__ __forceinline__ f16x8 dequant8_channel_f32(uint32_t w, const float4 *sz) {
#pragma clang fp contract(off)
  const uint32_t e = w & 0x33333333u;
  const uint32_t o = (w >> 2) & 0x33333333u;
  constexpr int b0 = 2 * HALF;
  // element pairs (0,1) (2,3) (4,5) (6,7) <-> codes (8h+0, 8h+2) (8h+4, 8h+6) (8h+1, 8h+3) (8h+5, 8h+7)
  const f32x2 c[4] = {__builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e, 2.0f, b0), __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e, 2.0f, b0 + 1),
                      __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(o, 2.0f, b0), __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(o, 2.0f, b0 + 1)};
  const float sv[8] = {sz[0].x, sz[0].y, sz[0].z, sz[0].w, sz[1].x, sz[1].y, sz[1].z, sz[1].w};
  const float zv[8] = {sz[2].x, sz[2].y, sz[2].z, sz[2].w, sz[3].x, sz[3].y, sz[3].z, sz[3].w};
  u32x4 r;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float a0 = c[q][0] * sv[2 * q], a1 = c[q][1] * sv[2 * q + 1];
    r[q] = pk_f16_bits(a0 + zv[2 * q], a1 + zv[2 * q + 1]);
  }
  return __builtin_bit_cast(f16x8, r);
}

// Position of token t (0..63) inside a page row of g32 scales / zeros.  Tile-major:
// the scores of MFMA tile tau hold tokens 16k + 4u + tau (u = 0..3), whose scales
// then sit at 16k + 4tau + u, one 8-byte load per lane and tile.
__host__ __device__ constexpr int scale_pos(int t) { return 16 * (t >> 4) + 4 * (t & 3) + ((t >> 2) & 3); }

// OCC = 4 asks the compiler for four waves per SIMD (at most 128 registers), so that four
// workgroups share a CU (29 KB of LDS each): used when the grid has more workgroups than two per
// CU can hold (large batches), where it trades a few spilled registers for two more workgroups
// in flight.
// SPEC (the builds for two-chunk spans, q2fp8_decode_2span_kernel: paged g32 and the contiguous
// per-channel layouts): waves 2 and 3 own the two chunks and score them and the probe windows;
// waves 0 and 1, which would own none, load the residual and V rows of chunk wv (the chunk of wave
// wv + 2) right after the operand barrier, before the prune decides it, and refine that chunk from
// their registers if it is kept.
template <int LAYOUT, int SMODE, int RES, int VT, int OCC, bool SPEC>
__device__ __forceinline__ void q2fp8_decode_body(const DecodeParams &p) {
  static_assert(!SPEC || (OCC == 1 && (LAYOUT == kPaged) == (SMODE == kG32)),
                "the two-chunk builds: paged g32, contiguous per-channel");
  typedef VTraits<VT> VTr;
#ifdef FFA_TIMELINE
  unsigned long long st_[16] = {0};
  int n_exact_ = 0;
#endif
  constexpr bool kG = SMODE == kG32;
  constexpr bool kCF = SMODE == kChannelF32;  // per-channel fp32 / bf16 scales: dequantized in fp32
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // grid (span, KV head, sequence); the paged layouts (small grids aside) place the workgroups
  // with the KV head fastest, so that a (sequence, KV head)'s partials stay in one XCD's L2 for
  // the merge (grid_pos)
  const GridPos gp = grid_pos<LAYOUT == kPaged>();
  const int cg = gp.cg;  // workgroup index along the sequence = partial slot
  const DecodeUnit un = decode_unit(p, gp.y);  // KV head and the (at most 4) query rows of this workgroup
  const int hkv = un.hkv;
  const int b = gp.b;
  // span: chunks of this workgroup (8, or 4 / 2 for small grids, where each wave owns one chunk and
  // waves past the span own none); slot (w, j) = wave w's j-th chunk
  const int span = SPEC ? kMinSpan : decode_span(p);
  const int ppw = span >= kChunksPerWG ? kPPW : 1;
  const int cw = cg * span;  // first chunk of the workgroup
  // the wave's place in the chunk order: its own index, or (SPEC) waves 2, 3 first
  const int wch = SPEC ? (wv ^ 2) : wv;
  const int c0 = cw + wch * ppw;  // first chunk scored by this wave
  const int SBS = p.SBS;
  bool own[kPPW];
#pragma unroll
  for (int j = 0; j < kPPW; ++j) own[j] = j < ppw && wch * ppw + j < span;
  auto slot_chunk = [&](int sl) { return cw + (sl >> 1) * ppw + (sl & 1); };  // chunk of slot sl
  auto slot_owned = [&](int sl) { return (sl & 1) < ppw && (sl >> 1) * ppw + (sl & 1) < span; };

  const int mrow = lane & 15;  // MFMA row (A) / column (B) index
  const int kc = lane >> 4;    // k-chunk of the operands == channel group of the A lane
  const int n = mrow;          // output column = (j, i)
  const int jg = n >> 2;
  const int ir = n & 3;
  const bool row_ok = ir < un.Gu;
  const int hq = un.row0 + (row_ok ? ir : 0);

  __shared__ uint4 s_qr[4][64];                    // B operands of the 4 residual MFMAs (g32)
  __shared__ uint4 s_sp[kG || kCF ? 1 : 4][kG || kCF ? 1 : 64];   // channel scales: fp16 (scale, scale) pairs of 8 channels
  __shared__ uint4 s_zp2[kG || kCF ? 1 : 4][kG || kCF ? 1 : 64];  // channel scales: fp16 (zero, zero) pairs
  // fp32 channel scales: [channel group kc][operand][s of elements 0-3, 4-7, z of 0-3, 4-7] (the
  // lanes of one kc share them: broadcast reads)
  __shared__ float4 s_cf[kCF ? 4 : 1][kCF ? 4 : 1][4];
  __shared__ float s_probe[2][4];
  __shared__ float s_wmax[kWaves][4];
  __shared__ int s_keep[kChunksPerWG * kPage / 16];  // pass 2: block decisions of the span
  __shared__ int s_kept[kChunksPerWG];             // chunk kept (some prune block survives)
  __shared__ int s_pgid[kChunksPerWG];             // pool page of the chunk
  __shared__ uint32_t s_bal[kChunksPerWG][2];      // survivor ballot of the chunk
  // g32: coarse scores of kept chunks, [q4][4 kc + row]: after the group sums the four lanes of a
  // query row (one per group) hold its scores, and only group 0's lanes reach the partials
  __shared__ float4 s_R[kG ? kChunksPerWG : 1][4][16];
  __shared__ uint64_t s_x[kG ? 1 : kChunksPerWG][kG ? 1 : 4][kG ? 1 : 64];  // channel: codes of kept chunks
  __shared__ float s_pm[kChunksPerWG][4], s_pl[kChunksPerWG][4];
  __shared__ float s_am[kWaves][4], s_al[kWaves][4];  // mean-V: pruned-token mass per wave and row
  __shared__ __attribute__((aligned(16))) float s_po[kChunksPerWG][4][128];
  // B operands of the 4 score MFMAs, per lane: read once after the operand barrier, long
  // before the exact pass writes s_po (two barriers later), so they share its storage
  uint4(*const s_qa)[64] = reinterpret_cast<uint4(*)[64]>(&s_po[0][0][0]);
  // g32: partial sums of q16 over 8 channels (read with the operands), after s_qa
  float(*const s_zs)[64] = reinterpret_cast<float(*)[64]>(&s_po[2][0][0]);
  __shared__ __attribute__((aligned(16))) uint8_t s_vstage[LAYOUT == kContig ? kWaves * kPage * kVRowHalf : 16];

  // Workgroup barrier for LDS traffic only: __syncthreads() would also wait for every
  // outstanding global load of the wave (s_waitcnt vmcnt(0)), serialising the page loads
  // issued ahead of it.
  auto lds_barrier = []() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

  // ------------------------------------------------ phase 1: loads
  // Every vector load is issued on every path; validity (sequence end, kept or pruned) is
  // the size of the buffer resource, so the compiler waits for one load group at a time.
  // Groups are issued in the order they are consumed: page ids (paged layout), q window (and
  // channel scales), the caller's threshold, probe windows, page 0, page 1.
  // The q window is channels [32kc + 16h, +16) of the lane's row, h = wave / 2: it holds
  // every element of the operand this wave builds.
  const int Tb = p.seq_lens ? min(max(p.seq_lens[b], 0), p.T) : p.T;  // lengths beyond T are clamped to T
  if (cg > 0 && cw * kPage >= Tb) {  // every token past the sequence end: mask bytes only
    if (p.pass != 1 && un.quad == 0) write_empty_mask(p.mask + ((size_t)b * p.HKV + hkv) * p.ntbs, cg, SBS, p.ntbs, span);
    return;
  }
  FFA_STAMP(0);
  if (threadIdx.x < kChunksPerWG * kPage / 16) s_keep[threadIdx.x] = 0;
  const int NTB = div_bs(p, Tb + p.BS - 1);
  const int NTBS_b = NTB * div_pow2(p.BS, p.SBS);
  // probe windows: waves 0 and 1 (SPEC: 2 and 3, which score)
  const bool do_probe = (p.th_in == nullptr) && wch < 2;
  const int pa = wch == 0 ? 0 : max(NTB - 1, 0) * 16;  // probe window (attn_kernel...q2fp8.py:58-73)
  int nv[kPPW];  // valid tokens of the wave's chunks (0 for a chunk it does not own)
#pragma unroll
  for (int j = 0; j < kPPW; ++j) nv[j] = own[j] ? min(max(Tb - (c0 + j) * kPage, 0), kPage) : 0;
  // SPEC: the chunk whose residual and V^T waves 0 and 1 load (chunk wv), and its valid tokens
  const int lc = cw + (wv & 1);
  const int nl = SPEC && wv < 2 ? min(max(Tb - lc * kPage, 0), kPage) : 0;

  int pg[kPPW] = {0, 0};
  int ppg = 0;
  uint32_t pg_lane = 0;
  if constexpr (LAYOUT == kPaged) {
    // page ids: one vector load per wave, issued first (lanes 0, 1: the wave's chunks, lane 2: its
    // probe window; the other lanes read past the resource and get 0)
    // (SPEC, waves 0 and 1: lane 0 reads the page of chunk lc)
    const bool ld = SPEC && wv < 2;
    const bool need = lane < kPPW ? (ld ? lane == 0 && nl > 0 : nv[lane & 1] > 0) : (lane == kPPW && do_probe && pa < Tb);
    const int idx = lane < kPPW ? (ld ? lc : c0 + lane) : (pa >> 6);
    pg_lane = bload4(make_rsrc(p.bt + (size_t)b * p.bt_stride, p.bt_stride * 4), need ? idx * 4 : p.bt_stride * 4);
    pg_lane = pg_lane < (uint32_t)p.num_pages ? pg_lane : 0u;  // ids outside the pools read page 0
  }
  const uint32_t es_q = p.q_dtype == 2 ? 4u : 2u;
  const int hwin = wv >> 1;
  Raw16 qraw, sraw, zraw;
  raw16_load(qraw, make_rsrc((const char *)p.q + (size_t)b * p.HQ * kD * es_q, p.HQ * kD * es_q),
             (hq * kD + 32 * kc + 16 * hwin) * es_q, es_q, p.HQ * kD * es_q);
  if constexpr (!kG) {
    const uint32_t es_s = p.s_dtype == 2 ? 4u : 2u;
    const size_t so = ((size_t)b * p.HKV + hkv) * kD * es_s;
    raw16_load(sraw, make_rsrc((const char *)p.ks + so, kD * es_s), (32 * kc + 16 * hwin) * es_s, es_s, kD * es_s);
    raw16_load(zraw, make_rsrc((const char *)p.kz + so, kD * es_s), (32 * kc + 16 * hwin) * es_s, es_s, kD * es_s);
  }
  // caller's threshold of the lane's query row (zeros when none is given)
  const float th_pre = __uint_as_float(
      bload8(make_rsrc(p.th_in + (p.th_in ? (size_t)b * p.HQ : 0), p.th_in ? p.HQ * 4 : 0), hq * 4).x);
  // the q (and channel scale) loads go out before the wait for the page ids and before the code
  // loads, whose waits would otherwise cover them
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (LAYOUT == kPaged) {
#pragma unroll
    for (int j = 0; j < kPPW; ++j) pg[j] = __builtin_amdgcn_readlane(pg_lane, j);
    ppg = __builtin_amdgcn_readlane(pg_lane, kPPW);
    FFA_STAMP(1);
  }
  // probe tile: MFMA row m <-> token pa + 4(m & 3) + (m >> 2), so that the output rows
  // 4kc + u hold tokens pa + 4u + kc, whose g32 scales are contiguous (scale_pos)
  uint64_t px;
  uint2 pgs = make_uint2(0, 0), pgz = make_uint2(0, 0);
  {
    const int tok = pa + 4 * (mrow & 3) + (mrow >> 2);
    const bool pv = do_probe && pa < Tb;
    if constexpr (LAYOUT == kPaged) {
      const size_t blk = (size_t)ppg * p.HKV + hkv;
      px = bload8u(make_rsrc(p.kq + blk * (4 * kPage * 8), pv ? 4 * kPage * 8 : 0), codes_off(kc, tok & (kPage - 1)));
      if constexpr (kG) {
        const uint32_t so = gscale_off(jg, (pa & (kPage - 1)) + 4 * kc) * 2;  // 4 consecutive slots
        pgs = bload8(make_rsrc((const uint16_t *)p.ks + blk * (4 * kPage), pv ? 4 * kPage * 2 : 0), so);
        pgz = bload8(make_rsrc((const uint16_t *)p.kz + blk * (4 * kPage), pv ? 4 * kPage * 2 : 0), so);
      }
    } else {
      const int nt = pv ? min(16, Tb - pa) : 0;
      const size_t base = (((size_t)b * p.T + pa) * p.HKV + hkv) * 32;
      px = bload8u(make_rsrc(p.kq + base, nt > 0 ? ((nt - 1) * p.HKV + 1) * 32 : 0), (tok - pa) * p.HKV * 32 + 8 * kc);
    }
  }
  // own chunks: the token of MFMA row m in tile tau is 4m + tau
  uint64_t x[kPPW][4];
  uint4 gs[kPPW][2], gz[kPPW][2];  // g32 scale/zero of group jg, tokens 16kc + 4u + tau at [tau/2].(2 words)
#pragma unroll
  for (int j = 0; j < kPPW; ++j) {
    const int t0 = (c0 + j) * kPage;
    if constexpr (LAYOUT == kPaged) {
      const size_t blk = (size_t)pg[j] * p.HKV + hkv;
      const brsrc rc = make_rsrc(p.kq + blk * (4 * kPage * 8), nv[j] > 0 ? 4 * kPage * 8 : 0);
      // tokens 4 mrow + (0, 1) and 4 mrow + (2, 3) of group kc: two 1 KB blocks, lane-ordered
      const uint4 q0 = bload16_nt(rc, lane * 16), q1 = bload16_nt(rc, (64 + lane) * 16);
      x[j][0] = ((uint64_t)q0.y << 32) | q0.x;
      x[j][1] = ((uint64_t)q0.w << 32) | q0.z;
      x[j][2] = ((uint64_t)q1.y << 32) | q1.x;
      x[j][3] = ((uint64_t)q1.w << 32) | q1.z;
      if constexpr (kG) {
        const brsrc rs = make_rsrc((const uint16_t *)p.ks + blk * (4 * kPage), nv[j] > 0 ? 4 * kPage * 2 : 0);
        const brsrc rz = make_rsrc((const uint16_t *)p.kz + blk * (4 * kPage), nv[j] > 0 ? 4 * kPage * 2 : 0);
        // slots 16 kc + (0..7) and 16 kc + (8..15) of group jg
        const uint32_t so0 = gscale_off(jg, 16 * kc) * 2, so1 = gscale_off(jg, 16 * kc + 8) * 2;
        gs[j][0] = bload16_nt(rs, so0);
        gs[j][1] = bload16_nt(rs, so1);
        gz[j][0] = bload16_nt(rz, so0);
        gz[j][1] = bload16_nt(rz, so1);
      }
    } else {
      const size_t base = (((size_t)b * p.T + t0) * p.HKV + hkv) * 32;
      const brsrc rc = make_rsrc(p.kq + base, nv[j] > 0 ? ((nv[j] - 1) * p.HKV + 1) * 32 : 0);
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) x[j][tau] = bload8u(rc, (4 * mrow + tau) * p.HKV * 32 + 8 * kc);
    }
  }

  // ------------------------------------------------ phase 2a: B operands, built once per workgroup
  // wave w = 2h + s builds, for every lane, the operand of MFMA m' = w (channels relative to
  // the lane's group 32kc):
  //   g32 score:     element 2q+half <-> channel 16h + 4s + q + 8half, times 4^-q
  //   channel score: element e <-> channel 8w + e
  //   residual:      element e <-> channel 8w + e (every column)
  // Score operands are nonzero only on the column's own group (kc == j).
  auto build_operands = [&](auto W) {
    constexpr int w = decltype(W)::value;  // compile-time: only the needed elements are converted
    constexpr int s = w & 1;
    float qv[16];  // channels 32kc + 16h + (0..15)
    raw16_to_f32(qraw, p.q_dtype, qv);
    u32x4 a4, r4;
    if constexpr (kG) {
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const float inv = qq == 0 ? 1.f : (qq == 1 ? 0.25f : (qq == 2 ? 0.0625f : 0.015625f));
        float e2[2];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const float q16 = (float)(_Float16)qv[4 * s + qq + 8 * half];
          e2[half] = (row_ok && kc == jg) ? q16 * inv : 0.f;
        }
        a4[qq] = f32_to_f16_bits(e2[0]) | (f32_to_f16_bits(e2[1]) << 16);
      }
      float zs = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) zs += (float)(_Float16)qv[8 * s + e];
      s_zs[w][lane] = row_ok ? zs : 0.f;
    } else {
      // element order kChanPerm, as dequant16_channel produces the codes
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const float e0 = (row_ok && kc == jg) ? (float)(_Float16)qv[8 * s + kChanPerm(2 * qq)] : 0.f;
        const float e1 = (row_ok && kc == jg) ? (float)(_Float16)qv[8 * s + kChanPerm(2 * qq + 1)] : 0.f;
        a4[qq] = f32_to_f16_bits(e0) | (f32_to_f16_bits(e1) << 16);
      }
      float sv[16], zv[16];
      raw16_to_f32(sraw, p.s_dtype, sv);
      raw16_to_f32(zraw, p.s_dtype, zv);
      if constexpr (kCF) {
        if (mrow == 0) {
          float se[8], ze[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            se[e] = sv[8 * s + kChanPerm(e)];
            ze[e] = zv[8 * s + kChanPerm(e)];
          }
          s_cf[kc][w][0] = make_float4(se[0], se[1], se[2], se[3]);
          s_cf[kc][w][1] = make_float4(se[4], se[5], se[6], se[7]);
          s_cf[kc][w][2] = make_float4(ze[0], ze[1], ze[2], ze[3]);
          s_cf[kc][w][3] = make_float4(ze[4], ze[5], ze[6], ze[7]);
        }
      } else {
        uint32_t spw[4], zpw[4];
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          spw[qq] = f32_to_f16_bits(sv[8 * s + kChanPerm(2 * qq)]) | (f32_to_f16_bits(sv[8 * s + kChanPerm(2 * qq + 1)]) << 16);
          zpw[qq] = f32_to_f16_bits(zv[8 * s + kChanPerm(2 * qq)]) | (f32_to_f16_bits(zv[8 * s + kChanPerm(2 * qq + 1)]) << 16);
        }
        s_sp[w][lane] = make_uint4(spw[0], spw[1], spw[2], spw[3]);
        s_zp2[w][lane] = make_uint4(zpw[0], zpw[1], zpw[2], zpw[3]);
      }
    }
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const float e0 = row_ok ? (float)(_Float16)qv[8 * s + 2 * qq] : 0.f;
      const float e1 = row_ok ? (float)(_Float16)qv[8 * s + 2 * qq + 1] : 0.f;
      r4[qq] = f32_to_f16_bits(e0) | (f32_to_f16_bits(e1) << 16);
    }
    s_qa[w][lane] = make_uint4(a4[0], a4[1], a4[2], a4[3]);
    s_qr[w][lane] = make_uint4(r4[0], r4[1], r4[2], r4[3]);
  };
  switch (wv) {
    case 0: build_operands(std::integral_constant<int, 0>()); break;
    case 1: build_operands(std::integral_constant<int, 1>()); break;
    case 2: build_operands(std::integral_constant<int, 2>()); break;
    default: build_operands(std::integral_constant<int, 3>()); break;
  }
  lds_barrier();
  FFA_STAMP(2);
  // SPEC: waves 0 and 1 load the residual and V^T pages of chunk lc now (after the operand barrier:
  // issued before it, they would sit between the q loads and the operand build's wait).  Nothing
  // these waves wait for before the exact pass comes after them; the chunk waves issue none.
  uint4 srr[4][2], svv[8][2];
  if constexpr (SPEC && LAYOUT == kPaged) {
    if (wv < 2) {
      const size_t blk = (size_t)pg[0] * p.HKV + hkv;
      if constexpr (RES != kResNone) {
        const brsrc rs = make_rsrc(p.kr + blk * (kPage * kD), nl > 0 ? kPage * kD : 0);
#pragma unroll
        for (int tau = 0; tau < 4; ++tau) {
          srr[tau][0] = bload16_nt(rs, ((tau * 2 + 0) * 64 + lane) * 16);
          srr[tau][1] = bload16_nt(rs, ((tau * 2 + 1) * 64 + lane) * 16);
        }
      }
      const brsrc vs = make_rsrc((const uint16_t *)p.v + blk * (kD * kPage), nl > 0 ? kD * kPage * 2 : 0);
#pragma unroll
      for (int nu = 0; nu < 8; ++nu)
#pragma unroll
        for (int kap = 0; kap < 2; ++kap) svv[nu][kap] = bload16_nt(vs, ((nu * 2 + kap) * 64 + lane) * 16);
    }
  } else if constexpr (SPEC) {  // contiguous rows of tokens lc * 64 .. (the exact pass's load pattern)
    if (wv < 2) {
      const size_t row0 = ((size_t)b * p.T + (size_t)lc * kPage) * p.HKV + hkv;
      if constexpr (RES != kResNone) {
        const brsrc rs = make_rsrc(p.kr + row0 * kD, nl > 0 ? ((nl - 1) * p.HKV + 1) * kD : 0);
#pragma unroll
        for (int tau = 0; tau < 4; ++tau) {
          const uint32_t ro = (4 * mrow + tau) * p.HKV * kD + 32 * kc;
          srr[tau][0] = bload16_nt(rs, ro);
          srr[tau][1] = bload16_nt(rs, ro + 16);
        }
      }
      const brsrc vs = make_rsrc((const uint16_t *)p.v + row0 * kD, nl > 0 ? ((nl - 1) * p.HKV + 1) * kD * 2 : 0);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int idx = r * 64 + lane;
        const int tk = idx >> 4, vc = idx & 15;
        svv[r >> 1][r & 1] = bload16_nt(vs, tk * p.HKV * kD * 2 + 16 * vc);
      }
    }
  }
  f16x8 qa[4];
  uint32_t spair[16], zpair[16];
  float zq = 0.f;
#pragma unroll
  for (int mp = 0; mp < 4; ++mp) {
    const uint4 a = s_qa[mp][lane];
    qa[mp] = __builtin_bit_cast(f16x8, u32x4{a.x, a.y, a.z, a.w});
    if constexpr (!kG && !kCF) {
      const uint4 sp = s_sp[mp][lane], zp = s_zp2[mp][lane];
      spair[4 * mp + 0] = sp.x; spair[4 * mp + 1] = sp.y; spair[4 * mp + 2] = sp.z; spair[4 * mp + 3] = sp.w;
      zpair[4 * mp + 0] = zp.x; zpair[4 * mp + 1] = zp.y; zpair[4 * mp + 2] = zp.z; zpair[4 * mp + 3] = zp.w;
    }
  }
  if constexpr (kG) {
    const int src = (jg << 4) | n;  // lane of the column's own group, same query row
    zq = ((s_zs[0][src] + s_zs[1][src]) + (s_zs[2][src] + s_zs[3][src])) * (1.0f / 16777216.f);
  }

  // per-channel k_hat of the lane's 32 channels (two code words) as the four score operands
  auto dequant_tile = [&](uint32_t wlo, uint32_t whi, f16x8 *k) {
    if constexpr (kCF) {
      k[0] = dequant8_channel_f32<0>(wlo, &s_cf[kc][0][0]);
      k[1] = dequant8_channel_f32<1>(wlo, &s_cf[kc][1][0]);
      k[2] = dequant8_channel_f32<0>(whi, &s_cf[kc][2][0]);
      k[3] = dequant8_channel_f32<1>(whi, &s_cf[kc][3][0]);
    } else {
      dequant16_channel(wlo, spair + 0, zpair + 0, k[0], k[1]);
      dequant16_channel(whi, spair + 8, zpair + 8, k[2], k[3]);
    }
  };

  // raw scores of one 16-token tile for the lane's column, summed over groups:
  //   g32: R' = sum_j s_j * D_j + z_j * zq_j   (units of 2^-24 of the dot product)
  //   channel: R = sum_j D_j                    (dot product)
  // s2/z2: fp16 (s, z) of the 4 output rows u, packed (u=0,1), (u=2,3)
  auto score_tile = [&](uint64_t xx, uint32_t s2lo, uint32_t s2hi, uint32_t z2lo, uint32_t z2hi, float *out) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const uint32_t wlo = (uint32_t)xx, whi = (uint32_t)(xx >> 32);
    if constexpr (kG) {
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes_to_f16x8(wlo, 0), qa[0], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes_to_f16x8(wlo, 1), qa[1], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes_to_f16x8(whi, 0), qa[2], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes_to_f16x8(whi, 1), qa[3], acc, 0, 0, 0);
    } else {
      f16x8 k[4];
      dequant_tile(wlo, whi, k);
#pragma unroll
      for (int mp = 0; mp < 4; ++mp) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k[mp], qa[mp], acc, 0, 0, 0);
    }
#pragma unroll
    for (int uu = 0; uu < 4; ++uu) {
      float r;
      if constexpr (kG) {
        const uint32_t sw = uu < 2 ? s2lo : s2hi, zw = uu < 2 ? z2lo : z2hi;
        const float su = f16_bits_to_f32((sw >> (16 * (uu & 1))) & 0xffffu);
        const float zu = f16_bits_to_f32((zw >> (16 * (uu & 1))) & 0xffffu);
        // z * zq as an fma with a zero addend: one mixed-precision op on the fp16 zero
        r = __builtin_fmaf(su, acc[uu], __builtin_fmaf(zu, zq, 0.0f));
      } else {
        r = acc[uu];
      }
      r += dpp<kRowRor4>(r);
      r += dpp<kRowRor8>(r);
      out[uu] = r;
    }
  };
  const float cs1 = kG ? p.scale * 16777216.f : p.scale;  // (R * cs1) * log2e = log2-scaled score

  // ------------------------------------------------ phase 2b: probe, scores, prune
  float R[kPPW][16];
  uint64_t bal[kPPW] = {0, 0};
  float th = INFINITY;

  // probe windows (waves 0 and 1)
  if (do_probe) {
    float r4[4];
    score_tile(px, pgs.x, pgs.y, pgz.x, pgz.y, r4);
    float mx = -INFINITY;
#pragma unroll
    for (int uu = 0; uu < 4; ++uu) {
      const int t = pa + 4 * uu + kc;
      mx = fmaxf(mx, t < Tb ? (r4[uu] * cs1) * kLog2e : -INFINITY);
    }
    mx = xor_max(mx, 16);
    mx = xor_max(mx, 32);
    if (lane < 4) s_probe[wch][lane] = mx;  // lane == ir here
  }

  // R[j][k] = raw score of token (c0+j)*64 + 16kc + k (k = 4u + tau)
  auto score_page = [&](auto J) {
    constexpr int j = decltype(J)::value;
    const int t0 = (c0 + j) * kPage;
    if (nv[j] > 0) {
      const uint32_t sw[8] = {gs[j][0].x, gs[j][0].y, gs[j][0].z, gs[j][0].w,
                              gs[j][1].x, gs[j][1].y, gs[j][1].z, gs[j][1].w};
      const uint32_t zw[8] = {gz[j][0].x, gz[j][0].y, gz[j][0].z, gz[j][0].w,
                              gz[j][1].x, gz[j][1].y, gz[j][1].z, gz[j][1].w};
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) {
        float r4[4];
        score_tile(x[j][tau], sw[2 * tau], sw[2 * tau + 1], zw[2 * tau], zw[2 * tau + 1], r4);
#pragma unroll
        for (int uu = 0; uu < 4; ++uu) R[j][4 * uu + tau] = r4[uu];
      }
      if (t0 + kPage > Tb) [[unlikely]] {  // tokens past the sequence end (page slots hold no data)
#pragma unroll
        for (int k = 0; k < 16; ++k)
          if (t0 + 16 * kc + k >= Tb) R[j][k] = -INFINITY;
      }
    }  // a page past the sequence end leaves R[j] unset: lane_max gives -inf and it is never kept
  };
  // maximum (log2-scaled) of the lane's 16 tokens, reduced over the lanes of one prune block
  // when the block spans several 16-token sub-blocks
  auto lane_max = [&](auto J) -> float {
    constexpr int j = decltype(J)::value;
    if (nv[j] <= 0) return -INFINITY;
    float m = R[j][0];
#pragma unroll
    for (int k = 1; k < 16; ++k) m = fmaxf(m, R[j][k]);
    return (m * cs1) * kLog2e;
  };
  const std::integral_constant<int, 0> J0;
  const std::integral_constant<int, 1> J1;
  score_page(J0);
  score_page(J1);
  float mb[kPPW];  // max of the prune block holding the lane's tokens, per chunk
  mb[0] = lane_max(J0);
  mb[1] = lane_max(J1);
  if (SBS >= 32) {
    mb[0] = xor_max(mb[0], 16);
    mb[1] = xor_max(mb[1], 16);
  }
  if (SBS >= 64) {
    mb[0] = xor_max(mb[0], 32);
    mb[1] = xor_max(mb[1], 32);
  }
  if (SBS >= 128) mb[0] = mb[1] = fmaxf(mb[0], mb[1]);
  if (SBS > 128 && lane < 4) s_wmax[wv][lane] = mb[0];
  FFA_STAMP(3);
  lds_barrier();  // probe maxima (and per-wave block maxima)
  FFA_STAMP(4);
  if (p.th_in != nullptr) {
    th = row_ok ? th_pre : INFINITY;
  } else {
    th = row_ok ? fmaxf(s_probe[0][ir], s_probe[1][ir]) - p.delta : INFINITY;
  }
  if (SBS > 128) {
    const int wpb = min(div_pow2(SBS, kPage * kPPW), kWaves);  // waves per block (a block of several spans: all)
    const int w0 = wv & ~(wpb - 1);  // wpb is 1, 2 or 4
    float m2 = -INFINITY;
    for (int w = w0; w < w0 + wpb; ++w) m2 = fmaxf(m2, s_wmax[w][ir]);
    mb[0] = mb[1] = m2;
  }
  if (p.pass == 1) {  // two-pass decode, first pass: block maxima and thresholds only
    if (row_ok && jg == 0) write_piece_max(p, (size_t)b * p.HQ + hq, c0, cg, wv, kc, mb);
    if (p.th_out != nullptr && cg == 0 && threadIdx.x < un.Gu) p.th_out[(size_t)b * p.HQ + un.row0 + threadIdx.x] = th;
    return;
  }
  if (p.pass == 2) {  // second pass: decide from every row's maxima
    decide_blocks(p, b, hkv, cw, Tb, s_keep);
    lds_barrier();
  }
  // prune iff every row of the group is below its threshold (strict <); rows >= G do not vote
#pragma unroll
  for (int j = 0; j < kPPW; ++j) bal[j] = nv[j] > 0 ? chunk_ballot(p, row_ok, mb[j], th, s_keep, cw, c0 + j, kc) : 0;
  // whether the prune block holding the lane's 16 tokens survives, from a chunk's ballot
  auto lane_kept = [&](uint64_t bl) {
    return SBS == 16   ? ((bl >> (16 * kc)) & 0xffffull) != 0
           : SBS == 32 ? ((bl >> (32 * (kc >> 1))) & 0xffffffffull) != 0
                       : bl != 0;
  };

  // mean-V fallback (attn_kernel_v1210_meanv_bsz_q2fp8.py:109-119): the softmax mass of the
  // wave's pruned tokens on their coarse scores, max am and sum 2^(s - am) per query row (every
  // lane of a row holds its scores; the reductions run over the row's four token quarters)
  if (p.v_mean != nullptr) {
    bool pr[kPPW];
    float am = -INFINITY;
#pragma unroll
    for (int j = 0; j < kPPW; ++j) {
      const int tl = (c0 + j) * kPage + 16 * kc;  // the lane's first token
      pr[j] = row_ok && nv[j] > 0 && !lane_kept(bal[j]);
      if (pr[j]) {
#pragma unroll
        for (int k = 0; k < 16; ++k)
          if (tl + k < Tb) am = fmaxf(am, (R[j][k] * cs1) * kLog2e);
      }
    }
    am = xor_max(am, 16);
    am = xor_max(am, 32);
    float al = 0.f;
#pragma unroll
    for (int j = 0; j < kPPW; ++j) {
      const int tl = (c0 + j) * kPage + 16 * kc;
      if (pr[j]) {
#pragma unroll
        for (int k = 0; k < 16; ++k)
          if (tl + k < Tb) al += exp2_hw((R[j][k] * cs1) * kLog2e - am);
      }
    }
    al = xor_sum(al, 16);
    al = xor_sum(al, 32);
    if (lane < 4) {  // lane == ir
      s_am[wv][lane] = am;
      s_al[wv][lane] = al;
    }
  }

  // publish the kept chunks: coarse scores (g32) or codes (channel scales), page, ballot
#pragma unroll
  for (int j = 0; j < kPPW; ++j) {
    const int slot = wch * kPPW + j;
    const bool kept = nv[j] > 0 && bal[j] != 0;
    if (lane == 0) {
      s_kept[slot] = kept ? 1 : 0;
      s_pgid[slot] = pg[j];
      s_bal[slot][0] = (uint32_t)bal[j];
      s_bal[slot][1] = (uint32_t)(bal[j] >> 32);
    }
    if (kept) {
      if constexpr (kG) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          if (jg == 0) s_R[slot][q4][4 * kc + ir] = make_float4(R[j][4 * q4], R[j][4 * q4 + 1], R[j][4 * q4 + 2], R[j][4 * q4 + 3]);
      } else {
#pragma unroll
        for (int tau = 0; tau < 4; ++tau) s_x[slot][tau][lane] = x[j][tau];
      }
    } else if (lane < 4) {
      s_pm[slot][lane] = -INFINITY;
      s_pl[slot][lane] = 0.f;
    }
  }
  lds_barrier();
  FFA_STAMP(5);

  // ------------------------------------------------ phase 3: exact pass over the kept chunks
  // The i-th kept chunk of the workgroup (in chunk order) goes to wave i % 4, so a
  // workgroup's kept chunks are spread over its waves whichever wave scored them.
  uint32_t km = 0;
#pragma unroll
  for (int sl = 0; sl < kChunksPerWG; ++sl) km |= (s_kept[sl] != 0 ? 1u : 0u) << sl;
  km = __builtin_amdgcn_readfirstlane(km);

  // Survivor mask, one byte per prune block (attn_kernel...q2fp8.py:99-104): final once the chunks
  // are published, so each thread's byte and address are worked out here, off the workgroup's
  // tail, and stored in phase 4 (stores come last).  mask_at < 0: this thread writes no byte.
  int mask_at = -1;
  int8_t mask_byte = 0;
  if (un.quad == 0) {
    const int t = threadIdx.x;
    if (SBS <= kPage) {
      const int lp = SBS == 16 ? 2 : (SBS == 32 ? 1 : 0);  // blocks per chunk = 1 << lp
      const int slot = t >> lp, k = t & ((1 << lp) - 1);
      if (t < (kChunksPerWG << lp) && slot_owned(slot)) {
        const uint64_t bl = ((uint64_t)s_bal[slot][1] << 32) | s_bal[slot][0];
        const int jb = (slot_chunk(slot) << lp) + k;
        const bool kk = SBS == 16   ? ((bl >> (16 * k)) & 0xffffull) != 0
                        : SBS == 32 ? ((bl >> (32 * k)) & 0xffffffffull) != 0
                                    : bl != 0;
        if (jb < p.ntbs) {
          mask_at = jb;
          mask_byte = (jb < NTBS_b && kk) ? 1 : 0;
        }
      }
    } else if (t < kChunksPerWG && (((cw + t) * kPage) & (SBS - 1)) == 0) {
      const int jb = div_pow2((cw + t) * kPage, SBS);
      const bool kk = (s_bal[t][0] | s_bal[t][1]) != 0;
      if (jb < p.ntbs) {
        mask_at = jb;
        mask_byte = (jb < NTBS_b && kk) ? 1 : 0;
      }
    }
  }

  auto exact_chunk = [&](int slot) {
    const int t0 = slot_chunk(slot) * kPage;
    const int nvs = min(Tb - t0, kPage);
    const int pgs_ = __builtin_amdgcn_readfirstlane(s_pgid[slot]);
    const bool keep16 = lane_kept(((uint64_t)s_bal[slot][1] << 32) | s_bal[slot][0]);
    // residual + V loads (the chunk is kept: whole resource).  In the large-batch build they are
    // issued at raised wave priority, so that the arbiter favours them over the scoring of the
    // other workgroups on the CU (config 5's decode 658 -> 599 us; at config 2, where every
    // workgroup reaches its exact pass at about the same time, it cost 0.2 us)
    if constexpr (OCC > 1) __builtin_amdgcn_s_setprio(2);
    // the chunk's residual and V rows (SPEC: loaded by this wave after the operand barrier, used in
    // place, so that the refine waits for the residual alone and P.V for V)
    uint4(&rr)[4][2] = srr;
    uint4(&vv)[8][2] = svv;
    // paged V^T: VH column blocks (of 8) are loaded with the residual; the large-batch build loads
    // the second half after the first half's products, which keeps 32 fewer registers live
    constexpr int VH = (LAYOUT == kPaged && OCC > 1) ? 4 : 8;
    brsrc vs_p;
    if constexpr (!SPEC) {
    if constexpr (RES != kResNone) {
      brsrc rr_s;
      uint32_t ro[4];
      if constexpr (LAYOUT == kPaged) {
        rr_s = make_rsrc(p.kr + ((size_t)pgs_ * p.HKV + hkv) * (kPage * kD), kPage * kD);
      } else {
        rr_s = make_rsrc(p.kr + (((size_t)b * p.T + t0) * p.HKV + hkv) * kD, ((nvs - 1) * p.HKV + 1) * kD);
#pragma unroll
        for (int tau = 0; tau < 4; ++tau) ro[tau] = (4 * mrow + tau) * p.HKV * kD + 32 * kc;
      }
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) {
        if constexpr (LAYOUT == kPaged) {  // token 4 mrow + tau, channels 32 kc + 16 h + (0..15): block (tau, h)
          rr[tau][0] = bload16_nt(rr_s, ((tau * 2 + 0) * 64 + lane) * 16);
          rr[tau][1] = bload16_nt(rr_s, ((tau * 2 + 1) * 64 + lane) * 16);
        } else {
          rr[tau][0] = bload16_nt(rr_s, ro[tau]);
          rr[tau][1] = bload16_nt(rr_s, ro[tau] + 16);
        }
      }
    }
    if constexpr (LAYOUT == kPaged) {
      vs_p = make_rsrc((const uint16_t *)p.v + ((size_t)pgs_ * p.HKV + hkv) * (kD * kPage), kD * kPage * 2);
#pragma unroll
      for (int nu = 0; nu < VH; ++nu)
#pragma unroll
        for (int kap = 0; kap < 2; ++kap) vv[nu][kap] = bload16_nt(vs_p, ((nu * 2 + kap) * 64 + lane) * 16);  // block (nu, kap)
    } else {
      const brsrc vs = make_rsrc((const uint16_t *)p.v + (((size_t)b * p.T + t0) * p.HKV + hkv) * kD,
                                 ((nvs - 1) * p.HKV + 1) * kD * 2);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int idx = r * 64 + lane;
        const int tk = idx >> 4, vc = idx & 15;
        vv[r >> 1][r & 1] = bload16_nt(vs, tk * p.HKV * kD * 2 + 16 * vc);
      }
    }
    }
    if constexpr (OCC > 1) __builtin_amdgcn_s_setprio(0);  // back to normal once the chunk's loads are out
    __builtin_amdgcn_sched_barrier(0);  // every load of the chunk goes out before the refine
    FFA_STAMP(6);
    // refined scores
    float Rj[16];
    if constexpr (kG) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float4 r4 = s_R[slot][q4][4 * kc + ir];
        Rj[4 * q4] = r4.x;
        Rj[4 * q4 + 1] = r4.y;
        Rj[4 * q4 + 2] = r4.z;
        Rj[4 * q4 + 3] = r4.w;
      }
    }
    if constexpr (RES != kResNone) {
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) {
        if constexpr (kG) {
          // refined = coarse + q . r   (exact fp16 residual, every column carries q_i)
          f16x8 qr[4];
#pragma unroll
          for (int mp = 0; mp < 4; ++mp) {
            const uint4 r = s_qr[mp][lane];
            qr[mp] = __builtin_bit_cast(f16x8, u32x4{r.x, r.y, r.z, r.w});
          }
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(fp8x8_to_f16x8<RES>(rr[tau][0].x, rr[tau][0].y), qr[0], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(fp8x8_to_f16x8<RES>(rr[tau][0].z, rr[tau][0].w), qr[1], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(fp8x8_to_f16x8<RES>(rr[tau][1].x, rr[tau][1].y), qr[2], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(fp8x8_to_f16x8<RES>(rr[tau][1].z, rr[tau][1].w), qr[3], acc, 0, 0, 0);
#pragma unroll
          for (int uu = 0; uu < 4; ++uu) Rj[4 * uu + tau] = __builtin_fmaf(acc[uu], 1.0f / 16777216.f, Rj[4 * uu + tau]);
        } else {
          // reference: k_tilde = fp16(k_hat + fp16(res)) (attn_kernel...q2fp8.py:109-115), full re-score
          const uint64_t xx = s_x[slot][tau][lane];
          const uint32_t wlo = (uint32_t)xx, whi = (uint32_t)(xx >> 32);
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
          f16x8 k[4];
          dequant_tile(wlo, whi, k);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(add_f16x8(k[0], fp8x8_to_f16x8_perm<RES>(rr[tau][0].x, rr[tau][0].y)), qa[0], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(add_f16x8(k[1], fp8x8_to_f16x8_perm<RES>(rr[tau][0].z, rr[tau][0].w)), qa[1], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(add_f16x8(k[2], fp8x8_to_f16x8_perm<RES>(rr[tau][1].x, rr[tau][1].y)), qa[2], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(add_f16x8(k[3], fp8x8_to_f16x8_perm<RES>(rr[tau][1].z, rr[tau][1].w)), qa[3], acc, 0, 0, 0);
#pragma unroll
          for (int uu = 0; uu < 4; ++uu) {
            float r = acc[uu];
            r += dpp<kRowRor4>(r);
            r += dpp<kRowRor8>(r);
            Rj[4 * uu + tau] = r;
          }
        }
      }
    } else if constexpr (!kG) {
      // no residual: the coarse scores of the chunk again, from its codes
      const uint32_t zero8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) {
        float r4[4];
        score_tile(s_x[slot][tau][lane], zero8[0], zero8[0], zero8[0], zero8[0], r4);
#pragma unroll
        for (int uu = 0; uu < 4; ++uu) Rj[4 * uu + tau] = r4[uu];
      }
    }
    // softmax partial over the active tokens (valid, in a kept prune block, a row of the group)
    const int nact = (row_ok && keep16) ? min(max(Tb - (t0 + 16 * kc), 0), 16) : 0;
    float P[16], mrow_max, lsum;
    FFA_STAMP(7);
    // (the large-batch build keeps one masked copy of the softmax and of P.V: the fast copies' extra
    // registers would spill at 128)
    chunk_softmax<OCC == 1>(Rj, cs1, nact, P, mrow_max, lsum);
    FFA_STAMP(8);
    // P operand (A) of P.V for K-chunk kap: element e <-> token 16*kc + 8*kap + e
    typename VTr::vec pa2[2];
#pragma unroll
    for (int kap = 0; kap < 2; ++kap) {
      u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = VTr::pack2(P[8 * kap + 2 * e], P[8 * kap + 2 * e + 1]);
      pa2[kap] = __builtin_bit_cast(typename VTr::vec, w);
    }
    const bool partial = nvs < kPage;
    f32x4 oacc[8];
#pragma unroll
    for (int nu = 0; nu < 8; ++nu) oacc[nu] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (LAYOUT == kPaged) {
      // a partial page ANDs each lane's V words with the mask of its valid tokens; two copies of the
      // loop, so that the full pages' loop holds no per-element test (the large-batch build, at 128
      // registers: one copy with a uniform branch per V block)
      auto pv_loop = [&](auto PART) {
        constexpr bool kPart = decltype(PART)::value;
        u32x4 keepw[2];
        if (kPart && (OCC == 1 || partial)) partial_page_masks(kc, nvs, keepw);
#pragma unroll
        for (int nu = 0; nu < 8; ++nu) {
          if (nu == VH) {  // the second half of V^T, into the registers the first half has freed
#pragma unroll
            for (int n2 = VH; n2 < 8; ++n2)
#pragma unroll
              for (int kap = 0; kap < 2; ++kap) vv[n2][kap] = bload16_nt(vs_p, ((n2 * 2 + kap) * 64 + lane) * 16);
          }
#pragma unroll
          for (int kap = 0; kap < 2; ++kap) {
            const uint4 v4 = vv[nu][kap];
            u32x4 w = {v4.x, v4.y, v4.z, v4.w};
            if (kPart && (OCC == 1 || partial)) w &= keepw[kap];
            oacc[nu] = VTr::mfma(pa2[kap], VTr::operand(w), oacc[nu]);
          }
        }
      };
      if (OCC > 1 || partial) [[unlikely]]
        pv_loop(std::true_type());
      else
        pv_loop(std::false_type());
    } else {
      // contiguous layout: stage the V tile through LDS one half at a time ([64 tokens][64
      // columns], a 132-byte row pitch keeps banks apart), then read columns (rows past the
      // sequence end were loaded as zeros).  Half tiles keep two workgroups per CU in LDS.
      uint8_t *st = s_vstage + wv * kPage * kVRowHalf;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int idx = r * 64 + lane;
          const int tk = idx >> 4, vc = idx & 15;
          if ((vc >> 3) == hf) {
            const uint4 v4 = vv[r >> 1][r & 1];
            uint2 *d = (uint2 *)(st + tk * kVRowHalf + 16 * (vc & 7));  // rows are 8-byte aligned
            d[0] = make_uint2(v4.x, v4.y);
            d[1] = make_uint2(v4.z, v4.w);
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int nl = 0; nl < 4; ++nl) {
          const int nu = 4 * hf + nl;
#pragma unroll
          for (int kap = 0; kap < 2; ++kap)
            oacc[nu] = VTr::mfma(pa2[kap], VTr::operand(vt_operand_lds(st, kVRowHalf, nl, kap, kc, n)), oacc[nu]);
        }
        // the other half (and the next kept chunk) reuses the staging buffer
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    }
    FFA_STAMP(9);
    // chunk partial into LDS: lanes 0..15 hold rows 0..3 of columns 16*nu + n
    if (lane < 16) {
#pragma unroll
      for (int uu = 0; uu < 4; ++uu)
#pragma unroll
        for (int nu = 0; nu < 8; ++nu) s_po[slot][uu][16 * nu + n] = oacc[nu][uu];
    }
    if (lane < 4) {  // lane == ir, kc == 0, jg == 0
      s_pm[slot][lane] = row_ok ? mrow_max : -INFINITY;
      s_pl[slot][lane] = row_ok ? lsum : 0.f;
    }
  };
  if constexpr (SPEC) {
    // waves 0 and 1 refine chunk wv (slot 2 wv), whose residual and V^T they hold, if it is kept
    if (wv < 2 && ((km >> (2 * wv)) & 1u)) {
      exact_chunk(2 * wv);
#ifdef FFA_TIMELINE
      ++n_exact_;
#endif
    }
  } else {
    // this wave's kept chunks: the (wv + 4a)-th set bit of km
    int rank = 0;
#pragma unroll 1
    for (int sl = 0; sl < kChunksPerWG; ++sl) {
      if ((km >> sl) & 1u) {
        if ((rank & (kWaves - 1)) == wv) {
          exact_chunk(sl);
#ifdef FFA_TIMELINE
          ++n_exact_;
#endif
        }
        ++rank;
      }
    }
  }

  // ------------------------------------------------ phase 4: workgroup partial (8 chunks) -> global
  FFA_STAMP(10);
  // Global stores come last: on gfx9 stores share the vector memory counter with loads, and a
  // pending store would make every later load wait a full write round trip.
  __syncthreads();
  FFA_STAMP(11);
  if (mask_at >= 0) p.mask[((size_t)b * p.HKV + hkv) * p.ntbs + mask_at] = mask_byte;
  if (p.pass == 0 && p.th_out != nullptr && cg == 0 && threadIdx.x < un.Gu)
    p.th_out[(size_t)b * p.HQ + un.row0 + threadIdx.x] = th;  // (pass 2: written by pass 1)
  {
    const int i = wv;         // query row handled by this wave
    const int c2 = 2 * lane;  // columns c2, c2 + 1
    if (i < un.Gu) {
      // Every slot's m, l and o columns in one batch of LDS reads, then selects: reads issued slot
      // by slot behind branches on l were ~40 dependent LDS round trips (about 1 us) at the end of
      // every workgroup with a kept chunk.  The arithmetic runs only for kept slots (km, uniform:
      // scalar branches), and a workgroup without one skips the merge.  A kept slot's l may still
      // be 0 (no active token of this row); its o is then selected away, not weighted by 0.
      float M = -INFINITY, A = 0.f, ox = 0.f, oy = 0.f;
      if (km != 0u) {
        float pm[kChunksPerWG], pl[kChunksPerWG];
        float2 po[kChunksPerWG];
#pragma unroll
        for (int ps = 0; ps < kChunksPerWG; ++ps) {
          pm[ps] = s_pm[ps][i];
          pl[ps] = s_pl[ps][i];
          po[ps] = *reinterpret_cast<const float2 *>(&s_po[ps][i][c2]);
        }
#pragma unroll
        for (int ps = 0; ps < kChunksPerWG; ++ps)
          if ((km >> ps) & 1u) M = pl[ps] > 0.f ? fmaxf(M, pm[ps]) : M;
#pragma unroll
        for (int ps = 0; ps < kChunksPerWG; ++ps) {
          if (!((km >> ps) & 1u)) continue;
          const bool use = pl[ps] > 0.f;
          const float wgt = exp2_hw(use ? pm[ps] - M : -INFINITY);
          A = use ? __builtin_fmaf(pl[ps], wgt, A) : A;
          ox = use ? __builtin_fmaf(po[ps].x, wgt, ox) : ox;
          oy = use ? __builtin_fmaf(po[ps].y, wgt, oy) : oy;
        }
      }
      const size_t row = (size_t)b * p.HQ + un.row0 + i;
      if (lane == 0) {
        p.m_buf[row * p.nparts + cg] = A > 0.f ? M : -INFINITY;
        p.l_buf[row * p.nparts + cg] = A;
        if (p.v_mean != nullptr) {  // the four waves' pruned-token masses of the row
          float am[kWaves], al[kWaves];  // one batch of LDS reads, as above
#pragma unroll
          for (int w = 0; w < kWaves; ++w) {
            am[w] = s_am[w][i];
            al[w] = s_al[w][i];
          }
          float AM = -INFINITY, AL = 0.f;
#pragma unroll
          for (int w = 0; w < kWaves; ++w) AM = al[w] > 0.f ? fmaxf(AM, am[w]) : AM;
#pragma unroll
          for (int w = 0; w < kWaves; ++w)
            AL = al[w] > 0.f ? __builtin_fmaf(al[w], exp2_hw(am[w] - AM), AL) : AL;
          p.am_buf[row * p.nparts + cg] = AL > 0.f ? AM : -INFINITY;
          p.al_buf[row * p.nparts + cg] = AL;
        }
      }
      if (A > 0.f) *(float2 *)(p.o_buf + (row * p.nparts + cg) * 128 + c2) = make_float2(ox, oy);
    }
  }
#ifdef FFA_TIMELINE
  FFA_STAMP(12);
  if (g_timeline != nullptr && lane == 0) {
    st_[13] = (unsigned long long)n_exact_;
    st_[14] = (unsigned long long)__builtin_popcount(km);
    st_[15] = ((unsigned long long)__builtin_amdgcn_s_getreg((31 << 11) | 20) << 32) |
              (unsigned long long)__builtin_amdgcn_s_getreg((31 << 11) | 4);
    const size_t wid = (((size_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * 4 + wv;
#pragma unroll
    for (int i = 0; i < 16; ++i) g_timeline[wid * 16 + i] = st_[i];
  }
#endif
}

template <int LAYOUT, int SMODE, int RES, int VT, int OCC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OCC))) void q2fp8_decode_kernel(
    const DecodeParams p) {
  q2fp8_decode_body<LAYOUT, SMODE, RES, VT, OCC, false>(p);
}

// the decode of two-chunk spans (small grids of at most one workgroup per CU): paged g32 and the
// contiguous per-channel layouts
template <int LAYOUT, int SMODE, int RES, int VT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1))) void q2fp8_decode_2span_kernel(
    const DecodeParams p) {
  q2fp8_decode_body<LAYOUT, SMODE, RES, VT, 1, true>(p);
}

// --------------------------------------------------------------------------
// Log-sum-exp merge of the workgroup partials (attn_kernel...q2fp8.py:142-171).
// One wave per (sequence, query head, 16-column slab): lane k owns partials k,
// k + 64, ...; m, l and (small batches) the first 64 partials' columns are loaded in one
// batch of unconditional buffer loads (validity = resource size), the maxima and sums go
// through register exchanges, the column sums over lanes through LDS.
// --------------------------------------------------------------------------
template <bool LAZY>
__device__ __forceinline__ void merge_partials(const DecodeParams &p) {
  // grid (KV head, 8 x query row of the group + slab, sequence), the KV head fastest: the paged
  // decoders' partials of a KV head sit in one XCD's L2, and so does every slab workgroup of a row
  // (one read of its m and l from the HBM)
  const int slab = blockIdx.y & 7;  // 16-column slab
  const int b = blockIdx.z;
  const int row = b * p.HQ + (int)blockIdx.x * p.G + (int)(blockIdx.y >> 3);  // b * HQ + hq
  const int lane = threadIdx.x;
  const int span_tok = decode_span(p) * kPage;
  // the launch's slots (from T): the m, l (and eager o) loads are sized by them and issued before
  // the sequence length arrives; slots past the sequence's own partials (stale workspace) are
  // masked to l = 0 once it has
  const int nslots = min(div_pow2(p.T + span_tok - 1, span_tok), p.nparts);
  const int Tb = p.seq_lens ? min(max(p.seq_lens[b], 0), p.T) : p.T;  // lengths beyond T are clamped to T
  const int nparts = min(div_pow2(Tb + span_tok - 1, span_tok), p.nparts);
  const brsrc rm = make_rsrc(p.m_buf + (size_t)row * p.nparts, nslots * 4);
  const brsrc rl = make_rsrc(p.l_buf + (size_t)row * p.nparts, nslots * 4);
  const brsrc ro = make_rsrc(p.o_buf + (size_t)row * p.nparts * 128 + 16 * slab, nslots > 0 ? ((nslots - 1) * 128 + 16) * 4 : 0);
  __shared__ float s_o[64][17];

  // The lane's partials k = lane + 64 i (slots past nparts read as l = 0) in batches of four per
  // lane: one round trip for a batch's m and l, one for the columns of its kept partials (l > 0;
  // a slot whose span kept nothing holds no defined o), with the running maximum rescaled
  // between batches.  Eager (small batches): the first partial's columns go out with its m and l,
  // kept or not.  LAZY (many rows): only kept partials' columns are read, since most slots of
  // long sequences hold pruned spans and reading them all would dominate the traffic.
  constexpr int kNB = 4;  // partials per lane and batch
  const uint32_t o_oob = nslots > 0 ? ((nslots - 1) * 128 + 16) * 4 : 0;  // offset past ro: zeros, no access
  float M = -INFINITY, A = 0.f;
  float acc[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) acc[c] = 0.f;
  if (nslots <= 64) {  // one partial per lane (uniform): a single round trip, no rescaling
    const float m0 = __uint_as_float(bload4(rm, lane * 4));
    const float l0 = __uint_as_float(bload4(rl, lane * 4));
    const bool keep = lane < nparts && l0 > 0.f;
    uint4 o0[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o0[e] = bload16(ro, (!LAZY || keep) ? (lane * 128 + 4 * e) * 4 : o_oob);
    M = wave_max(keep ? m0 : -INFINITY);
    const float wgt = keep ? exp2_hw(m0 - M) : 0.f;
    A = keep ? l0 * wgt : 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[4 * e + 0] = keep ? __uint_as_float(o0[e].x) * wgt : 0.f;
      acc[4 * e + 1] = keep ? __uint_as_float(o0[e].y) * wgt : 0.f;
      acc[4 * e + 2] = keep ? __uint_as_float(o0[e].z) * wgt : 0.f;
      acc[4 * e + 3] = keep ? __uint_as_float(o0[e].w) * wgt : 0.f;
    }
  }
  for (int kb = 0; nslots > 64 && kb < nslots; kb += 64 * kNB) {
    const int nb = min(kNB, (nslots - kb + 63) >> 6);  // partials per lane in this batch (uniform)
    float l[kNB], m[kNB];
    uint4 o[kNB][4];
#pragma unroll
    for (int i = 0; i < kNB; ++i) {
      const int k = kb + 64 * i + lane;
      l[i] = 0.f;
      m[i] = -INFINITY;
      if (i < nb) {
        l[i] = __uint_as_float(bload4(rl, k * 4));
        m[i] = __uint_as_float(bload4(rm, k * 4));
      }
    }
#pragma unroll
    for (int i = 0; i < kNB; ++i)
      if (kb + 64 * i + lane >= nparts) l[i] = 0.f;  // past the sequence's partials
    if (!LAZY && kb == 0) {
#pragma unroll
      for (int e = 0; e < 4; ++e) o[0][e] = bload16(ro, (lane * 128 + 4 * e) * 4);
    }
#pragma unroll
    for (int i = 0; i < kNB; ++i) {
      if ((!LAZY && kb == 0 && i == 0) || i >= nb) continue;
      const uint32_t base = l[i] > 0.f ? (uint32_t)(kb + 64 * i + lane) * 128 * 4 : o_oob;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[i][e] = bload16(ro, l[i] > 0.f ? base + 16 * e : o_oob);
    }
    float Mb = -INFINITY;
#pragma unroll
    for (int i = 0; i < kNB; ++i) Mb = (i < nb && l[i] > 0.f) ? fmaxf(Mb, m[i]) : Mb;
    const float Mn = fmaxf(M, wave_max(Mb));
    if (Mn == -INFINITY) continue;  // nothing kept so far (uniform)
    const float rs = M == -INFINITY ? 0.f : exp2_hw(M - Mn);  // earlier batches to the new maximum
    A *= rs;
#pragma unroll
    for (int c = 0; c < 16; ++c) acc[c] *= rs;
#pragma unroll
    for (int i = 0; i < kNB; ++i) {
      if (i >= nb) continue;  // uniform
      const bool keep = l[i] > 0.f;
      const float wgt = keep ? exp2_hw(m[i] - Mn) : 0.f;
      A = keep ? __builtin_fmaf(l[i], wgt, A) : A;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[4 * e + 0] = keep ? __builtin_fmaf(__uint_as_float(o[i][e].x), wgt, acc[4 * e + 0]) : acc[4 * e + 0];
        acc[4 * e + 1] = keep ? __builtin_fmaf(__uint_as_float(o[i][e].y), wgt, acc[4 * e + 1]) : acc[4 * e + 1];
        acc[4 * e + 2] = keep ? __builtin_fmaf(__uint_as_float(o[i][e].z), wgt, acc[4 * e + 2]) : acc[4 * e + 2];
        acc[4 * e + 3] = keep ? __builtin_fmaf(__uint_as_float(o[i][e].w), wgt, acc[4 * e + 3]) : acc[4 * e + 3];
      }
    }
    M = Mn;
  }
  A = wave_sum(A);
  // mean-V fallback: the pruned tokens' mass of every slot (attn_kernel_v1210_meanv_bsz_q2fp8.py:
  // 172-191, the approximate blocks' running max and sum)
  float AM = -INFINITY, AL = 0.f;
  if (p.v_mean != nullptr) {
    const brsrc ram = make_rsrc(p.am_buf + (size_t)row * p.nparts, nparts * 4);
    const brsrc ral = make_rsrc(p.al_buf + (size_t)row * p.nparts, nparts * 4);
    // the lane's (max, sum) pairs in batches of four per lane, one round trip each, with the
    // running maximum rescaled between batches (the pairs are small: read whether or not l > 0)
    for (int kb = 0; kb < nparts; kb += 64 * kNB) {
      float l[kNB], m[kNB];
#pragma unroll
      for (int i = 0; i < kNB; ++i) {
        const int k = kb + 64 * i + lane;
        l[i] = __uint_as_float(bload4(ral, k * 4));
        m[i] = __uint_as_float(bload4(ram, k * 4));
      }
      float Mb = -INFINITY;
#pragma unroll
      for (int i = 0; i < kNB; ++i) Mb = l[i] > 0.f ? fmaxf(Mb, m[i]) : Mb;
      const float Mn = fmaxf(AM, wave_max(Mb));
      if (Mn == -INFINITY) continue;  // no pruned mass so far (uniform)
      AL *= AM == -INFINITY ? 0.f : exp2_hw(AM - Mn);
#pragma unroll
      for (int i = 0; i < kNB; ++i) AL = l[i] > 0.f ? __builtin_fmaf(l[i], exp2_hw(m[i] - Mn), AL) : AL;
      AM = Mn;
    }
    AL = wave_sum(AL);
  }
  // column sums over the 64 lanes through LDS: lane 16 q + c sums column c of lanes 16 q .. 16 q + 15,
  // then the four quarters are added by register exchanges
#pragma unroll
  for (int e = 0; e < 16; ++e) s_o[lane][e] = acc[e];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  const int c = lane & 15, h = lane >> 4;
  float sum = 0.f;
#pragma unroll 8
  for (int k = 16 * h; k < 16 * h + 16; ++k) sum += s_o[k][c];
  sum += __shfl_xor(sum, 16);
  sum += __shfl_xor(sum, 32);
  if (lane < 16) {
    float val;
    if (p.v_mean == nullptr) {
      val = A == 0.f ? 0.f : sum / A;
    } else {
      // kept blocks' o and mass, plus the pruned mass times v_mean, each rescaled to the common
      // maximum (attn_kernel_v1210_meanv_bsz_q2fp8.py:192-202)
      const float Mx = fmaxf(A > 0.f ? M : -INFINITY, AL > 0.f ? AM : -INFINITY);
      const float re = A > 0.f ? exp2_hw(M - Mx) : 0.f;
      const float ra = AL > 0.f ? exp2_hw(AM - Mx) : 0.f;
      const int hkv = (row - b * p.HQ) / p.G;
      const float vm = load_any(p.v_mean, ((size_t)b * p.HKV + hkv) * 128 + 16 * slab + c, p.vm_dtype);
      const float den = A * re + AL * ra;
      val = den > 0.f ? (sum * re + vm * (AL * ra)) / den : 0.f;
    }
    store_any(p.out, (size_t)row * 128 + 16 * slab + c, p.out_dtype, val);
  }
}

__global__ __launch_bounds__(64) void q2fp8_merge_kernel(const DecodeParams p) { merge_partials<false>(p); }
__global__ __launch_bounds__(64) void q2fp8_merge_sparse_kernel(const DecodeParams p) { merge_partials<true>(p); }

// more than 256 query rows (8 sequences of 32 heads): the lazy merge
hipError_t launch_merge(const DecodeParams &p, hipStream_t st) {
  const dim3 grid((unsigned)p.HKV, (unsigned)(8 * p.G), (unsigned)p.B);
  if (p.B * p.HQ > 256)
    hipLaunchKernelGGL(q2fp8_merge_sparse_kernel, grid, dim3(64), 0, st, p);
  else
    hipLaunchKernelGGL(q2fp8_merge_kernel, grid, dim3(64), 0, st, p);
  return hipGetLastError();
}

}  // namespace ffa

// ============================================================================
// C ABI
// ============================================================================
static thread_local char g_err[512];

static int set_err(int code, const char *msg) {
  snprintf(g_err, sizeof(g_err), "%s", msg);
  return code;
}

extern "C" const char *ffa_last_error(void) { return g_err; }
extern "C" __attribute__((visibility("hidden"))) int ffa_set_error_internal(int code, const char *msg) {
  return set_err(code, msg);
}
extern "C" const char *ffa_version(void) { return "ffa_mi355x 0.1 (gfx950)"; }

// Partial slots per query row of a launch whose workgroups cover `span` chunks: the sub-blocks
// cover ceil(T/BS)*BS tokens.
extern "C" __attribute__((visibility("hidden"))) int ffa_decode_slots(int T, int BS, int span) {
  if (T <= 0 || BS <= 0 || span <= 0) return 0;
  const long tokens = (long)((T + BS - 1) / BS) * BS;
  const long span_tok = (long)span * ffa::kPage;
  return (int)((tokens + span_tok - 1) / span_tok);
}

extern "C" int ffa_q2fp8_decode_nparts(int T, int BS, int SBS) {
  if (T <= 0 || BS <= 0 || SBS <= 0) return 0;
  // short sequences may decode with two-chunk workgroups (small grids): room for their slots
  const long tokens = (long)((T + BS - 1) / BS) * BS;
  return ffa_decode_slots(T, BS, tokens <= ffa::kSmallSpanTokens ? ffa::kMinSpan : ffa::kChunksPerWG);
}

extern "C" int ffa_q2fp8_decode_pieces(int HQ, int HKV, int T, int BS, int SBS) {
  if (HQ <= 0 || HKV <= 0 || HQ % HKV || T <= 0 || BS <= 0 || SBS <= 0 || BS % SBS) return 0;
  const int G = HQ / HKV;
  const int span = ffa::kChunksPerWG * ffa::kPage;
  if (G <= 4 && SBS <= span) return 0;  // one pass
  if (SBS > span) return ffa_decode_slots(T, BS, ffa::kChunksPerWG);  // one piece per 512-token span
  return (int)(((long)T + BS - 1) / BS * (BS / SBS));
}

// Shared validation of the decode shape (both the q2 and the other-format decoders): group size,
// block sizes, two-pass scratch and grid limits; fills the two-pass fields of p.
extern "C" __attribute__((visibility("hidden"))) int ffa_decode_shape_check(int B, int T, int HQ, int HKV, int BS,
                                                                           int SBS, float *piece_max, int npieces,
                                                                           const float *th_in, const float *th_out,
                                                                           ffa::DecodeParams *p) {
  if (B <= 0 || T <= 0 || HQ <= 0 || HKV <= 0) return set_err(FFA_E_INVALID, "bad dims");
  if (HQ % HKV) return set_err(FFA_E_INVALID, "HQ must be a multiple of HKV");
  const int G = HQ / HKV;
  if (G > 16) return set_err(FFA_E_UNSUPPORTED, "GQA group size > 16 is not implemented (the reference's row tile is 16)");
  if (SBS < 16 || (SBS & (SBS - 1)) != 0) return set_err(FFA_E_UNSUPPORTED, "SBS must be a power of two >= 16");
  if (BS <= 0 || BS % SBS) return set_err(FFA_E_UNSUPPORTED, "BS must be a multiple of SBS");
  const int nq = (G + 3) / 4;
  if (B > 65535 || (long)HKV * nq > 65535)
    return set_err(FFA_E_UNSUPPORTED, "B and HKV * ceil(G / 4) are grid dimensions (at most 65535)");
  const int need = ffa_q2fp8_decode_pieces(HQ, HKV, T, BS, SBS);
  if (need > 0) {
    if (!piece_max || npieces < need)
      return set_err(FFA_E_INVALID, "a decode with G > 4 or SBS > 512 runs in two passes and needs piece_max "
                                    "scratch [B, HQ, npieces >= ffa_q2fp8_decode_pieces()]");
    if (!th_in && !th_out)
      return set_err(FFA_E_INVALID, "a two-pass decode (G > 4 or SBS > 512) needs threshold_out (or threshold_in)");
  }
  p->nq = nq;
  p->pass = 0;
  p->pmax = need > 0 ? piece_max : nullptr;
  p->npieces = need > 0 ? npieces : 0;
  return FFA_OK;
}

namespace ffa {
int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 0;
    cache[dev] = cus;
  }
  return cache[dev];
}
}  // namespace ffa

template <int L, int S, int R, int V>
static hipError_t launch_decode(const ffa::DecodeParams &p, dim3 g0, hipStream_t st) {
  // the paged builds place the KV head fastest: grid (unit, span, sequence) (grid_pos)
  const dim3 grid = L == ffa::kPaged ? dim3(g0.y, g0.x, g0.z) : g0;
  // paged g32 with more workgroups than two per CU: the four-per-CU build of the kernel
  if constexpr (L == ffa::kPaged && S == ffa::kG32) {
    const int cus = ffa::device_cus();
    if (cus > 0 && grid.x * grid.y * grid.z > 2u * (unsigned)cus) {
      hipLaunchKernelGGL((ffa::q2fp8_decode_kernel<L, S, R, V, 4>), grid, dim3(256), 0, st, p);
      return hipGetLastError();
    }
  }
  // two-chunk spans, at most one workgroup per CU: the role-split build (paged g32, contiguous)
  if constexpr ((L == ffa::kPaged) == (S == ffa::kG32)) {
    const int cus = ffa::device_cus();
    if (p.span == ffa::kMinSpan && cus > 0 && grid.x * grid.y * grid.z <= (unsigned)cus) {
      hipLaunchKernelGGL((ffa::q2fp8_decode_2span_kernel<L, S, R, V>), grid, dim3(256), 0, st, p);
      return hipGetLastError();
    }
  }
  // fp32 channel scales: held to two workgroups per CU (the fp32 dequantization's temporaries would
  // otherwise take the kernel to 256 registers, one workgroup per CU)
  constexpr int occ = S == ffa::kChannelF32 ? 2 : 1;
  hipLaunchKernelGGL((ffa::q2fp8_decode_kernel<L, S, R, V, occ>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

template <int L, int S>
static hipError_t dispatch_rv(const ffa::DecodeParams &p, int res, int vdt, dim3 grid, hipStream_t st) {
  const int r = res == FFA_DT_FP8_E4M3 ? ffa::kResE4M3 : (res == FFA_DT_FP8_E5M2 ? ffa::kResE5M2 : ffa::kResNone);
  const int v = vdt == FFA_DT_BF16 ? ffa::kVBF16 : ffa::kVF16;
#define FFA_CASE(RR, VV) \
  if (r == RR && v == VV) return launch_decode<L, S, RR, VV>(p, grid, st);
  FFA_CASE(ffa::kResE4M3, ffa::kVBF16)
  FFA_CASE(ffa::kResE4M3, ffa::kVF16)
  FFA_CASE(ffa::kResE5M2, ffa::kVBF16)
  FFA_CASE(ffa::kResE5M2, ffa::kVF16)
  FFA_CASE(ffa::kResNone, ffa::kVBF16)
  FFA_CASE(ffa::kResNone, ffa::kVF16)
#undef FFA_CASE
  return hipErrorInvalidValue;
}

// Validates the arguments and fills the kernel parameters; returns FFA_OK or an error code.
static int decode_params(const ffa_q2fp8_decode_args *a, ffa::DecodeParams &p) {
  if (!a) return set_err(FFA_E_INVALID, "null args");
  p = ffa::DecodeParams{};
  const int rc0 = ffa_decode_shape_check(a->B, a->T, a->HQ, a->HKV, a->BS, a->SBS, a->piece_max, a->npieces,
                                         a->threshold_in, a->threshold_out, &p);
  if (rc0 != FFA_OK) return rc0;
  const int G = a->HQ / a->HKV;
  if (!(a->q_dtype >= FFA_DT_F16 && a->q_dtype <= FFA_DT_F32)) return set_err(FFA_E_INVALID, "q dtype");
  if (!(a->out_dtype >= FFA_DT_F16 && a->out_dtype <= FFA_DT_F32)) return set_err(FFA_E_INVALID, "out dtype");
  if (!(a->v_dtype == FFA_DT_F16 || a->v_dtype == FFA_DT_BF16)) return set_err(FFA_E_INVALID, "v dtype");
  if (!(a->res_dtype == FFA_DT_FP8_E4M3 || a->res_dtype == FFA_DT_FP8_E5M2 || a->res_dtype == FFA_DT_NONE))
    return set_err(FFA_E_INVALID, "residual dtype");
  if (a->res_dtype != FFA_DT_NONE && !a->k_residual) return set_err(FFA_E_INVALID, "residual pointer is null");
  if (a->layout == FFA_LAYOUT_PAGED && !a->block_table) return set_err(FFA_E_INVALID, "paged layout needs a block table");
  if (a->layout == FFA_LAYOUT_PAGED && a->num_pages <= 0)
    return set_err(FFA_E_INVALID, "paged layout needs num_pages > 0 (pages in each pool)");
  if (a->layout == FFA_LAYOUT_PAGED && (long)a->bt_stride * ffa::kPage < a->T)
    return set_err(FFA_E_INVALID, "block table has fewer than ceil(T/64) columns");
  if (a->layout == FFA_LAYOUT_CONTIG && a->scale_mode != FFA_SCALE_CHANNEL)
    return set_err(FFA_E_UNSUPPORTED, "contiguous layout supports per-channel scales only");
  if (a->scale_mode == FFA_SCALE_G32 && a->scale_dtype != FFA_DT_F16)
    return set_err(FFA_E_INVALID, "g32 scales must be fp16");
  const int need = ffa_decode_slots(a->T, a->BS, ffa::kChunksPerWG);
  if (a->nparts < need) return set_err(FFA_E_INVALID, "scratch holds too few partial slots");
  const int ntbs = ((a->T + a->BS - 1) / a->BS) * (a->BS / a->SBS);
  if (a->ntbs < ntbs) return set_err(FFA_E_INVALID, "mask holds too few blocks");
  if (a->v_mean != nullptr) {
    if (!(a->v_mean_dtype >= FFA_DT_F16 && a->v_mean_dtype <= FFA_DT_F32)) return set_err(FFA_E_INVALID, "v_mean dtype");
    if (!a->approx_m || !a->approx_l)
      return set_err(FFA_E_INVALID, "the mean-V fallback needs approx_m / approx_l scratch [B, HQ, nparts]");
  }

  p.q = a->q;
  p.kq = a->k_q;
  p.ks = a->k_scale;
  p.kz = a->k_zero;
  p.kr = a->k_residual;
  p.v = a->v;
  p.bt = a->block_table;
  p.seq_lens = a->seq_lens;
  p.th_in = a->threshold_in;
  p.th_out = a->threshold_out;
  p.out = a->out;
  p.m_buf = a->m_buf;
  p.l_buf = a->l_buf;
  p.o_buf = a->o_buf;
  p.mask = a->mask;
  p.q_dtype = a->q_dtype;
  p.s_dtype = a->scale_dtype;
  p.out_dtype = a->out_dtype;
  p.bt_stride = a->bt_stride;
  p.num_pages = a->layout == FFA_LAYOUT_PAGED ? a->num_pages : 0;
  p.B = a->B;
  p.T = a->T;
  p.HQ = a->HQ;
  p.HKV = a->HKV;
  p.G = G;
  p.scale = a->scale;
  p.BS = a->BS;
  p.SBS = a->SBS;
  p.delta = a->delta;
  p.nparts = a->nparts;
  p.ntbs = a->ntbs;
  p.nwg = need;
  p.span = ffa::kChunksPerWG;
  // small grids (fewer workgroups than CUs): shorter spans, one chunk per wave, while the slots fit
  // the caller's scratch.  One pass with prune blocks of at most one chunk only.
  if (p.pmax == nullptr && a->SBS <= ffa::kPage) {
    const int cus = ffa::device_cus();
    const long units = (long)a->B * a->HKV * p.nq;
    for (int span = ffa::kChunksPerWG / 2; span >= ffa::kMinSpan; span /= 2) {
      if (cus <= 0 || units * p.nwg >= cus) break;
      const int slots = ffa_decode_slots(a->T, a->BS, span);
      if (slots > a->nparts) break;
      p.span = span;
      p.nwg = slots;
    }
  }
  p.v_mean = a->v_mean;
  p.vm_dtype = a->v_mean_dtype;
  p.am_buf = a->v_mean ? a->approx_m : nullptr;
  p.al_buf = a->v_mean ? a->approx_l : nullptr;
  return FFA_OK;
}

static int launch_stage1(const ffa_q2fp8_decode_args *a, const ffa::DecodeParams &p0, hipStream_t st) {
  dim3 grid(p0.nwg, a->HKV * p0.nq, a->B);
  if ((long long)grid.x * grid.y * grid.z > 0x7fffffffLL)  // the kernels number workgroups in 32 bits
    return ffa_set_error_internal(FFA_E_UNSUPPORTED, "decode grid of more than 2^31 - 1 workgroups");
  if (grid.x > 65535)  // the builds that place the KV head fastest launch the spans as grid y
    return ffa_set_error_internal(FFA_E_UNSUPPORTED, "more than 65535 workgroup spans per sequence");
  // one pass (pass 0), or (G > 4, SBS > 512) the maxima pass 1 and then the deciding pass 2
  const bool two = p0.pmax != nullptr;
  for (int pass = two ? 1 : 0; pass <= (two ? 2 : 0); ++pass) {
    ffa::DecodeParams p = p0;
    p.pass = pass;
    hipError_t e;
    // channel scales: the packed fp16 dequantization for fp16 scale / zero, and for bf16 / fp32 ones
    // that the caller declares exactly representable in fp16 (scale_exact_f16); otherwise fp32
    // arithmetic, as the reference dequantizes (fp16(fp32(fp32(c s) + z)))
    const bool f16_scales = a->scale_dtype == FFA_DT_F16 || a->scale_exact_f16 != 0;
    if (a->layout == FFA_LAYOUT_PAGED) {
      if (a->scale_mode == FFA_SCALE_G32)
        e = dispatch_rv<ffa::kPaged, ffa::kG32>(p, a->res_dtype, a->v_dtype, grid, st);
      else if (f16_scales)
        e = dispatch_rv<ffa::kPaged, ffa::kChannel>(p, a->res_dtype, a->v_dtype, grid, st);
      else
        e = dispatch_rv<ffa::kPaged, ffa::kChannelF32>(p, a->res_dtype, a->v_dtype, grid, st);
    } else if (f16_scales) {
      e = dispatch_rv<ffa::kContig, ffa::kChannel>(p, a->res_dtype, a->v_dtype, grid, st);
    } else {
      e = dispatch_rv<ffa::kContig, ffa::kChannelF32>(p, a->res_dtype, a->v_dtype, grid, st);
    }
    if (e != hipSuccess) return set_err(FFA_E_LAUNCH, hipGetErrorString(e));
  }
  return FFA_OK;
}

static int launch_stage2(const ffa_q2fp8_decode_args *a, const ffa::DecodeParams &p, hipStream_t st) {
  (void)a;
  const hipError_t e = ffa::launch_merge(p, st);
  if (e != hipSuccess) return set_err(FFA_E_LAUNCH, hipGetErrorString(e));
  return FFA_OK;
}

extern "C" int ffa_q2fp8_decode_stage1(const ffa_q2fp8_decode_args *a, void *stream) {
  ffa::DecodeParams p;
  const int rc = decode_params(a, p);
  return rc != FFA_OK ? rc : launch_stage1(a, p, (hipStream_t)stream);
}

extern "C" int ffa_q2fp8_decode_stage2(const ffa_q2fp8_decode_args *a, void *stream) {
  ffa::DecodeParams p;
  const int rc = decode_params(a, p);
  return rc != FFA_OK ? rc : launch_stage2(a, p, (hipStream_t)stream);
}

extern "C" int ffa_q2fp8_decode(const ffa_q2fp8_decode_args *a, void *stream) {
  ffa::DecodeParams p;
  int rc = decode_params(a, p);
  if (rc != FFA_OK) return rc;
  rc = launch_stage1(a, p, (hipStream_t)stream);
  return rc != FFA_OK ? rc : launch_stage2(a, p, (hipStream_t)stream);
}

// ============================================================================
// Decode without allocations: the scratch lives in a static device array
// ============================================================================
// For callers that cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc).  The per-call scratch of ffa_q2fp8_decode -- partials,
// two-pass block maxima, and the survivor mask / thresholds when the caller passes none -- is
// carved out of `scratch`, one copy per GPU for the life of the process.  Its device address is
// taken once per device with hipGetSymbolAddress and only that address reaches the kernels (the
// array's name in host code is a host-side stand-in).  Nothing in it has to start at zero: every
// slot a kernel reads is written earlier in the same call.  Calls that overlap on one GPU (two
// streams, two host threads) share the array and race.
namespace {
constexpr size_t kStaticScratchBytes = FFA_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch_ptr[kMaxDevices] = {};

int static_scratch_of_current_device(uint8_t **out, hipStream_t st) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_err(FFA_E_LAUNCH, "no current HIP device for the static scratch");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    // the address is resolved on the first call on a device, which must not be under stream capture
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
      return set_err(FFA_E_INVALID, "ffa_q2fp8_decode_noalloc: the first call on a device must run outside stream "
                                    "capture (it resolves the static scratch's device address)");
    if (ffa::device_cus() <= 0) return set_err(FFA_E_LAUNCH, "hipDeviceGetAttribute(multiprocessor count) failed");
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) return set_err(FFA_E_LAUNCH, "hipGetSymbolAddress(scratch) failed");
    g_scratch_ptr[dev] = static_cast<uint8_t *>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return FFA_OK;
}
}  // namespace

extern "C" int ffa_q2fp8_decode_noalloc(const ffa_q2fp8_decode_args *a, void *stream) {
  if (!a) return set_err(FFA_E_INVALID, "null args");
  if (a->B <= 0 || a->T <= 0 || a->HQ <= 0 || a->HKV <= 0 || a->BS <= 0 || a->SBS <= 0)
    return set_err(FFA_E_INVALID, "bad dims");
  const size_t B = (size_t)a->B, HQ = (size_t)a->HQ, HKV = (size_t)a->HKV;
  const size_t nparts = (size_t)ffa_q2fp8_decode_nparts(a->T, a->BS, a->SBS);
  const size_t ntbs = (size_t)((a->T + a->BS - 1) / a->BS) * (size_t)(a->BS / a->SBS);
  const size_t npieces = (size_t)ffa_q2fp8_decode_pieces(a->HQ, a->HKV, a->T, a->BS, a->SBS);
  // the size in floating point first, so that no product of the dimensions can wrap
  const double rows = (double)B * (double)HQ;
  const double need = rows * (double)nparts * (a->v_mean ? 132.0 : 130.0) * 4.0 +
                      (double)B * (double)HKV * (double)ntbs + rows * 4.0 + rows * (double)npieces * 4.0;
  if (need > (double)kStaticScratchBytes) {
    char msg[200];
    snprintf(msg, sizeof(msg), "ffa_q2fp8_decode_noalloc: this shape needs %.0f bytes of scratch, the static array holds %zu",
             need, kStaticScratchBytes);
    return set_err(FFA_E_UNSUPPORTED, msg);
  }
  size_t used = 0;
  auto take = [&](size_t bytes) {  // 256-byte aligned regions
    const size_t at = used;
    used += (bytes + 255) & ~size_t(255);
    return at;
  };
  const size_t m_at = take(B * HQ * nparts * 4), l_at = take(B * HQ * nparts * 4);
  const size_t o_at = take(B * HQ * nparts * 128 * 4);
  const size_t mask_at = a->mask ? 0 : take(B * HKV * ntbs);
  const size_t th_at = a->threshold_out ? 0 : take(B * HQ * 4);
  const size_t pm_at = npieces ? take(B * HQ * npieces * 4) : 0;
  const size_t am_at = a->v_mean ? take(B * HQ * nparts * 4) : 0;
  const size_t al_at = a->v_mean ? take(B * HQ * nparts * 4) : 0;
  if (used > kStaticScratchBytes) {
    char msg[200];
    snprintf(msg, sizeof(msg), "ffa_q2fp8_decode_noalloc: this shape needs %zu bytes of scratch, the static array holds %zu",
             used, kStaticScratchBytes);
    return set_err(FFA_E_UNSUPPORTED, msg);
  }
  uint8_t *base = nullptr;
  const int rc = static_scratch_of_current_device(&base, (hipStream_t)stream);
  if (rc != FFA_OK) return rc;
  ffa_q2fp8_decode_args s = *a;
  s.m_buf = reinterpret_cast<float *>(base + m_at);
  s.l_buf = reinterpret_cast<float *>(base + l_at);
  s.o_buf = reinterpret_cast<float *>(base + o_at);
  s.nparts = (int)nparts;
  if (!a->mask) {
    s.mask = reinterpret_cast<int8_t *>(base + mask_at);
    s.ntbs = (int)ntbs;
  }
  if (!a->threshold_out) s.threshold_out = reinterpret_cast<float *>(base + th_at);
  s.piece_max = npieces ? reinterpret_cast<float *>(base + pm_at) : nullptr;
  s.npieces = (int)npieces;
  s.approx_m = a->v_mean ? reinterpret_cast<float *>(base + am_at) : nullptr;
  s.approx_l = a->v_mean ? reinterpret_cast<float *>(base + al_at) : nullptr;
  return ffa_q2fp8_decode(&s, stream);
}

#ifdef FFA_TIMELINE
// Timeline build only: the buffer (16 words per wave of a stage-1 grid) the q2 decode writes to.
extern "C" int ffa_debug_set_timeline(void *ptr) {
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_timeline), &ptr, sizeof(ptr));
}
#endif
