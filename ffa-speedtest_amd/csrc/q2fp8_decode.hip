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
//   * partials (m, l, o) per 64-token chunk, merged by a second kernel that
//     compacts the kept chunks with a wave ballot.
#include "ffa_common.h"
#include "ffa_mi355x.h"

#include <stdio.h>

namespace ffa {

constexpr int kD = 128;
constexpr int kPage = 64;
constexpr int kWaves = 4;
constexpr int kVRow = 260;  // LDS row pitch (bytes) of the staged V tile: 256 + 4 keeps banks apart

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
  int B, T, HQ, HKV, G;
  float scale;
  int BS, SBS;
  float delta;
  int nch, ntbs;
};

enum { kContig = 0, kPaged = 1 };
enum { kChannel = 0, kG32 = 1 };
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

template <int VT>
struct VTraits;
template <>
struct VTraits<kVBF16> {
  typedef bf16x8 vec;
  __device__ static __forceinline__ f32x4 mfma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack2(float x, float y) {
    return f32_to_bf16_bits(x) | (f32_to_bf16_bits(y) << 16);
  }
};
template <>
struct VTraits<kVF16> {
  typedef f16x8 vec;
  __device__ static __forceinline__ f32x4 mfma(vec a, vec b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack2(float x, float y) {
    return f32_to_f16_bits(x) | (f32_to_f16_bits(y) << 16);
  }
};

template <int LAYOUT, int SMODE, int RES, int VT>
__global__ __launch_bounds__(256) void q2fp8_decode_kernel(const DecodeParams p) {
  typedef VTraits<VT> VTr;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int bh = blockIdx.y;
  const int b = bh / p.HKV;
  const int hkv = bh - b * p.HKV;
  const int G = p.G;
  const int chunk = blockIdx.x * kWaves + wv;
  const int t0 = chunk * kPage;
  const int Tb = p.seq_lens ? p.seq_lens[b] : p.T;
  const int NTB = (Tb + p.BS - 1) / p.BS;
  const int NTBS_b = NTB * (p.BS / p.SBS);

  const int mrow = lane & 15;  // MFMA row / column index inside a 16-lane group
  const int kc = lane >> 4;    // k-chunk of the MFMA operands == channel group
  const int n = mrow;          // output column = (j, i)
  const int jg = n >> 2;       // channel group of the output column
  const int ir = n & 3;        // query row of the output column
  const bool row_ok = ir < G;

  __shared__ float s_probe[2][4];
  __shared__ float s_pmax[kWaves][4];
  __shared__ uint8_t s_vstage[LAYOUT == kContig ? kWaves * kPage * kVRow : 4];

  // ---------------------------------------------------------------- q setup
  // Lane (kc, n=(j,i)) holds q_i on channels 32*kc .. 32*kc+31.
  const int hq = hkv * G + ir;
  float qv[32];
  float sc[32];  // per-channel scale (channel mode) for the folded operand
  float zsum = 0.f;
  {
    const size_t qbase = ((size_t)b * p.HQ + (row_ok ? hq : hkv * G)) * kD + 32 * kc;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      float x = load_any(p.q, qbase + e, p.q_dtype);
      qv[e] = row_ok ? (float)(_Float16)x : 0.f;  // q16 (attn_kernel...q2fp8.py:47)
    }
    if constexpr (SMODE == kChannel) {
      const size_t sbase = ((size_t)b * p.HKV + hkv) * kD + 32 * kc;
#pragma unroll
      for (int e = 0; e < 32; ++e) {
        sc[e] = load_any(p.ks, sbase + e, p.s_dtype);
        zsum += qv[e] * load_any(p.kz, sbase + e, p.s_dtype);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 32; ++e) {
        sc[e] = 1.f;
        zsum += qv[e];
      }
    }
  }
  // Coarse operand for MFMA m' = 2h + s: element 2q+half <-> channel 32kc + 16h + 4s + q + 8half,
  // divided by 4^q; nonzero only when kc == j (the column's group).
  f16x8 qa[4];
#pragma unroll
  for (int mp = 0; mp < 4; ++mp) {
    const int h = mp >> 1, s = mp & 1;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int ch = 16 * h + 4 * s + qq + 8 * half;
        const float inv = qq == 0 ? 1.f : (qq == 1 ? 0.25f : (qq == 2 ? 0.0625f : 0.015625f));
        float val = (kc == jg) ? (qv[ch] * sc[ch]) * inv : 0.f;
        qa[mp][2 * qq + half] = (_Float16)val;
      }
    }
  }
  // Refine operand for MFMA m': element e <-> channel 32kc + 8m' + e (all groups).
  f16x8 qr[4];
#pragma unroll
  for (int mp = 0; mp < 4; ++mp)
#pragma unroll
    for (int e = 0; e < 8; ++e) qr[mp][e] = (_Float16)qv[8 * mp + e];
  // Per-(j,i) constant of the epilogue: sum_{d in group j} q16 (g32) or
  // sum_{d in chunk j} q16 * z (channel); computed by the lanes with kc == j.
  const float zq = __shfl(zsum, (jg << 4) | n);

  const float qk_scale = p.scale;

  // ------------------------------------------------------- coarse score tile
  // Computes raw scores (before *scale*log2e) of 16 tokens for the lane's column.
  //   tok_row(mrow) : token handled by MFMA row `mrow`
  //   outputs racc[u] for rows 4*kc + u
  auto score_tile = [&](const uint64_t x, const float *s4, const float *z4, float *racc) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const uint32_t wlo = (uint32_t)x, whi = (uint32_t)(x >> 32);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes_to_f16x8(wlo, 0), qa[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes_to_f16x8(wlo, 1), qa[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes_to_f16x8(whi, 0), qa[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes_to_f16x8(whi, 1), qa[3], acc, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float r;
      if constexpr (SMODE == kG32) {
        r = (s4[u] * 16777216.f) * acc[u] + z4[u] * zq;
      } else {
        r = 16777216.f * acc[u] + zq;
      }
      r += dpp<kRowRor4>(r);
      r += dpp<kRowRor8>(r);
      racc[u] = r;
    }
  };

  auto token_codes = [&](int tok, int pg) -> uint64_t {
    // 32 codes of channel group kc for token `tok` (sequence position)
    if constexpr (LAYOUT == kPaged) {
      const size_t off = (((size_t)pg * p.HKV + hkv) * 4 + kc) * (kPage * 8) + (size_t)(tok & (kPage - 1)) * 8;
      return *(const uint64_t *)(p.kq + off);
    } else {
      const int t = min(tok, Tb - 1);
      const size_t off = (((size_t)b * p.T + t) * p.HKV + hkv) * 32 + 8 * kc;
      return *(const uint64_t *)(p.kq + off);
    }
  };

  // ------------------------------------------------------------ probe windows
  if (p.th_in == nullptr && wv < 2) {
    const int a = wv == 0 ? 0 : (NTB - 1) * 16;  // attn_kernel...q2fp8.py:58-73
    const int pg = (LAYOUT == kPaged) ? p.bt[(size_t)b * p.bt_stride + (a >> 6)] : 0;
    const uint64_t x = token_codes(a + mrow, pg);
    float s4[4] = {1.f, 1.f, 1.f, 1.f}, z4[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (SMODE == kG32) {
      const size_t sb = (((size_t)pg * p.HKV + hkv) * 4 + jg) * kPage + ((a & (kPage - 1)) + 4 * kc);
      const uint2 sv = *(const uint2 *)((const uint16_t *)p.ks + sb);
      const uint2 zv = *(const uint2 *)((const uint16_t *)p.kz + sb);
      s4[0] = f16_bits_to_f32(sv.x & 0xffff);
      s4[1] = f16_bits_to_f32(sv.x >> 16);
      s4[2] = f16_bits_to_f32(sv.y & 0xffff);
      s4[3] = f16_bits_to_f32(sv.y >> 16);
      z4[0] = f16_bits_to_f32(zv.x & 0xffff);
      z4[1] = f16_bits_to_f32(zv.x >> 16);
      z4[2] = f16_bits_to_f32(zv.y & 0xffff);
      z4[3] = f16_bits_to_f32(zv.y >> 16);
    }
    float r[4];
    score_tile(x, s4, z4, r);
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = a + 4 * kc + u;
      const float sv = (r[u] * qk_scale) * kLog2e;
      mx = fmaxf(mx, t < Tb ? sv : -INFINITY);
    }
    mx = xor_max(mx, 16);
    mx = xor_max(mx, 32);
    if (lane < 4) s_probe[wv][lane] = mx;  // lane == ir here (kc == 0, jg == 0)
  }

  // ---------------------------------------------------------- chunk scores
  const bool active = t0 < Tb;
  float R[16];  // raw coarse scores of tokens t0 + 16*kc + k, column (j,i) (identical across j)
  int pg = 0;
  if (active) {
    if constexpr (LAYOUT == kPaged) pg = p.bt[(size_t)b * p.bt_stride + chunk];
    // token of MFMA row m in tile tau is 4m + tau (within the chunk)
    uint64_t x[4];
    if constexpr (LAYOUT == kPaged) {
      const size_t off = (((size_t)pg * p.HKV + hkv) * 4 + kc) * (kPage * 8) + (size_t)(4 * mrow) * 8;
      const uint4 v0 = *(const uint4 *)(p.kq + off);
      const uint4 v1 = *(const uint4 *)(p.kq + off + 16);
      x[0] = ((uint64_t)v0.y << 32) | v0.x;
      x[1] = ((uint64_t)v0.w << 32) | v0.z;
      x[2] = ((uint64_t)v1.y << 32) | v1.x;
      x[3] = ((uint64_t)v1.w << 32) | v1.z;
    } else {
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) x[tau] = token_codes(t0 + 4 * mrow + tau, 0);
    }
    float s16[16], z16[16];
    if constexpr (SMODE == kG32) {
      const size_t sb = (((size_t)pg * p.HKV + hkv) * 4 + jg) * kPage + 16 * kc;
      const uint4 *sp = (const uint4 *)((const uint16_t *)p.ks + sb);
      const uint4 *zp = (const uint4 *)((const uint16_t *)p.kz + sb);
      uint32_t sw[8], zw[8];
      const uint4 s0 = sp[0], s1 = sp[1], z0 = zp[0], z1 = zp[1];
      sw[0] = s0.x; sw[1] = s0.y; sw[2] = s0.z; sw[3] = s0.w;
      sw[4] = s1.x; sw[5] = s1.y; sw[6] = s1.z; sw[7] = s1.w;
      zw[0] = z0.x; zw[1] = z0.y; zw[2] = z0.z; zw[3] = z0.w;
      zw[4] = z1.x; zw[5] = z1.y; zw[6] = z1.z; zw[7] = z1.w;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        s16[k] = f16_bits_to_f32((sw[k >> 1] >> (16 * (k & 1))) & 0xffff);
        z16[k] = f16_bits_to_f32((zw[k >> 1] >> (16 * (k & 1))) & 0xffff);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        s16[k] = 1.f;
        z16[k] = 0.f;
      }
    }
#pragma unroll
    for (int tau = 0; tau < 4; ++tau) {
      float s4[4], z4[4], r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        s4[u] = s16[4 * u + tau];
        z4[u] = z16[4 * u + tau];
      }
      score_tile(x[tau], s4, z4, r);
#pragma unroll
      for (int u = 0; u < 4; ++u) R[4 * u + tau] = r[u];
    }
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) R[k] = 0.f;
  }

  // coarse log2-scaled scores, masked
  float S[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int t = t0 + 16 * kc + k;
    const float sv = (R[k] * qk_scale) * kLog2e;
    S[k] = (active && t < Tb && row_ok) ? sv : -INFINITY;
  }

  __syncthreads();
  float th;
  if (p.th_in != nullptr) {
    th = row_ok ? p.th_in[(size_t)b * p.HQ + hq] : INFINITY;
  } else {
    th = row_ok ? fmaxf(s_probe[0][ir], s_probe[1][ir]) - p.delta : INFINITY;
  }
  if (p.th_out != nullptr && blockIdx.x == 0 && threadIdx.x < G) {
    p.th_out[(size_t)b * p.HQ + hkv * G + threadIdx.x] = th;  // lane == ir for threadIdx < 4
  }

  // ------------------------------------------------------------------ prune
  // block max over the lane's 16 tokens, then over lane groups per SBS
  float mx = S[0];
#pragma unroll
  for (int k = 1; k < 16; ++k) mx = fmaxf(mx, S[k]);
  const int SBS = p.SBS;
  if (SBS >= 32) mx = xor_max(mx, 16);
  if (SBS >= 64) mx = xor_max(mx, 32);
  if (SBS > kPage) {
    if (lane < 4) s_pmax[wv][lane] = mx;
  }
  __syncthreads();
  if (SBS > kPage) {
    const int wpb = SBS / kPage;  // waves per block
    const int w0 = (wv / wpb) * wpb;
    float m2 = -INFINITY;
    for (int w = w0; w < w0 + wpb; ++w) m2 = fmaxf(m2, s_pmax[w][ir]);
    mx = m2;
  }
  // "prune iff all rows below" (strict <), rows >= G do not vote
  const bool notbelow = row_ok && !(mx < th);
  const uint64_t bal = __ballot(notbelow);
  // keep flag of the sub-block holding the lane's tokens
  uint32_t keep16;
  if (SBS == 16) {
    keep16 = ((bal >> (16 * kc)) & 0xffffull) != 0;
  } else if (SBS == 32) {
    keep16 = ((bal >> (32 * (kc >> 1))) & 0xffffffffull) != 0;
  } else {
    keep16 = bal != 0;
  }
  // mask entries of the sub-blocks starting in this chunk
  {
    int8_t *mrow_ptr = p.mask + ((size_t)b * p.HKV + hkv) * p.ntbs;
    if (SBS <= kPage) {
      const int per = kPage / SBS;
      const int jb = t0 / SBS;
      if (lane < per && jb + lane < p.ntbs) {
        const int sub = lane;  // sub-block index inside the chunk
        const int kcs = sub * (SBS / 16);
        const bool kk = SBS == 16   ? ((bal >> (16 * kcs)) & 0xffffull) != 0
                        : SBS == 32 ? ((bal >> (16 * kcs)) & 0xffffffffull) != 0
                                    : bal != 0;
        mrow_ptr[jb + lane] = (jb + lane < NTBS_b && kk) ? 1 : 0;
      }
    } else if ((t0 % SBS) == 0 && lane == 0) {
      const int jb = t0 / SBS;
      if (jb < p.ntbs) mrow_ptr[jb] = (jb < NTBS_b && bal != 0) ? 1 : 0;
    }
  }
  const bool any_keep = __ballot(keep16 != 0) != 0;

  const size_t row_base = (size_t)b * p.HQ + hkv * G;  // first query row of the group
  if (!any_keep || !active) {
    if (kc == 0 && jg == 0 && row_ok && chunk < p.nch) {
      p.m_buf[(row_base + ir) * p.nch + chunk] = -INFINITY;
      p.l_buf[(row_base + ir) * p.nch + chunk] = 0.f;
    }
    return;
  }

  // ------------------------------------------------------------- exact pass
  // refined raw score = coarse raw + q . r   (r = fp8 residual, exact in fp16)
  if constexpr (RES != kResNone) {
    uint4 rr[4][2];
#pragma unroll
    for (int tau = 0; tau < 4; ++tau) {
      const int tk = 4 * mrow + tau;  // token inside the chunk
      size_t off;
      if constexpr (LAYOUT == kPaged) {
        off = (((size_t)pg * p.HKV + hkv) * kPage + tk) * kD + 32 * kc;
      } else {
        const int t = min(t0 + tk, Tb - 1);
        off = (((size_t)b * p.T + t) * p.HKV + hkv) * kD + 32 * kc;
      }
      rr[tau][0] = *(const uint4 *)(p.kr + off);
      rr[tau][1] = *(const uint4 *)(p.kr + off + 16);
    }
#pragma unroll
    for (int tau = 0; tau < 4; ++tau) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(fp8x8_to_f16x8<RES>(rr[tau][0].x, rr[tau][0].y), qr[0], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(fp8x8_to_f16x8<RES>(rr[tau][0].z, rr[tau][0].w), qr[1], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(fp8x8_to_f16x8<RES>(rr[tau][1].x, rr[tau][1].y), qr[2], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(fp8x8_to_f16x8<RES>(rr[tau][1].z, rr[tau][1].w), qr[3], acc, 0, 0, 0);
#pragma unroll
      for (int u = 0; u < 4; ++u) R[4 * u + tau] += acc[u];
    }
  }
  // active tokens: valid and inside a kept sub-block
  float P[16];
  float mrow_max = -INFINITY;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int t = t0 + 16 * kc + k;
    const float sv = (R[k] * qk_scale) * kLog2e;
    const bool act = row_ok && t < Tb && keep16;
    P[k] = act ? sv : -INFINITY;
    mrow_max = fmaxf(mrow_max, P[k]);
  }
  mrow_max = xor_max(mrow_max, 16);
  mrow_max = xor_max(mrow_max, 32);
  float lsum = 0.f;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const float e = (P[k] == -INFINITY) ? 0.f : exp2f(P[k] - mrow_max);
    P[k] = e;
    lsum += e;
  }
  lsum = xor_sum(lsum, 16);
  lsum = xor_sum(lsum, 32);

  // P operand (A) of the P.V MFMA for K-chunk kap: element e <-> token 16*kc + 8*kap + e
  typename VTr::vec pa[2];
#pragma unroll
  for (int kap = 0; kap < 2; ++kap) {
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = VTr::pack2(P[8 * kap + 2 * e], P[8 * kap + 2 * e + 1]);
    pa[kap] = __builtin_bit_cast(typename VTr::vec, w);
  }

  const bool partial = (t0 + kPage) > Tb;
  f32x4 oacc[8];
#pragma unroll
  for (int nu = 0; nu < 8; ++nu) oacc[nu] = f32x4{0.f, 0.f, 0.f, 0.f};

  if constexpr (LAYOUT == kPaged) {
    const uint16_t *vp = (const uint16_t *)p.v + (((size_t)pg * p.HKV + hkv) * 128) * kPage;
#pragma unroll
    for (int nu = 0; nu < 8; ++nu) {
#pragma unroll
      for (int kap = 0; kap < 2; ++kap) {
        const int vcol = 16 * nu + n;
        const int tk = 16 * kc + 8 * kap;
        uint4 vv = *(const uint4 *)(vp + (size_t)vcol * kPage + tk);
        if (partial) {
          // zero V of tokens past the sequence end (their page slots are not data)
          uint32_t w4[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int ta = t0 + tk + 2 * e;
            if (ta >= Tb) w4[e] &= 0xffff0000u;
            if (ta + 1 >= Tb) w4[e] &= 0x0000ffffu;
          }
          vv = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
        u32x4 w = {vv.x, vv.y, vv.z, vv.w};
        oacc[nu] = VTr::mfma(pa[kap], __builtin_bit_cast(typename VTr::vec, w), oacc[nu]);
      }
    }
  } else {
    // stage the chunk's V tile [64 tokens][128] into LDS (row pitch kVRow), then read columns
    uint8_t *st = s_vstage + wv * kPage * kVRow;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int idx = r * 64 + lane;
      const int tk = idx >> 4, vc = idx & 15;
      const int t = min(t0 + tk, Tb - 1);
      const uint4 vv = *(const uint4 *)((const uint16_t *)p.v + (((size_t)b * p.T + t) * p.HKV + hkv) * 128 + 8 * vc);
      uint32_t *d = (uint32_t *)(st + tk * kVRow + 16 * vc);
      const bool ok = (t0 + tk) < Tb;
      d[0] = ok ? vv.x : 0u;
      d[1] = ok ? vv.y : 0u;
      d[2] = ok ? vv.z : 0u;
      d[3] = ok ? vv.w : 0u;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int nu = 0; nu < 8; ++nu) {
#pragma unroll
      for (int kap = 0; kap < 2; ++kap) {
        const int vcol = 16 * nu + n;
        const int tk = 16 * kc + 8 * kap;
        u32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = *(const uint16_t *)(st + (tk + 2 * e) * kVRow + 2 * vcol);
          const uint32_t hi = *(const uint16_t *)(st + (tk + 2 * e + 1) * kVRow + 2 * vcol);
          w[e] = lo | (hi << 16);
        }
        oacc[nu] = VTr::mfma(pa[kap], __builtin_bit_cast(typename VTr::vec, w), oacc[nu]);
      }
    }
  }

  // write the chunk partial: lanes 0..15 hold rows 0..3 of columns 16*nu + n
  if (chunk < p.nch) {
    if (lane < 16) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (u < G) {
          float *op = p.o_buf + ((row_base + u) * p.nch + chunk) * 128 + n;
#pragma unroll
          for (int nu = 0; nu < 8; ++nu) op[16 * nu] = oacc[nu][u];
        }
      }
    }
    if (kc == 0 && jg == 0 && row_ok) {
      p.m_buf[(row_base + ir) * p.nch + chunk] = mrow_max;
      p.l_buf[(row_base + ir) * p.nch + chunk] = lsum;
    }
  }
}

// --------------------------------------------------------------------------
// Log-sum-exp merge of the chunk partials (attn_kernel...q2fp8.py:142-171).
// One workgroup (128 threads = 2 waves) per (sequence, query head).  Kept
// chunks (l > 0) are compacted with a wave ballot into LDS, in chunk order.
// --------------------------------------------------------------------------
constexpr int kMergeSeg = 1024;

__global__ __launch_bounds__(128) void q2fp8_merge_kernel(const DecodeParams p) {
  const int row = blockIdx.x;  // b * HQ + hq
  const int b = row / p.HQ;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6;
  const int Tb = p.seq_lens ? p.seq_lens[b] : p.T;
  const int nchb = min((Tb + kPage - 1) / kPage, p.nch);
  const float *mrow = p.m_buf + (size_t)row * p.nch;
  const float *lrow = p.l_buf + (size_t)row * p.nch;
  const float *orow = p.o_buf + (size_t)row * p.nch * 128;

  __shared__ int s_list[kMergeSeg];
  __shared__ float s_w[kMergeSeg];
  __shared__ float s_red[2];
  __shared__ int s_cnt[2];

  float Mrun = -INFINITY, Arun = 0.f, Orun = 0.f;
  for (int seg = 0; seg < nchb; seg += kMergeSeg) {
    const int segn = min(kMergeSeg, nchb - seg);
    // pass 1: segment max over kept chunks
    float mloc = -INFINITY;
    for (int c = tid; c < segn; c += 128) {
      const float l = lrow[seg + c];
      if (l > 0.f) mloc = fmaxf(mloc, mrow[seg + c]);
    }
    for (int o = 32; o >= 1; o >>= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, o));
    if (lane == 0) s_red[wv] = mloc;
    __syncthreads();
    const float Mseg = fmaxf(s_red[0], s_red[1]);
    // pass 2: compact kept chunks, in order, with their weights 2^(m - Mseg)
    int base = 0;
    for (int c0 = 0; c0 < segn; c0 += 128) {
      const int c = c0 + tid;
      bool keep = false;
      float wgt = 0.f;
      if (c < segn) {
        const float l = lrow[seg + c];
        keep = l > 0.f;
        if (keep) wgt = exp2f(mrow[seg + c] - Mseg);
      }
      const uint64_t bal = __ballot(keep);
      const int before = __popcll(bal & ((1ull << lane) - 1ull));
      if (lane == 0) s_cnt[wv] = __popcll(bal);
      __syncthreads();
      const int off = base + (wv ? s_cnt[0] : 0) + before;
      if (keep) {
        s_list[off] = seg + c;
        s_w[off] = wgt;
      }
      base += s_cnt[0] + s_cnt[1];
      __syncthreads();
    }
    // pass 3: accumulate (every thread owns one output column)
    float A = 0.f, O = 0.f;
    for (int k = 0; k < base; ++k) {
      const int c = s_list[k];
      const float wgt = s_w[k];
      A += lrow[c] * wgt;
      O += orow[(size_t)c * 128 + tid] * wgt;
    }
    if (base > 0) {
      const float Mn = fmaxf(Mrun, Mseg);
      const float a = (Mrun == -INFINITY) ? 0.f : exp2f(Mrun - Mn);
      const float bb = exp2f(Mseg - Mn);
      Arun = Arun * a + A * bb;
      Orun = Orun * a + O * bb;
      Mrun = Mn;
    }
    __syncthreads();
  }
  const float res = (Arun == 0.f) ? 0.f : Orun / Arun;
  store_any(p.out, (size_t)row * 128 + tid, p.out_dtype, res);
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

extern "C" int ffa_q2fp8_decode_nchunks(int T, int BS, int SBS) {
  if (T <= 0 || BS <= 0 || SBS <= 0) return 0;
  const long ntb = (T + BS - 1) / BS;
  const long tokens = ntb * BS;  // the sub-blocks cover ceil(T/BS)*BS tokens
  const long wgs = (tokens + ffa::kWaves * ffa::kPage - 1) / (ffa::kWaves * ffa::kPage);
  return (int)(wgs * ffa::kWaves);
}

template <int L, int S, int R, int V>
static hipError_t launch_decode(const ffa::DecodeParams &p, dim3 grid, hipStream_t st) {
  hipLaunchKernelGGL((ffa::q2fp8_decode_kernel<L, S, R, V>), grid, dim3(256), 0, st, p);
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

extern "C" int ffa_q2fp8_decode(const ffa_q2fp8_decode_args *a, void *stream) {
  if (!a) return set_err(FFA_E_INVALID, "null args");
  if (a->B <= 0 || a->T <= 0 || a->HQ <= 0 || a->HKV <= 0) return set_err(FFA_E_INVALID, "bad dims");
  if (a->HQ % a->HKV) return set_err(FFA_E_INVALID, "HQ must be a multiple of HKV");
  const int G = a->HQ / a->HKV;
  if (G > 4) return set_err(FFA_E_UNSUPPORTED, "GQA group size > 4 is not implemented");
  if (a->SBS <= 0 || a->BS <= 0 || a->BS % a->SBS) return set_err(FFA_E_UNSUPPORTED, "BS must be a multiple of SBS");
  if (!(a->SBS == 16 || a->SBS == 32 || a->SBS == 64 || a->SBS == 128 || a->SBS == 256))
    return set_err(FFA_E_UNSUPPORTED, "SBS must be one of 16, 32, 64, 128, 256");
  if (!(a->q_dtype >= FFA_DT_F16 && a->q_dtype <= FFA_DT_F32)) return set_err(FFA_E_INVALID, "q dtype");
  if (!(a->out_dtype >= FFA_DT_F16 && a->out_dtype <= FFA_DT_F32)) return set_err(FFA_E_INVALID, "out dtype");
  if (!(a->v_dtype == FFA_DT_F16 || a->v_dtype == FFA_DT_BF16)) return set_err(FFA_E_INVALID, "v dtype");
  if (!(a->res_dtype == FFA_DT_FP8_E4M3 || a->res_dtype == FFA_DT_FP8_E5M2 || a->res_dtype == FFA_DT_NONE))
    return set_err(FFA_E_INVALID, "residual dtype");
  if (a->res_dtype != FFA_DT_NONE && !a->k_residual) return set_err(FFA_E_INVALID, "residual pointer is null");
  if (a->layout == FFA_LAYOUT_PAGED && !a->block_table) return set_err(FFA_E_INVALID, "paged layout needs a block table");
  if (a->layout == FFA_LAYOUT_CONTIG && a->scale_mode != FFA_SCALE_CHANNEL)
    return set_err(FFA_E_UNSUPPORTED, "contiguous layout supports per-channel scales only");
  if (a->scale_mode == FFA_SCALE_G32 && a->scale_dtype != FFA_DT_F16)
    return set_err(FFA_E_INVALID, "g32 scales must be fp16");
  const int need = ffa_q2fp8_decode_nchunks(a->T, a->BS, a->SBS);
  if (a->nchunks < need) return set_err(FFA_E_INVALID, "scratch holds too few chunks");
  const int ntbs = ((a->T + a->BS - 1) / a->BS) * (a->BS / a->SBS);
  if (a->ntbs < ntbs) return set_err(FFA_E_INVALID, "mask holds too few blocks");

  ffa::DecodeParams p;
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
  p.B = a->B;
  p.T = a->T;
  p.HQ = a->HQ;
  p.HKV = a->HKV;
  p.G = G;
  p.scale = a->scale;
  p.BS = a->BS;
  p.SBS = a->SBS;
  p.delta = a->delta;
  p.nch = a->nchunks;
  p.ntbs = a->ntbs;

  hipStream_t st = (hipStream_t)stream;
  dim3 grid(need / ffa::kWaves, a->B * a->HKV);
  hipError_t e;
  if (a->layout == FFA_LAYOUT_PAGED) {
    if (a->scale_mode == FFA_SCALE_G32)
      e = dispatch_rv<ffa::kPaged, ffa::kG32>(p, a->res_dtype, a->v_dtype, grid, st);
    else
      e = dispatch_rv<ffa::kPaged, ffa::kChannel>(p, a->res_dtype, a->v_dtype, grid, st);
  } else {
    e = dispatch_rv<ffa::kContig, ffa::kChannel>(p, a->res_dtype, a->v_dtype, grid, st);
  }
  if (e != hipSuccess) return set_err(FFA_E_LAUNCH, hipGetErrorString(e));
  hipLaunchKernelGGL(ffa::q2fp8_merge_kernel, dim3(a->B * a->HQ), dim3(128), 0, st, p);
  e = hipGetLastError();
  if (e != hipSuccess) return set_err(FFA_E_LAUNCH, hipGetErrorString(e));
  return FFA_OK;
}
