// Pruned decode attention for the other K formats of the reference, on gfx950:
//   fp8 base + fp8 residual   ffa-fp8fp8/attn_kernel/attn_kernel_v1210_fused_bsz_fp8fp8.py:10-136
//   nvfp4 (e2m1 x block scale) ffa-nvfp4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nvfp4fp8.py:10-169
//   nf4 (codebook x channel)  ffa-nf4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nf4fp8.py:41-167
// and a variant of the fp8 base with one fp16 scale per token and KV head, plus two paged
// modes (no reference counterpart): nvfp4 with one
// e4m3 scale per 16 channels of each token, nf4 with one fp16 scale per 64 channels, in
// 64-token pages (codes [P, HKV, 64, 64], scales [P, HKV, 64, 8 | 2], residual [P, HKV, 64, 128],
// V^T [P, HKV, 128, 64]; codes, residual and V in the page-internal orders of decode_common.h)
// read through a block table.
//
// Every format dequantizes to the fp16 K the reference feeds its dot products,
// k_hat = fp16(f32(value) * f32(scale)), and then follows the q2fp8 path: the probe
// threshold (nvfp4 scores its second probe window with the scale of block NTB-1,
// :96-97), group prune, refined K fp16(k_hat + fp16(res)), exp2 softmax, P.V, and the
// shared log-sum-exp merge kernel.  Contiguous token-major layouts as in the reference
// ([B, T, HKV, row]) or the pages above; one workgroup = 4 waves = 8 chunks of 64 tokens
// of one (sequence, KV head), the partial layout of the q2fp8 kernel.
//
// MFMA layout (as the q2fp8 kernel's per-channel mode): rows of a 16x16x32 f16 MFMA are
// tokens (row m of tile tau = token 4m + tau), the lane of k-chunk kc holds channels
// [32kc, 32kc + 32) of its token, and MFMA m' takes channels 32kc + 8m' + e; the q operand
// of column (group j, query row i) is nonzero only for kc == j, so the four groups come out
// in separate columns and are summed with DPP row rotations.
#include "decode_common.h"
#include "ffa_mi355x.h"

#include <type_traits>

extern "C" int ffa_set_error_internal(int code, const char *msg);
extern "C" int ffa_decode_shape_check(int B, int T, int HQ, int HKV, int BS, int SBS, float *piece_max, int npieces,
                                      const float *th_in, const float *th_out, ffa::DecodeParams *p);
extern "C" int ffa_decode_slots(int T, int BS, int span);

// Timeline build (-DFFA_TIMELINE only): per-wave s_memrealtime stamps at the FFA_STAMP points, 16
// words per wave into the buffer ffa_debug_set_timeline_kfmt sets (stamps 0-12, the chunks the wave
// refined, 0, and XCC_ID << 32 | HW_ID), as in the q2 decoder.
#ifdef FFA_TIMELINE
__device__ unsigned long long *g_timeline_k = nullptr;
#define FFA_STAMP(i) (st_[i] = __builtin_amdgcn_s_memrealtime())
#else
#define FFA_STAMP(i) ((void)0)
#endif

namespace ffa {

enum { kF8E4M3 = 0, kF8E5M2 = 1, kFP4 = 2, kNF4 = 3 };
enum { kSclNone = 0, kSclToken = 1, kSclBlock = 2, kSclChannel = 3, kSclG16 = 4, kSclG64 = 5 };

// fp16(a * sa) in the low half and fp16(b * sb) in the high half: the compiler turns each rounded
// fma with a zero addend into v_fma_mixlo_f16 / v_fma_mixhi_f16, which write one half and keep the
// other (no shift and OR to pack two separately rounded halves).  Written in C rather than inline
// assembly so that the compiler sees the two VALU writes and pads them before the MFMA that reads
// the register: an asm block is opaque to its hazard checks, and with one wait state between the
// asm's write and the MFMA (two are required) the MFMA could read the register's previous value.
__device__ __forceinline__ uint32_t mul_pack_f16(float a, float sa, float b, float sb) {
  const _Float16 lo = (_Float16)__builtin_fmaf(a, sa, 0.f);
  const _Float16 hi = (_Float16)__builtin_fmaf(b, sb, 0.f);
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, h2{lo, hi});
}

// QLoRA NF4 levels (the published 16 normal-float values), as fp32
__constant__ float kNF4Levels[16] = {
    -1.0f, -0.6961928009986877f, -0.5229921340942383f, -0.39491748809814453f, -0.28444138169288635f,
    -0.18477343022823334f, -0.09105003625154495f, 0.0f, 0.07958029955625534f, 0.16093020141124725f,
    0.24611230194568634f, 0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,
    0.7229568362236023f, 1.0f};

// two fp8 values (bytes 2*HI, 2*HI+1 of w) -> f32, exact
template <bool E4M3, bool HI>
__device__ __forceinline__ f32x2 fp8pair_f32(uint32_t w) {
  if constexpr (E4M3) return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, HI);
  else return __builtin_amdgcn_cvt_scalef32_pk_f32_bf8(w, 1.0f, HI);
}

__device__ __forceinline__ uint32_t pack_f16(float a, float b) {  // two RNE conversions, one instruction
  return pk_f16_bits(a, b);
}

// Scale value i of a float tensor of dtype dt (0=f16, 1=bf16, 2=f32), in two steps: scale_word
// loads the aligned 32-bit word holding it, scale_value converts it (odd = i & 1 picks the upper
// half of a 16-bit pair).  The conversion branches on the dtype, and a wait inside such a branch
// covers every load issued before it, so a group's words are converted only once all of the
// group's loads are out.
__device__ __forceinline__ uint32_t scale_word(brsrc rs, uint32_t i, int dt) {
  return bload4(rs, dt == 2 ? i * 4u : (i * 2u) & ~3u);
}
__device__ __forceinline__ float scale_value(uint32_t w, uint32_t odd, int dt) {
  const uint32_t bits = dt == 2 ? w : (odd ? (w >> 16) : (w & 0xffffu));
  return dt == 2 ? __uint_as_float(bits) : (dt == 1 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits));
}

// RELOAD: the exact pass loads a kept chunk's codes and scales again instead of keeping the
// scoring registers of the wave's other chunk, which roughly halves the registers.  RELOAD builds
// serve grids larger than the CU count: the paged one with four waves per SIMD (at most 128
// registers, one or two spilled) and the whole 8-chunk span as a constant, the contiguous one (54.7
// KB of LDS) with two workgroups per CU.  Small grids (at most one workgroup per CU) take the other
// build, with the span a runtime value: contiguous layouts keep the scoring registers, one latency
// chain per wave being all they have (the paged exact pass reloads its page either way).
// SPEC (contiguous, two-chunk spans only, where two of the four waves would own no chunk): a split by
// role.  Waves 2 and 3 own the two chunks: they load q, a probe window each and their chunk's codes,
// build all four q operands themselves and score.  Waves 0 and 1 load the residual and V rows of
// chunk wv (the chunk of wave wv + 2) before the prune decides it, and stage them in LDS: the
// residual before the probe barrier, the V tile rounded to fp16 after it (a second barrier hands
// it over).  Every load a chunk wave waits for is then its own, and the V rounding and staging
// leave its path.
template <int LAYOUT, int FMT, int SCL, int RES, int VT, bool RELOAD, bool SPEC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(LAYOUT == kPaged && RELOAD ? 4 : (RELOAD ? 2 : 1))))
void kfmt_decode_kernel(const DecodeParams p) {
  static_assert(!SPEC || !RELOAD, "speculative loads go with the small-grid build");
  typedef VTraits<VT> VTr;
#ifdef FFA_TIMELINE
  unsigned long long st_[16] = {0};
  int n_exact_ = 0;
#endif
  constexpr bool k4 = FMT == kFP4 || FMT == kNF4;
  constexpr bool kGrp = SCL == kSclG16 || SCL == kSclG64;  // per-token group scales (paged modes)
  static_assert(kGrp == (LAYOUT == kPaged), "group scales go with the paged layout");
  static_assert(SCL != kSclG16 || FMT == kFP4, "g16 scales are nvfp4's");
  static_assert(SCL != kSclG64 || FMT == kNF4, "g64 scales are nf4's");
  constexpr int kRow = k4 ? 64 : 128;  // K bytes of one token and KV head
  constexpr int kLane = kRow / 4;      // bytes of one lane's 32 channels
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // grid (span, KV head, sequence), the span fastest (consecutive workgroups on different XCDs);
  // the contiguous 8-bit formats, whose K and V rows of a token give each KV head whole lines, and
  // the paged small-grid builds place the KV head fastest instead, so that a (sequence, KV head)'s
  // partials stay in one XCD's L2 for the merge (grid_pos).  In the paged large-batch build the KV
  // head fastest took config 4 from 139.8 to 141.7 us (config 3 86.6 -> 86.1 us)
  const GridPos gp = grid_pos<(LAYOUT == kContig && !k4) || (LAYOUT == kPaged && !RELOAD)>();
  const int cg = gp.cg;  // workgroup index along the sequence = partial slot
  const DecodeUnit un = decode_unit(p, gp.y);  // KV head and the (at most 4) query rows of this workgroup
  const int hkv = un.hkv;
  const int b = gp.b;
  // span: chunks of this workgroup (8, or 4 / 2 for small grids, where each wave owns one chunk
  // and waves past the span own none); slot (w, j) = the j-th chunk of the wave in place w of the
  // chunk order (wch below: the wave itself, or in SPEC wave w ^ 2).  The paged large-batch build
  // keeps the whole span as a constant (the runtime form costs it registers)
  constexpr bool kPagedBig = LAYOUT == kPaged && RELOAD;
  const int span = kPagedBig ? kChunksPerWG : (SPEC ? kMinSpan : decode_span(p));
  const int ppw = span >= kChunksPerWG ? kPPW : 1;
  const int cw = cg * span;
  // the wave's place in the chunk order: its own index, or (SPEC) waves 2, 3 first
  const int wch = SPEC ? (wv ^ 2) : wv;
  const int c0 = cw + wch * ppw;
  const int SBS = p.SBS;
  bool own[kPPW];
#pragma unroll
  for (int j = 0; j < kPPW; ++j) own[j] = j < ppw && wch * ppw + j < span;
  // first chunk of slot sl (and whether the slot holds a chunk of this workgroup)
  auto slot_chunk = [&](int sl) { return cw + (sl >> 1) * ppw + (sl & 1); };
  auto slot_owned = [&](int sl) { return (sl & 1) < ppw && (sl >> 1) * ppw + (sl & 1) < span; };

  const int mrow = lane & 15;
  const int kc = lane >> 4;
  const int n = mrow;
  const int jg = n >> 2;
  const int ir = n & 3;
  const bool row_ok = ir < un.Gu;
  const int hq = un.row0 + (row_ok ? ir : 0);

  __shared__ uint4 s_qa[4][64];
  __shared__ float s_probe[2][4];
  __shared__ float s_wmax[kWaves][4];
  __shared__ int s_keep[kChunksPerWG * kPage / 16];  // pass 2: block decisions of the span
  __shared__ uint32_t s_bal[kChunksPerWG][2];
  __shared__ float s_pm[kChunksPerWG][4], s_pl[kChunksPerWG][4];
  __shared__ float s_po[kChunksPerWG][4][128];
  // nf4: the codebook levels of both nibbles of every code byte, (low, high) at [byte]
  __shared__ float2 s_cb2[FMT == kNF4 ? 256 : 1];
  // V staging (contiguous layouts), and in SPEC the residual and V handed from waves 0 and 1 to
  // waves 2 and 3: per-wave regions of kStage bytes (a row-major V tile, or a paged V^T block of
  // 16 KB in the lanes' load order)
  constexpr int kStage = LAYOUT == kContig ? kPage * (RELOAD ? kVRowHalf : kVRow) : (SPEC ? kPage * kD * 2 : 0);
  __shared__ __attribute__((aligned(16))) uint8_t s_vstage[kStage > 0 ? kWaves * kStage : 16];

  auto lds_barrier = []() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

  // ------------------------------------------------ phase 1: loads (issued on every path)
  const int Tb = p.seq_lens ? min(max(p.seq_lens[b], 0), p.T) : p.T;  // lengths beyond T are clamped to T
  if (cg > 0 && cw * kPage >= Tb) {  // every token past the sequence end: mask bytes only
    if (p.pass != 1 && un.quad == 0) write_empty_mask(p.mask + ((size_t)b * p.HKV + hkv) * p.ntbs, cg, SBS, p.ntbs, span);
    return;
  }
  FFA_STAMP(0);
  if (threadIdx.x < kChunksPerWG * kPage / 16) s_keep[threadIdx.x] = 0;
  const int NTB = div_bs(p, Tb + p.BS - 1);
  const int NTBS_b = NTB * div_pow2(p.BS, p.SBS);
  const int NTBk = div_bs(p, p.T + p.BS - 1);  // blocks of the block-scale tensor
  // probe windows: waves 0 and 1 (SPEC: 2 and 3, the waves with the operands)
  const bool do_probe = (p.th_in == nullptr) && wch < 2;
  const int pa = wch == 0 ? 0 : max(NTB - 1, 0) * 16;  // probe window (attn_kernel...q2fp8.py:58-73)
  int nv[kPPW];  // valid tokens of the wave's chunks (0 for a chunk it does not own)
#pragma unroll
  for (int j = 0; j < kPPW; ++j) nv[j] = own[j] ? min(max(Tb - (c0 + j) * kPage, 0), kPage) : 0;

  // nf4: this thread's entries of the LDS level-pair table, loaded (constant memory) before every
  // other load, so that writing the table later waits for these loads only (loaded after the code
  // rows, the write waited for the codes and held the operand build behind them)
  float2 cbv[SPEC ? 4 : 1];
  if constexpr (FMT == kNF4) {
#pragma unroll
    for (int r = 0; r < (SPEC ? 4 : 1); ++r) {
      const int i = SPEC ? lane + 64 * r : (int)threadIdx.x;
      cbv[r] = make_float2(kNF4Levels[i & 15], kNF4Levels[i >> 4]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  uint32_t pg_lane = 0;
  if constexpr (LAYOUT == kPaged) {
    // page ids: one vector load per wave, issued first (lanes 0, 1: the wave's chunks, lane 2: its
    // probe window; the other lanes read past the resource and get 0)
    // (SPEC, waves 0 and 1: lane 0 reads the page of chunk cw + wv, whose rows they load)
    const bool ld = SPEC && wv < 2;
    const int lc = cw + (wv & 1);
    const bool need = lane < kPPW ? (ld ? lane == 0 && lc * kPage < Tb : nv[lane & 1] > 0)
                                  : (lane == kPPW && do_probe && pa < Tb);
    const int idx = lane < kPPW ? (ld ? lc : c0 + lane) : (pa >> 6);
    pg_lane = bload4(make_rsrc(p.bt + (size_t)b * p.bt_stride, p.bt_stride * 4), need ? idx * 4 : p.bt_stride * 4);
    pg_lane = pg_lane < (uint32_t)p.num_pages ? pg_lane : 0u;  // ids outside the pools read page 0
  }
  const uint32_t es_q = p.q_dtype == 2 ? 4u : 2u;
  const int hwin = wv >> 1;
  // the lane's 16 q channels of its wave's operand (SPEC: the 32 of all four operands, in waves 2
  // and 3; waves 0 and 1 read nothing)
  Raw16 qraw, qraw2;
  {
    const uint32_t qb = p.HQ * kD * es_q;
    const brsrc qrs = make_rsrc((const char *)p.q + (size_t)b * p.HQ * kD * es_q, SPEC && wv < 2 ? 0u : qb);
    if constexpr (SPEC) {
      raw16_load(qraw, qrs, (hq * kD + 32 * kc) * es_q, es_q, qb);
      raw16_load(qraw2, qrs, (hq * kD + 32 * kc + 16) * es_q, es_q, qb);
    } else {
      raw16_load(qraw, qrs, (hq * kD + 32 * kc + 16 * hwin) * es_q, es_q, qb);
    }
  }
  const float th_pre = __uint_as_float(
      bload8(make_rsrc(p.th_in + (p.th_in ? (size_t)b * p.HQ : 0), p.th_in ? p.HQ * 4 : 0), hq * 4).x);
  int pg[kPPW] = {0, 0};
  int ppg = 0;
  // the q loads go out before the wait for the page ids and before the code loads, whose waits
  // would otherwise cover them
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (LAYOUT == kPaged) {
#pragma unroll
    for (int j = 0; j < kPPW; ++j) pg[j] = __builtin_amdgcn_readlane(pg_lane, j);
    ppg = __builtin_amdgcn_readlane(pg_lane, kPPW);
  }
  // pool block (page, head) of the paged layout: kPage rows of kRow bytes
  auto page_rows = [&](const uint8_t *pool, int page, int row_bytes, bool valid) -> brsrc {
    return make_rsrc(pool + ((size_t)page * p.HKV + hkv) * kPage * row_bytes, valid ? kPage * row_bytes : 0);
  };
  // group scales of the lane's 32 channels for one token of a page: (scale of channels
  // [32kc, 32kc + 16), scale of [32kc + 16, 32kc + 32)) -- e4m3 per 16 channels, or fp16 per 64
  auto group_scales = [&](const brsrc &rs, int tok) -> f32x2 {
    if constexpr (SCL == kSclG16) {
      const uint32_t w = bload4(rs, tok * 8 + 4 * (kc >> 1));
      return fp8pair_f32<true, false>((kc & 1) ? (w >> 16) : w);
    } else {
      const uint32_t w = bload4(rs, tok * 4);
      const float sc = f16_bits_to_f32((kc >> 1) ? (w >> 16) : (w & 0xffffu));
      return f32x2{sc, sc};
    }
  };
  // per-channel scales of the lane's 32 channels (nf4): eight 16-byte loads whatever the dtype,
  // converted in phase 2b (a conversion here would hold the code loads behind their round trip)
  float sch[32];
  uint4 sraw[8];
  if constexpr (SCL == kSclChannel) {
    const uint32_t es = p.s_dtype == 2 ? 4u : 2u;
    const brsrc rs = make_rsrc((const char *)p.ks + ((size_t)b * p.HKV + hkv) * kD * es, kD * es);
#pragma unroll
    for (int i = 0; i < 8; ++i) sraw[i] = bload16(rs, 32 * kc * es + 16 * i);
  }
  const brsrc rsc = make_rsrc(p.ks, SCL == kSclToken ? (uint32_t)(p.B * p.T * p.HKV) * (p.s_dtype == 2 ? 4u : 2u)
                                   : SCL == kSclBlock ? (uint32_t)(p.B * NTBk * p.HKV) * (p.s_dtype == 2 ? 4u : 2u)
                                                      : 0u);
  // element index of the scale of token t (token mode) or of block blk (block mode)
  constexpr bool kTokScale = SCL == kSclToken || SCL == kSclBlock;
  auto scale_index = [&](int t, int blk) -> uint32_t {
    if constexpr (SCL == kSclToken) return ((uint32_t)b * p.T + (uint32_t)min(t, p.T - 1)) * p.HKV + hkv;
    else return ((uint32_t)b * NTBk + (uint32_t)blk) * p.HKV + hkv;
  };
  // probe tile: MFMA row m <-> token pa + m
  uint4 pxa, pxb = make_uint4(0, 0, 0, 0);
  float psc = 1.f;
  uint32_t psw = 0, psodd = 0;  // probe scale word, converted after the chunk loads
  f32x2 pgs = {1.f, 1.f};
  {
    const bool pv = do_probe && pa < Tb;
    if constexpr (LAYOUT == kPaged) {
      // the 16 window tokens lie in one page (pa is a multiple of 16); rows past the sequence
      // end hold no data, their scores are masked below
      const int tok = (pa & (kPage - 1)) + mrow;
      pxa = bload16(page_rows(p.kq, ppg, kRow, pv), k4_off(tok, 16 * kc));
      pgs = group_scales(page_rows((const uint8_t *)p.ks, ppg, SCL == kSclG16 ? 8 : 4, pv), tok);
    } else {
      const int nt = pv ? min(16, Tb - pa) : 0;
      const brsrc rc = make_rsrc(p.kq + (((size_t)b * p.T + pa) * p.HKV + hkv) * kRow, nt > 0 ? ((nt - 1) * p.HKV + 1) * kRow : 0);
      const uint32_t off = mrow * p.HKV * kRow + kLane * kc;
      pxa = bload16(rc, off);
      if constexpr (!k4) pxb = bload16(rc, off + 16);
      // nvfp4: window 0 uses block 0's scale, window 1 block NTB-1's (attn_kernel...nvfp4fp8.py:86-97)
      if constexpr (kTokScale) {
        const uint32_t si = scale_index(pa + mrow, wch == 0 ? 0 : max(NTB - 1, 0));
        psw = scale_word(rsc, si, p.s_dtype);
        psodd = si & 1u;
      }
    }
  }
  // residual and V loads of one chunk (page pg, or the contiguous rows of tokens t0 .. t0 + nvs;
  // nvs = 0 gives empty resources: the loads return zeros without a memory access)
  auto issue_res = [&](int pgid, int t0, int nvs, uint4 (&rr)[4][2]) {
    if constexpr (RES != kResNone) {
      const brsrc rs = LAYOUT == kPaged ? page_rows(p.kr, pgid, kD, !SPEC || nvs > 0)
                                        : make_rsrc(p.kr + (((size_t)b * p.T + t0) * p.HKV + hkv) * kD,
                                                    nvs > 0 ? ((nvs - 1) * p.HKV + 1) * kD : 0);
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) {
        if constexpr (LAYOUT == kPaged) {  // blocks (tau, h) of the page's residual
          rr[tau][0] = bload16_nt(rs, ((tau * 2 + 0) * 64 + lane) * 16);
          rr[tau][1] = bload16_nt(rs, ((tau * 2 + 1) * 64 + lane) * 16);
        } else {  // two loads of alternate 16-byte pieces of the same lines: default cache policy
          const uint32_t off = (4 * mrow + tau) * p.HKV * kD + 32 * kc;
          rr[tau][0] = bload16(rs, off);
          rr[tau][1] = bload16(rs, off + 16);
        }
      }
    }
  };
  auto issue_v = [&](int pgid, int t0, int nvs, uint4 (&vv)[8][2]) {
    if constexpr (LAYOUT == kPaged) {
      // V^T page: lane (n, kc) reads column 16 nu + n, tokens 16 kc + 8 kap .. + 8 (vt_off order)
      const brsrc vs = make_rsrc((const uint16_t *)p.v + ((size_t)pgid * p.HKV + hkv) * (kD * kPage), !SPEC || nvs > 0 ? kD * kPage * 2 : 0);
#pragma unroll
      for (int nu = 0; nu < 8; ++nu)
#pragma unroll
        for (int kap = 0; kap < 2; ++kap) vv[nu][kap] = bload16_nt(vs, ((nu * 2 + kap) * 64 + lane) * 16);  // block (nu, kap)
    } else {
      const brsrc vs = make_rsrc((const uint16_t *)p.v + (((size_t)b * p.T + t0) * p.HKV + hkv) * kD,
                                 nvs > 0 ? ((nvs - 1) * p.HKV + 1) * kD * 2 : 0);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int idx = r * 64 + lane;
        const int tk = idx >> 4, vc = idx & 15;
        vv[r >> 1][r & 1] = bload16_nt(vs, tk * p.HKV * kD * 2 + 16 * vc);
      }
    }
  };
  // the contiguous V tile [64 tokens][128] loaded by issue_v, row-major into LDS rows of kVRow bytes,
  // rounded to fp16 (rows past the sequence end were loaded as zeros)
  auto stage_v_f16 = [&](const uint4 (&vv)[8][2], uint8_t *st) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int idx = r * 64 + lane;
      const int tk = idx >> 4, vc = idx & 15;
      const uint4 v4 = vv[r >> 1][r & 1];
      const u32x4 w = __builtin_bit_cast(u32x4, VTr::operand(u32x4{v4.x, v4.y, v4.z, v4.w}));
      uint2 *d = (uint2 *)(st + tk * kVRow + 16 * vc);  // rows are 8-byte aligned
      d[0] = make_uint2(w[0], w[1]);
      d[1] = make_uint2(w[2], w[3]);
    }
  };
  uint4 xa[kPPW][4], xb[kPPW][4];
  float xs[kPPW][4];
  uint32_t xsw[kPPW][4], xsodd = 0;  // token / block scale words (bit 4j + tau of xsodd: odd index)
  f32x2 xg[kPPW][4];  // group scales (paged modes)
#pragma unroll
  for (int j = 0; j < kPPW; ++j) {
    const int t0 = (c0 + j) * kPage;
    if constexpr (LAYOUT == kPaged) {
      const brsrc rc = page_rows(p.kq, pg[j], kRow, nv[j] > 0);
      const brsrc rs = page_rows((const uint8_t *)p.ks, pg[j], SCL == kSclG16 ? 8 : 4, nv[j] > 0);
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) {
        xa[j][tau] = bload16_nt(rc, (tau * 64 + lane) * 16);  // block tau: token 4 mrow + tau, bytes 16 kc + (0..15)
        xb[j][tau] = make_uint4(0, 0, 0, 0);
        xs[j][tau] = 1.f;
        xg[j][tau] = group_scales(rs, 4 * mrow + tau);
      }
    } else {
      const brsrc rc = make_rsrc(p.kq + (((size_t)b * p.T + t0) * p.HKV + hkv) * kRow,
                                 nv[j] > 0 ? ((nv[j] - 1) * p.HKV + 1) * kRow : 0);
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) {
        const uint32_t off = (4 * mrow + tau) * p.HKV * kRow + kLane * kc;
        xa[j][tau] = bload16(rc, off);
        xb[j][tau] = make_uint4(0, 0, 0, 0);
        if constexpr (!k4) xb[j][tau] = bload16(rc, off + 16);
        const int t = t0 + 4 * mrow + tau;
        xs[j][tau] = 1.f;
        if constexpr (kTokScale) {
          const uint32_t si = scale_index(t, div_bs(p, min(t, max(Tb - 1, 0))));
          xsw[j][tau] = scale_word(rsc, si, p.s_dtype);
          xsodd |= (si & 1u) << (4 * j + tau);
        }
        xg[j][tau] = f32x2{1.f, 1.f};
      }
    }
  }
  // SPEC: waves 0 and 1 load the residual and V rows of the chunk of wave wv + 2, before the prune
  // decides it, and stage them in LDS for that wave (the chunk waves' own loads, issued above on
  // empty resources in waves 0 and 1, go out first; no load follows them in waves 2 and 3).  They
  // sleep about 0.25 us first, so that the chunk waves' code rows, which gate the decision, meet
  // fewer of these rows in the memory queues (config 1: 10.27 -> 10.14 us per step; twice as long
  // gave nothing)
  uint4 srr[4][2], svv[8][2];
  if constexpr (SPEC) {
    if (wv < 2) {
      __builtin_amdgcn_s_sleep(10);
      const int lc = cw + wv;
      const int nl = min(max(Tb - lc * kPage, 0), kPage);
      issue_res(pg[0], lc * kPage, nl, srr);
      issue_v(pg[0], lc * kPage, nl, svv);
    }
  }
  if constexpr (FMT == kNF4) {
    if constexpr (SPEC) {  // no barrier before the scoring: each chunk wave writes the whole table
      if (wv >= 2)
#pragma unroll
        for (int r = 0; r < 4; ++r) s_cb2[lane + 64 * r] = cbv[r];
    } else {
      s_cb2[threadIdx.x] = cbv[0];
    }
  }

  FFA_STAMP(1);
  // ------------------------------------------------ phase 2a: q operands (one per wave)
  // operand of MFMA m' = 2h + s from the lane's 16 channels 32kc + 16h + (0..15)
  auto operand_of = [&](const Raw16 &raw, auto S) -> u32x4 {
    constexpr int s = decltype(S)::value;
    float qv[16];
    raw16_to_f32(raw, p.q_dtype, qv);
    u32x4 a4;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const float e0 = (row_ok && kc == jg) ? (float)(_Float16)qv[8 * s + 2 * qq] : 0.f;
      const float e1 = (row_ok && kc == jg) ? (float)(_Float16)qv[8 * s + 2 * qq + 1] : 0.f;
      a4[qq] = f32_to_f16_bits(e0) | (f32_to_f16_bits(e1) << 16);
    }
    return a4;
  };
  f16x8 qa[4];
  if constexpr (SPEC) {  // waves 2 and 3 build all four (waves 0 and 1 score nothing)
    if (wv >= 2) {
      qa[0] = __builtin_bit_cast(f16x8, operand_of(qraw, std::integral_constant<int, 0>()));
      qa[1] = __builtin_bit_cast(f16x8, operand_of(qraw, std::integral_constant<int, 1>()));
      qa[2] = __builtin_bit_cast(f16x8, operand_of(qraw2, std::integral_constant<int, 0>()));
      qa[3] = __builtin_bit_cast(f16x8, operand_of(qraw2, std::integral_constant<int, 1>()));
    }
    FFA_STAMP(2);
  } else {  // one per wave, shared through LDS
    u32x4 a4;
    if (wv & 1) a4 = operand_of(qraw, std::integral_constant<int, 1>());
    else a4 = operand_of(qraw, std::integral_constant<int, 0>());
    s_qa[wv][lane] = make_uint4(a4[0], a4[1], a4[2], a4[3]);
    lds_barrier();
    FFA_STAMP(2);
#pragma unroll
    for (int mp = 0; mp < 4; ++mp) {
      const uint4 a = s_qa[mp][lane];
      qa[mp] = __builtin_bit_cast(f16x8, u32x4{a.x, a.y, a.z, a.w});
    }
  }

  // fp16 K of MFMA m' (channels 32kc + 8m' + e) from the lane's row bytes
  auto dequant = [&](const uint4 &a, const uint4 &bq, int mp, float sc, f32x2 gs) -> f16x8 {
    u32x4 r;
    if constexpr (kGrp) sc = mp < 2 ? gs[0] : gs[1];  // channels 32kc + 8mp + e lie in the first or second half
    if constexpr (!k4) {
      const uint4 &src = mp < 2 ? a : bq;
      const uint32_t lo = (mp & 1) ? src.z : src.x, hi = (mp & 1) ? src.w : src.y;
      if constexpr (SCL == kSclNone) {
        return fp8x8_to_f16x8<FMT == kF8E4M3 ? kResE4M3 : kResE5M2>(lo, hi);
      } else {
        const f32x2 v0 = fp8pair_f32<FMT == kF8E4M3, false>(lo), v1 = fp8pair_f32<FMT == kF8E4M3, true>(lo);
        const f32x2 v2 = fp8pair_f32<FMT == kF8E4M3, false>(hi), v3 = fp8pair_f32<FMT == kF8E4M3, true>(hi);
        r[0] = pack_f16(v0[0] * sc, v0[1] * sc);
        r[1] = pack_f16(v1[0] * sc, v1[1] * sc);
        r[2] = pack_f16(v2[0] * sc, v2[1] * sc);
        r[3] = pack_f16(v3[0] * sc, v3[1] * sc);
      }
    } else {
      const uint32_t w = mp == 0 ? a.x : mp == 1 ? a.y : mp == 2 ? a.z : a.w;
      if constexpr (FMT == kFP4 && SCL == kSclG16) {
        // e2m1 pairs of each byte (low nibble first) to fp16 (exact), times the e4m3 group scale
        // in fp16: both have at most 4 significant bits and the product lies in [2^-10, 2688],
        // so it is exact in fp16 and equals the reference's product rounded to fp16
        const f16x2 s2 = {(_Float16)sc, (_Float16)sc};
        r[0] = f16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 0) * s2);
        r[1] = f16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 1) * s2);
        r[2] = f16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 2) * s2);
        r[3] = f16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 3) * s2);
      } else if constexpr (FMT == kFP4) {
        // e2m1 pairs of each byte (low nibble first), exact in f32, times the scale, RNE to fp16
        const f32x2 v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
        const f32x2 v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
        const f32x2 v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
        const f32x2 v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
        r[0] = pack_f16(v0[0] * sc, v0[1] * sc);
        r[1] = pack_f16(v1[0] * sc, v1[1] * sc);
        r[2] = pack_f16(v2[0] * sc, v2[1] * sc);
        r[3] = pack_f16(v3[0] * sc, v3[1] * sc);
      }
      if constexpr (FMT == kNF4) {
        // one 8-byte read per code byte: the levels of its low and high nibbles
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const float2 lv = s_cb2[(w >> (8 * h)) & 0xffu];
          const float l0 = lv.x, l1 = lv.y;
          const float s0 = kGrp ? sc : sch[8 * mp + 2 * h], s1 = kGrp ? sc : sch[8 * mp + 2 * h + 1];
          r[h] = mul_pack_f16(l0, s0, l1, s1);
        }
      }
    }
    return __builtin_bit_cast(f16x8, r);
  };
  // dot products of one 16-token tile with the lane's column, summed over the four groups
  // (kh: where to keep the tile's fp16 K operands, or nullptr)
  auto score_tile = [&](const uint4 &a, const uint4 &bq, float sc, f32x2 gs, float *out, f16x8 *kh) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int mp = 0; mp < 4; ++mp) {
      const f16x8 k = dequant(a, bq, mp, sc, gs);
      if (kh != nullptr) kh[mp] = k;
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k, qa[mp], acc, 0, 0, 0);
    }
#pragma unroll
    for (int uu = 0; uu < 4; ++uu) {
      float r = acc[uu];
      r += dpp<kRowRor4>(r);
      r += dpp<kRowRor8>(r);
      out[uu] = r;
    }
  };
  const float cs1 = p.scale;

  // ------------------------------------------------ phase 2b: probe, scores, prune
  float R[kPPW][16];
  // SPEC with a residual: the chunk's fp16 K operands from the scoring, kept for the refine (a
  // second dequantization would sit on the wave's chain after the prune decision)
  constexpr bool kKeepK = SPEC && RES != kResNone;
  f16x8 khat[4][4];
  uint64_t bal[kPPW] = {0, 0};
  float th = INFINITY;
  float mb[kPPW] = {-INFINITY, -INFINITY};
  if (!SPEC || wv >= 2) {  // (SPEC: waves 0 and 1 stage the residual rows instead, below)
  // token / block scales: converted here, after the operands, so that the dtype branches' waits
  // (which cover every load issued before them) come after the q operands are built
  if constexpr (LAYOUT != kPaged && kTokScale) {
    __builtin_amdgcn_sched_barrier(0);
    psc = scale_value(psw, psodd, p.s_dtype);
#pragma unroll
    for (int j = 0; j < kPPW; ++j)
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) xs[j][tau] = scale_value(xsw[j][tau], (xsodd >> (4 * j + tau)) & 1u, p.s_dtype);
  }
  if constexpr (SCL == kSclChannel) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t w[4] = {sraw[i].x, sraw[i].y, sraw[i].z, sraw[i].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (p.s_dtype == 2) {
          sch[4 * i + k] = __uint_as_float(w[k]);
        } else if (i < 4) {
          const uint32_t lo = w[k] & 0xffffu, hi = w[k] >> 16;
          sch[8 * i + 2 * k] = p.s_dtype == 1 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
          sch[8 * i + 2 * k + 1] = p.s_dtype == 1 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
        }
      }
    }
  }
  if (do_probe) {
    float r4[4];
    score_tile(pxa, pxb, psc, pgs, r4, nullptr);
    float mx = -INFINITY;
#pragma unroll
    for (int uu = 0; uu < 4; ++uu) {
      const int t = pa + 4 * kc + uu;  // output row 4kc + uu
      mx = fmaxf(mx, t < Tb ? (r4[uu] * cs1) * kLog2e : -INFINITY);
    }
    mx = xor_max(mx, 16);
    mx = xor_max(mx, 32);
    if (lane < 4) s_probe[wch][lane] = mx;
  }
  // R[j][k] = raw score of token (c0+j)*64 + 16kc + k (k = 4u + tau)
  auto score_page = [&](auto J) {
    constexpr int j = decltype(J)::value;
    const int t0 = (c0 + j) * kPage;
    if (nv[j] > 0) {
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) {
        float r4[4];
        score_tile(xa[j][tau], xb[j][tau], xs[j][tau], xg[j][tau], r4, kKeepK && j == 0 ? khat[tau] : nullptr);
#pragma unroll
        for (int uu = 0; uu < 4; ++uu) R[j][4 * uu + tau] = r4[uu];
      }
      if (t0 + kPage > Tb) [[unlikely]] {  // tokens past the sequence end
#pragma unroll
        for (int k = 0; k < 16; ++k)
          if (t0 + 16 * kc + k >= Tb) R[j][k] = -INFINITY;
      }
    }  // a page past the sequence end leaves R[j] unset: lane_max gives -inf and it is never kept
  };
  auto lane_max = [&](int j) -> float {
    if (nv[j] <= 0) return -INFINITY;
    float m = R[j][0];
#pragma unroll
    for (int k = 1; k < 16; ++k) m = fmaxf(m, R[j][k]);
    return (m * cs1) * kLog2e;
  };
  score_page(std::integral_constant<int, 0>());
  score_page(std::integral_constant<int, 1>());
  mb[0] = lane_max(0);
  mb[1] = lane_max(1);
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
  } else if constexpr (SPEC) {
    // the residual rows of the chunk of wave wv + 2 into LDS, in the lane order of the loads (the
    // staging buffer of this wave, unused otherwise)
    uint4 *dst = (uint4 *)(s_vstage + wv * kStage);
#pragma unroll
    for (int tau = 0; tau < 4; ++tau)
#pragma unroll
      for (int h = 0; h < 2; ++h) dst[(tau * 2 + h) * 64 + lane] = srr[tau][h];
  }
  FFA_STAMP(3);
  lds_barrier();  // probe maxima (and per-wave block maxima)
  FFA_STAMP(4);
  if (p.th_in != nullptr) th = row_ok ? th_pre : INFINITY;
  else th = row_ok ? fmaxf(s_probe[0][ir], s_probe[1][ir]) - p.delta : INFINITY;
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
  for (int j = 0; j < kPPW; ++j) {
    bal[j] = chunk_ballot(p, row_ok, mb[j], th, s_keep, cw, c0 + j, kc);
    if (nv[j] <= 0) bal[j] = 0;  // past the sequence end, or not this wave's chunk
    const int slot = wch * kPPW + j;
    if (lane == 0) {
      s_bal[slot][0] = (uint32_t)bal[j];
      s_bal[slot][1] = (uint32_t)(bal[j] >> 32);
    }
  }

  // ------------------------------------------------ phase 3: exact pass over this wave's kept chunks
  auto exact_chunk = [&](auto J) {
    FFA_STAMP(5);
#ifdef FFA_TIMELINE
    ++n_exact_;
#endif
    constexpr int j = decltype(J)::value;
    const int slot = wch * kPPW + j;
    const int t0 = (c0 + j) * kPage;
    const int nvs = min(Tb - t0, kPage);
    const uint64_t bl = bal[j];
    const bool keep16 = SBS == 16   ? ((bl >> (16 * kc)) & 0xffffull) != 0
                        : SBS == 32 ? ((bl >> (32 * (kc >> 1))) & 0xffffffffull) != 0
                                    : bl != 0;
    uint4 rr[4][2];
    uint4 vv[8][2];
    // the chunk's codes and scales again (cache-hot), so that the scoring registers of the
    // wave's other chunk are not held through this exact pass
    uint4 ka[4], kb[4];
    float ksc[4];
    f32x2 kg[4];
    uint32_t ksw[4], ksodd = 0;  // reloaded scale words, converted once the residual and V loads are out
    if constexpr (kKeepK) {
      // the fp16 K operands kept from the scoring (khat): no codes or scales here
    } else if constexpr (LAYOUT == kPaged) {
      const brsrc rc = page_rows(p.kq, pg[j], kRow, true);
      const brsrc rs = page_rows((const uint8_t *)p.ks, pg[j], SCL == kSclG16 ? 8 : 4, true);
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) {
        ka[tau] = bload16(rc, (tau * 64 + lane) * 16);
        kb[tau] = make_uint4(0, 0, 0, 0);
        ksc[tau] = 1.f;
        kg[tau] = group_scales(rs, 4 * mrow + tau);
      }
    } else if constexpr (!RELOAD) {
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) {
        ka[tau] = xa[j][tau];
        kb[tau] = xb[j][tau];
        ksc[tau] = xs[j][tau];
        kg[tau] = xg[j][tau];
      }
    } else {
      const brsrc rc = make_rsrc(p.kq + (((size_t)b * p.T + t0) * p.HKV + hkv) * kRow, ((nvs - 1) * p.HKV + 1) * kRow);
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) {
        const uint32_t off = (4 * mrow + tau) * p.HKV * kRow + kLane * kc;
        ka[tau] = bload16(rc, off);
        kb[tau] = make_uint4(0, 0, 0, 0);
        if constexpr (!k4) kb[tau] = bload16(rc, off + 16);
        const int t = t0 + 4 * mrow + tau;
        ksc[tau] = 1.f;
        if constexpr (kTokScale) {
          const uint32_t si = scale_index(t, div_bs(p, min(t, max(Tb - 1, 0))));
          ksw[tau] = scale_word(rsc, si, p.s_dtype);
          ksodd |= (si & 1u) << tau;
        }
        kg[tau] = f32x2{1.f, 1.f};
      }
    }
    if constexpr (SPEC) {  // staged by wave wv - 2 before the probe barrier
      const uint4 *src = (const uint4 *)(s_vstage + (wv - 2) * kStage);
#pragma unroll
      for (int tau = 0; tau < 4; ++tau)
#pragma unroll
        for (int h = 0; h < 2; ++h) rr[tau][h] = src[(tau * 2 + h) * 64 + lane];
    } else {
      issue_res(pg[j], t0, nvs, rr);
      issue_v(pg[j], t0, nvs, vv);
    }
    if constexpr (LAYOUT != kPaged && RELOAD && kTokScale) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) ksc[tau] = scale_value(ksw[tau], (ksodd >> tau) & 1u, p.s_dtype);
    }
    FFA_STAMP(6);
    float Rj[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) Rj[k] = R[j][k];
    if constexpr (RES != kResNone) {
      // reference: k_tilde = fp16(k_hat + fp16(res)), full re-score (attn_kernel...fp8fp8.py:109-116)
#pragma unroll
      for (int tau = 0; tau < 4; ++tau) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mp = 0; mp < 4; ++mp) {
          const uint4 &rs4 = rr[tau][mp >> 1];
          const uint32_t lo = (mp & 1) ? rs4.z : rs4.x, hi = (mp & 1) ? rs4.w : rs4.y;
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              add_f16x8(kKeepK && j == 0 ? khat[tau][mp] : dequant(ka[tau], kb[tau], mp, ksc[tau], kg[tau]),
                        fp8x8_to_f16x8<RES>(lo, hi)),
              qa[mp], acc, 0, 0, 0);
        }
#pragma unroll
        for (int uu = 0; uu < 4; ++uu) {
          float r = acc[uu];
          r += dpp<kRowRor4>(r);
          r += dpp<kRowRor8>(r);
          Rj[4 * uu + tau] = r;
        }
      }
    }
    FFA_STAMP(7);
    // softmax partial over the active tokens (valid, in a kept prune block, a row of the group)
    const int nact = (row_ok && keep16) ? min(max(Tb - (t0 + 16 * kc), 0), 16) : 0;
    float P[16], mrow_max, lsum;
    // (the paged large-batch build, at 128 registers, keeps one masked copy of the softmax)
    chunk_softmax<!kPagedBig>(Rj, cs1, nact, P, mrow_max, lsum);
    FFA_STAMP(8);
    typename VTr::vec pa2[2];
#pragma unroll
    for (int kap = 0; kap < 2; ++kap) {
      u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = VTr::pack2(P[8 * kap + 2 * e], P[8 * kap + 2 * e + 1]);
      pa2[kap] = __builtin_bit_cast(typename VTr::vec, w);
    }
    f32x4 oacc[8];
#pragma unroll
    for (int nu = 0; nu < 8; ++nu) oacc[nu] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (LAYOUT == kPaged) {
      // a partial page ANDs each lane's V words with the mask of its valid tokens (one copy of the
      // loop, at 128 registers: a uniform branch per V block; always ANDing measured 3 % slower at
      // configs 3 and 4)
      const bool partial = nvs < kPage;
      u32x4 keepw[2];
      if (partial) partial_page_masks(kc, nvs, keepw);
      if constexpr (SPEC) {  // the V^T page staged by wave wv - 2 in the lanes' load order
        lds_barrier();
        const uint4 *src = (const uint4 *)(s_vstage + wv * kStage);
#pragma unroll
        for (int nu = 0; nu < 8; ++nu)
#pragma unroll
          for (int kap = 0; kap < 2; ++kap) vv[nu][kap] = src[(nu * 2 + kap) * 64 + lane];
      }
#pragma unroll
      for (int nu = 0; nu < 8; ++nu) {
#pragma unroll
        for (int kap = 0; kap < 2; ++kap) {
          const uint4 v4 = vv[nu][kap];
          u32x4 w = u32x4{v4.x, v4.y, v4.z, v4.w};
          if (partial) w &= keepw[kap];
          oacc[nu] = VTr::mfma(pa2[kap], VTr::operand(w), oacc[nu]);
        }
      }
    } else if constexpr (SPEC) {
      // the V tile staged in fp16 by wave wv - 2, visible after this barrier (which the other waves
      // reach after staging, or after an empty chunk)
      lds_barrier();
      const uint8_t *st = s_vstage + wv * kStage;
#pragma unroll
      for (int nu = 0; nu < 8; ++nu)
#pragma unroll
        for (int kap = 0; kap < 2; ++kap)
          oacc[nu] = VTr::mfma(pa2[kap], VTraits<kVF16>::operand(vt_operand_lds(st, kVRow, nu, kap, kc, n)), oacc[nu]);
    } else {
    // stage the V tile [64 tokens][128] through LDS (rows past the sequence end were loaded as
    // zeros): whole in the register-holding build (one workgroup per CU anyway), one half of the
    // columns at a time in the RELOAD build, so that two workgroups fit in a CU's LDS
    constexpr int kHalves = RELOAD ? 2 : 1;
    constexpr int kPitch = RELOAD ? kVRowHalf : kVRow;
    constexpr int kPieces = 16 / kHalves;  // 16-byte column pieces of a row staged per pass
    uint8_t *st = s_vstage + wv * kPage * kPitch;
#pragma unroll
    for (int hf = 0; hf < kHalves; ++hf) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int idx = r * 64 + lane;
        const int tk = idx >> 4, vc = idx & 15;
        if (kHalves == 1 || (vc >> 3) == hf) {
          const uint4 v4 = vv[r >> 1][r & 1];
          uint2 *d = (uint2 *)(st + tk * kPitch + 16 * (vc % kPieces));  // rows are 8-byte aligned
          d[0] = make_uint2(v4.x, v4.y);
          d[1] = make_uint2(v4.z, v4.w);
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int nl = 0; nl < 8 / kHalves; ++nl) {
        const int nu = (8 / kHalves) * hf + nl;
#pragma unroll
        for (int kap = 0; kap < 2; ++kap)
          oacc[nu] = VTr::mfma(pa2[kap], VTr::operand(vt_operand_lds(st, kPitch, nl, kap, kc, n)), oacc[nu]);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    }
    FFA_STAMP(9);
    if (lane < 16) {
#pragma unroll
      for (int uu = 0; uu < 4; ++uu)
#pragma unroll
        for (int nu = 0; nu < 8; ++nu) s_po[slot][uu][16 * nu + n] = oacc[nu][uu];
    }
    if (lane < 4) {
      s_pm[slot][lane] = row_ok ? mrow_max : -INFINITY;
      s_pl[slot][lane] = row_ok ? lsum : 0.f;
    }
  };
  auto empty_chunk = [&](int slot) {
    if (lane < 4) {
      s_pm[slot][lane] = -INFINITY;
      s_pl[slot][lane] = 0.f;
    }
  };
  if constexpr (SPEC) {
    // one chunk per wave of 2 and 3; waves 0 and 1 stage their V tiles.  Every wave reaches the V
    // barrier once (inside exact_chunk before P.V, or here).
    if (wv < 2) {
      if constexpr (LAYOUT == kPaged) {
        uint4 *dst = (uint4 *)(s_vstage + (wv + 2) * kStage);
#pragma unroll
        for (int nu = 0; nu < 8; ++nu)
#pragma unroll
          for (int kap = 0; kap < 2; ++kap) dst[(nu * 2 + kap) * 64 + lane] = svv[nu][kap];
      } else {
        stage_v_f16(svv, s_vstage + (wv + 2) * kStage);
      }
      empty_chunk(wch * kPPW);
      lds_barrier();
    } else if (nv[0] > 0 && bal[0] != 0) {
      exact_chunk(std::integral_constant<int, 0>());
    } else {
      empty_chunk(wch * kPPW);
      lds_barrier();
    }
    empty_chunk(wch * kPPW + 1);
  } else {
    if (nv[0] > 0 && bal[0] != 0) exact_chunk(std::integral_constant<int, 0>());
    else empty_chunk(wch * kPPW);
    if (nv[1] > 0 && bal[1] != 0) exact_chunk(std::integral_constant<int, 1>());
    else empty_chunk(wch * kPPW + 1);
  }

  FFA_STAMP(10);
  // ------------------------------------------------ phase 4: mask, threshold, workgroup partial
  __syncthreads();
  FFA_STAMP(11);
  if (un.quad == 0) {
    int8_t *mrow_ptr = p.mask + ((size_t)b * p.HKV + hkv) * p.ntbs;
    const int t = threadIdx.x;
    if (SBS <= kPage) {
      const int per = div_pow2(kPage, SBS);
      if (t < kChunksPerWG * per && slot_owned(div_pow2(t, per))) {
        const int slot = div_pow2(t, per), k = t & (per - 1);
        const uint64_t bl = ((uint64_t)s_bal[slot][1] << 32) | s_bal[slot][0];
        const int jb = slot_chunk(slot) * per + k;
        const bool kk = SBS == 16   ? ((bl >> (16 * k)) & 0xffffull) != 0
                        : SBS == 32 ? ((bl >> (32 * k)) & 0xffffffffull) != 0
                                    : bl != 0;
        if (jb < p.ntbs) mrow_ptr[jb] = (jb < NTBS_b && kk) ? 1 : 0;
      }
    } else if (t < kChunksPerWG && (((cw + t) * kPage) & (SBS - 1)) == 0) {
      const int jb = div_pow2((cw + t) * kPage, SBS);
      const bool kk = (s_bal[t][0] | s_bal[t][1]) != 0;
      if (jb < p.ntbs) mrow_ptr[jb] = (jb < NTBS_b && kk) ? 1 : 0;
    }
  }
  if (p.pass == 0 && p.th_out != nullptr && cg == 0 && threadIdx.x < un.Gu)
    p.th_out[(size_t)b * p.HQ + un.row0 + threadIdx.x] = th;  // (pass 2: written by pass 1)
  {
    const int i = wv;
    const int c2 = 2 * lane;
    if (i < un.Gu) {
      // Every slot's m, l and o columns in one batch of LDS reads, then selects (reads issued slot by
      // slot behind branches on l were dependent LDS round trips at the end of every workgroup).  A
      // slot without a kept chunk has l = 0 (empty_chunk); its o was never written and is selected
      // away, not weighted by 0.
      float pm[kChunksPerWG], pl[kChunksPerWG];
      float2 po[kChunksPerWG];
#pragma unroll
      for (int ps = 0; ps < kChunksPerWG; ++ps) {
        pm[ps] = s_pm[ps][i];
        pl[ps] = s_pl[ps][i];
        po[ps] = *reinterpret_cast<const float2 *>(&s_po[ps][i][c2]);
      }
      float M = -INFINITY;
#pragma unroll
      for (int ps = 0; ps < kChunksPerWG; ++ps) M = pl[ps] > 0.f ? fmaxf(M, pm[ps]) : M;
      float A = 0.f, ox = 0.f, oy = 0.f;
#pragma unroll
      for (int ps = 0; ps < kChunksPerWG; ++ps) {
        const bool use = pl[ps] > 0.f;
        const float wgt = exp2_hw(use ? pm[ps] - M : -INFINITY);
        A = use ? __builtin_fmaf(pl[ps], wgt, A) : A;
        ox = use ? __builtin_fmaf(po[ps].x, wgt, ox) : ox;
        oy = use ? __builtin_fmaf(po[ps].y, wgt, oy) : oy;
      }
      const size_t row = (size_t)b * p.HQ + un.row0 + i;
      if (lane == 0) {
        p.m_buf[row * p.nparts + cg] = A > 0.f ? M : -INFINITY;
        p.l_buf[row * p.nparts + cg] = A;
      }
      if (A > 0.f) *(float2 *)(p.o_buf + (row * p.nparts + cg) * 128 + c2) = make_float2(ox, oy);
    }
  }
#ifdef FFA_TIMELINE
  FFA_STAMP(12);
  if (g_timeline_k != nullptr && lane == 0) {
    st_[13] = (unsigned long long)n_exact_;
    st_[14] = 0;
    st_[15] = ((unsigned long long)__builtin_amdgcn_s_getreg((31 << 11) | 20) << 32) |
              (unsigned long long)__builtin_amdgcn_s_getreg((31 << 11) | 4);
    const size_t wid = (((size_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * 4 + wv;
#pragma unroll
    for (int i = 0; i < 16; ++i) g_timeline_k[wid * 16 + i] = st_[i];
  }
#endif
}

}  // namespace ffa

// --------------------------------------------------------------------------
// C ABI
// --------------------------------------------------------------------------
template <int L, int F, int S, int R, int V>
static hipError_t kfmt_launch(const ffa::DecodeParams &p, dim3 grid, hipStream_t st) {
  // the builds that place the KV head fastest (grid_pos) take the grid (unit, span, sequence)
  const dim3 gsw(grid.y, grid.x, grid.z);
  if constexpr (L == ffa::kPaged) {
    // the runtime-span build for small grids and for every span shorter than 8 chunks (the last
    // halving of a small grid's span can take it past the CU count); the large-batch build's span
    // is the constant 8
    const int cus = ffa::device_cus();
    const bool small = cus > 0 && grid.x * grid.y * grid.z <= (unsigned)cus;
    if (small && p.span == ffa::kMinSpan)  // the role split of two-chunk spans
      hipLaunchKernelGGL((ffa::kfmt_decode_kernel<L, F, S, R, V, false, true>), gsw, dim3(256), 0, st, p);
    else if (small || p.span < ffa::kChunksPerWG)
      hipLaunchKernelGGL((ffa::kfmt_decode_kernel<L, F, S, R, V, false, false>), gsw, dim3(256), 0, st, p);
    else
      hipLaunchKernelGGL((ffa::kfmt_decode_kernel<L, F, S, R, V, true, false>), grid, dim3(256), 0, st, p);
  } else {
    constexpr bool k4 = F == ffa::kFP4 || F == ffa::kNF4;
    const dim3 g = k4 ? grid : gsw;  // the contiguous 8-bit formats place the KV head fastest
    const int cus = ffa::device_cus();
    if (cus > 0 && grid.x * grid.y * grid.z > (unsigned)cus)
      hipLaunchKernelGGL((ffa::kfmt_decode_kernel<L, F, S, R, V, true, false>), g, dim3(256), 0, st, p);
    else if (p.span == ffa::kMinSpan)
      hipLaunchKernelGGL((ffa::kfmt_decode_kernel<L, F, S, R, V, false, true>), g, dim3(256), 0, st, p);
    else
      hipLaunchKernelGGL((ffa::kfmt_decode_kernel<L, F, S, R, V, false, false>), g, dim3(256), 0, st, p);
  }
  return hipGetLastError();
}

template <int L, int F, int S>
static hipError_t kfmt_dispatch_rv(const ffa::DecodeParams &p, int res, int vdt, dim3 grid, hipStream_t st) {
  const int r = res == FFA_DT_FP8_E4M3 ? ffa::kResE4M3 : (res == FFA_DT_FP8_E5M2 ? ffa::kResE5M2 : ffa::kResNone);
  const int v = vdt == FFA_DT_BF16 ? ffa::kVBF16 : ffa::kVF16;
#define FFA_CASE(RR, VV) \
  if (r == RR && v == VV) return kfmt_launch<L, F, S, RR, VV>(p, grid, st);
  FFA_CASE(ffa::kResE4M3, ffa::kVBF16)
  FFA_CASE(ffa::kResE4M3, ffa::kVF16)
  FFA_CASE(ffa::kResE5M2, ffa::kVBF16)
  FFA_CASE(ffa::kResE5M2, ffa::kVF16)
  FFA_CASE(ffa::kResNone, ffa::kVBF16)
  FFA_CASE(ffa::kResNone, ffa::kVF16)
#undef FFA_CASE
  return hipErrorInvalidValue;
}

// one launch of the decoder instance of a K format and scale granularity (hipErrorInvalidValue
// for a combination without an instance)
static hipError_t kfmt_launch_format(const ffa::DecodeParams &p, int fmt, int sk, int res, int vdt, dim3 grid,
                                     hipStream_t st) {
  constexpr int C = ffa::kContig, PG = ffa::kPaged;
  if (fmt == FFA_KFMT_FP8_E4M3 && sk == FFA_KSCALE_NONE)
    return kfmt_dispatch_rv<C, ffa::kF8E4M3, ffa::kSclNone>(p, res, vdt, grid, st);
  if (fmt == FFA_KFMT_FP8_E4M3 && sk == FFA_KSCALE_TOKEN)
    return kfmt_dispatch_rv<C, ffa::kF8E4M3, ffa::kSclToken>(p, res, vdt, grid, st);
  if (fmt == FFA_KFMT_FP8_E5M2 && sk == FFA_KSCALE_NONE)
    return kfmt_dispatch_rv<C, ffa::kF8E5M2, ffa::kSclNone>(p, res, vdt, grid, st);
  if (fmt == FFA_KFMT_FP8_E5M2 && sk == FFA_KSCALE_TOKEN)
    return kfmt_dispatch_rv<C, ffa::kF8E5M2, ffa::kSclToken>(p, res, vdt, grid, st);
  if (fmt == FFA_KFMT_NVFP4 && sk == FFA_KSCALE_BLOCK)
    return kfmt_dispatch_rv<C, ffa::kFP4, ffa::kSclBlock>(p, res, vdt, grid, st);
  if (fmt == FFA_KFMT_NF4 && sk == FFA_KSCALE_CHANNEL)
    return kfmt_dispatch_rv<C, ffa::kNF4, ffa::kSclChannel>(p, res, vdt, grid, st);
  if (fmt == FFA_KFMT_NVFP4 && sk == FFA_KSCALE_G16)
    return kfmt_dispatch_rv<PG, ffa::kFP4, ffa::kSclG16>(p, res, vdt, grid, st);
  if (fmt == FFA_KFMT_NF4 && sk == FFA_KSCALE_G64)
    return kfmt_dispatch_rv<PG, ffa::kNF4, ffa::kSclG64>(p, res, vdt, grid, st);
  return hipErrorInvalidValue;
}

extern "C" int ffa_kfmt_decode(const ffa_kfmt_decode_args *a, void *stream) {
  if (!a) return ffa_set_error_internal(FFA_E_INVALID, "null args");
  ffa::DecodeParams p = {};
  const int rc0 = ffa_decode_shape_check(a->B, a->T, a->HQ, a->HKV, a->BS, a->SBS, a->piece_max, a->npieces,
                                         a->threshold_in, a->threshold_out, &p);
  if (rc0 != FFA_OK) return rc0;
  const int G = a->HQ / a->HKV;
  if (!(a->q_dtype >= FFA_DT_F16 && a->q_dtype <= FFA_DT_F32)) return ffa_set_error_internal(FFA_E_INVALID, "q dtype");
  if (!(a->out_dtype >= FFA_DT_F16 && a->out_dtype <= FFA_DT_F32))
    return ffa_set_error_internal(FFA_E_INVALID, "out dtype");
  if (!(a->v_dtype == FFA_DT_F16 || a->v_dtype == FFA_DT_BF16)) return ffa_set_error_internal(FFA_E_INVALID, "v dtype");
  if (!(a->res_dtype == FFA_DT_FP8_E4M3 || a->res_dtype == FFA_DT_FP8_E5M2 || a->res_dtype == FFA_DT_NONE))
    return ffa_set_error_internal(FFA_E_INVALID, "residual dtype");
  if (a->res_dtype != FFA_DT_NONE && !a->k_residual) return ffa_set_error_internal(FFA_E_INVALID, "residual pointer is null");
  const bool scaled = a->scale_kind != FFA_KSCALE_NONE;
  if (scaled && !(a->scale_dtype >= FFA_DT_F16 && a->scale_dtype <= FFA_DT_F32))
    return ffa_set_error_internal(FFA_E_INVALID, "scale dtype");
  if (scaled && !a->k_scale) return ffa_set_error_internal(FFA_E_INVALID, "scale pointer is null");
  const int need = ffa_decode_slots(a->T, a->BS, ffa::kChunksPerWG);
  if (a->nparts < need) return ffa_set_error_internal(FFA_E_INVALID, "scratch holds too few partial slots");
  const int ntbs = ((a->T + a->BS - 1) / a->BS) * (a->BS / a->SBS);
  if (a->ntbs < ntbs) return ffa_set_error_internal(FFA_E_INVALID, "mask holds too few blocks");
  const bool paged = a->layout == FFA_LAYOUT_PAGED;
  if (!paged && a->layout != FFA_LAYOUT_CONTIG) return ffa_set_error_internal(FFA_E_INVALID, "layout");
  if (paged && !a->block_table) return ffa_set_error_internal(FFA_E_INVALID, "paged layout needs a block table");
  if (paged && a->num_pages <= 0)
    return ffa_set_error_internal(FFA_E_INVALID, "paged layout needs num_pages > 0 (pages in each pool)");
  if (paged && (long)a->bt_stride * ffa::kPage < a->T)
    return ffa_set_error_internal(FFA_E_INVALID, "block table has fewer than ceil(T/64) columns");
  if (paged != (a->scale_kind == FFA_KSCALE_G16 || a->scale_kind == FFA_KSCALE_G64))
    return ffa_set_error_internal(FFA_E_UNSUPPORTED,
                                  "the paged layout takes the per-token group scales (G16 / G64) and only it");

  p.q = a->q;
  p.kq = a->k;
  p.ks = a->k_scale;
  p.kr = a->k_residual;
  p.v = a->v;
  p.bt = a->block_table;
  p.bt_stride = a->bt_stride;
  p.num_pages = paged ? a->num_pages : 0;
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
  // the caller's scratch.  One pass with prune blocks of at most one chunk only (the longer blocks'
  // maxima span two chunks of a wave).
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

  hipStream_t st = (hipStream_t)stream;
  const dim3 grid(p.nwg, a->HKV * p.nq, a->B);
  if ((long long)grid.x * grid.y * grid.z > 0x7fffffffLL)  // the kernels number workgroups in 32 bits
    return ffa_set_error_internal(FFA_E_UNSUPPORTED, "decode grid of more than 2^31 - 1 workgroups");
  if (grid.x > 65535)  // the builds that place the KV head fastest launch the spans as grid y
    return ffa_set_error_internal(FFA_E_UNSUPPORTED, "more than 65535 workgroup spans per sequence");
  // one pass (pass 0), or (G > 4, SBS > 512) the maxima pass 1 and then the deciding pass 2
  const bool two = p.pmax != nullptr;
  for (int pass = two ? 1 : 0; pass <= (two ? 2 : 0); ++pass) {
    ffa::DecodeParams pp = p;
    pp.pass = pass;
    const hipError_t e = kfmt_launch_format(pp, a->k_format, a->scale_kind, a->res_dtype, a->v_dtype, grid, st);
    if (e == hipErrorInvalidValue)
      return ffa_set_error_internal(FFA_E_UNSUPPORTED, "unsupported K format / scale granularity combination");
    if (e != hipSuccess) return ffa_set_error_internal(FFA_E_LAUNCH, hipGetErrorString(e));
  }
  const hipError_t e = ffa::launch_merge(p, st);
  if (e != hipSuccess) return ffa_set_error_internal(FFA_E_LAUNCH, hipGetErrorString(e));
  return FFA_OK;
}

#ifdef FFA_TIMELINE
// Timeline build only: the buffer (16 words per wave of a stage-1 grid) the other-format decode writes to.
extern "C" int ffa_debug_set_timeline_kfmt(void *ptr) {
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_timeline_k), &ptr, sizeof(ptr));
}
#endif
