// 2-bit K quantizers and the fused K-projection + RoPE producers for gfx950.
//
//  * per-channel quantizer, bit-exact with the reference's torch op sequence
//    (ffa-q2fp8/run_attn_bench_q2.py:78-105): every op that torch runs in the
//    K dtype tau is rounded to tau here; no FMA contraction (the file is built
//    with `fp contract(off)`); divisions are IEEE round-to-nearest.
//  * fused K-proj + RoPE (ffa-q2fp8/fused_kproj_rope_q2fp8.py:103-399, which
//    runs the GEMM twice): one MFMA GEMM pass writes the rotated K, then the
//    per-channel quantizer runs on it.
//  * fused K-proj + RoPE + g32 quantize + append into the paged cache
//    (the decode-time producer): per-token groups make the append local, so GEMM,
//    RoPE, quantization and the page writes are one kernel.
#include "decode_common.h"
#include "ffa_common.h"
#include "ffa_mi355x.h"

#include <stdio.h>

#pragma clang fp contract(off)

namespace ffa {

// ---------------------------------------------------------------------------
// per-channel quantizer
// ---------------------------------------------------------------------------
constexpr int kQTok = 256;  // tokens per min/max split

__global__ __launch_bounds__(256) void q2_minmax_kernel(const void *k, int kdt, int T, int C, int nsplit,
                                                         float *minmax) {
  // grid (nsplit, B, ceil(C/256)); thread = column
  const int split = blockIdx.x, b = blockIdx.y;
  const int c = blockIdx.z * 256 + threadIdx.x;
  if (c >= C) return;
  const int tper = (T + nsplit - 1) / nsplit;
  const int ta = split * tper, tb = min(T, ta + tper);
  float mn = INFINITY, mx = -INFINITY;
  for (int t = ta; t < tb; ++t) {
    const float v = load_any(k, ((size_t)b * T + t) * C + c, kdt);
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
  const int B = gridDim.y;
  minmax[((size_t)b * nsplit + split) * C + c] = mn;
  minmax[((size_t)(B + b) * nsplit + split) * C + c] = mx;
}

__global__ __launch_bounds__(256) void q2_scale_kernel(const float *minmax, int B, int nsplit, int C, int kdt,
                                                        void *scale, void *zero) {
  const int b = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  float mn = INFINITY, mx = -INFINITY;
  for (int s = 0; s < nsplit; ++s) {
    mn = fminf(mn, minmax[((size_t)b * nsplit + s) * C + c]);
    mx = fmaxf(mx, minmax[((size_t)(B + b) * nsplit + s) * C + c]);
  }
  // scale = tau(tau(tau(max - min).clamp_min(1e-6)) / 3.0)   (run_attn_bench_q2.py:82)
  const float diff = round_to(mx - mn, kdt);
  const float cl = round_to(fmaxf(diff, 1e-6f), kdt);
  const float sc = round_to(__fdiv_rn(cl, 3.0f), kdt);
  store_any(scale, (size_t)b * C + c, kdt, sc);
  store_any(zero, (size_t)b * C + c, kdt, mn);
}

// one thread per (token, packed byte) of a [B, T, HKV, D] tensor
// One packed byte (channels 4 byte .. 4 byte + 3) of one K row under per-channel scale / zero
// (tau values at sz_off + d): codes and residuals with the reference's per-element ops.  The
// full quantizer runs it with K's own scale / zero, the per-channel append with the cache's.
__device__ __forceinline__ void quant_channel_byte(const void *k, int kdt, size_t k_row, int D, int byte,
                                                   const void *scale, const void *zero, size_t sz_off,
                                                   uint8_t *kq_byte, uint8_t *res_row, int res_e4m3) {
  uint32_t packed = 0;
  for (int e = 0; e < 4; ++e) {
    const int d = 4 * byte + e;
    if (d >= D) break;
    const float kv = load_any(k, k_row * D + d, kdt);
    const float sc = load_any(scale, sz_off + d, kdt);
    const float zr = load_any(zero, sz_off + d, kdt);
    const float xs = round_to(kv - zr, kdt);               // (k - zero) in tau
    const float xd = round_to(__fdiv_rn(xs, sc), kdt);     // / scale in tau
    const float cq = fminf(fmaxf(__builtin_rintf(xd), 0.f), 3.f);  // round (RNE), clamp(0,3)
    const float deq = (cq * sc) + zr;                      // two fp32 roundings
    res_row[d] = (uint8_t)f32_to_fp8(kv - deq, res_e4m3);
    packed |= ((uint32_t)cq) << (2 * e);
  }
  *kq_byte = (uint8_t)packed;
}

__global__ __launch_bounds__(256) void q2_quant_channel_kernel(const void *k, int kdt, int B, int T, int HKV,
                                                                int D, const void *scale, const void *zero,
                                                                uint8_t *kq, uint8_t *res, int res_e4m3) {
  const int DP = (D + 3) / 4;
  const size_t total = (size_t)B * T * HKV * DP;
  const size_t id = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= total) return;
  const int byte = (int)(id % DP);
  const size_t row = id / DP;  // (b, t, hkv)
  const int hkv = (int)(row % HKV);
  const int b = (int)(row / ((size_t)HKV * T));
  quant_channel_byte(k, kdt, row, D, byte, scale, zero, ((size_t)b * HKV + hkv) * D, kq + row * DP + byte,
                     res + row * D, res_e4m3);
}

// Reference-layout append: token n of sequence b (k_new [B, Tn, HKV, D]) is quantized with the
// cache's per-channel scale / zero [B, HKV, D] and written at position pos[b] + n of
// k_q [B, T_cap, HKV, ceil(D/4)] and residual [B, T_cap, HKV, D]; positions outside
// [0, T_cap) are not written.
__global__ __launch_bounds__(256) void q2_append_channel_kernel(const void *k_new, int kdt, int B, int Tn, int HKV,
                                                                 int D, const int32_t *pos, int T_cap,
                                                                 const void *scale, const void *zero, uint8_t *kq,
                                                                 uint8_t *res, int res_e4m3) {
  const int DP = (D + 3) / 4;
  const size_t total = (size_t)B * Tn * HKV * DP;
  const size_t id = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= total) return;
  const int byte = (int)(id % DP);
  const size_t row = id / DP;  // (b, n, hkv) of k_new
  const int hkv = (int)(row % HKV);
  const int n = (int)((row / HKV) % Tn);
  const int b = (int)(row / ((size_t)HKV * Tn));
  const int t = pos[b] + n;
  if (t < 0 || t >= T_cap) return;
  const size_t dst = ((size_t)b * T_cap + t) * HKV + hkv;
  quant_channel_byte(k_new, kdt, row, D, byte, scale, zero, ((size_t)b * HKV + hkv) * D, kq + dst * DP + byte,
                     res + dst * D, res_e4m3);
}

// K projection GEMM tile: 16 tokens x 32 output channels per 512-thread workgroup.  The 32-wide k
// steps are dealt round-robin to the 8 waves (wave w takes steps w, w + 8, ...), so even a handful of
// tokens keeps 8 waves per tile streaming W; each wave accumulates its steps with MFMA 16x16x32 into
// two 16x16 tiles, and the 8 partial tiles are summed in wave order through LDS, so the result does
// not depend on timing.  Returns the fp32 product for row threadIdx.x >> 5 (token m0 + row) and
// column threadIdx.x & 31 (output channel n0 + column).  w is [N, H] (out, in), rows of H elements.
// ---------------------------------------------------------------------------
constexpr int kKpWaves = 8;

template <int HDT>
__device__ __forceinline__ f32x4 kp_mfma(uint4 a, uint4 b, f32x4 c) {
  const u32x4 av = {a.x, a.y, a.z, a.w}, bv = {b.x, b.y, b.z, b.w};
  if constexpr (HDT == FFA_DT_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av), __builtin_bit_cast(f16x8, bv), c, 0,
                                                  0, 0);
}

// Operand loads read 4 lanes per row (lane L: row L >> 2, 16-byte piece L & 3 of the step's
// 64 bytes), so a 16-lane quarter of the wave touches 4 rows; the MFMA layout (lane L: row
// L & 15, piece L >> 4) puts 16 rows in each quarter, which the memory pipeline serves about
// twice as slowly.  A cross-lane permute then moves each piece to its MFMA lane.
__device__ __forceinline__ uint4 kp_to_mfma_layout(uint4 v) {
  const int lane = threadIdx.x & 63;
  const int src = (4 * (lane & 15) + (lane >> 4)) << 2;  // byte address of the source lane
  return make_uint4((uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)v.x),
                    (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)v.y),
                    (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)v.z),
                    (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)v.w));
}

// NB k steps of one wave: all 3 * NB loads are issued before the first MFMA waits.
template <int NB, int HDT>
__device__ __forceinline__ void kp_steps(const uint16_t *hp, const uint16_t *wp0, const uint16_t *wp1, int wv, int i,
                                         f32x4 &acc0, f32x4 &acc1) {
  uint4 a[NB], b0[NB], b1[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int k0 = 32 * (wv + kKpWaves * (i + j));
    a[j] = *(const uint4 *)(hp + k0);
    b0[j] = *(const uint4 *)(wp0 + k0);
    b1[j] = *(const uint4 *)(wp1 + k0);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const uint4 aj = kp_to_mfma_layout(a[j]);
    acc0 = kp_mfma<HDT>(aj, kp_to_mfma_layout(b0[j]), acc0);
    acc1 = kp_mfma<HDT>(aj, kp_to_mfma_layout(b1[j]), acc1);
  }
}

template <int HDT>
__device__ __forceinline__ float kproj_tile32(const void *h, const void *w, int M, int H, int m0, int n0,
                                              float (*red)[16][33]) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  // load layout: lane L reads row L >> 2, elements 8 (L & 3) .. + 8 of each 32-wide k step
  const int mrow = min(m0 + (lane >> 2), M - 1);
  const int kq = 8 * (lane & 3);
  const uint16_t *hp = (const uint16_t *)h + (size_t)mrow * H + kq;
  const uint16_t *wp0 = (const uint16_t *)w + (size_t)(n0 + (lane >> 2)) * H + kq;
  const uint16_t *wp1 = wp0 + (size_t)16 * H;
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  const int nsteps = H / 32;
  const int mine = (nsteps - wv + kKpWaves - 1) / kKpWaves;  // steps of this wave (16 at H = 4096)
  int i = 0;
  for (; i + 16 <= mine; i += 16) kp_steps<16, HDT>(hp, wp0, wp1, wv, i, acc0, acc1);
  for (; i + 4 <= mine; i += 4) kp_steps<4, HDT>(hp, wp0, wp1, wv, i, acc0, acc1);
  for (; i < mine; ++i) kp_steps<1, HDT>(hp, wp0, wp1, wv, i, acc0, acc1);
  // MFMA 16x16 result: acc[u] is row 4 * (lane >> 4) + u, column lane & 15
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    red[wv][4 * (lane >> 4) + u][lane & 15] = acc0[u];
    red[wv][4 * (lane >> 4) + u][16 + (lane & 15)] = acc1[u];
  }
  __syncthreads();
  const int row = threadIdx.x >> 5, col = threadIdx.x & 31;
  float sum = red[0][row][col];
#pragma unroll
  for (int x = 1; x < kKpWaves; ++x) sum += red[x][row][col];
  return sum;
}

// blockIdx.x -> (column tile ct, token tile mt).  Workgroups go to the 8 XCDs round-robin; when the
// column tiles split evenly over the XCDs, all token tiles of one column tile run on one XCD and share
// its L2, so each slice of W is read from HBM once.
__device__ __forceinline__ void kproj_tile_of(int bid, int nct, int &ct, int &mt) {
  if ((nct & 7) == 0) {
    const int per = nct >> 3, j = bid >> 3;
    ct = (bid & 7) + 8 * (j % per);
    mt = j / per;
  } else {
    ct = bid % nct;
    mt = bid / nct;
  }
}

// g32 quantization of one (token, KV head, group) held by the 32 lanes of a half wave (lane e of the
// half holds channel 32 g + e), and its page writes:
//   zero = fp16(min), scale = fp16(max(max - zero, 1e-6) / 3), c = clamp(rne((k - zero)/scale), 0, 3),
//   residual = fp8(k - (c*scale + zero)) with two fp32 roundings;
// min / max by shuffles, 2-bit codes OR-reduced over 16 lanes, residual bytes stored by each lane.
// All 64 lanes must call it; `store` masks the writes.
__device__ __forceinline__ void g32_quantize_lanes(float x, bool store, int page, int slot, int hkv, int HKV, int g,
                                                   uint8_t *kq_pages, uint16_t *s_pages, uint16_t *z_pages,
                                                   uint8_t *r_pages, int res_e4m3) {
  constexpr int D = 128;
  const int e = threadIdx.x & 31;
  float mn = x, mx = x;
#pragma unroll
  for (int m = 1; m < 32; m <<= 1) {
    mn = fminf(mn, __shfl_xor(mn, m));
    mx = fmaxf(mx, __shfl_xor(mx, m));
  }
  const float zr = (float)(_Float16)mn;
  const float sc = (float)(_Float16)__fdiv_rn(fmaxf(mx - zr, 1e-6f), 3.0f);
  const float cq = fminf(fmaxf(__builtin_rintf(__fdiv_rn(x - zr, sc)), 0.f), 3.f);
  const float deq = (cq * sc) + zr;
  const uint32_t rb = f32_to_fp8(x - deq, res_e4m3);
  uint32_t word = ((uint32_t)cq) << (2 * (e & 15));
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) word |= (uint32_t)__shfl_xor((int)word, m);
  if (!store) return;
  const size_t blk = (size_t)page * HKV + hkv;
  r_pages[blk * (64 * D) + res_off(slot, 32 * g + e)] = (uint8_t)rb;
  if ((e & 15) == 0) *(uint32_t *)(kq_pages + blk * (4 * 64 * 8) + codes_off(g, slot) + 4 * (e >> 4)) = word;
  if (e == 0) {
    const int ss = 16 * (slot >> 4) + 4 * (slot & 3) + ((slot >> 2) & 3);  // tile-major scale slot
    const size_t so = blk * (4 * 64) + gscale_off(g, ss);
    s_pages[so] = (uint16_t)f32_to_f16_bits(sc);
    z_pages[so] = (uint16_t)f32_to_f16_bits(zr);
  }
}

// RoPE of one element given its pair partner (fused_kproj_rope_q2fp8.py:26-37):
//   out[2i]   = x[2i]  *cos[2i]   + (-x[2i+1])*sin[2i]
//   out[2i+1] = x[2i+1]*cos[2i+1] +   x[2i]   *sin[2i+1]
// each product and the sum are rounded to the promoted dtype `odt`.
__device__ __forceinline__ float rope_one(float x, float partner, bool odd, float c, float s, int odt) {
  const float t1 = round_to(x * c, odt);
  const float rot = odd ? partner : -partner;
  const float t2 = round_to(rot * s, odt);
  return round_to(t1 + t2, odt);
}

// Rotated K of the reference producer -> k_scratch [M, N] in dtype odt.  One 512-thread workgroup per
// (16 tokens, 32 output channels); grid = (N / 32) * ceil(M / 16).
template <int HDT>
__global__ __launch_bounds__(512) void kproj_rope_kernel(const void *h, const void *w, const void *bias, const void *cos,
                                                         const void *sin, int csdt, int M, int T, int H, int N, int D,
                                                         void *kout, int odt) {
  __shared__ float red[kKpWaves][16][33];
  int ct, mt;
  kproj_tile_of(blockIdx.x, N / 32, ct, mt);
  const int m0 = mt * 16, n0 = ct * 32;
  const float acc = kproj_tile32<HDT>(h, w, M, H, m0, n0, red);
  const int m = m0 + (threadIdx.x >> 5), col = n0 + (threadIdx.x & 31);
  const float bv = bias ? load_any(bias, col, HDT) : 0.f;
  const float x = round_to(acc + bv, HDT);  // F.linear output in the h dtype
  const float partner = __shfl_xor(x, 1);   // channel col ^ 1 (D is even, so the RoPE pair)
  if (m < M) {
    const int d = col % D, t = m % T;
    const float c = load_any(cos, (size_t)t * D + d, csdt);
    const float s = load_any(sin, (size_t)t * D + d, csdt);
    store_any(kout, (size_t)m * N + col, odt, rope_one(x, partner, (d & 1) != 0, c, s, odt));
  }
}

// K-proj + RoPE (fp32 cos/sin rows per token) + g32 quantize + paged append; the 32 channels of a
// workgroup are one g32 group of one KV head, so quantization needs no other workgroup.
template <int HDT>
__global__ __launch_bounds__(512) void kproj_append_kernel(const void *h, const void *w, const void *bias,
                                                           const float *cos, const float *sin, int M, int Tn, int H,
                                                           int HKV, const int32_t *pos, const int32_t *bt, int bt_stride,
                                                           int num_pages, uint8_t *kq_pages, uint16_t *s_pages,
                                                           uint16_t *z_pages, uint8_t *r_pages, int res_e4m3,
                                                           const void *v_new, void *v_pages) {
  constexpr int D = 128;
  __shared__ float red[kKpWaves][16][33];
  int ct, mt;
  kproj_tile_of(blockIdx.x, HKV * (D / 32), ct, mt);
  const int m0 = mt * 16, n0 = ct * 32;
  const int hkv = n0 / D, g = (n0 % D) / 32;
  const int e = threadIdx.x & 31, d = 32 * g + e;
  const int m = m0 + (threadIdx.x >> 5), mc = min(m, M - 1);
  // the epilogue's inputs are fetched before the GEMM so their latency hides behind it
  const float bv = bias ? load_any(bias, n0 + e, HDT) : 0.f;
  const float cv = cos[(size_t)mc * D + d], sv = sin[(size_t)mc * D + d];
  const int b = mc / Tn, nn = mc % Tn;
  const int P = pos[b] + nn;
  const uint16_t vv = v_new != nullptr ? ((const uint16_t *)v_new)[((size_t)mc * HKV + hkv) * D + d] : 0;
  const float acc = kproj_tile32<HDT>(h, w, M, H, m0, n0, red);
  const float x = round_to(acc + bv, HDT);
  const float partner = __shfl_xor(x, 1);
  // fp32 cos / sin promote the rotation to fp32
  const float k = rope_one(x, partner, (d & 1) != 0, cv, sv, FFA_DT_F32);
  const int page = append_page(bt, bt_stride, num_pages, b, P);
  const int slot = P & 63;
  const bool wr = m < M && page >= 0;  // uniform over the 32 lanes of a token's group
  g32_quantize_lanes(k, wr, page, slot, hkv, HKV, g, kq_pages, s_pages, z_pages, r_pages, res_e4m3);
  if (v_new != nullptr && wr)  // V^T pages: this workgroup's 32 channels of each token
    ((uint16_t *)v_pages)[((size_t)page * HKV + hkv) * (D * 64) + vt_off(d, slot)] = vv;
}


// g32 quantize + append of given K rows (no projection): 128 threads per (token row, KV head),
// one channel each (coalesced loads; the quantization of a 32-channel group runs across the 32
// lanes of a half wave, g32_quantize_lanes).  k [B, Tn, HKV, 128] (dtype kdt).
__global__ __launch_bounds__(256) void q2_g32_append_kernel(const void *k, int kdt, int M, int Tn, int HKV,
                                                             const int32_t *pos, const int32_t *bt, int bt_stride,
                                                             int num_pages, uint8_t *kq_pages, uint16_t *s_pages,
                                                             uint16_t *z_pages, uint8_t *r_pages, int res_e4m3,
                                                             const void *v_new, void *v_pages) {
  constexpr int D = 128;
  const size_t rowid = (size_t)blockIdx.x * 2 + (threadIdx.x >> 7);  // (token row, head)
  if (rowid >= (size_t)M * HKV) return;  // whole waves (a row is two waves)
  const int c = threadIdx.x & 127, g = c >> 5;
  const int hkv = (int)(rowid % HKV);
  const int m = (int)(rowid / HKV);
  const int b = m / Tn, nn = m % Tn;
  const int P = pos[b] + nn;
  const int page = append_page(bt, bt_stride, num_pages, b, P);
  const int slot = P & 63;
  const float x = load_any(k, rowid * D + c, kdt);
  g32_quantize_lanes(x, page >= 0, page, slot, hkv, HKV, g, kq_pages, s_pages, z_pages, r_pages, res_e4m3);
  if (v_new != nullptr && page >= 0)
    ((uint16_t *)v_pages)[((size_t)page * HKV + hkv) * (D * 64) + vt_off(c, slot)] = ((const uint16_t *)v_new)[rowid * D + c];
}


// Paged g32 cache -> contiguous K and V (the exact-attention path of the HF integration, which the
// reference feeds with dequantized keys: ffa-fp8fp8/e2e/fp8fp8_cache.py:60-69, returned by update at
// :84-89).  One workgroup per (sequence, page of the sequence, KV head): K = c * s + z + r in fp32
// (c * s is exact, so the fma rounds once, as the sum does), then one rounding to the output dtype;
// V read from the V^T page through shared memory so that both outputs are written as rows.  Tokens at
// or past the sequence's length are written as zeros; block-table entries outside the pool read page 0.
__global__ __launch_bounds__(256) void q2_paged_dequant_kernel(const uint8_t *kq_pages, const uint16_t *s_pages,
                                                               const uint16_t *z_pages, const uint8_t *r_pages,
                                                               int res_e4m3, const uint16_t *v_pages, int vdt,
                                                               const int32_t *bt, int bt_stride, int num_pages,
                                                               const int32_t *seq_lens, int T, int HKV, void *k_out,
                                                               void *v_out, int odt) {
  constexpr int D = 128;
  const int j = blockIdx.x, hkv = blockIdx.y, b = blockIdx.z;
  const int Tb = seq_lens ? min(max(seq_lens[b], 0), T) : T;
  int page = bt[(size_t)b * bt_stride + j];
  page = (unsigned)page < (unsigned)num_pages ? page : 0;
  const size_t blk = (size_t)page * HKV + hkv;
  __shared__ uint16_t s_v[64][D + 2];
  // V^T: 1024 16-byte pieces (8 tokens of one column); piece P holds column 16 (P >> 7) + (P & 15),
  // tokens 16 ((P >> 4) & 3) + 8 ((P >> 6) & 1) + (0..7)
  const uint4 *vp = (const uint4 *)(v_pages + blk * (D * 64));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int P = threadIdx.x + 256 * i;
    const int c = 16 * (P >> 7) + (P & 15), t0 = 16 * ((P >> 4) & 3) + 8 * ((P >> 6) & 1);
    const uint4 w = vp[P];
    const uint32_t e[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      s_v[t0 + 2 * k][c] = (uint16_t)(e[k] & 0xffffu);
      s_v[t0 + 2 * k + 1][c] = (uint16_t)(e[k] >> 16);
    }
  }
  // K: thread (token t, group g) dequantizes 32 channels
  const int t = threadIdx.x >> 2, g = threadIdx.x & 3;
  const int tok = 64 * j + t;
  const bool valid = tok < Tb;
  const uint2 cw = *(const uint2 *)(kq_pages + blk * (4 * 64 * 8) + codes_off(g, t));
  const int ss = 16 * (t >> 4) + 4 * (t & 3) + ((t >> 2) & 3);  // tile-major scale slot, as appended
  const float sc = f16_bits_to_f32(s_pages[blk * (4 * 64) + gscale_off(g, ss)]);
  const float zr = f16_bits_to_f32(z_pages[blk * (4 * 64) + gscale_off(g, ss)]);
  const uint4 r0 = *(const uint4 *)(r_pages + blk * (64 * D) + res_off(t, 32 * g));
  const uint4 r1 = *(const uint4 *)(r_pages + blk * (64 * D) + res_off(t, 32 * g + 16));
  const uint32_t rw[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
  const uint32_t cwords[2] = {cw.x, cw.y};
  const size_t orow = ((size_t)b * T + tok) * HKV + hkv;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const f16x8 rv = res_e4m3 ? fp8x8_to_f16x8<kResE4M3>(rw[2 * a], rw[2 * a + 1])
                              : fp8x8_to_f16x8<kResE5M2>(rw[2 * a], rw[2 * a + 1]);  // exact
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int i = 8 * a + e;
      const uint32_t code = (cwords[i >> 4] >> (2 * (i & 15))) & 3u;
      const float k = __builtin_fmaf((float)code, sc, zr) + (float)rv[e];
      store_any(k_out, orow * D + 32 * g + i, odt, valid ? k : 0.f);
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const uint32_t bits = s_v[t][32 * g + i];
    const float x = vdt == FFA_DT_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
    store_any(v_out, orow * D + 32 * g + i, odt, valid ? x : 0.f);
  }
}
}  // namespace ffa

// ============================================================================
// C ABI
// ============================================================================
// errors of this translation unit are reported through the decode unit's buffer
extern "C" __attribute__((visibility("hidden"))) int ffa_set_error_internal(int code, const char *msg);

extern "C" int ffa_q2_quantize_nsplit(int T) {
  int s = (T + ffa::kQTok - 1) / ffa::kQTok;
  return s < 1 ? 1 : (s > 64 ? 64 : s);
}

static int launch_quant_channel(const void *k, int kdt, int B, int T, int HKV, int D, uint8_t *k_q, void *scale,
                                void *zero, uint8_t *residual, int res_dtype, float *minmax, hipStream_t st) {
  const int C = HKV * D;
  const int nsplit = ffa_q2_quantize_nsplit(T);
  hipLaunchKernelGGL(ffa::q2_minmax_kernel, dim3(nsplit, B, (C + 255) / 256), dim3(256), 0, st, k, kdt, T, C, nsplit,
                     minmax);
  hipLaunchKernelGGL(ffa::q2_scale_kernel, dim3((C + 255) / 256, B), dim3(256), 0, st, (const float *)minmax, B,
                     nsplit, C, kdt, scale, zero);
  const size_t total = (size_t)B * T * HKV * ((D + 3) / 4);
  hipLaunchKernelGGL(ffa::q2_quant_channel_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, k, kdt, B,
                     T, HKV, D, (const void *)scale, (const void *)zero, k_q, residual,
                     res_dtype == FFA_DT_FP8_E4M3 ? 1 : 0);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return ffa_set_error_internal(FFA_E_LAUNCH, hipGetErrorString(e));
  return FFA_OK;
}

extern "C" int ffa_q2_append_channel(const void *k_new, int k_dtype, int B, int Tn, int HKV, int D, const int32_t *pos,
                                     int T_cap, const void *scale, const void *zero, uint8_t *k_q, uint8_t *residual,
                                     int res_dtype, void *stream) {
  if (B <= 0 || Tn <= 0 || HKV <= 0 || D <= 0 || T_cap <= 0) return ffa_set_error_internal(FFA_E_INVALID, "bad dims");
  if (!(k_dtype >= FFA_DT_F16 && k_dtype <= FFA_DT_F32)) return ffa_set_error_internal(FFA_E_INVALID, "k dtype");
  if (!(res_dtype == FFA_DT_FP8_E4M3 || res_dtype == FFA_DT_FP8_E5M2))
    return ffa_set_error_internal(FFA_E_INVALID, "residual dtype");
  if (!k_new || !pos || !scale || !zero || !k_q || !residual) return ffa_set_error_internal(FFA_E_INVALID, "null pointer");
  const size_t total = (size_t)B * Tn * HKV * ((D + 3) / 4);
  hipLaunchKernelGGL(ffa::q2_append_channel_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, k_new, k_dtype, B, Tn, HKV, D, pos, T_cap, scale, zero, k_q, residual,
                     res_dtype == FFA_DT_FP8_E4M3 ? 1 : 0);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FFA_OK : ffa_set_error_internal(FFA_E_LAUNCH, hipGetErrorString(e));
}

extern "C" int ffa_q2_quantize_channel(const void *k, int k_dtype, int B, int T, int HKV, int D, uint8_t *k_q,
                                       void *scale, void *zero, uint8_t *residual, int res_dtype, float *minmax,
                                       void *stream) {
  if (B <= 0 || T <= 0 || HKV <= 0 || D <= 0) return ffa_set_error_internal(FFA_E_INVALID, "bad dims");
  if (!(k_dtype >= FFA_DT_F16 && k_dtype <= FFA_DT_F32)) return ffa_set_error_internal(FFA_E_INVALID, "k dtype");
  if (!(res_dtype == FFA_DT_FP8_E4M3 || res_dtype == FFA_DT_FP8_E5M2))
    return ffa_set_error_internal(FFA_E_INVALID, "residual dtype must be fp8");
  return launch_quant_channel(k, k_dtype, B, T, HKV, D, k_q, scale, zero, residual, res_dtype, minmax,
                              (hipStream_t)stream);
}

extern "C" int ffa_kproj_rope(const void *h, const void *w_k, const void *bias, int h_dtype, const void *cos,
                              const void *sin, int cs_dtype, int B, int T, int H, int HKV, int D, void *k_out,
                              void *stream) {
  if (B <= 0 || T <= 0 || H <= 0 || HKV <= 0 || D <= 0) return ffa_set_error_internal(FFA_E_INVALID, "bad dims");
  if (!(h_dtype == FFA_DT_F16 || h_dtype == FFA_DT_BF16))
    return ffa_set_error_internal(FFA_E_UNSUPPORTED, "h must be fp16 or bf16");
  if (!(cs_dtype == FFA_DT_F32 || cs_dtype == h_dtype))
    return ffa_set_error_internal(FFA_E_UNSUPPORTED, "cos/sin must be fp32 or the dtype of h");
  if (D % 2 || (HKV * D) % 32 || H % 32)
    return ffa_set_error_internal(FFA_E_UNSUPPORTED, "needs even D, HKV*D % 32 == 0, H % 32 == 0");
  const int M = B * T, N = HKV * D;
  const int odt = cs_dtype == FFA_DT_F32 ? FFA_DT_F32 : h_dtype;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)((N / 32) * ((M + 15) / 16)));
  if (h_dtype == FFA_DT_BF16)
    hipLaunchKernelGGL(ffa::kproj_rope_kernel<FFA_DT_BF16>, grid, dim3(512), 0, st, h, w_k, bias, cos, sin, cs_dtype, M,
                       T, H, N, D, k_out, odt);
  else
    hipLaunchKernelGGL(ffa::kproj_rope_kernel<FFA_DT_F16>, grid, dim3(512), 0, st, h, w_k, bias, cos, sin, cs_dtype, M,
                       T, H, N, D, k_out, odt);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return ffa_set_error_internal(FFA_E_LAUNCH, hipGetErrorString(e));
  return FFA_OK;
}

extern "C" int ffa_kproj_rope_q2_channel(const void *h, const void *w_k, const void *bias, int h_dtype, const void *cos,
                                         const void *sin, int cs_dtype, int B, int T, int H, int HKV, int D,
                                         void *k_scratch, uint8_t *k_q, void *scale, void *zero, uint8_t *residual,
                                         int res_dtype, float *minmax, void *stream) {
  if (!(res_dtype == FFA_DT_FP8_E4M3 || res_dtype == FFA_DT_FP8_E5M2))
    return ffa_set_error_internal(FFA_E_INVALID, "residual dtype must be fp8");
  const int rc = ffa_kproj_rope(h, w_k, bias, h_dtype, cos, sin, cs_dtype, B, T, H, HKV, D, k_scratch, stream);
  if (rc != FFA_OK) return rc;
  const int odt = cs_dtype == FFA_DT_F32 ? FFA_DT_F32 : h_dtype;
  return launch_quant_channel(k_scratch, odt, B, T, HKV, D, k_q, scale, zero, residual, res_dtype, minmax,
                              (hipStream_t)stream);
}

extern "C" int ffa_kproj_rope_q2_append(const void *h, const void *w_k, const void *bias, int h_dtype, const float *cos,
                                        const float *sin, int B, int Tn, int H, int HKV, const int32_t *pos,
                                        const int32_t *block_table, int bt_stride, int num_pages,
                                        uint8_t *k_q_pages, void *scale_pages, void *zero_pages, uint8_t *res_pages,
                                        int res_dtype, const void *v_new, void *v_pages, int v_dtype, void *stream) {
  if (B <= 0 || Tn <= 0 || H <= 0 || HKV <= 0) return ffa_set_error_internal(FFA_E_INVALID, "bad dims");
  if (bt_stride <= 0 || num_pages <= 0) return ffa_set_error_internal(FFA_E_INVALID, "empty block table or pool");
  if (!(h_dtype == FFA_DT_F16 || h_dtype == FFA_DT_BF16))
    return ffa_set_error_internal(FFA_E_UNSUPPORTED, "h must be fp16 or bf16");
  if (H % 32) return ffa_set_error_internal(FFA_E_UNSUPPORTED, "H must be a multiple of 32");
  if (!(res_dtype == FFA_DT_FP8_E4M3 || res_dtype == FFA_DT_FP8_E5M2))
    return ffa_set_error_internal(FFA_E_INVALID, "residual dtype must be fp8");
  if (v_new != nullptr && !(v_dtype == FFA_DT_F16 || v_dtype == FFA_DT_BF16))
    return ffa_set_error_internal(FFA_E_UNSUPPORTED, "V pages must be fp16 or bf16");
  const int M = B * Tn;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)(HKV * 4 * ((M + 15) / 16)));
  if (h_dtype == FFA_DT_BF16)
    hipLaunchKernelGGL(ffa::kproj_append_kernel<FFA_DT_BF16>, grid, dim3(512), 0, st, h, w_k, bias, cos, sin, M, Tn, H,
                       HKV, pos, block_table, bt_stride, num_pages, k_q_pages, (uint16_t *)scale_pages,
                       (uint16_t *)zero_pages,
                       res_pages, res_dtype == FFA_DT_FP8_E4M3 ? 1 : 0, v_new, v_pages);
  else
    hipLaunchKernelGGL(ffa::kproj_append_kernel<FFA_DT_F16>, grid, dim3(512), 0, st, h, w_k, bias, cos, sin, M, Tn, H,
                       HKV, pos, block_table, bt_stride, num_pages, k_q_pages, (uint16_t *)scale_pages,
                       (uint16_t *)zero_pages,
                       res_pages, res_dtype == FFA_DT_FP8_E4M3 ? 1 : 0, v_new, v_pages);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return ffa_set_error_internal(FFA_E_LAUNCH, hipGetErrorString(e));
  return FFA_OK;
}

extern "C" int ffa_q2_quantize_g32_append(const void *k, int k_dtype, int B, int Tn, int HKV, const int32_t *pos,
                                          const int32_t *block_table, int bt_stride, int num_pages,
                                          uint8_t *k_q_pages, void *scale_pages, void *zero_pages, uint8_t *res_pages,
                                          int res_dtype, const void *v_new, void *v_pages, void *stream) {
  if (B <= 0 || Tn <= 0 || HKV <= 0) return ffa_set_error_internal(FFA_E_INVALID, "bad dims");
  if (bt_stride <= 0 || num_pages <= 0) return ffa_set_error_internal(FFA_E_INVALID, "empty block table or pool");
  if (!(k_dtype >= FFA_DT_F16 && k_dtype <= FFA_DT_F32)) return ffa_set_error_internal(FFA_E_INVALID, "k dtype");
  if (!(res_dtype == FFA_DT_FP8_E4M3 || res_dtype == FFA_DT_FP8_E5M2))
    return ffa_set_error_internal(FFA_E_INVALID, "residual dtype must be fp8");
  const size_t rows = (size_t)B * Tn * HKV;
  hipLaunchKernelGGL(ffa::q2_g32_append_kernel, dim3((unsigned)((rows + 1) / 2)), dim3(256), 0,
                     (hipStream_t)stream, k, k_dtype, B * Tn, Tn, HKV, pos, block_table, bt_stride, num_pages, k_q_pages,
                     (uint16_t *)scale_pages, (uint16_t *)zero_pages, res_pages, res_dtype == FFA_DT_FP8_E4M3 ? 1 : 0,
                     v_new, v_pages);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return ffa_set_error_internal(FFA_E_LAUNCH, hipGetErrorString(e));
  return FFA_OK;
}

extern "C" int ffa_q2_paged_dequant(const uint8_t *k_q_pages, const void *scale_pages, const void *zero_pages,
                                    const uint8_t *res_pages, int res_dtype, const void *v_pages, int v_dtype,
                                    const int32_t *block_table, int bt_stride, int num_pages, const int32_t *seq_lens,
                                    int B, int T, int HKV, void *k_out, void *v_out, int out_dtype, void *stream) {
  if (B <= 0 || T <= 0 || HKV <= 0) return ffa_set_error_internal(FFA_E_INVALID, "bad dims");
  if (B > 65535 || HKV > 65535) return ffa_set_error_internal(FFA_E_UNSUPPORTED, "B and HKV are grid dimensions");
  if (bt_stride <= 0 || num_pages <= 0) return ffa_set_error_internal(FFA_E_INVALID, "empty block table or pool");
  if ((long)bt_stride * ffa::kPage < T) return ffa_set_error_internal(FFA_E_INVALID, "block table has fewer than ceil(T/64) columns");
  if (!(res_dtype == FFA_DT_FP8_E4M3 || res_dtype == FFA_DT_FP8_E5M2))
    return ffa_set_error_internal(FFA_E_INVALID, "residual dtype must be fp8");
  if (!(v_dtype == FFA_DT_F16 || v_dtype == FFA_DT_BF16)) return ffa_set_error_internal(FFA_E_INVALID, "v dtype");
  if (!(out_dtype >= FFA_DT_F16 && out_dtype <= FFA_DT_F32)) return ffa_set_error_internal(FFA_E_INVALID, "out dtype");
  if (!k_q_pages || !scale_pages || !zero_pages || !res_pages || !v_pages || !block_table || !k_out || !v_out)
    return ffa_set_error_internal(FFA_E_INVALID, "null pointer");
  if (T % ffa::kPage) return ffa_set_error_internal(FFA_E_INVALID, "T must be a multiple of the 64-token page");
  hipLaunchKernelGGL(ffa::q2_paged_dequant_kernel, dim3((unsigned)(T / ffa::kPage), (unsigned)HKV, (unsigned)B),
                     dim3(256), 0, (hipStream_t)stream, k_q_pages, (const uint16_t *)scale_pages,
                     (const uint16_t *)zero_pages, res_pages, res_dtype == FFA_DT_FP8_E4M3 ? 1 : 0,
                     (const uint16_t *)v_pages, v_dtype, block_table, bt_stride, num_pages, seq_lens, T, HKV, k_out,
                     v_out, out_dtype);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FFA_OK : ffa_set_error_internal(FFA_E_LAUNCH, hipGetErrorString(e));
}
