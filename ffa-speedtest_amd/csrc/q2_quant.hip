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
//    per-token groups make the append local, so GEMM,
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
  const int C = HKV * D;
  uint32_t packed = 0;
  for (int e = 0; e < 4; ++e) {
    const int d = 4 * byte + e;
    if (d >= D) break;
    const float kv = load_any(k, row * D + d, kdt);
    const float sc = load_any(scale, (size_t)b * C + hkv * D + d, kdt);
    const float zr = load_any(zero, (size_t)b * C + hkv * D + d, kdt);
    const float xs = round_to(kv - zr, kdt);               // (k - zero) in tau
    const float xd = round_to(__fdiv_rn(xs, sc), kdt);     // / scale in tau
    const float cq = fminf(fmaxf(__builtin_rintf(xd), 0.f), 3.f);  // round (RNE), clamp(0,3)
    const float deq = (cq * sc) + zr;                      // two fp32 roundings
    res[row * D + d] = (uint8_t)f32_to_fp8(kv - deq, res_e4m3);
    packed |= ((uint32_t)cq) << (2 * e);
  }
  kq[row * DP + byte] = (uint8_t)packed;
}

// ---------------------------------------------------------------------------
// g32 quantization of one (token, KV head, group) and its page writes.
// zero = fp16(min), scale = fp16(max(max - zero, 1e-6) / 3), c = clamp(rne((k - zero)/scale), 0, 3),
// residual = fp8(k - (c*scale + zero)) with two fp32 roundings.
__device__ __forceinline__ void g32_quantize_store(const float *kv, int page, int slot, int hkv, int HKV, int g,
                                                   uint8_t *kq_pages, uint16_t *s_pages, uint16_t *z_pages,
                                                   uint8_t *r_pages, int res_e4m3) {
  constexpr int D = 128;
  float mn = INFINITY, mx = -INFINITY;
  for (int e = 0; e < 32; ++e) {
    mn = fminf(mn, kv[e]);
    mx = fmaxf(mx, kv[e]);
  }
  const float zr = (float)(_Float16)mn;
  const float sc = (float)(_Float16)__fdiv_rn(fmaxf(mx - zr, 1e-6f), 3.0f);
  uint32_t words[2] = {0u, 0u};
  uint32_t rw[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  for (int e = 0; e < 32; ++e) {
    const float cq = fminf(fmaxf(__builtin_rintf(__fdiv_rn(kv[e] - zr, sc)), 0.f), 3.f);
    const float deq = (cq * sc) + zr;
    rw[e >> 2] |= f32_to_fp8(kv[e] - deq, res_e4m3) << (8 * (e & 3));
    words[e >> 4] |= ((uint32_t)cq) << (2 * (e & 15));
  }
  // page-internal orders: decode_common.h (res_off, codes_off, gscale_off)
  const size_t blk = (size_t)page * HKV + hkv;
  uint8_t *rp = r_pages + blk * (64 * D);
  *(uint4 *)(rp + res_off(slot, 32 * g)) = make_uint4(rw[0], rw[1], rw[2], rw[3]);
  *(uint4 *)(rp + res_off(slot, 32 * g + 16)) = make_uint4(rw[4], rw[5], rw[6], rw[7]);
  *(uint2 *)(kq_pages + blk * (4 * 64 * 8) + codes_off(g, slot)) = make_uint2(words[0], words[1]);
  const int ss = 16 * (slot >> 4) + 4 * (slot & 3) + ((slot >> 2) & 3);  // tile-major scale slot
  const size_t so = blk * (4 * 64) + gscale_off(g, ss);
  s_pages[so] = (uint16_t)f32_to_f16_bits(sc);
  z_pages[so] = (uint16_t)f32_to_f16_bits(zr);
}

// K projection GEMM tile: 16 tokens x 128 output channels per workgroup,
// 4 waves x 2 MFMA column tiles of 16.  acc[tile][u] = row 4*(lane>>4)+u,
// column n0 + 32*wave + 16*tile + (lane & 15).
// ---------------------------------------------------------------------------
template <int HDT>
__device__ __forceinline__ void kproj_tile(const void *h, const void *w, int M, int H, int m0, int n0,
                                           f32x4 acc[2]) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int mrow = min(m0 + (lane & 15), M - 1);
  const int kq = 8 * (lane >> 4);
  const uint16_t *hp = (const uint16_t *)h + (size_t)mrow * H + kq;
  const uint16_t *wp0 = (const uint16_t *)w + (size_t)(n0 + 32 * wv + (lane & 15)) * H + kq;
  const uint16_t *wp1 = wp0 + (size_t)16 * H;
  acc[0] = f32x4{0.f, 0.f, 0.f, 0.f};
  acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int k0 = 0; k0 < H; k0 += 32) {
    const uint4 a = *(const uint4 *)(hp + k0);
    const uint4 b0 = *(const uint4 *)(wp0 + k0);
    const uint4 b1 = *(const uint4 *)(wp1 + k0);
    const u32x4 av = {a.x, a.y, a.z, a.w}, bv0 = {b0.x, b0.y, b0.z, b0.w}, bv1 = {b1.x, b1.y, b1.z, b1.w};
    if constexpr (HDT == FFA_DT_BF16) {
      acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv0),
                                                       acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv1),
                                                       acc[1], 0, 0, 0);
    } else {
      acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av), __builtin_bit_cast(f16x8, bv0),
                                                      acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av), __builtin_bit_cast(f16x8, bv1),
                                                      acc[1], 0, 0, 0);
    }
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

// Rotated K of the reference producer -> k_scratch [M, N] in dtype odt.
template <int HDT>
__global__ __launch_bounds__(256) void kproj_rope_kernel(const void *h, const void *w, const void *bias, const void *cos,
                                                         const void *sin, int csdt, int M, int T, int H, int N, int D,
                                                         void *kout, int odt) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int m0 = blockIdx.y * 16, n0 = blockIdx.x * 128;
  f32x4 acc[2];
  kproj_tile<HDT>(h, w, M, H, m0, n0, acc);
#pragma unroll
  for (int tile = 0; tile < 2; ++tile) {
    const int col = n0 + 32 * wv + 16 * tile + (lane & 15);
    const float bv = bias ? load_any(bias, col, HDT) : 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int m = m0 + 4 * (lane >> 4) + u;
      // F.linear output in the h dtype
      const float x = round_to(acc[tile][u] + bv, HDT);
      const float partner = __shfl_xor(x, 1);
      const int d = col % D;
      const int t = m % T;
      const float c = load_any(cos, (size_t)t * D + d, csdt);
      const float s = load_any(sin, (size_t)t * D + d, csdt);
      const float r = rope_one(x, partner, (d & 1) != 0, c, s, odt);
      if (m < M) store_any(kout, (size_t)m * N + col, odt, r);
    }
  }
}

// K-proj + RoPE (fp32 cos/sin rows per token) + g32 quantize + paged append.
template <int HDT>
__global__ __launch_bounds__(256) void kproj_append_kernel(const void *h, const void *w, const void *bias,
                                                           const float *cos, const float *sin, int M, int Tn, int H,
                                                           int HKV, const int32_t *pos, const int32_t *bt, int bt_stride,
                                                           uint8_t *kq_pages, uint16_t *s_pages, uint16_t *z_pages,
                                                           uint8_t *r_pages, int res_e4m3, const void *v_new,
                                                           void *v_pages, int vdt) {
  constexpr int D = 128;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int m0 = blockIdx.y * 16;
  const int hkv = blockIdx.x;  // one head (128 channels) per workgroup column
  const int n0 = hkv * D;
  const int N = HKV * D;
  __shared__ float s_k[16][D + 1];
  f32x4 acc[2];
  kproj_tile<HDT>(h, w, M, H, m0, n0, acc);
#pragma unroll
  for (int tile = 0; tile < 2; ++tile) {
    const int d = 32 * wv + 16 * tile + (lane & 15);
    const float bv = bias ? load_any(bias, n0 + d, HDT) : 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int r = 4 * (lane >> 4) + u;
      const int m = min(m0 + r, M - 1);
      const float x = round_to(acc[tile][u] + bv, HDT);
      const float partner = __shfl_xor(x, 1);
      const float c = cos[(size_t)m * D + d];
      const float s = sin[(size_t)m * D + d];
      s_k[r][d] = rope_one(x, partner, (d & 1) != 0, c, s, FFA_DT_F32);  // fp32 cos promotes to fp32
    }
  }
  __syncthreads();
  // one thread per (token row, group): 16 x 4 = 64 threads
  if (threadIdx.x < 64) {
    const int r = threadIdx.x >> 2, g = threadIdx.x & 3;
    const int m = m0 + r;
    if (m < M) {
      const int b = m / Tn, nn = m % Tn;
      const int P = pos[b] + nn;
      const int page = bt[(size_t)b * bt_stride + (P >> 6)];
      const int slot = P & 63;
      float kv[32];
      for (int e = 0; e < 32; ++e) kv[e] = s_k[r][32 * g + e];
      g32_quantize_store(kv, page, slot, hkv, HKV, g, kq_pages, s_pages, z_pages, r_pages, res_e4m3);
    }
  }
  // V append into V^T pages: thread -> (token row, 8 channels)
  if (v_new != nullptr) {
    const int r = threadIdx.x >> 4, c8 = (threadIdx.x & 15) * 8;
    const int m = m0 + r;
    if (m < M) {
      const int b = m / Tn, nn = m % Tn;
      const int P = pos[b] + nn;
      const int page = bt[(size_t)b * bt_stride + (P >> 6)];
      const int slot = P & 63;
      const uint16_t *vs = (const uint16_t *)v_new + ((size_t)m * HKV + hkv) * D + c8;
      uint16_t *vd = (uint16_t *)v_pages + ((size_t)page * HKV + hkv) * (D * 64);
      for (int e = 0; e < 8; ++e) vd[vt_off(c8 + e, slot)] = vs[e];
    }
  }
  (void)N;
  (void)vdt;
}


// g32 quantize + append of given K rows (no projection): one thread per
// (token row, KV head, group).  k [B, Tn, HKV, 128] (dtype kdt).
__global__ __launch_bounds__(256) void q2_g32_append_kernel(const void *k, int kdt, int M, int Tn, int HKV,
                                                             const int32_t *pos, const int32_t *bt, int bt_stride,
                                                             uint8_t *kq_pages, uint16_t *s_pages, uint16_t *z_pages,
                                                             uint8_t *r_pages, int res_e4m3, const void *v_new,
                                                             void *v_pages) {
  constexpr int D = 128;
  const size_t id = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= (size_t)M * HKV * 4) return;
  const int g = (int)(id & 3);
  const int hkv = (int)((id >> 2) % HKV);
  const int m = (int)((id >> 2) / HKV);
  const int b = m / Tn, nn = m % Tn;
  const int P = pos[b] + nn;
  const int page = bt[(size_t)b * bt_stride + (P >> 6)];
  const int slot = P & 63;
  float kv[32];
  for (int e = 0; e < 32; ++e) kv[e] = load_any(k, ((size_t)m * HKV + hkv) * D + 32 * g + e, kdt);
  g32_quantize_store(kv, page, slot, hkv, HKV, g, kq_pages, s_pages, z_pages, r_pages, res_e4m3);
  if (v_new != nullptr) {
    const uint16_t *vs = (const uint16_t *)v_new + ((size_t)m * HKV + hkv) * D + 32 * g;
    uint16_t *vd = (uint16_t *)v_pages + ((size_t)page * HKV + hkv) * (D * 64);
    for (int e = 0; e < 32; ++e) vd[vt_off(32 * g + e, slot)] = vs[e];
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
  if (D % 2 || (HKV * D) % 128 || H % 32) return ffa_set_error_internal(FFA_E_UNSUPPORTED, "needs even D, HKV*D % 128 == 0, H % 32 == 0");
  const int M = B * T, N = HKV * D;
  const int odt = cs_dtype == FFA_DT_F32 ? FFA_DT_F32 : h_dtype;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid(N / 128, (M + 15) / 16);
  if (h_dtype == FFA_DT_BF16)
    hipLaunchKernelGGL(ffa::kproj_rope_kernel<FFA_DT_BF16>, grid, dim3(256), 0, st, h, w_k, bias, cos, sin, cs_dtype, M,
                       T, H, N, D, k_out, odt);
  else
    hipLaunchKernelGGL(ffa::kproj_rope_kernel<FFA_DT_F16>, grid, dim3(256), 0, st, h, w_k, bias, cos, sin, cs_dtype, M,
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
                                        const int32_t *block_table, int bt_stride, uint8_t *k_q_pages,
                                        void *scale_pages, void *zero_pages, uint8_t *res_pages, int res_dtype,
                                        const void *v_new, void *v_pages, int v_dtype, void *stream) {
  if (!(h_dtype == FFA_DT_F16 || h_dtype == FFA_DT_BF16))
    return ffa_set_error_internal(FFA_E_UNSUPPORTED, "h must be fp16 or bf16");
  if (H % 32) return ffa_set_error_internal(FFA_E_UNSUPPORTED, "H must be a multiple of 32");
  if (!(res_dtype == FFA_DT_FP8_E4M3 || res_dtype == FFA_DT_FP8_E5M2))
    return ffa_set_error_internal(FFA_E_INVALID, "residual dtype must be fp8");
  const int M = B * Tn;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid(HKV, (M + 15) / 16);
  if (h_dtype == FFA_DT_BF16)
    hipLaunchKernelGGL(ffa::kproj_append_kernel<FFA_DT_BF16>, grid, dim3(256), 0, st, h, w_k, bias, cos, sin, M, Tn, H,
                       HKV, pos, block_table, bt_stride, k_q_pages, (uint16_t *)scale_pages, (uint16_t *)zero_pages,
                       res_pages, res_dtype == FFA_DT_FP8_E4M3 ? 1 : 0, v_new, v_pages, v_dtype);
  else
    hipLaunchKernelGGL(ffa::kproj_append_kernel<FFA_DT_F16>, grid, dim3(256), 0, st, h, w_k, bias, cos, sin, M, Tn, H,
                       HKV, pos, block_table, bt_stride, k_q_pages, (uint16_t *)scale_pages, (uint16_t *)zero_pages,
                       res_pages, res_dtype == FFA_DT_FP8_E4M3 ? 1 : 0, v_new, v_pages, v_dtype);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return ffa_set_error_internal(FFA_E_LAUNCH, hipGetErrorString(e));
  return FFA_OK;
}

extern "C" int ffa_q2_quantize_g32_append(const void *k, int k_dtype, int B, int Tn, int HKV, const int32_t *pos,
                                          const int32_t *block_table, int bt_stride, uint8_t *k_q_pages,
                                          void *scale_pages, void *zero_pages, uint8_t *res_pages, int res_dtype,
                                          const void *v_new, void *v_pages, void *stream) {
  if (B <= 0 || Tn <= 0 || HKV <= 0) return ffa_set_error_internal(FFA_E_INVALID, "bad dims");
  if (!(k_dtype >= FFA_DT_F16 && k_dtype <= FFA_DT_F32)) return ffa_set_error_internal(FFA_E_INVALID, "k dtype");
  if (!(res_dtype == FFA_DT_FP8_E4M3 || res_dtype == FFA_DT_FP8_E5M2))
    return ffa_set_error_internal(FFA_E_INVALID, "residual dtype must be fp8");
  const size_t total = (size_t)B * Tn * HKV * 4;
  hipLaunchKernelGGL(ffa::q2_g32_append_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, k, k_dtype, B * Tn, Tn, HKV, pos, block_table, bt_stride, k_q_pages,
                     (uint16_t *)scale_pages, (uint16_t *)zero_pages, res_pages, res_dtype == FFA_DT_FP8_E4M3 ? 1 : 0,
                     v_new, v_pages);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return ffa_set_error_internal(FFA_E_LAUNCH, hipGetErrorString(e));
  return FFA_OK;
}
