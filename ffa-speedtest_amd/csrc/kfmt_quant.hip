// K quantizers of the fp8, nvfp4 and nf4 formats for gfx950 (reference layouts).
//
// Each one is bit-exact with the reference's torch op sequence:
//  * fp8 base + fp8 residual (ffa-fp8fp8/fused_kproj_rope_fp8fp8.py:58-64):
//      base = fp8(k), residual = fp8(f32(k) - f32(base)).
//  * nvfp4 (ffa-nvfp4fp8/fused_kproj_rope_nvfp4fp8.py:62-114): one scale per
//    (sequence, page of page_size tokens, KV head) over page x D, every op in the
//    K dtype tau: s = max(tau(amax / 6), tau(1e-6)), x = tau(k / s),
//    code = #{e2m1 midpoints <= |x|} | sign << 3, residual = fp8(tau(k - tau(+-level * s))).
//  * nf4 (ffa-nf4fp8/fused_kproj_rope_nf4fp8.py:72-96): fp32 per-channel absmax
//    over T, s = max(absmax, 1e-6), x = clamp(k / s, -1, 1),
//    code = #{codebook midpoints < x}, residual = fp8(k - codebook[code] * s); the
//    scale is stored in tau.
// No FMA contraction in this file; divisions are IEEE round-to-nearest.
#include "decode_common.h"
#include "ffa_common.h"
#include "ffa_mi355x.h"

#pragma clang fp contract(off)

namespace ffa {

// exact fp8 -> f32 from the format definitions (OCP e4m3fn: bias 7, no infinities,
// S.1111.111 = NaN; e5m2: the high byte of the fp16 with the same value)
__device__ __forceinline__ float fp8_bits_to_f32(uint32_t b, int e4m3) {
  if (!e4m3) return f16_bits_to_f32(b << 8);
  const uint32_t s = b >> 7, e = (b >> 3) & 15u, m = b & 7u;
  float v;
  if (e == 15u && m == 7u) v = __builtin_nanf("");
  else if (e == 0u) v = (float)m * 0x1p-9f;
  else v = __uint_as_float(((e + 120u) << 23) | (m << 20));  // (1 + m/8) * 2^(e-7)
  return s ? -v : v;
}

// ---------------------------------------------------------------------------
// fp8 base + fp8 residual: 4 elements per thread
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fp8fp8_quant_kernel(const void *k, int kdt, size_t n, uint8_t *base,
                                                            uint8_t *res, int e4m3) {
  const size_t i0 = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i0 >= n) return;
  uint32_t bw = 0, rw = 0;
  const int cnt = (int)min((size_t)4, n - i0);
  for (int e = 0; e < cnt; ++e) {
    const float x = load_any(k, i0 + e, kdt);
    const uint32_t bb = f32_to_fp8(x, e4m3);
    const uint32_t rb = f32_to_fp8(x - fp8_bits_to_f32(bb, e4m3), e4m3);
    bw |= bb << (8 * e);
    rw |= rb << (8 * e);
  }
  if (cnt == 4 && (((uintptr_t)(base + i0) | (uintptr_t)(res + i0)) & 3u) == 0) {
    *(uint32_t *)(base + i0) = bw;
    *(uint32_t *)(res + i0) = rw;
  } else {
    for (int e = 0; e < cnt; ++e) {
      base[i0 + e] = (uint8_t)(bw >> (8 * e));
      res[i0 + e] = (uint8_t)(rw >> (8 * e));
    }
  }
}

// ---------------------------------------------------------------------------
// per-token-scaled fp8 (no reference counterpart): for each row of D values (one token and
// KV head) s = max(fp16(max(amax |k|, 1e-6) / fmax), 2^-14) (fmax = 448 for e4m3, 57344 for
// e5m2), base = fp8(k / s), residual = fp8(k - value(base) * s); the product is exact (at most
// 4 x 11 significant bits).  The floor (the smallest normal fp16) keeps s non-zero for all-zero
// and tiny rows and |k / s| within fmax (1 + 2^-11), which rounds to fmax: a subnormal s could
// sit half a quantum below amax / fmax and push k / s past fmax (NaN in e4m3).
// One wave per row, lane e holds elements e, e + 64, ...
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fp8_scaled_quant_kernel(const void *k, int kdt, size_t rows, int D,
                                                               uint8_t *base, uint16_t *scale, uint8_t *res,
                                                               int e4m3) {
  const size_t row = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves
  const int lane = threadIdx.x & 63;
  const size_t r0 = row * (size_t)D;
  float amax = 0.f;
  for (int d = lane; d < D; d += 64) amax = fmaxf(amax, fabsf(load_any(k, r0 + d, kdt)));
  amax = wave_max(amax);
  const float s = fmaxf((float)(_Float16)__fdiv_rn(fmaxf(amax, 1e-6f), e4m3 ? 448.f : 57344.f), 0x1p-14f);
  for (int d = lane; d < D; d += 64) {
    const float x = load_any(k, r0 + d, kdt);
    const uint32_t bb = f32_to_fp8(__fdiv_rn(x, s), e4m3);
    base[r0 + d] = (uint8_t)bb;
    res[r0 + d] = (uint8_t)f32_to_fp8(x - fp8_bits_to_f32(bb, e4m3) * s, e4m3);
  }
  if (lane == 0) scale[row] = (uint16_t)f32_to_f16_bits(s);
}

// ---------------------------------------------------------------------------
// nvfp4: one workgroup per (sequence, page, KV head)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float fp4_level(int i) {
  // e2m1 magnitudes of codes 0..7
  return i < 4 ? 0.5f * (float)i : (i == 4 ? 2.f : (i == 5 ? 3.f : (i == 6 ? 4.f : 6.f)));
}

__global__ __launch_bounds__(256) void nvfp4_quant_kernel(const void *k, int kdt, int T, int HKV, int D, int page,
                                                           uint8_t *packed, void *scale, uint8_t *res, int e4m3) {
  const int hkv = blockIdx.x, pg = blockIdx.y, b = blockIdx.z;
  const int npg = gridDim.y;
  const int t0 = pg * page;
  const int nt = min(page, T - t0);  // tokens of the page inside the sequence (padding tokens are zeros)
  const int DP = (D + 1) / 2;
  __shared__ float s_red[256 / 64];
  // amax over the page's tokens x D
  float mx = 0.f;
  for (int i = threadIdx.x; i < nt * D; i += 256) {
    const int t = i / D, d = i - t * D;
    mx = fmaxf(mx, fabsf(load_any(k, (((size_t)b * T + t0 + t) * HKV + hkv) * D + d, kdt)));
  }
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  // scale = (amax / 6).clamp_min(1e-6), both in tau
  const float sc = fmaxf(round_to(__fdiv_rn(mx, 6.0f), kdt), round_to(1e-6f, kdt));
  if (threadIdx.x == 0) store_any(scale, ((size_t)b * npg + pg) * HKV + hkv, kdt, sc);
  // codes and residuals, one packed byte (two channels) per thread and step
  for (int i = threadIdx.x; i < nt * DP; i += 256) {
    const int t = i / DP, byte = i - t * DP;
    const size_t row = ((size_t)b * T + t0 + t) * HKV + hkv;
    uint32_t pk = 0;
    for (int e = 0; e < 2; ++e) {
      const int d = 2 * byte + e;
      if (d >= D) break;  // odd D pads a zero nibble
      const float kv = load_any(k, row * D + d, kdt);
      const float xs = round_to(__fdiv_rn(kv, sc), kdt);
      const float ax = fabsf(xs);
      // bucketize(|x|, midpoints, right=True): count of midpoints <= |x|
      const int idx = (ax >= 0.25f) + (ax >= 0.75f) + (ax >= 1.25f) + (ax >= 1.75f) + (ax >= 2.5f) + (ax >= 3.5f) +
                      (ax >= 5.0f);
      const bool neg = xs < 0.f;
      const float deq = round_to((neg ? -fp4_level(idx) : fp4_level(idx)) * sc, kdt);
      res[row * D + d] = (uint8_t)f32_to_fp8(round_to(kv - deq, kdt), e4m3);
      pk |= (uint32_t)(idx | (neg ? 8 : 0)) << (4 * e);
    }
    packed[row * DP + byte] = (uint8_t)pk;
  }
}

// ---------------------------------------------------------------------------
// nf4: per-channel absmax over T (splits, then a final pass), then codes
// ---------------------------------------------------------------------------
__constant__ float kNF4Book[16] = {-1.0f,
                                   -0.6961928009986877f,
                                   -0.5229921340942383f,
                                   -0.39491748809814453f,
                                   -0.28444138169288635f,
                                   -0.18477343022823334f,
                                   -0.09105003625154495f,
                                   0.0f,
                                   0.07958029955625534f,
                                   0.16093020141124725f,
                                   0.24611230194568634f,
                                   0.33791524171829224f,
                                   0.44070982933044434f,
                                   0.5626170039176941f,
                                   0.7229568362236023f,
                                   1.0f};
constexpr int kNF4Tok = 256;  // tokens per absmax split

__global__ __launch_bounds__(256) void nf4_absmax_kernel(const void *k, int kdt, int T, int C, int nsplit,
                                                          float *amax) {
  // grid (nsplit, B, ceil(C/256)); thread = channel (h, d)
  const int split = blockIdx.x, b = blockIdx.y;
  const int c = blockIdx.z * 256 + threadIdx.x;
  if (c >= C) return;
  const int tper = (T + nsplit - 1) / nsplit;
  const int ta = split * tper, tb = min(T, ta + tper);
  float mx = 0.f;
  for (int t = ta; t < tb; ++t) mx = fmaxf(mx, fabsf(load_any(k, ((size_t)b * T + t) * C + c, kdt)));
  amax[((size_t)b * nsplit + split) * C + c] = mx;
}

// final scale: fp32 s = max(absmax, 1e-6) back into split 0 of the scratch, tau(s) to the output
__global__ __launch_bounds__(256) void nf4_scale_kernel(float *amax, int nsplit, int C, int kdt, void *scale) {
  const int b = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  float mx = 0.f;
  for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, amax[((size_t)b * nsplit + s) * C + c]);
  const float sc = fmaxf(mx, 1e-6f);
  amax[(size_t)b * nsplit * C + c] = sc;
  store_any(scale, (size_t)b * C + c, kdt, sc);
}

// one thread per (token, packed byte)
__global__ __launch_bounds__(256) void nf4_quant_kernel(const void *k, int kdt, int B, int T, int HKV, int D,
                                                         const float *amax, int nsplit, uint8_t *packed, uint8_t *res,
                                                         int e4m3) {
  const int DP = (D + 1) / 2;
  const size_t total = (size_t)B * T * HKV * DP;
  const size_t id = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= total) return;
  const int byte = (int)(id % DP);
  const size_t row = id / DP;  // (b, t, hkv)
  const int hkv = (int)(row % HKV);
  const int b = (int)(row / ((size_t)HKV * T));
  const int C = HKV * D;
  uint32_t pk = 0;
  for (int e = 0; e < 2; ++e) {
    const int d = 2 * byte + e;
    if (d >= D) break;
    const float kv = load_any(k, row * D + d, kdt);
    const float sc = amax[(size_t)b * nsplit * C + hkv * D + d];
    const float x = fminf(fmaxf(__fdiv_rn(kv, sc), -1.0f), 1.0f);
    // bucketize(x, midpoints) (right=False): count of midpoints < x
    int idx = 0;
#pragma unroll
    for (int j = 0; j < 15; ++j) idx += ((kNF4Book[j] + kNF4Book[j + 1]) * 0.5f < x) ? 1 : 0;
    res[row * D + d] = (uint8_t)f32_to_fp8(kv - kNF4Book[idx] * sc, e4m3);
    pk |= (uint32_t)idx << (4 * e);
  }
  packed[row * DP + byte] = (uint8_t)pk;
}

// ---------------------------------------------------------------------------
// Paged group-scale modes (no reference counterpart): quantize K rows and append them,
// with V, into 64-token pages.  One thread per (token row, KV head, 16 channels);
// the 8 threads of a row and head are consecutive lanes of one wave.
//   nvfp4-g16: s = e4m3(min(amax16 / 6, 448)), x = k / s (0 where s == 0),
//              code = #{e2m1 midpoints <= |x|} | sign << 3, residual = fp8(k - (+-level * s))
//   nf4-g64:   s = fp16(max(amax64, 1e-6)), x = clamp(k / s, -1, 1),
//              code = #{codebook midpoints < x}, residual = fp8(k - codebook[code] * s)
// Pools: codes [P, HKV, 64, 64] u8 (token-major, low nibble first), scales [P, HKV, 64, 8] e4m3
// (nvfp4) or [P, HKV, 64, 2] fp16 (nf4), residual [P, HKV, 64, 128] fp8, V^T [P, HKV, 128, 64].
// ---------------------------------------------------------------------------
template <bool NF4>
__global__ __launch_bounds__(256) void kfmt_group_append_kernel(const void *k, int kdt, int M, int Tn, int HKV,
                                                                 const int32_t *pos, const int32_t *bt, int bt_stride,
                                                                 int num_pages, uint8_t *k_pages, void *s_pages,
                                                                 uint8_t *r_pages, int res_e4m3, const void *v_new,
                                                                 void *v_pages) {
  constexpr int D = 128;
  const size_t id = (size_t)blockIdx.x * 256 + threadIdx.x;
  const bool live = id < (size_t)M * HKV * 8;  // whole groups of 8 lanes are live or not
  const size_t idc = live ? id : 0;
  const int c16 = (int)(idc & 7);
  const int hkv = (int)((idc >> 3) % HKV);
  const int m = (int)((idc >> 3) / HKV);
  const int b = m / Tn, nn = m - b * Tn;
  const int P = pos[b] + nn;
  const int page = append_page(bt, bt_stride, num_pages, b, P);
  const bool wr = live && page >= 0;  // whole groups of 8 lanes (one token and head) write or not
  const int slot = P & 63;
  const size_t prow = ((size_t)page * HKV + hkv) * 64 + slot;  // (page, head, token) row of the pools
  float kv[16];
  float amax = 0.f;
  for (int e = 0; e < 16; ++e) {
    kv[e] = load_any(k, ((size_t)m * HKV + hkv) * D + 16 * c16 + e, kdt);
    amax = fmaxf(amax, fabsf(kv[e]));
  }
  uint32_t cw[2] = {0u, 0u};
  uint32_t rw[4] = {0u, 0u, 0u, 0u};
  if constexpr (NF4) {
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    const float sc = (float)(_Float16)fmaxf(amax, 1e-6f);
    for (int e = 0; e < 16; ++e) {
      const float x = fminf(fmaxf(__fdiv_rn(kv[e], sc), -1.0f), 1.0f);
      int idx = 0;
#pragma unroll
      for (int j = 0; j < 15; ++j) idx += ((kNF4Book[j] + kNF4Book[j + 1]) * 0.5f < x) ? 1 : 0;
      rw[e >> 2] |= f32_to_fp8(kv[e] - kNF4Book[idx] * sc, res_e4m3) << (8 * (e & 3));
      cw[e >> 3] |= (uint32_t)idx << (4 * (e & 7));
    }
    if (wr && (c16 & 3) == 0) ((uint16_t *)s_pages)[prow * 2 + (c16 >> 2)] = (uint16_t)f32_to_f16_bits(sc);
  } else {
    const uint32_t sb = f32_to_fp8(fminf(__fdiv_rn(amax, 6.0f), 448.0f), 1);
    const float sc = fp8_bits_to_f32(sb, 1);
    for (int e = 0; e < 16; ++e) {
      const float x = sc > 0.f ? __fdiv_rn(kv[e], sc) : 0.f;
      const float ax = fabsf(x);
      const int idx = (ax >= 0.25f) + (ax >= 0.75f) + (ax >= 1.25f) + (ax >= 1.75f) + (ax >= 2.5f) + (ax >= 3.5f) +
                      (ax >= 5.0f);
      const bool neg = x < 0.f;
      const float deq = (neg ? -fp4_level(idx) : fp4_level(idx)) * sc;  // exact
      rw[e >> 2] |= f32_to_fp8(kv[e] - deq, res_e4m3) << (8 * (e & 3));
      cw[e >> 3] |= (uint32_t)(idx | (neg ? 8 : 0)) << (4 * (e & 7));
    }
    if (wr) ((uint8_t *)s_pages)[prow * 8 + c16] = (uint8_t)sb;
  }
  if (!wr) return;
  // page-internal orders: decode_common.h (k4_off, res_off, vt_off)
  const size_t blk = (size_t)page * HKV + hkv;
  *(uint2 *)(k_pages + blk * (64 * 64) + k4_off(slot, 8 * c16)) = make_uint2(cw[0], cw[1]);
  *(uint4 *)(r_pages + blk * (64 * D) + res_off(slot, 16 * c16)) = make_uint4(rw[0], rw[1], rw[2], rw[3]);
  if (v_new != nullptr) {
    const uint16_t *vs = (const uint16_t *)v_new + ((size_t)m * HKV + hkv) * D + 16 * c16;
    uint16_t *vd = (uint16_t *)v_pages + blk * (D * 64);
    for (int e = 0; e < 16; ++e) vd[vt_off(16 * c16 + e, slot)] = vs[e];
  }
}

}  // namespace ffa

// ============================================================================
// C ABI
// ============================================================================
extern "C" __attribute__((visibility("hidden"))) int ffa_set_error_internal(int code, const char *msg);

static int launch_status() {
  const hipError_t e = hipGetLastError();
  return e != hipSuccess ? ffa_set_error_internal(FFA_E_LAUNCH, hipGetErrorString(e)) : FFA_OK;
}

static bool is_fp8(int dt) { return dt == FFA_DT_FP8_E4M3 || dt == FFA_DT_FP8_E5M2; }
static bool is_float(int dt) { return dt >= FFA_DT_F16 && dt <= FFA_DT_F32; }

extern "C" int ffa_fp8fp8_quantize(const void *k, int k_dtype, size_t n, uint8_t *base, uint8_t *residual,
                                   int fp8_dtype, void *stream) {
  if (!is_float(k_dtype)) return ffa_set_error_internal(FFA_E_INVALID, "k dtype");
  if (!is_fp8(fp8_dtype)) return ffa_set_error_internal(FFA_E_INVALID, "fp8 dtype");
  if (n == 0) return FFA_OK;
  const size_t threads = (n + 3) / 4;
  hipLaunchKernelGGL(ffa::fp8fp8_quant_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, k, k_dtype, n, base, residual, fp8_dtype == FFA_DT_FP8_E4M3 ? 1 : 0);
  return launch_status();
}

extern "C" int ffa_fp8_scaled_quantize(const void *k, int k_dtype, size_t rows, int D, uint8_t *base, void *scale,
                                       uint8_t *residual, int fp8_dtype, void *stream) {
  if (D <= 0) return ffa_set_error_internal(FFA_E_INVALID, "bad dims");
  if (!is_float(k_dtype)) return ffa_set_error_internal(FFA_E_INVALID, "k dtype");
  if (!is_fp8(fp8_dtype)) return ffa_set_error_internal(FFA_E_INVALID, "fp8 dtype");
  if (rows == 0) return FFA_OK;
  hipLaunchKernelGGL(ffa::fp8_scaled_quant_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                     k, k_dtype, rows, D, base, (uint16_t *)scale, residual, fp8_dtype == FFA_DT_FP8_E4M3 ? 1 : 0);
  return launch_status();
}

extern "C" int ffa_nvfp4_quantize(const void *k, int k_dtype, int B, int T, int HKV, int D, int page_size,
                                  uint8_t *k_packed, void *scale, uint8_t *residual, int res_dtype, void *stream) {
  if (B <= 0 || T <= 0 || HKV <= 0 || D <= 0 || page_size <= 0) return ffa_set_error_internal(FFA_E_INVALID, "bad dims");
  if (!is_float(k_dtype)) return ffa_set_error_internal(FFA_E_INVALID, "k dtype");
  if (!is_fp8(res_dtype)) return ffa_set_error_internal(FFA_E_INVALID, "residual dtype must be fp8");
  const int npg = (T + page_size - 1) / page_size;
  hipLaunchKernelGGL(ffa::nvfp4_quant_kernel, dim3(HKV, npg, B), dim3(256), 0, (hipStream_t)stream, k, k_dtype, T,
                     HKV, D, page_size, k_packed, scale, residual, res_dtype == FFA_DT_FP8_E4M3 ? 1 : 0);
  return launch_status();
}

extern "C" int ffa_nf4_quantize_nsplit(int T) {
  const int s = (T + ffa::kNF4Tok - 1) / ffa::kNF4Tok;
  return s < 1 ? 1 : (s > 64 ? 64 : s);
}

extern "C" int ffa_nf4_quantize(const void *k, int k_dtype, int B, int T, int HKV, int D, uint8_t *k_packed,
                                void *scale, uint8_t *residual, int res_dtype, float *absmax, void *stream) {
  if (B <= 0 || T <= 0 || HKV <= 0 || D <= 0) return ffa_set_error_internal(FFA_E_INVALID, "bad dims");
  if (!is_float(k_dtype)) return ffa_set_error_internal(FFA_E_INVALID, "k dtype");
  if (!is_fp8(res_dtype)) return ffa_set_error_internal(FFA_E_INVALID, "residual dtype must be fp8");
  hipStream_t st = (hipStream_t)stream;
  const int C = HKV * D;
  const int nsplit = ffa_nf4_quantize_nsplit(T);
  hipLaunchKernelGGL(ffa::nf4_absmax_kernel, dim3(nsplit, B, (C + 255) / 256), dim3(256), 0, st, k, k_dtype, T, C,
                     nsplit, absmax);
  hipLaunchKernelGGL(ffa::nf4_scale_kernel, dim3((C + 255) / 256, B), dim3(256), 0, st, absmax, nsplit, C, k_dtype,
                     scale);
  const size_t total = (size_t)B * T * HKV * ((D + 1) / 2);
  hipLaunchKernelGGL(ffa::nf4_quant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, k, k_dtype, B, T,
                     HKV, D, (const float *)absmax, nsplit, k_packed, residual, res_dtype == FFA_DT_FP8_E4M3 ? 1 : 0);
  return launch_status();
}

static int group_append(bool nf4, const void *k, int k_dtype, int B, int Tn, int HKV, const int32_t *pos,
                        const int32_t *block_table, int bt_stride, int num_pages, uint8_t *k_pages,
                        void *scale_pages, uint8_t *res_pages, int res_dtype, const void *v_new, void *v_pages,
                        void *stream) {
  if (B <= 0 || Tn <= 0 || HKV <= 0) return ffa_set_error_internal(FFA_E_INVALID, "bad dims");
  if (bt_stride <= 0 || num_pages <= 0) return ffa_set_error_internal(FFA_E_INVALID, "empty block table or pool");
  if (!is_float(k_dtype)) return ffa_set_error_internal(FFA_E_INVALID, "k dtype");
  if (!is_fp8(res_dtype)) return ffa_set_error_internal(FFA_E_INVALID, "residual dtype must be fp8");
  const size_t total = (size_t)B * Tn * HKV * 8;
  const dim3 grid((unsigned)((total + 255) / 256));
  const int e4 = res_dtype == FFA_DT_FP8_E4M3 ? 1 : 0;
  if (nf4)
    hipLaunchKernelGGL(ffa::kfmt_group_append_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, k, k_dtype, B * Tn,
                       Tn, HKV, pos, block_table, bt_stride, num_pages, k_pages, scale_pages, res_pages, e4, v_new,
                       v_pages);
  else
    hipLaunchKernelGGL(ffa::kfmt_group_append_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, k, k_dtype,
                       B * Tn, Tn, HKV, pos, block_table, bt_stride, num_pages, k_pages, scale_pages, res_pages, e4,
                       v_new, v_pages);
  return launch_status();
}

extern "C" int ffa_nvfp4_g16_append(const void *k, int k_dtype, int B, int Tn, int HKV, const int32_t *pos,
                                    const int32_t *block_table, int bt_stride, int num_pages, uint8_t *k_pages,
                                    uint8_t *scale_pages, uint8_t *res_pages, int res_dtype, const void *v_new,
                                    void *v_pages, void *stream) {
  return group_append(false, k, k_dtype, B, Tn, HKV, pos, block_table, bt_stride, num_pages, k_pages, scale_pages,
                      res_pages, res_dtype, v_new, v_pages, stream);
}

extern "C" int ffa_nf4_g64_append(const void *k, int k_dtype, int B, int Tn, int HKV, const int32_t *pos,
                                  const int32_t *block_table, int bt_stride, int num_pages, uint8_t *k_pages,
                                  void *scale_pages, uint8_t *res_pages, int res_dtype, const void *v_new,
                                  void *v_pages, void *stream) {
  return group_append(true, k, k_dtype, B, Tn, HKV, pos, block_table, bt_stride, num_pages, k_pages, scale_pages,
                      res_pages, res_dtype, v_new, v_pages, stream);
}
