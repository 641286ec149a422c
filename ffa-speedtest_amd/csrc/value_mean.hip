// Mean over tokens of V: the value that the mean-V fallback gives the softmax mass of pruned blocks
// (ffa-q2fp8-meanv/attn_kernel/attn_kernel_v1210_meanv_bsz_q2fp8.py:332,
// v.mean(dim=1, dtype=float32).to(v.dtype)).
//
// Two launches, no atomics (the result does not depend on scheduling):
//   * partial sums: workgroup (split s, sequence b, KV head) sums tokens [s * span, (s + 1) * span)
//     of its sequence in fp32 into partial[b, hkv, s, 128];
//   * finalize: one workgroup per (b, KV head) adds the splits in order, divides by the length and
//     rounds once to the output type.
// The contiguous layout reads one 256-byte token row per 16 lanes (16-byte loads); the paged layout
// reads whole V^T page blocks (16 KB, every lane 16-byte pieces of 8 tokens of one column).
#include "decode_common.h"
#include "ffa_mi355x.h"

namespace ffa {

constexpr int kMeanThreads = 256;
constexpr int kMeanMinSpan = 512;   // tokens per split at least
constexpr int kMeanMaxSplits = 256;

__device__ __forceinline__ void add8_16bit(float *acc, uint4 w, bool bf16) {
  const uint32_t x[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (bf16) {
      acc[2 * e] += __uint_as_float(x[e] << 16);
      acc[2 * e + 1] += __uint_as_float(x[e] & 0xffff0000u);
    } else {
      acc[2 * e] += f16_bits_to_f32(x[e] & 0xffffu);
      acc[2 * e + 1] += f16_bits_to_f32(x[e] >> 16);
    }
  }
}

// v [B, T, HKV, 128]: thread (r, cg) adds the 8 columns 8 cg .. 8 cg + 7 of tokens t0 + r, + 16, ...
__global__ __launch_bounds__(kMeanThreads) void vmean_partial_contig(const uint16_t *v, int bf16,
                                                                     const int32_t *seq_lens, int T, int HKV,
                                                                     int span, float *part, int nsplit) {
  const int s = blockIdx.x, bh = blockIdx.y;
  const int b = bh / HKV, hkv = bh - b * HKV;
  const int Tb = seq_lens ? min(max(seq_lens[b], 0), T) : T;
  const int t0 = s * span, t1 = min(t0 + span, Tb);
  const int r = threadIdx.x >> 4, cg = threadIdx.x & 15;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const uint16_t *row0 = v + ((size_t)b * T * HKV + hkv) * kD + 8 * cg;
  const size_t stride = (size_t)HKV * kD;
  for (int t = t0 + r; t < t1; t += 64) {  // four token rows in flight per thread
    uint4 w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int tt = t + 16 * u;
      w[u] = tt < t1 ? *(const uint4 *)(row0 + (size_t)tt * stride) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) add8_16bit(acc, w[u], bf16 != 0);
  }
  __shared__ float s_red[16][kD + 4];
#pragma unroll
  for (int e = 0; e < 8; ++e) s_red[r][8 * cg + e] = acc[e];
  __syncthreads();
  if (threadIdx.x < kD) {
    const int c = threadIdx.x;
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) sum += s_red[k][c];
    part[((size_t)bh * nsplit + s) * kD + c] = sum;
  }
}

// V^T pages [P, HKV, 128, 64] (vt_off order): 16-byte unit U of a page block holds tokens
// 8 g8 .. 8 g8 + 7 of column c, with c = 16 (U >> 7) + (U & 15) and g8 = 2 ((U >> 4) & 3) +
// ((U >> 6) & 1).  Thread th reads units th + 256 i (i = 0..3): the same 8 tokens of four columns
// 16 (th >> 7) + 32 i + (th & 15) in every page.
__global__ __launch_bounds__(kMeanThreads) void vmean_partial_paged(const uint16_t *v, int bf16, const int32_t *bt,
                                                                    int bt_stride, int num_pages,
                                                                    const int32_t *seq_lens, int T, int HKV,
                                                                    int span, float *part, int nsplit) {
  const int s = blockIdx.x, bh = blockIdx.y;
  const int b = bh / HKV, hkv = bh - b * HKV;
  const int Tb = seq_lens ? min(max(seq_lens[b], 0), T) : T;
  const int t0 = s * span, t1 = min(t0 + span, Tb);
  const int th = threadIdx.x;
  const int g8 = 2 * ((th >> 4) & 3) + ((th >> 6) & 1);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int pt = t0; pt < t1; pt += kPage) {  // span is a multiple of 64: pt is a page start
    int page = bt[(size_t)b * bt_stride + pt / kPage];
    page = (unsigned)page < (unsigned)num_pages ? page : 0;  // the decode's rule for ids outside the pool
    const int nv = min(t1 - pt, kPage) - 8 * g8;              // valid tokens of this thread's 8
    const uint4 *blk = (const uint4 *)(v + ((size_t)page * HKV + hkv) * (kD * kPage));
    uint4 w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = nv > 0 ? blk[th + kMeanThreads * i] : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      add8_16bit(x, w[i], bf16 != 0);
      float sum8 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) sum8 += e < nv ? x[e] : 0.f;
      acc[i] += sum8;
    }
  }
  __shared__ float s_red[4][kMeanThreads];
#pragma unroll
  for (int i = 0; i < 4; ++i) s_red[i][th] = acc[i];
  __syncthreads();
  if (th < kD) {
    const int c = th, q = c >> 4;
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) sum += s_red[q >> 1][((q & 1) << 7) | (k << 4) | (c & 15)];
    part[((size_t)bh * nsplit + s) * kD + c] = sum;
  }
}

__global__ __launch_bounds__(kD) void vmean_finalize(const float *part, int nsplit, const int32_t *seq_lens, int T,
                                                     int HKV, void *out, int out_dtype) {
  const int bh = blockIdx.x, b = bh / HKV, c = threadIdx.x;
  const int Tb = seq_lens ? min(max(seq_lens[b], 0), T) : T;
  float sum = 0.f;
  for (int s = 0; s < nsplit; ++s) sum += part[((size_t)bh * nsplit + s) * kD + c];
  store_any(out, (size_t)bh * kD + c, out_dtype, Tb > 0 ? sum / (float)Tb : 0.f);
}

}  // namespace ffa

extern "C" __attribute__((visibility("hidden"))) int ffa_set_error_internal(int code, const char *msg);

extern "C" int ffa_v_mean_nsplit(int T) {
  if (T <= 0) return 0;
  const int n = (T + ffa::kMeanMinSpan - 1) / ffa::kMeanMinSpan;
  return n < ffa::kMeanMaxSplits ? n : ffa::kMeanMaxSplits;
}

extern "C" int ffa_v_mean(const void *v, int v_dtype, int layout, const int32_t *block_table, int bt_stride,
                          int num_pages, const int32_t *seq_lens, int B, int T, int HKV, float *partial, int nsplit,
                          void *out, int out_dtype, void *stream) {
  if (!v || !out || !partial) return ffa_set_error_internal(FFA_E_INVALID, "null pointer");
  if (B <= 0 || T <= 0 || HKV <= 0) return ffa_set_error_internal(FFA_E_INVALID, "bad dims");
  if (B > 65535 || (long)B * HKV > 65535) return ffa_set_error_internal(FFA_E_UNSUPPORTED, "B * HKV above 65535");
  if (!(v_dtype == FFA_DT_F16 || v_dtype == FFA_DT_BF16)) return ffa_set_error_internal(FFA_E_INVALID, "v dtype");
  if (!(out_dtype >= FFA_DT_F16 && out_dtype <= FFA_DT_F32)) return ffa_set_error_internal(FFA_E_INVALID, "out dtype");
  const int need = ffa_v_mean_nsplit(T);
  if (nsplit < need) return ffa_set_error_internal(FFA_E_INVALID, "partial holds fewer than ffa_v_mean_nsplit(T) splits");
  // every split but the last covers `span` tokens, a multiple of the page
  const int per = (T + need - 1) / need;
  const int span = (per + ffa::kPage - 1) / ffa::kPage * ffa::kPage;
  const int used = (T + span - 1) / span;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)used, (unsigned)(B * HKV));
  if (layout == FFA_LAYOUT_PAGED) {
    if (!block_table || num_pages <= 0) return ffa_set_error_internal(FFA_E_INVALID, "paged layout needs a block table and pool");
    if ((long)bt_stride * ffa::kPage < T) return ffa_set_error_internal(FFA_E_INVALID, "block table has fewer than ceil(T/64) columns");
    hipLaunchKernelGGL(ffa::vmean_partial_paged, grid, dim3(ffa::kMeanThreads), 0, st, (const uint16_t *)v,
                       v_dtype == FFA_DT_BF16 ? 1 : 0, block_table, bt_stride, num_pages, seq_lens, T, HKV, span,
                       partial, used);
  } else if (layout == FFA_LAYOUT_CONTIG) {
    hipLaunchKernelGGL(ffa::vmean_partial_contig, grid, dim3(ffa::kMeanThreads), 0, st, (const uint16_t *)v,
                       v_dtype == FFA_DT_BF16 ? 1 : 0, seq_lens, T, HKV, span, partial, used);
  } else {
    return ffa_set_error_internal(FFA_E_INVALID, "layout");
  }
  const hipError_t e1 = hipGetLastError();  // the finalize pass would read partials never written
  if (e1 != hipSuccess) return ffa_set_error_internal(FFA_E_LAUNCH, hipGetErrorString(e1));
  hipLaunchKernelGGL(ffa::vmean_finalize, dim3((unsigned)(B * HKV)), dim3(ffa::kD), 0, st, partial, used, seq_lens, T,
                     HKV, out, out_dtype);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return ffa_set_error_internal(FFA_E_LAUNCH, hipGetErrorString(e));
  return FFA_OK;
}
