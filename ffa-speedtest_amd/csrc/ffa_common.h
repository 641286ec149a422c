// Shared device helpers for the gfx950 kernels of this library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ffa {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// scalar conversions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  // round-to-nearest-even, NaN kept quiet (same rule as torch's bf16 cast)
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// fp16(a) in the low half and fp16(b) in the high half, each rounded to nearest even as
// f32_to_f16_bits rounds it: gfx950 converts the pair with one v_cvt_pk_f16_f32 (two conversions,
// a shift and an OR otherwise)
__device__ __forceinline__ uint32_t pk_f16_bits(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
}

// load element i of a float tensor of runtime dtype (0=f16, 1=bf16, 2=f32)
__device__ __forceinline__ float load_any(const void *p, size_t i, int dt) {
  if (dt == 2) return ((const float *)p)[i];
  uint32_t b = ((const uint16_t *)p)[i];
  return dt == 1 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

__device__ __forceinline__ void store_any(void *p, size_t i, int dt, float v) {
  if (dt == 2) {
    ((float *)p)[i] = v;
  } else if (dt == 1) {
    ((uint16_t *)p)[i] = (uint16_t)f32_to_bf16_bits(v);
  } else {
    ((uint16_t *)p)[i] = (uint16_t)f32_to_f16_bits(v);
  }
}

// round a float to the given float dtype and back (0=f16, 1=bf16, 2=f32)
__device__ __forceinline__ float round_to(float v, int dt) {
  if (dt == 2) return v;
  if (dt == 1) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  return (float)(_Float16)v;
}

// ---------------------------------------------------------------------------
// fp8 (OCP e4m3fn / e5m2) encode with torch's rules: RNE, e4m3fn overflow -> NaN,
// e5m2 overflow -> inf.  Written from the format definitions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t f32_to_fp8(float x, int e4m3) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  const int mbits = e4m3 ? 3 : 2;
  const int bias = e4m3 ? 7 : 15;
  const int emin = 1 - bias;  // smallest normal exponent
  if (a > 0x7f800000u) return sign | 0x7fu;  // NaN
  if (a == 0x7f800000u) return e4m3 ? (sign | 0x7fu) : (sign | 0x7cu);
  const int e = (int)(a >> 23) - 127;  // unbiased exponent of the input (normal inputs)
  uint32_t bits;
  if (a < 0x00800000u || e < emin) {
    // result is subnormal (or zero) in fp8: a multiple of the quantum 2^(emin - mbits),
    // rounded to nearest even in units of the quantum
    const float q = __uint_as_float((uint32_t)(127 + emin - mbits) << 23);  // 2^(emin-mbits)
    const float r = __uint_as_float(a) / q;                                 // exact (power of 2)
    const float ri = __builtin_rintf(r);                                    // RNE
    bits = (uint32_t)ri;  // may equal 1 << mbits => smallest normal, encodes correctly
  } else {
    // normal: keep mbits of mantissa with RNE
    const uint32_t shift = 23 - mbits;
    uint32_t mant = a & 0x7fffffu;
    uint32_t keep = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    uint32_t exp8 = (uint32_t)(e + bias);
    if (rem > half || (rem == half && (keep & 1u))) {
      keep += 1;
      if (keep == (1u << mbits)) {
        keep = 0;
        exp8 += 1;
      }
    }
    bits = (exp8 << mbits) | keep;
  }
  if (e4m3) {
    if (bits > 0x7eu) return sign | 0x7fu;  // beyond 448 -> NaN
  } else {
    if (bits > 0x7bu) return sign | 0x7cu;  // beyond 57344 -> inf
  }
  return sign | bits;
}

// ---------------------------------------------------------------------------
// lane exchange
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
constexpr int kRowRor4 = 0x124;
constexpr int kRowRor8 = 0x128;

// Lane i combined with lane i ^ m.  For m = 16 and 32 a single register-to-register exchange:
// v_permlane16_swap / v_permlane32_swap (gfx950) of x with itself leaves x_i in one result and
// x_(i^m) in the other; other distances go through __shfl_xor (an LDS-pipe permute).
template <int M>
__device__ __forceinline__ void xor_pair(float x, float &a, float &b) {
  if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  } else if constexpr (M == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  } else {
    a = x;
    b = __shfl_xor(x, M);
  }
}
__device__ __forceinline__ float xor_max(float x, int m) {
  float a, b;
  if (m == 16) xor_pair<16>(x, a, b);
  else if (m == 32) xor_pair<32>(x, a, b);
  else { a = x; b = __shfl_xor(x, m); }
  return fmaxf(a, b);
}
__device__ __forceinline__ float xor_sum(float x, int m) {
  float a, b;
  if (m == 16) xor_pair<16>(x, a, b);
  else if (m == 32) xor_pair<32>(x, a, b);
  else { a = x; b = __shfl_xor(x, m); }
  return a + b;
}

// Whole-wave max / sum with register-to-register exchanges: lane i with i ^ 32 and i ^ 16,
// then DPP row rotations by 8, 4, 2, 1 inside each 16-lane row.  Every lane ends with the
// result.
constexpr int kRowRor1 = 0x121;
constexpr int kRowRor2 = 0x122;
__device__ __forceinline__ float wave_max(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto c = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(c[0]), __uint_as_float(c[1]));
  x = fmaxf(x, dpp<kRowRor8>(x));
  x = fmaxf(x, dpp<kRowRor4>(x));
  x = fmaxf(x, dpp<kRowRor2>(x));
  return fmaxf(x, dpp<kRowRor1>(x));
}
__device__ __forceinline__ float wave_sum(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto c = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(c[0]) + __uint_as_float(c[1]);
  x += dpp<kRowRor8>(x);
  x += dpp<kRowRor4>(x);
  x += dpp<kRowRor2>(x);
  return x + dpp<kRowRor1>(x);
}
// lane i + lane (i ^ 32), for every lane
__device__ __forceinline__ float swap32_sum(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}

// Raw buffer resource over [base, base + bytes) (gfx9 word 3: 32-bit data format, no
// swizzle).  A load at an offset past `bytes` returns zeros without a memory access, so a
// load group can be issued on every path with its validity carried by the size; the
// compiler then counts outstanding loads exactly and waits for one group at a time.
typedef __amdgpu_buffer_rsrc_t brsrc;
__device__ __forceinline__ brsrc make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bload16(brsrc r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t bload4(brsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint2 bload8(brsrc r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint64_t bload8u(brsrc r, uint32_t off) {
  const uint2 v = bload8(r, off);
  return ((uint64_t)v.y << 32) | v.x;
}
// The same loads with the non-temporal hint (cache-policy bit 1, `nt` on gfx950), for data one
// workgroup reads once in whole cache lines per load: the paged (page, KV head) blocks of codes,
// scales, residual and V, and the contiguous layouts' V rows.  Data that several workgroups read
// keeps the default policy: q, probe windows, page ids, and the reference layout's code rows, whose
// cache lines hold several KV heads' codes; so do the other-format decoder's contiguous residual
// rows, which a wave reads in two loads of alternate 16-byte pieces of each line (with the hint, a
// load-only probe of config 1's reads took 4.55 against 4.10 us; the q2 decoder's contiguous
// residual, read for about a tenth of the chunks at config 2, measured 0.15 us slower without it).
constexpr int kNonTemporal = 2;
__device__ __forceinline__ uint4 bload16_nt(brsrc r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kNonTemporal);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 bload8_nt(brsrc r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, kNonTemporal);
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint64_t bload8u_nt(brsrc r, uint32_t off) {
  const uint2 v = bload8_nt(r, off);
  return ((uint64_t)v.y << 32) | v.x;
}

}  // namespace ffa
