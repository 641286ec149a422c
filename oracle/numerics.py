"""Bit-level number formats for the CPU oracle (numpy only).

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this package, and only as the checker.

The reference computes with torch dtypes (bf16, fp16, float8_e4m3fn,
float8_e5m2).  numpy has float16 but no bf16/fp8, so those roundings are
written here from the IEEE-754 / OCP-FP8 definitions:

* bf16: round-to-nearest-even of the fp32 bit pattern, NaN kept quiet.
* fp8 e4m3fn (OCP): 4 exponent bits (bias 7), 3 mantissa bits, no inf;
  0x7F/0xFF are NaN, max finite 448.  A finite input whose RNE result would
  exceed 448 becomes NaN (this is what torch's float->float8_e4m3fn cast
  does; pinned by tests/test_oracle_numerics.py against torch).
* fp8 e5m2: 5 exponent bits (bias 15), 2 mantissa bits, inf/NaN like
  IEEE; an RNE result above 57344 becomes +-inf.

The reference's residual cast `(k.to(float32) - k_dequant).to(fp8_dtype)`
(ffa-q2fp8/run_attn_bench_q2.py:88) is exactly `fp8_encode(x_f32)` here.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32

# ----------------------------------------------------------------------------
# bf16 / fp16 / fp32 "tau" roundings.  Values are carried as float32 arrays
# whose elements are exactly representable in the named dtype.
# ----------------------------------------------------------------------------


def f32_to_bf16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=F32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) & 0xFFFF
    nan = np.isnan(x)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(F32)


def round_bf16(x) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def round_f16(x) -> np.ndarray:
    return np.asarray(x, dtype=F32).astype(np.float16).astype(F32)


def round_to(x, dtype: str) -> np.ndarray:
    """Round float32 values to `dtype` in {'fp32','fp16','bf16'} (RNE)."""
    x = np.asarray(x, dtype=F32)
    if dtype == "fp32":
        return x
    if dtype == "fp16":
        return round_f16(x)
    if dtype == "bf16":
        return round_bf16(x)
    raise ValueError(f"unknown dtype {dtype}")


# ----------------------------------------------------------------------------
# fp8
# ----------------------------------------------------------------------------

_FP8 = {
    # name: (exp_bits, man_bits, bias, max_finite, has_inf)
    "e4m3fn": (4, 3, 7, 448.0, False),
    "e5m2": (5, 2, 15, 57344.0, True),
}


def _fp8_decode_table(fmt: str) -> np.ndarray:
    eb, mb, bias, _, has_inf = _FP8[fmt]
    out = np.empty(256, dtype=np.float64)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> mb) & ((1 << eb) - 1)
        m = b & ((1 << mb) - 1)
        if has_inf and e == (1 << eb) - 1:
            out[b] = s * np.inf if m == 0 else np.nan
        elif (not has_inf) and (b & 0x7F) == 0x7F:
            out[b] = np.nan
        elif e == 0:
            out[b] = s * m * 2.0 ** (1 - bias - mb)
        else:
            out[b] = s * (1.0 + m / (1 << mb)) * 2.0 ** (e - bias)
    return out.astype(F32)


FP8_DECODE = {fmt: _fp8_decode_table(fmt) for fmt in _FP8}


def fp8_decode(b, fmt: str) -> np.ndarray:
    """uint8 fp8 codes -> float32 values (exact)."""
    return FP8_DECODE[fmt][np.asarray(b, dtype=np.uint8)]


def fp8_encode(x, fmt: str) -> np.ndarray:
    """float32 -> fp8 code (uint8), round-to-nearest-even."""
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        return _fp8_encode(x, fmt)


def _fp8_encode(x, fmt: str) -> np.ndarray:
    eb, mb, bias, maxf, has_inf = _FP8[fmt]
    x = np.asarray(x, dtype=F32).astype(np.float64)
    sign = np.signbit(x)
    a = np.abs(x)
    nan = np.isnan(a)
    inf = np.isinf(a)
    a = np.where(nan | inf, 0.0, a)
    emin = 1 - bias  # exponent of the smallest normal
    # a = m * 2^e with m in [0.5, 1): the binade of a is 2^(e-1)
    _, e = np.frexp(a)
    e = np.maximum(e - 1, emin)
    r = np.ldexp(np.rint(np.ldexp(a, mb - e)), e - mb)  # RNE to mb mantissa bits (exact in float64)
    over = (r > maxf) | inf
    r = np.where(over, 0.0, r)
    _, er = np.frexp(r)
    er = er - 1
    normal = r >= 2.0 ** emin
    m_norm = np.ldexp(r, mb - er) - (1 << mb)  # integer mantissa field
    bits_norm = ((er + bias).astype(np.int64) << mb) | m_norm.astype(np.int64)
    bits_sub = np.ldexp(r, mb - emin).astype(np.int64)
    bits = np.where(normal, bits_norm, bits_sub)
    if has_inf:
        bits = np.where(over, (((1 << eb) - 1) << mb), bits)
        bits = np.where(nan, 0x7F, bits)
    else:
        bits = np.where(over | nan, 0x7F, bits)
    bits = bits | np.where(sign, 0x80, 0)
    return bits.astype(np.uint8)


FP8_FORMATS = ("e4m3fn", "e5m2")
