"""CPU restatement of the other K formats' quantizers and dequantizers (numpy).

TEST INFRASTRUCTURE.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker.

Every format's decode is the q2fp8 decode with a different dequantized K:
`k_hat = fp16(f32(value) * f32(scale))`, then the same probe threshold, group
prune, refine `fp16(k_hat + fp16(res))`, exp2 softmax and merge
(q2fp8.decode(khat=...)).  What each function restates (paths relative to the
reference checkout):

* quantize_fp8fp8   ffa-fp8fp8/fused_kproj_rope_fp8fp8.py:58-64
* khat_fp8          ffa-fp8fp8/attn_kernel/attn_kernel_v1210_fused_bsz_fp8fp8.py:87-90 (fp8 -> fp16, exact)
* quantize_fp8_scaled / khat_fp8_scaled
                    per-token variant (no reference counterpart): e4m3 with one fp16
                    scale per token and KV head, fp16(amax / 448)
* quantize_nvfp4    ffa-nvfp4fp8/fused_kproj_rope_nvfp4fp8.py:62-114 (all arithmetic in k's dtype)
* khat_nvfp4        ffa-nvfp4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nvfp4fp8.py:10-21, 80-81, 123;
                    the second probe window takes the scale of block NTB-1 (:96-97)
* quantize_nf4      ffa-nf4fp8/fused_kproj_rope_nf4fp8.py:72-96 (fp32 arithmetic; the residual uses
                    the fp32 scale, the decode the scale rounded to k's dtype)
* khat_nf4          ffa-nf4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nf4fp8.py:80-81, 93, 121
* quantize_nvfp4_g16 / khat_nvfp4_g16
                    paged nvfp4 mode (no reference counterpart): e2m1 with one e4m3 scale per
                    16 channels of each token, s = e4m3(amax / 6); the codes follow the
                    reference encoder's midpoint rule (bucketize right=True), k_hat = fp16(level * s)
* quantize_nf4_g64 / khat_nf4_g64
                    paged nf4 mode (no reference counterpart): NF4 with one fp16 absmax scale
                    per 64 channels of each token, s = fp16(max(amax, 1e-6)); codes by the
                    reference encoder's rule (clamp to [-1, 1], bucketize right=False),
                    k_hat = fp16(codebook[c] * s)
"""
from __future__ import annotations

import numpy as np

from .numerics import F32, fp8_decode, fp8_encode, round_f16, round_to

FP4_POS_LEVELS = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], F32)  # e2m1 magnitudes
FP4_THRESHOLDS = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], F32)  # midpoints of the levels
# QLoRA NF4 codebook (the 16 published normal-float levels), as fp32
NF4_CODEBOOK = np.array([
    -1.0, -0.6961928009986877, -0.5229921340942383, -0.39491748809814453, -0.28444138169288635,
    -0.18477343022823334, -0.09105003625154495, 0.0, 0.07958029955625534, 0.16093020141124725,
    0.24611230194568634, 0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
    0.7229568362236023, 1.0], F32)


# ----------------------------------------------------------------------------- nibble packing
def pack_4bit(codes: np.ndarray) -> np.ndarray:
    """[..., D] codes 0..15 -> [..., ceil(D/2)] bytes, low nibble first (zero nibble pads odd D)."""
    codes = np.asarray(codes, np.uint8)
    D = codes.shape[-1]
    if D % 2:
        codes = np.concatenate([codes, np.zeros(codes.shape[:-1] + (1,), np.uint8)], axis=-1)
    c = codes.reshape(codes.shape[:-1] + (-1, 2))
    return (c[..., 0] | (c[..., 1] << 4)).astype(np.uint8)


def unpack_4bit(packed: np.ndarray, D: int) -> np.ndarray:
    p = np.asarray(packed, np.uint8)
    out = np.stack([p & 0xF, p >> 4], axis=-1).reshape(p.shape[:-1] + (-1,))
    return out[..., :D]


# ----------------------------------------------------------------------------- fp8 base
def quantize_fp8fp8(k: np.ndarray, fmt: str = "e5m2"):
    """base = fp8(k); residual = fp8(f32(k) - f32(base)).  k holds values of k's dtype (as f32)."""
    k = np.asarray(k, F32)
    base = fp8_encode(k, fmt)
    res = fp8_encode((k - fp8_decode(base, fmt)).astype(F32), fmt)
    return base, res


def khat_fp8(base: np.ndarray, fmt: str) -> np.ndarray:
    return fp8_decode(base, fmt).astype(F32)  # every fp8 value is an fp16 value


def quantize_fp8_scaled(k: np.ndarray, fmt: str = "e4m3fn"):
    """Per-token-scaled fp8: s = max(fp16(max(amax_d |k|, 1e-6) / fmax), 2^-14) per (b, t, h)
    (fmax = 448 for e4m3fn, 57344 for e5m2); base = fp8(k / s); residual = fp8(k - base * s).
    Returns (base u8 [B,T,HKV,D], scale f32 [B,T,HKV], residual u8).

    The floor 2^-14 (the smallest normal fp16) keeps s non-zero for all-zero and tiny rows, and
    keeps k / s within fmax: a subnormal fp16 s can be up to half its quantum (2^-25) below
    amax / fmax, which for amax = 3.5e-5 would give k / s = 587 > 448, a NaN in e4m3fn.  With a
    normal s the rounding is at most 2^-11 relative, so |k / s| <= fmax * (1 + 2^-11), which both
    formats round to fmax."""
    k = np.asarray(k, F32)
    fmax = 448.0 if fmt == "e4m3fn" else 57344.0
    s = round_f16((np.maximum(np.abs(k).max(axis=-1), F32(1e-6)) / F32(fmax)).astype(F32))
    s = np.maximum(s, F32(2.0**-14)).astype(F32)
    base = fp8_encode((k / s[..., None]).astype(F32), fmt)
    deq = (fp8_decode(base, fmt) * s[..., None]).astype(F32)  # exact: 4 x 11 significant bits
    res = fp8_encode((k - deq).astype(F32), fmt)
    return base, s, res


def khat_fp8_scaled(base: np.ndarray, scale: np.ndarray, fmt: str) -> np.ndarray:
    return round_f16((fp8_decode(base, fmt) * np.asarray(scale, F32)[..., None]).astype(F32))


# ----------------------------------------------------------------------------- nvfp4
def fp4_decode(codes: np.ndarray) -> np.ndarray:
    """e2m1 nibble -> value: sign bit 3, exponent bits 1-2 (bias 1), mantissa bit 0, subnormal at e=0."""
    c = np.asarray(codes, np.int64)
    mag = FP4_POS_LEVELS[c & 7]
    return np.where((c >> 3) & 1, -mag, mag).astype(F32)


def quantize_nvfp4(k: np.ndarray, tau: str, fmt: str = "e5m2", page_size: int = 128):
    """Per-(b, page, h) scale over page x D, every op rounded to tau.

    Returns (packed u8 [B,T,HKV,D/2], scale f32 [B,NTB,HKV] (tau values), residual u8 [B,T,HKV,D]).
    """
    k = np.asarray(k, F32)
    B, T, HKV, D = k.shape
    npg = -(-T // page_size)
    kp = np.zeros((B, npg * page_size, HKV, D), F32)
    kp[:, :T] = k
    kb = kp.reshape(B, npg, page_size, HKV, D)
    max_abs = np.abs(kb).max(axis=(2, 4))  # exact in tau
    scale = round_to(max_abs / F32(6.0), tau)
    scale = np.maximum(scale, round_to(np.full_like(scale, 1e-6), tau))  # clamp_min in tau
    sb = scale[:, :, None, :, None]
    ks = round_to(kb / sb, tau)
    idx = np.searchsorted(round_to(FP4_THRESHOLDS, tau), np.abs(ks), side="right")  # bucketize(right=True)
    sign = ks < 0
    codes = (idx | (sign.astype(np.int64) << 3)).astype(np.uint8)
    deq = round_to(np.where(sign, -FP4_POS_LEVELS[idx], FP4_POS_LEVELS[idx]).astype(F32) * sb, tau)
    res = fp8_encode(round_to(kb - deq, tau), fmt)
    codes = codes.reshape(B, npg * page_size, HKV, D)[:, :T]
    res = res.reshape(B, npg * page_size, HKV, D)[:, :T]
    return pack_4bit(codes), scale.astype(F32), res


def khat_nvfp4(packed: np.ndarray, scale: np.ndarray, BS: int, D: int, seq_lens=None):
    """k_hat = fp16(f32(e2m1) * f32(scale[b, t // BS, h])) and the probe variant whose second window
    uses scale[b, NTB_b - 1, h] for every token.  Returns (khat, khat_probe1), each [B, T, HKV, D]."""
    v = fp4_decode(unpack_4bit(packed, D))  # [B, T, HKV, D]
    B, T = v.shape[:2]
    lens = [T] * B if seq_lens is None else [int(x) for x in seq_lens]
    scale = np.asarray(scale, F32)
    tb = np.minimum(np.arange(T) // BS, scale.shape[1] - 1)
    s_tok = scale[:, tb, :]  # [B, T, HKV]
    khat = round_f16((v * s_tok[..., None]).astype(F32))
    s_last = np.stack([scale[b, max(-(-lens[b] // BS) - 1, 0)] for b in range(B)])  # [B, HKV]
    khat_p1 = round_f16((v * s_last[:, None, :, None]).astype(F32))
    return khat, khat_p1


# ----------------------------------------------------------------------------- nf4
def quantize_nf4(k: np.ndarray, tau: str, fmt: str = "e5m2"):
    """Per-(b, h, d) absmax over T in fp32; bucketize on the codebook midpoints (right=False).

    Returns (packed u8 [B,T,HKV,D/2], scale f32 [B,HKV,D] (tau values), residual u8 [B,T,HKV,D]).
    """
    k = np.asarray(k, F32)
    scale = np.maximum(np.abs(k).max(axis=1), F32(1e-6)).astype(F32)  # [B, HKV, D]
    scale_out = round_to(scale, tau)
    norm = np.clip((k / scale[:, None]).astype(F32), NF4_CODEBOOK[0], NF4_CODEBOOK[-1])
    bounds = ((NF4_CODEBOOK[:-1] + NF4_CODEBOOK[1:]).astype(F32) * F32(0.5)).astype(F32)
    idx = np.searchsorted(bounds, norm, side="left")  # bucketize(right=False)
    deq = (NF4_CODEBOOK[idx] * scale[:, None]).astype(F32)
    res = fp8_encode((k - deq).astype(F32), fmt)
    return pack_4bit(idx.astype(np.uint8)), scale_out.astype(F32), res


def khat_nf4(packed: np.ndarray, scale: np.ndarray, D: int) -> np.ndarray:
    """k_hat = fp16(f32(codebook[c]) * f32(scale[b, h, d]))."""
    c = unpack_4bit(packed, D).astype(np.int64)
    return round_f16((NF4_CODEBOOK[c] * np.asarray(scale, F32)[:, None]).astype(F32))


# ----------------------------------------------------------------------------- per-token group scales (paged modes)
def quantize_nvfp4_g16(k: np.ndarray, fmt: str = "e4m3fn"):
    """k [..., 128] (values of k's dtype) -> (packed u8 [..., 64], scale bytes u8 [..., 8] (e4m3),
    residual u8 [..., 128]).  Per 16-channel block: s = e4m3(min(amax / 6, 448)); x = k / s (0 where
    s == 0); code = #{midpoints <= |x|} | sign(x) << 3; residual = fp8(k - (+-level * s))."""
    k = np.asarray(k, F32)
    kb = k.reshape(k.shape[:-1] + (-1, 16))
    amax = np.abs(kb).max(axis=-1)
    sbytes = fp8_encode(np.minimum((amax / F32(6.0)).astype(F32), F32(448.0)), "e4m3fn")
    s = fp8_decode(sbytes, "e4m3fn")[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        x = np.where(s > 0, (kb / s).astype(F32), F32(0.0))
    idx = np.searchsorted(FP4_THRESHOLDS, np.abs(x), side="right")
    neg = x < 0
    deq = (np.where(neg, -FP4_POS_LEVELS[idx], FP4_POS_LEVELS[idx]) * s).astype(F32)  # exact
    res = fp8_encode((kb - deq).astype(F32), fmt).reshape(k.shape)
    codes = (idx | (neg.astype(np.int64) << 3)).astype(np.uint8).reshape(k.shape)
    return pack_4bit(codes), sbytes.astype(np.uint8), res


def khat_nvfp4_g16(packed: np.ndarray, sbytes: np.ndarray) -> np.ndarray:
    """k_hat = fp16(f32(e2m1) * f32(e4m3 scale of the channel's 16-block)) -- exact (<= 5 significant bits)."""
    v = fp4_decode(unpack_4bit(packed, 2 * np.asarray(packed).shape[-1]))
    s = np.repeat(fp8_decode(sbytes, "e4m3fn"), 16, axis=-1)
    return round_f16((v * s).astype(F32))


def quantize_nf4_g64(k: np.ndarray, fmt: str = "e4m3fn"):
    """k [..., 128] -> (packed u8 [..., 64], scale f32 [..., 2] (fp16 values), residual u8 [..., 128]).
    Per 64-channel block: s = fp16(max(amax, 1e-6)); x = clamp(k / s, -1, 1);
    code = #{codebook midpoints < x}; residual = fp8(k - codebook[code] * s)."""
    k = np.asarray(k, F32)
    kb = k.reshape(k.shape[:-1] + (-1, 64))
    s = round_f16(np.maximum(np.abs(kb).max(axis=-1), F32(1e-6)).astype(F32))  # [..., 2]
    x = np.clip((kb / s[..., None]).astype(F32), F32(-1.0), F32(1.0))
    bounds = ((NF4_CODEBOOK[:-1] + NF4_CODEBOOK[1:]).astype(F32) * F32(0.5)).astype(F32)
    idx = np.searchsorted(bounds, x, side="left")
    deq = (NF4_CODEBOOK[idx] * s[..., None]).astype(F32)
    res = fp8_encode((kb - deq).astype(F32), fmt).reshape(k.shape)
    return pack_4bit(idx.astype(np.uint8).reshape(k.shape)), s.astype(F32), res


def khat_nf4_g64(packed: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """k_hat = fp16(f32(codebook[c]) * f32(fp16 scale of the channel's 64-block))."""
    c = unpack_4bit(packed, 2 * np.asarray(packed).shape[-1]).astype(np.int64)
    s = np.repeat(np.asarray(scale, F32), 64, axis=-1)
    return round_f16((NF4_CODEBOOK[c] * s).astype(F32))
