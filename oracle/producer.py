"""CPU restatement of the K producers (numpy).

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker.

* kproj_rope   ffa-q2fp8/fused_kproj_rope_q2fp8.py:402-424 (F.linear + apply_rope),
               with RoPE as at :26-37 (interleaved pairs, cos/sin indexed by d).
               The GEMM is accumulated exactly (float64) and rounded once to
               fp32 and then to the dtype of h; the kernels accumulate in fp32
               in their own order, so the GEMM part is compared with a
               tolerance and the quantization part bit-exactly.
"""
from __future__ import annotations

import numpy as np

from .numerics import F32, round_to


def promote(h_dtype: str, cs_dtype: str) -> str:
    if "fp32" in (h_dtype, cs_dtype):
        return "fp32"
    if h_dtype != cs_dtype:
        raise ValueError("mixed fp16/bf16 promotion is not used by the reference")
    return h_dtype


def linear(h: np.ndarray, w: np.ndarray, bias, h_dtype: str) -> np.ndarray:
    """F.linear(h, w, bias) in h_dtype: exact accumulation, one rounding."""
    acc = h.astype(np.float64) @ w.astype(np.float64).T
    if bias is not None:
        acc = acc + bias.astype(np.float64)
    return round_to(acc.astype(F32), h_dtype)


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, odt: str) -> np.ndarray:
    """x [..., D]; cos/sin broadcastable to x.  out = tau(tau(x*cos) + tau(rot(x)*sin))."""
    rot = np.empty_like(x)
    rot[..., 0::2] = -x[..., 1::2]
    rot[..., 1::2] = x[..., 0::2]
    t1 = round_to((x * cos).astype(F32), odt)
    t2 = round_to((rot * sin).astype(F32), odt)
    return round_to((t1 + t2).astype(F32), odt)


def kproj_rope(h, w, cos, sin, HKV: int, D: int, bias=None, h_dtype="bf16", cs_dtype="fp32"):
    """h [B, T, H], w [HKV*D, H], cos/sin [T, D] -> rotated K [B, T, HKV, D] (promoted dtype)."""
    B, T, _ = h.shape
    odt = promote(h_dtype, cs_dtype)
    k = linear(h, w, bias, h_dtype).reshape(B, T, HKV, D)
    return apply_rope(k, cos[None, :, None, :], sin[None, :, None, :], odt), odt


def kproj_rope_rows(h, w, cos_rows, sin_rows, HKV: int, bias=None, h_dtype="bf16"):
    """Append form: h [B, Tn, H], cos/sin rows [B, Tn, 128] fp32 -> K [B, Tn, HKV, 128] fp32."""
    B, Tn, _ = h.shape
    k = linear(h, w, bias, h_dtype).reshape(B, Tn, HKV, 128)
    return apply_rope(k, cos_rows[:, :, None, :], sin_rows[:, :, None, :], "fp32")
