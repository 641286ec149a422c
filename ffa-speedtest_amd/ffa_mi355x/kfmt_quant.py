"""Host side of the fp8 / nvfp4 / nf4 K quantizers and the shared K-proj + RoPE kernel.

Each function launches HIP kernels through the C ABI (include/ffa_mi355x.h) and returns
tensors in the reference's layouts:
  quantize_fp8fp8  ffa-fp8fp8/fused_kproj_rope_fp8fp8.py:58-64
  encode_nvfp4     ffa-nvfp4fp8/fused_kproj_rope_nvfp4fp8.py:62-114
  encode_nf4       ffa-nf4fp8/fused_kproj_rope_nf4fp8.py:72-96
  kproj_rope       F.linear + apply_rope of every producer (e.g. ffa-nf4fp8/fused_kproj_rope_nf4fp8.py:428-436)
"""
from __future__ import annotations

import torch

from . import _native as N
from .quant import _normalize_k_weight

_FP8 = (torch.float8_e4m3fn, torch.float8_e5m2)


def _check_k(k: torch.Tensor, fp8_dtype) -> torch.Tensor:
    if not k.is_cuda:
        raise ValueError("k must be a CUDA tensor")
    if fp8_dtype not in _FP8:
        raise NotImplementedError(f"fp8_dtype must be float8_e4m3fn or float8_e5m2, got {fp8_dtype}")
    if k.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"k must be fp16, bf16 or fp32, got {k.dtype}")
    return k.contiguous()


def quantize_fp8fp8(k: torch.Tensor, fp8_dtype=torch.float8_e5m2):
    """(base, residual): base = fp8(k), residual = fp8(f32(k) - f32(base)), both shaped like k."""
    k = _check_k(k, fp8_dtype)
    base = torch.empty(k.shape, dtype=fp8_dtype, device=k.device)
    res = torch.empty(k.shape, dtype=fp8_dtype, device=k.device)
    rc = N.lib().ffa_fp8fp8_quantize(k.data_ptr(), N.dtype_code(k.dtype), k.numel(), base.data_ptr(), res.data_ptr(),
                                     N.dtype_code(fp8_dtype), N.stream_of(k.device))
    N.check(rc, "ffa_fp8fp8_quantize")
    return base, res


def quantize_fp8_scaled(k: torch.Tensor, fp8_dtype=torch.float8_e4m3fn):
    """k [..., D] -> (base fp8 [..., D], scale fp16 [...], residual fp8 [..., D]) with one fp16 scale per
    row (token and KV head): s = fp16(max(amax, 1e-6) / fmax), base = fp8(k / s), residual = fp8(k - base * s)."""
    k = _check_k(k, fp8_dtype)
    D = k.shape[-1]
    rows = k.numel() // D if D else 0
    base = torch.empty(k.shape, dtype=fp8_dtype, device=k.device)
    res = torch.empty(k.shape, dtype=fp8_dtype, device=k.device)
    scale = torch.empty(k.shape[:-1], dtype=torch.float16, device=k.device)
    rc = N.lib().ffa_fp8_scaled_quantize(k.data_ptr(), N.dtype_code(k.dtype), rows, D, base.data_ptr(),
                                         scale.data_ptr(), res.data_ptr(), N.dtype_code(fp8_dtype),
                                         N.stream_of(k.device))
    N.check(rc, "ffa_fp8_scaled_quantize")
    return base, scale, res


def encode_nvfp4(k: torch.Tensor, fp8_dtype, page_size: int):
    """(packed [B,T,HKV,ceil(D/2)] u8, scale [B,ceil(T/page),HKV] in k.dtype, residual [B,T,HKV,D] fp8)."""
    k = _check_k(k, fp8_dtype)
    if k.ndim != 4:
        raise ValueError(f"k must be [B, T, HKV, D], got {tuple(k.shape)}")
    B, T, HKV, D = k.shape
    page_size = int(page_size)
    if page_size <= 0:
        raise ValueError("page_size must be positive")
    npg = -(-T // page_size)
    dev = k.device
    packed = torch.empty((B, T, HKV, (D + 1) // 2), dtype=torch.uint8, device=dev)
    scale = torch.empty((B, npg, HKV), dtype=k.dtype, device=dev)
    res = torch.empty((B, T, HKV, D), dtype=fp8_dtype, device=dev)
    rc = N.lib().ffa_nvfp4_quantize(k.data_ptr(), N.dtype_code(k.dtype), B, T, HKV, D, page_size, packed.data_ptr(),
                                    scale.data_ptr(), res.data_ptr(), N.dtype_code(fp8_dtype), N.stream_of(dev))
    N.check(rc, "ffa_nvfp4_quantize")
    return packed, scale, res


def encode_nf4(k: torch.Tensor, fp8_dtype):
    """(packed [B,T,HKV,ceil(D/2)] u8, scale [B,HKV,D] in k.dtype, residual [B,T,HKV,D] fp8)."""
    k = _check_k(k, fp8_dtype)
    if k.ndim != 4:
        raise ValueError(f"k must be [B, T, HKV, D], got {tuple(k.shape)}")
    B, T, HKV, D = k.shape
    dev = k.device
    L = N.lib()
    nsplit = L.ffa_nf4_quantize_nsplit(T)
    packed = torch.empty((B, T, HKV, (D + 1) // 2), dtype=torch.uint8, device=dev)
    scale = torch.empty((B, HKV, D), dtype=k.dtype, device=dev)
    res = torch.empty((B, T, HKV, D), dtype=fp8_dtype, device=dev)
    absmax = torch.empty((B, nsplit, HKV * D), dtype=torch.float32, device=dev)
    rc = L.ffa_nf4_quantize(k.data_ptr(), N.dtype_code(k.dtype), B, T, HKV, D, packed.data_ptr(), scale.data_ptr(),
                            res.data_ptr(), N.dtype_code(fp8_dtype), absmax.data_ptr(), N.stream_of(dev))
    N.check(rc, "ffa_nf4_quantize")
    return packed, scale, res


def kproj_rope(h, w_k, cos, sin, num_kv_heads, head_dim, bias=None):
    """RoPE(h W_k^T + b) as [B, T, HKV, D] in the promoted dtype of h and cos (one MFMA GEMM pass)."""
    if not h.is_cuda:
        raise ValueError("kernel requires CUDA tensors.")
    if head_dim % 2 != 0:
        raise ValueError(f"head_dim must be even for RoPE, got {head_dim}")
    w_k = _normalize_k_weight(w_k, h.shape[-1]).to(h.dtype).contiguous()
    B, T, H = h.shape
    HKV, D = int(num_kv_heads), int(head_dim)
    if w_k.shape[0] != HKV * D:
        raise ValueError(f"w_k out_dim mismatch: got {w_k.shape[0]}, expected {HKV * D}")
    if bias is not None and bias.numel() != HKV * D:
        raise ValueError(f"bias length mismatch: got {bias.numel()}, expected {HKV * D}")
    if cos.dtype not in (torch.float32, h.dtype):
        cos, sin = cos.float(), sin.float()
    odt = torch.float32 if cos.dtype == torch.float32 else h.dtype
    h, cos, sin = h.contiguous(), cos.contiguous(), sin.contiguous()
    bias = bias.to(h.dtype).contiguous() if bias is not None else None
    k = torch.empty((B, T, HKV, D), dtype=odt, device=h.device)
    rc = N.lib().ffa_kproj_rope(h.data_ptr(), w_k.data_ptr(), N.ptr(bias), N.dtype_code(h.dtype), cos.data_ptr(),
                                sin.data_ptr(), N.dtype_code(cos.dtype), B, T, H, HKV, D, k.data_ptr(),
                                N.stream_of(h.device))
    N.check(rc, "ffa_kproj_rope")
    return k
