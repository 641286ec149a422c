"""Drop-in for ffa-q2fp8/fused_kproj_rope_q2fp8.py on MI355X (no Triton).

Same names and signatures:
  build_rope_cache, rotate_half, apply_rope             (reference :10-37, torch host helpers)
  quantize_k_2bit_fp8_residual                          (:40-68)   -> HIP quantizer, bit-exact
  kproj_rope_quantize_reference                         (:402-424) -> torch GEMM + RoPE, HIP quantizer
  kproj_rope_quantize_triton / kproj_rope_quantize_fused (:427-566) -> one fused HIP GEMM+RoPE pass
                                                          + HIP quantizer (tuning kwargs accepted, ignored)
  run_smoke_test, parse_args, main  (entry names of :569-664; the check is ffa_mi355x.producer_check)
"""
import argparse
import sys
from pathlib import Path
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))  # ffa-speedtest_amd/
from ffa_mi355x import producer_check as _check  # noqa: E402
from ffa_mi355x import quant as _Q  # noqa: E402


def build_rope_cache(
    seq_len: int,
    head_dim: int,
    base: float = 10000.0,
    device: Optional[torch.device] = None,
    dtype: torch.dtype = torch.float32,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables [seq_len, head_dim] with emb = cat(freqs, freqs) (reference :10-23)."""
    if head_dim % 2 != 0:
        raise ValueError(f"head_dim must be even for RoPE, got {head_dim}")
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, device=device, dtype=dtype) / head_dim))
    positions = torch.arange(seq_len, device=device, dtype=dtype)
    freqs = torch.outer(positions, inv_freq)
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos(), emb.sin()


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """Interleaved pair rotation (x0, x1) -> (-x1, x0) (reference :26-30)."""
    x_even = x[..., ::2]
    x_odd = x[..., 1::2]
    return torch.stack((-x_odd, x_even), dim=-1).flatten(-2)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    if cos.ndim == 2:
        cos = cos[None, :, None, :]
        sin = sin[None, :, None, :]
    return (x * cos) + (rotate_half(x) * sin)


def quantize_k_2bit_fp8_residual(k: torch.Tensor, fp8_dtype: torch.dtype = torch.float8_e5m2):
    """(k_q_packed, scale, zero, k_residual) of k [B, T, HKV, K] -- HIP kernels, bit-exact with the reference."""
    return _Q.quantize_per_channel(k, fp8_dtype)


def _normalize_k_weight(w_k: torch.Tensor, in_dim: int) -> torch.Tensor:
    return _Q._normalize_k_weight(w_k, in_dim)


def _resolve_fp8_dtype(device: torch.device) -> torch.dtype:
    return torch.float8_e5m2


def kproj_rope_quantize_reference(h, w_k, cos, sin, num_kv_heads, head_dim, bias=None, fp8_dtype=None):
    if fp8_dtype is None:
        fp8_dtype = _resolve_fp8_dtype(h.device)
    w_k = _normalize_k_weight(w_k, h.shape[-1])
    k_linear = F.linear(h, w_k, bias)
    B, T, _ = k_linear.shape
    if k_linear.shape[-1] != num_kv_heads * head_dim:
        raise ValueError(
            f"projection out_dim must be num_kv_heads*head_dim, got {k_linear.shape[-1]} "
            f"vs {num_kv_heads}*{head_dim}"
        )
    k = apply_rope(k_linear.view(B, T, num_kv_heads, head_dim), cos, sin)
    return quantize_k_2bit_fp8_residual(k, fp8_dtype)


def kproj_rope_quantize_triton(h, w_k, cos, sin, num_kv_heads, head_dim, bias=None, fp8_dtype=None, block_t=16,
                               block_h=32, block_pair=16, num_warps=4, num_stages=2):
    """Fused producer (reference :427-544).  Tuning arguments are accepted for signature
    compatibility; the HIP kernel has its own tiling."""
    if not h.is_cuda:
        raise ValueError("Triton kernel requires CUDA tensors.")
    if block_pair % 2 != 0:
        raise ValueError("block_pair must be even to pack int2 values.")
    if fp8_dtype is None:
        fp8_dtype = _resolve_fp8_dtype(h.device)
    return _Q.kproj_rope_q2_channel(h, w_k, cos, sin, num_kv_heads, head_dim, bias=bias, fp8_dtype=fp8_dtype)


def kproj_rope_quantize_fused(h, w_k, cos, sin, num_kv_heads, head_dim, bias=None, fp8_dtype=None):
    return kproj_rope_quantize_triton(h=h, w_k=w_k, cos=cos, sin=sin, num_kv_heads=num_kv_heads,
                                      head_dim=head_dim, bias=bias, fp8_dtype=fp8_dtype)


def run_smoke_test(device, dtype, fp8_dtype, B, T, H, HKV, K, seed=0) -> None:
    """Torch producer against the fused HIP producer on one seeded case (ffa_mi355x.producer_check)."""
    _check.run("q2fp8 producer", kproj_rope_quantize_reference, kproj_rope_quantize_triton,
               ("codes", "scale", "scale", "residual"), device, dtype, fp8_dtype, B, T, H, HKV, K, seed=seed)


def parse_args(argv=None) -> argparse.Namespace:
    return _check.parse("q2fp8 producer", argv)


def main(argv=None) -> None:
    ns = parse_args(argv)
    _check.main_for("q2fp8 producer", lambda *a: run_smoke_test(*a, seed=ns.seed), ns)


if __name__ == "__main__":
    main()
