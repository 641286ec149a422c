"""Drop-in for ffa-nvfp4fp8/fused_kproj_rope_nvfp4fp8.py on MI355X (no Triton).

Same names and signatures:
  build_rope_cache, rotate_half, apply_rope        (reference :12-39, torch host helpers)
  encode_k_nvfp4_fp8_residual                      (:62-114)  -> HIP quantizer, bit-exact
  kproj_rope_quantize_reference                    (:117-140) -> torch GEMM + RoPE, HIP quantizer
  kproj_rope_quantize_triton / _fused              (:143-190) -> HIP GEMM + RoPE kernel, HIP quantizer
  run_smoke_test, parse_args, main  (entry names of :193-290; the check is ffa_mi355x.producer_check)
The reference's "triton" producer is a placeholder that calls its torch path; here it is
a real fused kernel, so the two producers agree to the GEMM's last bit, not bitwise.
"""
import argparse
import sys
from pathlib import Path
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))  # ffa-speedtest_amd/
from ffa_mi355x import kfmt_quant as _KQ  # noqa: E402
from ffa_mi355x import producer_check as _check  # noqa: E402
from ffa_mi355x.quant import _normalize_k_weight  # noqa: E402,F401
from ffa_mi355x.rope import apply_rope, build_rope_cache, rotate_half  # noqa: E402,F401


def _resolve_fp8_dtype(device: torch.device) -> torch.dtype:
    return torch.float8_e5m2


def encode_k_nvfp4_fp8_residual(
    k: torch.Tensor,
    fp8_dtype: torch.dtype,
    page_size: int,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(k_packed [B,T,HKV,ceil(K/2)] u8, k_scale [B,ceil(T/page_size),HKV] k.dtype, k_residual fp8)."""
    return _KQ.encode_nvfp4(k, fp8_dtype, page_size)


def _project(h, w_k, cos, sin, num_kv_heads, head_dim, bias):
    w_k = _normalize_k_weight(w_k, h.shape[-1])
    k_linear = F.linear(h, w_k, bias)
    B, T, _ = k_linear.shape
    if k_linear.shape[-1] != num_kv_heads * head_dim:
        raise ValueError(
            f"projection out_dim must be num_kv_heads*head_dim, got {k_linear.shape[-1]} "
            f"vs {num_kv_heads}*{head_dim}"
        )
    return apply_rope(k_linear.view(B, T, num_kv_heads, head_dim), cos, sin)


def kproj_rope_quantize_reference(
    h: torch.Tensor,
    w_k: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    num_kv_heads: int,
    head_dim: int,
    page_size: int,
    bias: Optional[torch.Tensor] = None,
    fp8_dtype: Optional[torch.dtype] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    if fp8_dtype is None:
        fp8_dtype = _resolve_fp8_dtype(h.device)
    k = _project(h, w_k, cos, sin, num_kv_heads, head_dim, bias)
    return encode_k_nvfp4_fp8_residual(k, fp8_dtype, page_size)


def kproj_rope_quantize_triton(
    h: torch.Tensor,
    w_k: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    num_kv_heads: int,
    head_dim: int,
    page_size: int,
    bias: Optional[torch.Tensor] = None,
    fp8_dtype: Optional[torch.dtype] = None,
    **_kwargs,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """HIP GEMM + RoPE (ffa_kproj_rope) then the HIP quantizer; tuning kwargs are accepted and ignored."""
    if fp8_dtype is None:
        fp8_dtype = _resolve_fp8_dtype(h.device)
    k = _KQ.kproj_rope(h, w_k, cos, sin, num_kv_heads, head_dim, bias=bias)
    return encode_k_nvfp4_fp8_residual(k, fp8_dtype, page_size)


def kproj_rope_quantize_fused(
    h: torch.Tensor,
    w_k: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    num_kv_heads: int,
    head_dim: int,
    page_size: int,
    bias: Optional[torch.Tensor] = None,
    fp8_dtype: Optional[torch.dtype] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return kproj_rope_quantize_triton(h=h, w_k=w_k, cos=cos, sin=sin, num_kv_heads=num_kv_heads,
                                      head_dim=head_dim, page_size=page_size, bias=bias, fp8_dtype=fp8_dtype)


def run_smoke_test(device, dtype, fp8_dtype, B, T, H, HKV, K, page_size, seed=0) -> None:
    """Torch producer against the fused HIP producer on one seeded case (ffa_mi355x.producer_check)."""
    _check.run("nvfp4fp8 producer", kproj_rope_quantize_reference, kproj_rope_quantize_triton,
               ("codes", "scale", "residual"), device, dtype, fp8_dtype, B, T, H, HKV, K, seed=seed,
               page_size=page_size)


def parse_args(argv=None) -> argparse.Namespace:
    return _check.parse("nvfp4fp8 producer", argv, page_size=True)


def main(argv=None) -> None:
    ns = parse_args(argv)
    _check.main_for("nvfp4fp8 producer", lambda *a, **kw: run_smoke_test(*a, seed=ns.seed, **kw), ns)


if __name__ == "__main__":
    main()
