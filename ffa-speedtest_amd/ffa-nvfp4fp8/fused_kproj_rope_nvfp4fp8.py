"""Drop-in for ffa-nvfp4fp8/fused_kproj_rope_nvfp4fp8.py on MI355X (no Triton).

Same names and signatures:
  build_rope_cache, rotate_half, apply_rope        (reference :12-39, torch host helpers)
  encode_k_nvfp4_fp8_residual                      (:62-114)  -> HIP quantizer, bit-exact
  kproj_rope_quantize_reference                    (:117-140) -> torch GEMM + RoPE, HIP quantizer
  kproj_rope_quantize_triton / _fused              (:143-190) -> HIP GEMM + RoPE kernel, HIP quantizer
  run_smoke_test, parse_args, main                 (:193-290)
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


def run_smoke_test(device, dtype, fp8_dtype, B, T, H, HKV, K, page_size) -> None:
    """Torch-GEMM producer vs the fused HIP producer.  The quantizer is bit-exact on the same K;
    the two GEMMs may differ in the last bit, so a few codes may flip (the nf4 reference's
    smoke tolerances, ffa-nf4fp8/fused_kproj_rope_nf4fp8.py:620-628)."""
    torch.manual_seed(0)
    h = torch.randn(B, T, H, device=device, dtype=dtype)
    w_k = torch.randn(HKV * K, H, device=device, dtype=dtype)
    cos, sin = build_rope_cache(T, K, device=device, dtype=dtype)
    k_fp4_ref, k_scale_ref, k_res_ref = kproj_rope_quantize_reference(
        h=h, w_k=w_k, cos=cos, sin=sin, num_kv_heads=HKV, head_dim=K, page_size=page_size, fp8_dtype=fp8_dtype)
    k_fp4_fused, k_scale_fused, k_res_fused = kproj_rope_quantize_triton(
        h=h, w_k=w_k, cos=cos, sin=sin, num_kv_heads=HKV, head_dim=K, page_size=page_size, fp8_dtype=fp8_dtype)
    packed_mismatch = (k_fp4_ref != k_fp4_fused).float().mean().item()
    scale_max = (k_scale_ref.float() - k_scale_fused.float()).abs().max().item()
    res_mean = (k_res_ref.float() - k_res_fused.float()).abs().mean().item()
    if packed_mismatch > 0.01 or scale_max > 0.05 or res_mean > 0.05:
        raise AssertionError(
            "fused output mismatch: "
            f"packed_mismatch={packed_mismatch:.6f}, scale_max={scale_max:.6f}, res_mean={res_mean:.6f}")
    print(f"[OK] nvfp4 base/scale/residual outputs match reference (packed_mismatch={packed_mismatch:.6f}, "
          f"scale_max={scale_max:.6f}, res_mean={res_mean:.6f})")
    print(f"device={device}, dtype={dtype}, fp8_dtype={fp8_dtype}, B={B}, T={T}, H={H}, HKV={HKV}, K={K}, "
          f"page_size={page_size}")


def parse_args() -> argparse.Namespace:
    p = argparse.ArgumentParser(description="Fuse K projection + RoPE + nvfp4/fp8 split and test.")
    p.add_argument("--device", type=str, default="cuda" if torch.cuda.is_available() else "cpu")
    p.add_argument("--dtype", type=str, default="fp16", choices=["fp16", "bf16", "fp32"])
    p.add_argument("--B", type=int, default=2)
    p.add_argument("--T", type=int, default=32)
    p.add_argument("--H", type=int, default=256)
    p.add_argument("--HKV", type=int, default=4)
    p.add_argument("--K", type=int, default=64)
    p.add_argument("--page-size", type=int, default=128)
    return p.parse_args()


def main() -> None:
    args = parse_args()
    dtype = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[args.dtype]
    device = torch.device(args.device)
    if device.type == "cpu":
        raise RuntimeError("This test requires a CUDA device for fp8 storage.")
    run_smoke_test(device=device, dtype=dtype, fp8_dtype=_resolve_fp8_dtype(device), B=args.B, T=args.T, H=args.H,
                   HKV=args.HKV, K=args.K, page_size=args.page_size)


if __name__ == "__main__":
    main()
