"""Drop-in for ffa-nf4fp8/fused_kproj_rope_nf4fp8.py on MI355X (no Triton).

Same names and signatures:
  NF4_CODEBOOK_VALUES, _get_nf4_tables             (reference :10-39)
  build_rope_cache, rotate_half, apply_rope        (:42-69, torch host helpers)
  encode_k_nf4_fp8_residual                        (:72-96)   -> HIP quantizer, bit-exact
  kproj_rope_nf4_reference                         (:415-437) -> torch GEMM + RoPE, HIP quantizer
  kproj_rope_nf4_triton / kproj_rope_nf4_fused     (:440-580) -> HIP GEMM + RoPE kernel, HIP quantizer
  run_smoke_test, parse_args, main  (entry names of :583-677; the check is ffa_mi355x.producer_check)
The fused producer quantizes the rotated K with the torch path's rules (the reference's
two Triton kernels round their own way); its scale has the dtype of h, as in the reference.
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

# the published 16-level NF4 (QLoRA) codebook, as float32 values
NF4_CODEBOOK_VALUES = (
    -1.0,
    -0.6961928009986877,
    -0.5229921340942383,
    -0.39491748809814453,
    -0.28444138169288635,
    -0.18477343022823334,
    -0.09105003625154495,
    0.0,
    0.07958029955625534,
    0.16093020141124725,
    0.24611230194568634,
    0.33791524171829224,
    0.44070982933044434,
    0.5626170039176941,
    0.7229568362236023,
    1.0,
)

_NF4_TABLE_CACHE = {}


def _get_nf4_tables(device: torch.device) -> Tuple[torch.Tensor, torch.Tensor]:
    """(codebook f32 [16], midpoints f32 [15]) on `device`, cached per device."""
    key = (device.type, device.index)
    if key not in _NF4_TABLE_CACHE:
        codebook = torch.tensor(NF4_CODEBOOK_VALUES, device=device, dtype=torch.float32)
        _NF4_TABLE_CACHE[key] = (codebook, (codebook[:-1] + codebook[1:]) * 0.5)
    return _NF4_TABLE_CACHE[key]


def _resolve_fp8_dtype(device: torch.device) -> torch.dtype:
    return torch.float8_e5m2


def encode_k_nf4_fp8_residual(k: torch.Tensor, fp8_dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(k_nf4_packed [B,T,HKV,ceil(K/2)] u8, scale [B,HKV,K] k.dtype, k_residual fp8)."""
    return _KQ.encode_nf4(k, fp8_dtype)


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


def kproj_rope_nf4_reference(
    h: torch.Tensor,
    w_k: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    num_kv_heads: int,
    head_dim: int,
    bias: Optional[torch.Tensor] = None,
    fp8_dtype: Optional[torch.dtype] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    if fp8_dtype is None:
        fp8_dtype = _resolve_fp8_dtype(h.device)
    return encode_k_nf4_fp8_residual(_project(h, w_k, cos, sin, num_kv_heads, head_dim, bias), fp8_dtype)


def kproj_rope_nf4_triton(
    h: torch.Tensor,
    w_k: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    num_kv_heads: int,
    head_dim: int,
    bias: Optional[torch.Tensor] = None,
    fp8_dtype: Optional[torch.dtype] = None,
    block_t: int = 16,
    block_h: int = 32,
    block_pair: int = 16,
    num_warps: int = 4,
    num_stages: int = 2,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """HIP GEMM + RoPE (ffa_kproj_rope) then the HIP nf4 quantizer.  The reference's argument
    checks are kept; the tiling arguments are accepted and ignored."""
    if not h.is_cuda:
        raise ValueError("Triton kernel requires CUDA tensors.")
    if head_dim % 2 != 0:
        raise ValueError(f"head_dim must be even for RoPE, got {head_dim}")
    if block_pair <= 0:
        raise ValueError("block_pair must be positive.")
    w_k = _normalize_k_weight(w_k, h.shape[-1])
    out_dim = num_kv_heads * head_dim
    if w_k.shape[0] != out_dim:
        raise ValueError(f"w_k out_dim mismatch: got {w_k.shape[0]}, expected {out_dim}")
    if bias is not None and bias.numel() != out_dim:
        raise ValueError(f"bias length mismatch: got {bias.numel()}, expected {out_dim}")
    if fp8_dtype is None:
        fp8_dtype = _resolve_fp8_dtype(h.device)
    k = _KQ.kproj_rope(h, w_k, cos, sin, num_kv_heads, head_dim, bias=bias)
    packed, scale, res = encode_k_nf4_fp8_residual(k, fp8_dtype)
    return packed, scale.to(h.dtype), res


def kproj_rope_nf4_fused(
    h: torch.Tensor,
    w_k: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    num_kv_heads: int,
    head_dim: int,
    bias: Optional[torch.Tensor] = None,
    fp8_dtype: Optional[torch.dtype] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return kproj_rope_nf4_triton(h=h, w_k=w_k, cos=cos, sin=sin, num_kv_heads=num_kv_heads, head_dim=head_dim,
                                 bias=bias, fp8_dtype=fp8_dtype)


def run_smoke_test(device, dtype, fp8_dtype, B, T, H, HKV, K, seed=0) -> None:
    """Torch producer against the fused HIP producer on one seeded case (ffa_mi355x.producer_check)."""
    _check.run("nf4fp8 producer", kproj_rope_nf4_reference, kproj_rope_nf4_triton, ("codes", "scale", "residual"),
               device, dtype, fp8_dtype, B, T, H, HKV, K, seed=seed)


def parse_args(argv=None) -> argparse.Namespace:
    return _check.parse("nf4fp8 producer", argv)


def main(argv=None) -> None:
    ns = parse_args(argv)
    _check.main_for("nf4fp8 producer", lambda *a: run_smoke_test(*a, seed=ns.seed), ns)


if __name__ == "__main__":
    main()
