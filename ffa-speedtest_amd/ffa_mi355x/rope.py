"""RoPE host helpers shared by every drop-in producer.

All four reference producers define the same three functions
(ffa-q2fp8/fused_kproj_rope_q2fp8.py:10-37, ffa-fp8fp8/fused_kproj_rope_fp8fp8.py:8-35,
ffa-nvfp4fp8/fused_kproj_rope_nvfp4fp8.py:12-39, ffa-nf4fp8/fused_kproj_rope_nf4fp8.py:42-69);
they are part of each module's interface, so the drop-ins re-export these.
`rope_rows` gives the same angles for arbitrary positions in fp32 (the paged append's
cos/sin rows), so positions above 65504 (fp16's range) stay exact.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch


def build_rope_cache(
    seq_len: int,
    head_dim: int,
    base: float = 10000.0,
    device: Optional[torch.device] = None,
    dtype: torch.dtype = torch.float32,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables [seq_len, head_dim]: angle(t, d) = t * base^(-2(d mod D/2)/D), i.e. emb = cat(freqs, freqs)."""
    if head_dim % 2 != 0:
        raise ValueError(f"head_dim must be even for RoPE, got {head_dim}")
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, device=device, dtype=dtype) / head_dim))
    positions = torch.arange(seq_len, device=device, dtype=dtype)
    freqs = torch.outer(positions, inv_freq)
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos(), emb.sin()


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """Interleaved pair rotation (x0, x1) -> (-x1, x0)."""
    x_even = x[..., ::2]
    x_odd = x[..., 1::2]
    return torch.stack((-x_odd, x_even), dim=-1).flatten(-2)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x * cos + rotate_half(x) * sin; [T, D] tables broadcast over [B, T, H, D]."""
    if cos.ndim == 2:
        cos = cos[None, :, None, :]
        sin = sin[None, :, None, :]
    return (x * cos) + (rotate_half(x) * sin)


def rope_rows(positions: torch.Tensor, head_dim: int = 128, base: float = 10000.0):
    """positions [...] int -> (cos, sin) [..., head_dim] fp32 (same frequencies as build_rope_cache)."""
    inv = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=positions.device) / head_dim))
    ang = positions.to(torch.float32)[..., None] * inv
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos(), emb.sin()
