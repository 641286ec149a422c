"""RoPE angle rows for given positions (host helper; the tables are kernel inputs).

Same frequencies as build_rope_cache (ffa-q2fp8/fused_kproj_rope_q2fp8.py:10-23):
inv_freq = 1 / base^(2i/D), emb = cat(freqs, freqs), computed in fp32 so that
positions above 65504 (fp16's range) stay exact.
"""
from __future__ import annotations

import torch


def rope_rows(positions: torch.Tensor, head_dim: int = 128, base: float = 10000.0):
    """positions [...] int -> (cos, sin) [..., head_dim] fp32."""
    inv = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=positions.device) / head_dim))
    ang = positions.to(torch.float32)[..., None] * inv
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos(), emb.sin()
