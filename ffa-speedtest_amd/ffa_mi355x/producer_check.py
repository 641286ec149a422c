"""Agreement check between a drop-in's torch producer and its fused HIP producer.

Both producers of a format hand K = RoPE(h W_k^T) to the same HIP quantizer; they differ only
in how K is formed (torch's GEMM against the library's MFMA GEMM, whose fp32 sums may round
differently).  A K value that moves across a rounding boundary changes one code and the residual
that goes with it, so the check bounds the disagreement instead of asking for equality:

  codes      share of differing bytes                              <= 1/64
  scale      largest |difference| / largest |torch value|          <= 1/64
  residual   mean |difference| / mean |torch residual|             <= 1/8

Inputs come from a seeded ``torch.Generator`` on the CPU (h ~ N(0, 1), W_k ~ N(0, 1/H), so K has
unit scale as in a trained projection) and are then moved to the device, so a seed names the
same case on every device.  The per-module entry points ``run_smoke_test``, ``parse_args`` and
``main`` of the four producer drop-ins call into this module.
"""
from __future__ import annotations

import argparse
from typing import Callable, Dict, Sequence

import torch

from .rope import build_rope_cache

LIMITS = {"codes": 1.0 / 64, "scale": 1.0 / 64, "residual": 1.0 / 8}
DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
FP8 = {"e4m3fn": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def _measure(kind: str, ref: torch.Tensor, got: torch.Tensor) -> float:
    if ref.shape != got.shape:
        raise AssertionError(f"output shapes differ: torch producer {tuple(ref.shape)}, fused {tuple(got.shape)}")
    if kind == "codes":
        return (ref.contiguous().view(torch.uint8) != got.contiguous().view(torch.uint8)).float().mean().item()
    a, b = ref.float(), got.float()
    if kind == "scale":
        return ((a - b).abs().max() / a.abs().max().clamp_min(1e-30)).item()
    if kind == "residual":
        return ((a - b).abs().mean() / a.abs().mean().clamp_min(1e-30)).item()
    raise ValueError(f"unknown output kind {kind!r}")


def run(label: str, reference_fn: Callable, fused_fn: Callable, kinds: Sequence[str], device, dtype: torch.dtype,
        fp8_dtype: torch.dtype, B: int, T: int, H: int, HKV: int, K: int, seed: int = 0, verbose: bool = True,
        **extra) -> Dict[str, float]:
    """Run both producers on one seeded case and compare output by output (``kinds`` names each
    output: "codes", "scale" or "residual").  Raises AssertionError past a limit; returns the
    measured ratios keyed "<index>:<kind>"."""
    device = torch.device(device)
    if device.type != "cuda":
        raise RuntimeError("the fused producer runs on the GPU: pass a cuda device")
    gen = torch.Generator().manual_seed(seed)
    h = torch.randn(B, T, H, generator=gen).to(device=device, dtype=dtype)
    w_k = (torch.randn(HKV * K, H, generator=gen) * H ** -0.5).to(device=device, dtype=dtype)
    cos, sin = build_rope_cache(T, K, device=device, dtype=dtype)
    args = dict(h=h, w_k=w_k, cos=cos, sin=sin, num_kv_heads=HKV, head_dim=K, fp8_dtype=fp8_dtype, **extra)
    ref = reference_fn(**args)
    got = fused_fn(**args)
    if len(ref) != len(kinds) or len(got) != len(kinds):
        raise AssertionError(f"expected {len(kinds)} outputs, got {len(ref)} (torch) and {len(got)} (fused)")
    ratios = {f"{i}:{kind}": _measure(kind, r, g) for i, (kind, r, g) in enumerate(zip(kinds, ref, got))}
    over = {k: v for k, v in ratios.items() if v > LIMITS[k.split(":")[1]]}
    summary = ", ".join(f"{k}={v:.2e}" for k, v in ratios.items())
    if over:
        raise AssertionError(f"{label}: fused and torch producers disagree beyond the limits {LIMITS}: {summary}")
    if verbose:
        print(f"{label}: producers agree ({summary}); B={B} T={T} H={H} HKV={HKV} K={K} {dtype} {fp8_dtype}")
    return ratios


def parse(label: str, argv=None, page_size: bool = False) -> argparse.Namespace:
    """Command line of a producer self-check: --shape B,T,H,HKV,K (default 2,32,256,4,64), --dtype,
    --fp8, --seed, --device and, for nvfp4, --page-size."""
    ap = argparse.ArgumentParser(description=f"{label}: compare the fused HIP producer with the torch producer")
    ap.add_argument("--shape", default="2,32,256,4,64", help="B,T,H,HKV,K (comma separated)")
    ap.add_argument("--dtype", choices=sorted(DTYPES), default="fp16")
    ap.add_argument("--fp8", choices=sorted(FP8), default="e5m2", help="residual format")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--device", default="cuda")
    if page_size:
        ap.add_argument("--page-size", type=int, default=128)
    ns = ap.parse_args(argv)
    dims = [int(x) for x in ns.shape.split(",")]
    if len(dims) != 5 or min(dims) <= 0:
        ap.error("--shape takes five positive integers B,T,H,HKV,K")
    ns.B, ns.T, ns.H, ns.HKV, ns.K = dims
    return ns


def main_for(label: str, smoke: Callable, ns: argparse.Namespace) -> None:
    if not torch.cuda.is_available() or torch.device(ns.device).type != "cuda":
        raise SystemExit(f"{label}: a GPU is required (the fused producer is a HIP kernel)")
    extra = {"page_size": ns.page_size} if hasattr(ns, "page_size") else {}
    smoke(torch.device(ns.device), DTYPES[ns.dtype], FP8[ns.fp8], ns.B, ns.T, ns.H, ns.HKV, ns.K, **extra)
