# attn_kernel_v1210_fused_bsz_nf4fp8.py -- MI355X drop-in.
# NF4 K with fp8 residual refinement; the kernels are hand-written HIP for gfx950 in
# libffa_mi355x.so (no Triton).
"""Drop-in for ffa-nf4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nf4fp8.py.

`attn_forward_decode_nf4` keeps the reference signature, defaults, scale-shape
normalisation and exception types (reference :202-330).  K is packed NF4 codes (low
nibble first) with one scale per (sequence, KV head, channel).  Extension through
**kwargs: seq_lens=[B] int32, workspace=DecodeWorkspace; block_table=[B, n] int32 (with
T= or seq_lens=) selects the paged layout (64-token page pools, one fp16 absmax per 64 channels), where k_nf4 / k_scale / k_residual / v are
the page pools of ffa_mi355x.paged_kfmt.PagedKfmtCache("nf4", ...).
"""
import math
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))  # ffa-speedtest_amd/
from ffa_mi355x import _native as _N  # noqa: E402
from ffa_mi355x.decode import DecodeWorkspace, decode_ntbs  # noqa: E402
from ffa_mi355x.kfmt import run_kfmt_decode  # noqa: E402
from ffa_mi355x.paged_kfmt import decode_pools  # noqa: E402

__all__ = ["attn_forward_decode_nf4", "NF4_CODEBOOK_VALUES"]

# QLoRA NF4 levels (the published 16 normal-float values); the kernel holds the same table
NF4_CODEBOOK_VALUES = (
    -1.0, -0.6961928009986877, -0.5229921340942383, -0.39491748809814453, -0.28444138169288635,
    -0.18477343022823334, -0.09105003625154495, 0.0, 0.07958029955625534, 0.16093020141124725,
    0.24611230194568634, 0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
    0.7229568362236023, 1.0,
)


def _normalize_scale(k_scale: torch.Tensor, expect_shape):
    """[B, 1, HKV, K] is accepted for [B, HKV, K] (reference :202-209)."""
    if k_scale.ndim == 4 and k_scale.shape[1] == 1:
        k_scale = k_scale.squeeze(1)
    if k_scale.shape != expect_shape:
        raise ValueError(f"Unsupported k_scale shape: {k_scale.shape}, expected {expect_shape}")
    return k_scale.contiguous()


def attn_forward_decode_nf4(
    q: torch.Tensor,           # [B, 1, HQ, K]
    k_nf4: torch.Tensor,       # [B, T, HKV, ceil(K / (8 / k_bits))], packed NF4 codes
    k_scale: torch.Tensor,     # [B, HKV, K] (token dimension removed)
    v: torch.Tensor,           # [B, T, HKV, V]
    k_residual: torch.Tensor | None = None,  # [B, T, HKV, K], fp8 residual
    k_bits: int = 4,
    scale: float = None,
    BS: int = 128,
    SBS: int | None = None,
    delta: float = 5.0,
    return_skip_ratio: bool = False,
    precomputed_threshold: torch.Tensor | None = None,
    use_fp8_residual: bool = True,
    **kwargs,
):
    assert q.is_cuda and k_nf4.is_cuda and v.is_cuda
    if k_residual is not None and not k_residual.is_cuda:
        raise ValueError("k_residual must be a CUDA tensor when provided")
    if k_bits != 4:
        raise ValueError(f"attn_forward_decode_nf4 currently supports 4-bit keys, got k_bits={k_bits}")
    assert k_scale.is_cuda, "k_scale must be a CUDA tensor"
    if not k_scale.is_floating_point():
        raise ValueError("k_scale must be a floating point tensor for dequantization")
    if k_nf4.is_floating_point():
        raise ValueError("k_nf4 must contain packed NF4 codes in an integer tensor (e.g., uint8)")
    if k_residual is not None and not k_residual.is_floating_point():
        raise ValueError("k_residual must be a floating point tensor (e.g., fp8/fp16/bf16)")

    if kwargs.get("block_table") is not None:
        # paged layout (per-token group scales; no reference counterpart)
        if use_fp8_residual and k_residual is None:
            raise ValueError("use_fp8_residual=True requires k_residual")
        workspace = kwargs.get("workspace")
        if workspace is not None and not isinstance(workspace, DecodeWorkspace):
            raise TypeError("workspace must be a DecodeWorkspace")
        seq_lens = kwargs.get("seq_lens")
        ws = decode_pools("nf4", q, k_nf4, k_scale, v, k_residual, kwargs["block_table"], seq_lens, T=kwargs.get("T"),
                          scale=scale, BS=BS, SBS=SBS, delta=delta, precomputed_threshold=precomputed_threshold,
                          use_fp8_residual=use_fp8_residual, workspace=workspace)
        if return_skip_ratio:
            kept = ws.mask_buf.to(torch.int32).sum()
            sl = seq_lens.tolist() if seq_lens is not None else [ws.T] * q.shape[0]
            total = sum(decode_ntbs(int(t), BS, BS if SBS is None else SBS) for t in sl) * k_nf4.shape[1]
            return ws.o, float((1.0 - (kept.float() / float(total))).item())
        return ws.o

    B, Tq, HQ, K = q.shape
    Bk, T, HKV, K_packed = k_nf4.shape
    Bv, Tv, HKVv, V = v.shape
    vals_per_byte = 8 // k_bits
    expected_k_packed = (K + vals_per_byte - 1) // vals_per_byte
    if K_packed != expected_k_packed:
        raise ValueError(
            f"k_nf4 packed dim mismatch: got {K_packed}, expected {expected_k_packed} for K={K}, k_bits={k_bits}")
    if k_residual is not None:
        Bk_r, T_r, HKV_r, K_r = k_residual.shape
        assert (B == Bk == Bv == Bk_r and Tq == 1 and Tv == T == T_r and HKVv == HKV == HKV_r
                and K == K_r), "K/V layouts must be [B, T, HKV, D]"
    else:
        assert B == Bk == Bv and Tq == 1 and Tv == T and HKVv == HKV, "K/V layouts must be [B, T, HKV, D]"
    k_scale = _normalize_scale(k_scale, (B, HKV, K))
    if scale is None:
        scale = 1.0 / math.sqrt(K)
    if SBS is None:
        SBS = BS
    assert q.is_contiguous() and k_nf4.is_contiguous() and v.is_contiguous()
    if use_fp8_residual and k_residual is None:
        raise ValueError("use_fp8_residual=True requires k_residual")
    if k_residual is not None:
        assert k_residual.is_contiguous()
    use_res = bool(use_fp8_residual and k_residual is not None)
    if precomputed_threshold is not None:
        assert precomputed_threshold.is_cuda and precomputed_threshold.shape == (B, HQ)
    seq_lens = kwargs.get("seq_lens")
    if seq_lens is not None:
        seq_lens = seq_lens.to(device=q.device, dtype=torch.int32).contiguous()
    workspace = kwargs.get("workspace")
    if workspace is not None and not isinstance(workspace, DecodeWorkspace):
        raise TypeError("workspace must be a DecodeWorkspace")

    ws = run_kfmt_decode(
        q=q[:, 0], k=k_nf4, k_format=_N.KFMT_NF4, k_scale=k_scale, scale_kind=_N.KSCALE_CHANNEL, v=v,
        k_residual=k_residual, use_res=use_res, T=T, HKV=HKV, scale=scale, BS=BS, SBS=SBS, delta=delta,
        precomputed_threshold=precomputed_threshold, seq_lens=seq_lens, workspace=workspace)
    if return_skip_ratio:
        kept = ws.mask_buf.to(torch.int32).sum()
        total = ws.mask_buf.numel() if seq_lens is None else \
            sum(decode_ntbs(int(t), BS, SBS) for t in seq_lens.tolist()) * HKV
        return ws.o, float((1.0 - (kept.float() / float(total))).item())
    return ws.o
