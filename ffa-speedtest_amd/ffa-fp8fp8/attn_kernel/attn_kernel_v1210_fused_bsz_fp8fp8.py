# attn_kernel_v1210_fused_bsz_fp8fp8.py -- MI355X drop-in.
# FP8 K with FP8 residual refinement; the kernels are hand-written HIP for gfx950 in
# libffa_mi355x.so (no Triton).
"""Drop-in for ffa-fp8fp8/attn_kernel/attn_kernel_v1210_fused_bsz_fp8fp8.py.

`attn_forward_decode_fp8fp8` keeps the reference signature, defaults and exception
types (reference :180-312).  Extension through **kwargs: k_scale=[B, T, HKV] (one scale
per token and KV head, no reference counterpart), so that k_hat = fp16(k_fp8 * k_scale);
seq_lens=[B] int32 (ragged lengths).
"""
import math
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))  # ffa-speedtest_amd/
from ffa_mi355x import _native as _N  # noqa: E402
from ffa_mi355x.decode import DecodeWorkspace, decode_ntbs  # noqa: E402
from ffa_mi355x.kfmt import fp8_format_of, run_kfmt_decode  # noqa: E402

__all__ = ["attn_forward_decode_fp8fp8"]


def attn_forward_decode_fp8fp8(
    q: torch.Tensor,  # [B, 1, HQ, K]
    k_fp8: torch.Tensor,  # [B, T, HKV, K]
    v: torch.Tensor,  # [B, T, HKV, V]
    *,
    k_residual: torch.Tensor | None = None,  # [B, T, HKV, K]
    scale: float | None = None,
    BS: int = 128,
    SBS: int | None = None,
    delta: float = 5.0,
    return_skip_ratio: bool = False,
    precomputed_threshold: torch.Tensor | None = None,
    use_fp8_residual: bool = True,
    **kwargs,
):
    assert q.is_cuda and k_fp8.is_cuda and v.is_cuda
    if k_residual is not None and not k_residual.is_cuda:
        raise ValueError("k_residual must be a CUDA tensor when provided")
    if not k_fp8.is_floating_point():
        raise ValueError("k_fp8 must be a floating point tensor (fp8/fp16/bf16)")
    if k_residual is not None and not k_residual.is_floating_point():
        raise ValueError("k_residual must be a floating point tensor (fp8/fp16/bf16)")

    B, Tq, HQ, K = q.shape
    Bk, T, HKV, Kk = k_fp8.shape
    Bv, Tv, HKVv, V = v.shape
    if k_residual is not None:
        Bk_r, T_r, HKV_r, K_r = k_residual.shape
        assert (B == Bk == Bv == Bk_r and Tq == 1 and Tv == T == T_r and HKVv == HKV == HKV_r
                and K == Kk == K_r), "K/V layouts must be [B, T, HKV, D]"
    else:
        assert B == Bk == Bv and Tq == 1 and Tv == T and HKVv == HKV and K == Kk, "K/V layouts must be [B, T, HKV, D]"
    if HQ % HKV != 0:
        raise ValueError(f"HQ ({HQ}) must be divisible by HKV ({HKV}) for GQA")
    if scale is None:
        scale = 1.0 / math.sqrt(K)
    if SBS is None:
        SBS = BS
    assert q.is_contiguous() and k_fp8.is_contiguous() and v.is_contiguous()
    if use_fp8_residual and k_residual is None:
        raise ValueError("use_fp8_residual=True requires k_residual")
    if k_residual is not None:
        assert k_residual.is_contiguous()
    use_res = bool(use_fp8_residual and k_residual is not None)
    if precomputed_threshold is not None:
        assert precomputed_threshold.is_cuda and precomputed_threshold.shape == (B, HQ)

    k_scale = kwargs.get("k_scale")
    if k_scale is not None:
        if tuple(k_scale.shape) != (B, T, HKV):
            raise ValueError(f"k_scale must be [B, T, HKV] = {(B, T, HKV)}, got {tuple(k_scale.shape)}")
        k_scale = k_scale.contiguous()
    seq_lens = kwargs.get("seq_lens")
    if seq_lens is not None:
        seq_lens = seq_lens.to(device=q.device, dtype=torch.int32).contiguous()
    workspace = kwargs.get("workspace")
    if workspace is not None and not isinstance(workspace, DecodeWorkspace):
        raise TypeError("workspace must be a DecodeWorkspace")

    ws = run_kfmt_decode(
        q=q[:, 0], k=k_fp8, k_format=fp8_format_of(k_fp8.dtype), k_scale=k_scale,
        scale_kind=_N.KSCALE_TOKEN if k_scale is not None else _N.KSCALE_NONE, v=v, k_residual=k_residual,
        use_res=use_res, T=T, HKV=HKV, scale=scale, BS=BS, SBS=SBS, delta=delta,
        precomputed_threshold=precomputed_threshold, seq_lens=seq_lens, workspace=workspace)
    if return_skip_ratio:
        kept = ws.mask_buf.to(torch.int32).sum()
        total = ws.mask_buf.numel() if seq_lens is None else \
            sum(decode_ntbs(int(t), BS, SBS) for t in seq_lens.tolist()) * HKV
        return ws.o, float((1.0 - (kept.float() / float(total))).item())
    return ws.o
