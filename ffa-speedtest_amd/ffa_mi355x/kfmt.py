"""Host side of the pruned decode over the other K formats (fp8 base, nvfp4, nf4).

One C-ABI call (`ffa_kfmt_decode`) replaces the two Triton launches of
ffa-fp8fp8/attn_kernel/attn_kernel_v1210_fused_bsz_fp8fp8.py:263-309,
ffa-nvfp4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nvfp4fp8.py:316-363 and
ffa-nf4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nf4fp8.py:300-326.  The scratch
layout is the q2fp8 decode's (`DecodeWorkspace`).
"""
from __future__ import annotations

import ctypes

import torch

from . import _native as N
from .decode import HEAD_DIM, DecodeWorkspace

_FP8_FORMAT = {torch.float8_e4m3fn: N.KFMT_FP8_E4M3, torch.float8_e5m2: N.KFMT_FP8_E5M2}


def fp8_format_of(dtype: torch.dtype) -> int:
    try:
        return _FP8_FORMAT[dtype]
    except KeyError:
        raise NotImplementedError(f"fp8 K base must be float8_e4m3fn or float8_e5m2, got {dtype}") from None


def run_kfmt_decode(
    *,
    q: torch.Tensor,  # [B, HQ, 128]
    k: torch.Tensor,  # [B, T, HKV, 128] fp8 or [B, T, HKV, 64] u8 nibbles (paged: [P, HKV, 64, 64] pool)
    k_format: int,
    k_scale,  # tensor or None
    scale_kind: int,
    v: torch.Tensor,  # [B, T, HKV, 128]
    k_residual,
    use_res: bool,
    T: int,
    HKV: int,
    scale: float,
    BS: int,
    SBS: int,
    delta: float,
    precomputed_threshold=None,
    seq_lens=None,
    workspace: DecodeWorkspace | None = None,
    layout: int = N.LAYOUT_CONTIG,
    block_table=None,
) -> DecodeWorkspace:
    B, HQ, D = q.shape
    vdim = v.shape[-2] if layout == N.LAYOUT_PAGED else v.shape[-1]  # V^T pages [P, HKV, 128, 64]
    if D != HEAD_DIM or vdim != HEAD_DIM:
        raise NotImplementedError(f"head_dim {D} / value dim {vdim} not supported (this build implements 128)")
    if workspace is None:
        workspace = DecodeWorkspace(B, HQ, HKV, T, BS, SBS, q.device, q.dtype)
    elif not workspace.matches(B, HQ, HKV, T, BS, SBS, q.device, q.dtype):
        raise ValueError("workspace shape/device/dtype mismatch")
    th_in = precomputed_threshold.to(torch.float32).contiguous() if precomputed_threshold is not None else None
    if use_res and k_residual.dtype not in (torch.float8_e4m3fn, torch.float8_e5m2):
        raise NotImplementedError(f"k_residual must be float8_e4m3fn or float8_e5m2, got {k_residual.dtype}")
    a = N.KfmtArgs()
    a.q, a.q_dtype = q.data_ptr(), N.dtype_code(q.dtype)
    a.k, a.k_format = k.data_ptr(), k_format
    a.k_scale = k_scale.data_ptr() if k_scale is not None else None
    a.scale_dtype = N.dtype_code(k_scale.dtype) if k_scale is not None else N.DT_F16
    a.scale_kind = scale_kind
    a.k_residual = k_residual.data_ptr() if use_res else None
    a.res_dtype = N.dtype_code(k_residual.dtype) if use_res else N.DT_NONE
    a.v, a.v_dtype = v.data_ptr(), N.dtype_code(v.dtype)
    a.seq_lens = seq_lens.data_ptr() if seq_lens is not None else None
    a.B, a.T, a.HQ, a.HKV = B, int(T), HQ, int(HKV)
    a.scale, a.BS, a.SBS, a.delta = float(scale), int(BS), int(SBS), float(delta)
    a.threshold_in = th_in.data_ptr() if th_in is not None else None
    a.threshold_out = workspace.threshold_buf.data_ptr()
    a.out, a.out_dtype = workspace.o.data_ptr(), N.dtype_code(workspace.o.dtype)
    a.m_buf, a.l_buf, a.o_buf = workspace.m_buf.data_ptr(), workspace.l_buf.data_ptr(), workspace.o_buf.data_ptr()
    a.nparts = workspace.nparts
    a.mask, a.ntbs = workspace.mask_buf.data_ptr(), workspace.NTBS
    a.piece_max = workspace.piece_max.data_ptr() if workspace.piece_max is not None else None
    a.npieces = workspace.npieces
    a.layout = layout
    a.block_table = block_table.data_ptr() if block_table is not None else None
    a.bt_stride = block_table.shape[1] if block_table is not None else 0
    if layout == N.LAYOUT_PAGED:  # pages every pool holds: the kernel reads ids beyond them as page 0
        pools = [k, v] + ([k_scale] if k_scale is not None else []) + ([k_residual] if use_res else [])
        a.num_pages = min(int(t.shape[0]) for t in pools)
    rc = N.lib().ffa_kfmt_decode(ctypes.byref(a), ctypes.c_void_p(N.stream_of(q.device)))
    N.check(rc, "ffa_kfmt_decode")
    return workspace


def skip_ratio(workspace: DecodeWorkspace, seq_lens=None) -> float:
    """1 - kept / total blocks (the reference's formula, ragged lengths counting their own blocks)."""
    from .decode import skip_ratio_of

    return skip_ratio_of(workspace.mask_buf, seq_lens, workspace.BS, workspace.SBS)
