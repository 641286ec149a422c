"""Host side of the q2fp8 pruned decode: validation, scratch, one C-ABI call.

The launch sequence replaces stage1 + stage2 of
ffa-q2fp8/attn_kernel/attn_kernel_v1210_fused_bsz_q2fp8.py:283-304; the
argument checks mirror :211-281 (same exception types).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from . import _native as N

HEAD_DIM = 128
_STAGE_FN = {"both": "ffa_q2fp8_decode", "stage1": "ffa_q2fp8_decode_stage1", "stage2": "ffa_q2fp8_decode_stage2"}


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def decode_nparts(T: int, BS: int, SBS: int) -> int:
    """Partial slots per query row (one per 512-token workgroup of the decode kernel)."""
    return int(N.lib().ffa_q2fp8_decode_nparts(int(T), int(BS), int(SBS)))


def decode_ntbs(T: int, BS: int, SBS: int) -> int:
    return _cdiv(T, BS) * _cdiv(BS, SBS)


def decode_pieces(HQ: int, HKV: int, T: int, BS: int, SBS: int) -> int:
    """Per-row slots of the two-pass scratch (GQA groups above 4 rows or SBS > 512), else 0."""
    return int(N.lib().ffa_q2fp8_decode_pieces(int(HQ), int(HKV), int(T), int(BS), int(SBS)))


class DecodeWorkspace:
    """Caller-owned scratch of one decode shape (graph-capture friendly).

    Mirrors Q2FP8DecodeWorkspace (ffa-q2fp8-h100/attn_kernel/attn_kernel_v1210_fused_bsz_q2fp8.py:232-257):
    o, m_buf, l_buf, o_buf, mask_buf, threshold_buf.  Partials are kept per
    512-token span (m_buf/l_buf [B, HQ, nparts], o_buf [B, HQ, nparts, 128]),
    mask_buf holds one byte per prune block [B, HKV, NTBS].  GQA groups of more
    than 4 query rows and prune blocks longer than 512 tokens decode in two
    passes and add piece_max [B, HQ, npieces] (the first pass's block maxima).
    approx_m / approx_l [B, HQ, nparts] hold the pruned tokens' softmax mass of the mean-V
    fallback (used only when a decode is given v_mean).
    """

    def __init__(self, B, HQ, HKV, T, BS, SBS, device, dtype):
        self.B, self.HQ, self.HKV, self.T = int(B), int(HQ), int(HKV), int(T)
        self.BS, self.SBS = int(BS), int(SBS)
        self.V = HEAD_DIM
        self.device = torch.device(device)
        self.dtype = dtype
        self.nparts = decode_nparts(T, BS, SBS)
        self.NTBS = decode_ntbs(T, BS, SBS)
        self.o = torch.empty((B, HQ, HEAD_DIM), device=device, dtype=dtype)
        self.m_buf = torch.empty((B, HQ, self.nparts), device=device, dtype=torch.float32)
        self.l_buf = torch.empty((B, HQ, self.nparts), device=device, dtype=torch.float32)
        self.o_buf = torch.empty((B, HQ, self.nparts, HEAD_DIM), device=device, dtype=torch.float32)
        self.mask_buf = torch.empty((B, HKV, self.NTBS), device=device, dtype=torch.int8)
        self.threshold_buf = torch.empty((B, HQ), device=device, dtype=torch.float32)
        self.npieces = decode_pieces(HQ, HKV, T, BS, SBS)
        self.piece_max = (torch.empty((B, HQ, self.npieces), device=device, dtype=torch.float32)
                          if self.npieces else None)
        self.approx_m = torch.empty((B, HQ, self.nparts), device=device, dtype=torch.float32)
        self.approx_l = torch.empty((B, HQ, self.nparts), device=device, dtype=torch.float32)

    def matches(self, B, HQ, HKV, T, BS, SBS, device, dtype) -> bool:
        return (
            self.B == int(B)
            and self.HQ == int(HQ)
            and self.HKV == int(HKV)
            and self.nparts >= decode_nparts(T, BS, SBS)
            and self.NTBS == decode_ntbs(T, BS, SBS)
            and self.npieces >= decode_pieces(HQ, HKV, T, BS, SBS)
            and self.device == torch.device(device)
            and self.dtype == dtype
        )


def _res_code(k_residual, use_res: bool) -> int:
    if not use_res:
        return N.DT_NONE
    if k_residual.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        return N.dtype_code(k_residual.dtype)
    raise ValueError(f"k_residual must be float8_e4m3fn or float8_e5m2, got {k_residual.dtype}")


def run_decode(*, workspace: DecodeWorkspace | None = None, stage: str = "both", **kw) -> DecodeWorkspace:
    """Launch one decode step; returns the workspace holding o / mask / thresholds.

    stage: "both" (stage 1 + stage 2), or "stage1" / "stage2" alone, the two launches of
    attn_forward_decode_quantized (attn_kernel...q2fp8.py:283-304).  Keyword arguments as
    decode_args.
    """
    if stage not in _STAGE_FN:
        raise ValueError(f"stage must be one of {sorted(_STAGE_FN)}")
    a, workspace = decode_args(workspace=workspace, **kw)
    fn = _STAGE_FN[stage]
    rc = getattr(N.lib(), fn)(ctypes.byref(a), ctypes.c_void_p(N.stream_of(kw["q"].device)))
    N.check(rc, fn)
    return workspace


_EXACT_ATTR = "_ffa_scales_exact_f16"


def scales_exact_f16(k_scale: torch.Tensor, k_zero: torch.Tensor) -> bool:
    """Whether every per-channel scale and zero point is exactly representable in fp16.

    The decode then dequantizes bf16 / fp32 scales as it does fp16 ones (one packed fp16 FMA per
    channel pair, the reference's k_hat for such values); otherwise it keeps fp32 arithmetic
    (attn_kernel_v1210_fused_bsz_q2fp8.py:52-53, 93).  fp16 tensors are exact by definition.  The
    answer is computed on the device once (a synchronising reduction) and remembered on the scale
    tensor (and its base) with both tensors' version counters, so that an in-place change of either
    checks again; during stream capture an unknown answer is False (fp32 arithmetic, correct for
    any values), as a capture cannot synchronise."""
    if k_scale.dtype == torch.float16 and k_zero.dtype == torch.float16:
        return True
    key = (k_scale.data_ptr(), tuple(k_scale.shape), k_scale._version, k_scale.dtype,
           k_zero.data_ptr(), tuple(k_zero.shape), k_zero._version, k_zero.dtype)
    for t in (k_scale, k_scale._base):
        memo = getattr(t, _EXACT_ATTR, None) if t is not None else None
        if memo is not None and memo[0] == key:
            return memo[1]
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        return False

    def exact(t):
        return bool(torch.equal(t.to(torch.float16).to(t.dtype), t))

    ok = exact(k_scale) and exact(k_zero)
    for t in (k_scale, k_scale._base):
        if t is not None:
            setattr(t, _EXACT_ATTR, (key, ok))
    return ok


def decode_args(
    *,
    q: torch.Tensor,  # [B, HQ, 128]
    k_q: torch.Tensor,
    k_scale: torch.Tensor,
    k_zero: torch.Tensor,
    v: torch.Tensor,
    k_residual,
    layout: int,
    scale_mode: int,
    T: int,
    HKV: int,
    scale: float,
    BS: int,
    SBS: int,
    delta: float,
    use_res: bool,
    precomputed_threshold=None,
    block_table=None,
    seq_lens=None,
    workspace: DecodeWorkspace | None = None,
    v_mean: torch.Tensor | None = None,
):
    """Validate one decode step and fill its C argument struct; returns (args, workspace).  The
    struct holds raw pointers of the tensors passed in: keep them alive until the call.

    v_mean [B, HKV, 128] (optional) turns on the mean-V fallback: pruned blocks keep their
    coarse-score softmax mass with v_mean as value (ffa-q2fp8-meanv/attn_kernel/
    attn_kernel_v1210_meanv_bsz_q2fp8.py:109-119, 156-202)."""
    B, HQ, D = q.shape
    if D != HEAD_DIM:
        raise NotImplementedError(f"head_dim {D} is not supported (this build implements {HEAD_DIM})")
    if v.shape[-1 if layout == N.LAYOUT_CONTIG else -2] != HEAD_DIM:
        raise NotImplementedError("value head dim must be 128")
    if workspace is None:
        workspace = DecodeWorkspace(B, HQ, HKV, T, BS, SBS, q.device, q.dtype)
    elif not workspace.matches(B, HQ, HKV, T, BS, SBS, q.device, q.dtype):
        raise ValueError("workspace shape/device/dtype mismatch")
    th_in = None
    if precomputed_threshold is not None:
        th_in = precomputed_threshold.to(torch.float32).contiguous()
    a = N.DecodeArgs()
    a.q = q.data_ptr()
    a.q_dtype = N.dtype_code(q.dtype)
    a.k_q = k_q.data_ptr()
    a.k_scale = k_scale.data_ptr()
    a.k_zero = k_zero.data_ptr()
    a.scale_dtype = N.dtype_code(k_scale.dtype)
    a.scale_mode = scale_mode
    if scale_mode == N.SCALE_CHANNEL and k_scale.dtype != torch.float16:
        a.scale_exact_f16 = 1 if scales_exact_f16(k_scale, k_zero) else 0
    a.k_residual = k_residual.data_ptr() if use_res else None
    a.res_dtype = _res_code(k_residual, use_res)
    a.v = v.data_ptr()
    a.v_dtype = N.dtype_code(v.dtype)
    a.layout = layout
    a.block_table = block_table.data_ptr() if block_table is not None else None
    a.bt_stride = block_table.shape[1] if block_table is not None else 0
    if layout == N.LAYOUT_PAGED:  # pages every pool holds: the kernels read ids beyond them as page 0
        pools = [k_q, v] + ([k_scale, k_zero] if scale_mode == N.SCALE_G32 else []) + ([k_residual] if use_res else [])
        a.num_pages = min(int(t.shape[0]) for t in pools)
    a.seq_lens = seq_lens.data_ptr() if seq_lens is not None else None
    a.B, a.T, a.HQ, a.HKV = B, int(T), HQ, int(HKV)
    a.scale = float(scale)
    a.BS, a.SBS = int(BS), int(SBS)
    a.delta = float(delta)
    a.threshold_in = th_in.data_ptr() if th_in is not None else None
    a.threshold_out = workspace.threshold_buf.data_ptr()
    a.out = workspace.o.data_ptr()
    a.out_dtype = N.dtype_code(workspace.o.dtype)
    a.m_buf = workspace.m_buf.data_ptr()
    a.l_buf = workspace.l_buf.data_ptr()
    a.o_buf = workspace.o_buf.data_ptr()
    a.nparts = workspace.nparts
    a.mask = workspace.mask_buf.data_ptr()
    a.ntbs = workspace.NTBS
    a.piece_max = workspace.piece_max.data_ptr() if workspace.piece_max is not None else None
    a.npieces = workspace.npieces
    if v_mean is not None:
        if tuple(v_mean.shape) != (B, int(HKV), HEAD_DIM) or v_mean.device != q.device:
            raise ValueError(f"v_mean must be [B, HKV, {HEAD_DIM}] on the query's device, got {tuple(v_mean.shape)}")
        if not v_mean.is_contiguous():
            raise ValueError("v_mean must be contiguous")
        a.v_mean = v_mean.data_ptr()
        a.v_mean_dtype = N.dtype_code(v_mean.dtype)
        a.approx_m = workspace.approx_m.data_ptr()
        a.approx_l = workspace.approx_l.data_ptr()
    a._keep = th_in  # the converted threshold must outlive the call
    return a, workspace


def skip_ratio_of(mask: torch.Tensor, seq_lens=None, BS=None, SBS=None) -> float:
    """1 - kept/total blocks (attn_kernel...q2fp8.py:293-297); ragged lengths count their own blocks."""
    kept = mask.to(torch.int32).sum()
    if seq_lens is None:
        total = mask.numel()
    else:
        HKV = mask.shape[1]
        total = sum(decode_ntbs(int(t), BS, SBS) for t in seq_lens.tolist()) * HKV
    return float((1.0 - kept.float() / float(total)).item())


def default_scale(D: int) -> float:
    return 1.0 / math.sqrt(D)
