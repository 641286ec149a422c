"""Host side of the mean-V fallback (ffa-q2fp8-meanv): v_mean and the approximated-block ratio.

In the mean-V variant a pruned block is not dropped: its softmax mass on the coarse (2-bit)
scores stays in the normalizer and its value is the mean of V over the sequence
(ffa-q2fp8-meanv/attn_kernel/attn_kernel_v1210_meanv_bsz_q2fp8.py:109-119, 156-202, 332).  The
decode kernels do this when given v_mean (decode.decode_args); this module computes v_mean with
the `ffa_v_mean` kernels and the variant's skip ratio.
"""
from __future__ import annotations

import math

import torch

from . import _native as N
from .decode import HEAD_DIM, decode_ntbs

PAGE = 64


def value_mean(v: torch.Tensor, *, block_table: torch.Tensor | None = None, seq_lens: torch.Tensor | None = None,
               T: int | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Mean over tokens of V, [B, HKV, 128] in out_dtype (default v.dtype), with fp32 sums
    (reference :332, v.mean(dim=1, dtype=torch.float32).to(v.dtype)).

    Contiguous: v [B, T, HKV, 128].  Paged: v is the V^T pool [P, HKV, 128, 64] and block_table
    [B, n] names each sequence's pages; T defaults to the table's capacity.  seq_lens [B]
    (optional) gives each sequence's own length; an empty sequence's mean is 0."""
    if v.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"v must be float16 or bfloat16, got {v.dtype}")
    if not v.is_contiguous():
        raise ValueError("v must be contiguous")
    out_dtype = v.dtype if out_dtype is None else out_dtype
    if block_table is None:
        if v.ndim != 4 or v.shape[-1] != HEAD_DIM:
            raise ValueError(f"v must be [B, T, HKV, {HEAD_DIM}], got {tuple(v.shape)}")
        B, Tv, HKV, _ = v.shape
        T = Tv
        layout, bt_ptr, bt_stride, num_pages = N.LAYOUT_CONTIG, None, 0, 0
    else:
        if v.ndim != 4 or tuple(v.shape[2:]) != (HEAD_DIM, PAGE):
            raise ValueError(f"paged v must be [P, HKV, {HEAD_DIM}, {PAGE}] (V^T pages), got {tuple(v.shape)}")
        block_table = block_table.to(device=v.device, dtype=torch.int32).contiguous()
        B, HKV = block_table.shape[0], v.shape[1]
        T = int(block_table.shape[1]) * PAGE if T is None else int(T)
        if T > block_table.shape[1] * PAGE:
            raise ValueError("T exceeds the block table's capacity")
        layout, bt_ptr, bt_stride, num_pages = N.LAYOUT_PAGED, block_table.data_ptr(), block_table.shape[1], v.shape[0]
    if seq_lens is not None:
        seq_lens = seq_lens.to(device=v.device, dtype=torch.int32).contiguous()
    out = torch.empty((B, HKV, HEAD_DIM), device=v.device, dtype=out_dtype)
    nsplit = int(N.lib().ffa_v_mean_nsplit(int(T)))
    partial = torch.empty((B, HKV, max(nsplit, 1), HEAD_DIM), device=v.device, dtype=torch.float32)
    rc = N.lib().ffa_v_mean(v.data_ptr(), N.dtype_code(v.dtype), layout, bt_ptr, bt_stride, num_pages,
                            N.ptr(seq_lens), B, int(T), HKV, partial.data_ptr(), max(nsplit, 1), out.data_ptr(),
                            N.dtype_code(out_dtype), N.stream_of(v.device))
    N.check(rc, "ffa_v_mean")
    return out


def approx_ratio(mask: torch.Tensor, T: int, BS: int, SBS: int, seq_lens=None) -> float:
    """Fraction of prune blocks that the mean-V variant approximates: pruned blocks that hold
    tokens (reference :119 sets the approx flag there, :326-330's ratio is approx.sum() /
    approx.numel()); ragged lengths count their own blocks."""
    B, HKV, _ = mask.shape
    kept = int(mask.to(torch.int64).sum().item())
    if seq_lens is None:
        with_tokens = B * HKV * math.ceil(T / SBS)
        total = mask.numel()
    else:
        lens = [min(max(int(t), 0), T) for t in seq_lens.tolist()]
        with_tokens = HKV * sum(math.ceil(t / SBS) for t in lens)
        total = HKV * sum(decode_ntbs(t, BS, SBS) for t in lens)
    return max(with_tokens - kept, 0) / max(total, 1)


def approx_flags(mask: torch.Tensor, T: int, BS: int, SBS: int, seq_lens=None):
    """The mean-V variant's per-block flags, from the survivor mask the decode writes (1 = refined
    exactly): approx = pruned blocks that hold tokens (reference :117-119 writes approx_buf = 1 there,
    :151-152 writes 0 for exact blocks), and the variant's own mask_buf = exact or approximated
    (reference :118, :151).  Returns (mask_meanv, approx), int8 [B, HKV, NTBS]; blocks past a
    sequence's last token are 0 in both."""
    B, HKV, NTBS = mask.shape
    lens = [T] * B if seq_lens is None else [min(max(int(t), 0), T) for t in seq_lens.tolist()]
    nblk = torch.tensor([math.ceil(t / SBS) for t in lens], device=mask.device)
    has_tokens = torch.arange(NTBS, device=mask.device)[None, :] < nblk[:, None]  # [B, NTBS]
    kept = mask != 0
    approx = has_tokens[:, None, :] & ~kept
    return (kept | approx).to(torch.int8), approx.to(torch.int8)
