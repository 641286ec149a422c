"""Paged nvfp4 / nf4 KV caches (64-token pages, per-token group scales; no reference counterpart).

The reference keeps one contiguous cache per batch with one nvfp4 scale per
(sequence, BS-token block, KV head) or one nf4 scale per (sequence, KV head, channel)
(ffa-nvfp4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nvfp4fp8.py:225-231,
ffa-nf4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nf4fp8.py:212-217).  These caches keep
one page pool shared by all sequences, with scales along head_dim instead:

    k        [P, HKV, 64, 64]   u8    packed 4-bit codes, token-major (low nibble first)
    k_scale  [P, HKV, 64, 8]    e4m3  nvfp4: scale of each 16-channel block
             [P, HKV, 64, 2]    f16   nf4:   absmax scale of each 64-channel block
    k_res    [P, HKV, 64, 128]  fp8   residual (e4m3fn by default)
    v        [P, HKV, 128, 64]  fp16  V^T pages (token-minor; fp16 by default, the P.V operand type)

block_table[b, i] is the pool page of tokens [64 i, 64 i + 64) of sequence b.
Quantization rules: ffa_nvfp4_g16_append / ffa_nf4_g64_append in include/ffa_mi355x.h.
"""
from __future__ import annotations

import math

import torch

from . import _native as N
from .decode import HEAD_DIM, DecodeWorkspace
from .kfmt import run_kfmt_decode
from .paged import PAGE, check_append_fits

FORMATS = ("nvfp4", "nf4")


def decode_pools(fmt, q, k, k_scale, v, k_res, block_table, seq_lens=None, *, T=None, scale=None, BS=64, SBS=None,
                 delta=5.0, precomputed_threshold=None, use_fp8_residual=True,
                 workspace: DecodeWorkspace | None = None) -> DecodeWorkspace:
    """Pruned decode of q [B, HQ, 128] (or [B, 1, HQ, 128]) over the page pools above."""
    if fmt not in FORMATS:
        raise ValueError(f"fmt must be one of {FORMATS}")
    if q.ndim == 4:
        if q.shape[1] != 1:
            raise AssertionError("decode takes one query token per sequence")
        q = q[:, 0]
    q = q.contiguous()
    B, HQ, D = q.shape
    P, HKV = k.shape[0], k.shape[1]
    want_scale = (P, HKV, PAGE, 8) if fmt == "nvfp4" else (P, HKV, PAGE, 2)
    if k.shape != (P, HKV, PAGE, HEAD_DIM // 2) or k.dtype != torch.uint8:
        raise ValueError(f"k must be a uint8 pool [P, HKV, 64, 64], got {tuple(k.shape)} {k.dtype}")
    if tuple(k_scale.shape) != want_scale:
        raise ValueError(f"k_scale must be {want_scale}, got {tuple(k_scale.shape)}")
    if v.shape != (P, HKV, HEAD_DIM, PAGE):
        raise ValueError(f"v must be a V^T pool [P, HKV, 128, 64], got {tuple(v.shape)}")
    use_res = bool(use_fp8_residual)
    if use_res and (k_res is None or k_res.shape != (P, HKV, PAGE, HEAD_DIM)):
        raise ValueError("use_fp8_residual=True needs a residual pool [P, HKV, 64, 128]")
    SBS = BS if SBS is None else SBS
    block_table = block_table.to(torch.int32).contiguous()
    if seq_lens is not None:
        seq_lens = seq_lens.to(device=q.device, dtype=torch.int32).contiguous()
    if T is None:
        if seq_lens is None:
            raise ValueError("give T or seq_lens")
        T = int(seq_lens.max().item())
    if block_table.shape[0] != B or block_table.shape[1] * PAGE < T:
        raise ValueError("block_table must be [B, >= ceil(T/64)]")
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    if fmt == "nvfp4":
        if k_scale.dtype not in (torch.uint8, torch.float8_e4m3fn):
            raise ValueError("nvfp4 page scales are e4m3 bytes")
        # the kernel reads the e4m3 bytes directly; the ABI's float scale dtype is not used by them
        ks, kf, sk = k_scale.contiguous().view(torch.uint8).view(torch.float16), N.KFMT_NVFP4, N.KSCALE_G16
    else:
        if k_scale.dtype != torch.float16:
            raise ValueError("nf4 page scales are fp16")
        ks, kf, sk = k_scale.contiguous(), N.KFMT_NF4, N.KSCALE_G64
    ws = run_kfmt_decode(q=q, k=k.contiguous(), k_format=kf, k_scale=ks, scale_kind=sk, v=v.contiguous(),
                         k_residual=k_res, use_res=use_res, T=T, HKV=HKV, scale=scale, BS=BS, SBS=SBS, delta=delta,
                         precomputed_threshold=precomputed_threshold, seq_lens=seq_lens, workspace=workspace,
                         layout=N.LAYOUT_PAGED, block_table=block_table)
    return ws


class PagedKfmtCache:
    """Page pools of one format ("nvfp4" or "nf4"), with append (quantize + write) and decode."""

    def __init__(self, fmt, num_pages, HKV, device, res_dtype=torch.float8_e4m3fn, v_dtype=torch.float16):
        if fmt not in FORMATS:
            raise ValueError(f"fmt must be one of {FORMATS}")
        self.fmt = fmt
        self.P, self.HKV = int(num_pages), int(HKV)
        self.device = torch.device(device)
        self.res_dtype, self.v_dtype = res_dtype, v_dtype
        P, H = self.P, self.HKV
        self.k = torch.zeros((P, H, PAGE, HEAD_DIM // 2), dtype=torch.uint8, device=device)
        if fmt == "nvfp4":
            self.k_scale = torch.zeros((P, H, PAGE, 8), dtype=torch.float8_e4m3fn, device=device)
        else:
            self.k_scale = torch.zeros((P, H, PAGE, 2), dtype=torch.float16, device=device)
        self.k_res = torch.zeros((P, H, PAGE, HEAD_DIM), dtype=res_dtype, device=device)
        self.v = torch.zeros((P, H, HEAD_DIM, PAGE), dtype=v_dtype, device=device)

    def nbytes_per_page(self) -> int:
        return sum(t[0].numel() * t.element_size() for t in (self.k, self.k_scale, self.k_res, self.v))

    def append(self, k: torch.Tensor, v: torch.Tensor | None, pos: torch.Tensor, block_table: torch.Tensor):
        """Quantize k [B, Tn, HKV, 128] and write it (and v) at positions pos[b] + n."""
        B, Tn, HKV, D = k.shape
        if HKV != self.HKV or D != HEAD_DIM:
            raise ValueError("k shape does not match the cache")
        k = k.contiguous()
        if v is not None:
            if v.shape != k.shape:
                raise ValueError("v must have the shape of k")
            v = v.to(self.v_dtype).contiguous()
        pos = pos.to(device=k.device, dtype=torch.int32).contiguous()
        block_table = block_table.to(device=k.device, dtype=torch.int32).contiguous()
        check_append_fits(pos, Tn, block_table, self.P)
        fn = N.lib().ffa_nvfp4_g16_append if self.fmt == "nvfp4" else N.lib().ffa_nf4_g64_append
        rc = fn(k.data_ptr(), N.dtype_code(k.dtype), B, Tn, HKV, pos.data_ptr(), block_table.data_ptr(),
                block_table.shape[1], self.P, self.k.data_ptr(), self.k_scale.data_ptr(), self.k_res.data_ptr(),
                N.dtype_code(self.res_dtype), N.ptr(v), self.v.data_ptr(), N.stream_of(k.device))
        N.check(rc, f"ffa_{self.fmt}_append")

    def decode(self, q, block_table, seq_lens=None, **kw) -> DecodeWorkspace:
        return decode_pools(self.fmt, q, self.k, self.k_scale, self.v, self.k_res, block_table, seq_lens, **kw)
