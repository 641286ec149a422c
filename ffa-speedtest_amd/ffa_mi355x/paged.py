"""Paged q2fp8 KV cache (64-token pages) and its decode / append entry points.

The reference keeps one contiguous [B, T, HKV, D] cache per batch
(ffa-q2fp8/attn_kernel/attn_kernel_v1210_fused_bsz_q2fp8.py:192-197).  This
build adds a page pool shared by all sequences, laid out for the gfx950
kernels (all per (page, KV head) blocks contiguous):

    k_q      [P, HKV, 4, 64, 8]  u8    2-bit codes, group-major (32 codes/8 bytes per token and group)
    k_scale  [P, HKV, 4, 64]     f16   g32 scale per token and group (slot order below)
    k_zero   [P, HKV, 4, 64]     f16   g32 zero point (slot order below)
    k_res    [P, HKV, 64, 128]   fp8   residual (e4m3fn by default)
    v        [P, HKV, 128, 64]   fp16  V^T pages (token-minor); fp16 by default, since the decode
                                       computes P.V on fp16(V) as the reference does (bf16 pages
                                       are accepted and rounded to fp16 in registers)

block_table[b, i] is the pool page of tokens [64 i, 64 i + 64) of sequence b;
seq_lens[b] is its length.  Token t of a page keeps its scale/zero in slot
scale_pos(t) = 16*(t//16) + 4*(t%4) + (t//4)%4 (the order the decode kernel's
MFMA tiles consume them in).  Inside each (page, head) block the data are stored in
the order the decode's load instructions read them (every instruction reads whole
1 KB / 256 B blocks): RES_ORDER, VT_ORDER, CODES_ORDER, GSCALE_ORDER and K4_ORDER
give the position of each logical element (the mirror of decode_common.h);
`to_logical` / `to_tiled` convert whole pools.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import _native as N
from .decode import HEAD_DIM, DecodeWorkspace, run_decode

PAGE = 64


def _orders():
    t = np.arange(64)[:, None]
    c = np.arange(128)[None, :]
    res = (((t & 3) * 2 + ((c >> 4) & 1)) * 64 + (c >> 5) * 16 + (t >> 2)) * 16 + (c & 15)  # [t, c] byte
    cc = np.arange(128)[:, None]
    tt = np.arange(64)[None, :]
    vt = (((cc >> 4) * 2 + ((tt >> 3) & 1)) * 64 + (tt >> 4) * 16 + (cc & 15)) * 8 + (tt & 7)  # [c, t] element
    g = np.arange(4)[:, None]
    codes = ((((tt >> 1) & 1) * 64 + g * 16 + (tt >> 2)) * 2 + (tt & 1))  # [g, t] 8-byte unit
    gscale = ((((tt >> 3) & 1) * 4 + g) * 4 + (tt >> 4)) * 8 + (tt & 7)  # [g, slot] element
    b = np.arange(64)[None, :]
    k4 = ((t & 3) * 64 + (b >> 4) * 16 + (t >> 2)) * 16 + (b & 15)  # [t, byte] byte
    return res, vt, codes, gscale, k4


RES_ORDER, VT_ORDER, CODES_ORDER, GSCALE_ORDER, K4_ORDER = _orders()


def to_tiled(logical: np.ndarray, order: np.ndarray, unit: int = 1) -> np.ndarray:
    """Pool in logical page order [..., *order.shape (, unit)] -> the stored order (same shape)."""
    lead = logical.shape[: logical.ndim - order.ndim - (1 if unit > 1 else 0)]
    flat = logical.reshape(lead + (order.size, unit))
    out = np.empty_like(flat)
    out[..., order.ravel(), :] = flat
    return out.reshape(logical.shape)


def to_logical(stored: np.ndarray, order: np.ndarray, unit: int = 1) -> np.ndarray:
    """Pool in stored order -> logical page order (inverse of to_tiled)."""
    lead = stored.shape[: stored.ndim - order.ndim - (1 if unit > 1 else 0)]
    flat = stored.reshape(lead + (order.size, unit))
    return flat[..., order.ravel(), :].reshape(stored.shape)


def scale_pos(t):
    """Slot of token t (0..63) in a page row of g32 scales / zeros (an involution)."""
    return 16 * (t // 16) + 4 * (t % 4) + (t // 4) % 4


def check_append_fits(pos: torch.Tensor, Tn: int, block_table: torch.Tensor, num_pages: int) -> None:
    """Host-side bounds check of an append (positions and page ids must stay inside the table / pool)."""
    if block_table.shape[0] != pos.shape[0]:
        raise ValueError("block_table must have one row per sequence")
    last = int(pos.max().item()) + Tn - 1
    if int(pos.min().item()) < 0 or last >= block_table.shape[1] * PAGE:
        raise ValueError("append positions exceed the block table")
    used = block_table[:, : last // PAGE + 1]
    if int(used.min().item()) < 0 or int(used.max().item()) >= num_pages:
        raise ValueError("block table references pages outside the pool")


class PagedQ2Cache:
    def __init__(self, num_pages, HKV, device, res_dtype=torch.float8_e4m3fn, v_dtype=torch.float16):
        self.P, self.HKV = int(num_pages), int(HKV)
        self.device = torch.device(device)
        self.res_dtype, self.v_dtype = res_dtype, v_dtype
        P, H = self.P, self.HKV
        self.k_q = torch.zeros((P, H, 4, PAGE, 8), dtype=torch.uint8, device=device)
        self.k_scale = torch.zeros((P, H, 4, PAGE), dtype=torch.float16, device=device)
        self.k_zero = torch.zeros((P, H, 4, PAGE), dtype=torch.float16, device=device)
        self.k_res = torch.zeros((P, H, PAGE, HEAD_DIM), dtype=res_dtype, device=device)
        self.v = torch.zeros((P, H, HEAD_DIM, PAGE), dtype=v_dtype, device=device)

    def nbytes_per_page(self) -> int:
        return sum(t[0].numel() * t.element_size() for t in (self.k_q, self.k_scale, self.k_zero, self.k_res, self.v))

    # ------------------------------------------------------------------ writes
    def append(self, k: torch.Tensor, v: torch.Tensor | None, pos: torch.Tensor, block_table: torch.Tensor):
        """g32-quantize k [B, Tn, HKV, 128] and write it (and v) at positions pos[b] + n."""
        B, Tn, HKV, D = k.shape
        if HKV != self.HKV or D != HEAD_DIM:
            raise ValueError("k shape does not match the cache")
        k = k.contiguous()
        if v is not None:
            if v.shape != k.shape:
                raise ValueError("v must have the shape of k")
            v = v.to(self.v_dtype).contiguous()
        pos = pos.to(torch.int32).contiguous()
        block_table = block_table.to(torch.int32).contiguous()
        check_append_fits(pos, Tn, block_table, self.P)
        rc = N.lib().ffa_q2_quantize_g32_append(
            k.data_ptr(), N.dtype_code(k.dtype), B, Tn, HKV, pos.data_ptr(), block_table.data_ptr(),
            block_table.shape[1], self.P, self.k_q.data_ptr(), self.k_scale.data_ptr(), self.k_zero.data_ptr(),
            self.k_res.data_ptr(), N.dtype_code(self.res_dtype), N.ptr(v), self.v.data_ptr(),
            N.stream_of(k.device))
        N.check(rc, "ffa_q2_quantize_g32_append")

    def dequantize(self, block_table: torch.Tensor, T: int, seq_lens: torch.Tensor | None = None,
                   out_dtype: torch.dtype = torch.float32):
        """K and V [B, T', HKV, 128] of the first T tokens of every sequence (T' = T rounded up to a
        page), K = codes * scale + zero + residual in fp32 rounded once to out_dtype, V from the V^T
        pages; tokens at or past seq_lens[b] are zeros.  The keys an exact attention over the cache
        sees (the reference returns its cache's dequantized keys from update: ffa-fp8fp8/e2e/
        fp8fp8_cache.py:60-69, 84-89)."""
        block_table = block_table.to(torch.int32).contiguous()
        B = block_table.shape[0]
        Tp = -(-int(T) // PAGE) * PAGE
        if Tp > block_table.shape[1] * PAGE:
            raise ValueError("T exceeds the block table")
        if seq_lens is not None:
            seq_lens = seq_lens.to(device=self.device, dtype=torch.int32).contiguous()
        k = torch.empty((B, Tp, self.HKV, HEAD_DIM), dtype=out_dtype, device=self.device)
        v = torch.empty_like(k)
        rc = N.lib().ffa_q2_paged_dequant(
            self.k_q.data_ptr(), self.k_scale.data_ptr(), self.k_zero.data_ptr(), self.k_res.data_ptr(),
            N.dtype_code(self.res_dtype), self.v.data_ptr(), N.dtype_code(self.v_dtype), block_table.data_ptr(),
            block_table.shape[1], self.P, N.ptr(seq_lens), B, Tp, self.HKV, k.data_ptr(), v.data_ptr(),
            N.dtype_code(out_dtype), N.stream_of(self.device))
        N.check(rc, "ffa_q2_paged_dequant")
        return k, v

    # ------------------------------------------------------------------ decode
    def value_mean(self, block_table, seq_lens=None, *, T=None, out_dtype=None):
        """Mean over each sequence's tokens of its V pages, [B, HKV, 128] (the mean-V fallback's v_mean)."""
        from .meanv import value_mean

        return value_mean(self.v, block_table=block_table, seq_lens=seq_lens, T=T, out_dtype=out_dtype)

    def decode(self, q, block_table, seq_lens=None, *, T=None, scale=None, BS=64, SBS=None, delta=5.0,
               precomputed_threshold=None, use_fp8_residual=True, workspace: DecodeWorkspace | None = None,
               stage="both", v_mean=None):
        """Pruned decode of q [B, HQ, 128] (or [B, 1, HQ, 128]) over the paged cache.

        stage: "both", or "stage1" (scores, prune, exact partials) / "stage2" (merge) alone.
        v_mean [B, HKV, 128] (optional): the mean-V fallback (pruned blocks keep their coarse-score
        mass with v_mean as value), e.g. from value_mean().
        """
        if q.ndim == 4:
            if q.shape[1] != 1:
                raise AssertionError("decode takes one query token per sequence")
            q = q[:, 0]
        q = q.contiguous()
        B, HQ, D = q.shape
        SBS = BS if SBS is None else SBS
        block_table = block_table.to(torch.int32).contiguous()
        if seq_lens is not None:
            seq_lens = seq_lens.to(torch.int32).contiguous()
        if T is None:
            if seq_lens is None:
                raise ValueError("give T or seq_lens")
            T = int(seq_lens.max().item())
        if block_table.shape[0] != B or block_table.shape[1] * PAGE < T:
            raise ValueError("block_table must be [B, >= ceil(T/64)]")
        scale = 1.0 / math.sqrt(D) if scale is None else scale
        return run_decode(
            q=q, k_q=self.k_q, k_scale=self.k_scale, k_zero=self.k_zero, v=self.v, k_residual=self.k_res,
            layout=N.LAYOUT_PAGED, scale_mode=N.SCALE_G32, T=T, HKV=self.HKV, scale=scale, BS=BS, SBS=SBS,
            delta=delta, use_res=use_fp8_residual, precomputed_threshold=precomputed_threshold,
            block_table=block_table, seq_lens=seq_lens, workspace=workspace, stage=stage, v_mean=v_mean)
