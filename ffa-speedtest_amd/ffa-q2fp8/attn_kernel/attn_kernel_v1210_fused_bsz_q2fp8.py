# attn_kernel_v1210_fused_bsz_q2fp8.py -- MI355X drop-in.
# 2-bit quantized K with fp8 residual refinement; the kernels are hand-written
# HIP for gfx950 in libffa_mi355x.so (no Triton).
"""Drop-in for ffa-q2fp8/attn_kernel/attn_kernel_v1210_fused_bsz_q2fp8.py.

`attn_forward_decode_quantized` keeps the reference signature, tensor layouts,
defaults and exception types (reference :191-309).  The H100 variant's
workspace API (ffa-q2fp8-h100/attn_kernel/attn_kernel_v1210_fused_bsz_q2fp8.py:232-277,
295, 359-376) is available too.

Extensions, all through **kwargs (reference :206):
  block_table=[B, npages] int32  -> paged cache (ffa_mi355x.paged layout): k_q,
                                    k_scale, k_zero, k_residual and v are the page
                                    pools; k_scale/k_zero [P,HKV,4,64] fp16 (g32).
  seq_lens=[B] int32             -> ragged lengths.
  T=int                          -> longest length a paged call may see; default the block
                                    table's capacity, block_table.shape[1] * 64 (lengths past
                                    T are clamped to T).
"""
import math
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))  # ffa-speedtest_amd/
from ffa_mi355x import _native as _N  # noqa: E402
from ffa_mi355x.decode import DecodeWorkspace, decode_ntbs, run_decode  # noqa: E402

__all__ = [
    "attn_forward_decode_quantized",
    "Q2FP8DecodeWorkspace",
    "allocate_q2fp8_decode_workspace",
]


class Q2FP8DecodeWorkspace(DecodeWorkspace):
    """Reusable scratch (ffa-q2fp8-h100 ...q2fp8.py:232-257); attributes o, m_buf, l_buf,
    o_buf, mask_buf, threshold_buf.  Partials are kept per 512-token span here."""

    def __init__(self, B, HQ, HKV, V, T, BS, SBS, device, dtype):
        if V != 128:
            raise NotImplementedError("value head dim must be 128")
        super().__init__(B, HQ, HKV, T, BS, SBS, device, dtype)


def allocate_q2fp8_decode_workspace(q, k_q, v, BS: int = 128, SBS=None, **kwargs) -> Q2FP8DecodeWorkspace:
    """ffa-q2fp8-h100 ...q2fp8.py:260-277 (plus block_table/T for paged caches)."""
    B, Tq, HQ, _ = q.shape
    if SBS is None:
        SBS = BS
    if kwargs.get("block_table") is not None:
        HKV = k_q.shape[1]
        V = v.shape[2]
        T = _paged_T(kwargs["block_table"], kwargs.get("T"))
        if Tq != 1:
            raise ValueError("K/V layouts must be [B, T, HKV, D]")
    else:
        Bk, T, HKV, _ = k_q.shape
        Bv, Tv, HKVv, V = v.shape
        if B != Bk or B != Bv or Tq != 1 or T != Tv or HKV != HKVv:
            raise ValueError("K/V layouts must be [B, T, HKV, D]")
    return Q2FP8DecodeWorkspace(B, HQ, HKV, V, T, BS, SBS, q.device, q.dtype)


def _paged_T(block_table: torch.Tensor, T=None) -> int:
    """Longest length of a paged call: the caller's T, else the block table's capacity (no host sync,
    and the same value for a workspace allocated ahead and for the calls that use it)."""
    return int(T) if T is not None else int(block_table.shape[1]) * 64


def _check_paged_pools(q, k_q, k_scale, k_zero, v, k_residual, g32: bool) -> None:
    """Shapes and dtypes of the page pools (ffa_mi355x.paged): k_q [P, HKV, 4, 64, 8] u8, g32
    k_scale / k_zero [P, HKV, 4, 64] fp16 (or per-channel [B, HKV, 128]), k_residual
    [P, HKV, 64, 128] fp8, v [P, HKV, 128, 64] (V^T pages)."""
    assert q.is_contiguous() and k_q.is_contiguous() and v.is_contiguous(), "paged pools and q must be contiguous"
    if k_q.ndim != 5 or tuple(k_q.shape[2:]) != (4, 64, 8) or k_q.dtype != torch.uint8:
        raise ValueError(f"paged k_q must be [P, HKV, 4, 64, 8] uint8, got {tuple(k_q.shape)} {k_q.dtype}")
    P, HKV = k_q.shape[:2]
    if v.ndim != 4 or v.shape[1] != HKV or tuple(v.shape[2:]) != (128, 64):
        raise ValueError(f"paged v must be [P, HKV, 128, 64] (V^T pages), got {tuple(v.shape)}")
    if g32:
        for name, t in (("k_scale", k_scale), ("k_zero", k_zero)):
            if t.ndim != 4 or t.shape[1] != HKV or tuple(t.shape[2:]) != (4, 64) or t.dtype != torch.float16:
                raise ValueError(f"paged g32 {name} must be [P, HKV, 4, 64] float16, got {tuple(t.shape)} {t.dtype}")
            assert t.is_contiguous(), f"{name} must be contiguous"
    if k_residual is not None:
        if k_residual.ndim != 4 or k_residual.shape[1] != HKV or tuple(k_residual.shape[2:]) != (64, 128):
            raise ValueError(f"paged k_residual must be [P, HKV, 64, 128], got {tuple(k_residual.shape)}")
        assert k_residual.is_contiguous(), "k_residual must be contiguous"


def _normalize_scale_zero(k_scale: torch.Tensor, k_zero: torch.Tensor, expect_shape):
    """Ensure scale / zero_point tensors are contiguous and have shape [B, HKV, K] (reference :174-188)."""
    if k_scale.ndim == 4 and k_scale.shape[1] == 1:
        k_scale = k_scale.squeeze(1)
    if k_zero.ndim == 4 and k_zero.shape[1] == 1:
        k_zero = k_zero.squeeze(1)
    if k_scale.shape != expect_shape or k_zero.shape != expect_shape:
        raise ValueError(
            f"Unsupported k_scale/k_zero shapes: {k_scale.shape=} {k_zero.shape=}, expected {expect_shape}"
        )
    return k_scale.contiguous(), k_zero.contiguous()


def _decode(q, k_q, k_scale, k_zero, v, k_residual, k_bits, scale, BS, SBS, delta, precomputed_threshold,
            use_fp8_residual, workspace, v_mean_of=None, **kwargs):
    """Argument checks of reference :211-281 and one decode; returns (workspace, seq_lens, HKV, T, BS, SBS).

    v_mean_of(v, layout, block_table, seq_lens, T) (optional, after the checks) gives the mean-V
    fallback's v_mean [B, HKV, 128]."""
    assert q.is_cuda and k_q.is_cuda and v.is_cuda
    if k_residual is not None and not k_residual.is_cuda:
        raise ValueError("k_residual must be a CUDA tensor when provided")
    if k_bits != 2:
        raise ValueError(f"attn_forward_decode_quantized currently supports 2-bit keys, got k_bits={k_bits}")
    assert k_scale.is_cuda and k_zero.is_cuda, "k_scale/k_zero must be CUDA tensors"
    if not k_scale.is_floating_point() or not k_zero.is_floating_point():
        raise ValueError("k_scale and k_zero must be floating point tensors for dequantization")
    if k_q.is_floating_point():
        raise ValueError("k_q must contain integer quantized values (e.g., uint8/int8)")
    if k_residual is not None and not k_residual.is_floating_point():
        raise ValueError("k_residual must be a floating point tensor (e.g., fp8/fp16/bf16)")

    block_table = kwargs.get("block_table")
    seq_lens = kwargs.get("seq_lens")
    B, Tq, HQ, K = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(K)
    if SBS is None:
        SBS = BS
    if use_fp8_residual and k_residual is None:
        raise ValueError("use_fp8_residual=True requires k_residual")
    use_res = bool(use_fp8_residual and k_residual is not None)
    assert Tq == 1, "K/V layouts must be [B, T, HKV, D]"

    if block_table is None:
        Bk, T, HKV, K_packed = k_q.shape
        Bv, Tv, HKVv, V = v.shape
        vals_per_byte = 8 // k_bits
        expected_k_packed = (K + vals_per_byte - 1) // vals_per_byte
        if K_packed != expected_k_packed:
            raise ValueError(
                f"k_q packed dim mismatch: got {K_packed}, expected {expected_k_packed} for K={K}, k_bits={k_bits}")
        if k_residual is not None:
            Bk_r, T_r, HKV_r, K_r = k_residual.shape
            assert (B == Bk == Bv == Bk_r and Tv == T == T_r and HKVv == HKV == HKV_r and K == K_r), \
                "K/V layouts must be [B, T, HKV, D]"
        else:
            assert B == Bk == Bv and Tv == T and HKVv == HKV, "K/V layouts must be [B, T, HKV, D]"
        k_scale, k_zero = _normalize_scale_zero(k_scale, k_zero, (B, HKV, K))
        assert q.is_contiguous() and k_q.is_contiguous() and v.is_contiguous()
        if k_residual is not None:
            assert k_residual.is_contiguous()
        if seq_lens is not None:
            seq_lens = seq_lens.to(device=q.device, dtype=torch.int32).contiguous()
        layout, smode = _N.LAYOUT_CONTIG, _N.SCALE_CHANNEL
    else:
        smode = _N.SCALE_G32 if k_scale.ndim == 4 else _N.SCALE_CHANNEL
        _check_paged_pools(q, k_q, k_scale, k_zero, v, k_residual if use_res else None, smode == _N.SCALE_G32)
        HKV = k_q.shape[1]
        if smode == _N.SCALE_CHANNEL:
            k_scale, k_zero = _normalize_scale_zero(k_scale, k_zero, (B, HKV, K))
        block_table = block_table.to(device=q.device, dtype=torch.int32).contiguous()
        if seq_lens is not None:
            seq_lens = seq_lens.to(device=q.device, dtype=torch.int32).contiguous()
        T = _paged_T(block_table, kwargs.get("T"))
        layout = _N.LAYOUT_PAGED
    if precomputed_threshold is not None:
        assert precomputed_threshold.is_cuda and precomputed_threshold.shape == (B, HQ)

    if workspace is not None and not isinstance(workspace, DecodeWorkspace):
        raise TypeError("workspace must be a Q2FP8DecodeWorkspace")
    v_mean = v_mean_of(v, layout, block_table, seq_lens, T) if v_mean_of is not None else None
    ws = run_decode(
        q=q[:, 0], k_q=k_q, k_scale=k_scale, k_zero=k_zero, v=v, k_residual=k_residual, layout=layout,
        scale_mode=smode, T=T, HKV=HKV, scale=scale, BS=BS, SBS=SBS, delta=delta, use_res=use_res,
        precomputed_threshold=precomputed_threshold, block_table=block_table, seq_lens=seq_lens,
        workspace=workspace, v_mean=v_mean)
    return ws, seq_lens, HKV, T, BS, SBS


def attn_forward_decode_quantized(
    q: torch.Tensor,           # [B, 1, HQ, K]
    k_q: torch.Tensor,         # [B, T, HKV, ceil(K / (8 / k_bits))], packed quantized ints
    k_scale: torch.Tensor,     # [B, HKV, K] (token dimension removed)
    k_zero: torch.Tensor,      # same shape as k_scale
    v: torch.Tensor,           # [B, T, HKV, V]
    k_residual: torch.Tensor | None = None,  # [B, T, HKV, K], fp8 residual
    k_bits: int = 2,
    scale: float = None,
    BS: int = 128,
    SBS: int | None = None,
    delta: float = 5.0,
    return_skip_ratio: bool = False,
    precomputed_threshold: torch.Tensor | None = None,
    use_fp8_residual: bool = True,
    workspace: Q2FP8DecodeWorkspace | None = None,
    **kwargs,
):
    ws, seq_lens, HKV, T, BS, SBS = _decode(q, k_q, k_scale, k_zero, v, k_residual, k_bits, scale, BS, SBS, delta,
                                           precomputed_threshold, use_fp8_residual, workspace, **kwargs)
    o = ws.o

    if return_skip_ratio:
        mask_buf = ws.mask_buf
        kept = mask_buf.to(torch.int32).sum()
        if seq_lens is None:
            total = mask_buf.numel()
        else:
            total = sum(decode_ntbs(int(t), BS, SBS) for t in seq_lens.tolist()) * HKV
        skip_ratio = float((1.0 - (kept.float() / float(total))).item())
        return o, skip_ratio
    return o
