"""Host side of the 2-bit K quantizers and the fused K-proj + RoPE producers."""
from __future__ import annotations

import torch

from . import _native as N
from .paged import PagedQ2Cache, check_append_fits


def _normalize_k_weight(w_k: torch.Tensor, in_dim: int) -> torch.Tensor:
    """Accept W_k as [out, in] or [in, out] (ffa-q2fp8/fused_kproj_rope_q2fp8.py:71-78)."""
    if w_k.ndim != 2:
        raise ValueError(f"w_k must be 2D, got {w_k.shape}")
    if w_k.shape[1] == in_dim:
        return w_k
    if w_k.shape[0] == in_dim:
        return w_k.t().contiguous()
    raise ValueError(f"w_k shape {w_k.shape} is incompatible with in_dim={in_dim}")


def quantize_per_channel(k: torch.Tensor, fp8_dtype=torch.float8_e5m2):
    """Reference quantizer on the GPU, bit-exact with ffa-q2fp8/run_attn_bench_q2.py:78-105.

    k [B, T, HKV, D] (fp16/bf16/fp32) -> (k_q [B,T,HKV,ceil(D/4)] u8, scale [B,HKV,D], zero [B,HKV,D]
    in k.dtype, residual [B,T,HKV,D] fp8).
    """
    if not k.is_cuda:
        raise ValueError("k must be a CUDA tensor")
    k = k.contiguous()
    B, T, HKV, D = k.shape
    L = N.lib()
    nsplit = L.ffa_q2_quantize_nsplit(T)
    dev = k.device
    k_q = torch.empty((B, T, HKV, (D + 3) // 4), dtype=torch.uint8, device=dev)
    scale = torch.empty((B, HKV, D), dtype=k.dtype, device=dev)
    zero = torch.empty((B, HKV, D), dtype=k.dtype, device=dev)
    res = torch.empty((B, T, HKV, D), dtype=fp8_dtype, device=dev)
    minmax = torch.empty((2, B, nsplit, HKV * D), dtype=torch.float32, device=dev)
    rc = L.ffa_q2_quantize_channel(k.data_ptr(), N.dtype_code(k.dtype), B, T, HKV, D, k_q.data_ptr(),
                                   scale.data_ptr(), zero.data_ptr(), res.data_ptr(), N.dtype_code(fp8_dtype),
                                   minmax.data_ptr(), N.stream_of(dev))
    N.check(rc, "ffa_q2_quantize_channel")
    return k_q, scale, zero, res


def append_per_channel(k_q: torch.Tensor, k_scale: torch.Tensor, k_zero: torch.Tensor, k_residual: torch.Tensor,
                       k_new: torch.Tensor, pos, v: torch.Tensor | None = None, v_new: torch.Tensor | None = None):
    """Append new tokens to a reference-layout cache (k_q [B, T_cap, HKV, ceil(D/4)], residual
    [B, T_cap, HKV, D], per-channel scale / zero [B, HKV, D] as quantize_per_channel made them), in place.

    No reference counterpart (incremental quantization is a TODO there, ffa-q2fp8/OPTIMIZATION_NOTES.md:
    23-26).  Policy: the scale / zero stay as they are and the new tokens k_new [B, Tn, HKV, D] are
    quantized with them by the reference's per-element ops, so a value outside [zero, zero + 3 scale]
    takes code 0 or 3 and the fp8 residual carries the difference (e5m2 reaches 57344, e4m3 448).
    Token n of sequence b goes to position pos[b] + n (pos: int or [B] int tensor); v_new [B, Tn, HKV, DV]
    is copied into v at the same positions.  Positions must fit the cache (checked on the host).
    """
    for t, name in ((k_q, "k_q"), (k_scale, "k_scale"), (k_zero, "k_zero"), (k_residual, "k_residual"),
                    (k_new, "k_new")):
        if not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous CUDA tensor")
    B, T_cap, HKV, DP = k_q.shape
    Bn, Tn, HKVn, D = k_new.shape
    if Bn != B or HKVn != HKV or DP != (D + 3) // 4 or tuple(k_residual.shape) != (B, T_cap, HKV, D):
        raise ValueError("k_new [B, Tn, HKV, D] must match the cache [B, T_cap, HKV, ceil(D/4)] / [B, T_cap, HKV, D]")
    if tuple(k_scale.shape) != (B, HKV, D) or tuple(k_zero.shape) != (B, HKV, D):
        raise ValueError("k_scale / k_zero must be [B, HKV, D]")
    if k_scale.dtype != k_new.dtype or k_zero.dtype != k_new.dtype:
        raise ValueError("k_scale / k_zero must have k_new's dtype (the quantizer's arithmetic type)")
    dev = k_q.device
    pos_t = torch.full((B,), int(pos), dtype=torch.int32) if isinstance(pos, int) else pos.to(torch.int32).cpu()
    if pos_t.shape != (B,) or int(pos_t.min()) < 0 or int(pos_t.max()) + Tn > T_cap:
        raise ValueError(f"positions pos + {Tn} tokens must lie in [0, {T_cap}]")
    pos_d = pos_t.to(dev)
    rc = N.lib().ffa_q2_append_channel(k_new.data_ptr(), N.dtype_code(k_new.dtype), B, Tn, HKV, D, pos_d.data_ptr(),
                                       T_cap, k_scale.data_ptr(), k_zero.data_ptr(), k_q.data_ptr(),
                                       k_residual.data_ptr(), N.dtype_code(k_residual.dtype), N.stream_of(dev))
    N.check(rc, "ffa_q2_append_channel")
    if v_new is not None:
        if v is None or v.shape[0] != B or v.shape[2:] != v_new.shape[2:] or v_new.shape[1] != Tn:
            raise ValueError("v_new [B, Tn, HKV, DV] needs v [B, T_cap, HKV, DV]")
        for b in range(B):
            p0 = int(pos_t[b])
            v[b, p0:p0 + Tn].copy_(v_new[b])
    return k_q, k_residual


def kproj_rope_q2_channel(h, w_k, cos, sin, num_kv_heads, head_dim, bias=None, fp8_dtype=torch.float8_e5m2,
                          return_k=False):
    """K = RoPE(h W_k^T + b) then the per-channel q2 quantizer, on the GPU (one GEMM pass).

    h [B, T, H] fp16/bf16; cos/sin [T, D] (fp32 or h.dtype).  The rotated K has
    the promoted dtype of h and cos, as in the reference torch path
    (ffa-q2fp8/fused_kproj_rope_q2fp8.py:402-424).
    """
    if not h.is_cuda:
        raise ValueError("kernel requires CUDA tensors.")
    if head_dim % 2 != 0:
        raise ValueError(f"head_dim must be even for RoPE, got {head_dim}")
    w_k = _normalize_k_weight(w_k, h.shape[-1]).to(h.dtype).contiguous()
    B, T, H = h.shape
    HKV, D = int(num_kv_heads), int(head_dim)
    if w_k.shape[0] != HKV * D:
        raise ValueError(f"w_k out_dim mismatch: got {w_k.shape[0]}, expected {HKV * D}")
    if bias is not None and bias.numel() != HKV * D:
        raise ValueError(f"bias length mismatch: got {bias.numel()}, expected {HKV * D}")
    if cos.dtype not in (torch.float32, h.dtype):
        cos, sin = cos.float(), sin.float()
    odt = torch.float32 if cos.dtype == torch.float32 else h.dtype
    h, cos, sin = h.contiguous(), cos.contiguous(), sin.contiguous()
    bias = bias.to(h.dtype).contiguous() if bias is not None else None
    dev = h.device
    L = N.lib()
    nsplit = L.ffa_q2_quantize_nsplit(T)
    k_scr = torch.empty((B, T, HKV, D), dtype=odt, device=dev)
    k_q = torch.empty((B, T, HKV, (D + 3) // 4), dtype=torch.uint8, device=dev)
    scale = torch.empty((B, HKV, D), dtype=odt, device=dev)
    zero = torch.empty((B, HKV, D), dtype=odt, device=dev)
    res = torch.empty((B, T, HKV, D), dtype=fp8_dtype, device=dev)
    minmax = torch.empty((2, B, nsplit, HKV * D), dtype=torch.float32, device=dev)
    rc = L.ffa_kproj_rope_q2_channel(h.data_ptr(), w_k.data_ptr(), N.ptr(bias), N.dtype_code(h.dtype),
                                     cos.data_ptr(), sin.data_ptr(), N.dtype_code(cos.dtype), B, T, H, HKV, D,
                                     k_scr.data_ptr(), k_q.data_ptr(), scale.data_ptr(), zero.data_ptr(),
                                     res.data_ptr(), N.dtype_code(fp8_dtype), minmax.data_ptr(), N.stream_of(dev))
    N.check(rc, "ffa_kproj_rope_q2_channel")
    out = (k_q, scale, zero, res)
    return (out, k_scr) if return_k else out


def kproj_rope_q2_append(cache: PagedQ2Cache, h, w_k, cos_rows, sin_rows, pos, block_table, bias=None, v_new=None,
                         validate=True):
    """Project, rotate, g32-quantize and append Tn new tokens per sequence into a paged cache.

    h [B, Tn, H]; cos_rows/sin_rows [B, Tn, 128] fp32 (angles of positions pos[b] + n);
    v_new [B, Tn, HKV, 128] or None.  validate=False skips the host-side check that the positions and
    page ids stay inside the table and the pool (it reads them back, which graph capture forbids): the
    caller must have checked the same pos / block_table before.
    """
    if not h.is_cuda:
        raise ValueError("kernel requires CUDA tensors.")
    B, Tn, H = h.shape
    HKV = cache.HKV
    w_k = _normalize_k_weight(w_k, H).to(h.dtype).contiguous()
    if w_k.shape[0] != HKV * 128:
        raise ValueError("w_k out_dim must be HKV * 128")
    cos_rows = cos_rows.float().reshape(B, Tn, 128).contiguous()
    sin_rows = sin_rows.float().reshape(B, Tn, 128).contiguous()
    pos = pos.to(device=h.device, dtype=torch.int32).contiguous()
    block_table = block_table.to(device=h.device, dtype=torch.int32).contiguous()
    if validate:
        check_append_fits(pos, Tn, block_table, cache.P)
    if v_new is not None:
        v_new = v_new.to(cache.v_dtype).contiguous()
    bias = bias.to(h.dtype).contiguous() if bias is not None else None
    h = h.contiguous()
    rc = N.lib().ffa_kproj_rope_q2_append(
        h.data_ptr(), w_k.data_ptr(), N.ptr(bias), N.dtype_code(h.dtype), cos_rows.data_ptr(), sin_rows.data_ptr(),
        B, Tn, H, HKV, pos.data_ptr(), block_table.data_ptr(), block_table.shape[1], cache.P, cache.k_q.data_ptr(),
        cache.k_scale.data_ptr(), cache.k_zero.data_ptr(), cache.k_res.data_ptr(), N.dtype_code(cache.res_dtype),
        N.ptr(v_new), cache.v.data_ptr(), N.dtype_code(cache.v_dtype), N.stream_of(h.device))
    N.check(rc, "ffa_kproj_rope_q2_append")
