"""CPU restatement of the q2fp8 pruned decode path (numpy).

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker.  The
product path (ffa-speedtest_amd/) never calls it.

What each function restates (reference paths are relative to the reference
checkout):

* quantize_per_channel   ffa-q2fp8/run_attn_bench_q2.py:78-105
                         (== ffa-q2fp8/fused_kproj_rope_q2fp8.py:40-68)
* quantize_g32           paged-cache layout (2-bit, groups of 32 along D, fp16
                         scale/zero per token).  The reference has no such
                         quantizer; the rules mirror the per-channel one.
* decode                 ffa-q2fp8/attn_kernel/attn_kernel_v1210_fused_bsz_q2fp8.py
                         stage1 :10-139, stage2 :142-171, wrapper :191-309.
                         per_channel mode rounds dequantized and refined K to fp16
                         as the reference's tl.dot inputs do (:93, :109-115); g32 mode
                         (no reference counterpart) keeps them exact.
  decode(v_mean=...)     the mean-V variant, ffa-q2fp8-meanv/attn_kernel/
                         attn_kernel_v1210_meanv_bsz_q2fp8.py stage1 :109-152, stage2 :156-202
* value_mean             the same file :332 (v.mean(dim=1, dtype=float32).to(v.dtype))
* threshold_external     ffa-fp8/attn_kernel/attn_kernel_v1208_fused_bsz_fp8.py:174-234
* decode_bruteforce      same semantics as `decode`, written as scalar loops
                         for tiny shapes (an independent second statement).

Values of a torch dtype `tau` are carried as float32 arrays whose elements
are exactly representable in tau; every torch op that the reference runs in
tau is followed here by an explicit rounding to tau (`round_to`).
"""
from __future__ import annotations

import math

import numpy as np

from .numerics import F32, fp8_decode, fp8_encode, round_f16, round_to

L2E = np.float32(1.4426950408889634)  # RCP_LN2, attn_kernel_v1210_fused_bsz_q2fp8.py:30
T_BS = 16  # probe window length, attn_kernel_v1210_fused_bsz_q2fp8.py:20


# ----------------------------------------------------------------------------
# 2-bit packing
# ----------------------------------------------------------------------------


def pack_2bit(codes: np.ndarray) -> np.ndarray:
    """[..., D] codes in 0..3 -> [..., ceil(D/4)] bytes, c0 | c1<<2 | c2<<4 | c3<<6.

    run_attn_bench_q2.py:91-104 (zero codes pad D up to a multiple of 4).
    """
    codes = np.asarray(codes, dtype=np.uint8)
    D = codes.shape[-1]
    Dp = (D + 3) // 4
    pad = Dp * 4 - D
    if pad:
        codes = np.concatenate([codes, np.zeros(codes.shape[:-1] + (pad,), np.uint8)], axis=-1)
    c = codes.reshape(codes.shape[:-1] + (Dp, 4))
    return (c[..., 0] | (c[..., 1] << 2) | (c[..., 2] << 4) | (c[..., 3] << 6)).astype(np.uint8)


def unpack_2bit(packed: np.ndarray, D: int) -> np.ndarray:
    """Inverse of pack_2bit: code d is (byte[d//4] >> 2*(d%4)) & 3 (attn_kernel...q2fp8.py:43-44, 91-92)."""
    packed = np.asarray(packed, dtype=np.uint8)
    sh = np.array([0, 2, 4, 6], dtype=np.uint8)
    c = (packed[..., :, None] >> sh) & 3
    return c.reshape(packed.shape[:-1] + (-1,))[..., :D]


# ----------------------------------------------------------------------------
# Quantizers
# ----------------------------------------------------------------------------


def quantize_per_channel(k: np.ndarray, tau: str, fp8: str = "e5m2"):
    """Reference quantizer, run_attn_bench_q2.py:78-105.

    k: [B, T, HKV, D] float32 holding tau values.  Returns
    (k_q_packed u8 [B,T,HKV,ceil(D/4)], scale [B,HKV,D], zero [B,HKV,D]
    (tau values as float32), k_residual fp8 bytes [B,T,HKV,D]).
    """
    k = np.asarray(k, dtype=F32)
    k_min = k.min(axis=1)  # :80 amin over T (exact)
    k_max = k.max(axis=1)  # :81
    diff = round_to(k_max - k_min, tau)  # :82 (k_max - k_min) in tau
    clamped = round_to(np.maximum(diff, F32(1e-6)), tau)  # .clamp_min(1e-6)
    scale = round_to(clamped / F32(3.0), tau)  # / 3.0 in tau
    zero = k_min  # :83
    packed, res = quantize_with_channel_scale(k, scale, zero, tau, fp8)
    return packed, scale.astype(F32), zero.astype(F32), res


def quantize_with_channel_scale(k: np.ndarray, scale: np.ndarray, zero: np.ndarray, tau: str, fp8: str = "e5m2"):
    """Codes and residual of K [B, T, HKV, D] under given per-channel scale / zero [B, HKV, D] (tau
    values), with the reference quantizer's per-element ops (run_attn_bench_q2.py:84-88):
    c = clamp(rne(tau(tau(k - zero) / scale)), 0, 3); res = fp8(f32(k) - (f32(c * scale) + zero)).
    quantize_per_channel runs it with the scale / zero of K itself; the per-channel append runs it
    on new tokens with the cache's existing scale / zero, so a value outside [zero, zero + 3 scale]
    takes code 0 or 3 and the residual carries the rest (no reference counterpart: incremental
    quantization is a TODO there, ffa-q2fp8/OPTIMIZATION_NOTES.md:23-26).  Returns
    (packed u8 [B, T, HKV, ceil(D/4)], residual fp8 bytes [B, T, HKV, D])."""
    k = np.asarray(k, dtype=F32)
    scale = np.asarray(scale, F32)
    zero = np.asarray(zero, F32)
    xs = round_to(k - zero[:, None], tau)  # (k - zero) in tau
    xd = round_to(xs / scale[:, None], tau)  # / scale in tau
    codes = np.clip(np.rint(xd), 0, 3).astype(np.uint8)  # torch.round = RNE; clamp(0,3)
    deq = (codes.astype(F32) * scale[:, None]).astype(F32) + zero[:, None]  # :85-87, no FMA
    res = fp8_encode((k - deq).astype(F32), fp8)  # :88
    return pack_2bit(codes), res


def append_per_channel(k_q: np.ndarray, k_res: np.ndarray, k_new: np.ndarray, scale: np.ndarray, zero: np.ndarray,
                       pos, tau: str, fp8: str = "e5m2"):
    """Reference-layout cache append: tokens k_new [B, Tn, HKV, D] go to positions pos[b] .. pos[b] + Tn - 1
    of k_q [B, T_cap, HKV, ceil(D/4)] / k_res [B, T_cap, HKV, D] (copies are returned), quantized by
    quantize_with_channel_scale with the cache's scale / zero; positions past T_cap are dropped."""
    k_q = np.array(k_q, copy=True)
    k_res = np.array(k_res, copy=True)
    pk, rr = quantize_with_channel_scale(k_new, scale, zero, tau, fp8)
    T_cap = k_q.shape[1]
    for b in range(k_new.shape[0]):
        for n in range(k_new.shape[1]):
            t = int(pos[b]) + n
            if 0 <= t < T_cap:
                k_q[b, t] = pk[b, n]
                k_res[b, t] = rr[b, n]
    return k_q, k_res


def quantize_g32(k: np.ndarray, fp8: str = "e4m3fn", group: int = 32):
    """Paged-cache q2 layout: groups of `group` along D, fp16 scale/zero per token.

    k: [..., D] float32 (any tau).  Per group g of one token:
      zero  = fp16(min_g k)
      scale = fp16(max(fp32(max_g k) - fp32(zero), 1e-6) / 3)
      c     = clamp(rne((fp32(k) - fp32(zero)) / fp32(scale)), 0, 3)
      deq   = fp32(fp32(c) * fp32(scale)) + fp32(zero)      (two roundings)
      res   = fp8(fp32(k) - deq)
    Returns (packed u8 [..., D/4], scale f32 [..., D/group], zero f32 [..., D/group], res u8 [..., D]).
    """
    k = np.asarray(k, dtype=F32)
    D = k.shape[-1]
    if D % group:
        raise ValueError("D must be a multiple of the group size")
    kg = k.reshape(k.shape[:-1] + (D // group, group))
    zero = round_f16(kg.min(axis=-1))
    scale = round_f16(np.maximum(kg.max(axis=-1) - zero, F32(1e-6)).astype(F32) / F32(3.0))
    x = ((kg - zero[..., None]).astype(F32) / scale[..., None]).astype(F32)
    codes = np.clip(np.rint(x), 0, 3).astype(np.uint8)
    deq = (codes.astype(F32) * scale[..., None]).astype(F32) + zero[..., None]
    res = fp8_encode((kg - deq).astype(F32), fp8).reshape(k.shape)
    codes = codes.reshape(k.shape)
    return pack_2bit(codes), scale.astype(F32), zero.astype(F32), res


def dequant(codes_packed, scale, zero, D: int, mode: str):
    """Dequantized 2-bit K.

    per_channel (reference, attn_kernel...q2fp8.py:93): k_hat = fp16(fp32(fp32(c) * s) + z),
        scale/zero [B, HKV, D] broadcast over T.
    g32 (this build's paged format): k_hat = c * s + z evaluated exactly (float64), no
        fp16 rounding; scale/zero [B, T, HKV, D/32] fp16 values, one per token and group.
    """
    c = unpack_2bit(codes_packed, D).astype(F32)
    if mode == "per_channel":
        s = np.asarray(scale, F32)[:, None]
        z = np.asarray(zero, F32)[:, None]
        return round_f16((c * s).astype(F32) + z)
    if mode == "g32":
        g = D // np.asarray(scale).shape[-1]
        s = np.repeat(np.asarray(scale, np.float64), g, axis=-1)
        z = np.repeat(np.asarray(zero, np.float64), g, axis=-1)
        return c.astype(np.float64) * s + z
    raise ValueError(mode)


# ----------------------------------------------------------------------------
# Paged layout (this build's format; the reference is contiguous only)
# ----------------------------------------------------------------------------


def gather_pages(pages: np.ndarray, block_table: np.ndarray, T: int, page: int = 64, v_transposed=False):
    """Paged pool -> contiguous [T, HKV, X] for one sequence.

    pages: [P, HKV, page, X]  (codes / residual / g32 scales-by-token)
       or  [P, HKV, X, page]  when v_transposed (V^T pages).
    Token t lives in page block_table[t // page], slot t % page.
    """
    npg = (T + page - 1) // page
    sel = pages[np.asarray(block_table[:npg], dtype=np.int64)]
    if v_transposed:
        sel = np.swapaxes(sel, -1, -2)
    # [npg, HKV, page, X] -> [npg*page, HKV, X]
    out = np.swapaxes(sel, 1, 2).reshape(npg * page, sel.shape[1], sel.shape[-1])
    return out[:T]


# ----------------------------------------------------------------------------
# Decode
# ----------------------------------------------------------------------------


def _subblock_tokens(T: int, BS: int, SBS: int):
    """Token index matrix [NTBS, SBS] and validity (attn_kernel...q2fp8.py:84-86, 104, 254-256)."""
    NTB = -(-T // BS)
    NSB = -(-BS // SBS)
    j = np.arange(NTB * NSB)
    start = (j // NSB) * BS + (j % NSB) * SBS
    idx = start[:, None] + np.arange(SBS)[None, :]
    valid = idx < T
    return NTB, NSB, np.where(valid, idx, 0), valid


def _score(qrows16: np.ndarray, k16: np.ndarray, scale: np.float32) -> np.ndarray:
    """f32(f32(dot(q16, k16)) * scale) * L2E ; dot accumulated exactly (float64)."""
    dot = (k16.astype(np.float64) @ qrows16.astype(np.float64).T).astype(F32)  # [T, G]
    return ((dot * scale).astype(F32) * L2E).astype(F32)


def _probe_windows(T: int, NTB: int):
    w0 = np.arange(0, min(T_BS, T))
    lo = (NTB - 1) * T_BS  # attn_kernel...q2fp8.py:70-73 ("last block" quirk)
    w1 = np.arange(lo, lo + T_BS)
    w1 = w1[w1 < T]
    return w0, w1


def decode(
    q,
    k_q,
    k_scale,
    k_zero,
    v,
    k_residual=None,
    *,
    res_fmt: str = "e5m2",
    scale=None,
    BS: int = 128,
    SBS=None,
    delta: float = 5.0,
    precomputed_threshold=None,
    use_fp8_residual: bool = True,
    scale_mode: str = "per_channel",
    seq_lens=None,
    out_dtype: str = "fp16",
    force_mask=None,
    khat=None,
    khat_probe1=None,
    pv_dtype: str = "fp16",
    v_mean=None,
):
    """Appendix-A decode semantics over the contiguous layout.

    khat [B,T,HKV,D] (optional) replaces the 2-bit dequantization with another format's
    fp16 K (the other formats share the decode, oracle/formats.py); khat_probe1 (optional)
    is the K used for the second probe window (nvfp4 takes the last block's scale there).
    With khat, the refined K is fp16(khat + fp16(res)) as in per_channel mode.

    q [B,HQ,D]; k_q [B,T,HKV,ceil(D/4)] u8; k_scale/k_zero per_channel
    [B,HKV,D] or g32 [B,T,HKV,D/32]; v [B,T,HKV,DV]; k_residual [B,T,HKV,D]
    fp8 bytes.  seq_lens (optional) gives each sequence its own length.
    force_mask [B,HKV,NTBS] (optional) replaces the prune decision, so that an
    implementation's arithmetic can be checked under its own block mask.
    pv_dtype: the type p and v are rounded to for P.V, "fp16" as the reference casts
    both (attn_kernel...q2fp8.py:130-131); "bf16" exists only for tests that show a
    bf16 P operand is caught.
    v_mean [B,HKV,DV] (optional): the mean-V variant (..._meanv_bsz_q2fp8.py): a pruned
    block holding tokens keeps m = max of its coarse scores and l = sum 2^(s - m) (:109-119);
    stage 2 merges kept and approximated blocks apart and folds l with v_mean (:172-202).
    diag then has 'approx' [B,HKV,NTBS] and 'approx_ratio' = approx.sum()/approx.size (:326-330).

    Returns (o [B,HQ,DV] float32 holding out_dtype values, diag dict with
    'mask' [B,HKV,NTBS] int8, 'threshold' [B,HQ], 'block_max' [B,HQ,NTBS]
    (coarse), 'margin' [B,HKV,NTBS] = max_g(block_max - th), 'skip_ratio',
    'm','l' per kept block [B,HQ,NTBS] and 'ntbs' per sequence).
    """
    q = np.asarray(q, F32)
    B, HQ, D = q.shape
    _, T, HKV, _ = k_q.shape
    DV = v.shape[-1]
    G = HQ // HKV
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    scale = F32(scale)
    if SBS is None:
        SBS = BS
    use_res = bool(use_fp8_residual and k_residual is not None)
    lens = [T] * B if seq_lens is None else [int(x) for x in seq_lens]
    NSB = -(-BS // SBS)
    NTBS_max = max(-(-t // BS) for t in lens) * NSB

    o = np.zeros((B, HQ, DV), F32)
    mask = np.zeros((B, HKV, NTBS_max), np.int8)
    thr = np.zeros((B, HQ), F32)
    bmax = np.full((B, HQ, NTBS_max), -np.inf, F32)
    margin = np.full((B, HKV, NTBS_max), -np.inf, F32)
    m_out = np.full((B, HQ, NTBS_max), -np.inf, F32)
    l_out = np.zeros((B, HQ, NTBS_max), F32)
    approx = np.zeros((B, HKV, NTBS_max), np.int8)
    ntbs = []
    kept_total = 0
    blocks_total = 0

    for b in range(B):
        Tb = lens[b]
        if Tb == 0:
            # an empty sequence (ragged batches only): no blocks, both probe windows empty so the
            # threshold is -inf, and the merge of no partials gives 0 (attn_kernel...q2fp8.py:167-171)
            ntbs.append(0)
            thr[b] = -np.inf
            continue
        NTB, NSB_, idx, valid = _subblock_tokens(Tb, BS, SBS)
        NTBS = idx.shape[0]
        ntbs.append(NTBS)
        blocks_total += HKV * NTBS
        w0, w1 = _probe_windows(Tb, NTB)
        for h in range(HKV):
            if khat is not None:
                kh = np.asarray(khat[b, :Tb, h], F32)
            elif scale_mode == "per_channel":
                kh = dequant(k_q[b:b + 1, :Tb, h:h + 1], k_scale[b:b + 1, h:h + 1], k_zero[b:b + 1, h:h + 1], D,
                             "per_channel")[0, :, 0]
            else:
                kh = dequant(k_q[b, :Tb, h], k_scale[b, :Tb, h], k_zero[b, :Tb, h], D, "g32")
            q16 = round_f16(q[b, h * G:(h + 1) * G])  # [G, D]  (:47)
            Sq = _score(q16, kh, scale)  # [Tb, G] (:94)
            if precomputed_threshold is not None:
                th = np.asarray(precomputed_threshold, F32)[b, h * G:(h + 1) * G]
            else:
                Sp1 = Sq if khat_probe1 is None else _score(q16, np.asarray(khat_probe1[b, :Tb, h], F32), scale)
                m0 = Sq[w0].max(axis=0) if len(w0) else np.full(G, -np.inf, F32)
                m1 = Sp1[w1].max(axis=0) if len(w1) else np.full(G, -np.inf, F32)
                th = (np.maximum(m0, m1) - F32(delta)).astype(F32)  # :82
            thr[b, h * G:(h + 1) * G] = th
            Sb = np.where(valid[:, :, None], Sq[idx], -np.inf)  # [NTBS, SBS, G]
            mb = Sb.max(axis=1)  # [NTBS, G] (:97)
            bmax[b, h * G:(h + 1) * G, :NTBS] = mb.T
            # diagnostic only: NaN where an empty block (-inf) meets an infinite threshold (delta = +inf
            # makes th = -inf); the keep rule below does not use it
            with np.errstate(invalid="ignore"):
                margin[b, h, :NTBS] = (mb - th[None, :]).max(axis=1)
            keep = ~np.all(mb < th[None, :], axis=1)  # prune iff all rows below (:99-102)
            if force_mask is not None:
                keep = np.asarray(force_mask)[b, h, :NTBS].astype(bool)
            mask[b, h, :NTBS] = keep
            kept = np.nonzero(keep)[0]
            kept_total += len(kept)
            # mean-V: pruned blocks holding tokens, their coarse max and mass (meanv :109-119)
            Mp = np.full(G, -np.inf)
            Ap = np.zeros(G)
            if v_mean is not None:
                apx = np.nonzero(~keep & valid.any(axis=1))[0]
                approx[b, h, apx] = 1
                if len(apx):
                    Sa = np.where(valid[apx][:, :, None], Sq[idx[apx]], -np.inf).astype(np.float64)  # [A, SBS, G]
                    ma = Sa.max(axis=1)  # [A, G]
                    la = np.where(valid[apx][:, :, None], np.exp2(Sa - ma[:, None, :]), 0.0).astype(F32).astype(
                        np.float64).sum(axis=1)  # [A, G]
                    Mp = ma.max(axis=0)
                    Ap = (la * np.exp2(ma - Mp[None, :])).sum(axis=0)
            if len(kept) == 0:
                if v_mean is not None:
                    vm = np.asarray(v_mean, np.float64)[b, h]  # [DV]
                    with np.errstate(invalid="ignore", divide="ignore"):
                        out = np.where(Ap[:, None] > 0, (vm[None, :] * Ap[:, None]) / Ap[:, None], 0.0)
                    o[b, h * G:(h + 1) * G] = round_to(out.astype(F32), out_dtype)
                continue
            if use_res:
                r16 = fp8_decode(k_residual[b, :Tb, h], res_fmt)  # exact in fp16
                if khat is not None or scale_mode == "per_channel":
                    ktil = round_f16(kh + r16)  # (:109-115)
                else:
                    ktil = kh + r16.astype(np.float64)  # g32: exact
                S = _score(q16, ktil, scale)
            else:
                S = Sq
            Sk = np.where(valid[kept][:, :, None], S[idx[kept]], -np.inf)  # [K, SBS, G]
            m = Sk.max(axis=1)  # [K, G]
            with np.errstate(invalid="ignore"):
                p = np.where(valid[kept][:, :, None], np.exp2((Sk - m[:, None, :]).astype(np.float64)), 0.0)
            p = p.astype(F32)
            lsum = p.astype(np.float64).sum(axis=1).astype(F32)  # [K, G] (:124)
            v16 = round_to(np.asarray(v[b, :Tb, h][idx[kept]], F32), pv_dtype)  # [K, SBS, DV]
            v16 = np.where(valid[kept][:, :, None], v16, 0.0)
            ob = np.einsum("kug,kuv->kgv", round_to(p, pv_dtype).astype(np.float64), v16.astype(np.float64))  # (:131)
            m_out[b, h * G:(h + 1) * G][:, kept] = m.T
            l_out[b, h * G:(h + 1) * G][:, kept] = lsum.T
            # stage 2 merge (:156-169), evaluated exactly
            mf = np.where(np.isfinite(m), m, -np.inf).astype(np.float64)
            M = mf.max(axis=0)  # [G]
            with np.errstate(invalid="ignore"):
                w = np.where(np.isfinite(mf), np.exp2(mf - M[None, :]), 0.0)  # [K, G]
            A = (lsum.astype(np.float64) * w).sum(axis=0)
            O = (ob * w[:, :, None]).sum(axis=0)  # [G, DV]
            if v_mean is not None:  # meanv stage 2 fold (:192-202)
                vm = np.asarray(v_mean, np.float64)[b, h]
                Mx = np.maximum(np.where(A > 0, M, -np.inf), np.where(Ap > 0, Mp, -np.inf))
                with np.errstate(invalid="ignore"):
                    rb = np.where(A > 0, np.exp2(M - Mx), 0.0)
                    rp = np.where(Ap > 0, np.exp2(Mp - Mx), 0.0)
                O = O * rb[:, None] + vm[None, :] * (Ap * rp)[:, None]
                A = A * rb + Ap * rp
            with np.errstate(invalid="ignore", divide="ignore"):
                out = np.where(A[:, None] == 0.0, 0.0, O / A[:, None])
            o[b, h * G:(h + 1) * G] = round_to(out.astype(F32), out_dtype)

    diag = dict(
        mask=mask,
        threshold=thr,
        block_max=bmax,
        margin=margin,
        m=m_out,
        l=l_out,
        ntbs=ntbs,
        skip_ratio=1.0 - kept_total / max(blocks_total, 1),
    )
    if v_mean is not None:
        diag["approx"] = approx
        diag["approx_ratio"] = float(approx.sum()) / max(blocks_total, 1)
    return o, diag


def value_mean(v, seq_lens=None, out_dtype: str = "bf16"):
    """Mean over tokens of v [B,T,HKV,DV] per (b, head), rounded once to out_dtype
    (..._meanv_bsz_q2fp8.py:332; the sum is exact here, fp32 in the reference).  With seq_lens each
    sequence averages its own tokens, and an empty one gives 0."""
    v = np.asarray(v, np.float64)
    B, T = v.shape[:2]
    lens = [T] * B if seq_lens is None else [min(max(int(x), 0), T) for x in seq_lens]
    out = np.zeros((B,) + v.shape[2:], np.float64)
    for b, L in enumerate(lens):
        if L > 0:
            out[b] = v[b, :L].sum(axis=0) / L
    return round_to(out.astype(F32), out_dtype)


def threshold_external(q, k_fp16, scale, NTB, delta, HKV, HQ, T_BS_: int = T_BS):
    """Host threshold of ffa-fp8/attn_kernel/attn_kernel_v1208_fused_bsz_fp8.py:174-234.

    th = max(max_{t in tb0} q.k, max_{t in tb_last} q.k) * (scale*RCP_LN2) - delta,
    tb0 = [0, T_BS), tb_last = [(NTB-1)*T_BS, (NTB-1)*T_BS + T_BS) clipped to [0, T).
    Computed in fp32 (the product in fp32, as at :222-229).
    """
    q = np.asarray(q, F32)
    k = np.asarray(k_fp16, F32)
    B, _, D = q.shape
    T = k.shape[1]
    G = HQ // HKV
    c = F32(float(scale) * 1.4426950408889634)
    t0 = np.arange(0, min(T_BS_, T))
    lo = max(0, (NTB - 1) * T_BS_)
    t1 = np.arange(lo, min(lo + T_BS_, T))
    th = np.empty((B, HQ), F32)
    for b in range(B):
        for h in range(HKV):
            qr = q[b, h * G:(h + 1) * G].astype(np.float64)
            def mx(ts):
                if len(ts) == 0:
                    return np.full(G, -np.inf)
                s = (qr @ k[b, ts, h].astype(np.float64).T).astype(F32) * c
                return s.max(axis=1)
            th[b, h * G:(h + 1) * G] = (np.maximum(mx(t0), mx(t1)) - F32(delta)).astype(F32)
    return th


def decode_bruteforce(q, k_q, k_scale, k_zero, v, k_residual=None, *, res_fmt="e5m2", scale=None, BS=128,
                      SBS=None, delta=5.0, use_fp8_residual=True, scale_mode="per_channel", out_dtype="fp16"):
    """Scalar-loop statement of the same semantics, for tiny shapes only.

    Written token by token from attn_kernel_v1210_fused_bsz_q2fp8.py:10-171 without
    reshapes or vectorised gathers, to cross-check `decode`.
    """
    B, HQ, D = q.shape
    _, T, HKV, _ = k_q.shape
    DV = v.shape[-1]
    G = HQ // HKV
    sc = F32(1.0 / math.sqrt(D) if scale is None else scale)
    SBS = BS if SBS is None else SBS
    NTB = -(-T // BS)
    NSB = -(-BS // SBS)
    use_res = use_fp8_residual and k_residual is not None
    out = np.zeros((B, HQ, DV), F32)
    f16 = lambda x: float(np.float16(np.float32(x)))

    def khat(b, t, h, d):
        byte = int(k_q[b, t, h, d // 4])
        c = (byte >> (2 * (d % 4))) & 3
        if scale_mode == "per_channel":
            s, z = k_scale[b, h, d], k_zero[b, h, d]
            return f16(np.float32(np.float32(np.float32(c) * np.float32(s)) + np.float32(z)))
        s, z = k_scale[b, t, h, d // 32], k_zero[b, t, h, d // 32]
        return float(c) * float(s) + float(z)

    def score(b, h, g, t, refined):
        acc = 0.0
        for d in range(D):
            kv = khat(b, t, h, d)
            if refined:
                r = float(fp8_decode(k_residual[b, t, h, d], res_fmt))
                kv = f16(np.float32(kv) + r) if scale_mode == "per_channel" else kv + r
            acc += f16(q[b, h * G + g, d]) * kv
        return float(np.float32(np.float32(np.float32(acc) * sc) * L2E))

    for b in range(B):
        for h in range(HKV):
            th = []
            for g in range(G):
                cand = [score(b, h, g, t, False) for t in range(0, min(16, T))]
                lo = (NTB - 1) * 16
                cand += [score(b, h, g, t, False) for t in range(lo, min(lo + 16, T))]
                th.append(float(np.float32(max(cand) - np.float32(delta))))
            parts = []
            for tb in range(NTB):
                for sb in range(NSB):
                    toks = [t for t in range(tb * BS + sb * SBS, tb * BS + sb * SBS + SBS) if t < T]
                    below = 0
                    for g in range(G):
                        mb = max([score(b, h, g, t, False) for t in toks], default=-math.inf)
                        below += mb < th[g]
                    if below == G:
                        continue
                    for g in range(G):
                        S = [score(b, h, g, t, use_res) for t in toks]
                        m = max(S, default=-math.inf)
                        p = [2.0 ** (s - m) for s in S]
                        l = sum(p)
                        o = [sum(f16(pp) * f16(v[b, t, h, dv]) for pp, t in zip(p, toks)) for dv in range(DV)]
                        parts.append((g, m, l, o))
            for g in range(G):
                pg = [(m, l, o) for (gg, m, l, o) in parts if gg == g]
                if not pg:
                    continue
                M = max(m for m, _, _ in pg)
                A = sum(l * 2.0 ** (m - M) for m, l, _ in pg)
                if A == 0:
                    continue
                for dv in range(DV):
                    out[b, h * G + g, dv] = sum(o[dv] * 2.0 ** (m - M) for m, _, o in pg) / A
    return round_to(out, out_dtype)
