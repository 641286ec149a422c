"""Shared builders for the parity tests: seeded inputs, oracle quantization, page pools."""
from __future__ import annotations

import numpy as np
import torch

from ffa_mi355x import synth
from ffa_mi355x.paged import scale_pos
from oracle import q2fp8 as O

TORCH_DT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}
FP8_DT = {"e4m3fn": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}

# Decode tolerances: output within max-abs 2e-2 and mean-abs 2e-3;
# survivor mask identical except blocks within 1e-3 (log2 units) of the threshold.
OUT_MAX_ABS = 2e-2
OUT_MEAN_ABS = 2e-3
NEAR_TH = 1e-3


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def contig_case(B=1, T=1024, HQ=32, HKV=8, tau="bf16", res="e5m2", seed=0, n_heavy=0, seq_lens=None):
    """Reference layout: per-channel q2 + fp8 residual (run_attn_bench_q2.py:78-105)."""
    q, k, v = synth.attention_inputs(B=B, T=T, HQ=HQ, HKV=HKV, seed=seed, n_heavy=n_heavy, dtype=TORCH_DT[tau],
                                     seq_lens=seq_lens)
    pk, s, z, r = O.quantize_per_channel(f32(k), tau, res)
    return dict(q=q, k=k, v=v, k_q=pk, k_scale=s, k_zero=z, k_res=r, tau=tau, res=res)


def to_gpu_contig(case, dev):
    tau = TORCH_DT[case["tau"]]
    return dict(
        q=case["q"].to(dev).unsqueeze(1).contiguous(),
        k_q=torch.from_numpy(case["k_q"]).to(dev),
        k_scale=torch.from_numpy(case["k_scale"]).to(tau).to(dev),
        k_zero=torch.from_numpy(case["k_zero"]).to(tau).to(dev),
        k_residual=torch.from_numpy(case["k_res"]).view(FP8_DT[case["res"]]).to(dev),
        v=case["v"].to(dev),
    )


def paged_case(B=1, T=2048, HQ=32, HKV=8, seed=0, n_heavy=16, res="e4m3fn", seq_lens=None, garbage=True,
               interleave=True):
    """Benchmark layout: g32 q2 + fp8 residual in 64-token pages with a random page table."""
    q, k, v = synth.attention_inputs(B=B, T=T, HQ=HQ, HKV=HKV, seed=seed, n_heavy=n_heavy, seq_lens=seq_lens)
    lens = [T] * B if seq_lens is None else [int(x) for x in seq_lens]
    pk, s, z, r = O.quantize_g32(f32(k), res)  # [B,T,HKV,32], [B,T,HKV,4] x2, [B,T,HKV,128]
    bt, P = synth.page_tables(lens, seed=seed, interleave=interleave)
    rng = np.random.default_rng(seed + 7)
    if garbage:
        kq_pool = rng.integers(0, 256, (P, HKV, 4, 64, 8), dtype=np.uint8)
        s_pool = rng.integers(0, 65536, (P, HKV, 4, 64), dtype=np.uint16)  # includes NaN/inf patterns
        z_pool = rng.integers(0, 65536, (P, HKV, 4, 64), dtype=np.uint16)
        r_pool = rng.integers(0, 256, (P, HKV, 64, 128), dtype=np.uint8)
        v_pool = rng.integers(0, 65536, (P, HKV, 128, 64), dtype=np.uint16)
    else:
        kq_pool = np.zeros((P, HKV, 4, 64, 8), np.uint8)
        s_pool = np.zeros((P, HKV, 4, 64), np.uint16)
        z_pool = np.zeros((P, HKV, 4, 64), np.uint16)
        r_pool = np.zeros((P, HKV, 64, 128), np.uint8)
        v_pool = np.zeros((P, HKV, 128, 64), np.uint16)
    vb = v.view(torch.int16).numpy().view(np.uint16)  # bf16 bits [B,T,HKV,128]
    spos = np.array([scale_pos(t) for t in range(64)])
    s16 = s.astype(np.float16).view(np.uint16)
    z16 = z.astype(np.float16).view(np.uint16)
    for b in range(B):
        for t0 in range(0, lens[b], 64):
            page = int(bt[b, t0 // 64])
            t1 = min(t0 + 64, lens[b])
            n = t1 - t0
            kq_pool[page, :, :, :n, :] = pk[b, t0:t1].reshape(n, HKV, 4, 8).transpose(1, 2, 0, 3)
            s_pool[page][:, :, spos[:n]] = s16[b, t0:t1].transpose(1, 2, 0)
            z_pool[page][:, :, spos[:n]] = z16[b, t0:t1].transpose(1, 2, 0)
            r_pool[page, :, :n, :] = r[b, t0:t1].transpose(1, 0, 2)
            v_pool[page, :, :, :n] = vb[b, t0:t1].transpose(1, 2, 0)
    # the pools keep each (page, head) block in the decode's load order
    from ffa_mi355x.paged import CODES_ORDER, GSCALE_ORDER, RES_ORDER, VT_ORDER, to_tiled

    pools = dict(k_q=to_tiled(kq_pool, CODES_ORDER, 8), k_scale=to_tiled(s_pool, GSCALE_ORDER),
                 k_zero=to_tiled(z_pool, GSCALE_ORDER), k_res=to_tiled(r_pool, RES_ORDER), v=to_tiled(v_pool, VT_ORDER))
    return dict(q=q, k=k, v=v, k_q=pk, k_scale=s, k_zero=z, k_res=r, res=res, lens=lens, block_table=bt,
                pools=pools, P=P)


def paged_channel_case(B=1, T=2048, HQ=32, HKV=8, tau="bf16", res="e5m2", seed=0, n_heavy=16, seq_lens=None):
    """Per-channel q2 (the reference quantizer, scale / zero [B, HKV, 128]) with its codes, residual and
    V in the paged pools: codes pack as in the reference layout, so they scatter like the g32 codes."""
    q, k, v = synth.attention_inputs(B=B, T=T, HQ=HQ, HKV=HKV, seed=seed, n_heavy=n_heavy, dtype=TORCH_DT[tau],
                                     seq_lens=seq_lens)
    lens = [T] * B if seq_lens is None else [int(x) for x in seq_lens]
    pk, s, z, r = O.quantize_per_channel(f32(k), tau, res)
    bt, P = synth.page_tables(lens, seed=seed, interleave=True)
    rng = np.random.default_rng(seed + 7)
    kq_pool = rng.integers(0, 256, (P, HKV, 4, 64, 8), dtype=np.uint8)
    r_pool = rng.integers(0, 256, (P, HKV, 64, 128), dtype=np.uint8)
    v_pool = rng.integers(0, 65536, (P, HKV, 128, 64), dtype=np.uint16)
    vb = v.view(torch.int16).numpy().view(np.uint16)
    for b in range(B):
        for t0 in range(0, lens[b], 64):
            page = int(bt[b, t0 // 64])
            n = min(t0 + 64, lens[b]) - t0
            kq_pool[page, :, :, :n, :] = pk[b, t0:t0 + n].reshape(n, HKV, 4, 8).transpose(1, 2, 0, 3)
            r_pool[page, :, :n, :] = r[b, t0:t0 + n].transpose(1, 0, 2)
            v_pool[page, :, :, :n] = vb[b, t0:t0 + n].transpose(1, 2, 0)
    from ffa_mi355x.paged import CODES_ORDER, RES_ORDER, VT_ORDER, to_tiled

    pools = dict(k_q=to_tiled(kq_pool, CODES_ORDER, 8), k_res=to_tiled(r_pool, RES_ORDER), v=to_tiled(v_pool, VT_ORDER))
    return dict(q=q, k=k, v=v, k_q=pk, k_scale=s, k_zero=z, k_res=r, tau=tau, res=res, lens=lens, block_table=bt,
                pools=pools, P=P)


def to_gpu_paged(case, dev):
    from ffa_mi355x.paged import PagedQ2Cache

    P = case["P"]
    HKV = case["k_q"].shape[2]
    cache = PagedQ2Cache(P, HKV, dev, res_dtype=FP8_DT[case["res"]])
    p = case["pools"]
    cache.k_q.copy_(torch.from_numpy(p["k_q"]))
    cache.k_scale.copy_(torch.from_numpy(p["k_scale"].view(np.int16)).view(torch.float16))
    cache.k_zero.copy_(torch.from_numpy(p["k_zero"].view(np.int16)).view(torch.float16))
    cache.k_res.copy_(torch.from_numpy(p["k_res"]).view(FP8_DT[case["res"]]))
    cache.v.copy_(torch.from_numpy(p["v"].view(np.int16)).view(torch.bfloat16))  # stored as the pool dtype
    return cache


def oracle_paged(case, **kw):
    lens = case["lens"]
    return O.decode(f32(case["q"]), case["k_q"], case["k_scale"], case["k_zero"], f32(case["v"]), case["k_res"],
                    res_fmt=case["res"], scale_mode="g32", seq_lens=None if len(set(lens)) == 1 else lens,
                    out_dtype="bf16", **kw)


def compare_masks(mask_gpu: np.ndarray, diag: dict):
    """Return (n_mismatch_far, n_mismatch_near, n_near_total)."""
    mo = diag["mask"]
    marg = diag["margin"]
    mg = mask_gpu[..., : mo.shape[-1]]
    diff = mg != mo
    near = np.abs(marg) <= NEAR_TH
    return int((diff & ~near).sum()), int((diff & near).sum()), int(near.sum())


def assert_out_close(o_gpu: np.ndarray, o_ref: np.ndarray, what=""):
    d = np.abs(o_gpu.astype(np.float64) - o_ref.astype(np.float64))
    assert np.isfinite(o_gpu).all(), f"{what}: non-finite output"
    assert d.max() <= OUT_MAX_ABS, f"{what}: max abs diff {d.max():.3e} > {OUT_MAX_ABS}"
    assert d.mean() <= OUT_MEAN_ABS, f"{what}: mean abs diff {d.mean():.3e} > {OUT_MEAN_ABS}"
    return float(d.max()), float(d.mean())
