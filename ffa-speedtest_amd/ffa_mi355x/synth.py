"""Seeded synthetic inputs for the benchmark and test workloads (no recorded data).

The reference benchmarks recorded Llama layers (ffa-q2fp8/run_attn_bench_q2.py:26-29),
which are not available; these generators build inputs of the same shapes.
Everything is drawn on the CPU from torch.Generator(seed) so that every
machine produces the same tensors, then moved to `device`.

Heavy tokens (configs 2-5): per query head, `n_heavy` positions whose key is
a cosine-`cos` blend of that head's query direction and a random direction
orthogonal to it, with the norm of the key it replaces.  One of them lies in
tokens 0..15 (the first probe window, attn_kernel_v1210_fused_bsz_q2fp8.py:58-68)
so the threshold sees a heavy score and pruning engages.
"""
from __future__ import annotations

import math

import torch


def _plant_heavy(q, k, lens, n_heavy, cos, g):
    """q [B, HQ, D] f32, k [B, T, HKV, D] f32 (in place)."""
    B, HQ, D = q.shape
    HKV = k.shape[2]
    G = HQ // HKV
    sin = math.sqrt(max(0.0, 1.0 - cos * cos))
    for b in range(B):
        T = int(lens[b])
        for h in range(HKV):
            first = torch.randperm(min(16, T), generator=g)[:G]
            rest = 16 + torch.randperm(max(T - 16, 0), generator=g)[: G * (n_heavy - 1)] if T > 16 else first[:0]
            for gi in range(G):
                hq = h * G + gi
                qh = q[b, hq] / q[b, hq].norm()
                # sequences shorter than the group (or empty) get fewer heavy tokens
                pos = [int(x) for x in first[gi:gi + 1]] + [int(x) for x in rest[gi * (n_heavy - 1):(gi + 1) * (n_heavy - 1)]]
                for t in pos:
                    u = torch.randn(D, generator=g)
                    u = u - (u @ qh) * qh
                    u = u / u.norm()
                    k[b, t, h] = k[b, t, h].norm() * (cos * qh + sin * u)


def attention_inputs(B=1, T=32768, HQ=32, HKV=8, D=128, seed=0, n_heavy=16, cos=0.8, seq_lens=None,
                     outlier_channels=0, outlier_scale=10.0, dtype=torch.bfloat16, device="cpu"):
    """q [B, HQ, D], k/v [B, T, HKV, D] ~ N(0, 1) in `dtype`, optional heavy tokens / outliers.

    seq_lens: per-sequence lengths (ragged); positions >= seq_lens[b] are still
    filled but never used.
    """
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, HQ, D, generator=g)
    k = torch.randn(B, T, HKV, D, generator=g)
    v = torch.randn(B, T, HKV, D, generator=g)
    if outlier_channels:
        ch = torch.randperm(D, generator=g)[:outlier_channels]
        k[..., ch] *= outlier_scale
    lens = [T] * B if seq_lens is None else [int(x) for x in seq_lens]
    if n_heavy:
        _plant_heavy(q, k, lens, n_heavy, cos, g)
    return q.to(dtype).to(device), k.to(dtype).to(device), v.to(dtype).to(device)


def ragged_lengths(B, lo, hi, seed=0):
    g = torch.Generator().manual_seed(seed + 1)
    return torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int32)


def page_tables(seq_lens, page=64, seed=0, interleave=True, base=0):
    """Block tables for sequences of the given lengths over one page pool.

    Pages are drawn from a seeded random permutation of the pool, so
    consecutive pages of a sequence are scattered and sequences interleave.
    Returns (block_table [B, max_pages] int32, num_pages).
    """
    lens = [int(x) for x in seq_lens]
    npg = [-(-t // page) for t in lens]
    total = sum(npg)
    g = torch.Generator().manual_seed(seed + 2)
    perm = torch.randperm(total, generator=g) if interleave else torch.arange(total)
    bt = torch.zeros((len(lens), max(npg)), dtype=torch.int32)
    o = 0
    for b, n in enumerate(npg):
        bt[b, :n] = perm[o:o + n].to(torch.int32) + base
        o += n
    return bt, total


def sequence_inputs_device(q_seq, T, HKV=8, D=128, seed=0, n_heavy=16, cos=0.8, dtype=torch.bfloat16):
    """k, v [1, T, HKV, D] of one sequence, drawn on q_seq's device (for benchmark shapes too large to
    draw on the host).

    q_seq [HQ, D].  Same construction as `attention_inputs` (N(0, 1) K and V, n_heavy heavy keys per
    query head at cosine `cos` with it, one inside tokens 0..15) with the device's generator, so the
    values differ from the host-drawn ones of the same seed.
    """
    dev = q_seq.device
    g = torch.Generator(device=dev).manual_seed(seed)
    k = torch.randn((T, HKV, D), generator=g, device=dev)
    v = torch.randn((T, HKV, D), generator=g, device=dev, dtype=torch.float32).to(dtype)
    HQ = q_seq.shape[0]
    G = HQ // HKV
    sin = math.sqrt(max(0.0, 1.0 - cos * cos))
    if n_heavy and T > 16:
        qn = q_seq.float() / q_seq.float().norm(dim=-1, keepdim=True)  # [HQ, D]
        for h in range(HKV):
            first = torch.randperm(16, generator=g, device=dev)[:G]
            rest = 16 + torch.randperm(T - 16, generator=g, device=dev)[: G * (n_heavy - 1)]
            pos = torch.cat([first.view(G, 1), rest.view(G, n_heavy - 1)], 1)  # [G, n_heavy]
            qh = qn[h * G:(h + 1) * G].unsqueeze(1).expand(G, n_heavy, D)
            u = torch.randn((G, n_heavy, D), generator=g, device=dev)
            u = u - (u * qh).sum(-1, keepdim=True) * qh
            u = u / u.norm(dim=-1, keepdim=True)
            kn = k[pos, h].norm(dim=-1, keepdim=True)
            k[pos.reshape(-1), h] = (kn * (cos * qh + sin * u)).reshape(-1, D)
    return k.to(dtype).unsqueeze(0), v.unsqueeze(0)
