"""Pins of the oracle's mean-V variant (ffa-q2fp8-meanv/attn_kernel/attn_kernel_v1210_meanv_bsz_q2fp8.py).

The variant's output is softmax attention in which the tokens of pruned blocks keep their coarse
(2-bit) scores and take the mean of V as their value, while kept blocks use the refined scores
and their own V.  These tests state that directly with torch (K rebuilt from the codes without
the oracle's dequantization) and check the special cases it reduces to: nothing pruned is the
q2fp8 decode, everything pruned is v_mean.  A planted mistake, the refined scores for pruned
tokens, has to miss the tolerance.
"""
import math

import numpy as np
import torch

from helpers import FP8_DT, contig_case, f32
from oracle import q2fp8 as O


def _case(seed=5, T=300):
    return contig_case(B=2, T=T, HQ=8, HKV=2, tau="bf16", res="e5m2", seed=seed, n_heavy=2)


def _np(c):
    return f32(c["q"]), c["k_q"], c["k_scale"], c["k_zero"], f32(c["v"]), c["k_res"]


def _k_torch(c):
    """(coarse k_hat, refined k_tilde) [B, T, HKV, D] from the packed codes with torch ops."""
    kq = torch.from_numpy(c["k_q"]).long()
    codes = torch.stack([(kq >> (2 * i)) & 3 for i in range(4)], dim=-1).flatten(-2)[..., :128].float()
    khat = (codes * torch.from_numpy(c["k_scale"])[:, None] + torch.from_numpy(c["k_zero"])[:, None]).half()
    res = torch.from_numpy(c["k_res"]).view(FP8_DT[c["res"]]).half()
    return khat.double(), (khat + res).double()


def _softmax_with_mean(c, keep, v_mean, SBS, pruned_scores="coarse"):
    """out[b, hq] = sum_t w_t val_t with w = softmax over the sequence's tokens of s_t (coarse for the
    tokens of pruned blocks, refined for kept ones), val_t = v_t (kept) or v_mean (pruned)."""
    q, _, _, _, v, _ = _np(c)
    khat, ktil = _k_torch(c)
    qh = torch.from_numpy(q).half().double()
    vv = torch.from_numpy(v).half().double()
    vm = torch.from_numpy(np.asarray(v_mean, np.float64))
    B, HQ, D = q.shape
    T, HKV = khat.shape[1], khat.shape[2]
    G = HQ // HKV
    out = np.zeros((B, HQ, 128))
    blk = torch.arange(T) // SBS
    for b in range(B):
        for hq in range(HQ):
            h = hq // G
            kept_tok = torch.from_numpy(keep[b, h].astype(bool))[blk]
            k_pr = khat if pruned_scores == "coarse" else ktil
            kk = torch.where(kept_tok[:, None], ktil[b, :, h], k_pr[b, :, h])
            w = torch.softmax((kk @ qh[b, hq]) / math.sqrt(D), 0)
            val = torch.where(kept_tok[:, None], vv[b, :, h], vm[b, h][None, :])
            out[b, hq] = (w @ val).numpy()
    return out


def test_meanv_is_softmax_with_pruned_tokens_on_coarse_scores_and_mean_value():
    c = _case()
    q, kq, s, z, v, r = _np(c)
    BS = SBS = 32
    ntbs = math.ceil(300 / SBS)
    keep = (np.random.default_rng(0).random((2, 2, ntbs)) < 0.5).astype(np.int8)
    keep[:, :, 0] = 1  # some mass on exact blocks
    vmean = O.value_mean(v, out_dtype="bf16")
    o, diag = O.decode(q, kq, s, z, v, r, res_fmt="e5m2", BS=BS, SBS=SBS, delta=5.0, out_dtype="fp32",
                       force_mask=keep, v_mean=vmean)
    want = _softmax_with_mean(c, keep, vmean, SBS)
    err = np.abs(o - want).max()
    assert err < 5e-4, err  # fp16 rounding of the kept blocks' p only
    planted = _softmax_with_mean(c, keep, vmean, SBS, pruned_scores="refined")
    assert np.abs(o - planted).max() > 20 * 5e-4  # refined scores for pruned tokens would be caught
    assert np.array_equal(diag["approx"], (1 - keep).astype(np.int8))  # every block holds tokens here
    assert diag["approx_ratio"] == float((1 - keep).sum()) / keep.size


def test_meanv_nothing_pruned_is_the_q2fp8_decode():
    c = _case(seed=6)
    q, kq, s, z, v, r = _np(c)
    vmean = O.value_mean(v)
    a, _ = O.decode(q, kq, s, z, v, r, res_fmt="e5m2", BS=64, SBS=32, delta=math.inf, out_dtype="bf16")
    b, diag = O.decode(q, kq, s, z, v, r, res_fmt="e5m2", BS=64, SBS=32, delta=math.inf, out_dtype="bf16",
                       v_mean=vmean)
    assert np.array_equal(a, b) and diag["approx"].sum() == 0


def test_meanv_everything_pruned_is_v_mean():
    c = _case(seed=7)
    q, kq, s, z, v, r = _np(c)
    vmean = O.value_mean(v, out_dtype="bf16")
    o, diag = O.decode(q, kq, s, z, v, r, res_fmt="e5m2", BS=64, SBS=32, delta=-math.inf, out_dtype="fp32",
                       v_mean=vmean)
    G = 4
    assert np.array_equal(o, np.repeat(vmean, G, axis=1))
    # BS=64 over T=300: 5 threshold blocks x 2 prune blocks of 32; the last, [288, 320), still holds
    # tokens 288..299, so all 10 blocks are approximated
    assert diag["approx_ratio"] == 1.0


def test_meanv_empty_blocks_are_not_approximated():
    c = contig_case(B=1, T=70, HQ=4, HKV=1, tau="bf16", res="e5m2", seed=8)
    q, kq, s, z, v, r = _np(c)
    o, diag = O.decode(q, kq, s, z, v, r, res_fmt="e5m2", BS=128, SBS=32, delta=-math.inf, out_dtype="fp32",
                       v_mean=O.value_mean(v))
    # blocks of 32: [0,32) [32,64) [64,96) hold tokens, [96,128) does not
    assert diag["approx"][0, 0].tolist() == [1, 1, 1, 0]
    assert diag["approx_ratio"] == 3 / 4


def test_value_mean_matches_torch_mean():
    g = torch.Generator().manual_seed(0)
    v = torch.randn(2, 777, 3, 128, generator=g).bfloat16()
    want = v.mean(dim=1, dtype=torch.float32).to(torch.bfloat16).float().numpy()  # reference :332
    got = O.value_mean(f32(v), out_dtype="bf16")
    diff = np.abs(got - want)
    ulp = np.abs(want) * 2.0 ** -7 + 1e-30
    assert (diff <= ulp).all() and (diff == 0).mean() > 0.99
    # integer data: the mean is exact
    vi = torch.arange(40, dtype=torch.float32).reshape(1, 10, 1, 4).repeat(1, 1, 1, 32)
    m = O.value_mean(vi.numpy(), out_dtype="fp32")
    assert np.array_equal(m[0, 0], vi[0, :, 0].mean(0).numpy())
    # ragged: each sequence its own tokens, an empty one 0
    m2 = O.value_mean(f32(v), seq_lens=[5, 0], out_dtype="fp32")
    assert np.allclose(m2[0], f32(v)[0, :5].mean(0), atol=1e-6) and (m2[1] == 0).all()
