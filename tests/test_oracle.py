"""Pins of the CPU oracle (no GPU).

The reference ships no golden vectors or known-answer tests for this path
(its only checks are CUDA smoke tests, ffa-q2fp8/fused_kproj_rope_q2fp8.py:569-625),
so the oracle is pinned by:
  * library routines that implement the same number formats (torch casts),
  * the reference's own torch op sequence for the quantizer, run by torch on
    the CPU (run_attn_bench_q2.py:78-105 restated),
  * hand-built known answers (ties, clamps, padding, constant channels),
  * special cases that reduce to textbook attention (delta=+inf -> softmax
    over refined K; delta=-inf -> all pruned -> zeros),
  * the reference's host threshold (ffa-fp8 ...v1208_fused_bsz_fp8.py:174-234),
  * an independent scalar-loop statement on tiny shapes,
  * invariants of the merge and of paging.
"""
import math

import numpy as np
import pytest
import torch

from helpers import FP8_DT, TORCH_DT, contig_case, f32, paged_case
from oracle import numerics as NM
from oracle import q2fp8 as O


# ----------------------------------------------------------------------------- formats
@pytest.mark.parametrize("fmt", ["e4m3fn", "e5m2"])
def test_fp8_encode_matches_torch_on_every_fp16(fmt):
    h = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    ref = torch.from_numpy(h).to(FP8_DT[fmt]).view(torch.uint8).numpy()
    assert (NM.fp8_encode(h, fmt) == ref).all()


@pytest.mark.parametrize("fmt", ["e4m3fn", "e5m2"])
def test_fp8_encode_random_f32_and_decode(fmt):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(200_000) * np.exp(rng.uniform(-30, 14, 200_000))).astype(np.float32)
    ref = torch.from_numpy(x).to(FP8_DT[fmt]).view(torch.uint8).numpy()
    assert (NM.fp8_encode(x, fmt) == ref).all()
    dec = NM.fp8_decode(np.arange(256), fmt)
    tdec = torch.arange(256, dtype=torch.uint8).view(FP8_DT[fmt]).float().numpy()
    assert ((dec == tdec) | (np.isnan(dec) & np.isnan(tdec))).all()


def test_fp8_golden_table():
    """Committed fixture: torch's fp16 -> fp8 tables (tests/golden/fp8_from_fp16.npz)."""
    from pathlib import Path

    g = np.load(Path(__file__).parent / "golden" / "fp8_from_fp16.npz")
    h = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    assert (NM.fp8_encode(h, "e4m3fn") == g["e4m3fn"]).all()
    assert (NM.fp8_encode(h, "e5m2") == g["e5m2"]).all()


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(500_000) * np.exp(rng.uniform(-40, 40, 500_000))).astype(np.float32)
    assert (NM.round_bf16(x) == torch.from_numpy(x).bfloat16().float().numpy()).all()


# ----------------------------------------------------------------------------- quantizer
def _torch_reference_quantizer(k, fp8):
    """The reference's op sequence (run_attn_bench_q2.py:78-105), run by torch on the CPU."""
    k_min = k.amin(dim=1)
    k_max = k.amax(dim=1)
    scale = ((k_max - k_min).clamp_min(1e-6) / 3.0).contiguous()
    zero = k_min.contiguous()
    k_q = torch.round((k - zero[:, None]) / scale[:, None]).clamp(0, 3).to(torch.uint8)
    k_dequant = k_q.to(torch.float32) * scale[:, None].to(torch.float32) + zero[:, None].to(torch.float32)
    k_residual = (k.to(torch.float32) - k_dequant).to(fp8).contiguous()
    B, T, HKV, K = k_q.shape
    kp = (K + 3) // 4
    pad = kp * 4 - K
    if pad:
        k_q = torch.cat([k_q, torch.zeros((B, T, HKV, pad), dtype=k_q.dtype)], dim=-1)
    k_q = k_q.view(B, T, HKV, kp, 4)
    packed = (k_q[..., 0] | (k_q[..., 1] << 2) | (k_q[..., 2] << 4) | (k_q[..., 3] << 6)).contiguous()
    return packed, scale, zero, k_residual


@pytest.mark.parametrize("tau", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("fmt", ["e5m2", "e4m3fn"])
def test_quantizer_matches_torch_ops(tau, fmt):
    g = torch.Generator().manual_seed(11)
    k = (torch.randn(2, 333, 3, 130, generator=g) * 3).to(TORCH_DT[tau])
    k[:, :, 1, 7] = 0.5  # constant channel -> clamp_min(1e-6)
    k[0, :, 2, 9] = torch.linspace(-1, 1, 333).to(TORCH_DT[tau])
    pk, s, z, r = O.quantize_per_channel(f32(k), tau, fmt)
    tp, ts, tz, tr = _torch_reference_quantizer(k, FP8_DT[fmt])
    assert (pk == tp.numpy()).all()
    assert (s == ts.float().numpy()).all()
    assert (z == tz.float().numpy()).all()
    assert (r == tr.view(torch.uint8).numpy()).all()


def test_quantizer_known_answers():
    # one channel over T = 5 tokens: values 0, 1, 1.5, 2.5, 3  -> zero 0, scale 1
    k = np.array([0.0, 1.0, 1.5, 2.5, 3.0], np.float32).reshape(1, 5, 1, 1)
    k = np.concatenate([k, np.zeros((1, 5, 1, 5), np.float32)], axis=-1)  # D = 6 (pads to 8)
    pk, s, z, r = O.quantize_per_channel(k, "fp32", "e4m3fn")
    c = O.unpack_2bit(pk, 6)[0, :, 0, 0]
    assert s[0, 0, 0] == 1.0 and z[0, 0, 0] == 0.0
    assert list(c) == [0, 1, 2, 2, 3]  # 1.5 -> 2 and 2.5 -> 2 (round half to even)
    res = NM.fp8_decode(r[0, :, 0, 0], "e4m3fn")
    assert list(res) == [0.0, 0.0, -0.5, 0.5, 0.0]
    # constant channels: scale = 1e-6/3 rounded, codes 0, residual 0
    assert (O.unpack_2bit(pk, 6)[0, :, 0, 1:] == 0).all()
    assert np.isclose(s[0, 0, 1], np.float32(np.float32(1e-6) / np.float32(3.0)))
    # padding codes of the last byte are zero
    assert (pk[..., 1] >> 4 == 0).all()


@pytest.mark.parametrize("tau", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("fmt", ["e5m2", "e4m3fn"])
def test_channel_append_matches_torch_ops_with_the_cache_scale(tau, fmt):
    """New tokens quantized with an existing cache's scale / zero: the reference's op sequence
    (run_attn_bench_q2.py:84-88) run by torch with those scale / zero, including values outside
    [zero, zero + 3 scale] (codes clamp to 0 / 3, the residual carries the rest)."""
    g = torch.Generator().manual_seed(12)
    k0 = (torch.randn(2, 200, 3, 130, generator=g) * 2).to(TORCH_DT[tau])
    _, s, z, _ = O.quantize_per_channel(f32(k0), tau, fmt)
    k_new = (torch.randn(2, 9, 3, 130, generator=g) * 4).to(TORCH_DT[tau])  # many outside the cache's range
    pk, rr = O.quantize_with_channel_scale(f32(k_new), s, z, tau, fmt)
    ts, tz = torch.from_numpy(s).to(TORCH_DT[tau]), torch.from_numpy(z).to(TORCH_DT[tau])
    c = torch.round((k_new - tz[:, None]) / ts[:, None]).clamp(0, 3).to(torch.uint8)
    deq = c.to(torch.float32) * ts[:, None].to(torch.float32) + tz[:, None].to(torch.float32)
    tr = (k_new.to(torch.float32) - deq).to(FP8_DT[fmt])
    cu = O.unpack_2bit(pk, 130)
    assert (cu == c.numpy()).all()
    assert (rr == tr.view(torch.uint8).numpy()).all()
    assert (cu == 0).any() and (cu == 3).any()


def test_channel_append_reproduces_the_quantizer_and_drops_positions_past_the_end():
    rng = np.random.default_rng(13)
    k = NM.round_bf16(rng.standard_normal((2, 100, 2, 128)).astype(np.float32))
    pk, s, z, r = O.quantize_per_channel(k, "bf16", "e5m2")
    # re-appending tokens 60..99 of each sequence over a cache that holds only tokens 0..59
    kq0 = pk.copy()
    kr0 = r.copy()
    kq0[:, 60:] = 0
    kr0[:, 60:] = 0
    kq1, kr1 = O.append_per_channel(kq0, kr0, k[:, 60:], s, z, [60, 60], "bf16", "e5m2")
    assert np.array_equal(kq1, pk) and np.array_equal(kr1, r)
    # positions beyond the cache are dropped, earlier positions overwritten
    kq2, kr2 = O.append_per_channel(pk, r, k[:, :5], s, z, [97, -2], "bf16", "e5m2")
    assert np.array_equal(kq2[0, 97:], pk[0, :3]) and np.array_equal(kq2[0, :97], pk[0, :97])
    assert np.array_equal(kq2[1, :3], pk[1, 2:5]) and np.array_equal(kq2[1, 3:], pk[1, 3:])


def test_channel_append_known_answers():
    # one channel with zero 0 and scale 1 (cache values 0 .. 3): a new token's -2 takes code 0 and
    # residual -2, 7 takes code 3 and residual 4, 1.5 takes code 2 (half to even) and residual -0.5;
    # 7.5 also takes code 3, its residual 4.5 rounds to 4 in e5m2 (half to even)
    s = np.ones((1, 1, 1), np.float32)
    z = np.zeros((1, 1, 1), np.float32)
    k_new = np.array([-2.0, 7.0, 1.5, 7.5], np.float32).reshape(1, 4, 1, 1)
    pk, rr = O.quantize_with_channel_scale(k_new, s, z, "fp32", "e5m2")
    assert list(O.unpack_2bit(pk, 1)[0, :, 0, 0]) == [0, 3, 2, 3]
    assert list(NM.fp8_decode(rr[0, :, 0, 0], "e5m2")) == [-2.0, 4.0, -0.5, 4.0]


def test_g32_quantizer_invariants():
    rng = np.random.default_rng(5)
    k = NM.round_bf16(rng.standard_normal((2, 70, 4, 128)).astype(np.float32) * 2)
    pk, s, z, r = O.quantize_g32(k, "e4m3fn")
    c = O.unpack_2bit(pk, 128).reshape(2, 70, 4, 4, 32)
    kg = k.reshape(2, 70, 4, 4, 32)
    deq = (c.astype(np.float32) * s[..., None]).astype(np.float32) + z[..., None]
    # codes hit 0 and 3 in every group that is not constant, the residual recovers k to fp8 precision
    assert (c.min(axis=-1) == 0).all() and (c.max(axis=-1) == 3).all()
    rr = NM.fp8_decode(r, "e4m3fn").reshape(kg.shape)
    assert np.abs(deq + rr - kg).max() <= np.abs(kg - deq).max() * 2 ** -3 + 1e-6
    assert (np.abs(kg - deq) <= s[..., None] * 0.5 + 1e-3).all()


# ----------------------------------------------------------------------------- decode
def _small():
    return contig_case(B=2, T=150, HQ=8, HKV=2, tau="bf16", res="e5m2", seed=4, n_heavy=2)


def _np_inputs(c):
    return f32(c["q"]), c["k_q"], c["k_scale"], c["k_zero"], f32(c["v"]), c["k_res"]


@pytest.mark.parametrize("BS,SBS,delta", [(64, 32, 1.0), (32, 32, 3.0), (48, 32, 2.0), (128, 64, 5.0)])
def test_decode_matches_scalar_statement(BS, SBS, delta):
    c = contig_case(B=1, T=150, HQ=4, HKV=2, tau="bf16", res="e5m2", seed=1, n_heavy=1)
    q, kq, s, z, v, r = _np_inputs(c)
    q, kq, s, z, v, r = q[:, :, :32], kq[..., :8], s[..., :32], z[..., :32], v[..., :16], r[..., :32]
    o, _ = O.decode(q, kq, s, z, v, r, res_fmt="e5m2", BS=BS, SBS=SBS, delta=delta, out_dtype="bf16")
    ob = O.decode_bruteforce(q, kq, s, z, v, r, res_fmt="e5m2", BS=BS, SBS=SBS, delta=delta, out_dtype="bf16")
    assert np.array_equal(o, ob)


def test_decode_g32_matches_scalar_statement():
    c = paged_case(B=1, T=100, HQ=4, HKV=2, seed=2, n_heavy=1)
    q, v = f32(c["q"]), f32(c["v"])
    o, _ = O.decode(q, c["k_q"], c["k_scale"], c["k_zero"], v, c["k_res"], res_fmt="e4m3fn", BS=32, SBS=32,
                    delta=2.0, scale_mode="g32", out_dtype="bf16")
    ob = O.decode_bruteforce(q, c["k_q"], c["k_scale"], c["k_zero"], v, c["k_res"], res_fmt="e4m3fn", BS=32, SBS=32,
                             delta=2.0, scale_mode="g32", out_dtype="bf16")
    assert np.array_equal(o, ob)


def _refined_k_torch(c):
    """k_tilde = fp16(fp16(c*s+z) + fp16(res)) rebuilt with torch ops (independent of the oracle's dequant)."""
    kq = torch.from_numpy(c["k_q"]).long()
    codes = torch.stack([(kq >> (2 * i)) & 3 for i in range(4)], dim=-1).flatten(-2)[..., :128].float()
    s = torch.from_numpy(c["k_scale"])[:, None]
    z = torch.from_numpy(c["k_zero"])[:, None]
    khat = (codes * s + z).half()
    res = torch.from_numpy(c["k_res"]).view(FP8_DT[c["res"]]).half()
    return (khat + res).double()


def test_no_pruning_equals_softmax_attention():
    """delta = +inf: threshold -inf, every block kept -> plain softmax attention over refined K."""
    c = _small()
    q, kq, s, z, v, r = _np_inputs(c)
    o, diag = O.decode(q, kq, s, z, v, r, res_fmt="e5m2", BS=64, SBS=32, delta=math.inf, out_dtype="fp32")
    assert diag["skip_ratio"] == 0.0
    kt = _refined_k_torch(c)  # [B, T, HKV, D]
    qh = torch.from_numpy(q).half().double()
    vv = torch.from_numpy(v).half().double()
    B, HQ, D = q.shape
    G = HQ // kt.shape[2]
    for b in range(B):
        for hq in range(HQ):
            sc = (kt[b, :, hq // G] @ qh[b, hq]) / math.sqrt(D)
            ref = torch.softmax(sc, 0) @ vv[b, :, hq // G]
            assert np.abs(o[b, hq] - ref.numpy()).max() < 2e-3


def test_all_pruned_gives_zero():
    c = _small()
    q, kq, s, z, v, r = _np_inputs(c)
    o, diag = O.decode(q, kq, s, z, v, r, res_fmt="e5m2", BS=64, SBS=32, delta=-math.inf, out_dtype="bf16")
    assert (o == 0).all() and diag["skip_ratio"] == 1.0 and diag["mask"].sum() == 0


def test_threshold_matches_reference_host_threshold():
    """Internal probe threshold == compute_threshold_external on the 2-bit K (ffa-fp8 v1208:174-234)."""
    c = contig_case(B=2, T=700, HQ=8, HKV=2, tau="bf16", res="e5m2", seed=9, n_heavy=3)
    q, kq, s, z, v, r = _np_inputs(c)
    BS = 64
    _, diag = O.decode(q, kq, s, z, v, r, res_fmt="e5m2", BS=BS, delta=4.0)
    khat = O.dequant(kq, s, z, 128, "per_channel")
    NTB = -(-700 // BS)
    th = O.threshold_external(NM.round_f16(q), khat, 1 / math.sqrt(128), NTB, 4.0, 2, 8)
    assert np.allclose(diag["threshold"], th, rtol=0, atol=2e-5)
    # the "last" probe window is [(NTB-1)*16, (NTB-1)*16+16), not the last block (quirk, :70-73)
    assert (NTB - 1) * 16 == 160


def test_precomputed_threshold_reproduces_mask():
    c = _small()
    q, kq, s, z, v, r = _np_inputs(c)
    o1, d1 = O.decode(q, kq, s, z, v, r, res_fmt="e5m2", BS=64, SBS=32, delta=2.0)
    o2, d2 = O.decode(q, kq, s, z, v, r, res_fmt="e5m2", BS=64, SBS=32, delta=123.0,
                      precomputed_threshold=d1["threshold"])
    assert np.array_equal(d1["mask"], d2["mask"]) and np.array_equal(o1, o2)


def test_merge_is_partition_invariant():
    """Kept-block partials merged by LSE equal the direct softmax over the kept tokens (SBS changes only the split)."""
    c = _small()
    q, kq, s, z, v, r = _np_inputs(c)
    o16, _ = O.decode(q, kq, s, z, v, r, res_fmt="e5m2", BS=64, SBS=16, delta=math.inf, out_dtype="fp32")
    o64, _ = O.decode(q, kq, s, z, v, r, res_fmt="e5m2", BS=64, SBS=64, delta=math.inf, out_dtype="fp32")
    assert np.abs(o16 - o64).max() < 5e-4  # only fp16(p) rounding of P.V differs


def test_paged_gather_is_layout_only():
    """The paged pools built for the GPU gather back to the contiguous arrays the oracle used."""
    from ffa_mi355x.paged import CODES_ORDER, RES_ORDER, VT_ORDER, to_logical

    c = paged_case(B=2, T=300, HQ=8, HKV=2, seed=3, n_heavy=2, seq_lens=[300, 130])
    p = dict(c["pools"])
    p["k_q"] = to_logical(p["k_q"], CODES_ORDER, 8)  # stored block order -> logical page order
    p["k_res"] = to_logical(p["k_res"], RES_ORDER)
    p["v"] = to_logical(p["v"], VT_ORDER)
    for b, T in enumerate(c["lens"]):
        bt = c["block_table"][b].numpy()
        kq = O.gather_pages(p["k_q"].reshape(*p["k_q"].shape[:2], 4, 64, 8).transpose(0, 1, 3, 2, 4).reshape(
            p["k_q"].shape[0], 2, 64, 32), bt, T)
        assert np.array_equal(kq, c["k_q"][b, :T])
        vv = O.gather_pages(p["v"], bt, T, v_transposed=True)
        assert np.array_equal(vv, c["v"][b, :T].view(torch.int16).numpy().view(np.uint16))
        rr = O.gather_pages(p["k_res"], bt, T)
        assert np.array_equal(rr, c["k_res"][b, :T])


def test_ragged_lengths_are_independent_sequences():
    c = paged_case(B=2, T=300, HQ=8, HKV=2, seed=3, n_heavy=2, seq_lens=[300, 130])
    q, v = f32(c["q"]), f32(c["v"])
    o, d = O.decode(q, c["k_q"], c["k_scale"], c["k_zero"], v, c["k_res"], res_fmt="e4m3fn", BS=64, scale_mode="g32",
                    seq_lens=c["lens"], out_dtype="bf16", delta=3.0)
    o1, _ = O.decode(q[1:], c["k_q"][1:, :130], c["k_scale"][1:, :130], c["k_zero"][1:, :130], v[1:, :130],
                     c["k_res"][1:, :130], res_fmt="e4m3fn", BS=64, scale_mode="g32", out_dtype="bf16", delta=3.0)
    assert np.array_equal(o[1:], o1)
    assert d["mask"][1, :, 3:].sum() == 0  # blocks past the sequence end do not exist


def test_empty_and_one_token_sequences():
    """An empty sequence gives zero output, no kept blocks and a -inf threshold; a one-token
    sequence attends to its only token (softmax weight 1: the output is that token's V in bf16),
    and the other sequences are unchanged by their presence."""
    c = paged_case(B=3, T=300, HQ=8, HKV=2, seed=4, n_heavy=2, seq_lens=[300, 0, 1])
    q, v = f32(c["q"]), f32(c["v"])
    o, d = O.decode(q, c["k_q"], c["k_scale"], c["k_zero"], v, c["k_res"], res_fmt="e4m3fn", BS=64, scale_mode="g32",
                    seq_lens=c["lens"], out_dtype="bf16", delta=3.0)
    assert (o[1] == 0).all() and d["mask"][1].sum() == 0 and np.isneginf(d["threshold"][1]).all()
    v1 = NM.round_bf16(v[2, 0])  # [HKV, 128]
    assert np.array_equal(o[2], np.repeat(v1, 4, axis=0))
    assert d["mask"][2, :, 0].all() and d["mask"][2, :, 1:].sum() == 0
    o0, _ = O.decode(q[:1], c["k_q"][:1], c["k_scale"][:1], c["k_zero"][:1], v[:1], c["k_res"][:1],
                     res_fmt="e4m3fn", BS=64, scale_mode="g32", out_dtype="bf16", delta=3.0)
    assert np.array_equal(o[:1], o0)
