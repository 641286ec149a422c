"""GPU parity of the mean-V variant (ffa-q2fp8-meanv) and of ffa_v_mean against the oracle.

v_mean: the kernels' fp32 sums against the oracle's exact mean, both rounded once to the output
type: equal but for rounding ties (at most one unit in the last place).  Decode: the survivor
mask as in the q2fp8 tests (no mismatch away from the threshold), the output under the GPU's own
mask and v_mean within the decode tolerance, and the approximated-block ratio.
"""
import math

import numpy as np
import pytest
import torch

from helpers import (assert_out_close, compare_masks, contig_case, f32, oracle_paged, paged_case, to_gpu_contig,
                     to_gpu_paged)
from oracle import q2fp8 as O

pytestmark = pytest.mark.gpu

ULP = {"bf16": 2.0 ** -7, "fp16": 2.0 ** -10}


def _meanv_module():
    from ffa_mi355x.dropins import _ROOT, _load

    return _load("ffa_mi355x_meanv_dropin", _ROOT / "ffa-q2fp8-meanv" / "attn_kernel" / "attn_kernel_v1210_meanv_bsz_q2fp8.py")


def _close_to_ulp(got, want, dt):
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    return bool((d <= np.abs(want) * ULP[dt] + 1e-30).all()), float((d == 0).mean())


@pytest.mark.parametrize("dt,lens", [("bf16", None), ("fp16", [1000, 37]), ("bf16", [0, 999])])
def test_value_mean_contiguous(gpu, dt, lens):
    from ffa_mi355x.meanv import value_mean

    g = torch.Generator().manual_seed(3)
    v = (torch.randn(2, 1000, 8, 128, generator=g) * 2).to({"bf16": torch.bfloat16, "fp16": torch.float16}[dt])
    sl = torch.tensor(lens, dtype=torch.int32, device=gpu) if lens is not None else None
    got = f32(value_mean(v.to(gpu), seq_lens=sl))
    want = O.value_mean(f32(v), seq_lens=lens, out_dtype=dt)
    ok, exact = _close_to_ulp(got, want, dt)
    print(f"[v_mean] contiguous {dt} lens={lens}: exact fraction {exact:.4f}")
    assert ok and exact > 0.98
    got32 = f32(value_mean(v.to(gpu), seq_lens=sl, out_dtype=torch.float32))
    want32 = O.value_mean(f32(v), seq_lens=lens, out_dtype="fp32")
    assert np.allclose(got32, want32, rtol=1e-5, atol=1e-6)


def test_value_mean_paged(gpu):
    c = paged_case(B=3, T=2500, HQ=32, HKV=8, seed=31, n_heavy=4, seq_lens=[2500, 700, 65])
    cache = to_gpu_paged(c, gpu)
    bt = c["block_table"].to(gpu)
    sl = torch.tensor(c["lens"], dtype=torch.int32, device=gpu)
    got = f32(cache.value_mean(bt, sl))
    vpool = f32(c["v"].to(cache.v.dtype))  # the pool holds V rounded to its dtype
    want = O.value_mean(vpool, seq_lens=c["lens"], out_dtype="fp16")
    ok, exact = _close_to_ulp(got, want, "fp16")
    print(f"[v_mean] paged: exact fraction {exact:.4f}")
    assert ok and exact > 0.98


@pytest.mark.parametrize(
    "T,HQ,BS,SBS,delta",
    [
        (1000, 32, 128, None, 5.0),   # reference defaults
        (4096, 32, 64, 64, 3.0),
        (2048, 32, 256, 32, 2.0),
        (3000, 64, 128, 128, 3.0),    # G = 8: two passes
        (4096, 32, 1024, None, 3.0),  # SBS = 1024: two passes
    ],
)
def test_meanv_contiguous_dropin(gpu, T, HQ, BS, SBS, delta):
    K = _meanv_module()
    case = contig_case(B=2, T=T, HQ=HQ, HKV=8, tau="bf16", res="e5m2", seed=T + HQ, n_heavy=8)
    g = to_gpu_contig(case, gpu)
    ws = K.allocate_q2fp8_decode_workspace(g["q"], g["k_q"], g["v"], BS=BS, SBS=SBS)
    o, ratio = K.attn_forward_decode_quantized(g["q"], g["k_q"], g["k_scale"], g["k_zero"], g["v"],
                                               k_residual=g["k_residual"], BS=BS, SBS=SBS, delta=delta,
                                               return_skip_ratio=True, workspace=ws)
    torch.cuda.synchronize()
    SBSv = BS if SBS is None else SBS
    q, v = f32(case["q"]), f32(case["v"])
    vmean = O.value_mean(v, out_dtype="bf16")
    args = (q, case["k_q"], case["k_scale"], case["k_zero"], v, case["k_res"])
    o_ref, diag = O.decode(*args, res_fmt="e5m2", BS=BS, SBS=SBSv, delta=delta, out_dtype="bf16", v_mean=vmean)
    mask = ws.mask_buf.cpu().numpy()
    far, near, n_near = compare_masks(mask, diag)
    print(f"[meanv] T={T} HQ={HQ} BS={BS} SBS={SBSv} approx={ratio:.3f} oracle={diag['approx_ratio']:.3f} "
          f"far={far} near={near}/{n_near}")
    assert far == 0
    if near == 0:
        assert abs(ratio - diag["approx_ratio"]) < 1e-9
        # the reference's per-block flags (approx_buf, and mask_buf = exact or approximated)
        from ffa_mi355x.meanv import approx_flags

        m_ref, apx = approx_flags(ws.mask_buf, T, BS, SBSv)
        n = diag["approx"].shape[-1]
        assert np.array_equal(apx.cpu().numpy()[..., :n], diag["approx"])
        assert np.array_equal(m_ref.cpu().numpy()[..., :n], diag["approx"] | diag["mask"])
        assert int(apx.sum()) == int(diag["approx"].sum())
    o_forced, _ = O.decode(*args, res_fmt="e5m2", BS=BS, SBS=SBSv, delta=delta, out_dtype="bf16", v_mean=vmean,
                           force_mask=mask)
    mx, mean = assert_out_close(f32(o), o_forced, "meanv contiguous")
    print(f"[out] max_abs={mx:.3e} mean_abs={mean:.3e}")
    # the variant differs from the q2fp8 decode wherever something was pruned
    o_plain, _ = O.decode(*args, res_fmt="e5m2", BS=BS, SBS=SBSv, delta=delta, out_dtype="bf16", force_mask=mask)
    if diag["approx_ratio"] > 0.2:
        assert np.abs(o_plain - o_forced).max() > 10 * np.abs(f32(o) - o_forced).max()


def test_meanv_paged_ragged_and_all_pruned(gpu):
    c = paged_case(B=3, T=3000, HQ=32, HKV=8, seed=41, n_heavy=8, seq_lens=[3000, 1111, 65])
    cache = to_gpu_paged(c, gpu)
    q = c["q"].to(gpu)
    bt = c["block_table"].to(gpu)
    sl = torch.tensor(c["lens"], dtype=torch.int32, device=gpu)
    vm = cache.value_mean(bt, sl, T=3000)
    ws = cache.decode(q, bt, sl, T=3000, BS=64, SBS=64, delta=3.0, v_mean=vm)
    torch.cuda.synchronize()
    mask = ws.mask_buf.cpu().numpy()
    o_ref, diag = oracle_paged(c, BS=64, SBS=64, delta=3.0, v_mean=f32(vm))
    far, near, n_near = compare_masks(mask, diag)
    assert far == 0
    o_forced, _ = oracle_paged(c, BS=64, SBS=64, delta=3.0, v_mean=f32(vm), force_mask=mask)
    mx, mean = assert_out_close(f32(ws.o), o_forced, "meanv paged")
    print(f"[meanv paged] far={far} near={near}/{n_near} max_abs={mx:.3e} mean_abs={mean:.3e}")
    # delta = -inf: every block pruned, every output row is its KV head's v_mean
    ws2 = cache.decode(q.float(), bt, sl, T=3000, BS=64, SBS=64, delta=-math.inf, v_mean=vm)
    torch.cuda.synchronize()
    assert int(ws2.mask_buf.sum().item()) == 0
    want = vm.float().repeat_interleave(4, dim=1)
    assert torch.allclose(ws2.o, want, rtol=1e-6, atol=0)



@pytest.mark.parametrize("B", [1, 9])  # 32 query rows (eager merge) / 288 rows (lazy merge)
@pytest.mark.parametrize("with_vmean", [False, True])
def test_merge_long_rows_in_batches(gpu, B, with_vmean):
    """Stage 2 alone on synthetic partials of 136,000-token rows: 266 partial slots per row, which
    the merge takes in two batches of four per lane with the running maximum rescaled between
    them.  Expected: the reference's log-sum-exp merge (attn_kernel...q2fp8.py:156-171, and the
    mean-V fold of attn_kernel_v1210_meanv_bsz_q2fp8.py:192-202) in float64."""
    from ffa_mi355x.decode import DecodeWorkspace
    from ffa_mi355x.paged import PagedQ2Cache

    T, HQ, HKV, D = 136_000, 32, 8, 128
    cache = PagedQ2Cache(4, HKV, gpu)  # stage 2 never reads the pools; the call only needs valid ones
    bt = torch.zeros((B, (T + 63) // 64), dtype=torch.int32, device=gpu)
    ws = DecodeWorkspace(B, HQ, HKV, T, 64, 64, gpu, torch.float32)
    n = -(-T // 512)
    assert ws.nparts >= n > 256
    rng = np.random.default_rng(61 + B)
    m = rng.normal(0.0, 3.0, (B, HQ, n)).astype(np.float32)
    kept = rng.random((B, HQ, n)) < 0.4
    kept[0, 0] = False  # one row with nothing kept
    l = np.where(kept, rng.uniform(0.5, 8.0, (B, HQ, n)), 0.0).astype(np.float32)
    m = np.where(kept, m, -np.inf).astype(np.float32)
    o = rng.normal(0.0, 1.0, (B, HQ, n, D)).astype(np.float32)
    ws.m_buf[..., :n].copy_(torch.from_numpy(m))
    ws.l_buf[..., :n].copy_(torch.from_numpy(l))
    ws.o_buf[..., :n, :].copy_(torch.from_numpy(o))
    vm = None
    if with_vmean:
        am = rng.normal(0.0, 3.0, (B, HQ, n)).astype(np.float32)
        al = np.where(rng.random((B, HQ, n)) < 0.7, rng.uniform(0.5, 8.0, (B, HQ, n)), 0.0).astype(np.float32)
        ws.approx_m[..., :n].copy_(torch.from_numpy(am))
        ws.approx_l[..., :n].copy_(torch.from_numpy(al))
        vm_np = rng.normal(0.0, 1.0, (B, HKV, D)).astype(np.float32)
        vm = torch.from_numpy(vm_np).to(gpu)
    q = torch.zeros((B, HQ, D), dtype=torch.float32, device=gpu)
    cache.decode(q, bt, None, T=T, BS=64, SBS=64, delta=5.0, workspace=ws, stage="stage2", v_mean=vm)
    torch.cuda.synchronize()
    got = ws.o.cpu().numpy().astype(np.float64)

    md, ld, od = m.astype(np.float64), l.astype(np.float64), o.astype(np.float64)
    want = np.zeros((B, HQ, D))
    for b in range(B):
        for h in range(HQ):
            k = ld[b, h] > 0
            M = md[b, h, k].max() if k.any() else -np.inf
            w = np.where(k, np.exp2(np.where(k, md[b, h], 0.0) - (M if k.any() else 0.0)), 0.0)
            A = (ld[b, h] * w).sum()
            acc = (od[b, h] * w[:, None]).sum(0)
            if not with_vmean:
                want[b, h] = acc / A if A > 0 else 0.0
                continue
            ka = al[b, h] > 0
            AM = am[b, h, ka].max() if ka.any() else -np.inf
            AL = (al[b, h, ka] * np.exp2(am[b, h, ka].astype(np.float64) - AM)).sum() if ka.any() else 0.0
            Mx = max(M if A > 0 else -np.inf, AM if AL > 0 else -np.inf)
            re = np.exp2(M - Mx) if A > 0 else 0.0
            ra = np.exp2(AM - Mx) if AL > 0 else 0.0
            den = A * re + AL * ra
            want[b, h] = (acc * re + vm_np[b, h // (HQ // HKV)] * AL * ra) / den if den > 0 else 0.0
    err = np.abs(got - want).max()
    print(f"[merge batches] B={B} v_mean={with_vmean} partials={n} max_abs={err:.3e}")
    assert np.isfinite(got).all()
    assert err < 1e-4
