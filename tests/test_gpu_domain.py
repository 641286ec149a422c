"""GPU parity over the reference's whole argument domain for the decode entry points.

The reference takes any GQA group up to its 16-row tile (attn_kernel_v1210_fused_bsz_q2fp8.py:19,
40-41) and any power-of-two prune block, with SBS defaulting to BS (:251-252); its own sweep runs
BS 64..4096 x SBS 64..512 (ffa-q2fp8/run_attn_bench_q2_cudagraph.sh:8-9), and run_attn_bench_q2.py
without --SBS makes SBS = BS up to 4096.  Groups above 4 rows and blocks above 512 tokens take the
two-pass path of the kernels (block maxima first, then the decision over every row); the bar is
the one of the other parity tests: masks identical to the oracle's away from the threshold,
thresholds to fp32 rounding, outputs within max-abs 2e-2 / mean-abs 2e-3 under the GPU's mask.
"""
import numpy as np
import pytest
import torch

from helpers import (FP8_DT, TORCH_DT, assert_out_close, compare_masks, contig_case, f32, oracle_paged, paged_case,
                     to_gpu_contig, to_gpu_paged)
from ffa_mi355x import synth
from oracle import formats as OF
from oracle import q2fp8 as O

pytestmark = pytest.mark.gpu

# (BS, SBS) of the reference's sweep script, plus SBS = BS (None) for the block sizes above 512
SWEEP = [(bs, sbs) for bs in (64, 128, 256, 512, 1024, 2048, 4096) for sbs in (64, 128, 256, 512) if sbs <= bs]
SWEEP += [(1024, None), (2048, None), (4096, None)]


def _contig_run(gpu, case, BS, SBS, delta, tau, res, what):
    import attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8 as K

    g = to_gpu_contig(case, gpu)
    SBSv = BS if SBS is None else SBS
    ws = K.allocate_q2fp8_decode_workspace(g["q"], g["k_q"], g["v"], BS=BS, SBS=SBS)
    o, sr = K.attn_forward_decode_quantized(g["q"], g["k_q"], g["k_scale"], g["k_zero"], g["v"],
                                            k_residual=g["k_residual"], BS=BS, SBS=SBS, delta=delta,
                                            return_skip_ratio=True, workspace=ws)
    torch.cuda.synchronize()
    q, v = f32(case["q"]), f32(case["v"])
    o_ref, diag = O.decode(q, case["k_q"], case["k_scale"], case["k_zero"], v, case["k_res"], res_fmt=res, BS=BS,
                           SBS=SBSv, delta=delta, out_dtype=tau)
    mask = ws.mask_buf.cpu().numpy()
    far, near, n_near = compare_masks(mask, diag)
    print(f"[mask] {what} skip={sr:.3f} oracle_skip={diag['skip_ratio']:.3f} far={far} near={near}/{n_near}")
    assert far == 0, f"{what}: {far} mask mismatches away from the threshold"
    assert mask.shape[-1] == diag["mask"].shape[-1]
    assert abs(sr - (1 - mask.sum() / mask.size)) < 1e-6
    assert np.abs(ws.threshold_buf.cpu().numpy() - diag["threshold"]).max() < 1e-4, f"{what}: threshold"
    o_forced, _ = O.decode(q, case["k_q"], case["k_scale"], case["k_zero"], v, case["k_res"], res_fmt=res, BS=BS,
                           SBS=SBSv, delta=delta, out_dtype=tau, force_mask=mask)
    mx, mean = assert_out_close(f32(o), o_forced, what)
    print(f"[out] {what} max_abs={mx:.3e} mean_abs={mean:.3e}")
    return mask


@pytest.mark.parametrize("T", [4096, 32768])
@pytest.mark.parametrize("BS,SBS", SWEEP)
def test_reference_sweep_grid(gpu, T, BS, SBS):
    """Every (BS, SBS) point of the reference's sweep in its own layout and defaults (fp16, e5m2)."""
    case = contig_case(B=1, T=T, HQ=32, HKV=8, tau="fp16", res="e5m2", seed=T + BS + (SBS or 0), n_heavy=16)
    _contig_run(gpu, case, BS, SBS, 5.0, "fp16", "e5m2", f"T={T} BS={BS} SBS={SBS}")


@pytest.mark.parametrize("HQ,HKV,T,BS,SBS,tau", [
    (40, 8, 1000, 128, 32, "bf16"),    # G = 5 (two units, the second with one row)
    (48, 8, 2048, 64, 64, "fp16"),     # G = 6
    (64, 8, 4096, 256, 128, "bf16"),   # G = 8 (Llama-3-70B's group)
    (32, 2, 1500, 1024, 1024, "fp16"),  # G = 16 with a block of two spans
    (24, 3, 777, 64, 16, "bf16"),      # G = 8, three KV heads, 16-token blocks
])
def test_contig_groups_above_four(gpu, HQ, HKV, T, BS, SBS, tau):
    case = contig_case(B=2, T=T, HQ=HQ, HKV=HKV, tau=tau, res="e5m2", seed=HQ * 3 + T, n_heavy=8)
    _contig_run(gpu, case, BS, SBS, 4.0, tau, "e5m2", f"contig G={HQ // HKV} T={T} BS={BS} SBS={SBS}")


@pytest.mark.parametrize("HQ,HKV,lens,BS,SBS", [
    (64, 8, [4096], 64, 64),                 # G = 8
    (48, 8, [2000, 700], 128, 32),           # G = 6, ragged
    (32, 2, [3000, 1, 0, 1500], 512, 256),   # G = 16, ragged with empty / one-token sequences
    (40, 8, [5000, 2100], 2048, 2048),       # G = 5, SBS = BS > 512
    (32, 8, [9000, 4500, 700], 4096, 4096),  # G = 4, SBS = BS = 4096 (two passes for the long blocks)
    (32, 8, [3000], 1024, 512),              # G = 4, one pass, SBS = 512 = one span
])
def test_paged_groups_and_long_blocks(gpu, HQ, HKV, lens, BS, SBS):
    T = max(lens)
    case = paged_case(B=len(lens), T=T, HQ=HQ, HKV=HKV, seed=HQ + T + BS, n_heavy=8, seq_lens=lens)
    cache = to_gpu_paged(case, gpu)
    sl = torch.tensor(lens, dtype=torch.int32, device=gpu)
    ws = cache.decode(case["q"].to(gpu), case["block_table"].to(gpu), sl, T=T, BS=BS, SBS=SBS, delta=4.0)
    torch.cuda.synchronize()
    what = f"paged G={HQ // HKV} lens={lens} BS={BS} SBS={SBS}"
    _, diag = oracle_paged(case, BS=BS, SBS=SBS, delta=4.0)
    mask = ws.mask_buf.cpu().numpy()
    far, near, n_near = compare_masks(mask, diag)
    print(f"[mask] {what} far={far} near={near}/{n_near} keep={mask.mean():.3f}")
    assert far == 0
    for b, t in enumerate(lens):
        if t == 0:
            assert mask[b].sum() == 0
        else:
            assert np.abs(ws.threshold_buf[b].cpu().numpy() - diag["threshold"][b]).max() < 1e-4
    o_forced, _ = oracle_paged(case, BS=BS, SBS=SBS, delta=4.0, force_mask=mask)
    mx, mean = assert_out_close(f32(ws.o), o_forced, what)
    print(f"[out] {what} max_abs={mx:.3e} mean_abs={mean:.3e}")


def test_two_pass_stage1_then_stage2_and_graph_runner(gpu):
    """Two-pass decodes through the stage entry points and the graph runner: stage 1 (both passes)
    then stage 2 equals the combined call, and graph replays equal eager calls."""
    import attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8 as K
    from attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8_cudagraph import CUDAGraphDecodeRunnerQ2FP8

    c = paged_case(B=2, T=2500, HQ=64, HKV=8, seed=41, n_heavy=8, seq_lens=[2500, 1300])
    cache = to_gpu_paged(c, gpu)
    q = c["q"].to(gpu)
    bt = c["block_table"].to(gpu)
    sl = torch.tensor(c["lens"], dtype=torch.int32, device=gpu)
    ws = cache.decode(q, bt, sl, T=2500, BS=1024, SBS=1024, delta=4.0)
    o_both, m_both = ws.o.clone(), ws.mask_buf.clone()
    cache.decode(q, bt, sl, T=2500, BS=1024, SBS=1024, delta=4.0, workspace=ws, stage="stage1")
    cache.decode(q, bt, sl, T=2500, BS=1024, SBS=1024, delta=4.0, workspace=ws, stage="stage2")
    torch.cuda.synchronize()
    assert torch.equal(o_both, ws.o) and torch.equal(m_both, ws.mask_buf)
    args = (q.unsqueeze(1).contiguous(), cache.k_q, cache.k_scale, cache.k_zero, cache.v)
    runner = CUDAGraphDecodeRunnerQ2FP8(*args, k_residual=cache.k_res, BS=1024, delta=4.0, block_table=bt,
                                        seq_lens=sl)
    for _ in range(3):
        got = runner(*args, k_residual=cache.k_res).clone()
        torch.cuda.synchronize()
        ref = K.attn_forward_decode_quantized(*args, k_residual=cache.k_res, BS=1024, delta=4.0, block_table=bt,
                                              seq_lens=sl)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
    o_ref, diag = oracle_paged(c, BS=1024, SBS=1024, delta=4.0, force_mask=m_both.cpu().numpy())
    assert_out_close(f32(o_both), o_ref, "two-pass G=8 SBS=1024")


def _kfmt_mod(rel, name):
    import importlib.util
    from pathlib import Path

    path = Path(__file__).resolve().parents[1] / "ffa-speedtest_amd" / rel
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("HQ,HKV,T,BS,SBS", [(64, 8, 2048, 128, 64), (48, 8, 1500, 2048, 2048), (32, 8, 3000, 1024, 1024)])
def test_fp8fp8_groups_and_long_blocks(gpu, HQ, HKV, T, BS, SBS):
    F8K = _kfmt_mod("ffa-fp8fp8/attn_kernel/attn_kernel_v1210_fused_bsz_fp8fp8.py", "dom_fp8fp8")
    q, k, v = synth.attention_inputs(B=2, T=T, HQ=HQ, HKV=HKV, seed=HQ + T, n_heavy=8, dtype=torch.bfloat16)
    base, res = OF.quantize_fp8fp8(f32(k), "e5m2")
    kh = OF.khat_fp8(base, "e5m2")
    kw = dict(res_fmt="e5m2", BS=BS, SBS=SBS, delta=4.0, khat=kh, out_dtype="bf16")
    _, diag = O.decode(f32(q), base, None, None, f32(v), res, **kw)
    ws = F8K.__dict__["DecodeWorkspace"](2, HQ, HKV, T, BS, SBS, gpu, torch.bfloat16)
    o = F8K.attn_forward_decode_fp8fp8(q.to(gpu).unsqueeze(1).contiguous(),
                                       torch.from_numpy(base).view(torch.float8_e5m2).to(gpu), v.to(gpu),
                                       k_residual=torch.from_numpy(res).view(torch.float8_e5m2).to(gpu), BS=BS, SBS=SBS,
                                       delta=4.0, workspace=ws)
    torch.cuda.synchronize()
    what = f"fp8fp8 G={HQ // HKV} BS={BS} SBS={SBS}"
    mask = ws.mask_buf.cpu().numpy()
    far, near, n_near = compare_masks(mask, diag)
    print(f"[mask] {what} far={far} near={near}/{n_near} keep={mask.mean():.3f}")
    assert far == 0
    assert np.abs(ws.threshold_buf.cpu().numpy() - diag["threshold"]).max() < 1e-4
    o_forced, _ = O.decode(f32(q), base, None, None, f32(v), res, force_mask=mask, **kw)
    mx, mean = assert_out_close(f32(o), o_forced, what)
    print(f"[out] {what} max_abs={mx:.3e} mean_abs={mean:.3e}")


@pytest.mark.parametrize("fmt", ["nvfp4", "nf4"])
@pytest.mark.parametrize("HQ,HKV,lens,BS,SBS", [(64, 8, [3000, 1200], 64, 32), (32, 4, [4500, 600], 2048, 1024)])
def test_paged_kfmt_groups_and_long_blocks(gpu, fmt, HQ, HKV, lens, BS, SBS):
    from test_gpu_kfmt_paged import _build  # each sequence appends its own tokens only

    T = max(lens)
    q, k, v, lens, bt, btd, cache = _build(fmt, len(lens), T, lens, seed=HQ + T, n_heavy=8, HQ=HQ, HKV=HKV)
    sl = torch.tensor(lens, dtype=torch.int32, device=gpu)
    ws = cache.decode(q.to(gpu), btd, sl, T=T, BS=BS, SBS=SBS, delta=4.0)
    torch.cuda.synchronize()
    kf = f32(k)
    if fmt == "nvfp4":
        codes, sc, res = OF.quantize_nvfp4_g16(kf, "e4m3fn")
        kh = OF.khat_nvfp4_g16(codes, sc)
    else:
        codes, sc, res = OF.quantize_nf4_g64(kf, "e4m3fn")
        kh = OF.khat_nf4_g64(codes, sc)
    kw = dict(res_fmt="e4m3fn", BS=BS, SBS=SBS, delta=4.0, khat=kh, out_dtype="bf16", seq_lens=lens)
    _, diag = O.decode(f32(q), codes, None, None, f32(v), res, **kw)
    mask = ws.mask_buf.cpu().numpy()
    far, near, n_near = compare_masks(mask, diag)
    what = f"paged {fmt} G={HQ // HKV} BS={BS} SBS={SBS}"
    print(f"[mask] {what} far={far} near={near}/{n_near}")
    assert far == 0
    assert np.abs(ws.threshold_buf.cpu().numpy() - diag["threshold"]).max() < 1e-4
    o_forced, _ = O.decode(f32(q), codes, None, None, f32(v), res, force_mask=mask, **kw)
    mx, mean = assert_out_close(f32(ws.o), o_forced, what)
    print(f"[out] {what} max_abs={mx:.3e} mean_abs={mean:.3e}")
