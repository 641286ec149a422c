"""GPU parity at the edges of the supported shapes: GQA groups of 1 to 4 with other head counts
than 32/8, and ragged batches holding empty, one-token and shorter-than-a-probe-window sequences
(paged q2, paged nvfp4 / nf4, reference-layout q2 and fp8).  Same bar as the other parity tests;
thresholds are compared where a sequence has tokens (an empty one has no blocks to prune)."""
import numpy as np
import pytest
import torch

from helpers import (FP8_DT, TORCH_DT, assert_out_close, compare_masks, contig_case, f32, oracle_paged, paged_case,
                     to_gpu_contig, to_gpu_paged)
from ffa_mi355x import synth
from oracle import formats as OF
from oracle import q2fp8 as O

pytestmark = pytest.mark.gpu


def _check(o_gpu, ws, o_ref, diag, lens, what):
    torch.cuda.synchronize()
    mask = ws.mask_buf.cpu().numpy()
    far, near, n_near = compare_masks(mask, diag)
    print(f"[mask] {what} far={far} near={near}/{n_near}")
    assert far == 0, f"{what}: {far} mask mismatches away from the threshold"
    for b, t in enumerate(lens):
        if t == 0:
            assert mask[b].sum() == 0, f"{what}: an empty sequence kept blocks"
        else:
            assert np.abs(ws.threshold_buf[b].cpu().numpy() - diag["threshold"][b]).max() < 1e-4, f"{what}: th"
    o = f32(o_gpu)
    for b, t in enumerate(lens):
        if t == 0:
            assert (o[b] == 0).all(), f"{what}: an empty sequence's output is not 0"
    mx, mean = assert_out_close(o, o_ref, what)
    print(f"[out] {what} max_abs={mx:.3e} mean_abs={mean:.3e}")


@pytest.mark.parametrize("HQ,HKV,lens", [
    (16, 8, [1000, 0, 1, 15]),   # G = 2
    (6, 2, [17, 1000, 64, 65]),  # G = 3
    (8, 8, [1, 1000, 0, 129]),   # G = 1
    (8, 2, [15, 16, 1000, 999]),  # G = 4, two KV heads
])
def test_paged_q2_gqa_groups_and_short_sequences(gpu, HQ, HKV, lens):
    T = max(lens)
    case = paged_case(B=len(lens), T=T, HQ=HQ, HKV=HKV, seed=HQ + HKV, n_heavy=4, seq_lens=lens)
    cache = to_gpu_paged(case, gpu)
    sl = torch.tensor(lens, dtype=torch.int32, device=gpu)
    ws = cache.decode(case["q"].to(gpu), case["block_table"].to(gpu), sl, T=T, BS=64, SBS=32, delta=4.0)
    torch.cuda.synchronize()
    _, diag = oracle_paged(case, BS=64, SBS=32, delta=4.0)
    o_forced, _ = oracle_paged(case, BS=64, SBS=32, delta=4.0, force_mask=ws.mask_buf.cpu().numpy())
    _check(ws.o, ws, o_forced, diag, lens, f"paged q2 {HQ}/{HKV}")


@pytest.mark.parametrize("HQ,HKV,T", [(8, 8, 777), (16, 8, 1000), (12, 4, 300), (4, 1, 129)])
def test_contig_q2_gqa_groups(gpu, HQ, HKV, T):
    import attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8 as K

    case = contig_case(B=2, T=T, HQ=HQ, HKV=HKV, tau="bf16", res="e5m2", seed=T + HQ, n_heavy=4)
    g = to_gpu_contig(case, gpu)
    ws = K.allocate_q2fp8_decode_workspace(g["q"], g["k_q"], g["v"], BS=64, SBS=64)
    o = K.attn_forward_decode_quantized(g["q"], g["k_q"], g["k_scale"], g["k_zero"], g["v"],
                                        k_residual=g["k_residual"], BS=64, SBS=64, delta=5.0, workspace=ws)
    torch.cuda.synchronize()
    q, v = f32(case["q"]), f32(case["v"])
    _, diag = O.decode(q, case["k_q"], case["k_scale"], case["k_zero"], v, case["k_res"], res_fmt="e5m2", BS=64,
                       SBS=64, delta=5.0, out_dtype="bf16")
    o_forced, _ = O.decode(q, case["k_q"], case["k_scale"], case["k_zero"], v, case["k_res"], res_fmt="e5m2", BS=64,
                           SBS=64, delta=5.0, out_dtype="bf16", force_mask=ws.mask_buf.cpu().numpy())
    _check(o.reshape(2, HQ, 128), ws, o_forced, diag, [T, T], f"contig q2 {HQ}/{HKV}")


@pytest.mark.parametrize("fmt", ["nvfp4", "nf4"])
def test_paged_kfmt_gqa_group_3_and_short_sequences(gpu, fmt):
    from test_gpu_kfmt_paged import QUANT, _build, _khat

    lens = [2000, 0, 1, 15]
    q, k, v, lens, bt, btd, cache = _build(fmt, 4, 2000, lens, seed=77, n_heavy=4, HQ=6, HKV=2)
    ws = cache.decode(q.to(gpu), btd, torch.tensor(lens, dtype=torch.int32, device=gpu), T=2000, BS=64, SBS=64,
                      delta=5.0)
    torch.cuda.synchronize()
    pk, sc, res = QUANT[fmt](f32(k))
    kh = _khat(fmt, pk, sc)
    _, diag = O.decode(f32(q), pk, None, None, f32(v), res, res_fmt="e4m3fn", BS=64, SBS=64, delta=5.0, khat=kh,
                       seq_lens=lens, out_dtype="bf16")
    o_forced, _ = O.decode(f32(q), pk, None, None, f32(v), res, res_fmt="e4m3fn", BS=64, SBS=64, delta=5.0, khat=kh,
                           seq_lens=lens, out_dtype="bf16", force_mask=ws.mask_buf.cpu().numpy())
    _check(ws.o, ws, o_forced, diag, lens, f"paged {fmt} 6/2")


@pytest.mark.parametrize("HQ,HKV", [(8, 4), (3, 1)])
def test_contig_fp8fp8_gqa_groups(gpu, HQ, HKV):
    from test_gpu_kfmt import F8K

    T = 1000
    q, k, v = synth.attention_inputs(B=2, T=T, HQ=HQ, HKV=HKV, seed=HQ * 10 + HKV, n_heavy=4)
    base, res = OF.quantize_fp8fp8(f32(k), "e4m3fn")
    kh = OF.khat_fp8(base, "e4m3fn")
    ws = F8K.__dict__["DecodeWorkspace"](2, HQ, HKV, T, 64, 64, gpu, torch.bfloat16)
    o = F8K.attn_forward_decode_fp8fp8(
        q.to(gpu).unsqueeze(1).contiguous(), torch.from_numpy(base).view(FP8_DT["e4m3fn"]).to(gpu), v.to(gpu),
        k_residual=torch.from_numpy(res).view(FP8_DT["e4m3fn"]).to(gpu), BS=64, SBS=64, delta=5.0, workspace=ws)
    torch.cuda.synchronize()
    _, diag = O.decode(f32(q), base, None, None, f32(v), res, res_fmt="e4m3fn", BS=64, SBS=64, delta=5.0, khat=kh,
                       out_dtype="bf16")
    o_forced, _ = O.decode(f32(q), base, None, None, f32(v), res, res_fmt="e4m3fn", BS=64, SBS=64, delta=5.0,
                           khat=kh, out_dtype="bf16", force_mask=ws.mask_buf.cpu().numpy())
    _check(o.reshape(2, HQ, 128), ws, o_forced, diag, [T, T], f"contig fp8fp8 {HQ}/{HKV}")
