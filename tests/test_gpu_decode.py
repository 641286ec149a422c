"""GPU parity of the q2fp8 pruned decode (HIP kernels through the C ABI) against the CPU oracle.

Bar: survivor mask identical except blocks whose
margin max_g(block_max - th) is within 1e-3 (their count is printed);
attention output within max-abs 2e-2 and mean-abs 2e-3 in bf16.  The output
is compared with the oracle evaluated under the GPU's own mask, so that a
near-threshold flip is not mistaken for an arithmetic error.
"""
import math

import numpy as np
import pytest
import torch

from helpers import (FP8_DT, TORCH_DT, assert_out_close, compare_masks, contig_case, f32, oracle_paged, paged_case,
                     paged_channel_case, to_gpu_contig, to_gpu_paged)
from oracle import q2fp8 as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize(
    "tau,res,T,BS,SBS,delta,heavy",
    [
        ("fp16", "e5m2", 1000, 128, None, 5.0, 0),   # reference defaults (BS=128, SBS=BS, e5m2)
        ("bf16", "e5m2", 4096, 64, 64, 5.0, 16),
        ("bf16", "e4m3fn", 4096, 64, 32, 3.0, 16),
        ("fp16", "e5m2", 777, 64, 16, 2.0, 4),
        ("bf16", "e5m2", 2048, 256, 128, 4.0, 8),
        ("bf16", "e5m2", 1300, 256, 256, 4.0, 8),
    ],
)
def test_contig_reference_layout(gpu, tau, res, T, BS, SBS, delta, heavy):
    import attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8 as K

    case = contig_case(B=2, T=T, HQ=32, HKV=8, tau=tau, res=res, seed=T, n_heavy=heavy)
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
    far, near, near_total = compare_masks(mask, diag)
    print(f"[mask] T={T} BS={BS} SBS={SBSv} skip={sr:.3f} oracle_skip={diag['skip_ratio']:.3f} "
          f"mismatch_far={far} mismatch_near={near} near_blocks={near_total}")
    assert far == 0
    assert abs(sr - (1 - mask[..., : diag['mask'].shape[-1]].sum() / diag['mask'].size)) < 1e-6
    # the GPU dequantizes K to fp16 exactly as the reference does: thresholds agree to fp32 rounding
    th_gpu = ws.threshold_buf.cpu().numpy()
    assert np.abs(th_gpu - diag["threshold"]).max() < 1e-4
    o_forced, _ = O.decode(q, case["k_q"], case["k_scale"], case["k_zero"], v, case["k_res"], res_fmt=res, BS=BS,
                           SBS=SBSv, delta=delta, out_dtype=tau, force_mask=mask)
    mx, mean = assert_out_close(f32(o), o_forced, "contig")
    print(f"[out] max_abs={mx:.3e} mean_abs={mean:.3e}")


@pytest.mark.parametrize(
    "B,T,seq_lens,BS,SBS,delta,interleave",
    [
        (1, 4096, None, 64, 64, 5.0, True),
        (2, 3000, [3000, 1111], 64, 64, 5.0, True),
        (3, 2500, [2500, 640, 65], 128, 32, 4.0, True),
        (1, 1024, None, 64, 16, 5.0, False),
    ],
)
def test_paged_g32(gpu, B, T, seq_lens, BS, SBS, delta, interleave):
    case = paged_case(B=B, T=T, HQ=32, HKV=8, seed=B * 7 + T, n_heavy=16, seq_lens=seq_lens, interleave=interleave)
    cache = to_gpu_paged(case, gpu)
    q = case["q"].to(gpu)
    bt = case["block_table"].to(gpu)
    sl = torch.tensor(case["lens"], dtype=torch.int32, device=gpu)
    ws = cache.decode(q, bt, sl, T=T, BS=BS, SBS=SBS, delta=delta)
    torch.cuda.synchronize()
    o_ref, diag = oracle_paged(case, BS=BS, SBS=SBS, delta=delta)
    assert np.abs(ws.threshold_buf.cpu().numpy() - diag["threshold"]).max() < 1e-4
    mask = ws.mask_buf.cpu().numpy()
    far, near, near_total = compare_masks(mask, diag)
    kept = mask.sum() / sum(-(-t // SBS) for t in case["lens"]) / 8
    print(f"[mask] B={B} T={T} keep={kept:.3f} oracle_skip={diag['skip_ratio']:.3f} mismatch_far={far} "
          f"mismatch_near={near} near_blocks={near_total}")
    assert far == 0
    o_forced, _ = oracle_paged(case, BS=BS, SBS=SBS, delta=delta, force_mask=mask)
    mx, mean = assert_out_close(f32(ws.o), o_forced, "paged")
    print(f"[out] max_abs={mx:.3e} mean_abs={mean:.3e}")


@pytest.mark.parametrize("tau,res,seq_lens", [("bf16", "e5m2", None), ("fp16", "e4m3fn", [2048, 777])])
def test_paged_per_channel(gpu, tau, res, seq_lens):
    """Paged pools with the reference's per-channel scale / zero ([B, HKV, 128]) through the drop-in:
    the per-channel dequantization and refine on codes gathered through the page table."""
    import attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8 as K

    case = paged_channel_case(B=2, T=2048, tau=tau, res=res, seed=23, n_heavy=16, seq_lens=seq_lens)
    p = case["pools"]
    dt = TORCH_DT[tau]
    k_q = torch.from_numpy(p["k_q"]).to(gpu)
    k_res = torch.from_numpy(p["k_res"]).view(FP8_DT[res]).to(gpu)
    v = torch.from_numpy(p["v"].view(np.int16)).view(dt).to(gpu)  # V^T pages in the cache's dtype
    s = torch.from_numpy(case["k_scale"]).to(dt).to(gpu)
    z = torch.from_numpy(case["k_zero"]).to(dt).to(gpu)
    kw = dict(block_table=torch.as_tensor(case["block_table"]).to(gpu), T=2048)
    if seq_lens is not None:
        kw["seq_lens"] = torch.tensor(case["lens"], dtype=torch.int32, device=gpu)
    q = case["q"].to(gpu).unsqueeze(1).contiguous()
    ws = K.allocate_q2fp8_decode_workspace(q, k_q, v, BS=64, SBS=64, **kw)
    o, sr = K.attn_forward_decode_quantized(q, k_q, s, z, v, k_residual=k_res, BS=64, SBS=64, delta=5.0,
                                            return_skip_ratio=True, workspace=ws, **kw)
    torch.cuda.synchronize()
    args = (f32(case["q"]), case["k_q"], case["k_scale"], case["k_zero"], f32(case["v"]), case["k_res"])
    okw = dict(res_fmt=res, scale_mode="per_channel", seq_lens=seq_lens, BS=64, SBS=64, delta=5.0, out_dtype=tau)
    _, diag = O.decode(*args, **okw)
    mask = ws.mask_buf.cpu().numpy()
    far, near, near_total = compare_masks(mask, diag)
    print(f"[paged per-channel] tau={tau} res={res} skip={sr:.3f} oracle_skip={diag['skip_ratio']:.3f} "
          f"mismatch_far={far} mismatch_near={near} near_blocks={near_total}")
    assert far == 0
    assert np.abs(ws.threshold_buf.cpu().numpy() - diag["threshold"]).max() < 1e-4
    o_forced, _ = O.decode(*args, force_mask=mask, **okw)
    assert_out_close(f32(o), o_forced, "paged per-channel")


def test_paged_page_permutation_invariance(gpu):
    """Identity and permuted page tables over the same logical cache give bit-identical outputs."""
    c1 = paged_case(B=1, T=2048, HQ=32, HKV=8, seed=5, n_heavy=16, interleave=False)
    c2 = paged_case(B=1, T=2048, HQ=32, HKV=8, seed=5, n_heavy=16, interleave=True)
    assert not np.array_equal(c1["block_table"].numpy(), c2["block_table"].numpy())
    outs = []
    for c in (c1, c2):
        cache = to_gpu_paged(c, gpu)
        ws = cache.decode(c["q"].to(gpu), c["block_table"].to(gpu), T=2048, BS=64, delta=5.0)
        torch.cuda.synchronize()
        outs.append((ws.o.clone(), ws.mask_buf.clone()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


def test_precomputed_threshold_and_no_residual(gpu):
    case = paged_case(B=1, T=2048, HQ=32, HKV=8, seed=13, n_heavy=16)
    cache = to_gpu_paged(case, gpu)
    q, bt = case["q"].to(gpu), case["block_table"].to(gpu)
    ws = cache.decode(q, bt, T=2048, BS=64, delta=5.0)
    th = ws.threshold_buf.clone()
    o1, m1 = ws.o.clone(), ws.mask_buf.clone()
    ws2 = cache.decode(q, bt, T=2048, BS=64, delta=99.0, precomputed_threshold=th)
    torch.cuda.synchronize()
    assert torch.equal(m1, ws2.mask_buf) and torch.equal(o1, ws2.o)
    ws3 = cache.decode(q, bt, T=2048, BS=64, delta=5.0, use_fp8_residual=False)
    torch.cuda.synchronize()
    o_ref, diag = oracle_paged(case, BS=64, delta=5.0, use_fp8_residual=False,
                               force_mask=ws3.mask_buf.cpu().numpy())
    assert_out_close(f32(ws3.o), o_ref, "no-residual")


def test_extreme_deltas(gpu):
    case = paged_case(B=1, T=1500, HQ=32, HKV=8, seed=21, n_heavy=4)
    cache = to_gpu_paged(case, gpu)
    q, bt = case["q"].to(gpu), case["block_table"].to(gpu)
    ws = cache.decode(q, bt, T=1500, BS=64, delta=-math.inf)
    torch.cuda.synchronize()
    assert ws.mask_buf.sum().item() == 0 and (ws.o == 0).all()
    ws = cache.decode(q, bt, T=1500, BS=64, delta=math.inf)
    torch.cuda.synchronize()
    assert ws.mask_buf.sum().item() == ws.mask_buf.numel()
    o_ref, _ = oracle_paged(case, BS=64, delta=math.inf)
    assert_out_close(f32(ws.o), o_ref, "delta=inf")


def test_stage1_then_stage2_equals_both(gpu):
    """The two entry points ffa_q2fp8_decode_stage1 / _stage2 in sequence give the combined call's results."""
    c = paged_case(B=2, T=1500, HQ=32, HKV=8, seed=11, n_heavy=16, seq_lens=[1500, 900])
    cache = to_gpu_paged(c, gpu)
    q, bt = c["q"].to(gpu), c["block_table"].to(gpu)
    lens = torch.tensor(c["lens"], dtype=torch.int32, device=gpu)
    ws = cache.decode(q, bt, lens, BS=64, delta=5.0)
    torch.cuda.synchronize()
    ref = (ws.o.clone(), ws.mask_buf.clone(), ws.threshold_buf.clone())
    ws.o.zero_()
    ws.mask_buf.fill_(-1)
    cache.decode(q, bt, lens, BS=64, delta=5.0, workspace=ws, stage="stage1")
    cache.decode(q, bt, lens, BS=64, delta=5.0, workspace=ws, stage="stage2")
    torch.cuda.synchronize()
    assert torch.equal(ws.o, ref[0]) and torch.equal(ws.mask_buf, ref[1]) and torch.equal(ws.threshold_buf, ref[2])


def test_cudagraph_runner_replays_match_eager(gpu):
    """CUDAGraphDecodeRunnerQ2FP8: every replay (new inputs, eager work in between) equals an eager call."""
    import attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8 as K
    from attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8_cudagraph import CUDAGraphDecodeRunnerQ2FP8

    cases = [to_gpu_contig(contig_case(B=2, T=1024, tau="bf16", res="e5m2", seed=s, n_heavy=8), gpu) for s in (0, 1, 2)]
    c0 = cases[0]
    runner = CUDAGraphDecodeRunnerQ2FP8(c0["q"], c0["k_q"], c0["k_scale"], c0["k_zero"], c0["v"],
                                        k_residual=c0["k_residual"], BS=64, delta=5.0)
    for rep in range(2):
        for c in cases:
            got = runner(c["q"], c["k_q"], c["k_scale"], c["k_zero"], c["v"], k_residual=c["k_residual"]).clone()
            torch.cuda.synchronize()
            _ = torch.randn(4096, device=gpu).sum()  # unrelated eager work between replays
            ref, sr = K.attn_forward_decode_quantized(c["q"], c["k_q"], c["k_scale"], c["k_zero"], c["v"],
                                                      k_residual=c["k_residual"], BS=64, delta=5.0,
                                                      return_skip_ratio=True)
            torch.cuda.synchronize()
            assert torch.equal(got, ref), f"replay {rep} differs from eager"
    c = cases[1]
    out, sr_g = runner(c["q"], c["k_q"], c["k_scale"], c["k_zero"], c["v"], k_residual=c["k_residual"],
                       return_skip_ratio=True)
    _, sr_e = K.attn_forward_decode_quantized(c["q"], c["k_q"], c["k_scale"], c["k_zero"], c["v"],
                                              k_residual=c["k_residual"], BS=64, delta=5.0, return_skip_ratio=True)
    assert sr_g == sr_e
    assert torch.equal(runner.replay_only(), out)


def test_cudagraph_runner_paged(gpu):
    """The runner over a paged g32 cache with a page table and ragged lengths (passed through **kwargs)."""
    import attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8 as K
    from attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8_cudagraph import CUDAGraphDecodeRunnerQ2FP8

    c = paged_case(B=2, T=1500, HQ=32, HKV=8, seed=21, n_heavy=16, seq_lens=[1500, 700])
    cache = to_gpu_paged(c, gpu)
    q = c["q"].to(gpu).unsqueeze(1).contiguous()
    bt = c["block_table"].to(gpu)
    lens = torch.tensor(c["lens"], dtype=torch.int32, device=gpu)
    args = (q, cache.k_q, cache.k_scale, cache.k_zero, cache.v)
    runner = CUDAGraphDecodeRunnerQ2FP8(*args, k_residual=cache.k_res, BS=64, delta=5.0, block_table=bt,
                                        seq_lens=lens)
    for _ in range(3):
        got = runner(*args, k_residual=cache.k_res).clone()
        torch.cuda.synchronize()
        ref = K.attn_forward_decode_quantized(*args, k_residual=cache.k_res, BS=64, delta=5.0, block_table=bt,
                                              seq_lens=lens)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
    o_ref, _ = oracle_paged(c, BS=64, SBS=64, delta=5.0)
    assert_out_close(f32(got), o_ref, "paged runner")


def test_cudagraph_runner_paged_growing_lengths(gpu):
    """Capture with short lengths, then replay as a decode loop does, with seq_lens growing past
    the capture-time maximum: every replay equals an eager call and the oracle at those lengths
    (the captured grid covers the block table's capacity)."""
    import attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8 as K
    from attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8_cudagraph import CUDAGraphDecodeRunnerQ2FP8

    c = paged_case(B=2, T=1500, HQ=32, HKV=8, seed=23, n_heavy=16)  # both sequences hold 1500 tokens
    cache = to_gpu_paged(c, gpu)
    q = c["q"].to(gpu).unsqueeze(1).contiguous()
    bt = c["block_table"].to(gpu)
    args = (q, cache.k_q, cache.k_scale, cache.k_zero, cache.v)
    lens0 = torch.tensor([700, 300], dtype=torch.int32, device=gpu)
    runner = CUDAGraphDecodeRunnerQ2FP8(*args, k_residual=cache.k_res, BS=64, delta=5.0, block_table=bt,
                                        seq_lens=lens0)
    for lens in ([700, 300], [701, 301], [1100, 900], [1500, 1500]):
        lt = torch.tensor(lens, dtype=torch.int32, device=gpu)
        got = runner(*args, k_residual=cache.k_res, seq_lens=lt).clone()
        torch.cuda.synchronize()
        ref = K.attn_forward_decode_quantized(*args, k_residual=cache.k_res, BS=64, delta=5.0, block_table=bt,
                                              seq_lens=lt)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"replay != eager at lengths {lens}"
        o_ref, _ = O.decode(f32(c["q"]), c["k_q"], c["k_scale"], c["k_zero"], f32(c["v"]), c["k_res"],
                            res_fmt=c["res"], scale_mode="g32", seq_lens=lens, out_dtype="bf16", BS=64, SBS=64,
                            delta=5.0)
        assert_out_close(f32(got), o_ref, f"growing lengths {lens}")


def test_workspace_allocated_ahead_matches_paged_call(gpu):
    """allocate_q2fp8_decode_workspace and the call agree on T for a paged cache (both default to the
    block table's capacity), so the H100-style allocate-then-call pattern works with seq_lens."""
    import attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8 as K

    c = paged_case(B=2, T=1000, HQ=32, HKV=8, seed=24, n_heavy=16, seq_lens=[1000, 450])
    cache = to_gpu_paged(c, gpu)
    q = c["q"].to(gpu).unsqueeze(1).contiguous()
    kw = dict(block_table=c["block_table"].to(gpu), seq_lens=torch.tensor(c["lens"], dtype=torch.int32, device=gpu))
    ws = K.allocate_q2fp8_decode_workspace(q, cache.k_q, cache.v, BS=64, **kw)
    o = K.attn_forward_decode_quantized(q, cache.k_q, cache.k_scale, cache.k_zero, cache.v, k_residual=cache.k_res,
                                        BS=64, delta=5.0, workspace=ws, **kw)
    o_ref, _ = oracle_paged(c, BS=64, SBS=64, delta=5.0)
    assert_out_close(f32(o), o_ref, "workspace allocated ahead")


def _pool_views(cache, P):
    """Replace the cache's pools by pages [1, P + 1) of allocations two pages larger, so that page
    ids -1 and P name real memory (allocation pages 0 and P + 1) outside the pools the library sees."""
    allocs = {}
    for name in ("k_q", "k_scale", "k_zero", "k_res", "v"):
        t = getattr(cache, name)
        big = torch.empty((P + 2,) + tuple(t.shape[1:]), dtype=t.dtype, device=t.device)
        big.view(torch.uint8).fill_(0x3C)  # finite in every dtype of the pools
        big[1:P + 1].copy_(t)
        allocs[name] = big
        setattr(cache, name, big[1:P + 1])
    return allocs


def test_page_ids_outside_the_pool(gpu):
    """Block-table entries outside [0, P): the decoder reads them as page 0 and the g32 append
    writes nothing for their tokens (no access outside the pools)."""
    from ffa_mi355x import _native as N

    case = paged_case(B=1, T=1024, HQ=32, HKV=8, seed=9, n_heavy=8)
    cache = to_gpu_paged(case, gpu)
    P = case["P"]
    allocs = _pool_views(cache, P)
    q = case["q"].to(gpu)
    bt = case["block_table"].to(gpu)
    bt_zero, bt_out = bt.clone(), bt.clone()
    bt_zero[0, 3] = 0
    bt_zero[0, 9] = 0
    bt_out[0, 3] = -1
    bt_out[0, 9] = P
    w0 = cache.decode(q, bt_zero, T=1024, BS=64, delta=5.0)
    o0, m0 = w0.o.clone(), w0.mask_buf.clone()
    w1 = cache.decode(q, bt_out, T=1024, BS=64, delta=5.0)
    torch.cuda.synchronize()
    assert torch.equal(o0, w1.o) and torch.equal(m0, w1.mask_buf)

    # append 128 tokens at positions 0..127 through pages bt_app = [P, 2]: page P is outside the pool
    before = {k: v.clone() for k, v in allocs.items()}
    k_new = torch.randn(1, 128, 8, 128, device=gpu, dtype=torch.bfloat16)
    bt_app = torch.tensor([[P, 2]], dtype=torch.int32, device=gpu)
    pos = torch.zeros(1, dtype=torch.int32, device=gpu)
    rc = N.lib().ffa_q2_quantize_g32_append(
        k_new.data_ptr(), N.DT_BF16, 1, 128, 8, pos.data_ptr(), bt_app.data_ptr(), 2, P, cache.k_q.data_ptr(),
        cache.k_scale.data_ptr(), cache.k_zero.data_ptr(), cache.k_res.data_ptr(), N.dtype_code(cache.res_dtype),
        None, cache.v.data_ptr(), N.stream_of(k_new.device))
    N.check(rc, "ffa_q2_quantize_g32_append")
    torch.cuda.synchronize()
    for name, big in allocs.items():
        b0 = before[name]
        changed = [i for i in range(P + 2) if not torch.equal(big[i].view(torch.uint8), b0[i].view(torch.uint8))]
        # only pool page 2 (allocation page 3) is written; the V pool is not (no v_new)
        assert changed == ([] if name == "v" else [3]), (name, changed)


# P.V operand pin: with fp32 output and prune blocks of one 64-token chunk (the kernel's softmax
# reference maximum is then the block maximum of the reference), the kernel's output agrees with
# the oracle's fp16 p / fp16 v to within PV_PIN_TOL, while the same oracle with bf16 p / bf16 v (the
# planted mistake) lies further away than that on the same inputs.
PV_PIN_TOL = 2e-4


@pytest.mark.parametrize("layout", ["paged", "contig"])
def test_pv_operands_are_fp16(gpu, layout):
    from ffa_mi355x import _native as N
    from ffa_mi355x.decode import run_decode

    T, BS, SBS, delta = 4096, 64, 64, 5.0
    if layout == "paged":
        case = paged_case(B=1, T=T, HQ=32, HKV=8, seed=11, n_heavy=16)
        cache = to_gpu_paged(case, gpu)
        bt = case["block_table"].to(gpu)
        ws = cache.decode(case["q"].float().to(gpu), bt, None, T=T, BS=BS, SBS=SBS, delta=delta)
        kw = dict(res_fmt=case["res"], scale_mode="g32")
    else:
        case = contig_case(B=1, T=T, HQ=32, HKV=8, tau="bf16", res="e5m2", seed=11, n_heavy=16)
        g = to_gpu_contig(case, gpu)
        ws = run_decode(q=g["q"][:, 0].float().contiguous(), k_q=g["k_q"], k_scale=g["k_scale"],
                        k_zero=g["k_zero"], v=g["v"], k_residual=g["k_residual"], layout=N.LAYOUT_CONTIG,
                        scale_mode=N.SCALE_CHANNEL, T=T, HKV=8, scale=1.0 / math.sqrt(128), BS=BS, SBS=SBS,
                        delta=delta, use_res=True)
        kw = dict(res_fmt=case["res"], scale_mode="per_channel")
    torch.cuda.synchronize()
    assert ws.o.dtype == torch.float32
    mask = ws.mask_buf.cpu().numpy()
    args = (f32(case["q"]), case["k_q"], case["k_scale"], case["k_zero"], f32(case["v"]), case["k_res"])
    o16, _ = O.decode(*args, BS=BS, SBS=SBS, delta=delta, out_dtype="fp32", force_mask=mask, **kw)
    ob, _ = O.decode(*args, BS=BS, SBS=SBS, delta=delta, out_dtype="fp32", force_mask=mask, pv_dtype="bf16", **kw)
    og = f32(ws.o)
    d16 = np.abs(og - o16).max()
    dbf = np.abs(og - ob).max()
    gap = np.abs(o16 - ob).max()
    print(f"[pv] {layout}: |gpu - oracle fp16 P| = {d16:.3e}, |gpu - oracle bf16 P| = {dbf:.3e}, "
          f"|oracle fp16 - bf16| = {gap:.3e}")
    assert gap > PV_PIN_TOL  # the tolerance tells the two operand precisions apart
    assert d16 <= PV_PIN_TOL
