"""Per-channel q2 decode with fp32 and bf16 scale / zero: the reference dequantizes with the scale
and zero in fp32, k_hat = fp16(fp32(fp32(c * s) + z)) (attn_kernel_v1210_fused_bsz_q2fp8.py:50-53,
93), so a kernel that narrows them to fp16 first gets other k_hat values.  Each case also checks,
on the CPU, that it tells the two apart: the oracle given fp16-narrowed scales (the planted
mistake) misses the true thresholds by more than the bar.

Cases: fp32 K quantized by the reference quantizer (fp32 scale / zero); bf16 K whose first 64
channels span less than 2^-17 per step (bf16 scales that fp16 holds only as subnormals, with
fewer bits), with q large on those channels so the dequantization shows in the scores; and the
fused producer's fp32 output (fp32 cos / sin, Q2F:15) fed straight to the decoder."""
import numpy as np
import pytest
import torch

from helpers import FP8_DT, assert_out_close, compare_masks, f32
from ffa_mi355x import synth
from oracle import q2fp8 as O

pytestmark = pytest.mark.gpu

TH_TOL = 1e-4  # thresholds: fp32 rounding of the same fp16 dot products


def _case(kind, T, seed):
    if kind == "fp32":
        q, k, v = synth.attention_inputs(B=2, T=T, HQ=32, HKV=8, seed=seed, n_heavy=16, dtype=torch.float32)
        tau = "fp32"
    else:  # bf16 with tiny channels
        q, k, v = synth.attention_inputs(B=2, T=T, HQ=32, HKV=8, seed=seed, n_heavy=16, dtype=torch.float32)
        k[..., :64] *= 2e-6
        q[..., :64] *= 3e3
        tau = "bf16"
        q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    pk, s, z, r = O.quantize_per_channel(f32(k), tau, "e5m2")
    if kind != "fp32":
        assert (np.abs(s[..., :64]) < 2.0 ** -17).all()  # below fp16's exact range for bf16 values
    return q.bfloat16(), v.bfloat16(), pk, s, z, r, tau


def _oracle(q, v, pk, s, z, r, **kw):
    return O.decode(f32(q), pk, s, z, f32(v), r, res_fmt="e5m2", scale_mode="per_channel", out_dtype="bf16", **kw)


@pytest.mark.parametrize("kind", ["fp32", "bf16_tiny"])
@pytest.mark.parametrize("layout", ["contig", "paged"])
def test_channel_scales_dequantized_in_fp32(gpu, kind, layout):
    import attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8 as K

    T = 2048
    q, v, pk, s, z, r, tau = _case(kind, T, seed=31 if kind == "fp32" else 37)
    dt = torch.float32 if tau == "fp32" else torch.bfloat16
    B, HKV = pk.shape[0], pk.shape[2]
    kw = {}
    if layout == "contig":
        k_q = torch.from_numpy(pk).to(gpu)
        k_res = torch.from_numpy(r).view(FP8_DT["e5m2"]).to(gpu)
        vg = v.to(gpu)
    else:
        from ffa_mi355x.paged import CODES_ORDER, RES_ORDER, VT_ORDER, to_tiled

        lens = [T] * B
        bt, P = synth.page_tables(lens, seed=5, interleave=True)
        kq_pool = np.zeros((P, HKV, 4, 64, 8), np.uint8)
        r_pool = np.zeros((P, HKV, 64, 128), np.uint8)
        v_pool = np.zeros((P, HKV, 128, 64), np.uint16)
        vb = v.view(torch.int16).numpy().view(np.uint16)
        for b in range(B):
            for t0 in range(0, T, 64):
                page = int(bt[b, t0 // 64])
                kq_pool[page] = pk[b, t0:t0 + 64].reshape(64, HKV, 4, 8).transpose(1, 2, 0, 3)
                r_pool[page] = r[b, t0:t0 + 64].transpose(1, 0, 2)
                v_pool[page] = vb[b, t0:t0 + 64].transpose(1, 2, 0)
        k_q = torch.from_numpy(to_tiled(kq_pool, CODES_ORDER, 8)).to(gpu)
        k_res = torch.from_numpy(to_tiled(r_pool, RES_ORDER)).view(FP8_DT["e5m2"]).to(gpu)
        vg = torch.from_numpy(to_tiled(v_pool, VT_ORDER).view(np.int16)).view(torch.bfloat16).to(gpu)
        kw = dict(block_table=bt.to(gpu), T=T)
    qg = q.to(gpu).unsqueeze(1).contiguous()
    sg = torch.from_numpy(s).to(dt).to(gpu)
    zg = torch.from_numpy(z).to(dt).to(gpu)
    assert sg.dtype == dt and torch.equal(sg.float().cpu(), torch.from_numpy(s))  # the scales as quantized
    ws = K.allocate_q2fp8_decode_workspace(qg, k_q, vg, BS=64, SBS=64, **kw)
    o = K.attn_forward_decode_quantized(qg, k_q, sg, zg, vg, k_residual=k_res, BS=64, SBS=64, delta=5.0,
                                        workspace=ws, **kw)
    torch.cuda.synchronize()
    _, diag = _oracle(q, v, pk, s, z, r, BS=64, SBS=64, delta=5.0)
    # the planted mistake (scale / zero narrowed to fp16 before the dequantization), on the CPU
    s16, z16 = s.astype(np.float16).astype(np.float32), z.astype(np.float16).astype(np.float32)
    _, diag16 = _oracle(q, v, pk, s16, z16, r, BS=64, SBS=64, delta=5.0)
    miss16 = np.abs(diag16["threshold"] - diag["threshold"]).max()
    th_gpu = ws.threshold_buf.cpu().numpy()
    err = np.abs(th_gpu - diag["threshold"]).max()
    mask = ws.mask_buf.cpu().numpy()
    far, near, near_total = compare_masks(mask, diag)
    print(f"[{layout} {kind}] threshold err {err:.2e} (fp16-narrowed oracle: {miss16:.2e}) "
          f"mismatch_far={far} mismatch_near={near} near_blocks={near_total} keep={diag['mask'].mean():.3f}")
    assert miss16 > TH_TOL, "the case does not tell fp32 from fp16-narrowed dequantization"
    assert err < TH_TOL
    assert far == 0
    o_forced, _ = _oracle(q, v, pk, s, z, r, BS=64, SBS=64, delta=5.0, force_mask=mask)
    mx, mean = assert_out_close(f32(o), o_forced, f"{layout} {kind}")
    print(f"[out] max_abs={mx:.3e} mean_abs={mean:.3e}")


def test_producer_fp32_output_feeds_decode(gpu):
    """ffa_kproj_rope_q2_channel with fp32 cos / sin (the producer's default cache dtype) emits fp32
    scale / zero; the decode of that cache matches the oracle on the producer's own bytes."""
    from ffa_mi355x import quant

    B, T, H, HKV, D, HQ = 1, 1536, 512, 8, 128, 32
    g = torch.Generator().manual_seed(11)
    h = torch.randn(B, T, H, generator=g).bfloat16()
    w = (torch.randn(HKV * D, H, generator=g) * 0.05).bfloat16()
    inv = 1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    ang = torch.outer(torch.arange(T, dtype=torch.float32), inv)
    emb = torch.cat([ang, ang], -1)
    cos, sin = emb.cos(), emb.sin()  # fp32
    kq, s, z, r = quant.kproj_rope_q2_channel(h.to(gpu), w.to(gpu), cos.to(gpu), sin.to(gpu), HKV, D,
                                              fp8_dtype=torch.float8_e5m2)
    assert s.dtype == torch.float32 and z.dtype == torch.float32
    q = torch.randn(B, 1, HQ, D, generator=g).bfloat16()
    v = torch.randn(B, T, HKV, D, generator=g).bfloat16()
    import attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8 as K

    qg, vg = q.to(gpu), v.to(gpu)
    ws = K.allocate_q2fp8_decode_workspace(qg, kq, vg, BS=64, SBS=64)
    o = K.attn_forward_decode_quantized(qg, kq, s, z, vg, k_residual=r, BS=64, SBS=64, delta=1.0, workspace=ws)
    torch.cuda.synchronize()
    pk, sn, zn = kq.cpu().numpy(), f32(s), f32(z)
    rn = r.view(torch.uint8).cpu().numpy()
    args = (f32(q[:, 0]), pk, sn, zn, f32(v), rn)
    okw = dict(res_fmt="e5m2", scale_mode="per_channel", BS=64, SBS=64, delta=1.0, out_dtype="bf16")
    _, diag = O.decode(*args, **okw)
    mask = ws.mask_buf.cpu().numpy()
    far, near, near_total = compare_masks(mask, diag)
    err = np.abs(ws.threshold_buf.cpu().numpy() - diag["threshold"]).max()
    print(f"[producer fp32] threshold err {err:.2e} mismatch_far={far} mismatch_near={near} "
          f"near_blocks={near_total} keep={diag['mask'].mean():.3f}")
    assert err < TH_TOL and far == 0
    o_forced, _ = O.decode(*args, force_mask=mask, **okw)
    mx, mean = assert_out_close(f32(o), o_forced, "producer fp32")
    print(f"[out] max_abs={mx:.3e} mean_abs={mean:.3e}")


@pytest.mark.parametrize("layout", ["contig"])
def test_exact_bf16_scales_take_the_fp16_dequantization(gpu, layout):
    """bf16 scale / zero within fp16's range (the usual case: bf16 K quantized per channel) are
    exactly fp16 values, for which the packed fp16 dequantization gives the reference's k_hat.
    decode_args marks them (scale_exact_f16 = 1); that decode must agree with the oracle and with
    the same call forced onto the fp32 arithmetic (flag cleared)."""
    import ctypes

    from ffa_mi355x import _native as N
    from ffa_mi355x.decode import DecodeWorkspace, decode_args, scales_exact_f16

    T = 2048
    q, k, v = synth.attention_inputs(B=2, T=T, HQ=32, HKV=8, seed=41, n_heavy=16)  # bf16
    pk, s, z, r = O.quantize_per_channel(f32(k), "bf16", "e5m2")
    qg = q.to(gpu)
    sg = torch.from_numpy(s).to(torch.bfloat16).to(gpu)
    zg = torch.from_numpy(z).to(torch.bfloat16).to(gpu)
    assert scales_exact_f16(sg, zg)
    k_q = torch.from_numpy(pk).to(gpu)
    k_res = torch.from_numpy(r).view(FP8_DT["e5m2"]).to(gpu)
    vg = v.to(gpu)
    B, HQ = q.shape[0], q.shape[1]
    outs = []
    for flag in (1, 0):
        ws = DecodeWorkspace(B, HQ, 8, T, 64, 64, gpu, torch.bfloat16)
        a, ws = decode_args(q=qg, k_q=k_q, k_scale=sg, k_zero=zg, v=vg, k_residual=k_res, layout=N.LAYOUT_CONTIG,
                            scale_mode=N.SCALE_CHANNEL, T=T, HKV=8, scale=1.0 / np.sqrt(128), BS=64, SBS=64,
                            delta=5.0, use_res=True, workspace=ws)
        assert a.scale_exact_f16 == 1
        a.scale_exact_f16 = flag
        N.check(N.lib().ffa_q2fp8_decode(ctypes.byref(a), ctypes.c_void_p(N.stream_of(gpu))), "ffa_q2fp8_decode")
        torch.cuda.synchronize()
        outs.append((f32(ws.o), ws.threshold_buf.cpu().numpy(), ws.mask_buf.cpu().numpy()))
    (o16, th16, m16), (o32, th32, m32) = outs
    _, diag = _oracle(q, v, pk, s, z, r, BS=64, SBS=64, delta=5.0)
    err = np.abs(th16 - diag["threshold"]).max()
    far, near, near_total = compare_masks(m16, diag)
    print(f"[{layout} bf16 exact] threshold err {err:.2e} mismatch_far={far} near={near}/{near_total}; "
          f"fp16 vs fp32 path: threshold {np.abs(th16 - th32).max():.2e} out {np.abs(o16 - o32).max():.2e}")
    assert err < TH_TOL and far == 0
    assert np.array_equal(m16, m32)
    assert np.abs(th16 - th32).max() <= 1e-6 and np.abs(o16 - o32).max() <= 1e-6
    o_forced, _ = _oracle(q, v, pk, s, z, r, BS=64, SBS=64, delta=5.0, force_mask=m16)
    assert_out_close(o16, o_forced, f"{layout} bf16 exact")
