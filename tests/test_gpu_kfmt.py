"""GPU parity of the fp8 / nvfp4 / nf4 decoders (drop-in modules -> C ABI -> HIP) against the oracle."""
import importlib.util
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import FP8_DT, TORCH_DT, assert_out_close, compare_masks, f32
from ffa_mi355x import synth
from oracle import formats as OF
from oracle import numerics as NM
from oracle import q2fp8 as O

pytestmark = pytest.mark.gpu
PKG = Path(__file__).resolve().parents[1] / "ffa-speedtest_amd"


def _load(rel, name):
    spec = importlib.util.spec_from_file_location(name, PKG / rel)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


F8K = _load("ffa-fp8fp8/attn_kernel/attn_kernel_v1210_fused_bsz_fp8fp8.py", "kfmt_fp8fp8")
NVK = _load("ffa-nvfp4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nvfp4fp8.py", "kfmt_nvfp4fp8")
NFK = _load("ffa-nf4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nf4fp8.py", "kfmt_nf4fp8")


def _inputs(B, T, tau, seed, n_heavy, seq_lens=None):
    q, k, v = synth.attention_inputs(B=B, T=T, HQ=32, HKV=8, seed=seed, n_heavy=n_heavy, dtype=TORCH_DT[tau],
                                     seq_lens=seq_lens)
    return q, k, v


def _check(o_gpu, ws, o_ref, diag, what):
    torch.cuda.synchronize()
    far, near, n_near = compare_masks(ws.mask_buf.cpu().numpy(), diag)
    print(f"[mask] {what} keep={ws.mask_buf.float().mean().item():.3f} far={far} near={near}/{n_near}")
    assert far == 0, f"{what}: {far} mask mismatches away from the threshold"
    th = ws.threshold_buf.cpu().numpy()
    assert np.abs(th - diag["threshold"]).max() < 1e-4, f"{what}: threshold"
    mx, mean = assert_out_close(f32(o_gpu), o_ref, what)
    print(f"[out] {what} max_abs={mx:.3e} mean_abs={mean:.3e}")


@pytest.mark.parametrize("fmt,tau,vdt,T,BS,SBS,delta", [
    ("e5m2", "fp16", "fp16", 1000, 128, None, 5.0),
    ("e4m3fn", "bf16", "bf16", 4096, 64, 64, 5.0),
    ("e5m2", "bf16", "bf16", 2048, 64, 32, 3.0),
    ("e4m3fn", "fp16", "fp16", 777, 64, 16, 2.0),
])
def test_fp8fp8_decoder(gpu, fmt, tau, vdt, T, BS, SBS, delta):
    q, k, v = _inputs(1, T, tau, 1, 16)
    base, res = OF.quantize_fp8fp8(f32(k), fmt)
    kh = OF.khat_fp8(base, fmt)
    o_ref, diag = O.decode(f32(q), base, None, None, f32(v), res, res_fmt=fmt, BS=BS, SBS=SBS, delta=delta,
                           khat=kh, out_dtype=tau)
    ws = F8K.__dict__["DecodeWorkspace"](1, 32, 8, T, BS, SBS or BS, gpu, TORCH_DT[tau])
    o = F8K.attn_forward_decode_fp8fp8(
        q.to(gpu).unsqueeze(1).contiguous(), torch.from_numpy(base).view(FP8_DT[fmt]).to(gpu),
        v.to(TORCH_DT[vdt]).to(gpu), k_residual=torch.from_numpy(res).view(FP8_DT[fmt]).to(gpu), BS=BS, SBS=SBS,
        delta=delta, workspace=ws)
    _check(o, ws, o_ref, diag, f"fp8fp8 {fmt} T={T}")


def test_fp8fp8_decoder_f32_query(gpu):
    """q in float32 (the 64-byte q window per lane, all four loads used) on the other-format decoder."""
    T, BS, SBS, delta, fmt = 1500, 64, 64, 4.0, "e4m3fn"
    q, k, v = _inputs(1, T, "bf16", 1, 16)
    base, res = OF.quantize_fp8fp8(f32(k), fmt)
    kh = OF.khat_fp8(base, fmt)
    o_ref, diag = O.decode(f32(q), base, None, None, f32(v), res, res_fmt=fmt, BS=BS, SBS=SBS, delta=delta,
                           khat=kh, out_dtype="fp32")
    qd = q.float().to(gpu).unsqueeze(1).contiguous()
    ws = F8K.__dict__["DecodeWorkspace"](1, 32, 8, T, BS, SBS, gpu, torch.float32)
    o = F8K.attn_forward_decode_fp8fp8(
        qd, torch.from_numpy(base).view(FP8_DT[fmt]).to(gpu), v.to(gpu),
        k_residual=torch.from_numpy(res).view(FP8_DT[fmt]).to(gpu), BS=BS, SBS=SBS, delta=delta, workspace=ws)
    assert o.dtype == torch.float32
    _check(o, ws, o_ref, diag, f"fp8fp8 f32 q T={T}")


def test_fp8_scaled_decoder_baseline_config1(gpu):
    """Benchmark config 1: e4m3 + one fp16 scale per token and KV head + e4m3 residual, 4 outlier channels."""
    T = 4096
    q, k, v = _inputs(1, T, "bf16", 0, 0)
    kf = f32(k)
    kf[..., :4] *= 10.0
    base, s, res = OF.quantize_fp8_scaled(kf, "e4m3fn")
    kh = OF.khat_fp8_scaled(base, s, "e4m3fn")
    o_ref, diag = O.decode(f32(q), base, None, None, f32(v), res, res_fmt="e4m3fn", BS=64, SBS=64, delta=5.0,
                           khat=kh, out_dtype="bf16")
    ws = F8K.__dict__["DecodeWorkspace"](1, 32, 8, T, 64, 64, gpu, torch.bfloat16)
    o = F8K.attn_forward_decode_fp8fp8(
        q.to(gpu).unsqueeze(1).contiguous(), torch.from_numpy(base).view(torch.float8_e4m3fn).to(gpu), v.to(gpu),
        k_residual=torch.from_numpy(res).view(torch.float8_e4m3fn).to(gpu), BS=64, delta=5.0,
        k_scale=torch.from_numpy(s).to(torch.float16).to(gpu), workspace=ws)
    _check(o, ws, o_ref, diag, "fp8 scaled (config 1)")


def test_fp8_scaled_decoder_zero_and_tiny_rows(gpu):
    """A config-1 cache holding an all-zero K row and a row of amplitude 3.5e-5 (whose fp16
    scale would be subnormal without the floor): the HIP quantizer's bytes decode to finite
    outputs that match the oracle on the same bytes."""
    from ffa_mi355x import kfmt_quant as KQ

    T = 1024
    q, k, v = _inputs(1, T, "bf16", 4, 16)
    k[0, 17, 3] = 0.0
    row = torch.randn(128)
    k[0, 300, 5] = (row * (3.5e-5 / row.abs().max())).to(torch.bfloat16)
    k[0, 301, 0] = 0.0
    base, s, res = KQ.quantize_fp8_scaled(k.to(gpu), torch.float8_e4m3fn)
    torch.cuda.synchronize()
    bo, so, ro = OF.quantize_fp8_scaled(f32(k), "e4m3fn")
    assert np.array_equal(base.view(torch.uint8).cpu().numpy(), bo)
    assert np.array_equal(f32(s), so) and np.array_equal(res.view(torch.uint8).cpu().numpy(), ro)
    kh = OF.khat_fp8_scaled(bo, so, "e4m3fn")
    o_ref, diag = O.decode(f32(q), bo, None, None, f32(v), ro, res_fmt="e4m3fn", BS=64, SBS=64, delta=5.0,
                           khat=kh, out_dtype="bf16")
    assert np.isfinite(o_ref).all()
    ws = F8K.__dict__["DecodeWorkspace"](1, 32, 8, T, 64, 64, gpu, torch.bfloat16)
    o = F8K.attn_forward_decode_fp8fp8(q.to(gpu).unsqueeze(1).contiguous(), base, v.to(gpu), k_residual=res,
                                       BS=64, delta=5.0, k_scale=s, workspace=ws)
    assert torch.isfinite(o.float()).all()
    _check(o, ws, o_ref, diag, "fp8 scaled with zero / tiny rows")


@pytest.mark.parametrize("tau,T,BS,SBS,delta", [
    ("bf16", 2048, 64, 64, 5.0),
    ("fp16", 1100, 128, 64, 4.0),  # NTB = 9 != HKV: see test_nvfp4_scale_normalisation_quirk
    ("bf16", 3000, 128, 128, 5.0),
    ("fp32", 700, 64, 32, 3.0),
])
def test_nvfp4_decoder(gpu, tau, T, BS, SBS, delta):
    q, k, v = _inputs(1, T, "bf16" if tau == "fp32" else tau, 2, 16)
    kt = NM.round_to(f32(k), tau)
    pk, sc, res = OF.quantize_nvfp4(kt, tau, "e5m2", BS)
    kh, kp1 = OF.khat_nvfp4(pk, sc, BS, 128)
    o_ref, diag = O.decode(f32(q), pk, None, None, f32(v), res, res_fmt="e5m2", BS=BS, SBS=SBS, delta=delta,
                           khat=kh, khat_probe1=kp1, out_dtype="bf16" if tau == "fp32" else tau)
    qd = q.to(gpu).unsqueeze(1).contiguous()
    o, sr = NVK.attn_forward_decode_nvfp4fp8(
        qd, torch.from_numpy(pk).to(gpu), torch.from_numpy(sc).to(TORCH_DT[tau]).to(gpu), v.to(gpu),
        k_residual=torch.from_numpy(res).view(torch.float8_e5m2).to(gpu), BS=BS, SBS=SBS, delta=delta,
        return_skip_ratio=True)
    ws = NVK.__dict__["DecodeWorkspace"](1, 32, 8, T, BS, SBS, gpu, qd.dtype)
    o = NVK.attn_forward_decode_nvfp4fp8(
        qd, torch.from_numpy(pk).to(gpu), torch.from_numpy(sc).to(TORCH_DT[tau]).to(gpu), v.to(gpu),
        k_residual=torch.from_numpy(res).view(torch.float8_e5m2).to(gpu), BS=BS, SBS=SBS, delta=delta, workspace=ws)
    _check(o, ws, o_ref, diag, f"nvfp4 {tau} T={T} BS={BS}")
    assert abs(sr - (1.0 - ws.mask_buf.float().mean().item())) < 1e-6  # return_skip_ratio of the first call


@pytest.mark.parametrize("tau,T,BS,SBS,delta,res_fmt", [
    ("bf16", 2048, 64, 64, 5.0, "e4m3fn"),
    ("fp16", 1300, 128, 32, 4.0, "e5m2"),
])
def test_nf4_decoder(gpu, tau, T, BS, SBS, delta, res_fmt):
    q, k, v = _inputs(1, T, tau, 3, 16)
    pk, sc, res = OF.quantize_nf4(f32(k), tau, res_fmt)
    kh = OF.khat_nf4(pk, sc, 128)
    o_ref, diag = O.decode(f32(q), pk, None, None, f32(v), res, res_fmt=res_fmt, BS=BS, SBS=SBS, delta=delta,
                           khat=kh, out_dtype=tau)
    ws = NFK.__dict__["DecodeWorkspace"](1, 32, 8, T, BS, SBS, gpu, TORCH_DT[tau])
    o = NFK.attn_forward_decode_nf4(
        q.to(gpu).unsqueeze(1).contiguous(), torch.from_numpy(pk).to(gpu), torch.from_numpy(sc).to(TORCH_DT[tau]).to(gpu),
        v.to(gpu), torch.from_numpy(res).view(FP8_DT[res_fmt]).to(gpu), BS=BS, SBS=SBS, delta=delta, workspace=ws)
    _check(o, ws, o_ref, diag, f"nf4 {tau} T={T}")


def test_kfmt_ragged_and_no_residual(gpu):
    """Ragged lengths (seq_lens) and use_fp8_residual=False on the nf4 decoder."""
    lens = [1500, 640]
    q, k, v = _inputs(2, 1500, "bf16", 4, 16, seq_lens=lens)
    pk, sc, res = OF.quantize_nf4(f32(k), "bf16", "e4m3fn")
    kh = OF.khat_nf4(pk, sc, 128)
    o_ref, diag = O.decode(f32(q), pk, None, None, f32(v), res, res_fmt="e4m3fn", BS=64, SBS=64, delta=5.0,
                           khat=kh, use_fp8_residual=False, seq_lens=lens, out_dtype="bf16")
    ws = NFK.__dict__["DecodeWorkspace"](2, 32, 8, 1500, 64, 64, gpu, torch.bfloat16)
    o = NFK.attn_forward_decode_nf4(
        q.to(gpu).unsqueeze(1).contiguous(), torch.from_numpy(pk).to(gpu), torch.from_numpy(sc).to(torch.bfloat16).to(gpu),
        v.to(gpu), torch.from_numpy(res).view(torch.float8_e4m3fn).to(gpu), BS=64, delta=5.0, use_fp8_residual=False,
        seq_lens=torch.tensor(lens, dtype=torch.int32, device=gpu), workspace=ws)
    _check(o, ws, o_ref, diag, "nf4 ragged no-residual")


@pytest.mark.parametrize("fmt", ["fp8_scaled", "nvfp4", "nf4"])
def test_contiguous_large_grid_reload_build(gpu, fmt):
    """More workgroups than CUs (B=6, T=3000: 6 x 8 x 6 = 288) selects the contiguous decoders' build that
    reloads a kept chunk's codes and scales in the exact pass; it must match the oracle as the other does."""
    B, T = 6, 3000
    q, k, v = _inputs(B, T, "bf16", 11, 16)
    qd = q.to(gpu).unsqueeze(1).contiguous()
    if fmt == "fp8_scaled":
        base, s, res = OF.quantize_fp8_scaled(f32(k), "e4m3fn")
        kh = OF.khat_fp8_scaled(base, s, "e4m3fn")
        o_ref, diag = O.decode(f32(q), base, None, None, f32(v), res, res_fmt="e4m3fn", BS=64, SBS=64, delta=5.0,
                               khat=kh, out_dtype="bf16")
        ws = F8K.__dict__["DecodeWorkspace"](B, 32, 8, T, 64, 64, gpu, torch.bfloat16)
        o = F8K.attn_forward_decode_fp8fp8(
            qd, torch.from_numpy(base).view(torch.float8_e4m3fn).to(gpu), v.to(gpu),
            k_residual=torch.from_numpy(res).view(torch.float8_e4m3fn).to(gpu), BS=64, delta=5.0,
            k_scale=torch.from_numpy(s).to(torch.float16).to(gpu), workspace=ws)
    elif fmt == "nvfp4":
        pk, sc, res = OF.quantize_nvfp4(f32(k), "bf16", "e5m2", 64)
        kh, kp1 = OF.khat_nvfp4(pk, sc, 64, 128)
        o_ref, diag = O.decode(f32(q), pk, None, None, f32(v), res, res_fmt="e5m2", BS=64, SBS=64, delta=5.0,
                               khat=kh, khat_probe1=kp1, out_dtype="bf16")
        ws = NVK.__dict__["DecodeWorkspace"](B, 32, 8, T, 64, 64, gpu, torch.bfloat16)
        o = NVK.attn_forward_decode_nvfp4fp8(
            qd, torch.from_numpy(pk).to(gpu), torch.from_numpy(sc).to(torch.bfloat16).to(gpu), v.to(gpu),
            k_residual=torch.from_numpy(res).view(torch.float8_e5m2).to(gpu), BS=64, delta=5.0, workspace=ws)
    else:
        pk, sc, res = OF.quantize_nf4(f32(k), "bf16", "e5m2")
        kh = OF.khat_nf4(pk, sc, 128)
        o_ref, diag = O.decode(f32(q), pk, None, None, f32(v), res, res_fmt="e5m2", BS=64, SBS=64, delta=5.0,
                               khat=kh, out_dtype="bf16")
        ws = NFK.__dict__["DecodeWorkspace"](B, 32, 8, T, 64, 64, gpu, torch.bfloat16)
        o = NFK.attn_forward_decode_nf4(
            qd, torch.from_numpy(pk).to(gpu), torch.from_numpy(sc).to(torch.bfloat16).to(gpu), v.to(gpu),
            k_residual=torch.from_numpy(res).view(torch.float8_e5m2).to(gpu), BS=64, delta=5.0, workspace=ws)
    _check(o, ws, o_ref, diag, f"{fmt} contiguous, large grid")


@pytest.mark.parametrize("T,th_given", [(4096, False), (4096, True), (8192, False), (16384, False)])
def test_fp8_scaled_small_grid_spans(gpu, T, th_given):
    """The contiguous small-grid builds at B=1, 8 KV heads: T=4096 gives two-chunk spans (waves 2
    and 3 score, waves 0 and 1 load and stage the residual / V rows before the prune), 8192
    four-chunk spans, 16384 eight-chunk spans in 256 workgroups (the register-holding build); with
    a caller's threshold the two-chunk build scores no probe window."""
    from ffa_mi355x import _native as N
    from ffa_mi355x.decode import DecodeWorkspace
    from ffa_mi355x.kfmt import run_kfmt_decode

    q, k, v = _inputs(1, T, "bf16", 12, 16)
    base, s, res = OF.quantize_fp8_scaled(f32(k), "e4m3fn")
    kh = OF.khat_fp8_scaled(base, s, "e4m3fn")
    th = None
    if th_given:
        _, d0 = O.decode(f32(q), base, None, None, f32(v), res, res_fmt="e4m3fn", BS=64, SBS=64, delta=5.0,
                         khat=kh, out_dtype="bf16")
        th = d0["threshold"] + 0.5  # a different threshold than the probe's: more blocks pruned
    o_ref, diag = O.decode(f32(q), base, None, None, f32(v), res, res_fmt="e4m3fn", BS=64, SBS=64, delta=5.0,
                           khat=kh, out_dtype="bf16", precomputed_threshold=th)
    ws = DecodeWorkspace(1, 32, 8, T, 64, 64, gpu, torch.bfloat16)
    run_kfmt_decode(q=q.to(gpu), k=torch.from_numpy(base).view(torch.float8_e4m3fn).to(gpu),
                    k_format=N.KFMT_FP8_E4M3, k_scale=torch.from_numpy(s).to(torch.float16).to(gpu),
                    scale_kind=N.KSCALE_TOKEN, v=v.to(gpu),
                    k_residual=torch.from_numpy(res).view(torch.float8_e4m3fn).to(gpu), use_res=True, T=T, HKV=8,
                    scale=128 ** -0.5, BS=64, SBS=64, delta=5.0,
                    precomputed_threshold=None if th is None else torch.from_numpy(th).to(gpu), workspace=ws)
    _check(ws.o, ws, o_ref, diag, f"fp8 scaled T={T} threshold given={th_given}")


def test_fp8_scaled_small_grid_ragged_with_empty_sequence(gpu):
    """Two-chunk spans (B=3, T=1024) over lengths 0, 37 and 1024: an empty sequence (output 0), a
    sequence inside its first chunk, and a full one."""
    from ffa_mi355x import _native as N
    from ffa_mi355x.decode import DecodeWorkspace
    from ffa_mi355x.kfmt import run_kfmt_decode

    lens = [0, 37, 1024]
    B, T = 3, 1024
    q, k, v = _inputs(B, T, "bf16", 13, 16, seq_lens=lens)
    base, s, res = OF.quantize_fp8_scaled(f32(k), "e4m3fn")
    kh = OF.khat_fp8_scaled(base, s, "e4m3fn")
    o_ref, diag = O.decode(f32(q), base, None, None, f32(v), res, res_fmt="e4m3fn", BS=64, SBS=64, delta=5.0,
                           khat=kh, out_dtype="bf16", seq_lens=lens)
    ws = DecodeWorkspace(B, 32, 8, T, 64, 64, gpu, torch.bfloat16)
    run_kfmt_decode(q=q.to(gpu), k=torch.from_numpy(base).view(torch.float8_e4m3fn).to(gpu),
                    k_format=N.KFMT_FP8_E4M3, k_scale=torch.from_numpy(s).to(torch.float16).to(gpu),
                    scale_kind=N.KSCALE_TOKEN, v=v.to(gpu),
                    k_residual=torch.from_numpy(res).view(torch.float8_e4m3fn).to(gpu), use_res=True, T=T, HKV=8,
                    scale=128 ** -0.5, BS=64, SBS=64, delta=5.0,
                    seq_lens=torch.tensor(lens, dtype=torch.int32, device=gpu), workspace=ws)
    torch.cuda.synchronize()
    assert torch.count_nonzero(ws.o[0]).item() == 0, "an empty sequence decodes to 0"
    far, near, n_near = compare_masks(ws.mask_buf.cpu().numpy(), diag)
    assert far == 0, f"{far} mask mismatches away from the threshold"
    th = ws.threshold_buf.cpu().numpy()[1:]
    assert np.abs(th - diag["threshold"][1:]).max() < 1e-4, "threshold"
    mx, mean = assert_out_close(f32(ws.o), o_ref, "fp8 scaled ragged small grid")
    print(f"[out] ragged small grid max_abs={mx:.3e} mean_abs={mean:.3e}")
