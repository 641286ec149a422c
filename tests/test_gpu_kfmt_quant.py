"""GPU quantizers and producers of the fp8 / nvfp4 / nf4 formats vs the CPU oracle.

The oracle quantizers (oracle/formats.py) are pinned against torch's own op
sequences on the CPU (tests/test_oracle_formats.py).  Given the same K, every
byte the HIP quantizers write (codes, scales, residuals) must equal the
oracle's.  The producers' GEMM accumulates in its own order, so their bytes are
compared against the oracle applied to the GPU's own rotated K.
"""
import importlib.util
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import FP8_DT, TORCH_DT, f32
from oracle import formats as OF
from oracle import numerics as NM
from oracle import producer as OP

pytestmark = pytest.mark.gpu
PKG = Path(__file__).resolve().parents[1] / "ffa-speedtest_amd"


def _load(rel, name):
    spec = importlib.util.spec_from_file_location(name, PKG / rel)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


F8P = _load("ffa-fp8fp8/fused_kproj_rope_fp8fp8.py", "prod_fp8fp8_gpu")
NVP = _load("ffa-nvfp4fp8/fused_kproj_rope_nvfp4fp8.py", "prod_nvfp4_gpu")
NFP = _load("ffa-nf4fp8/fused_kproj_rope_nf4fp8.py", "prod_nf4_gpu")


def _k(shape, tau, seed, outliers=True):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(shape, generator=g)
    if outliers:
        k[..., :4] *= 10.0
    return k.to(TORCH_DT[tau])


def _u8(t):
    return t.contiguous().view(torch.uint8).cpu().numpy()


@pytest.mark.parametrize("tau", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("fmt", ["e4m3fn", "e5m2"])
@pytest.mark.parametrize("D", [128, 77])
def test_fp8_scaled_quantizer_bit_exact(gpu, tau, fmt, D):
    """Per-token-scaled fp8 (one fp16 scale per token and KV head): base, scale and residual
    bytes equal the oracle's, with outlier channels, an all-zero row and a tiny row."""
    from ffa_mi355x import kfmt_quant as KQ

    k = _k((2, 300, 8, D), tau, 3)
    k[0, 5, 2] = 0.0  # amax 0: the scale floor 2^-14
    k[1, 7, 1] = (torch.randn(D) * 1e-7).to(TORCH_DT[tau])
    row = torch.randn(D)
    k[1, 9, 3] = (row * (3.5e-5 / row.abs().max())).to(TORCH_DT[tau])  # fp16(amax / 448) is subnormal
    base, sc, res = KQ.quantize_fp8_scaled(k.to(gpu), FP8_DT[fmt])
    torch.cuda.synchronize()
    ob, osc, orr = OF.quantize_fp8_scaled(f32(k), fmt)
    assert base.shape == k.shape and sc.shape == k.shape[:-1] and sc.dtype == torch.float16
    assert np.array_equal(_u8(base), ob)
    assert np.array_equal(f32(sc), osc)
    assert np.array_equal(_u8(res), orr)
    # no NaN / inf byte anywhere (e4m3fn: 0x7F / 0xFF; e5m2: exponent all ones)
    bad = (lambda b: (b & 0x7F) == 0x7F) if fmt == "e4m3fn" else (lambda b: (b & 0x7C) == 0x7C)
    assert not bad(_u8(base)).any() and not bad(_u8(res)).any()
    assert f32(sc).min() >= 2.0 ** -14


@pytest.mark.parametrize("tau", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("fmt", ["e4m3fn", "e5m2"])
def test_fp8fp8_quantizer_bit_exact(gpu, tau, fmt):
    k = _k((2, 77, 3, 128), tau, 1)
    # 1000 / -60000 overflow e4m3 (NaN base), 1e-9 underflows to zero
    k[0, 0, 0, :3] = torch.tensor([1000.0, -60000.0, 1e-9]).to(TORCH_DT[tau])
    base, res = F8P.quantize_k_fp8_fp8_residual(k.to(gpu), FP8_DT[fmt])
    torch.cuda.synchronize()
    ob, orr = OF.quantize_fp8fp8(f32(k), fmt)
    assert base.dtype == FP8_DT[fmt] and base.shape == k.shape
    assert np.array_equal(_u8(base), ob)
    # where the base is NaN the residual is NaN too (its sign bit is not specified): compare NaN-ness there
    nan = (lambda b: (b & 0x7F) == 0x7F) if fmt == "e4m3fn" else (lambda b: ((b & 0x7C) == 0x7C) & ((b & 3) != 0))
    g = _u8(res)
    assert np.array_equal(g[~nan(ob)], orr[~nan(ob)]) and nan(g[nan(ob)]).all() and nan(orr[nan(ob)]).all()


@pytest.mark.parametrize("tau", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("T,D,page", [(300, 128, 128), (129, 64, 16), (64, 63, 64)])
def test_nvfp4_quantizer_bit_exact(gpu, tau, T, D, page):
    k = _k((2, T, 3, D), tau, 2)
    k[1, :page, 2] = 0  # an all-zero block: scale clamps to tau(1e-6)
    packed, scale, res = NVP.encode_k_nvfp4_fp8_residual(k.to(gpu), torch.float8_e5m2, page)
    torch.cuda.synchronize()
    op, osc, orr = OF.quantize_nvfp4(f32(k), tau, "e5m2", page)
    assert packed.shape == op.shape and scale.dtype == TORCH_DT[tau] and scale.shape == osc.shape
    assert np.array_equal(packed.cpu().numpy(), op)
    assert np.array_equal(f32(scale), osc)
    assert np.array_equal(_u8(res), orr)


@pytest.mark.parametrize("tau", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("T,D,fmt", [(777, 128, "e4m3fn"), (40, 63, "e5m2")])
def test_nf4_quantizer_bit_exact(gpu, tau, T, D, fmt):
    k = _k((2, T, 3, D), tau, 3)
    k[0, :, 1, 5] = 0  # an all-zero channel: scale clamps to 1e-6
    packed, scale, res = NFP.encode_k_nf4_fp8_residual(k.to(gpu), FP8_DT[fmt])
    torch.cuda.synchronize()
    op, osc, orr = OF.quantize_nf4(f32(k), tau, fmt)
    assert scale.dtype == TORCH_DT[tau]
    assert np.array_equal(packed.cpu().numpy(), op)
    assert np.array_equal(f32(scale), osc)
    assert np.array_equal(_u8(res), orr)


@pytest.mark.parametrize("h_dtype,cs_dtype", [("bf16", "fp32"), ("fp16", "fp16")])
def test_format_producers_quantize_their_own_k_bit_exact(gpu, h_dtype, cs_dtype):
    """HIP K-proj + RoPE (ffa_kproj_rope) within a GEMM ulp of the oracle; each format's bytes
    equal the oracle quantizer applied to that K."""
    from ffa_mi355x import kfmt_quant as KQ

    B, T, H, HKV, D = 2, 50, 256, 4, 128
    g = torch.Generator().manual_seed(6)
    h = torch.randn(B, T, H, generator=g).to(TORCH_DT[h_dtype])
    w = (torch.randn(HKV * D, H, generator=g) * 0.05).to(TORCH_DT[h_dtype])
    cos, sin = (t.to(TORCH_DT[cs_dtype]) for t in NVP.build_rope_cache(T, D, base=500000.0))
    args = (h.to(gpu), w.to(gpu), cos.to(gpu), sin.to(gpu), HKV, D)
    k_gpu = KQ.kproj_rope(*args)
    torch.cuda.synchronize()
    k_ref, odt = OP.kproj_rope(f32(h), f32(w), f32(cos), f32(sin), HKV, D, h_dtype=h_dtype, cs_dtype=cs_dtype)
    kg = f32(k_gpu)
    tol = {"bf16": 2 ** -7, "fp16": 2 ** -10}[h_dtype] * 2
    assert np.abs(kg - k_ref).max() <= tol * (np.abs(k_ref).max() + 1e-3)
    base, res = F8P.kproj_rope_quantize_fused(*args, fp8_dtype=torch.float8_e4m3fn)
    ob, orr = OF.quantize_fp8fp8(kg, "e4m3fn")
    assert np.array_equal(_u8(base), ob) and np.array_equal(_u8(res), orr)
    pk, sc, res = NVP.kproj_rope_quantize_fused(*args, page_size=32, fp8_dtype=torch.float8_e5m2)
    op, osc, orr = OF.quantize_nvfp4(kg, odt, "e5m2", 32)
    assert np.array_equal(pk.cpu().numpy(), op) and np.array_equal(f32(sc), osc) and np.array_equal(_u8(res), orr)
    pk, sc, res = NFP.kproj_rope_nf4_fused(*args, fp8_dtype=torch.float8_e5m2)
    op, osc, orr = OF.quantize_nf4(kg, odt, "e5m2")
    assert sc.dtype == TORCH_DT[h_dtype]  # the reference's Triton producer returns the scale in h.dtype
    assert np.array_equal(pk.cpu().numpy(), op) and np.array_equal(_u8(res), orr)
    assert np.array_equal(f32(sc), NM.round_to(osc, h_dtype))


def test_format_producer_smoke_tests(gpu):
    """Each drop-in's run_smoke_test (torch-GEMM producer vs the fused HIP producer)."""
    F8P.run_smoke_test(gpu, torch.float16, torch.float8_e5m2, B=2, T=32, H=256, HKV=4, K=64)
    NVP.run_smoke_test(gpu, torch.float16, torch.float8_e5m2, B=2, T=32, H=256, HKV=4, K=64, page_size=128)
    NFP.run_smoke_test(gpu, torch.bfloat16, torch.float8_e5m2, B=2, T=32, H=256, HKV=4, K=64)


def test_nvfp4_producer_feeds_decoder(gpu):
    """Producer -> decoder: the HIP-encoded nvfp4 cache decodes like the oracle's encoding of the same K."""
    from helpers import assert_out_close, compare_masks
    from oracle import q2fp8 as O

    NVK = _load("ffa-nvfp4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nvfp4fp8.py", "dec_nvfp4_gpu")
    from ffa_mi355x import synth

    T, BS = 1100, 64
    q, k, v = synth.attention_inputs(B=1, T=T, HQ=32, HKV=8, seed=9, n_heavy=16, dtype=torch.bfloat16)
    pk, sc, res = NVP.encode_k_nvfp4_fp8_residual(k.to(gpu), torch.float8_e5m2, BS)
    ws = NVK.__dict__["DecodeWorkspace"](1, 32, 8, T, BS, BS, gpu, torch.bfloat16)
    o = NVK.attn_forward_decode_nvfp4fp8(q.to(gpu).unsqueeze(1).contiguous(), pk, sc, v.to(gpu), k_residual=res,
                                         BS=BS, delta=5.0, workspace=ws)
    torch.cuda.synchronize()
    opk, osc, orr = OF.quantize_nvfp4(f32(k), "bf16", "e5m2", BS)
    assert np.array_equal(pk.cpu().numpy(), opk)
    kh, kp1 = OF.khat_nvfp4(opk, osc, BS, 128)
    o_ref, diag = O.decode(f32(q), opk, None, None, f32(v), orr, res_fmt="e5m2", BS=BS, SBS=BS, delta=5.0,
                           khat=kh, khat_probe1=kp1, out_dtype="bf16")
    far, _, _ = compare_masks(ws.mask_buf.cpu().numpy(), diag)
    assert far == 0
    assert_out_close(f32(o), o_ref, "nvfp4 producer -> decoder")
