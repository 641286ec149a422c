"""GPU quantizers and K producers vs the CPU oracle.

Quantized bytes (codes, scale, zero, residual) must be bit-exact given the
same K; the K-projection GEMM accumulates in fp32 in its own order, so the
rotated K is compared with a tolerance and the bytes are compared against the
oracle quantizer applied to the GPU's own K.
"""
import numpy as np
import pytest
import torch

from helpers import FP8_DT, TORCH_DT, assert_out_close, f32
from oracle import producer as OP
from ffa_mi355x import quant as Q
from ffa_mi355x import synth
from ffa_mi355x.paged import scale_pos
from oracle import q2fp8 as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tau", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("fmt", ["e5m2", "e4m3fn"])
def test_quantize_per_channel_bit_exact(gpu, tau, fmt):
    from ffa_mi355x import quant

    g = torch.Generator().manual_seed(1)
    k = (torch.randn(2, 1500, 8, 128, generator=g) * 2).to(TORCH_DT[tau])
    k[:, :, 3, 5] = 0.25  # constant channel
    kq, s, z, r = quant.quantize_per_channel(k.to(gpu), FP8_DT[fmt])
    torch.cuda.synchronize()
    pk, so, zo, ro = O.quantize_per_channel(f32(k), tau, fmt)
    assert np.array_equal(kq.cpu().numpy(), pk)
    assert np.array_equal(f32(s), so) and np.array_equal(f32(z), zo)
    assert np.array_equal(r.view(torch.uint8).cpu().numpy(), ro)


def test_quantize_per_channel_odd_head_dim(gpu):
    from ffa_mi355x import quant

    g = torch.Generator().manual_seed(2)
    k = torch.randn(1, 77, 2, 6, generator=g).half()
    kq, s, z, r = quant.quantize_per_channel(k.to(gpu), torch.float8_e5m2)
    pk, so, zo, ro = O.quantize_per_channel(f32(k), "fp16", "e5m2")
    assert np.array_equal(kq.cpu().numpy(), pk) and np.array_equal(r.view(torch.uint8).cpu().numpy(), ro)


def test_g32_append_bit_exact(gpu):
    from ffa_mi355x import synth
    from ffa_mi355x.paged import PagedQ2Cache

    B, T, HKV = 3, 300, 8
    g = torch.Generator().manual_seed(3)
    k = (torch.randn(B, T, HKV, 128, generator=g) * 3).bfloat16()
    v = torch.randn(B, T, HKV, 128, generator=g).bfloat16()
    bt, P = synth.page_tables([T] * B, seed=3)
    cache = PagedQ2Cache(P, HKV, gpu)
    # two appends: a prefix of 200 tokens, then the remaining 100 at position 200
    pos0 = torch.zeros(B, dtype=torch.int32)
    cache.append(k[:, :200].to(gpu), v[:, :200].to(gpu), pos0.to(gpu), bt.to(gpu))
    cache.append(k[:, 200:].to(gpu), v[:, 200:].to(gpu), (pos0 + 200).to(gpu), bt.to(gpu))
    torch.cuda.synchronize()
    pk, s, z, r = O.quantize_g32(f32(k), "e4m3fn")
    from ffa_mi355x.paged import CODES_ORDER, GSCALE_ORDER, RES_ORDER, VT_ORDER, to_logical

    kq_pool = to_logical(cache.k_q.cpu().numpy(), CODES_ORDER, 8)
    spos = np.array([scale_pos(t) for t in range(64)])
    s_pool = to_logical(cache.k_scale.float().cpu().numpy(), GSCALE_ORDER)[..., spos]  # back to token order
    z_pool = to_logical(cache.k_zero.float().cpu().numpy(), GSCALE_ORDER)[..., spos]
    r_pool = to_logical(cache.k_res.view(torch.uint8).cpu().numpy(), RES_ORDER)
    v_pool = to_logical(cache.v.view(torch.int16).cpu().numpy(), VT_ORDER)
    vb = v.to(cache.v.dtype).view(torch.int16).numpy()
    for b in range(B):
        for t in range(0, T, 64):
            page, n = int(bt[b, t // 64]), min(64, T - t)
            assert np.array_equal(kq_pool[page, :, :, :n].transpose(2, 0, 1, 3).reshape(n, HKV, 32), pk[b, t:t + n])
            assert np.array_equal(s_pool[page, :, :, :n].transpose(2, 0, 1), s[b, t:t + n])
            assert np.array_equal(z_pool[page, :, :, :n].transpose(2, 0, 1), z[b, t:t + n])
            assert np.array_equal(r_pool[page, :, :n].transpose(1, 0, 2), r[b, t:t + n])
            assert np.array_equal(v_pool[page, :, :, :n].transpose(2, 0, 1), vb[b, t:t + n])


@pytest.mark.parametrize("h_dtype,cs_dtype", [("bf16", "fp32"), ("fp16", "fp16"), ("bf16", "bf16")])
def test_kproj_rope_channel(gpu, h_dtype, cs_dtype):
    from ffa_mi355x import quant

    B, T, H, HKV, D = 2, 40, 512, 4, 64
    g = torch.Generator().manual_seed(4)
    h = torch.randn(B, T, H, generator=g).to(TORCH_DT[h_dtype])
    w = (torch.randn(HKV * D, H, generator=g) * 0.05).to(TORCH_DT[h_dtype])
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    ang = torch.outer(torch.arange(T, dtype=torch.float32), inv)
    emb = torch.cat([ang, ang], -1)
    cos, sin = emb.cos().to(TORCH_DT[cs_dtype]), emb.sin().to(TORCH_DT[cs_dtype])
    (kq, s, z, r), k_gpu = quant.kproj_rope_q2_channel(h.to(gpu), w.to(gpu), cos.to(gpu), sin.to(gpu), HKV, D,
                                                       fp8_dtype=torch.float8_e5m2, return_k=True)
    torch.cuda.synchronize()
    k_ref, odt = OP.kproj_rope(f32(h), f32(w), f32(cos), f32(sin), HKV, D, h_dtype=h_dtype, cs_dtype=cs_dtype)
    kg = f32(k_gpu)
    # GEMM accumulation order differs: allow one ulp of the h dtype (relative) after RoPE
    tol = {"bf16": 2 ** -7, "fp16": 2 ** -10, "fp32": 2 ** -7}[h_dtype] * 2
    assert np.abs(kg - k_ref).max() <= tol * (np.abs(k_ref).max() + 1e-3)
    assert (kg != k_ref).mean() < 0.05
    # quantization of the GPU's own K is bit-exact
    pk, so, zo, ro = O.quantize_per_channel(kg, odt, "e5m2")
    assert np.array_equal(kq.cpu().numpy(), pk)
    assert np.array_equal(f32(s), so) and np.array_equal(f32(z), zo)
    assert np.array_equal(r.view(torch.uint8).cpu().numpy(), ro)


def test_reference_smoke_test(gpu):
    """The drop-in's producer self-check (run_smoke_test): torch and fused HIP producers agree."""
    import fused_kproj_rope_q2fp8 as FK

    FK.run_smoke_test(gpu, torch.float16, torch.float8_e5m2, B=2, T=32, H=256, HKV=4, K=64)


@pytest.mark.parametrize("B,Tn,H,use_bias", [(3, 20, 4096, False), (2, 7, 288, True), (1, 64, 4096, True)])
def test_kproj_append_multi_token_bit_exact(gpu, B, Tn, H, use_bias):
    """Appends of several tokens per sequence (token tiles with a ragged last tile, page boundaries,
    H with whole and partial k batches, bias): every byte equals the oracle's g32 quantization of the
    rotated K that ffa_kproj_rope (the same GEMM tile) computes; V^T bytes are the new V."""
    from ffa_mi355x import kfmt_quant as KQ
    from ffa_mi355x import quant, synth
    from ffa_mi355x.paged import CODES_ORDER, GSCALE_ORDER, RES_ORDER, VT_ORDER, PagedQ2Cache, to_logical

    HKV = 8
    g = torch.Generator().manual_seed(B * 100 + Tn)
    h = torch.randn(B, Tn, H, generator=g).bfloat16()
    w = (torch.randn(HKV * 128, H, generator=g) * 0.02).bfloat16()  # [out, in] orientation
    bias = (torch.randn(HKV * 128, generator=g) * 0.1).bfloat16() if use_bias else None
    pos = torch.tensor([50 + 13 * b for b in range(B)], dtype=torch.int32)
    inv = 1.0 / (500000.0 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))
    ang = (pos[:, None].float() + torch.arange(Tn, dtype=torch.float32)[None, :])[..., None] * inv
    emb = torch.cat([ang, ang], -1)  # [B, Tn, 128]
    cos, sin = emb.cos(), emb.sin()
    lens = [int(p) + Tn for p in pos]
    bt, P = synth.page_tables(lens, seed=B)
    cache = PagedQ2Cache(P, HKV, gpu)
    v_new = torch.randn(B, Tn, HKV, 128, generator=g).bfloat16()
    quant.kproj_rope_q2_append(cache, h.to(gpu), w.to(gpu), cos.to(gpu), sin.to(gpu), pos.to(gpu), bt.to(gpu),
                               bias=None if bias is None else bias.to(gpu), v_new=v_new.to(gpu))
    M = B * Tn
    k_own = KQ.kproj_rope(h.view(1, M, H).to(gpu), w.to(gpu), cos.view(M, 128).to(gpu), sin.view(M, 128).to(gpu),
                          HKV, 128, bias=None if bias is None else bias.to(gpu))
    torch.cuda.synchronize()
    k_ref = OP.kproj_rope_rows(f32(h), f32(w), f32(cos), f32(sin), HKV, bias=None if bias is None else f32(bias))
    assert np.abs(f32(k_own).reshape(B, Tn, HKV, 128) - k_ref).max() < 2e-2 * max(1.0, np.abs(k_ref).max())
    pk, s, z, r = O.quantize_g32(f32(k_own).reshape(B, Tn, HKV, 128), "e4m3fn")
    kq_pool = to_logical(cache.k_q.cpu().numpy(), CODES_ORDER, 8)
    sp = [scale_pos(t) for t in range(64)]
    s_pool = to_logical(cache.k_scale.float().cpu().numpy(), GSCALE_ORDER)[..., sp]
    z_pool = to_logical(cache.k_zero.float().cpu().numpy(), GSCALE_ORDER)[..., sp]
    r_pool = to_logical(cache.k_res.view(torch.uint8).cpu().numpy(), RES_ORDER)
    v_pool = to_logical(cache.v.view(torch.int16).cpu().numpy(), VT_ORDER)
    vb = v_new.to(cache.v.dtype).view(torch.int16).numpy()
    for b in range(B):
        for n in range(Tn):
            t = int(pos[b]) + n
            page, slot = int(bt[b, t // 64]), t % 64
            assert np.array_equal(kq_pool[page, :, :, slot].reshape(HKV, 32), pk[b, n]), ("codes", b, n)
            assert np.array_equal(s_pool[page, :, :, slot], s[b, n]), ("scales", b, n)
            assert np.array_equal(z_pool[page, :, :, slot], z[b, n]), ("zeros", b, n)
            assert np.array_equal(r_pool[page, :, slot], r[b, n]), ("residual", b, n)
            assert np.array_equal(v_pool[page, :, :, slot], vb[b, n]), ("V", b, n)


def test_kproj_append_config5_small(gpu):
    """K-proj (theta 5e5, positions 65536+) + g32 quantize + paged append, then decode over the cache."""
    from ffa_mi355x import quant, synth
    from ffa_mi355x.paged import PagedQ2Cache

    B, H, HKV, T0 = 4, 512, 8, 700
    g = torch.Generator().manual_seed(5)
    h = torch.randn(B, 1, H, generator=g).bfloat16()
    w = (torch.randn(H, HKV * 128, generator=g) * 0.02).bfloat16()  # [in, out] orientation
    pos = torch.full((B,), T0, dtype=torch.int32) + torch.arange(B, dtype=torch.int32)
    inv = 1.0 / (500000.0 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))
    ang = pos.float()[:, None] * inv[None, :]
    emb = torch.cat([ang, ang], -1)[:, None, :]  # [B, 1, 128]
    cos, sin = emb.cos(), emb.sin()
    lens = [int(p) + 1 for p in pos]
    bt, P = synth.page_tables(lens, seed=5)
    cache = PagedQ2Cache(P, HKV, gpu)
    v_new = torch.randn(B, 1, HKV, 128, generator=g).bfloat16()
    quant.kproj_rope_q2_append(cache, h.to(gpu), w.to(gpu), cos.to(gpu), sin.to(gpu), pos.to(gpu), bt.to(gpu),
                               v_new=v_new.to(gpu))
    torch.cuda.synchronize()
    k_ref = OP.kproj_rope_rows(f32(h), f32(w).T, f32(cos), f32(sin), HKV)
    pk, s, z, r = O.quantize_g32(k_ref, "e4m3fn")
    from ffa_mi355x.paged import CODES_ORDER, GSCALE_ORDER, RES_ORDER, VT_ORDER, to_logical

    kq_pool = to_logical(cache.k_q.cpu().numpy(), CODES_ORDER, 8)
    s_pool = to_logical(cache.k_scale.float().cpu().numpy(), GSCALE_ORDER)[..., [scale_pos(t) for t in range(64)]]
    r_pool = to_logical(cache.k_res.view(torch.uint8).cpu().numpy(), RES_ORDER)
    v_pool = torch.from_numpy(to_logical(cache.v.view(torch.int16).cpu().numpy(), VT_ORDER)).view(cache.v.dtype)
    mism = 0
    for b in range(B):
        page, slot = int(bt[b, int(pos[b]) // 64]), int(pos[b]) % 64
        codes_gpu = O.unpack_2bit(kq_pool[page, :, :, slot].reshape(HKV, 32), 128)
        codes_ref = O.unpack_2bit(pk[b, 0], 128)
        mism += int((codes_gpu != codes_ref).sum())
        assert np.allclose(s_pool[page, :, :, slot], s[b, 0], rtol=2e-2, atol=1e-4)
        res_gpu = O.fp8_decode(r_pool[page, :, slot], "e4m3fn") if hasattr(O, "fp8_decode") else None
        assert res_gpu is not None
        deq_gpu = codes_gpu.astype(np.float32) * np.repeat(s_pool[page, :, :, slot], 32, -1)
        assert np.isfinite(deq_gpu).all()
        vg = v_pool[page, :, :, slot]
        assert torch.equal(vg, v_new[b, 0])
    assert mism <= 0.01 * B * HKV * 128
    # ffa_kproj_rope runs the same GEMM tile (same fp32 sums), so its rotated K, quantized by the oracle,
    # must give exactly the appended bytes
    from ffa_mi355x import kfmt_quant as KQ

    k_own = KQ.kproj_rope(h.view(1, B, H).to(gpu), w.to(gpu), cos.view(B, 128).to(gpu), sin.view(B, 128).to(gpu),
                          HKV, 128)
    torch.cuda.synchronize()
    pk2, s2, z2, r2 = O.quantize_g32(f32(k_own).reshape(B, 1, HKV, 128), "e4m3fn")
    z_pool = to_logical(cache.k_zero.float().cpu().numpy(), GSCALE_ORDER)[..., [scale_pos(t) for t in range(64)]]
    for b in range(B):
        page, slot = int(bt[b, int(pos[b]) // 64]), int(pos[b]) % 64
        assert np.array_equal(kq_pool[page, :, :, slot].reshape(HKV, 32), pk2[b, 0]), "codes"
        assert np.array_equal(s_pool[page, :, :, slot], s2[b, 0]), "scales"
        assert np.array_equal(z_pool[page, :, :, slot], z2[b, 0]), "zeros"
        assert np.array_equal(r_pool[page, :, slot], r2[b, 0]), "residual"


@pytest.mark.parametrize("tau", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("fmt", ["e5m2", "e4m3fn"])
def test_append_per_channel_bit_exact(gpu, tau, fmt):
    """Reference-layout append: new tokens (many outside the cache's per-channel range) quantized with
    the cache's scale / zero are byte-identical to the oracle's; an overwrite of earlier positions too."""
    g = torch.Generator().manual_seed(61)
    B, T0, Tcap, HKV, D = 2, 300, 400, 4, 128
    k0 = (torch.randn(B, T0, HKV, D, generator=g) * 2).to(TORCH_DT[tau])
    kq0, s, z, r0 = Q.quantize_per_channel(k0.to(gpu), FP8_DT[fmt])
    kq = torch.zeros((B, Tcap, HKV, D // 4), dtype=torch.uint8, device=gpu)
    kr = torch.zeros((B, Tcap, HKV, D), dtype=FP8_DT[fmt], device=gpu)
    kq[:, :T0].copy_(kq0)
    kr[:, :T0].copy_(r0)
    k_new = (torch.randn(B, 17, HKV, D, generator=g) * 4).to(TORCH_DT[tau])
    pos = torch.tensor([300, 250], dtype=torch.int32)
    Q.append_per_channel(kq, s, z, kr, k_new.to(gpu), pos)
    torch.cuda.synchronize()
    cache_q = np.concatenate([kq0.cpu().numpy(), np.zeros((B, Tcap - T0, HKV, D // 4), np.uint8)], axis=1)
    cache_r = np.concatenate([r0.view(torch.uint8).cpu().numpy(), np.zeros((B, Tcap - T0, HKV, D), np.uint8)], axis=1)
    oq, orr = O.append_per_channel(cache_q, cache_r, f32(k_new), f32(s), f32(z), pos.tolist(), tau, fmt)
    assert np.array_equal(kq.cpu().numpy(), oq)
    assert np.array_equal(kr.view(torch.uint8).cpu().numpy(), orr)
    c = O.unpack_2bit(oq[:, 300:317], D)
    assert (c == 0).any() and (c == 3).any()


def test_append_per_channel_then_decode(gpu):
    """A reference-layout cache filled by the quantizer over its first tokens and by appends for the
    rest decodes (through the drop-in) to the oracle's result on the oracle's appended cache."""
    import attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8 as K

    B, T0, T, HQ, HKV = 2, 1500, 2048, 32, 8
    q, k, v = synth.attention_inputs(B=B, T=T, HQ=HQ, HKV=HKV, seed=62, n_heavy=16, dtype=torch.float16)
    kd = k.to(gpu)
    kq0, s, z, r0 = Q.quantize_per_channel(kd[:, :T0].contiguous(), torch.float8_e5m2)
    kq = torch.zeros((B, T, HKV, 32), dtype=torch.uint8, device=gpu)
    kr = torch.zeros((B, T, HKV, 128), dtype=torch.float8_e5m2, device=gpu)
    vd = torch.zeros((B, T, HKV, 128), dtype=torch.float16, device=gpu)
    kq[:, :T0].copy_(kq0)
    kr[:, :T0].copy_(r0)
    vd[:, :T0].copy_(v[:, :T0].to(gpu))
    for a in range(T0, T, 200):  # appends of 200 tokens (the last one shorter)
        e = min(a + 200, T)
        Q.append_per_channel(kq, s, z, kr, kd[:, a:e].contiguous(), a, v=vd, v_new=v[:, a:e].to(gpu))
    qd = q.to(gpu).unsqueeze(1).contiguous()
    o = K.attn_forward_decode_quantized(qd, kq, s, z, vd, k_residual=kr, BS=64, delta=5.0)
    torch.cuda.synchronize()
    # the oracle's cache: its quantizer over the first T0 tokens, its append for the rest
    pk0, os_, oz, or0 = O.quantize_per_channel(f32(k[:, :T0]), "fp16", "e5m2")
    okq = np.concatenate([pk0, np.zeros((B, T - T0, HKV, 32), np.uint8)], axis=1)
    okr = np.concatenate([or0, np.zeros((B, T - T0, HKV, 128), np.uint8)], axis=1)
    okq, okr = O.append_per_channel(okq, okr, f32(k[:, T0:]), os_, oz, [T0, T0], "fp16", "e5m2")
    assert np.array_equal(kq.cpu().numpy(), okq) and np.array_equal(kr.view(torch.uint8).cpu().numpy(), okr)
    o_ref, diag = O.decode(f32(q), okq, os_, oz, f32(v), okr, res_fmt="e5m2", BS=64, SBS=64, delta=5.0,
                           out_dtype="fp16")
    mx, mean = assert_out_close(f32(o), o_ref, "appended reference-layout cache")
    print(f"[out] append + decode max_abs={mx:.3e} mean_abs={mean:.3e} skip={diag['skip_ratio']:.3f}")
