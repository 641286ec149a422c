"""CPU pins of the other formats' oracle (oracle/formats.py) and of the shared decode on them.

The reference holds no fixtures for these formats.  The quantizers are pinned by
running the same sequence of torch operations on the CPU (torch's own casts and
bucketize, an independent implementation of the roundings), by closed forms
(the e2m1 table, codebook midpoints) and by invariants; the decode by its
special cases (nothing pruned = plain softmax attention on the refined K, the
nvfp4 probe window taking the last block's scale).
"""
import math

import numpy as np
import pytest
import torch

from oracle import formats as OF
from oracle import numerics as NM
from oracle import q2fp8 as O

TD = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}
F8 = {"e4m3fn": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def _k(shape, tau, seed, outliers=False):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal(shape).astype(np.float32)
    if outliers:
        k[..., :4] *= 10.0
    return NM.round_to(k, tau)


def _bytes(t):
    return t.view(torch.uint8).numpy()


# ----------------------------------------------------------------------------- fp8 base
@pytest.mark.parametrize("tau", ["bf16", "fp16"])
@pytest.mark.parametrize("fmt", ["e4m3fn", "e5m2"])
def test_fp8fp8_quantizer_matches_torch(tau, fmt):
    k = _k((2, 40, 3, 128), tau, 1, outliers=True)
    base, res = OF.quantize_fp8fp8(k, fmt)
    kt = torch.from_numpy(k).to(TD[tau])
    bt = kt.to(F8[fmt])
    rt = (kt.to(torch.float32) - bt.to(torch.float32)).to(F8[fmt])  # fused_kproj_rope_fp8fp8.py:62-63
    assert np.array_equal(base, _bytes(bt)) and np.array_equal(res, _bytes(rt))
    # every fp8 value is an fp16 value: the decode's fp16 K is exact
    kh = OF.khat_fp8(base, fmt)
    assert np.array_equal(kh, NM.round_f16(kh))


def test_fp8_scaled_quantizer_invariants():
    k = _k((2, 33, 2, 128), "bf16", 2, outliers=True)
    base, s, res = OF.quantize_fp8_scaled(k, "e4m3fn")
    assert np.array_equal(s, NM.round_f16(s)) and (s > 0).all()
    deq = NM.fp8_decode(base, "e4m3fn") * s[..., None]
    # the largest |k| of each (token, head) maps near the top of the e4m3 range
    top = np.abs(NM.fp8_decode(base, "e4m3fn")).max(axis=-1)
    assert (top >= 416).all() and (top <= 448).all()
    # base + residual recovers k to e4m3 precision of the residual
    r = NM.fp8_decode(res, "e4m3fn")
    assert np.abs(deq + r - k).max() <= np.abs(k - deq).max() * 2.0 ** -3 + 1e-6
    kh = OF.khat_fp8_scaled(base, s, "e4m3fn")
    assert np.array_equal(kh, NM.round_f16(deq))


@pytest.mark.parametrize("fmt", ["e4m3fn", "e5m2"])
def test_fp8_scaled_zero_and_tiny_rows_stay_finite(fmt):
    """All-zero rows and rows whose amax / fmax is an fp16 subnormal: the scale is floored at
    the smallest normal fp16, so no byte is NaN / inf and k / s never passes fmax."""
    fmax = 448.0 if fmt == "e4m3fn" else 57344.0
    rng = np.random.default_rng(5)
    k = rng.standard_normal((1, 6, 1, 128)).astype(np.float32)
    k[0, 0] = 0.0
    k[0, 1] *= 3.5e-5 / np.abs(k[0, 1]).max()  # amax 3.5e-5: fp16(amax / 448) is one subnormal quantum
    k[0, 2] *= 1e-7
    k[0, 3] *= 1e-3
    base, s, res = OF.quantize_fp8_scaled(k, fmt)
    assert (s >= 2.0 ** -14).all() and np.array_equal(s, NM.round_f16(s))
    b, r = NM.fp8_decode(base, fmt), NM.fp8_decode(res, fmt)
    assert np.isfinite(b).all() and np.isfinite(r).all()
    assert np.abs(b).max() <= fmax
    assert (b[0, 0] == 0).all() and (r[0, 0] == 0).all()
    # the 3.5e-5 row: k / s is the plain quotient by 2^-14 (well inside the range), and base +
    # residual recovers k to the residual's precision
    assert np.array_equal(b[0, 1], NM.fp8_decode(NM.fp8_encode(k[0, 1] / np.float32(2.0 ** -14), fmt), fmt))
    rec = b * s[..., None] + r
    err = np.abs(rec - k)
    # the residual is RNE-rounded fp8: relative 2^-4 (e4m3) / 2^-3 (e5m2) of |k - base * s| for a
    # normal result, at most half the smallest subnormal (2^-10 / 2^-17) otherwise
    rel, sub = (2.0 ** -4, 2.0 ** -10) if fmt == "e4m3fn" else (2.0 ** -3, 2.0 ** -17)
    assert (err <= np.maximum(np.abs(k - b * s[..., None]) * rel, sub) + 1e-12).all()
    # a normal row keeps the old scale (fp16(amax / fmax) is normal for amax >= 448 * 2^-14 / 1)
    big = np.abs(k[0, 4:]).max(axis=-1)
    assert np.array_equal(s[0, 4:], NM.round_f16((big / np.float32(fmax)).astype(np.float32)).clip(2.0 ** -14))


# ----------------------------------------------------------------------------- nvfp4
def test_e2m1_decode_closed_form():
    codes = np.arange(16)
    got = OF.fp4_decode(codes)
    want = []
    for c in codes:
        s, e, m = c >> 3, (c >> 1) & 3, c & 1
        mag = m * 0.5 if e == 0 else 2.0 ** (e - 1) * (1 + m / 2)
        want.append(-mag if s else mag)
    assert np.array_equal(got, np.array(want, np.float32))
    assert np.array_equal(OF.FP4_THRESHOLDS, (OF.FP4_POS_LEVELS[:-1] + OF.FP4_POS_LEVELS[1:]) / 2)


@pytest.mark.parametrize("tau", ["bf16", "fp16", "fp32"])
def test_nvfp4_quantizer_matches_torch(tau):
    page = 16
    k = _k((2, 37, 2, 64), tau, 3)
    pk, scale, res = OF.quantize_nvfp4(k, tau, "e5m2", page)
    # the reference's sequence of torch ops (fused_kproj_rope_nvfp4fp8.py:62-114), in k's dtype
    kt = torch.from_numpy(k).to(TD[tau])
    B, T, H, D = kt.shape
    lv = torch.tensor(OF.FP4_POS_LEVELS.tolist(), dtype=kt.dtype)
    th = torch.tensor(OF.FP4_THRESHOLDS.tolist(), dtype=kt.dtype)
    npg = -(-T // page)
    kp = torch.cat([kt, torch.zeros((B, npg * page - T, H, D), dtype=kt.dtype)], dim=1)
    kb = kp.view(B, npg, page, H, D)
    sc = (kb.abs().amax(dim=(2, 4)) / lv[-1]).clamp_min(1e-6).to(kt.dtype)
    sb = sc[:, :, None, :, None]
    ks = kb / sb
    idx = torch.bucketize(ks.abs(), th, right=True)
    sign = ks < 0
    codes = (idx.to(torch.uint8) | (sign.to(torch.uint8) << 3)).view(B, npg * page, H, D)[:, :T]
    deq = lv[idx] * torch.where(sign, -torch.ones_like(ks), torch.ones_like(ks)) * sb
    rt = (kb - deq).to(torch.float8_e5m2).view(B, npg * page, H, D)[:, :T]
    assert np.array_equal(scale, sc.float().numpy())
    assert np.array_equal(OF.unpack_4bit(pk, D), codes.numpy())
    assert np.array_equal(res, _bytes(rt.contiguous()))


def test_4bit_packing_roundtrip_and_order():
    rng = np.random.default_rng(4)
    c = rng.integers(0, 16, (3, 5, 7))
    p = OF.pack_4bit(c)
    assert p.shape == (3, 5, 4) and np.array_equal(OF.unpack_4bit(p, 7), c)
    assert p[0, 0, 0] == (c[0, 0, 0] | (c[0, 0, 1] << 4))  # low nibble first
    assert (p[..., -1] >> 4 == 0).all()  # odd D pads a zero nibble


# ----------------------------------------------------------------------------- nf4
@pytest.mark.parametrize("tau", ["bf16", "fp16"])
def test_nf4_quantizer_matches_torch(tau):
    k = _k((2, 29, 2, 64), tau, 5)
    pk, scale, res = OF.quantize_nf4(k, tau, "e4m3fn")
    cb = torch.tensor(OF.NF4_CODEBOOK.tolist(), dtype=torch.float32)
    bounds = (cb[:-1] + cb[1:]) * 0.5
    kf = torch.from_numpy(k).to(TD[tau]).to(torch.float32)  # fused_kproj_rope_nf4fp8.py:77-87
    sc = kf.abs().amax(dim=1).clamp_min(1e-6)
    norm = (kf / sc[:, None]).clamp(cb[0].item(), cb[-1].item())
    idx = torch.bucketize(norm, bounds)
    rt = (kf - cb[idx] * sc[:, None]).to(torch.float8_e4m3fn)
    assert np.array_equal(scale, sc.to(TD[tau]).float().numpy())
    assert np.array_equal(OF.unpack_4bit(pk, 64), idx.numpy())
    assert np.array_equal(res, _bytes(rt))


def test_nf4_codes_are_nearest_levels():
    k = _k((1, 50, 1, 32), "fp32", 6)
    pk, scale, _ = OF.quantize_nf4(k, "fp32", "e4m3fn")
    c = OF.unpack_4bit(pk, 32)
    norm = k / np.maximum(np.abs(k).max(axis=1), 1e-6)[:, None]
    dist = np.abs(norm[..., None] - OF.NF4_CODEBOOK)
    assert np.all(dist[np.arange(1)[:, None, None, None], np.arange(50)[None, :, None, None],
                       np.arange(1)[None, None, :, None], np.arange(32)[None, None, None, :], c]
                  <= dist.min(axis=-1) + 1e-7)
    assert (c.max(axis=1) == 15).any() or (c.min(axis=1) == 0).any()  # absmax maps to an end level


# ----------------------------------------------------------------------------- decode on other formats
def _softmax_attn(q, kt, v, scale):
    s = (NM.round_f16(q).astype(np.float64) @ kt.astype(np.float64).T) * scale
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    return (p / p.sum(axis=-1, keepdims=True)) @ NM.round_f16(v).astype(np.float64)


@pytest.mark.parametrize("fmt", ["fp8", "nvfp4", "nf4"])
def test_decode_without_pruning_is_softmax_attention(fmt):
    B, T, HQ, HKV, D = 1, 200, 8, 2, 64
    rng = np.random.default_rng(7)
    q = rng.standard_normal((B, HQ, D)).astype(np.float32)
    k = NM.round_bf16(rng.standard_normal((B, T, HKV, D)).astype(np.float32))
    v = NM.round_bf16(rng.standard_normal((B, T, HKV, D)).astype(np.float32))
    probe = None
    if fmt == "fp8":
        base, res = OF.quantize_fp8fp8(k, "e5m2")
        kh, rf = OF.khat_fp8(base, "e5m2"), "e5m2"
    elif fmt == "nvfp4":
        pk, sc, res = OF.quantize_nvfp4(k, "bf16", "e5m2", 32)
        kh, probe = OF.khat_nvfp4(pk, sc, 32, D)
        rf = "e5m2"
    else:
        pk, sc, res = OF.quantize_nf4(k, "bf16", "e4m3fn")
        kh, rf = OF.khat_nf4(pk, sc, D), "e4m3fn"
    o, diag = O.decode(q, np.zeros((B, T, HKV, 1), np.uint8), None, None, v, res, res_fmt=rf, BS=32, SBS=32,
                       delta=math.inf, khat=kh, khat_probe1=probe, out_dtype="fp32")
    assert diag["skip_ratio"] == 0.0
    ktil = NM.round_f16(kh + NM.fp8_decode(res, rf))
    for h in range(HKV):
        ref = _softmax_attn(q[0, h * 4:(h + 1) * 4], ktil[0, :, h], v[0, :, h],
                            1 / math.sqrt(D))
        assert np.abs(o[0, h * 4:(h + 1) * 4] - ref).max() < 2e-3


def test_nvfp4_second_probe_window_uses_last_block_scale():
    """T=200, BS=32: NTB=7, the quirk window is tokens [96, 112) of block 3, scored with block 6's scale."""
    B, T, HQ, HKV, D, BS = 1, 200, 4, 1, 64, 32
    rng = np.random.default_rng(8)
    q = rng.standard_normal((B, HQ, D)).astype(np.float32)
    k = NM.round_bf16(rng.standard_normal((B, T, HKV, D)).astype(np.float32))
    k[:, 192:] *= 8.0  # the last block gets a much larger scale than block 3
    v = NM.round_bf16(rng.standard_normal((B, T, HKV, D)).astype(np.float32))
    pk, sc, res = OF.quantize_nvfp4(k, "bf16", "e5m2", BS)
    kh, kp1 = OF.khat_nvfp4(pk, sc, BS, D)
    assert sc[0, 6, 0] > 4 * sc[0, 3, 0]
    _, diag = O.decode(q, pk, None, None, v, res, res_fmt="e5m2", BS=BS, delta=2.0, khat=kh, khat_probe1=kp1)
    q16 = NM.round_f16(q[0])
    s = 1 / math.sqrt(D)
    sc_w0 = ((kh[0, 0:16, 0].astype(np.float64) @ q16.T.astype(np.float64)).astype(np.float32) * np.float32(s)
             ).astype(np.float32) * O.L2E
    w1 = OF.fp4_decode(OF.unpack_4bit(pk, D))[0, 96:112, 0] * sc[0, 6, 0]
    sc_w1 = ((NM.round_f16(w1).astype(np.float64) @ q16.T.astype(np.float64)).astype(np.float32) * np.float32(s)
             ).astype(np.float32) * O.L2E
    th = np.maximum(sc_w0.max(axis=0), sc_w1.max(axis=0)) - np.float32(2.0)
    assert np.array_equal(diag["threshold"][0], th.astype(np.float32))


# ----------------------------------------------------------------------------- benchmark group-scale modes
def test_nvfp4_g16_quantizer_pins():
    """Scales are torch's e4m3 cast of amax/6; codes are the nearest e2m1 level of k/s (ties to the
    larger level, the encoder's right=True rule); k_hat = level * s exactly; residual = torch's fp8 cast."""
    k = _k((2, 9, 3, 128), "bf16", 11, outliers=True)
    k[0, 0, 0, :16] = 0.0  # an all-zero block: scale 0, codes 0
    pk, sb, res = OF.quantize_nvfp4_g16(k)
    kb = torch.from_numpy(k).view(2, 9, 3, 8, 16)
    amax = kb.abs().amax(-1)
    assert np.array_equal(sb, _bytes((amax / 6.0).clamp(max=448.0).to(torch.float8_e4m3fn)))
    s = torch.from_numpy(sb).view(torch.float8_e4m3fn).float()[..., None]
    x = torch.where(s > 0, kb / s, torch.zeros_like(kb))
    codes = torch.from_numpy(OF.unpack_4bit(pk, 128)).view(2, 9, 3, 8, 16).long()
    lv = torch.from_numpy(OF.FP4_POS_LEVELS)
    mag = lv[codes & 7]
    d = (x.abs()[..., None] - lv).abs()  # brute force over the 8 levels
    best = d.min(-1).values
    assert torch.all((x.abs() - mag).abs() <= best + 1e-7)
    tie_hi = ((d - best[..., None]).abs() <= 1e-7).float().argmax(-1, keepdim=True)  # first (smaller) level
    n_tie = ((d - best[..., None]).abs() <= 1e-7).sum(-1)
    assert torch.all((n_tie < 2) | (codes & 7 > tie_hi[..., 0]))  # a tie takes the larger level
    assert torch.all(((codes >> 3) == 1) == (x < 0))
    kh = OF.khat_nvfp4_g16(pk, sb)
    exact = (torch.where(x < 0, -mag, mag) * s).reshape(2, 9, 3, 128).numpy()
    assert np.array_equal(kh, exact)  # fp16 rounding is a no-op here
    assert np.array_equal(res, _bytes((torch.from_numpy(k) - torch.from_numpy(exact)).to(torch.float8_e4m3fn)))
    assert (sb[0, 0, 0, 0] == 0) and (codes[0, 0, 0, 0] == 0).all()


def test_nf4_g64_quantizer_pins():
    """Scales are torch's fp16 cast of max(amax, 1e-6); codes are the nearest NF4 level of
    clamp(k/s, -1, 1) (ties to the smaller level, right=False); residual = torch's fp8 cast."""
    k = _k((2, 9, 3, 128), "bf16", 12, outliers=True)
    k[1, 2, 1, 64:] = 0.0  # zero block: s = fp16(1e-6), code 7 (level 0)
    pk, s, res = OF.quantize_nf4_g64(k)
    kb = torch.from_numpy(k).view(2, 9, 3, 2, 64)
    st = kb.abs().amax(-1).clamp(min=1e-6).to(torch.float16).float()
    assert np.array_equal(s, st.numpy())
    x = (kb / st[..., None]).clamp(-1.0, 1.0)
    codes = torch.from_numpy(OF.unpack_4bit(pk, 128)).view(2, 9, 3, 2, 64).long()
    cb = torch.from_numpy(OF.NF4_CODEBOOK)
    d = (x[..., None] - cb).abs()
    best = d.min(-1).values
    assert torch.all((x - cb[codes]).abs() <= best + 1e-7)
    deq = cb[codes] * st[..., None]
    assert np.array_equal(res, _bytes((kb - deq).reshape(2, 9, 3, 128).to(torch.float8_e4m3fn)))
    assert np.array_equal(OF.khat_nf4_g64(pk, s), deq.reshape(2, 9, 3, 128).to(torch.float16).float().numpy())
    assert (codes[1, 2, 1, 1] == 7).all() and s[1, 2, 1, 1] == np.float32(np.float16(1e-6))
