"""CPU pins of the producer oracle (K projection + RoPE, oracle/producer.py).

The reference has no fixtures for its producer; these checks tie the oracle to
what the mathematics fixes: exact integer GEMMs, RoPE as a rotation (identity at
angle 0, composition of angles, norm preservation) and the reference's cos/sin
cache with its interleaved-pair quirk (ffa-q2fp8/fused_kproj_rope_q2fp8.py:10-37).
"""
import numpy as np
import torch

from oracle import numerics as NM
from oracle import producer as OP


def _rot_tables(angles):
    """cos/sin [T, D] with both elements of each pair (2i, 2i+1) at the same angle."""
    return np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)


def test_linear_exact_on_integer_inputs():
    rng = np.random.default_rng(0)
    h = rng.integers(-8, 9, (2, 5, 64)).astype(np.float32)
    w = rng.integers(-8, 9, (48, 64)).astype(np.float32)
    bias = rng.integers(-8, 9, (48,)).astype(np.float32)
    exact = (h.astype(np.int64) @ w.astype(np.int64).T + bias.astype(np.int64)).astype(np.float32)
    # small integers: the fp32 result is exact; the bf16 result is that value rounded once
    got = OP.linear(h, w, bias, "fp32")
    assert np.array_equal(got, exact)
    got_bf16 = OP.linear(h, w, bias, "bf16")
    assert np.array_equal(got_bf16, NM.round_bf16(exact))


def test_linear_close_to_torch_fp32():
    rng = np.random.default_rng(1)
    h = rng.standard_normal((3, 7, 256)).astype(np.float32)
    w = (rng.standard_normal((128, 256)) * 0.02).astype(np.float32)
    got = OP.linear(h, w, None, "fp32")
    ref = torch.nn.functional.linear(torch.from_numpy(h), torch.from_numpy(w)).numpy()
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max() + 1e-6


def test_rope_zero_angle_is_identity():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 128)).astype(np.float32)
    cos, sin = np.ones((4, 128), np.float32), np.zeros((4, 128), np.float32)
    assert np.array_equal(OP.apply_rope(x, cos, sin, "fp32"), x)


def test_rope_is_a_rotation_of_each_pair():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 128)).astype(np.float64)
    a = rng.uniform(-3, 3, (6, 64))
    b = rng.uniform(-3, 3, (6, 64))
    ang_a, ang_b = np.repeat(a, 2, axis=1), np.repeat(b, 2, axis=1)  # pair (2i, 2i+1) shares angle i
    ca, sa = _rot_tables(ang_a)
    cb, sb = _rot_tables(ang_b)
    cab, sab = _rot_tables(ang_a + ang_b)
    xf = x.astype(np.float32)
    once = OP.apply_rope(xf, ca, sa, "fp32")
    twice = OP.apply_rope(once, cb, sb, "fp32")
    direct = OP.apply_rope(xf, cab, sab, "fp32")
    assert np.abs(twice - direct).max() < 1e-5
    # rotation keeps the norm of every pair and turns (x0, x1) by +angle: x0' = x0 cos - x1 sin
    n0 = xf[:, 0::2] ** 2 + xf[:, 1::2] ** 2
    n1 = once[:, 0::2] ** 2 + once[:, 1::2] ** 2
    assert np.abs(n0 - n1).max() < 1e-5 * n0.max()
    assert np.allclose(once[:, 0::2], xf[:, 0::2] * np.cos(a) - xf[:, 1::2] * np.sin(a), atol=1e-5)
    assert np.allclose(once[:, 1::2], xf[:, 1::2] * np.cos(a) + xf[:, 0::2] * np.sin(a), atol=1e-5)


def test_rope_reference_cache_pairs_use_two_frequencies():
    """With the reference cache (cos/sin of cat([f, f]), :19-23) element 2i takes angle f[2i mod D/2] and
    2i+1 takes f[(2i+1) mod D/2]: the pair is not a rotation (the reference's quirk, reproduced)."""
    import fused_kproj_rope_q2fp8 as FK

    T, D = 5, 128
    cos, sin = FK.build_rope_cache(T, D, base=500000.0, device=torch.device("cpu"), dtype=torch.float32)
    inv = 1.0 / (500000.0 ** (np.arange(0, D, 2, dtype=np.float64) / D))
    ang = np.arange(T)[:, None] * np.concatenate([inv, inv])[None, :]
    assert np.allclose(cos.numpy(), np.cos(ang), atol=1e-6) and np.allclose(sin.numpy(), np.sin(ang), atol=1e-6)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((T, D)).astype(np.float32)
    out = OP.apply_rope(x, cos.numpy(), sin.numpy(), "fp32")
    want0 = x[:, 0::2] * np.cos(ang[:, 0::2]) - x[:, 1::2] * np.sin(ang[:, 0::2])
    want1 = x[:, 1::2] * np.cos(ang[:, 1::2]) + x[:, 0::2] * np.sin(ang[:, 1::2])
    assert np.allclose(out[:, 0::2], want0, atol=1e-5) and np.allclose(out[:, 1::2], want1, atol=1e-5)
    # the pair norm changes for t > 0: not a rotation
    n0 = x[1:, 0::2] ** 2 + x[1:, 1::2] ** 2
    n1 = out[1:, 0::2] ** 2 + out[1:, 1::2] ** 2
    assert np.abs(n0 - n1).max() > 1e-3


def test_rope_rounds_each_op_in_the_output_dtype():
    """bf16 promotion: out = bf16(bf16(x cos) + bf16(rot(x) sin)), as torch evaluates x*cos + rot*sin in bf16."""
    rng = np.random.default_rng(5)
    x = NM.round_bf16(rng.standard_normal((3, 128)).astype(np.float32))
    c = NM.round_bf16(rng.uniform(-1, 1, (3, 128)).astype(np.float32))
    s = NM.round_bf16(rng.uniform(-1, 1, (3, 128)).astype(np.float32))
    got = OP.apply_rope(x, c, s, "bf16")
    xt, ct, st = (torch.from_numpy(a).to(torch.bfloat16) for a in (x, c, s))
    rot = torch.stack((-xt[..., 1::2], xt[..., 0::2]), dim=-1).flatten(-2)
    ref = (xt * ct + rot * st).float().numpy()
    assert np.array_equal(got, ref)
