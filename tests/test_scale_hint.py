"""CPU tests of the fp16-exactness hint for per-channel scales (ffa_mi355x.decode.scales_exact_f16):
which values count as exact, and that the remembered answer follows the tensors' versions."""
import torch

from ffa_mi355x import decode as D


def test_exact_values():
    s = torch.tensor([1.0, 2.5, -3.0, 6.5e4, 2.0 ** -14, 0.0], dtype=torch.bfloat16)
    z = torch.tensor([0.5, -1.0, 2.0, -4.0, 2.0 ** -17, 0.0], dtype=torch.bfloat16)  # 2^-17: an fp16 subnormal
    assert D.scales_exact_f16(s, z)
    assert D.scales_exact_f16(s.half(), z.half())
    # bf16 values fp16 holds only as subnormals with fewer bits, or not at all
    assert not D.scales_exact_f16(torch.tensor([1.00781250 * 2.0 ** -20], dtype=torch.bfloat16), z[:1])
    assert not D.scales_exact_f16(torch.tensor([1.0e5], dtype=torch.bfloat16), z[:1])
    assert not D.scales_exact_f16(s[:1], torch.tensor([float("nan")], dtype=torch.bfloat16))
    # fp32 values need 11 significant bits at most
    assert D.scales_exact_f16(torch.tensor([1.5, 0.125]), torch.tensor([-2.0, 3.0]))
    assert not D.scales_exact_f16(torch.tensor([1.0 + 2.0 ** -12]), torch.tensor([0.0]))


def test_memo_follows_versions(monkeypatch):
    s = torch.tensor([1.0, 2.5], dtype=torch.bfloat16)
    z = torch.tensor([0.5, -1.0], dtype=torch.bfloat16)
    calls = []
    real = torch.equal
    monkeypatch.setattr(torch, "equal", lambda a, b: calls.append(1) or real(a, b))
    assert D.scales_exact_f16(s, z) and len(calls) == 2
    assert D.scales_exact_f16(s, z) and len(calls) == 2  # remembered
    s.mul_(2.0 ** -30)  # in place: the version changes, the answer too
    assert not D.scales_exact_f16(s, z) and len(calls) == 3
    z2 = z.clone()
    D.scales_exact_f16(s.clone().fill_(1.0), z2)
    n = len(calls)
    base = torch.ones(2, 3, dtype=torch.bfloat16)
    assert D.scales_exact_f16(base[0], z2[:1].expand(3).contiguous())
    assert len(calls) > n
