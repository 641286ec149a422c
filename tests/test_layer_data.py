"""The recorded-layer loader (ffa-q2fp8/utils/load.py format) on files these tests write."""
import pickle

import pytest
import torch

from ffa_mi355x import layer_data as LD


def _write(root, n_layers=3, B=1, HQ=4, HKV=2, T=50, D=8, hidden=16):
    g = torch.Generator().manual_seed(0)
    layers = []
    for i in range(n_layers):
        t = dict(q_rope=torch.randn(B, HQ, T, D, generator=g), k_rope=torch.randn(B, HKV, T, D, generator=g),
                 q_unrope=torch.randn(B, HQ, T, D, generator=g), k_unrope=torch.randn(B, HKV, T, D, generator=g),
                 v=torch.randn(B, HKV, T, D, generator=g), h=torch.randn(B, T, hidden, generator=g))
        LD.save_layer(root, i, **{k: x.bfloat16() for k, x in t.items()})
        layers.append({k: x.bfloat16() for k, x in t.items()})
    return layers


def test_round_trip_and_truncation(tmp_path):
    layers = _write(tmp_path)
    got = list(LD.load_qkvh(tmp_path, start_layer=1, max_length=20))
    assert len(got) == 2
    for i, d in enumerate(got, start=1):
        assert set(d) == set(LD.LAYER_TENSORS)
        assert torch.equal(d["q_rope"], layers[i]["q_rope"][:, :, :20])
        assert torch.equal(d["v"], layers[i]["v"][:, :, :20])
        assert torch.equal(d["h"], layers[i]["h"][:, :20])  # [B, T, hidden]: the second-to-last axis
    full = next(LD.load_qkvh(tmp_path, max_length=None))
    assert full["k_rope"].shape[2] == 50
    assert LD.truncate_length(torch.zeros(3, 9), 4).shape == (3, 4)  # 2-D: the last axis
    assert LD.truncate_length(torch.zeros(9), 4).shape == (9,)


def test_layer_naming_and_range(tmp_path):
    _write(tmp_path, n_layers=2)
    with pytest.raises(ValueError):
        next(LD.load_qkvh(tmp_path, start_layer=2))
    (tmp_path / "layer_3").mkdir()  # a gap: layer_2 missing
    with pytest.raises(AssertionError):
        LD.layer_dirs(tmp_path)


def test_batch_and_decode_step_layout(tmp_path):
    layers = _write(tmp_path, n_layers=3, B=2)
    q, k, v = LD.load_layer_batch(tmp_path, [1, 2], torch.float16, max_length=40)
    assert q.shape == (4, 4, 40, 8) and q.dtype == torch.float16
    assert torch.equal(q[2:], layers[2]["q_rope"][:, :, :40].half())
    qd, kd, vd = LD.decode_step_inputs(q, k, v, L=33)
    assert qd.shape == (4, 4, 8) and kd.shape == (4, 33, 2, 8) and vd.shape == (4, 33, 2, 8)
    assert torch.equal(qd, q[:, :, 32]) and torch.equal(kd[:, 5, 1], k[:, 1, 5]) and torch.equal(vd[:, 32], v[:, :, 32])
    with pytest.raises(RuntimeError):
        LD.load_layer_batch(tmp_path, [2, 3], torch.float16)
    with pytest.raises(ValueError):
        LD.decode_step_inputs(q, k, v, L=41)


class _Payload:
    def __reduce__(self):
        return (print, ("executed",))


def test_files_are_loaded_as_tensors_only(tmp_path, capsys):
    """A layer file holding a pickled call is refused, not executed (weights_only loading)."""
    _write(tmp_path, n_layers=1)
    with open(tmp_path / "layer_0" / "v.pt", "wb") as f:
        pickle.dump(_Payload(), f, protocol=2)
    with pytest.raises(pickle.UnpicklingError):
        next(LD.load_qkvh(tmp_path))
    assert "executed" not in capsys.readouterr().out


def test_drop_in_module_names(tmp_path):
    import importlib.util

    from ffa_mi355x.dropins import _ROOT

    spec = importlib.util.spec_from_file_location("ffa_q2fp8_utils_load", _ROOT / "ffa-q2fp8" / "utils" / "load.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    _write(tmp_path, n_layers=1)
    assert mod.load_qkvh is LD.load_qkvh and mod.load_attn_input is LD.load_attn_input
    torch.save({"q": torch.ones(2)}, tmp_path / "layer_0" / "attn_input.pt")
    assert torch.equal(next(mod.load_attn_input(tmp_path))["q"], torch.ones(2))
