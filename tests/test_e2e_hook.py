"""The HF attention hook's guards (CPU): it takes the layer of the cache update that ran last on the
thread, checks it against the module's layer index and clears it, so a model run without a
Q2FP8Cache (or after another layer's update) raises instead of decoding over a stale layer."""
import importlib.util
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

E2E = Path(__file__).resolve().parents[1] / "ffa-speedtest_amd" / "ffa-q2fp8" / "e2e" / "q2fp8_cache.py"


def _load():
    spec = importlib.util.spec_from_file_location("q2fp8_cache_cpu", E2E)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _module(layer_idx, **settings):
    return SimpleNamespace(layer_idx=layer_idx, config=SimpleNamespace(attn_settings=settings))


def test_attention_without_a_cache_update_raises():
    C = _load()
    q = torch.zeros(1, 8, 1, 128)
    C._current.entry = None
    with pytest.raises(RuntimeError, match="needs a Q2FP8Cache"):
        C.ffa_q2fp8_attention(_module(0), q, q, q, None)


def test_attention_of_another_layer_raises_and_clears():
    C = _load()
    q = torch.zeros(1, 8, 1, 128)
    C._current.entry = (0, C.Q2FP8PagedLayer(1, 128))
    with pytest.raises(RuntimeError, match="layer 1 after the cache update of layer 0"):
        C.ffa_q2fp8_attention(_module(1), q, q, q, None)
    assert C._current.entry is None
    with pytest.raises(RuntimeError, match="needs a Q2FP8Cache"):  # the stale entry is gone
        C.ffa_q2fp8_attention(_module(0), q, q, q, None)


def test_pattern_layers_must_be_a_list():
    C = _load()
    q = torch.zeros(1, 8, 1, 128)
    C._current.entry = (0, C.Q2FP8PagedLayer(1, 128))
    with pytest.raises(TypeError, match="pattern_layers"):
        C.ffa_q2fp8_attention(_module(0, pattern_layers=3), q, q, q, None)
