"""Recorded attention inputs: the `layer_data/layer_i/*.pt` format of the reference's benchmarks.

Format (written by attn_analysis/dump_qkvh.py:50-60, read by ffa-q2fp8/utils/load.py:29-72):
one directory per decoder layer, `layer_0`, `layer_1`, ... (consecutive), each holding

    h.pt         [B, T, hidden]   the attention input hidden states
    q_unrope.pt  [B, HQ, T, D]    q before RoPE
    k_unrope.pt  [B, HKV, T, D]   k before RoPE
    v.pt         [B, HKV, T, D]
    q_rope.pt    [B, HQ, T, D]    q after RoPE
    k_rope.pt    [B, HKV, T, D]   k after RoPE

(or a single attn_input.pt per layer for `load_attn_input`).  Every file is read with
`torch.load(..., weights_only=True)`: tensors only, nothing in a file is executed.

`load_layer_batch` and `decode_step_inputs` turn the layers into one decode step as the
benchmarks do (ffa-q2fp8/run_attn_bench_q2.py:66-74, 146-170, 209-213): layers are stacked along
the batch, the query is the token at position L - 1 and K / V are the first L tokens, transposed
to the decode's [B, T, H, D] layout.
"""
from __future__ import annotations

from pathlib import Path
from typing import Iterator, Optional

import torch

LAYER_TENSORS = ("q_rope", "k_rope", "q_unrope", "k_unrope", "v", "h")


def layer_dirs(load_dir) -> list[Path]:
    """The `layer_<i>` subdirectories of load_dir in layer order; they must be layer_0 .. layer_{n-1}."""
    root = Path(load_dir)
    dirs = [x for x in root.iterdir() if x.is_dir() and x.name.startswith("layer")]
    try:
        dirs.sort(key=lambda x: int(x.name.split("_")[1]))
    except (IndexError, ValueError):
        raise AssertionError("Layer directories must be named layer_0, layer_1, ...") from None
    assert [p.name for p in dirs] == [f"layer_{i}" for i in range(len(dirs))], \
        "Layer directories must be named layer_0, layer_1, ..."
    return dirs


def _load(path: Path, device) -> torch.Tensor:
    return torch.load(path, weights_only=True, map_location=device)


def truncate_length(t: torch.Tensor, max_length: Optional[int]) -> torch.Tensor:
    """Cut the sequence axis to max_length (None or <= 0: unchanged): the second-to-last axis of a
    tensor of 3 or more dims, the last axis of a 2-D one (ffa-q2fp8/utils/load.py:56-63)."""
    if max_length is None or max_length <= 0:
        return t
    if t.dim() >= 3:
        return t[..., :max_length, :]
    if t.dim() == 2:
        return t[:, :max_length]
    return t


def load_attn_input(load_dir, device="cpu") -> Iterator:
    """Each layer's attn_input.pt, in layer order (ffa-q2fp8/utils/load.py:7-27)."""
    for d in layer_dirs(load_dir):
        yield _load(d / "attn_input.pt", device)


def load_qkvh(load_dir, device="cpu", start_layer: int = 0, max_length: Optional[int] = None) -> Iterator[dict]:
    """Dicts of q_rope, k_rope, q_unrope, k_unrope, v and h, one per layer from start_layer on, each
    cut to max_length tokens (ffa-q2fp8/utils/load.py:29-72)."""
    dirs = layer_dirs(load_dir)
    if not (0 <= start_layer < len(dirs)):
        raise ValueError(f"start_layer must be in [0, {len(dirs) - 1}], got {start_layer}")
    for d in dirs[start_layer:]:
        yield {name: truncate_length(_load(d / f"{name}.pt", device), max_length) for name in LAYER_TENSORS}


def save_layer(save_dir, layer_idx: int, **tensors: torch.Tensor) -> Path:
    """Write one layer in the format above (any subset of LAYER_TENSORS); returns its directory."""
    unknown = set(tensors) - set(LAYER_TENSORS) - {"attn_input"}
    if unknown:
        raise ValueError(f"unknown layer tensors {sorted(unknown)}; expected {LAYER_TENSORS}")
    d = Path(save_dir) / f"layer_{int(layer_idx)}"
    d.mkdir(parents=True, exist_ok=True)
    for name, t in tensors.items():
        torch.save(t.detach().contiguous(), d / f"{name}.pt")
    return d


def load_layer_batch(load_dir, layer_indices, dtype: torch.dtype, max_length: Optional[int] = None, device="cpu"):
    """q_rope, k_rope, v of consecutive layers stacked along the batch axis and cast to dtype
    (ffa-q2fp8/run_attn_bench_q2.py:146-170): [B * n, HQ, T, D], [B * n, HKV, T, D] x 2."""
    layer_indices = list(layer_indices)
    if layer_indices != list(range(layer_indices[0], layer_indices[0] + len(layer_indices))):
        raise ValueError("layer_indices must be consecutive")
    it = load_qkvh(load_dir, device=device, start_layer=layer_indices[0], max_length=max_length)
    qs, ks, vs = [], [], []
    for i, layer in enumerate(layer_indices):
        try:
            data = next(it)
        except StopIteration:
            raise RuntimeError(f"Not enough layers to form batch size {len(layer_indices)} starting from "
                               f"layer_{layer_indices[0]}. Only found {i} layers.") from None
        qs.append(data["q_rope"])
        ks.append(data["k_rope"])
        vs.append(data["v"])
    return (torch.cat(qs, 0).to(dtype=dtype), torch.cat(ks, 0).to(dtype=dtype), torch.cat(vs, 0).to(dtype=dtype))


def decode_step_inputs(q_rope: torch.Tensor, k_rope: torch.Tensor, v: torch.Tensor, L: Optional[int] = None):
    """The decode step at length L (default: every recorded token): q [B, HQ, D] of the token at
    L - 1, k and v [B, L, HKV, D] (ffa-q2fp8/run_attn_bench_q2.py:66-74, 209-213)."""
    B, HQ, T, D = q_rope.shape
    if k_rope.shape[0] != B or v.shape[0] != B or k_rope.shape[2] != T or v.shape[2] != T or v.shape[1] != k_rope.shape[1]:
        raise ValueError(f"q_rope {tuple(q_rope.shape)}, k_rope {tuple(k_rope.shape)} and v {tuple(v.shape)} "
                         "must be [B, H, T, D] with one T and one KV head count")
    L = T if L is None else int(L)
    if not 1 <= L <= T:
        raise ValueError(f"L must be in [1, {T}], got {L}")
    q = q_rope[:, :, L - 1, :].contiguous()
    k = k_rope[:, :, :L, :].permute(0, 2, 1, 3).contiguous()
    vv = v[:, :, :L, :].permute(0, 2, 1, 3).contiguous()
    return q, k, vv
