# attn_kernel_v1210_fused_bsz_q2fp8_cudagraph.py -- MI355X drop-in.
"""Graph-captured q2fp8 decode (drop-in for
ffa-q2fp8/attn_kernel/attn_kernel_v1210_fused_bsz_q2fp8_cudagraph.py:11-183).

`CUDAGraphDecodeRunnerQ2FP8` keeps the reference constructor, `replay` /
`__call__` / `replay_only` and `output`.  The decode's scratch (output,
partials, mask, thresholds) is one caller-owned workspace allocated before
capture, and the C ABI neither allocates nor synchronises, so the captured
graph holds only the two decode launches (plus a dtype cast of the external
threshold when it is not fp32).  The survivor mask is written by every
replay, so `return_skip_ratio=True` reads it instead of running the decode
again.  Paged caches pass block_table / seq_lens / T through **kwargs as in
`attn_forward_decode_quantized`.
"""
from __future__ import annotations

from typing import Optional

import torch

from .attn_kernel_v1210_fused_bsz_q2fp8 import (
    allocate_q2fp8_decode_workspace,
    attn_forward_decode_quantized,
)
from ffa_mi355x.decode import skip_ratio_of

__all__ = ["CUDAGraphDecodeRunnerQ2FP8"]


def _static_copy(t: Optional[torch.Tensor], device) -> Optional[torch.Tensor]:
    if t is None:
        return None
    s = torch.empty_like(t, device=device)
    s.copy_(t)
    return s


class CUDAGraphDecodeRunnerQ2FP8:
    """Capture one decode step on static buffers and replay it."""

    def __init__(
        self,
        q: torch.Tensor,
        k_q: torch.Tensor,
        k_scale: torch.Tensor,
        k_zero: torch.Tensor,
        v: torch.Tensor,
        *,
        k_residual: Optional[torch.Tensor] = None,
        precomputed_threshold: Optional[torch.Tensor] = None,
        k_bits: int = 2,
        scale: Optional[float] = None,
        BS: int = 128,
        SBS: Optional[int] = None,
        delta: float = 5.0,
        use_fp8_residual: bool = True,
        warmup: int = 2,
        **kwargs,
    ) -> None:
        if not torch.cuda.is_available():
            raise RuntimeError("CUDA is required for CUDAGraph capture.")
        if q.device.type != "cuda":
            raise ValueError("q must be a CUDA tensor.")
        if use_fp8_residual and k_residual is None:
            raise ValueError("use_fp8_residual=True requires k_residual")
        self._device = q.device
        self._use_res = use_fp8_residual
        self._use_ext_th = precomputed_threshold is not None
        self._BS = BS
        self._SBS = BS if SBS is None else SBS
        self._args = dict(k_bits=k_bits, scale=scale, BS=BS, SBS=SBS, delta=delta, use_fp8_residual=use_fp8_residual)

        dev = self._device
        self._q = _static_copy(q, dev)
        self._k_q = _static_copy(k_q, dev)
        self._k_scale = _static_copy(k_scale, dev)
        self._k_zero = _static_copy(k_zero, dev)
        self._v = _static_copy(v, dev)
        self._k_res = _static_copy(k_residual, dev) if use_fp8_residual else None
        self._th = _static_copy(precomputed_threshold, dev)
        # paged-cache extras: the page table and lengths are inputs too
        self._kw = {}
        for name in ("block_table", "seq_lens"):
            if kwargs.get(name) is not None:
                self._kw[name] = _static_copy(kwargs[name].to(device=dev, dtype=torch.int32), dev)
        # The captured grid and scratch are sized for T: the caller's, else the block table's
        # capacity, so replays may grow seq_lens up to the table's end (a decode loop appends a
        # token per step); lengths past T would be clamped to T.
        if kwargs.get("T") is not None:
            self._kw["T"] = int(kwargs["T"])
        elif "block_table" in self._kw:
            self._kw["T"] = int(self._kw["block_table"].shape[1]) * 64

        self._ws = allocate_q2fp8_decode_workspace(self._q, self._k_q, self._v, BS=BS, SBS=SBS, **self._kw)
        for _ in range(max(1, warmup)):
            self._launch()
        torch.cuda.synchronize(dev)

        self._graph = torch.cuda.CUDAGraph()
        self._pool = torch.cuda.graphs.graph_pool_handle()
        with torch.cuda.graph(self._graph, pool=self._pool):
            self._out = self._launch()

    def _launch(self) -> torch.Tensor:
        return attn_forward_decode_quantized(
            q=self._q, k_q=self._k_q, k_scale=self._k_scale, k_zero=self._k_zero, v=self._v,
            k_residual=self._k_res, return_skip_ratio=False, precomputed_threshold=self._th,
            workspace=self._ws, **self._args, **self._kw)

    @property
    def output(self) -> torch.Tensor:
        return self._out

    def replay(
        self,
        q: torch.Tensor,
        k_q: torch.Tensor,
        k_scale: torch.Tensor,
        k_zero: torch.Tensor,
        v: torch.Tensor,
        *,
        k_residual: Optional[torch.Tensor] = None,
        precomputed_threshold: Optional[torch.Tensor] = None,
        return_skip_ratio: bool = False,
        **kwargs,
    ):
        if q.device != self._device:
            raise ValueError("q must be on the same device as the captured graph.")
        if self._use_res and k_residual is None:
            raise ValueError("k_residual is required for this captured graph.")
        if self._use_ext_th and precomputed_threshold is None:
            raise ValueError("precomputed_threshold is required for this captured graph.")
        self._q.copy_(q)
        self._k_q.copy_(k_q)
        self._k_scale.copy_(k_scale)
        self._k_zero.copy_(k_zero)
        self._v.copy_(v)
        if self._use_res:
            self._k_res.copy_(k_residual)
        if self._use_ext_th:
            self._th.copy_(precomputed_threshold)
        for name in ("block_table", "seq_lens"):
            if kwargs.get(name) is not None:
                if name not in self._kw:
                    raise ValueError(f"{name} was not given at capture")
                self._kw[name].copy_(kwargs[name])
        self._graph.replay()
        if not return_skip_ratio:
            return self._out
        lens = self._kw.get("seq_lens")
        return self._out, skip_ratio_of(self._ws.mask_buf, lens, self._BS, self._SBS)

    __call__ = replay

    def replay_only(self) -> torch.Tensor:
        """Replay without updating static inputs."""
        self._graph.replay()
        return self._out
