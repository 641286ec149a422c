# attn_kernel_v1210_meanv_bsz_q2fp8.py -- MI355X drop-in.
# 2-bit quantized K with fp8 residual refinement + mean-V fallback; hand-written HIP for gfx950
# in libffa_mi355x.so (no Triton).
"""Drop-in for ffa-q2fp8-meanv/attn_kernel/attn_kernel_v1210_meanv_bsz_q2fp8.py.

`attn_forward_decode_quantized` keeps the reference signature, layouts, defaults and exception
types (reference :222-341; its checks are those of the q2fp8 decode).  The variant's semantics:

  * a prune block is pruned as in q2fp8 (every query row's coarse block maximum below its
    threshold), but a pruned block that holds tokens is approximated, not dropped: its softmax
    mass on the coarse scores, 2^(s - m) summed over its tokens, stays in the normalizer with the
    mean of V as its value (reference :109-119);
  * stage 2 merges kept blocks and approximated blocks separately and folds the latter with
    v_mean = mean over tokens of V, rounded to v.dtype (reference :156-202, :332);
  * return_skip_ratio gives the fraction of approximated blocks, approx.sum() / approx.numel()
    (reference :326-330).

Here the kernels are the q2fp8 decode's: stage 1 also writes, per query row and 512-token span,
the pruned tokens' maximum and mass; the merge folds them with v_mean.  v_mean comes from the
`ffa_v_mean` kernels (fp32 sums).

Extensions through **kwargs, as for the q2fp8 drop-in: block_table / seq_lens / T (paged pools,
ragged lengths), workspace; and v_mean=[B, HKV, V] to pass a mean the caller keeps (then V is not
read for it).

Block flags.  The reference keeps its mask_buf / approx_buf inside the call.  A workspace passed
here holds the q2fp8 decode's survivor mask: `workspace.mask_buf` = 1 for blocks refined exactly.
The reference's two flags follow from it with `ffa_mi355x.meanv.approx_flags(mask_buf, T, BS, SBS,
seq_lens)`: approx = pruned blocks that hold tokens (:117-119), and its mask_buf = exact or
approximated (:118, :151).
"""
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))  # ffa-speedtest_amd/
from ffa_mi355x import _native as _N  # noqa: E402
from ffa_mi355x.dropins import q2fp8_dropin  # noqa: E402
from ffa_mi355x.meanv import approx_ratio, value_mean  # noqa: E402

_q2 = q2fp8_dropin()
Q2FP8DecodeWorkspace = _q2.Q2FP8DecodeWorkspace
allocate_q2fp8_decode_workspace = _q2.allocate_q2fp8_decode_workspace

__all__ = ["attn_forward_decode_quantized", "Q2FP8DecodeWorkspace", "allocate_q2fp8_decode_workspace"]


def attn_forward_decode_quantized(
    q: torch.Tensor,           # [B, 1, HQ, K]
    k_q: torch.Tensor,         # [B, T, HKV, ceil(K / (8 / k_bits))], packed quantized ints
    k_scale: torch.Tensor,     # [B, HKV, K] (token dimension removed)
    k_zero: torch.Tensor,      # same shape as k_scale
    v: torch.Tensor,           # [B, T, HKV, V]
    k_residual: torch.Tensor | None = None,  # [B, T, HKV, K], fp8 residual
    k_bits: int = 2,
    scale: float = None,
    BS: int = 128,
    SBS: int | None = None,
    delta: float = 5.0,
    return_skip_ratio: bool = False,
    precomputed_threshold: torch.Tensor | None = None,
    use_fp8_residual: bool = True,
    **kwargs,
):
    given = kwargs.pop("v_mean", None)
    workspace = kwargs.pop("workspace", None)

    def v_mean_of(v_, layout, block_table, seq_lens, T):
        if given is not None:
            return given.contiguous()
        if layout == _N.LAYOUT_PAGED:
            return value_mean(v_, block_table=block_table, seq_lens=seq_lens, T=T)
        return value_mean(v_, seq_lens=seq_lens)

    ws, seq_lens, HKV, T, BS, SBS = _q2._decode(q, k_q, k_scale, k_zero, v, k_residual, k_bits, scale, BS, SBS, delta,
                                               precomputed_threshold, use_fp8_residual, workspace,
                                               v_mean_of=v_mean_of, **kwargs)
    o = ws.o
    if return_skip_ratio:
        return o, approx_ratio(ws.mask_buf, T, BS, SBS, seq_lens=seq_lens)
    return o
