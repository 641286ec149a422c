# attn_kernel_v1210_fused_bsz_q2fp8.py -- MI355X drop-in (mean-V variant's copy).
"""Drop-in for ffa-q2fp8-meanv/attn_kernel/attn_kernel_v1210_fused_bsz_q2fp8.py, which is the same
module as ffa-q2fp8's: this re-exports the q2fp8 drop-in (ffa-q2fp8/attn_kernel/...)."""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))  # ffa-speedtest_amd/
from ffa_mi355x.dropins import q2fp8_dropin  # noqa: E402

_m = q2fp8_dropin()
attn_forward_decode_quantized = _m.attn_forward_decode_quantized
Q2FP8DecodeWorkspace = _m.Q2FP8DecodeWorkspace
allocate_q2fp8_decode_workspace = _m.allocate_q2fp8_decode_workspace

__all__ = ["attn_forward_decode_quantized", "Q2FP8DecodeWorkspace", "allocate_q2fp8_decode_workspace"]
