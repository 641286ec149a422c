"""Write fp8_from_fp16.npz: torch's fp16 -> float8_e4m3fn / float8_e5m2 casts of all 65536 fp16 bit patterns.

These are library outputs (torch's casts), the number-format ground truth
the reference relies on for its residual (ffa-q2fp8/run_attn_bench_q2.py:88).
Run: python tests/golden/make_fp8_tables.py
"""
from pathlib import Path

import numpy as np
import torch

h = torch.from_numpy(np.arange(65536, dtype=np.uint16).view(np.int16)).view(torch.float16).float()
out = {
    "e4m3fn": h.to(torch.float8_e4m3fn).view(torch.uint8).numpy(),
    "e5m2": h.to(torch.float8_e5m2).view(torch.uint8).numpy(),
}
np.savez_compressed(Path(__file__).with_name("fp8_from_fp16.npz"), **out)
print({k: v.shape for k, v in out.items()})
