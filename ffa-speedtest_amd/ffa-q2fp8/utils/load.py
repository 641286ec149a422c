"""Drop-in for ffa-q2fp8/utils/load.py: the recorded-layer loaders the benchmarks import
(`from utils.load import load_qkvh`, run_attn_bench_q2.py:15), reading every file with
torch.load(weights_only=True).  The text / dataset helpers of that module (tokenize_text and the
LongBench / BABILong readers) serve data capture, not the decode path, and are not provided."""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))  # ffa-speedtest_amd/
from ffa_mi355x.layer_data import load_attn_input, load_qkvh  # noqa: E402,F401

__all__ = ["load_attn_input", "load_qkvh"]
