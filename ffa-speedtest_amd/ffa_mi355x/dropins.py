"""Access to the variant drop-in modules from other variants.

Each variant directory (ffa-q2fp8/, ffa-q2fp8-meanv/, ...) has its own `attn_kernel` package, as
in the reference, so one variant cannot import another's by package name.  The q2fp8 decode
drop-in is loaded here by path, once, under a name of its own.
"""
from __future__ import annotations

import importlib.util
import sys
import threading
from pathlib import Path

_ROOT = Path(__file__).resolve().parents[1]  # ffa-speedtest_amd/
_lock = threading.RLock()  # a drop-in may load another while it loads


def _load(name: str, path: Path):
    with _lock:
        mod = sys.modules.get(name)
        if mod is None:
            spec = importlib.util.spec_from_file_location(name, path)
            mod = importlib.util.module_from_spec(spec)
            sys.modules[name] = mod
            try:
                spec.loader.exec_module(mod)
            except BaseException:
                del sys.modules[name]
                raise
        return mod


def q2fp8_dropin():
    """ffa-q2fp8/attn_kernel/attn_kernel_v1210_fused_bsz_q2fp8.py (the q2fp8 decode drop-in)."""
    return _load("ffa_mi355x_q2fp8_dropin", _ROOT / "ffa-q2fp8" / "attn_kernel" / "attn_kernel_v1210_fused_bsz_q2fp8.py")
