"""Module resolution as the reference's benchmark scripts see it, with the drop-in directories on PYTHONPATH.

The reference's ffa-q2fp8/ holds namespace directories (no __init__.py): `utils/` with bench.py,
cache.py, flash.py, load.py, plot.py and `attn_kernel/` with the decode modules.  Its scripts run
from that directory (first on sys.path) and import `utils.bench`, `utils.cache`, `utils.load`, ...
(run_attn_bench_q2.py:12-16, run_attn_bench_q2_cudagraph.py:13-20).  With the drop-in directories
on PYTHONPATH, `utils.load` and the `attn_kernel` decode modules must come from the drop-in and
every other `utils` / `attn_kernel` module from the reference's copy beside the script.  The tree
below is a stand-in of that shape with stub modules (no reference file is read or run)."""
import json
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "ffa-speedtest_amd"
DROPIN = PKG / "ffa-q2fp8"

SCRIPT = r'''
import importlib.util, json, sys
from utils.bench import benchmark          # the reference's stub (run_attn_bench_q2.py:12)
from utils.cache import dtype_key           # (:13)
from utils.plot import plot_speed_curve      # relative import of .cache inside (utils/plot.py:7)
names = ["utils.bench", "utils.cache", "utils.flash", "utils.plot", "utils.load",
         "attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8",
         "attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8_cudagraph",
         "attn_kernel.attn_kernel_v0000_other"]
out = {n: importlib.util.find_spec(n).origin for n in names}
out["benchmark"] = benchmark()
out["plot"] = plot_speed_curve()
print(json.dumps(out))
'''


def _reference_shaped_tree(root: Path) -> Path:
    d = root / "ffa-q2fp8"
    (d / "utils").mkdir(parents=True)
    (d / "attn_kernel").mkdir()
    (d / "utils" / "bench.py").write_text("def benchmark():\n    return 'ref-bench'\n")
    (d / "utils" / "cache.py").write_text("def dtype_key():\n    return 'k'\n\ndef to_k_str(x):\n    return 'ref-cache'\n")
    (d / "utils" / "flash.py").write_text("def flash_attn_compute():\n    pass\n")
    (d / "utils" / "plot.py").write_text("from .cache import to_k_str\n\ndef plot_speed_curve():\n    return to_k_str(0)\n")
    (d / "utils" / "load.py").write_text("raise RuntimeError('the reference loader must not be imported')\n")
    for m in ("attn_kernel_v1210_fused_bsz_q2fp8", "attn_kernel_v1210_fused_bsz_q2fp8_cudagraph"):
        (d / "attn_kernel" / f"{m}.py").write_text("raise RuntimeError('the reference kernel must not be imported')\n")
    (d / "attn_kernel" / "attn_kernel_v0000_other.py").write_text("X = 1\n")
    (d / "run_probe.py").write_text(SCRIPT)
    return d


def test_reference_scripts_resolve_their_modules(tmp_path):
    ref = _reference_shaped_tree(tmp_path)
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([str(DROPIN), str(PKG)])  # the drop-in, then the package
    r = subprocess.run([sys.executable, "run_probe.py"], cwd=ref, env=env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stderr
    got = json.loads(r.stdout.strip().splitlines()[-1])
    for n in ("bench", "cache", "flash", "plot"):
        assert Path(got[f"utils.{n}"]) == ref / "utils" / f"{n}.py"
    assert Path(got["utils.load"]) == DROPIN / "utils" / "load.py"
    for m in ("attn_kernel_v1210_fused_bsz_q2fp8", "attn_kernel_v1210_fused_bsz_q2fp8_cudagraph"):
        assert Path(got[f"attn_kernel.{m}"]) == DROPIN / "attn_kernel" / f"{m}.py"
    assert Path(got["attn_kernel.attn_kernel_v0000_other"]) == ref / "attn_kernel" / "attn_kernel_v0000_other.py"
    assert got["benchmark"] == "ref-bench" and got["plot"] == "ref-cache"


def test_dropin_loader_imports_under_the_recipe(tmp_path):
    """`from utils.load import load_qkvh` executes the drop-in loader, not the reference's."""
    ref = _reference_shaped_tree(tmp_path)
    (ref / "run_load.py").write_text("from utils.load import load_qkvh\nprint(load_qkvh.__module__)\n")
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([str(DROPIN), str(PKG)])
    r = subprocess.run([sys.executable, "run_load.py"], cwd=ref, env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip().splitlines()[-1] == "ffa_mi355x.layer_data"
