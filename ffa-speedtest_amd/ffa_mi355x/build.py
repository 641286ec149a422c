"""Build libffa_mi355x.so (all HIP sources for gfx950) in-tree.

Usage: python -m ffa_mi355x.build   (from ffa-speedtest_amd/), or call build().
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent  # ffa-speedtest_amd/
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
LIB_NAME = "libffa_mi355x.so"
LIB_PATH = PKG_DIR / LIB_NAME

SOURCES = ["q2fp8_decode.hip", "kfmt_decode.hip", "q2_quant.hip", "kfmt_quant.hip", "value_mean.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 ops are disabled on purpose (see the kernels' build notes)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in arch VGPRs rather than AGPRs: the decode kernel then needs 196 registers
    # instead of 228 and no v_accvgpr_read copies (measured 2 % faster on the config-2 decode)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libffa_mi355x.so)")


def build(verbose: bool = False, jobs: int = 4, extra_flags=(), lib_path: Path = LIB_PATH) -> Path:
    """Compile every HIP source for gfx950 and link the shared library (extra_flags / lib_path: a
    variant build, such as the timeline build of ffa_mi355x.timeline)."""
    hipcc = _hipcc()
    lib_path = Path(lib_path)
    objdir = PKG_DIR / ("_obj" if lib_path == LIB_PATH else "_obj_" + lib_path.stem)
    objdir.mkdir(exist_ok=True)
    procs = []
    objs = []
    for src in SOURCES:
        obj = objdir / (Path(src).stem + ".o")
        objs.append(obj)
        cmd = [hipcc, *HIPCC_FLAGS, *extra_flags, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        if len(procs) >= jobs:
            _wait(procs.pop(0))
    for pr in procs:
        _wait(pr)
    tmp = lib_path.with_suffix(".so.tmp")
    cmd = [hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    _run(cmd)
    os.replace(tmp, lib_path)
    return lib_path


def _wait(item):
    src, p = item
    out, _ = p.communicate()
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{out}")


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed: {' '.join(cmd)}\n{r.stdout}")


if __name__ == "__main__":
    p = build(verbose="-v" in sys.argv)
    print(p)
