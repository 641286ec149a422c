"""Per-wave timeline of a decode's stage 1 (a diagnostic; the library never loads it).

    python -m ffa_mi355x.timeline build                      # CPU: compile the timeline library
    python -m ffa_mi355x.timeline run --workload config2     # GPU: benchmark config 2's stage 1
    python -m ffa_mi355x.timeline run --workload config1     # GPU: benchmark config 1's step
    python -m ffa_mi355x.timeline run --workload config2ref  # GPU: config 2's stage 1, reference layout

`build` compiles every HIP source with -DFFA_TIMELINE into libffa_mi355x_timeline.so beside the
library.  In that build each wave of the q2 and other-format decoders reads the 100 MHz constant
clock (s_memrealtime) at 13 points of its path and stores them, with the kept chunks it refined and
its hardware ids, into a buffer set through ffa_debug_set_timeline(_kfmt).  `run` replays a HIP
graph of 24 rotated stage-1 launches (config 2, as bench.py times its roofline) or steps (config 1),
keeps the stamps of the last launch and prints, in microseconds from the first wave's start, the
median / 90th percentile / maximum of every point, and (config 2 in either layout) the workgroups'
end times by kept chunks per workgroup, per CU and per XCD.  The stamps are scalar-memory reads that share lgkmcnt
with LDS traffic, so the timeline build runs a little slower than the library.
"""
from __future__ import annotations

import argparse
import ctypes
import sys
from pathlib import Path

import numpy as np

from . import build as B

LIB = B.PKG_DIR / "libffa_mi355x_timeline.so"
POINTS = {
    "config2": ["entry", "page ids in", "operands built", "pages scored", "probe barrier", "published",
                "chunk loads issued", "refined", "softmax", "P.V", "exact pass done", "final barrier", "end"],
    "config1": ["entry", "loads issued", "operands built", "pages scored", "probe barrier", "exact pass start",
                "chunk loads issued", "refined", "softmax", "P.V", "exact pass done", "final barrier", "end"],
    "config2ref": ["entry", "-", "operands built", "pages scored", "probe barrier", "published",
                   "chunk loads issued", "refined", "softmax", "P.V", "exact pass done", "final barrier", "end"],
}
# points recorded inside a wave's exact pass (only waves that refine a chunk have them)
EXACT_POINTS = {"config2": range(6, 10), "config1": range(5, 10), "config2ref": range(6, 10)}


def build_lib(verbose: bool = False) -> Path:
    return B.build(verbose=verbose, extra_flags=("-DFFA_TIMELINE",), lib_path=LIB)


def _graph(step, R):
    import torch

    for r in range(R):
        step(r)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        step(0)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=stream):
        for r in range(R):
            step(r)
    torch.cuda.synchronize()
    for _ in range(5):
        g.replay()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(20):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (20 * R)


def _config2(N, R=24):
    import torch

    from . import synth
    from .decode import DecodeWorkspace
    from .paged import PagedQ2Cache

    dev = torch.device("cuda:0")
    T, HKV = 32768, 8
    q, k, v = synth.attention_inputs(B=1, T=T, HQ=32, HKV=HKV, D=128, seed=0, n_heavy=16, cos=0.8)
    npg = -(-T // 64)
    bt0, _ = synth.page_tables([T], seed=0)
    cache = PagedQ2Cache(npg * R, HKV, dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    bts = [(bt0 + r * npg).to(dev) for r in range(R)]
    for bt in bts:
        cache.append(k.to(dev), v.to(dev), pos, bt)
    qd = q.to(dev)
    ws = DecodeWorkspace(1, 32, HKV, T, 64, 64, dev, torch.bfloat16)
    buf = torch.zeros(64 * HKV * 4 * 16, dtype=torch.int64, device=dev)
    N.lib().ffa_debug_set_timeline.argtypes = [ctypes.c_void_p]
    assert N.lib().ffa_debug_set_timeline(ctypes.c_void_p(buf.data_ptr())) == 0
    us = _graph(lambda r: cache.decode(qd, bts[r], None, T=T, BS=64, SBS=64, delta=5.0, workspace=ws,
                                       stage="stage1"), R)
    return us, buf.cpu().numpy().reshape(-1, 16).astype(np.int64), "stage 1 per launch"


def _config2ref(N, R=24):
    import torch

    from . import quant, synth
    from .decode import DecodeWorkspace, run_decode

    dev = torch.device("cuda:0")
    T, HKV = 32768, 8
    q, k, v = synth.attention_inputs(B=1, T=T, HQ=32, HKV=HKV, D=128, seed=0, n_heavy=16, cos=0.8)
    qd, vd = q.to(dev), v.to(dev)
    kq, ks, kz, kr = quant.quantize_per_channel(k.to(dev), torch.float8_e5m2)
    copies = [(kq.clone(), kr.clone(), vd.clone()) for _ in range(R)]
    ws = DecodeWorkspace(1, 32, HKV, T, 64, 64, dev, qd.dtype)
    buf = torch.zeros(64 * HKV * 4 * 16, dtype=torch.int64, device=dev)
    N.lib().ffa_debug_set_timeline.argtypes = [ctypes.c_void_p]
    assert N.lib().ffa_debug_set_timeline(ctypes.c_void_p(buf.data_ptr())) == 0

    def step(r):
        kq_, kr_, v_ = copies[r]
        run_decode(q=qd, k_q=kq_, k_scale=ks, k_zero=kz, v=v_, k_residual=kr_, layout=N.LAYOUT_CONTIG,
                   scale_mode=N.SCALE_CHANNEL, T=T, HKV=HKV, scale=128 ** -0.5, BS=64, SBS=64, delta=5.0,
                   use_res=True, workspace=ws, stage="stage1")

    us = _graph(step, R)
    return us, buf.cpu().numpy().reshape(-1, 16).astype(np.int64), "stage 1 per launch"


def _config1(N, R=24):
    import torch

    from . import kfmt_quant as KQ
    from . import synth
    from .decode import DecodeWorkspace
    from .kfmt import run_kfmt_decode

    dev = torch.device("cuda:0")
    T, HKV = 4096, 8
    q, k, v = synth.attention_inputs(B=1, T=T, HQ=32, HKV=HKV, D=128, seed=0, n_heavy=0, outlier_channels=4,
                                     outlier_scale=10.0)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    base, sc, res = KQ.quantize_fp8_scaled(kd, torch.float8_e4m3fn)
    copies = [(base.clone(), sc.clone(), res.clone(), vd.clone()) for _ in range(R)]
    ws = DecodeWorkspace(1, 32, HKV, T, 64, 64, dev, torch.bfloat16)
    buf = torch.zeros(4096 * 4 * 16, dtype=torch.int64, device=dev)
    N.lib().ffa_debug_set_timeline_kfmt.argtypes = [ctypes.c_void_p]
    assert N.lib().ffa_debug_set_timeline_kfmt(ctypes.c_void_p(buf.data_ptr())) == 0

    def step(r):
        b_, s_, r_, v_ = copies[r]
        run_kfmt_decode(q=qd, k=b_, k_format=N.KFMT_FP8_E4M3, k_scale=s_, scale_kind=N.KSCALE_TOKEN, v=v_,
                        k_residual=r_, use_res=True, T=T, HKV=HKV, scale=128 ** -0.5, BS=64, SBS=64, delta=5.0,
                        workspace=ws)

    us = _graph(step, R)
    st = buf.cpu().numpy().reshape(-1, 16).astype(np.int64)
    return us, st[st[:, 12] != 0], "step (stage 1 + merge) per launch"


def summarize(st: np.ndarray, names, per_wg: bool, exact_points=range(6, 10)) -> None:
    rel = (st[:, :13] - st[:, 0].min()) * 0.01  # 100 MHz ticks -> us
    nex = st[:, 13]
    print(f"{'point':22s} {'median':>7s} {'p90':>7s} {'max':>7s}   (us from the first wave's start)")
    for i, nm in enumerate(names):
        if nm == "-":  # a point this layout does not stamp
            continue
        col = rel[nex > 0, i] if i in exact_points else rel[:, i]
        print(f"{nm:22s} {np.median(col):7.2f} {np.percentile(col, 90):7.2f} {col.max():7.2f}")
    ex = nex > 0
    if ex.any():
        d = lambda a, b: np.median(rel[ex, b] - rel[ex, a])  # noqa: E731
        print(f"waves with a kept chunk: {int(ex.sum())}; medians: {names[5]} -> {names[6]} {d(5, 6):.2f}, "
              f"-> {names[7]} {d(6, 7):.2f}, -> {names[8]} {d(7, 8):.2f}, -> {names[9]} {d(8, 9):.2f}")
    if not per_wg:
        return
    nwg = len(st) // 4
    end = rel[:, 12].reshape(nwg, 4).max(1)
    kept = st[:, 14].reshape(nwg, 4)[:, 0]
    xcc = (st[:, 15] >> 32).reshape(nwg, 4)[:, 0] & 0xF
    hw = (st[:, 15] & 0xFFFFFFFF).reshape(nwg, 4)[:, 0]
    cu_key = xcc * 1000 + ((hw >> 13) & 0x7) * 100 + ((hw >> 8) & 0xF)
    for k in range(int(kept.max()) + 1):
        sel = kept == k
        if sel.any():
            print(f"workgroups with {k} kept chunks: {int(sel.sum()):4d}, end median {np.median(end[sel]):.2f} "
                  f"max {end[sel].max():.2f}")
    cus = {}
    for i in range(nwg):
        cus.setdefault(int(cu_key[i]), []).append(i)
    per_cu = [(sum(int(kept[i]) for i in v), max(end[i] for i in v)) for v in cus.values()]
    for k in sorted({p[0] for p in per_cu}):
        ends = [p[1] for p in per_cu if p[0] == k]
        print(f"CUs with {k} kept chunks: {len(ends):3d}, latest workgroup end median {np.median(ends):.2f} "
              f"max {max(ends):.2f}")
    xs = {int(x): (int(kept[xcc == x].sum()), round(float(end[xcc == x].max()), 2)) for x in np.unique(xcc)}
    print("per XCD (kept chunks, latest end):", xs)


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("cmd", choices=("build", "run"))
    ap.add_argument("--workload", choices=tuple(POINTS), default="config2")
    args = ap.parse_args(argv)
    if args.cmd == "build":
        print(build_lib(verbose=True))
        return
    from . import _native as N

    if not LIB.exists():
        raise SystemExit(f"{LIB} is missing: run `python -m ffa_mi355x.timeline build` first")
    N.LIB_PATH = LIB  # this process loads the timeline build instead of the library
    us, st, what = {"config2": _config2, "config1": _config1, "config2ref": _config2ref}[args.workload](N)
    print(f"{args.workload}: {us:.2f} us {what} in the timeline build; {len(st)} waves")
    summarize(st, POINTS[args.workload], per_wg=args.workload != "config1", exact_points=EXACT_POINTS[args.workload])


if __name__ == "__main__":
    main(sys.argv[1:])
