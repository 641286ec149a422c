#!/usr/bin/env python
"""Benchmark of the MI355X q2fp8 pruned decode (benchmark config 2).

Workload: one decode-attention step ("layer-step") of batch 1 over a 32K
context, 32 query / 8 KV heads, head dim 128.  K is 2-bit (groups of 32 along
D, fp16 scale/zero per token) plus an fp8 e4m3 residual, V is bf16 (held as
fp16, the type the decode's P.V uses, as the reference casts v to fp16), paged in
64-token pages through a seeded random page table; 16 heavy tokens per query
head are planted (cosine 0.8 with q).  Inputs are synthetic (seeded), already
resident in HBM when timing starts.

To keep the 256 MB Infinity Cache from serving repeated steps, R (default 24)
copies of the cache live in distinct pages and consecutive steps rotate over
them; the R steps are captured in one HIP graph that is replayed.

Prints one JSON line: value = microseconds per layer-step (lower is better),
with the achieved HBM bandwidth on the algorithmic bytes, the roofline object
of the decode and the CPU oracle timed on this host.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "ffa-speedtest_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E peak (AMD spec)
PAGE = 64


def algorithmic_bytes(T_list, HKV, HQ, kept_tokens_heads, D=128):
    """Bytes one layer-step must touch: every token's codes + g32 scale/zero, the fp8 residual and 16-bit V of
    kept tokens, q, o and the page table."""
    every = sum(T_list) * HKV * (D // 4 + (D // 32) * 4)
    kept = kept_tokens_heads * (D + 2 * D)
    consts = len(T_list) * HQ * D * 2 * 2 + sum(-(-t // PAGE) for t in T_list) * 4
    return every + kept + consts


def kept_token_heads(mask, T, SBS):
    """Tokens (x KV heads) inside kept blocks, counting only tokens < T."""
    import torch

    nb = mask.shape[-1]
    valid = torch.clamp(T - torch.arange(nb, device=mask.device) * SBS, min=0, max=SBS)
    return int((mask.to(torch.int64) * valid).sum().item())


def measured_traffic():
    """HBM bytes per stage-1 launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (or None)."""
    import re

    f = ROOT / "profiles" / "q2fp8_decode_kernel_config2_traffic.md"
    if not f.exists():
        return None
    m = re.search(r"^traffic_bytes_per_dispatch\s*=\s*(\d+)", f.read_text(), flags=re.M)
    return {"bytes": int(m.group(1)), "source": f"profiles/{f.name}"} if m else None


MIN_TIMED_STEPS = 200  # at least this many timed layer-steps, whatever --steps asks for
MIN_WARMUP_STEPS = 50


def host_cores() -> int:
    """Host cores this process may run on (16 at most: the GPU box's CPU share for one GPU)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def host_cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def oracle_decode_parallel(qf, pk, s, z, vf, r, HKV, threads, **kw):
    """The numpy oracle split by KV head over `threads` host threads (the (sequence, KV head) units are
    independent); numpy's per-element work releases the GIL, BLAS is held at one thread per task.
    Returns (o, mask [B, HKV, NTBS], margin [B, HKV, NTBS])."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    from threadpoolctl import threadpool_limits

    from oracle import q2fp8 as O

    G = qf.shape[1] // HKV
    khat = kw.pop("khat", None)

    def one(h):
        sl = slice(h, h + 1)
        cut = lambda a: None if a is None else a[:, :, sl]  # noqa: E731
        return O.decode(qf[:, h * G:(h + 1) * G], pk[:, :, sl], cut(s), cut(z), vf[:, :, sl], r[:, :, sl],
                        khat=cut(khat), **kw)

    with threadpool_limits(1), ThreadPoolExecutor(max_workers=threads) as ex:
        parts = list(ex.map(one, range(HKV)))
    o = np.concatenate([p_[0] for p_ in parts], axis=1)
    mask = np.concatenate([p_[1]["mask"] for p_ in parts], axis=1)
    margin = np.concatenate([p_[1]["margin"] for p_ in parts], axis=1)
    return o, mask, margin


def cpu_baseline(q, k, v, BS, SBS, delta, seconds):
    """The numpy oracle on this host's cores (split by KV head) on the same workload: microseconds per
    layer-step, the thread count, and the oracle's mask and margins of the last run."""
    from oracle import q2fp8 as O

    kf = k.float().numpy()
    pk, s, z, r = O.quantize_g32(kf, "e4m3fn")  # cache building, not timed
    qf, vf = q.float().numpy(), v.float().numpy()
    threads = host_cores()
    times = []
    t_end = time.perf_counter() + seconds
    while True:
        t0 = time.perf_counter()
        _, mask, margin = oracle_decode_parallel(qf, pk, s, z, vf, r, k.shape[2], threads, res_fmt="e4m3fn", BS=BS,
                                                 SBS=SBS, delta=delta, scale_mode="g32", out_dtype="bf16")
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end and len(times) >= 5:
            break
    return statistics.median(times) * 1e6, len(times), threads, mask, margin


WORKLOADS = {
    "config2ref": "benchmark config 2 in the reference's own layout: per-channel q2 scale/zero over T, e5m2 "
                  "residual, contiguous [B, T, HKV, D] cache (ffa-q2fp8/run_attn_bench_q2.py:78-105), bs=1, 32K ctx, "
                  "32/8/128, BS=SBS=64, delta=5",
    "config1": "benchmark config 1: fp8 e4m3 K with one fp16 scale per token and KV head + e4m3 residual, bf16 V, "
               "B=1, T=4096, 32/8/128, 4 of 128 K channels x10, contiguous cache, BS=SBS=64, delta=5",
    "config3": "benchmark config 3: nvfp4-g16 + e4m3 residual pruned decode, B=4 x 128K, 32/8/128, 64-token pages "
               "interleaved across sequences",
    "config4": "benchmark config 4: nf4-g64 + e4m3 residual pruned decode, B=16 ragged 8K-64K (seeded), 32/8/128, "
               "64-token pages interleaved across sequences",
    "config5": "benchmark config 5: K-proj (4096 -> 8x128) + RoPE (theta 5e5, positions 65536..65599) + g32 q2 + "
               "e4m3 quantize, appending token 65536+b to sequence b of 64, then one q2fp8 pruned decode over "
               "the 65537..65600-token contexts at B=64",
}
# bytes of one (token, KV head) that every step reads (codes + scales) and that a kept token adds (residual + V)
_EVERY = {"config3": 64 + 8, "config4": 64 + 4, "config5": 32 + 16}
_KEPT = 128 + 256


def _warm(R, per_graph=1):
    """Untimed steps before the timed replays: R eager steps plus the warm-up replays of _graph_time."""
    return R + max(1, math.ceil(MIN_WARMUP_STEPS / (R * per_graph))) * R * per_graph


def _reps(steps, R):
    """Graph replays of R steps that time at least MIN_TIMED_STEPS steps (and at least `steps`)."""
    return max(1, math.ceil(max(steps, MIN_TIMED_STEPS) / R))


def _graph_time(step, R, reps, stream, per_graph=1):
    """Microseconds per call of step(r): a HIP graph of `per_graph` rounds of step(0..R-1), replayed `reps`
    times, hipEvents around the replays (per_graph > 1 amortises the replay launch for short calls)."""
    import torch

    with torch.cuda.stream(stream):
        step(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for _ in range(per_graph):
            for r in range(R):
                step(r)
    torch.cuda.synchronize()
    for _ in range(max(1, math.ceil(MIN_WARMUP_STEPS / (R * per_graph)))):  # untimed warm-up replays
        g.replay()
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(cur)
    for _ in range(reps):
        g.replay()
    e1.record(cur)
    torch.cuda.synchronize()
    n = reps * R * per_graph
    return e0.elapsed_time(e1) * 1e3 / n, n


def bench_config2_reference_layout(args):
    """Config 2's inputs in the reference's contiguous per-channel layout, quantized by the HIP port of the
    reference quantizer and decoded through the stage-1 + merge launches; 24 rotated copies."""
    from ffa_mi355x import synth

    t_setup = time.perf_counter()
    q, k, v = synth.attention_inputs(B=1, T=args.T, HQ=32, HKV=8, D=128, seed=0, n_heavy=16, cos=0.8)
    _bench_contiguous(args, q, k, v, t_setup, WORKLOADS["config2ref"],
                      "config2 (reference layout) decode-attn us/step + HBM TB/s on the algorithmic bytes",
                      "synthetic (seeded N(0,1) bf16 with planted heavy tokens)")


def bench_layer_data(args):
    """Recorded layers (the reference's layer_data/layer_i/{q_rope,k_rope,v}.pt, read tensors-only by
    ffa_mi355x.layer_data): layers --layer .. --layer + --bsz - 1 stacked along the batch, the decode of the
    last recorded token (or --max-length) over the reference layout, as run_attn_bench_q2.py:146-170, 256-283
    does with these files."""
    import torch

    from ffa_mi355x import layer_data as LD

    if not args.layer_data:
        print(json.dumps({"error": "--workload layerdata needs --layer-data DIR (a layer_data directory)"}))
        sys.exit(2)
    t_setup = time.perf_counter()
    dt = {"bf16": torch.bfloat16, "fp16": torch.float16}[args.dtype]
    qr, kr, vr = LD.load_layer_batch(args.layer_data, range(args.layer, args.layer + args.bsz), dt,
                                     max_length=args.max_length)
    q, k, v = LD.decode_step_inputs(qr, kr, vr)
    B, HQ, D = q.shape
    T, HKV = k.shape[1], k.shape[2]
    desc = (f"recorded layers {args.layer}..{args.layer + args.bsz - 1} of {args.layer_data} as the batch "
            f"(B={B}, T={T}, {HQ}/{HKV}/{D}), reference per-channel layout, BS={args.BS}, SBS={args.SBS}, "
            f"delta={args.delta}")
    _bench_contiguous(args, q, k, v, t_setup, desc,
                      "recorded-layer q2fp8 decode-attn us/step + HBM TB/s on the algorithmic bytes",
                      f"recorded ({args.dtype})")


def _bench_contiguous(args, q, k, v, t_setup, workload, metric, data):
    """q [B, HQ, D], k / v [B, T, HKV, D] (host or device): the reference quantizer (HIP port), then the
    stage-1 + merge launches over R rotated copies of the cache in one HIP graph."""
    import torch

    from ffa_mi355x import _native as N
    from ffa_mi355x import quant
    from ffa_mi355x.decode import DecodeWorkspace, run_decode

    dev = torch.device("cuda:0")
    B, HQ, D = q.shape
    T, HKV = k.shape[1], k.shape[2]
    BS, SBS, R = args.BS, args.SBS, args.rotations
    qd, vd = q.to(dev), v.to(dev)
    kq, ks, kz, kr = quant.quantize_per_channel(k.to(dev), torch.float8_e5m2)
    copies = [(kq.clone(), kr.clone(), vd.clone()) for _ in range(R)]
    ws = DecodeWorkspace(B, HQ, HKV, T, BS, SBS, dev, qd.dtype)
    scale = 1.0 / math.sqrt(D)

    def step(r):
        kq_, kr_, v_ = copies[r]
        run_decode(q=qd, k_q=kq_, k_scale=ks, k_zero=kz, v=v_, k_residual=kr_, layout=N.LAYOUT_CONTIG,
                   scale_mode=N.SCALE_CHANNEL, T=T, HKV=HKV, scale=scale, BS=BS, SBS=SBS, delta=args.delta,
                   use_res=True, workspace=ws)

    for r in range(R):
        step(r)
    torch.cuda.synchronize()
    o0, mask = ws.o.clone(), ws.mask_buf.clone()
    stream = torch.cuda.Stream()
    setup_s = time.perf_counter() - t_setup
    us, steps = _graph_time(step, R, _reps(args.steps, R), stream)
    assert torch.equal(o0, ws.o), "graph replays must match the eager step"
    kept_th = kept_token_heads(mask, T, SBS)
    keep_frac = float(mask.float().mean().item())
    # every token's codes, the per-channel scale/zero once, residual + V of kept tokens, q and o
    nbytes = T * HKV * (D // 4) + B * HKV * D * 2 * 2 + kept_th * _KEPT + B * HQ * D * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    line = {
        "metric": metric,
        "value": round(us, 3), "unit": "us/step", "n_gpus": 1, "steps": steps, "warmup": _warm(R),
        "ms_per_step": round(us / 1e3, 6), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": f"q2 per-channel + e5m2 residual K, {str(vd.dtype).replace('torch.', '')} V; f16 MFMA (P.V on fp16 p "
                 "and fp16 v), f32 accumulate",
        "data": data,
        "config": {"workload": workload, "B": B, "T": T, "HQ": HQ, "HKV": HKV, "D": D, "BS": BS,
                   "SBS": SBS, "delta": args.delta, "keep_fraction": round(keep_frac, 4), "algorithmic_bytes": nbytes,
                   "rotations": R, "timing": "HIP graph of R steps (decode + merge), hipEvents over the replays"},
        "decode_hbm_tbps": round(gbs / 1e3, 4),
        "decode_hbm_pct_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "cpu_baseline": None,
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(line), flush=True)


def bench_config1(args):
    """Benchmark config 1 on the GPU (the reference runs it on the CPU): HIP quantizer, then the fp8 decode over
    the contiguous cache; 24 rotated copies defeat the MALL.  cpu_baseline: the numpy oracle, 1 thread."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_limits

    from ffa_mi355x import _native as N
    from ffa_mi355x import kfmt_quant as KQ
    from ffa_mi355x import synth
    from ffa_mi355x.decode import DecodeWorkspace
    from ffa_mi355x.kfmt import run_kfmt_decode

    dev = torch.device("cuda:0")
    B, HQ, HKV, D, T, BS, SBS, R = 1, 32, 8, 128, 4096, 64, 64, args.rotations
    t_setup = time.perf_counter()
    q, k, v = synth.attention_inputs(B=B, T=T, HQ=HQ, HKV=HKV, D=D, seed=0, n_heavy=0, outlier_channels=4,
                                     outlier_scale=10.0)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    base, sc, res = KQ.quantize_fp8_scaled(kd, torch.float8_e4m3fn)
    copies = [(base.clone(), sc.clone(), res.clone(), vd.clone()) for _ in range(R)]
    ws = DecodeWorkspace(B, HQ, HKV, T, BS, SBS, dev, torch.bfloat16)
    scale = 1.0 / math.sqrt(D)

    def step(r):
        b_, s_, r_, v_ = copies[r]
        run_kfmt_decode(q=qd, k=b_, k_format=N.KFMT_FP8_E4M3, k_scale=s_, scale_kind=N.KSCALE_TOKEN, v=v_,
                        k_residual=r_, use_res=True, T=T, HKV=HKV, scale=scale, BS=BS, SBS=SBS, delta=args.delta,
                        workspace=ws)

    for r in range(R):
        step(r)
    torch.cuda.synchronize()
    o0, mask = ws.o.clone(), ws.mask_buf.clone()
    stream = torch.cuda.Stream()
    setup_s = time.perf_counter() - t_setup
    us, steps = _graph_time(step, R, _reps(args.steps, R), stream)
    assert torch.equal(o0, ws.o), "graph replays must match the eager step"
    kept_th = kept_token_heads(mask, T, SBS)
    keep_frac = float(mask.float().mean().item())
    nbytes = T * HKV * (D + 2) + kept_th * _KEPT + B * HQ * D * 4
    gbs = nbytes / (us * 1e-6) / 1e9

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import formats as OF
        from oracle import q2fp8 as O

        kf, qf, vf = k.float().numpy(), q.float().numpy(), v.float().numpy()
        ob, osc, ores = OF.quantize_fp8_scaled(kf, "e4m3fn")  # cache building, not timed
        kh = OF.khat_fp8_scaled(ob, osc, "e4m3fn")
        threads = host_cores()
        times = []
        t_end = time.perf_counter() + args.cpu_seconds
        while True:
            t0 = time.perf_counter()
            oracle_decode_parallel(qf, ob, None, None, vf, ores, HKV, threads, res_fmt="e4m3fn", BS=BS, SBS=SBS,
                                   delta=args.delta, khat=kh, out_dtype="bf16")
            times.append(time.perf_counter() - t0)
            if time.perf_counter() > t_end and len(times) >= 5:
                break
        cpu = {"value": round(statistics.median(times) * 1e6, 1), "unit": "us/step", "cores": threads,
               "kind": "port", "cpu": host_cpu_model(), "torch": torch.__version__,
               "sample": f"full workload (B=1, T={T}, 32/8/128, per-token fp8 + e4m3 residual), numpy oracle split "
                         f"by KV head over {threads} threads, median of {len(times)} runs; cache quantization not timed"}
        del np
    line = {
        "metric": "config1 decode-attn us/step + HBM TB/s on the algorithmic bytes",
        "value": round(us, 3), "unit": "us/step", "n_gpus": 1, "steps": steps, "warmup": _warm(R),
        "ms_per_step": round(us / 1e3, 6), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "e4m3 K x fp16 token scale + e4m3 residual, bf16 V; f16 MFMA (P.V on fp16 p and fp16 v), f32 accumulate",
        "data": "synthetic (seeded N(0,1) bf16, 4 K channels x10)",
        "config": {"workload": WORKLOADS["config1"], "B": B, "T": T, "HQ": HQ, "HKV": HKV, "D": D, "BS": BS,
                   "SBS": SBS, "delta": args.delta, "keep_fraction": round(keep_frac, 4), "algorithmic_bytes": nbytes,
                   "rotations": R, "timing": "HIP graph of R steps (decode + merge), hipEvents over the replays"},
        "decode_hbm_tbps": round(gbs / 1e3, 4),
        "decode_hbm_pct_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "cpu_baseline": cpu,
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(line), flush=True)


def bench_workload(args):
    """Benchmark configs 3, 4 and 5 at their full sizes: one JSON line with the step time and its bandwidth.

    K and V are drawn on the device per sequence (synth.sequence_inputs_device), quantized and appended by
    the library's own append kernels, so no host copy of the multi-GB caches exists.
    """
    import torch

    from ffa_mi355x import synth
    from ffa_mi355x.decode import DecodeWorkspace, decode_ntbs

    dev = torch.device("cuda:0")
    wl = args.workload
    HQ, HKV, D, BS, SBS, delta = 32, 8, 128, 64, 64, args.delta
    t_setup = time.perf_counter()
    if wl == "config3":
        lens = [131072] * 4
    elif wl == "config4":
        lens = [int(x) for x in synth.ragged_lengths(16, 8192, 65536, seed=0)]
    else:
        lens = [65536 + b for b in range(64)]  # sequence b holds 65536 + b tokens before its append
    B = len(lens)
    final = [t + 1 for t in lens] if wl == "config5" else lens  # config 5 decodes after its append
    T = max(final)
    R = 1 if wl == "config5" else 2  # the caches (1.9-15.6 GB) dwarf the 256 MB MALL; 2 copies for 3 and 4
    bt0, npool = synth.page_tables(final, seed=0, interleave=True)
    g = torch.Generator().manual_seed(0)
    q = torch.randn(B, HQ, D, generator=g).to(torch.bfloat16)
    qd = q.to(dev)
    if wl == "config5":
        from ffa_mi355x import quant
        from ffa_mi355x.paged import PagedQ2Cache, check_append_fits

        cache = PagedQ2Cache(npool * R, HKV, dev)
    else:
        from ffa_mi355x.paged_kfmt import PagedKfmtCache

        cache = PagedKfmtCache("nvfp4" if wl == "config3" else "nf4", npool * R, HKV, dev)
    bts = [(bt0 + r * npool).to(dev) for r in range(R)]
    zero = torch.zeros(1, dtype=torch.int32, device=dev)
    for b in range(B):
        k, v = synth.sequence_inputs_device(qd[b], lens[b], HKV=HKV, D=D, seed=1000 + b)
        for r in range(R):
            cache.append(k, v, zero, bts[r][b:b + 1])
        del k, v
    lens_d = torch.tensor(final, dtype=torch.int32, device=dev)
    ws = DecodeWorkspace(B, HQ, HKV, T, BS, SBS, dev, torch.bfloat16)
    extra = {}

    def decode(r):
        cache.decode(qd, bts[r], lens_d, T=T, BS=BS, SBS=SBS, delta=delta, workspace=ws)

    if wl == "config5":
        H = 4096
        # one new token per sequence: token b of the 64 is rotated at, and appended to, position 65536 + b
        pos = torch.tensor(lens, dtype=torch.int32)
        h = (torch.randn(B, 1, H, generator=g)).to(torch.bfloat16).to(dev)
        # W_k [4096, 1024] ~ N(0, 0.02), held once in nn.Linear's [out, in] layout, whose rows the GEMM streams
        # (an [in, out] tensor would be transposed by the wrapper on every call, as the reference does)
        w = (torch.randn(H, HKV * D, generator=g) * 0.02).to(torch.bfloat16).t().contiguous().to(dev)
        inv = 1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
        ang = pos.float()[:, None] * inv[None, :]
        emb = torch.cat([ang, ang], -1)[:, None, :]
        cos, sin = emb.cos().to(dev), emb.sin().to(dev)
        v_new = torch.randn(B, 1, HKV, D, generator=g).to(torch.bfloat16).to(dev)
        pos_d = pos.to(dev)

        for r in range(R):  # host-side bounds check once, outside graph capture
            check_append_fits(pos_d, 1, bts[r], cache.P)

        def produce(r):
            quant.kproj_rope_q2_append(cache, h, w, cos, sin, pos_d, bts[r], v_new=v_new, validate=False)

        def step(r):
            produce(r)
            decode(r)
    else:
        step = decode

    for r in range(R):
        step(r)
    torch.cuda.synchronize()
    o0, mask = ws.o.clone(), ws.mask_buf.clone()
    stream = torch.cuda.Stream()
    setup_s = time.perf_counter() - t_setup
    reps = _reps(args.steps, R)
    us, steps = _graph_time(step, R, reps, stream)
    assert torch.equal(o0, ws.o), "graph replays must match the eager step"
    if wl == "config5":
        extra["producer_us"] = round(_graph_time(produce, R, 8, stream, per_graph=32)[0], 3)
        extra["decode_us"] = round(_graph_time(decode, R, reps, stream)[0], 3)

    valid = torch.zeros_like(mask, dtype=torch.int64)
    nb = mask.shape[-1]
    for b in range(B):
        valid[b] = torch.clamp(final[b] - torch.arange(nb, device=dev) * SBS, min=0, max=SBS)
    kept_th = int((mask.to(torch.int64) * valid).sum().item())
    total_blocks = sum(decode_ntbs(t, BS, SBS) for t in final) * HKV
    keep_frac = float(mask.to(torch.int64).sum().item()) / total_blocks
    nbytes = sum(final) * HKV * _EVERY[wl] + kept_th * _KEPT + B * HQ * D * 4 + sum(-(-t // PAGE) for t in final) * 4
    decode_us = extra.get("decode_us", us)
    gbs = nbytes / (decode_us * 1e-6) / 1e9
    line = {
        "metric": f"{wl} decode-attn us/step + HBM TB/s on the algorithmic bytes",
        "value": round(us, 3), "unit": "us/step", "n_gpus": 1, "steps": steps, "warmup": _warm(R),
        "ms_per_step": round(us / 1e3, 6), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": {"config3": "e2m1 K x e4m3 g16 scale + e4m3 residual, bf16 V held as fp16 V^T pages",
                  "config4": "nf4 K x fp16 g64 absmax + e4m3 residual, bf16 V held as fp16 V^T pages",
                  "config5": "bf16 K-proj (f32 accumulate); q2 g32 + e4m3 residual K, bf16 V held as fp16 V^T "
                             "pages"}[wl]
                 + "; f16 MFMA (P.V on fp16 p and fp16 v), f32 accumulate",
        "data": "synthetic (N(0,1) bf16 drawn on the device per sequence, 16 heavy tokens per query head)",
        "config": {"workload": WORKLOADS[wl], "B": B, "T_max": T, "tokens": sum(final), "HQ": HQ, "HKV": HKV,
                   "D": D, "BS": BS, "SBS": SBS, "delta": delta, "keep_fraction": round(keep_frac, 4),
                   "algorithmic_bytes": nbytes, "rotations": R,
                   "timing": "HIP graph of R steps, hipEvents over the replays"},
        "decode_hbm_tbps": round(gbs / 1e3, 4),
        "decode_hbm_pct_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "cpu_baseline": None,
        "setup_s": round(setup_s, 1),
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=480, help="timed layer-steps")
    ap.add_argument("--warmup", type=int, default=96, help="untimed layer-steps")
    ap.add_argument("--rotations", type=int, default=24, help="distinct cache copies (defeats the 256 MB MALL)")
    ap.add_argument("--T", type=int, default=32768)
    ap.add_argument("--BS", type=int, default=64)
    ap.add_argument("--SBS", type=int, default=64)
    ap.add_argument("--delta", type=float, default=5.0)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--kernel-launches", type=int, default=480, help="timed stage-1 launches (roofline)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run 5 device copies of 256 MiB (calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--workload", choices=("config2", "layerdata") + tuple(WORKLOADS), default="config2",
                    help="config2 (default) is the metric's line; config2ref, config1/3/4/5 time the other benchmark "
                         "decodes; layerdata times recorded layers (--layer-data)")
    ap.add_argument("--layer-data", default=None, help="layerdata: a layer_data directory (layer_0, layer_1, ...)")
    ap.add_argument("--layer", type=int, default=0, help="layerdata: first layer")
    ap.add_argument("--bsz", type=int, default=1, help="layerdata: consecutive layers stacked as the batch")
    ap.add_argument("--max-length", type=int, default=None, help="layerdata: cut the recorded tokens to this many")
    ap.add_argument("--dtype", choices=("bf16", "fp16"), default="bf16", help="layerdata: q / k / v dtype")
    args = ap.parse_args()
    if args.copy_probe:
        import torch

        src = torch.ones(64 * 2**20, dtype=torch.float32, device="cuda:0")  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": src.numel() * 4, "copies": 5}))
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU (the decode would shard by KV head or sequence "
                                   "without changing the per-GPU kernel); --gpus must be 1"}))
        sys.exit(2)

    if args.workload == "config1":
        bench_config1(args)
        return
    if args.workload == "config2ref":
        bench_config2_reference_layout(args)
        return
    if args.workload == "layerdata":
        bench_layer_data(args)
        return
    if args.workload != "config2":
        bench_workload(args)
        return

    import torch

    from ffa_mi355x import synth
    from ffa_mi355x.decode import DecodeWorkspace
    from ffa_mi355x.paged import PagedQ2Cache

    dev = torch.device("cuda:0")
    B, HQ, HKV, D, T, R = 1, 32, 8, 128, args.T, args.rotations
    t_setup = time.perf_counter()
    q, k, v = synth.attention_inputs(B=B, T=T, HQ=HQ, HKV=HKV, D=D, seed=0, n_heavy=16, cos=0.8)
    npg = -(-T // PAGE)
    bt0, _ = synth.page_tables([T], seed=0)
    cache = PagedQ2Cache(npg * R, HKV, dev)
    kd, vd = k.to(dev), v.to(dev)
    pos = torch.zeros(B, dtype=torch.int32, device=dev)
    bts = []
    for r in range(R):
        bt = (bt0 + r * npg).to(dev)
        cache.append(kd, vd, pos, bt)
        bts.append(bt)
    qd = q.to(dev)
    del kd, vd
    ws = DecodeWorkspace(B, HQ, HKV, T, args.BS, args.SBS, dev, torch.bfloat16)

    def step(r):
        cache.decode(qd, bts[r], None, T=T, BS=args.BS, SBS=args.SBS, delta=args.delta, workspace=ws)

    for r in range(R):  # eager warmup of every rotation
        step(r)
    step(0)
    torch.cuda.synchronize()
    outs = [ws.o.clone()]
    mask = ws.mask_buf.clone()
    step(R - 1)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], ws.o), "rotations must give identical outputs"

    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        step(0)  # prime on the capture stream
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        for r in range(R):
            step(r)
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup

    n_warm = max(1, math.ceil(max(args.warmup, MIN_WARMUP_STEPS) / R))
    n_rep = max(1, math.ceil(max(args.steps, MIN_TIMED_STEPS) / R))
    for _ in range(n_warm):
        graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(outs[0], ws.o), "graph replay must match eager"
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    start.record(cur)
    for _ in range(n_rep):
        graph.replay()
    end.record(cur)
    torch.cuda.synchronize()
    steps = n_rep * R
    ms_total = start.elapsed_time(end)
    us_per_step = ms_total * 1e3 / steps

    # dominant kernel (stage 1, q2fp8_decode_kernel) alone: a HIP graph of R back-to-back stage-1 launches
    # (the same rotations), hipEvents on the replay stream around the replays
    def stage1(r):
        cache.decode(qd, bts[r], None, T=T, BS=args.BS, SBS=args.SBS, delta=args.delta, workspace=ws,
                     stage="stage1")

    g1 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1, stream=stream):
        for r in range(R):
            stage1(r)
    torch.cuda.synchronize()
    n_k = max(1, math.ceil(args.kernel_launches / R))
    g1.replay()
    torch.cuda.synchronize()
    k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    k0.record(cur)
    for _ in range(n_k):
        g1.replay()
    k1.record(cur)
    torch.cuda.synchronize()
    kernel_us = k0.elapsed_time(k1) * 1e3 / (n_k * R)
    n_k *= R

    kept_th = kept_token_heads(mask, T, args.SBS)
    keep_frac = float(mask.float().mean().item())
    nbytes = algorithmic_bytes([T] * B, HKV, HQ, kept_th, D)
    achieved_gbs = nbytes / (us_per_step * 1e-6) / 1e9
    kernel_gbs = nbytes / (kernel_us * 1e-6) / 1e9
    traffic = measured_traffic()

    cpu = None
    mask_check = None
    if not args.no_cpu_baseline:
        import numpy as np
        import torch as _t

        cpu_us, n, threads, o_mask, o_margin = cpu_baseline(q, k, v, args.BS, args.SBS, args.delta, args.cpu_seconds)
        cpu = {"value": round(cpu_us, 1), "unit": "us/layer", "cores": threads, "kind": "port",
               "cpu": host_cpu_model(), "torch": _t.__version__,
               "sample": f"full workload (B=1, T={T}, 32/8/128, g32 q2 + e4m3 residual), numpy oracle split by KV "
                         f"head over {threads} threads, median of {n} runs; cache quantization not timed"}
        g_mask = mask.cpu().numpy()[..., : o_mask.shape[-1]]
        near = np.abs(o_margin) <= 1e-3
        differ = g_mask != o_mask
        mask_check = {"blocks": int(o_mask.size), "near_threshold_blocks": int(near.sum()),
                      "mismatch_far": int((differ & ~near).sum()), "mismatch_near": int((differ & near).sum()),
                      "rule": "survivor mask against the CPU oracle on the same inputs; near = |margin| <= 1e-3"}

    line = {
        "metric": "q2fp8 decode-attn us/layer + HBM TB/s (% of peak) at 32K ctx, bs=1",
        "value": round(us_per_step, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": steps,
        "warmup": n_warm * R,
        "ms_per_step": round(us_per_step / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q2+fp8(e4m3) K, bf16 V held as fp16 V^T pages; f16 MFMA (P.V on fp16 p and fp16 v), f32 accumulate",
        "data": "synthetic (seeded N(0,1) bf16 with planted heavy tokens)",
        "hbm_tbps": round(achieved_gbs / 1e3, 4),
        "hbm_pct_peak": round(100.0 * achieved_gbs / HBM_PEAK_GBS, 2),
        "config": {
            "workload": "benchmark config 2: q2fp8 pruned decode, bs=1, 32K ctx, 32/8/128, 64-token pages",
            "B": B, "T": T, "HQ": HQ, "HKV": HKV, "D": D, "BS": args.BS, "SBS": args.SBS, "delta": args.delta,
            "keep_fraction": round(keep_frac, 4), "algorithmic_bytes": nbytes, "rotations": R,
            "timing": "HIP graph of R rotated steps, hipEvent over the replays",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(kernel_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic["bytes"] if traffic else None,
            "kernel": "q2fp8_decode_kernel (stage 1: scores, prune, exact pass over kept pages)",
            "kernel_us": round(kernel_us, 3),
            "kernel_timing": f"HIP graph of {R} back-to-back stage-1 launches, hipEvents around {n_k} launches",
            "algorithmic_bytes_per_launch": nbytes,
            "traffic_source": traffic["source"] if traffic else None,
        },
        "cpu_baseline": cpu,
        "mask_vs_oracle": mask_check,
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
