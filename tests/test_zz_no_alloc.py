"""ffa_q2fp8_decode_noalloc (scratch in the library's static device array) against ffa_q2fp8_decode
(caller-owned scratch), through the C ABI: two calls in a row, the second with a smaller input
(and the two-pass path), outputs bit-identical; a shape beyond the static array is refused
before any launch; a call captured into a HIP graph (after one eager call has resolved the
scratch address) replays to the decode's output."""
import ctypes

import pytest
import torch

from helpers import paged_case, to_gpu_paged
from ffa_mi355x import _native as N
from ffa_mi355x import decode as D

pytestmark = pytest.mark.gpu


def _args(case, cache, gpu, BS, SBS, delta, lens=None):
    q = case["q"].to(gpu)
    bt = case["block_table"].to(gpu)
    sl = torch.tensor(lens, dtype=torch.int32, device=gpu) if lens is not None else None
    kw = dict(q=q, k_q=cache.k_q, k_scale=cache.k_scale, k_zero=cache.k_zero, v=cache.v, k_residual=cache.k_res,
              layout=N.LAYOUT_PAGED, scale_mode=N.SCALE_G32, T=int(bt.shape[1]) * 64, HKV=cache.k_q.shape[1],
              scale=D.default_scale(128), BS=BS, SBS=SBS, delta=delta, use_res=True, block_table=bt, seq_lens=sl)
    return kw, (q, bt, sl)


def _noalloc(kw, gpu, keep_mask: bool):
    """The no-allocation entry point on the same inputs: no scratch pointers; mask and thresholds
    into caller tensors (keep_mask) or left in the static scratch."""
    a, ws = D.decode_args(**kw)  # ws only supplies shapes; its scratch pointers are cleared below
    out = torch.full_like(ws.o, float("nan"))
    a.out = out.data_ptr()
    a.m_buf = a.l_buf = a.o_buf = None
    a.nparts = 0
    a.piece_max = None
    a.npieces = 0
    mask = th = None
    if keep_mask:
        mask = torch.full_like(ws.mask_buf, -1)
        th = torch.full_like(ws.threshold_buf, float("nan"))
        a.mask, a.ntbs, a.threshold_out = mask.data_ptr(), ws.NTBS, th.data_ptr()
    else:
        a.mask, a.threshold_out = None, None
    rc = N.lib().ffa_q2fp8_decode_noalloc(ctypes.byref(a), ctypes.c_void_p(N.stream_of(gpu)))
    N.check(rc, "ffa_q2fp8_decode_noalloc")
    torch.cuda.synchronize()
    return out, mask, th


def test_noalloc_matches_decode_twice_then_smaller(gpu):
    # first call: config-2 shape at 8K (G = 4, one pass), mask and thresholds returned to the caller
    c1 = paged_case(B=2, T=8192, HQ=32, HKV=8, seed=51, n_heavy=16, seq_lens=[8192, 5000])
    cache1 = to_gpu_paged(c1, gpu)
    kw1, _ = _args(c1, cache1, gpu, 64, 64, 5.0, c1["lens"])
    ws1 = D.run_decode(**kw1)
    torch.cuda.synchronize()
    out1, mask1, th1 = _noalloc(kw1, gpu, keep_mask=True)
    assert torch.equal(out1, ws1.o)
    assert torch.equal(mask1, ws1.mask_buf) and torch.equal(th1, ws1.threshold_buf)
    # second call, smaller: B = 1, 1000 tokens, G = 8 with SBS = 1024 (two passes: block maxima in the
    # static scratch too), mask and thresholds kept in the scratch
    c2 = paged_case(B=1, T=1000, HQ=64, HKV=8, seed=52, n_heavy=8)
    cache2 = to_gpu_paged(c2, gpu)
    kw2, _ = _args(c2, cache2, gpu, 1024, 1024, 4.0)
    ws2 = D.run_decode(**kw2)
    torch.cuda.synchronize()
    out2, _, _ = _noalloc(kw2, gpu, keep_mask=False)
    assert torch.equal(out2, ws2.o)
    # and the first shape again after the smaller one (the array keeps the last call's contents)
    out3, mask3, _ = _noalloc(kw1, gpu, keep_mask=True)
    assert torch.equal(out3, ws1.o) and torch.equal(mask3, ws1.mask_buf)


def test_noalloc_refuses_shapes_beyond_the_static_array(gpu):
    c = paged_case(B=1, T=256, HQ=32, HKV=8, seed=53, n_heavy=4)
    cache = to_gpu_paged(c, gpu)
    kw, _ = _args(c, cache, gpu, 64, 64, 5.0)
    a, ws = D.decode_args(**kw)
    a.out = ws.o.data_ptr()
    a.mask, a.threshold_out = None, None
    # 2^20 tokens: partials alone are 32 rows x 2048 spans x 520 B = 34 MB.  The block table still
    # covers 256 tokens only, so were the size check to pass, the decode's own block-table check
    # would refuse the call (-1) before any launch
    a.T = 1 << 20
    rc = N.lib().ffa_q2fp8_decode_noalloc(ctypes.byref(a), ctypes.c_void_p(N.stream_of(gpu)))
    assert rc == -2 and b"static array" in N.lib().ffa_last_error()


def test_noalloc_mean_v(gpu):
    """The mean-V fallback through the no-allocation entry point: its pruned-mass scratch is carved
    from the static array too (approx_m / approx_l cleared here); bit-identical to the decode."""
    c = paged_case(B=2, T=3000, HQ=32, HKV=8, seed=54, n_heavy=8, seq_lens=[3000, 1700])
    cache = to_gpu_paged(c, gpu)
    kw, (q, bt, sl) = _args(c, cache, gpu, 64, 64, 3.0, c["lens"])
    kw["v_mean"] = cache.value_mean(bt, sl, T=kw["T"])
    ws = D.run_decode(**kw)
    torch.cuda.synchronize()
    a, _ = D.decode_args(**kw)
    out = torch.full_like(ws.o, float("nan"))
    a.out = out.data_ptr()
    a.m_buf = a.l_buf = a.o_buf = a.approx_m = a.approx_l = None
    a.nparts = 0
    a.mask, a.threshold_out = None, None
    rc = N.lib().ffa_q2fp8_decode_noalloc(ctypes.byref(a), ctypes.c_void_p(N.stream_of(gpu)))
    N.check(rc, "ffa_q2fp8_decode_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(out, ws.o)


def test_noalloc_under_graph_capture(gpu):
    """Captured into a graph (torch.cuda.graph) after an eager call on the device, replayed three times
    with eager decodes of other inputs in between: every replay equals ffa_q2fp8_decode bit for bit."""
    c = paged_case(B=2, T=4096, HQ=32, HKV=8, seed=55, n_heavy=16, seq_lens=[4096, 2500])
    cache = to_gpu_paged(c, gpu)
    kw, _ = _args(c, cache, gpu, 64, 64, 5.0, c["lens"])
    ws = D.run_decode(**kw)
    torch.cuda.synchronize()
    out0, _, _ = _noalloc(kw, gpu, keep_mask=False)  # eager: resolves the static scratch address
    assert torch.equal(out0, ws.o)
    a, _ = D.decode_args(**kw)
    out = torch.full_like(ws.o, float("nan"))
    a.out = out.data_ptr()
    a.m_buf = a.l_buf = a.o_buf = None
    a.nparts = 0
    a.mask, a.threshold_out = None, None
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=s):
        rc = N.lib().ffa_q2fp8_decode_noalloc(ctypes.byref(a), ctypes.c_void_p(s.cuda_stream))
    N.check(rc, "ffa_q2fp8_decode_noalloc (captured)")
    c2 = paged_case(B=1, T=2000, HQ=32, HKV=8, seed=56, n_heavy=8)
    cache2 = to_gpu_paged(c2, gpu)
    kw2, _ = _args(c2, cache2, gpu, 64, 64, 4.0)
    for _ in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ws.o)
        D.run_decode(**kw2)  # eager work between replays, using the same library
        _noalloc(kw2, gpu, keep_mask=False)  # and the static scratch itself
        torch.cuda.synchronize()
