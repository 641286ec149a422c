"""GPU parity of the benchmark's paged nvfp4-g16 / nf4-g64 modes (configs 3 and 4) against the oracle.

Append: every byte written to the pools (codes, scales, residual, V^T) equals the
oracle's quantization of the same K (oracle/formats.py quantize_nvfp4_g16 /
quantize_nf4_g64, pinned on the CPU), also when the cache is filled by several
appends and the pools start with garbage.  Decode: mask identical to the oracle's
except near-threshold blocks, output within the decode tolerance; the oracle sees
the logical (contiguous) sequence, so the page table is only storage.
"""
import importlib.util
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import assert_out_close, compare_masks, f32
from ffa_mi355x import synth
from ffa_mi355x.paged_kfmt import PagedKfmtCache
from oracle import formats as OF
from oracle import q2fp8 as O

pytestmark = pytest.mark.gpu
PKG = Path(__file__).resolve().parents[1] / "ffa-speedtest_amd"
QUANT = {"nvfp4": OF.quantize_nvfp4_g16, "nf4": OF.quantize_nf4_g64}


def _khat(fmt, pk, sc):
    return OF.khat_nvfp4_g16(pk, sc) if fmt == "nvfp4" else OF.khat_nf4_g64(pk, sc)


def _build(fmt, B, T, lens, seed, n_heavy=16, chunks=1, interleave=True, HQ=32, HKV=8):
    q, k, v = synth.attention_inputs(B=B, T=T, HQ=HQ, HKV=HKV, seed=seed, n_heavy=n_heavy, seq_lens=lens)
    lens = [T] * B if lens is None else [int(x) for x in lens]
    bt, P = synth.page_tables(lens, seed=seed, interleave=interleave)
    dev = torch.device("cuda:0")
    cache = PagedKfmtCache(fmt, P, HKV, dev)
    g = torch.Generator().manual_seed(seed + 100)
    for t in (cache.k, cache.k_scale, cache.k_res, cache.v):  # garbage in every slot the appends do not write
        t.view(torch.uint8).copy_(torch.randint(0, 256, t.view(torch.uint8).shape, generator=g, dtype=torch.uint8))
    btd = bt.to(dev)
    # each sequence appends its own tokens, in `chunks` pieces [c_i, c_i+1) at position c_i
    for bi in range(B):
        cuts = np.linspace(0, lens[bi], chunks + 1).astype(int)
        for a, e in zip(cuts[:-1], cuts[1:]):
            if e > a:
                cache.append(k[bi:bi + 1, a:e].to(dev), v[bi:bi + 1, a:e].to(dev),
                             torch.tensor([int(a)], dtype=torch.int32, device=dev), btd[bi:bi + 1])
    return q, k, v, lens, bt, btd, cache


def _gather(pool, bt, lens, b, tok_axis=2):
    """Tokens 0..lens[b]-1 of sequence b from a [P, HKV, 64, X] pool -> [len, HKV, X]."""
    rows = []
    for t0 in range(0, lens[b], 64):
        page = int(bt[b, t0 // 64])
        n = min(64, lens[b] - t0)
        rows.append(pool[page, :, :n].transpose(1, 0, 2))
    return np.concatenate(rows, axis=0)


@pytest.mark.parametrize("fmt", ["nvfp4", "nf4"])
def test_paged_append_bit_exact(gpu, fmt):
    B, T = 2, 300
    q, k, v, lens, bt, btd, cache = _build(fmt, B, T, None, seed=21, chunks=3)
    torch.cuda.synchronize()
    pk, sc, res = QUANT[fmt](f32(k))
    from ffa_mi355x.paged import K4_ORDER, RES_ORDER, VT_ORDER, to_logical

    kpool = to_logical(cache.k.cpu().numpy(), K4_ORDER)
    spool = cache.k_scale.view(torch.uint8).cpu().numpy() if fmt == "nvfp4" else f32(cache.k_scale)
    rpool = to_logical(cache.k_res.view(torch.uint8).cpu().numpy(), RES_ORDER)
    vpool = to_logical(cache.v.view(torch.int16).cpu().numpy(), VT_ORDER)
    vb = v.to(cache.v.dtype).view(torch.int16).numpy()
    for b in range(B):
        assert np.array_equal(_gather(kpool, bt, lens, b), pk[b]), "codes"
        assert np.array_equal(_gather(spool, bt, lens, b), sc[b]), "scales"
        assert np.array_equal(_gather(rpool, bt, lens, b), res[b]), "residual"
        vt = _gather(vpool.transpose(0, 1, 3, 2), bt, lens, b)  # V^T pages -> [len, HKV, 128]
        assert np.array_equal(vt, vb[b]), "V^T"


@pytest.mark.parametrize("fmt", ["nvfp4", "nf4"])
@pytest.mark.parametrize("B,T,lens,BS,SBS,delta", [
    (2, 3000, [3000, 1777], 64, 64, 5.0),     # two-chunk spans, 384 workgroups (runtime-span build)
    (1, 4096, None, 128, 32, 4.0),            # two-chunk spans, 256 workgroups
    (3, 2500, [2500, 64, 1000], 64, 16, 3.0),
    (1, 8192, None, 64, 64, 5.0),             # four-chunk spans
    (2, 8192, [8192, 5000], 64, 64, 5.0),     # eight-chunk spans in 256 workgroups (runtime-span build)
])
def test_paged_decode_parity(gpu, fmt, B, T, lens, BS, SBS, delta):
    q, k, v, lens, bt, btd, cache = _build(fmt, B, T, lens, seed=T + B)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=gpu)
    ws = cache.decode(q.to(gpu), btd, lens_d, T=T, BS=BS, SBS=SBS, delta=delta)
    torch.cuda.synchronize()
    pk, sc, res = QUANT[fmt](f32(k))
    o_ref, diag = O.decode(f32(q), pk, None, None, f32(v), res, res_fmt="e4m3fn", BS=BS, SBS=SBS, delta=delta,
                           khat=_khat(fmt, pk, sc), seq_lens=lens, out_dtype="bf16")
    far, near, n_near = compare_masks(ws.mask_buf.cpu().numpy(), diag)
    print(f"[mask] {fmt} B={B} T={T} keep={ws.mask_buf.float().mean().item():.3f} far={far} near={near}/{n_near}")
    assert far == 0
    assert np.abs(ws.threshold_buf.cpu().numpy() - diag["threshold"]).max() < 1e-4
    mx, mean = assert_out_close(f32(ws.o), o_ref, f"{fmt} paged")
    print(f"[out] {fmt} paged max_abs={mx:.3e} mean_abs={mean:.3e}")


@pytest.mark.parametrize("fmt", ["nvfp4", "nf4"])
def test_paged_ragged_large_grid_items(gpu, fmt):
    """A ragged batch on the large-batch build (6 x 8 x 32 = 1536 workgroup spans): only the spans that
    hold tokens are launched as work, so the mask bytes past each sequence's end (written by its last
    span) and every row's partials must come out as the oracle's from a workspace holding garbage;
    lengths include an empty sequence, a one-page one and a partial last page."""
    from ffa_mi355x.decode import DecodeWorkspace

    B, T = 6, 16384
    lens = [16384, 0, 700, 9000, 64, 12345]
    q, k, v, lens, bt, btd, cache = _build(fmt, B, T, lens, seed=77)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=gpu)
    ws = DecodeWorkspace(B, 32, 8, T, 64, 64, gpu, torch.bfloat16)
    ws.mask_buf.fill_(5)
    for t in (ws.m_buf, ws.l_buf, ws.o_buf, ws.o, ws.threshold_buf):
        t.fill_(float("nan"))
    for rep in range(2):  # twice into the same workspace
        cache.decode(q.to(gpu), btd, lens_d, T=T, BS=64, SBS=64, delta=5.0, workspace=ws)
        torch.cuda.synchronize()
        if rep == 0:
            pk, sc, res = QUANT[fmt](f32(k))
            o_ref, diag = O.decode(f32(q), pk, None, None, f32(v), res, res_fmt="e4m3fn", BS=64, SBS=64,
                                   delta=5.0, khat=_khat(fmt, pk, sc), seq_lens=lens, out_dtype="bf16")
        m = ws.mask_buf.cpu().numpy()
        for b, L in enumerate(lens):
            assert (m[b, :, -(-L // 64):] == 0).all(), f"mask bytes past the end of sequence {b}"
        far, near, n_near = compare_masks(m, diag)
        print(f"[mask] {fmt} items rep={rep} keep={ws.mask_buf.float().mean().item():.3f} far={far} near={near}/{n_near}")
        assert far == 0
        full = [b for b, L in enumerate(lens) if L > 0]  # (an empty sequence's threshold is not defined)
        assert np.abs(ws.threshold_buf.cpu().numpy()[full] - diag["threshold"][full]).max() < 1e-4
        mx, mean = assert_out_close(f32(ws.o), o_ref, f"{fmt} paged items")
        print(f"[out] {fmt} paged items max_abs={mx:.3e} mean_abs={mean:.3e}")
        assert (f32(ws.o)[1] == 0).all(), "an empty sequence decodes to 0"


@pytest.mark.parametrize("fmt", ["nvfp4", "nf4"])
def test_paged_drop_in_block_table_kwargs(gpu, fmt):
    """The reference entry points with block_table= select the paged pools; skip ratio and the
    no-residual path follow the reference's rules."""
    rel, fn = {"nvfp4": ("ffa-nvfp4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nvfp4fp8.py",
                         "attn_forward_decode_nvfp4fp8"),
               "nf4": ("ffa-nf4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nf4fp8.py", "attn_forward_decode_nf4")}[fmt]
    spec = importlib.util.spec_from_file_location(f"paged_dropin_{fmt}", PKG / rel)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    f = getattr(mod, fn)
    B, T = 2, 1500
    q, k, v, lens, bt, btd, cache = _build(fmt, B, T, [1500, 700], seed=31)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=gpu)
    qd = q.to(gpu).unsqueeze(1).contiguous()
    o, sr = f(qd, cache.k, cache.k_scale, cache.v, k_residual=cache.k_res, BS=64, delta=5.0, return_skip_ratio=True,
              block_table=btd, seq_lens=lens_d, T=T)
    torch.cuda.synchronize()
    pk, sc, res = QUANT[fmt](f32(k))
    o_ref, diag = O.decode(f32(q), pk, None, None, f32(v), res, res_fmt="e4m3fn", BS=64, SBS=64, delta=5.0,
                           khat=_khat(fmt, pk, sc), seq_lens=lens, out_dtype="bf16")
    assert abs(sr - diag["skip_ratio"]) < 0.02
    assert_out_close(f32(o), o_ref, f"{fmt} drop-in")
    o2 = f(qd, cache.k, cache.k_scale, cache.v, k_residual=None, BS=64, delta=5.0, use_fp8_residual=False,
           block_table=btd, seq_lens=lens_d, T=T)
    torch.cuda.synchronize()
    o2_ref, _ = O.decode(f32(q), pk, None, None, f32(v), res, res_fmt="e4m3fn", BS=64, SBS=64, delta=5.0,
                         khat=_khat(fmt, pk, sc), seq_lens=lens, out_dtype="bf16", use_fp8_residual=False)
    assert_out_close(f32(o2), o2_ref, f"{fmt} drop-in no residual")
    with pytest.raises(ValueError):
        f(qd, cache.k, cache.k_scale, cache.v, k_residual=None, BS=64, block_table=btd, seq_lens=lens_d, T=T)
