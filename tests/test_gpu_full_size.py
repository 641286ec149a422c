"""GPU parity at the benchmark configs' full sizes (configs 2-5), through the library's own append and decode.

Config 2 (B=1, 32K) is small enough for the whole oracle: bytes, mask, threshold and output.
For configs 3-5 (0.5-4.2M tokens) the oracle quantizers would take minutes, so:
  * appended bytes are checked on a seeded sample of tokens against the oracle quantizer
    applied to those tokens' K rows;
  * one sequence is decoded by the oracle in full from the pools the GPU wrote (gathered
    back through the page table): mask (except near-threshold blocks), threshold, output;
  * size-independent properties, bit-exact: every sequence of the batch decoded alone equals
    its row of the batched decode, and a permutation of the pool's pages (with the block
    table permuted to match) gives the same outputs.
"""
import numpy as np
import pytest
import torch

from helpers import assert_out_close, compare_masks, f32
from ffa_mi355x import synth
from ffa_mi355x.paged import (CODES_ORDER, GSCALE_ORDER, K4_ORDER, RES_ORDER, VT_ORDER, scale_pos,
                              to_logical)
from oracle import formats as OF
from oracle import q2fp8 as O

pytestmark = pytest.mark.gpu
SPOS = np.array([scale_pos(t) for t in range(64)])


# ------------------------------------------------------------------ page pools -> logical sequence
def _pages(bt_row, L):
    return bt_row[: -(-L // 64)].long()


def q2_sequence(cache, bt_row, L):
    """(codes [L, HKV, 32], scale, zero [L, HKV, 4] f32, residual [L, HKV, 128] u8, v [L, HKV, 128] f32)."""
    pg = _pages(bt_row, L)
    n, H = pg.numel(), cache.HKV

    def tok(x):  # [n, HKV, 64, X] -> [L, HKV, X]
        return x.transpose(0, 2, 1, 3).reshape(n * 64, H, -1)[:L]

    kq = to_logical(cache.k_q[pg].cpu().numpy(), CODES_ORDER, 8)  # [n, HKV, 4, 64, 8]
    kq = kq.transpose(0, 3, 1, 2, 4).reshape(n * 64, H, 32)[:L]
    s = to_logical(cache.k_scale[pg].float().cpu().numpy(), GSCALE_ORDER)[..., SPOS]  # [n, HKV, 4, 64]
    z = to_logical(cache.k_zero[pg].float().cpu().numpy(), GSCALE_ORDER)[..., SPOS]
    s = s.transpose(0, 3, 1, 2).reshape(n * 64, H, 4)[:L]
    z = z.transpose(0, 3, 1, 2).reshape(n * 64, H, 4)[:L]
    r = tok(to_logical(cache.k_res[pg].view(torch.uint8).cpu().numpy(), RES_ORDER))
    v = to_logical(cache.v[pg].view(torch.int16).cpu().numpy(), VT_ORDER)  # [n, HKV, 128, 64]
    v = torch.from_numpy(np.ascontiguousarray(v.transpose(0, 3, 1, 2).reshape(n * 64, H, 128)[:L]))
    return kq, s, z, r, f32(v.view(cache.v.dtype))


def kfmt_sequence(cache, bt_row, L):
    """(codes [L, HKV, 64] u8, scales [L, HKV, 8] u8 | [L, HKV, 2] f32, residual u8, v f32)."""
    pg = _pages(bt_row, L)
    n, H = pg.numel(), cache.HKV

    def tok(x):
        return x.transpose(0, 2, 1, 3).reshape(n * 64, H, -1)[:L]

    k = tok(to_logical(cache.k[pg].cpu().numpy(), K4_ORDER))
    sc = cache.k_scale[pg]
    sc = tok(sc.view(torch.uint8).cpu().numpy() if cache.fmt == "nvfp4" else f32(sc))
    r = tok(to_logical(cache.k_res[pg].view(torch.uint8).cpu().numpy(), RES_ORDER))
    v = to_logical(cache.v[pg].view(torch.int16).cpu().numpy(), VT_ORDER)
    v = torch.from_numpy(np.ascontiguousarray(v.transpose(0, 3, 1, 2).reshape(n * 64, H, 128)[:L]))
    return k, sc, r, f32(v.view(cache.v.dtype))


def _fill(cache, q, lens, bt, seed):
    """K/V of every sequence drawn on the device and appended; returns the K tensors (device, bf16)."""
    ks = []
    zero = torch.zeros(1, dtype=torch.int32, device=q.device)
    for b, L in enumerate(lens):
        k, v = synth.sequence_inputs_device(q[b], L, seed=seed + b)
        cache.append(k, v, zero, bt[b:b + 1])
        ks.append(k[0])
    return ks


def _sample_rows(ks, lens, n, seed):
    rng = np.random.default_rng(seed)
    bs = rng.integers(0, len(lens), n)
    ts = np.array([rng.integers(0, lens[b]) for b in bs])
    rows = torch.stack([ks[b][t] for b, t in zip(bs, ts)]).float().cpu().numpy()  # [n, HKV, 128]
    return bs, ts, rows


def _permuted(make_empty, cache, bt, seed):
    """A copy of the pools with page p moved to perm[p], and the block table mapped the same way."""
    perm = torch.from_numpy(np.random.default_rng(seed).permutation(cache.P)).to(bt.device)
    other = make_empty()
    for name in ("k", "k_q", "k_scale", "k_zero", "k_res", "v"):
        if hasattr(cache, name):
            getattr(other, name)[perm] = getattr(cache, name)
    return other, perm[bt.long()].to(torch.int32)


# ------------------------------------------------------------------ config 2: whole oracle
def test_config2_full_size_vs_oracle(gpu):
    from ffa_mi355x.paged import PagedQ2Cache

    B, T = 1, 32768
    q, k, v = synth.attention_inputs(B=B, T=T, seed=0, n_heavy=16, cos=0.8)  # bench.py's inputs
    bt, P = synth.page_tables([T], seed=0)
    cache = PagedQ2Cache(P, 8, gpu)
    cache.append(k.to(gpu), v.to(gpu), torch.zeros(1, dtype=torch.int32, device=gpu), bt.to(gpu))
    ws = cache.decode(q.to(gpu), bt.to(gpu), None, T=T, BS=64, SBS=64, delta=5.0)
    torch.cuda.synchronize()
    pk, s, z, r = O.quantize_g32(f32(k), "e4m3fn")
    kq, sg, zg, rg, vg = q2_sequence(cache, bt[0], T)
    assert np.array_equal(kq, pk[0]) and np.array_equal(rg, r[0]), "codes / residual"
    assert np.array_equal(sg, s[0]) and np.array_equal(zg, z[0]), "scales / zeros"
    assert np.array_equal(vg, f32(v.to(cache.v.dtype))[0]), "V (rounded to the pool dtype)"
    o_ref, diag = O.decode(f32(q), pk, s, z, f32(v), r, res_fmt="e4m3fn", BS=64, SBS=64, delta=5.0,
                           scale_mode="g32", out_dtype="bf16")
    far, near, n_near = compare_masks(ws.mask_buf.cpu().numpy(), diag)
    print(f"[mask] config2 keep={ws.mask_buf.float().mean().item():.4f} far={far} near={near}/{n_near}")
    assert far == 0
    assert np.abs(ws.threshold_buf.cpu().numpy() - diag["threshold"]).max() < 1e-4
    mx, mean = assert_out_close(f32(ws.o), o_ref, "config 2")
    print(f"[out] config2 max_abs={mx:.3e} mean_abs={mean:.3e}")


# ------------------------------------------------------------------ configs 3 and 4
@pytest.mark.parametrize("fmt", ["nvfp4", "nf4"])
def test_config34_full_size(gpu, fmt):
    from ffa_mi355x.paged_kfmt import PagedKfmtCache

    if fmt == "nvfp4":
        lens = [131072] * 4  # config 3
    else:
        lens = [int(x) for x in synth.ragged_lengths(16, 8192, 65536, seed=0)]  # config 4
    B, T = len(lens), max(lens)
    bt, P = synth.page_tables(lens, seed=3, interleave=True)
    btd = bt.to(gpu)
    cache = PagedKfmtCache(fmt, P, 8, gpu)
    q = torch.randn(B, 32, 128, generator=torch.Generator().manual_seed(3)).bfloat16().to(gpu)
    ks = _fill(cache, q, lens, btd, seed=300)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=gpu)
    ws = cache.decode(q, btd, lens_d, T=T, BS=64, SBS=64, delta=5.0)
    o_all, m_all = ws.o.clone(), ws.mask_buf.clone()
    torch.cuda.synchronize()

    # appended bytes of 256 sampled tokens
    bs, ts, rows = _sample_rows(ks, lens, 256, seed=4)
    quant = OF.quantize_nvfp4_g16 if fmt == "nvfp4" else OF.quantize_nf4_g64
    pk, sc, res = quant(rows)
    for j in range(256):
        b, t = int(bs[j]), int(ts[j])
        page, slot = int(bt[b, t // 64]), t % 64
        kk = to_logical(cache.k[page].cpu().numpy(), K4_ORDER)[:, slot]
        assert np.array_equal(kk, pk[j]), ("codes", b, t)
        got_s = cache.k_scale[page, :, slot]
        got_s = got_s.view(torch.uint8).cpu().numpy() if fmt == "nvfp4" else f32(got_s)
        assert np.array_equal(got_s, sc[j]), ("scales", b, t)
        rr = to_logical(cache.k_res[page].view(torch.uint8).cpu().numpy(), RES_ORDER)[:, slot]
        assert np.array_equal(rr, res[j]), ("residual", b, t)

    # every sequence alone == its row of the batch (bit-exact)
    for b in range(B):
        w1 = cache.decode(q[b:b + 1], btd[b:b + 1], lens_d[b:b + 1], T=T, BS=64, SBS=64, delta=5.0)
        torch.cuda.synchronize()
        assert torch.equal(w1.o[0], o_all[b]), f"sequence {b} alone differs from the batch"
        assert torch.equal(w1.mask_buf[0], m_all[b])

    # permuted pool pages, same outputs (bit-exact)
    other, bt2 = _permuted(lambda: PagedKfmtCache(fmt, P, 8, gpu), cache, btd, seed=5)
    w2 = other.decode(q, bt2, lens_d, T=T, BS=64, SBS=64, delta=5.0)
    torch.cuda.synchronize()
    assert torch.equal(w2.o, o_all) and torch.equal(w2.mask_buf, m_all), "page permutation changed the output"
    del other

    # the longest sequence through the oracle, from the GPU's pools
    b = int(np.argmax(lens))
    L = lens[b]
    kc, scs, rg, vg = kfmt_sequence(cache, bt[b], L)
    sel = bs == b
    if sel.any():  # sampled tokens of this sequence, through the gathered view
        assert np.array_equal(kc[ts[sel]], pk[sel]) and np.array_equal(rg[ts[sel]], res[sel])
        assert np.array_equal(scs[ts[sel]], sc[sel])
    khat = OF.khat_nvfp4_g16(kc, scs) if fmt == "nvfp4" else OF.khat_nf4_g64(kc, scs)
    o_ref, diag = O.decode(f32(q[b:b + 1]), kc[None], None, None, vg[None], rg[None], res_fmt="e4m3fn", BS=64, SBS=64,
                           delta=5.0, khat=khat[None], out_dtype="bf16")
    far, near, n_near = compare_masks(m_all[b:b + 1].cpu().numpy(), diag)
    print(f"[mask] {fmt} full size b={b} L={L} keep={m_all.float().mean().item():.4f} far={far} near={near}/{n_near}")
    assert far == 0
    assert np.abs(ws.threshold_buf[b:b + 1].cpu().numpy() - diag["threshold"]).max() < 1e-4
    mx, mean = assert_out_close(f32(o_all[b:b + 1]), o_ref, f"{fmt} full size")
    print(f"[out] {fmt} full size max_abs={mx:.3e} mean_abs={mean:.3e}")


# ------------------------------------------------------------------ config 5
def test_config5_full_size(gpu):
    from ffa_mi355x import kfmt_quant as KQ
    from ffa_mi355x import quant
    from ffa_mi355x.paged import PagedQ2Cache

    B, H, HKV = 64, 4096, 8
    lens = [65536 + b for b in range(B)]  # tokens before the append
    final = [t + 1 for t in lens]
    T = max(final)
    bt, P = synth.page_tables(final, seed=5, interleave=True)
    btd = bt.to(gpu)
    cache = PagedQ2Cache(P, HKV, gpu)
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, 32, 128, generator=g).bfloat16().to(gpu)
    ks = _fill(cache, q, lens, btd, seed=500)
    # the producer: token b rotated at, and appended to, position 65536 + b
    h = torch.randn(B, 1, H, generator=g).bfloat16()
    w = (torch.randn(HKV * 128, H, generator=g) * 0.02).bfloat16()
    pos = torch.tensor(lens, dtype=torch.int32)
    inv = 1.0 / (500000.0 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))
    ang = pos.float()[:, None] * inv[None, :]
    emb = torch.cat([ang, ang], -1)[:, None, :]
    cos, sin = emb.cos(), emb.sin()
    v_new = torch.randn(B, 1, HKV, 128, generator=g).bfloat16()
    quant.kproj_rope_q2_append(cache, h.to(gpu), w.to(gpu), cos.to(gpu), sin.to(gpu), pos.to(gpu), btd,
                               v_new=v_new.to(gpu))
    k_own = KQ.kproj_rope(h.view(1, B, H).to(gpu), w.to(gpu), cos.view(B, 128).to(gpu), sin.view(B, 128).to(gpu),
                          HKV, 128)
    lens_d = torch.tensor(final, dtype=torch.int32, device=gpu)
    ws = cache.decode(q, btd, lens_d, T=T, BS=64, SBS=64, delta=5.0)
    o_all, m_all = ws.o.clone(), ws.mask_buf.clone()
    torch.cuda.synchronize()

    # the appended token of every sequence: the oracle's g32 quantization of the producer's K
    pk, s, z, r = O.quantize_g32(f32(k_own).reshape(B, 1, HKV, 128), "e4m3fn")
    for b in range(B):
        page, slot = int(bt[b, lens[b] // 64]), lens[b] % 64
        kq = to_logical(cache.k_q[page].cpu().numpy(), CODES_ORDER, 8)[:, :, slot].reshape(HKV, 32)
        assert np.array_equal(kq, pk[b, 0]), ("codes", b)
        rr = to_logical(cache.k_res[page].view(torch.uint8).cpu().numpy(), RES_ORDER)[:, slot]
        assert np.array_equal(rr, r[b, 0]), ("residual", b)
        sc = to_logical(cache.k_scale[page].float().cpu().numpy(), GSCALE_ORDER)[..., SPOS][:, :, slot]
        zc = to_logical(cache.k_zero[page].float().cpu().numpy(), GSCALE_ORDER)[..., SPOS][:, :, slot]
        assert np.array_equal(sc, s[b, 0]) and np.array_equal(zc, z[b, 0]), ("scale / zero", b)
    # sampled tokens of the bulk fill: every field
    bs, ts, rows = _sample_rows(ks, lens, 256, seed=6)
    pk2, s2, z2, r2 = O.quantize_g32(rows, "e4m3fn")
    for j in range(256):
        b, t = int(bs[j]), int(ts[j])
        page, slot = int(bt[b, t // 64]), t % 64
        kq = to_logical(cache.k_q[page].cpu().numpy(), CODES_ORDER, 8)[:, :, slot].reshape(HKV, 32)
        assert np.array_equal(kq, pk2[j]), ("codes", b, t)
        sc = to_logical(cache.k_scale[page].float().cpu().numpy(), GSCALE_ORDER)[..., SPOS][:, :, slot]
        assert np.array_equal(sc, s2[j]), ("scales", b, t)
        zc = to_logical(cache.k_zero[page].float().cpu().numpy(), GSCALE_ORDER)[..., SPOS][:, :, slot]
        assert np.array_equal(zc, z2[j]), ("zeros", b, t)
        rr = to_logical(cache.k_res[page].view(torch.uint8).cpu().numpy(), RES_ORDER)[:, slot]
        assert np.array_equal(rr, r2[j]), ("residual", b, t)

    # sequences alone == rows of the batch (a sample of 4), bit-exact
    for b in (0, 21, 42, 63):
        w1 = cache.decode(q[b:b + 1], btd[b:b + 1], lens_d[b:b + 1], T=T, BS=64, SBS=64, delta=5.0)
        torch.cuda.synchronize()
        assert torch.equal(w1.o[0], o_all[b]), f"sequence {b} alone differs from the batch"

    # two sequences through the oracle, from the GPU's pools (incl. the appended token)
    for b in (0, 63):
        L = final[b]
        kq, sg, zg, rg, vg = q2_sequence(cache, bt[b], L)
        o_ref, diag = O.decode(f32(q[b:b + 1]), kq[None], sg[None], zg[None], vg[None], rg[None], res_fmt="e4m3fn",
                               BS=64, SBS=64, delta=5.0, scale_mode="g32", out_dtype="bf16")
        far, near, n_near = compare_masks(m_all[b:b + 1].cpu().numpy(), diag)
        print(f"[mask] config5 b={b} far={far} near={near}/{n_near}")
        assert far == 0
        assert np.abs(ws.threshold_buf[b:b + 1].cpu().numpy() - diag["threshold"]).max() < 1e-4
        mx, mean = assert_out_close(f32(o_all[b:b + 1]), o_ref, f"config 5 b={b}")
        print(f"[out] config5 b={b} max_abs={mx:.3e} mean_abs={mean:.3e}")
