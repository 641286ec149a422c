"""A tiny randomly initialised Llama decoding through the paged q2fp8 cache and the registered
attention hook (ffa-speedtest_amd/ffa-q2fp8/e2e/q2fp8_cache.py; the reference's fp8fp8 integration
is ffa-fp8fp8/e2e/fp8fp8_cache.py:183-224 and ffa-fp8fp8/e2e/modeling_llama.py:293-321).

Every decode step of every layer is checked against the oracle on the same inputs: the K / V the
layer appended (rotated, as the model produced them), g32-quantized by the oracle, and the layer's
query; the pools are checked byte for byte against the oracle's quantization.  Bar: outputs within
max-abs 2e-2 / mean-abs 2e-3, masks identical away from the threshold."""
import importlib.util
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import assert_out_close, compare_masks, f32
from oracle import q2fp8 as O

pytestmark = pytest.mark.gpu
E2E = Path(__file__).resolve().parents[1] / "ffa-speedtest_amd" / "ffa-q2fp8" / "e2e" / "q2fp8_cache.py"


def _load():
    spec = importlib.util.spec_from_file_location("q2fp8_cache", E2E)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _pool_logical(layer, T):
    """Codes / g32 scale / zero / residual of the first T tokens of each sequence, from the layer's pools."""
    from ffa_mi355x.paged import CODES_ORDER, GSCALE_ORDER, RES_ORDER, scale_pos, to_logical

    pool = layer.pool
    kq = to_logical(pool.k_q.cpu().numpy(), CODES_ORDER, 8)  # [P, H, 4, 64, 8]
    ks = to_logical(pool.k_scale.view(torch.int16).cpu().numpy().view(np.uint16), GSCALE_ORDER)
    kz = to_logical(pool.k_zero.view(torch.int16).cpu().numpy().view(np.uint16), GSCALE_ORDER)
    kr = to_logical(pool.k_res.view(torch.uint8).cpu().numpy(), RES_ORDER)
    bt = layer.block_table.cpu().numpy()
    spos = np.array([scale_pos(t) for t in range(64)])
    out = []
    for b in range(bt.shape[0]):
        pk, s, z, r = [], [], [], []
        for t0 in range(0, T, 64):
            pg, n = int(bt[b, t0 // 64]), min(64, T - t0)
            pk.append(kq[pg][:, :, :n].transpose(2, 0, 1, 3).reshape(n, -1, 32))
            s.append(ks[pg][:, :, spos[:n]].transpose(2, 0, 1))
            z.append(kz[pg][:, :, spos[:n]].transpose(2, 0, 1))
            r.append(kr[pg][:, :n].transpose(1, 0, 2))
        out.append([np.concatenate(x) for x in (pk, s, z, r)])
    return [np.stack([o[i] for o in out]) for i in range(4)]


def test_llama_decode_through_the_q2fp8_cache(gpu):
    from transformers import LlamaConfig, LlamaForCausalLM

    C = _load()
    cfg = LlamaConfig(vocab_size=512, hidden_size=1024, intermediate_size=1536, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=128, max_position_embeddings=8192,
                      rope_theta=500000.0)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).to(device=gpu, dtype=torch.bfloat16).eval()
    B, L, steps = 2, 700, 3
    cache = C.Q2FP8Cache(num_layers=2, max_batch_size=B, max_cache_len=1024, page_seed=3)
    seen_k = {0: [], 1: []}
    seen_v = {0: [], 1: []}
    for i, layer in enumerate(cache.layers):  # record the rotated K / V each layer appends
        orig = layer.update

        def rec(k, v, *a, _i=i, _orig=orig, **kw):
            seen_k[_i].append(k.transpose(1, 2).float().cpu())
            seen_v[_i].append(v.transpose(1, 2).float().cpu())
            return _orig(k, v, *a, **kw)

        layer.update = rec
    decodes = []

    def on_decode(layer_idx, q, o, layer):
        decodes.append((layer_idx, q.float().cpu(), o.float().cpu(), layer.seq_len,
                        layer._workspace.mask_buf.cpu().numpy().copy(), layer._workspace.threshold_buf.cpu().numpy()))

    C.enable_ffa_q2fp8(model, BS=64, SBS=64, delta=5.0, on_decode=on_decode)
    ids = torch.randint(0, 512, (B, L), generator=torch.Generator().manual_seed(1)).to(gpu)
    with torch.no_grad():
        out = model(input_ids=ids, past_key_values=cache, use_cache=True)
        nxt = out.logits[:, -1].argmax(-1)
        for _ in range(steps):
            out = model(input_ids=nxt[:, None], past_key_values=cache, use_cache=True)
            nxt = out.logits[:, -1].argmax(-1)
    torch.cuda.synchronize()
    assert cache.get_seq_length() == L + steps and torch.isfinite(out.logits.float()).all()
    assert len(decodes) == 2 * steps
    for layer_idx, q, o, T, mask, th in decodes:
        k_all = torch.cat(seen_k[layer_idx], dim=1)[:, :T].numpy()
        v_all = torch.cat(seen_v[layer_idx], dim=1)[:, :T].numpy()
        pk, s, z, r = O.quantize_g32(k_all, "e4m3fn")
        o_ref, diag = O.decode(q.numpy(), pk, s, z, v_all, r, res_fmt="e4m3fn", scale_mode="g32", BS=64, SBS=64,
                               delta=5.0, out_dtype="bf16")
        far, near, n_near = compare_masks(mask, diag)
        assert far == 0, f"layer {layer_idx} T={T}: {far} mask mismatches"
        assert np.abs(th - diag["threshold"]).max() < 1e-4
        o_forced, _ = O.decode(q.numpy(), pk, s, z, v_all, r, res_fmt="e4m3fn", scale_mode="g32", BS=64, SBS=64,
                               delta=5.0, out_dtype="bf16", force_mask=mask)
        mx, mean = assert_out_close(o.numpy(), o_forced, f"llama layer {layer_idx} T={T}")
        print(f"[out] layer {layer_idx} T={T} keep={mask.mean():.3f} max_abs={mx:.2e} mean_abs={mean:.2e} near={near}")
    # the pools hold exactly the oracle's quantization of what the layers appended
    for i, layer in enumerate(cache.layers):
        T = layer.seq_len
        k_all = torch.cat(seen_k[i], dim=1).numpy()
        pk, s, z, r = O.quantize_g32(k_all, "e4m3fn")
        gk, gs, gz, gr = _pool_logical(layer, T)
        assert np.array_equal(gk, pk) and np.array_equal(gr, r)
        assert np.array_equal(gs, s.astype(np.float16).view(np.uint16))
        assert np.array_equal(gz, z.astype(np.float16).view(np.uint16))


def _exact_reference(q, k_all, v_all, S, L):
    """Causal attention (float64) of the L newest queries q [B, HQ, L, D] over the first S tokens of
    the oracle's dequantized cache: keys fp32(c * scale + zero + residual) of the oracle's g32
    quantization rounded to bf16 (the model dtype), values fp16 (the V pool's dtype) then bf16."""
    from oracle.numerics import fp8_decode, round_bf16, round_f16

    pk, s, z, r = O.quantize_g32(k_all[:, :S], "e4m3fn")
    khat = O.dequant(pk, s, z, 128, "g32").astype(np.float32)  # c * s + z, exact in fp32
    kt = round_bf16((khat + fp8_decode(r, "e4m3fn")).astype(np.float32)).astype(np.float64)
    vt = round_bf16(round_f16(v_all[:, :S])).astype(np.float64)
    B, HQ, _, D = q.shape
    G = HQ // kt.shape[2]
    kt = np.repeat(kt.transpose(0, 2, 1, 3), G, axis=1)  # [B, HQ, S, D]
    vt = np.repeat(vt.transpose(0, 2, 1, 3), G, axis=1)
    sc = np.einsum("bhld,bhsd->bhls", q.astype(np.float64), kt) / np.sqrt(D)
    qpos = np.arange(S - L, S)[:, None]
    sc = np.where(np.arange(S)[None, :] > qpos, -np.inf, sc)
    p = np.exp(sc - sc.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhls,bhsd->blhd", p, vt)


def _run_llama(gpu, C, steps, chunk, **settings):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=512, hidden_size=1024, intermediate_size=1536, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=128, max_position_embeddings=8192,
                      rope_theta=500000.0)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).to(device=gpu, dtype=torch.bfloat16).eval()
    B, L = 2, 300
    cache = C.Q2FP8Cache(num_layers=2, max_batch_size=B, max_cache_len=1024, page_seed=5)
    seen_k, seen_v = {0: [], 1: []}, {0: [], 1: []}
    for i, layer in enumerate(cache.layers):
        orig = layer.update

        def rec(k, v, *a, _i=i, _orig=orig, **kw):
            seen_k[_i].append(k.transpose(1, 2).float().cpu())
            seen_v[_i].append(v.transpose(1, 2).float().cpu())
            return _orig(k, v, *a, **kw)

        layer.update = rec
    calls = []
    C.enable_ffa_q2fp8(model, BS=64, SBS=64, delta=5.0, **settings,
                       on_decode=lambda li, q, o, lay: calls.append(("ffa", li, q.float().cpu(), o.float().cpu(),
                                                                      lay.seq_len, 1,
                                                                      lay._workspace.mask_buf.cpu().numpy().copy())),
                       on_exact=lambda li, q, o, lay: calls.append(("exact", li, q.float().cpu(), o.float().cpu(),
                                                                    lay.seq_len, q.shape[2], None)))
    g = torch.Generator().manual_seed(2)
    with torch.no_grad():
        out = model(input_ids=torch.randint(0, 512, (B, L), generator=g).to(gpu), past_key_values=cache, use_cache=True)
        nxt = out.logits[:, -1].argmax(-1)
        for _ in range(steps):
            out = model(input_ids=nxt[:, None], past_key_values=cache, use_cache=True)
            nxt = out.logits[:, -1].argmax(-1)
        # a second multi-token chunk after decode steps (chunked prefill over the cached past)
        out = model(input_ids=torch.randint(0, 512, (B, chunk), generator=g).to(gpu), past_key_values=cache,
                    use_cache=True)
    torch.cuda.synchronize()
    assert cache.get_seq_length() == L + steps + chunk and torch.isfinite(out.logits.float()).all()
    return calls, {i: torch.cat(seen_k[i], dim=1).numpy() for i in seen_k}, {i: torch.cat(seen_v[i], dim=1).numpy()
                                                                             for i in seen_v}


def _check_calls(calls, K, V):
    kinds = []
    for kind, li, q, o, S, L, mask in calls:
        kinds.append((kind, li, L))
        if kind == "exact":
            ref = _exact_reference(q.numpy(), K[li], V[li], S, L)
            mx, mean = assert_out_close(o.numpy(), ref, f"exact layer {li} S={S} L={L}")
            print(f"[exact] layer {li} S={S} L={L} max_abs={mx:.2e} mean_abs={mean:.2e}")
        else:
            pk, s, z, r = O.quantize_g32(K[li][:, :S], "e4m3fn")
            okw = dict(res_fmt="e4m3fn", scale_mode="g32", BS=64, SBS=64, delta=5.0, out_dtype="bf16")
            _, diag = O.decode(q.numpy(), pk, s, z, V[li][:, :S], r, **okw)
            far, near, _ = compare_masks(mask, diag)
            assert far == 0, f"ffa layer {li} S={S}: {far} mask mismatches"
            o_ref, _ = O.decode(q.numpy(), pk, s, z, V[li][:, :S], r, force_mask=mask, **okw)
            mx, mean = assert_out_close(o.numpy(), o_ref, f"ffa layer {li} S={S}")
            print(f"[ffa] layer {li} S={S} max_abs={mx:.2e} mean_abs={mean:.2e}")
    return kinds


def test_llama_pattern_layers_and_chunked_prefill(gpu):
    """pattern_layers=[0]: layer 0 decodes through the pruned kernel, layer 1 through exact attention
    over its dequantized cache (modeling_llama.py:281-293, 322-337); the prompt and a later 40-token
    chunk run exact attention over the cache with the causal offset."""
    C = _load()
    calls, K, V = _run_llama(gpu, C, steps=3, chunk=40, pattern_layers=[0])
    kinds = _check_calls(calls, K, V)
    assert kinds == ([("exact", 0, 300), ("exact", 1, 300)] + [("ffa", 0, 1), ("exact", 1, 1)] * 3
                     + [("exact", 0, 40), ("exact", 1, 40)])


def test_llama_without_ffa_decode(gpu):
    """use_ffa_decode=False: every step runs exact attention over the dequantized cache (the
    reference bench's A/B baseline, e2e/bench_llama_fp8fp8.py:178-189)."""
    C = _load()
    calls, K, V = _run_llama(gpu, C, steps=2, chunk=17, use_ffa_decode=False)
    kinds = _check_calls(calls, K, V)
    assert all(k[0] == "exact" for k in kinds) and len(kinds) == 2 * 4


def test_paged_dequantize_matches_the_oracle(gpu):
    """ffa_q2_paged_dequant: keys fp32(c * scale + zero) + residual rounded once to the output dtype,
    values from the V^T pages, zeros past each sequence's length; bit-exact against the oracle's
    g32 quantization of what was appended."""
    from oracle.numerics import fp8_decode, round_bf16

    from ffa_mi355x import synth
    from ffa_mi355x.paged import PagedQ2Cache

    B, T, HKV = 3, 700, 4
    lens = [700, 333, 64]
    _, k, v = synth.attention_inputs(B=B, T=T, HQ=8, HKV=HKV, seed=9, n_heavy=0)
    bt, P = synth.page_tables(lens, seed=9)
    cache = PagedQ2Cache(P, HKV, gpu)
    for b, n in enumerate(lens):  # each sequence's own tokens only (its table row ends at its pages)
        cache.append(k[b:b + 1, :n].to(gpu), v[b:b + 1, :n].to(gpu), torch.zeros(1, dtype=torch.int32, device=gpu),
                     bt[b:b + 1].to(gpu))
    sl = torch.tensor(lens, dtype=torch.int32, device=gpu)
    kf, vf = cache.dequantize(bt.to(gpu), T, sl, out_dtype=torch.float32)
    kb, vb = cache.dequantize(bt.to(gpu), T, sl, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    pk, s, z, r = O.quantize_g32(f32(k), "e4m3fn")
    kref = (O.dequant(pk, s, z, 128, "g32").astype(np.float32) + fp8_decode(r, "e4m3fn")).astype(np.float32)
    vref = v.to(torch.float16).float().numpy()
    kg, vg = f32(kf), f32(vf)
    assert kg.shape == (B, 704, HKV, 128)
    for b, n in enumerate(lens):
        assert np.array_equal(kg[b, :n], kref[b, :n])
        assert np.array_equal(vg[b, :n], vref[b, :n])
        assert not kg[b, n:].any() and not vg[b, n:].any()
    assert np.array_equal(f32(kb)[0, :700], round_bf16(kref[0, :700]))
