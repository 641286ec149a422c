"""Recorded-layer data through the decode: layers written in the reference's layer_data format,
read back with the loader, quantized on the GPU (reference per-channel quantizer) and decoded with
the q2fp8 drop-in, against the oracle on the same recorded tensors."""
import numpy as np
import pytest
import torch

from helpers import assert_out_close, compare_masks, f32
from ffa_mi355x import layer_data as LD
from ffa_mi355x import synth
from oracle import q2fp8 as O

pytestmark = pytest.mark.gpu


def _record(root, n_layers, T, HQ=32, HKV=8, D=128):
    for i in range(n_layers):
        q, k, v = synth.attention_inputs(B=1, T=T, HQ=HQ, HKV=HKV, D=D, seed=100 + i, n_heavy=16)
        g = torch.Generator().manual_seed(200 + i)
        q_rope = torch.randn(1, HQ, T, D, generator=g).bfloat16()
        q_rope[:, :, T - 1] = q  # the recorded query of the last position carries the planted heavy tokens
        LD.save_layer(root, i, q_rope=q_rope, k_rope=k.permute(0, 2, 1, 3), v=v.permute(0, 2, 1, 3),
                      q_unrope=q_rope, k_unrope=k.permute(0, 2, 1, 3), h=torch.zeros(1, T, 16).bfloat16())


@pytest.mark.parametrize("L", [3000, 1777])
def test_recorded_layers_decode(gpu, tmp_path, L):
    import attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8 as K
    from ffa_mi355x.quant import quantize_per_channel

    _record(tmp_path, 2, 3000)
    qr, kr, vr = LD.load_layer_batch(tmp_path, [0, 1], torch.bfloat16, max_length=None, device=gpu)
    q, k, v = LD.decode_step_inputs(qr, kr, vr, L=L)  # [2, 32, 128], [2, L, 8, 128] x 2
    k_q, k_scale, k_zero, k_res = quantize_per_channel(k)
    o, sr = K.attn_forward_decode_quantized(q.unsqueeze(1), k_q, k_scale, k_zero, v, k_residual=k_res, BS=128,
                                            delta=5.0, return_skip_ratio=True)
    torch.cuda.synchronize()
    pk, s, z, r = O.quantize_per_channel(f32(k), "bf16", "e5m2")
    assert np.array_equal(k_q.cpu().numpy(), pk)  # the GPU quantizer is bit-exact on recorded data too
    o_ref, diag = O.decode(f32(q), pk, s, z, f32(v), r, res_fmt="e5m2", BS=128, SBS=128, delta=5.0, out_dtype="bf16")
    ws = K.allocate_q2fp8_decode_workspace(q.unsqueeze(1), k_q, v, BS=128)
    K.attn_forward_decode_quantized(q.unsqueeze(1), k_q, k_scale, k_zero, v, k_residual=k_res, BS=128, delta=5.0,
                                    workspace=ws)
    torch.cuda.synchronize()
    mask = ws.mask_buf.cpu().numpy()
    far, near, n_near = compare_masks(mask, diag)
    print(f"[layer_data] L={L} skip={sr:.3f} oracle={diag['skip_ratio']:.3f} far={far} near={near}/{n_near}")
    assert far == 0
    o_forced, _ = O.decode(f32(q), pk, s, z, f32(v), r, res_fmt="e5m2", BS=128, SBS=128, delta=5.0, out_dtype="bf16",
                           force_mask=mask)
    assert_out_close(f32(o), o_forced, "recorded layers")


def test_bench_layerdata_line(gpu, tmp_path, capsys):
    """bench.py --workload layerdata on recorded files: one JSON line for the stacked layers."""
    import argparse
    import json

    import bench

    _record(tmp_path, 2, 2048)
    args = argparse.Namespace(layer_data=str(tmp_path), layer=0, bsz=2, max_length=1500, dtype="bf16", BS=64, SBS=64,
                              delta=5.0, rotations=2, steps=4)
    bench.bench_layer_data(args)
    line = json.loads(capsys.readouterr().out.strip().splitlines()[-1])
    assert line["config"]["B"] == 2 and line["config"]["T"] == 1500 and line["value"] > 0
    assert line["data"] == "recorded (bf16)" and 0.0 < line["config"]["keep_fraction"] <= 1.0
