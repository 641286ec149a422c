"""The per-channel q2 decoder dequantizes fp16 scale / zero with one packed fp16 FMA,
fp16(c * s + z) rounded once from the exact value, where the reference rounds twice,
fp16(fp32(fp32(c * s) + z)) (attn_kernel_v1210_fused_bsz_q2fp8.py:50-53, 93).  c * s is exact in fp32
(at most 13 significant bits); the two results can differ only where the fp32 sum drops a zero
point smaller than 2^-23 of c * s.  Checked here (CPU, numpy) for every finite fp16 z, c = 1..3 and
every 8th positive finite fp16 s: every difference has |z| < 2^-23 c s."""
import numpy as np


def test_single_rounding_equals_the_reference_unless_z_is_negligible():
    allh = np.arange(65536, dtype=np.uint16).view(np.float16)
    fin = allh[np.isfinite(allh)]
    S = fin[fin > 0][::8]
    z = fin.astype(np.float64)
    z32 = fin.astype(np.float32)
    differ = 0
    for i in range(0, S.size, 256):
        s = S[i:i + 256].astype(np.float64)[:, None]
        s32 = S[i:i + 256].astype(np.float32)[:, None]
        for c in (1.0, 2.0, 3.0):
            with np.errstate(over="ignore"):
                once = (c * s + z[None, :]).astype(np.float16)  # float64 holds c * s + z exactly
                twice = (np.float32(c) * s32 + z32[None, :]).astype(np.float16)  # fp32 mul, fp32 add
            d = (once != twice) & np.isfinite(once) & np.isfinite(twice)
            differ += int(d.sum())
            assert not (d & (np.abs(z)[None, :] >= 2.0 ** -23 * c * s)).any()
    assert differ > 0  # the case exists (c * s on an fp16 midpoint, z tiny): the bound is needed
