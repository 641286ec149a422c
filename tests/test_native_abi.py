"""The C-ABI library loads and exports what include/*.h declares (no GPU calls)."""
import ctypes
import inspect
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ffa_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    from ffa_mi355x import _native as N

    L = N.lib()
    declared = _declared_functions()
    assert declared, "no declarations found"
    missing = [n for n in declared if not hasattr(L, n)]
    assert not missing, f"missing exports: {missing}"
    assert set(N.EXPORTS) == declared


def test_ctypes_argtypes_match_header_parameter_lists():
    """Each function's ctypes argtypes have the header's parameter count, and the pointer /
    integer / size_t kinds in the same order."""
    from ffa_mi355x import _native as N

    L = N.lib()
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "ffa_mi355x.h").read_text(), flags=re.S)
    decls = re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ffa_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M)
    assert len(decls) == len(N.EXPORTS)
    for name, params in decls:
        params = [p.strip() for p in params.replace("\n", " ").split(",") if p.strip() not in ("", "void")]
        want = ["p" if "*" in p else ("z" if p.startswith("size_t") else "i") for p in params]
        kinds = {ctypes.c_void_p: "p", ctypes.c_int: "i", ctypes.c_size_t: "z", ctypes.c_float: "i"}
        got = [("p" if hasattr(t, "contents") or t is ctypes.c_void_p else kinds[t])
               for t in (getattr(L, name).argtypes or [])]
        assert got == want, name


@pytest.mark.parametrize("cname,pyname", [("ffa_q2fp8_decode_args", "DecodeArgs"),
                                           ("ffa_kfmt_decode_args", "KfmtArgs")])
def test_ctypes_argument_structs_match_header(tmp_path, cname, pyname):
    """Field names, offsets and size of the ctypes mirrors equal the C compiler's layout."""
    import shutil
    import subprocess

    from ffa_mi355x import _native as N

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    py = getattr(N, pyname)
    fields = [f[0] for f in py._fields_]
    body = "\n".join(f'  printf("%s %zu\\n", "{f}", offsetof({cname}, {f}));' for f in fields)
    src = tmp_path / "layout.c"
    src.write_text(f'#include <stddef.h>\n#include <stdio.h>\n#include "ffa_mi355x.h"\nint main(void) {{\n{body}\n'
                   f'  printf("sizeof %zu\\n", sizeof({cname}));\n  return 0;\n}}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    out = dict(line.split() for line in subprocess.run([str(exe)], check=True, capture_output=True,
                                                        text=True).stdout.splitlines())
    for f in fields:
        assert int(out[f]) == getattr(py, f).offset, f"{cname}.{f}"
    assert int(out["sizeof"]) == ctypes.sizeof(py)
    # every member of the C struct is mirrored
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "ffa_mi355x.h").read_text(), flags=re.S)
    decl = re.search(r"typedef struct %s \{(.*?)\} %s;" % (cname, cname), text, flags=re.S).group(1)
    members = []
    for d in decl.split(";"):
        d = d.strip()
        if d:
            head, *rest = d.split(",")
            members.append(re.findall(r"(\w+)\s*$", head)[0])
            members += [r.strip().lstrip("*").strip() for r in rest]
    assert members == fields


def test_host_only_helpers():
    from ffa_mi355x import _native as N

    L = N.lib()
    assert L.ffa_version().startswith(b"ffa_mi355x")
    # one partial slot per 512-token workgroup
    assert L.ffa_q2fp8_decode_nparts(32768, 64, 64) == 64
    assert L.ffa_q2fp8_decode_nparts(100, 128, 128) == 1
    assert L.ffa_q2fp8_decode_nparts(1000, 64, 64) == 8  # short sequences: room for two-chunk spans
    assert L.ffa_q2_quantize_nsplit(32768) == 64
    # two-pass scratch: none for G <= 4 and SBS <= 512; prune blocks (SBS <= 512) or 512-token spans
    assert L.ffa_q2fp8_decode_pieces(32, 8, 32768, 64, 64) == 0
    assert L.ffa_q2fp8_decode_pieces(32, 8, 32768, 512, 512) == 0
    assert L.ffa_q2fp8_decode_pieces(64, 8, 32768, 64, 64) == 512  # G = 8
    assert L.ffa_q2fp8_decode_pieces(48, 8, 1000, 128, 32) == 8 * 4  # G = 6, ceil(1000/128) * 4
    assert L.ffa_q2fp8_decode_pieces(32, 8, 5000, 4096, 4096) == 16  # SBS = 4096: ceil(5000/4096)*4096/512
    assert L.ffa_q2fp8_decode_pieces(32, 8, 5000, 2048, 1024) == 12


def test_invalid_arguments_are_rejected_without_launch():
    from ffa_mi355x import _native as N

    L = N.lib()
    a = N.DecodeArgs()
    a.B, a.T, a.HQ, a.HKV = 1, 128, 136, 8  # G = 17 -> beyond the reference's 16-row tile
    a.BS, a.SBS = 64, 64
    rc = L.ffa_q2fp8_decode(ctypes.byref(a), None)
    assert rc == -2 and b"group" in L.ffa_last_error()
    a.HQ = 40  # G = 5: two passes, which need the piece_max scratch
    assert L.ffa_q2fp8_decode(ctypes.byref(a), None) == -1 and b"piece_max" in L.ffa_last_error()
    a.HQ, a.BS, a.SBS = 32, 1024, 1024  # SBS > 512: two passes as well
    assert L.ffa_q2fp8_decode(ctypes.byref(a), None) == -1 and b"piece_max" in L.ffa_last_error()
    a.BS = 64
    a.SBS = 48
    assert L.ffa_q2fp8_decode(ctypes.byref(a), None) == -2
    a.SBS = 64
    a.q_dtype, a.out_dtype, a.v_dtype, a.res_dtype = 0, 0, 9, 3
    assert L.ffa_q2fp8_decode(ctypes.byref(a), None) == -1
    # paged: the pool size is required and the block table must cover T (checked before any launch)
    a.v_dtype, a.res_dtype, a.layout = N.DT_BF16, N.DT_NONE, N.LAYOUT_PAGED
    a.block_table, a.bt_stride, a.num_pages = 0x1000, 2, 0
    assert L.ffa_q2fp8_decode(ctypes.byref(a), None) == -1 and b"num_pages" in L.ffa_last_error()
    a.num_pages, a.bt_stride = 4, 1
    assert L.ffa_q2fp8_decode(ctypes.byref(a), None) == -1 and b"block table" in L.ffa_last_error()
    k = N.KfmtArgs()
    k.B, k.T, k.HQ, k.HKV, k.BS, k.SBS = 1, 128, 32, 8, 64, 64
    k.v_dtype, k.res_dtype, k.layout, k.block_table, k.bt_stride = N.DT_BF16, N.DT_NONE, N.LAYOUT_PAGED, 0x1000, 2
    k.nparts, k.ntbs = 1, 2
    assert L.ffa_kfmt_decode(ctypes.byref(k), None) == -1 and b"num_pages" in L.ffa_last_error()
    k.num_pages, k.bt_stride = 4, 1
    assert L.ffa_kfmt_decode(ctypes.byref(k), None) == -1 and b"block table" in L.ffa_last_error()
    # a grid of more than 2^31 - 1 workgroups (the kernels number them in 32 bits): 32768 spans of
    # 512 tokens x 8 KV heads x 65535 sequences, refused before any launch
    k = N.KfmtArgs()
    k.B, k.T, k.HQ, k.HKV, k.BS, k.SBS = 65535, 1 << 24, 32, 8, 64, 64
    k.q_dtype, k.out_dtype, k.v_dtype, k.res_dtype = N.DT_BF16, N.DT_BF16, N.DT_BF16, N.DT_NONE
    k.layout, k.k_format, k.scale_kind = N.LAYOUT_CONTIG, N.KFMT_FP8_E4M3, N.KSCALE_NONE
    k.nparts, k.ntbs = 1 << 15, (1 << 24) // 64
    assert L.ffa_kfmt_decode(ctypes.byref(k), None) == -2 and b"2^31" in L.ffa_last_error()
    a = N.DecodeArgs()
    a.B, a.T, a.HQ, a.HKV, a.BS, a.SBS = 65535, 1 << 24, 32, 8, 64, 64
    a.q_dtype, a.out_dtype, a.v_dtype, a.res_dtype = N.DT_BF16, N.DT_BF16, N.DT_BF16, N.DT_NONE
    a.scale_dtype, a.scale_mode, a.layout = N.DT_F16, N.SCALE_CHANNEL, N.LAYOUT_CONTIG
    a.nparts, a.ntbs = 1 << 15, (1 << 24) // 64
    assert L.ffa_q2fp8_decode(ctypes.byref(a), None) == -2 and b"2^31" in L.ffa_last_error()
    # more than 65535 spans of 512 tokens in one sequence (the span count is a grid dimension)
    a.B, a.T = 1, (1 << 25) + 512
    a.nparts, a.ntbs = 65537, a.T // 64
    assert L.ffa_q2fp8_decode(ctypes.byref(a), None) == -2 and b"65535 workgroup spans" in L.ffa_last_error()
    k.B, k.T = 1, (1 << 25) + 512
    k.nparts, k.ntbs = 65537, k.T // 64
    assert L.ffa_kfmt_decode(ctypes.byref(k), None) == -2 and b"65535 workgroup spans" in L.ffa_last_error()


def test_drop_in_signatures_match_reference():
    import attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8 as K

    params = list(inspect.signature(K.attn_forward_decode_quantized).parameters)
    ref = ["q", "k_q", "k_scale", "k_zero", "v", "k_residual", "k_bits", "scale", "BS", "SBS", "delta",
           "return_skip_ratio", "precomputed_threshold", "use_fp8_residual"]
    assert params[: len(ref)] == ref
    sig = inspect.signature(K.attn_forward_decode_quantized)
    assert sig.parameters["BS"].default == 128 and sig.parameters["delta"].default == 5.0
    assert sig.parameters["use_fp8_residual"].default is True


def test_meanv_drop_in_loads_and_keeps_the_reference_signature():
    """ffa-q2fp8-meanv's two modules load (the mean-V one loads the q2fp8 drop-in while it loads)
    and keep the reference signature (..._meanv_bsz_q2fp8.py:222-238)."""
    import torch

    from ffa_mi355x.dropins import _ROOT, _load

    base = _ROOT / "ffa-q2fp8-meanv" / "attn_kernel"
    M = _load("ffa_mi355x_meanv_dropin", base / "attn_kernel_v1210_meanv_bsz_q2fp8.py")
    F = _load("ffa_mi355x_meanv_fused_copy", base / "attn_kernel_v1210_fused_bsz_q2fp8.py")
    ref = ["q", "k_q", "k_scale", "k_zero", "v", "k_residual", "k_bits", "scale", "BS", "SBS", "delta",
           "return_skip_ratio", "precomputed_threshold", "use_fp8_residual"]
    for mod in (M, F):
        params = list(inspect.signature(mod.attn_forward_decode_quantized).parameters)
        assert params[: len(ref)] == ref
    assert inspect.signature(M.attn_forward_decode_quantized).parameters["BS"].default == 128
    with pytest.raises(AssertionError):  # CPU tensors, as the reference's first check
        M.attn_forward_decode_quantized(torch.zeros(1, 1, 4, 128), torch.zeros(1, 8, 1, 32, dtype=torch.uint8),
                                        torch.zeros(1, 1, 128), torch.zeros(1, 1, 128), torch.zeros(1, 8, 1, 128))


def test_drop_in_rejects_cpu_tensors():
    import torch

    import attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8 as K

    q = torch.zeros(1, 1, 4, 128)
    with pytest.raises(AssertionError):
        K.attn_forward_decode_quantized(q, torch.zeros(1, 8, 1, 32, dtype=torch.uint8), torch.zeros(1, 1, 128),
                                        torch.zeros(1, 1, 128), torch.zeros(1, 8, 1, 128))


def test_graph_runner_interface_matches_reference():
    """CUDAGraphDecodeRunnerQ2FP8 keeps the reference constructor and methods (..._cudagraph.py:19-183)."""
    from attn_kernel.attn_kernel_v1210_fused_bsz_q2fp8_cudagraph import CUDAGraphDecodeRunnerQ2FP8 as R

    params = inspect.signature(R.__init__).parameters
    assert list(params)[1:6] == ["q", "k_q", "k_scale", "k_zero", "v"]
    for name, default in [("k_residual", None), ("precomputed_threshold", None), ("k_bits", 2), ("scale", None),
                          ("BS", 128), ("SBS", None), ("delta", 5.0), ("use_fp8_residual", True), ("warmup", 2)]:
        assert params[name].default == default and params[name].kind == inspect.Parameter.KEYWORD_ONLY
    assert R.__call__ is R.replay and callable(R.replay_only) and isinstance(R.output, property)
    rp = inspect.signature(R.replay).parameters
    assert list(rp)[1:6] == ["q", "k_q", "k_scale", "k_zero", "v"] and rp["return_skip_ratio"].default is False


def test_other_format_drop_in_signatures():
    """fp8fp8 / nvfp4 / nf4 decoders keep the reference parameter order and defaults
    (F8K:180-194, NVK:225-241, NFK:212-227)."""
    import importlib.util

    pkg = ROOT / "ffa-speedtest_amd"

    def load(rel, name):
        spec = importlib.util.spec_from_file_location(name, pkg / rel)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        return mod

    f8 = load("ffa-fp8fp8/attn_kernel/attn_kernel_v1210_fused_bsz_fp8fp8.py", "sig_fp8fp8").attn_forward_decode_fp8fp8
    nv = load("ffa-nvfp4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nvfp4fp8.py", "sig_nvfp4").attn_forward_decode_nvfp4fp8
    nf = load("ffa-nf4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nf4fp8.py", "sig_nf4").attn_forward_decode_nf4
    tail = ["scale", "BS", "SBS", "delta", "return_skip_ratio", "precomputed_threshold", "use_fp8_residual"]
    assert list(inspect.signature(f8).parameters)[:-1] == ["q", "k_fp8", "v", "k_residual"] + tail
    assert list(inspect.signature(nv).parameters)[:-1] == ["q", "k_fp4", "k_scale", "v", "k_residual", "k_bits"] + tail
    assert list(inspect.signature(nf).parameters)[:-1] == ["q", "k_nf4", "k_scale", "v", "k_residual", "k_bits"] + tail
    for fn in (f8, nv, nf):
        ps = inspect.signature(fn).parameters
        assert ps["BS"].default == 128 and ps["delta"].default == 5.0 and ps["use_fp8_residual"].default is True
    assert inspect.signature(nv).parameters["k_bits"].default == 4
    assert inspect.signature(f8).parameters["k_residual"].kind == inspect.Parameter.KEYWORD_ONLY
    assert inspect.signature(nf).parameters["k_residual"].kind == inspect.Parameter.POSITIONAL_OR_KEYWORD


def test_nvfp4_scale_normalisation_quirk():
    """The nvfp4 drop-in normalises k_scale as the reference does (NVK:213-222): a [B, HKV, NTB]
    tensor is transposed to [B, NTB, HKV], so when NTB == HKV a correctly shaped [B, NTB, HKV]
    tensor is transposed too.  Kept on purpose: the drop-in computes what the reference computes."""
    import importlib.util

    import torch

    spec = importlib.util.spec_from_file_location(
        "quirk_nvfp4", ROOT / "ffa-speedtest_amd/ffa-nvfp4fp8/attn_kernel/attn_kernel_v1210_fused_bsz_nvfp4fp8.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    s = torch.arange(2 * 9 * 8, dtype=torch.float32).reshape(2, 9, 8)  # NTB = 9, HKV = 8
    assert torch.equal(mod._normalize_k_scale(s, (2, 9, 8)), s)
    assert torch.equal(mod._normalize_k_scale(s.permute(0, 2, 1).contiguous(), (2, 9, 8)), s)
    sq = torch.arange(2 * 8 * 8, dtype=torch.float32).reshape(2, 8, 8)  # NTB == HKV == 8
    assert torch.equal(mod._normalize_k_scale(sq, (2, 8, 8)), sq.permute(0, 2, 1))


def _load_dropin(rel, name):
    import importlib.util

    spec = importlib.util.spec_from_file_location(name, ROOT / "ffa-speedtest_amd" / rel)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_other_format_producer_signatures():
    """Producer drop-ins keep the reference names, parameter order and defaults
    (F8F:58-135, NVF:62-190, NFF:72-96, 415-580)."""
    f8 = _load_dropin("ffa-fp8fp8/fused_kproj_rope_fp8fp8.py", "prod_fp8fp8")
    nv = _load_dropin("ffa-nvfp4fp8/fused_kproj_rope_nvfp4fp8.py", "prod_nvfp4")
    nf = _load_dropin("ffa-nf4fp8/fused_kproj_rope_nf4fp8.py", "prod_nf4")
    head = ["h", "w_k", "cos", "sin", "num_kv_heads", "head_dim"]
    for fn in (f8.kproj_rope_quantize_reference, f8.kproj_rope_quantize_fused, nf.kproj_rope_nf4_reference,
               nf.kproj_rope_nf4_fused):
        assert list(inspect.signature(fn).parameters) == head + ["bias", "fp8_dtype"]
    for fn in (nv.kproj_rope_quantize_reference, nv.kproj_rope_quantize_fused):
        assert list(inspect.signature(fn).parameters) == head + ["page_size", "bias", "fp8_dtype"]
    assert list(inspect.signature(nf.kproj_rope_nf4_triton).parameters) == head + [
        "bias", "fp8_dtype", "block_t", "block_h", "block_pair", "num_warps", "num_stages"]
    assert list(inspect.signature(f8.quantize_k_fp8_fp8_residual).parameters) == ["k", "fp8_dtype"]
    assert list(inspect.signature(nv.encode_k_nvfp4_fp8_residual).parameters) == ["k", "fp8_dtype", "page_size"]
    assert list(inspect.signature(nf.encode_k_nf4_fp8_residual).parameters) == ["k", "fp8_dtype"]
    # the codebook literal is the published NF4 table: 16 increasing levels from -1 to 1 with 0 at index 7
    cb = nf.NF4_CODEBOOK_VALUES
    assert len(cb) == 16 and cb[0] == -1.0 and cb[7] == 0.0 and cb[15] == 1.0
    assert all(a < b for a, b in zip(cb, cb[1:]))
    from oracle import formats as OF

    assert np.array_equal(np.array(cb, np.float32), OF.NF4_CODEBOOK)


def test_rope_helpers_closed_form():
    """build_rope_cache / rotate_half / apply_rope: angle t * base^(-2i/D) for channels i and i + D/2,
    interleaved pair rotation, and a rotation preserves each pair's norm."""
    import torch

    from ffa_mi355x import rope

    T, D = 7, 8
    cos, sin = rope.build_rope_cache(T, D, base=500000.0)
    i = np.arange(D) % (D // 2)
    ang = np.arange(T)[:, None] * (1.0 / 500000.0 ** (2.0 * i / D))[None, :]
    assert np.allclose(cos.numpy(), np.cos(ang), atol=1e-6) and np.allclose(sin.numpy(), np.sin(ang), atol=1e-6)
    x = torch.arange(1, 9, dtype=torch.float32).view(1, 1, 1, 8)
    assert rope.rotate_half(x).flatten().tolist() == [-2, 1, -4, 3, -6, 5, -8, 7]
    xr = torch.randn(2, T, 3, D)
    y = rope.apply_rope(xr, cos, sin)
    # pairs (2j, 2j+1) use angles of channels 2j and 2j+1; with equal angles a pair keeps its norm
    c2, s2 = rope.build_rope_cache(T, 2)
    y2 = rope.apply_rope(xr[..., :2], c2, s2)
    assert torch.allclose(y2.norm(dim=-1), xr[..., :2].norm(dim=-1), atol=1e-5)
    assert y.shape == xr.shape
    # rope_rows: the rows of build_rope_cache's table at the given positions (fp32 angles)
    cr, sr = rope.rope_rows(torch.tensor([0, 3, 6]), head_dim=D, base=500000.0)
    assert torch.allclose(cr, cos[[0, 3, 6]], atol=1e-6) and torch.allclose(sr, sin[[0, 3, 6]], atol=1e-6)


def test_page_orders_match_the_kernels(tmp_path):
    """The numpy page orders (ffa_mi355x.paged) equal decode_common.h's offset functions, and each
    is a permutation of its block."""
    import shutil
    import subprocess

    from ffa_mi355x import paged as PG

    for order, n in ((PG.RES_ORDER, 8192), (PG.VT_ORDER, 8192), (PG.CODES_ORDER, 256), (PG.GSCALE_ORDER, 256),
                     (PG.K4_ORDER, 4096)):
        assert np.array_equal(np.sort(order.ravel()), np.arange(n))
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    src = tmp_path / "orders.cpp"
    src.write_text('#include <stdio.h>\n#include "decode_common.h"\nint main() {\n'
                   '  for (int t = 0; t < 64; ++t) for (int c = 0; c < 128; ++c) printf("%u ", ffa::res_off(t, c));\n'
                   '  printf("\\n");\n'
                   '  for (int c = 0; c < 128; ++c) for (int t = 0; t < 64; ++t) printf("%u ", ffa::vt_off(c, t));\n'
                   '  printf("\\n");\n'
                   '  for (int g = 0; g < 4; ++g) for (int t = 0; t < 64; ++t) printf("%u ", ffa::codes_off(g, t) / 8);\n'
                   '  printf("\\n");\n'
                   '  for (int g = 0; g < 4; ++g) for (int s = 0; s < 64; ++s) printf("%u ", ffa::gscale_off(g, s));\n'
                   '  printf("\\n");\n'
                   '  for (int t = 0; t < 64; ++t) for (int b = 0; b < 64; ++b) printf("%u ", ffa::k4_off(t, b));\n'
                   '  printf("\\n");\n  return 0;\n}\n')
    exe = tmp_path / "orders"
    csrc = ROOT / "ffa-speedtest_amd" / "csrc"
    r = subprocess.run([hipcc, "-x", "hip", "--offload-arch=gfx950", "-std=c++17", f"-I{csrc}", f"-I{ROOT / 'include'}",
                        str(src), "-o", str(exe)], capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip(f"host build of decode_common.h failed: {r.stderr[:200]}")
    lines = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines()
    got = [np.array(line.split(), dtype=np.int64) for line in lines]
    for g, order in zip(got, (PG.RES_ORDER, PG.VT_ORDER, PG.CODES_ORDER, PG.GSCALE_ORDER, PG.K4_ORDER)):
        assert np.array_equal(g, order.ravel())


def test_kernel_sources_have_no_register_writing_inline_asm():
    """Inline assembly is opaque to the compiler's hazard checks: a VALU write inside an asm block
    gets the wait states the compiler would give an unknown instruction, not the two an MFMA read of
    the same register needs, so the MFMA can read the register's previous value (a deterministic
    wrong score that comes and goes with register allocation).  The kernels keep only asm that
    writes no register: waits and barriers, and empty constraint-only statements."""
    allowed = {"", "s_waitcnt lgkmcnt(0)\\n\\ts_barrier"}
    found = []
    for src in sorted((ROOT / "ffa-speedtest_amd" / "csrc").glob("*.[hc]*")):
        text = re.sub(r"//[^\n]*", "", src.read_text())
        for m in re.finditer(r"\basm\s*(?:volatile\s*)?\(\s*\"((?:[^\"\\]|\\.)*)\"", text):
            found.append((src.name, m.group(1)))
    assert found, "no asm statements found: the pattern no longer matches the sources"
    bad = [(f, body) for f, body in found if body not in allowed]
    assert not bad, f"inline asm that emits instructions other than waits and barriers: {bad}"
