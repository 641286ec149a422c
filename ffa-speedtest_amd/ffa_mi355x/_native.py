"""ctypes binding of libffa_mi355x.so (the C ABI declared in include/ffa_mi355x.h).

The library is the only compute path: if it is missing or does not load,
every entry point raises; there is no CPU or PyTorch fallback.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libffa_mi355x.so"

# element type codes (ffa_mi355x.h)
DT_F16, DT_BF16, DT_F32, DT_FP8_E4M3, DT_FP8_E5M2, DT_NONE = range(6)
LAYOUT_CONTIG, LAYOUT_PAGED = 0, 1
SCALE_CHANNEL, SCALE_G32 = 0, 1
KFMT_FP8_E4M3, KFMT_FP8_E5M2, KFMT_NVFP4, KFMT_NF4 = range(4)
KSCALE_NONE, KSCALE_TOKEN, KSCALE_BLOCK, KSCALE_CHANNEL, KSCALE_G16, KSCALE_G64 = range(6)

EXPORTS = (
    "ffa_q2fp8_decode_nparts",
    "ffa_q2fp8_decode_pieces",
    "ffa_q2fp8_decode",
    "ffa_q2fp8_decode_stage1",
    "ffa_q2fp8_decode_stage2",
    "ffa_q2fp8_decode_noalloc",
    "ffa_v_mean_nsplit",
    "ffa_v_mean",
    "ffa_kfmt_decode",
    "ffa_q2_quantize_nsplit",
    "ffa_q2_quantize_channel",
    "ffa_q2_append_channel",
    "ffa_kproj_rope_q2_channel",
    "ffa_kproj_rope_q2_append",
    "ffa_q2_quantize_g32_append",
    "ffa_q2_paged_dequant",
    "ffa_kproj_rope",
    "ffa_fp8fp8_quantize",
    "ffa_fp8_scaled_quantize",
    "ffa_nvfp4_quantize",
    "ffa_nf4_quantize_nsplit",
    "ffa_nf4_quantize",
    "ffa_nvfp4_g16_append",
    "ffa_nf4_g64_append",
    "ffa_last_error",
    "ffa_version",
)

_TORCH_DT = {
    torch.float16: DT_F16,
    torch.bfloat16: DT_BF16,
    torch.float32: DT_F32,
    torch.float8_e4m3fn: DT_FP8_E4M3,
    torch.float8_e5m2: DT_FP8_E5M2,
}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _TORCH_DT[dt]
    except KeyError:
        raise ValueError(f"unsupported dtype {dt}") from None


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("q_dtype", ctypes.c_int),
        ("k_q", ctypes.c_void_p),
        ("k_scale", ctypes.c_void_p),
        ("k_zero", ctypes.c_void_p),
        ("scale_dtype", ctypes.c_int),
        ("scale_mode", ctypes.c_int),
        ("k_residual", ctypes.c_void_p),
        ("res_dtype", ctypes.c_int),
        ("v", ctypes.c_void_p),
        ("v_dtype", ctypes.c_int),
        ("layout", ctypes.c_int),
        ("block_table", ctypes.c_void_p),
        ("bt_stride", ctypes.c_int),
        ("seq_lens", ctypes.c_void_p),
        ("B", ctypes.c_int),
        ("T", ctypes.c_int),
        ("HQ", ctypes.c_int),
        ("HKV", ctypes.c_int),
        ("scale", ctypes.c_float),
        ("BS", ctypes.c_int),
        ("SBS", ctypes.c_int),
        ("delta", ctypes.c_float),
        ("threshold_in", ctypes.c_void_p),
        ("threshold_out", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("out_dtype", ctypes.c_int),
        ("m_buf", ctypes.c_void_p),
        ("l_buf", ctypes.c_void_p),
        ("o_buf", ctypes.c_void_p),
        ("nparts", ctypes.c_int),
        ("mask", ctypes.c_void_p),
        ("ntbs", ctypes.c_int),
        ("num_pages", ctypes.c_int),
        ("piece_max", ctypes.c_void_p),
        ("npieces", ctypes.c_int),
        ("v_mean", ctypes.c_void_p),
        ("v_mean_dtype", ctypes.c_int),
        ("approx_m", ctypes.c_void_p),
        ("approx_l", ctypes.c_void_p),
        ("scale_exact_f16", ctypes.c_int),
    ]


class KfmtArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("q_dtype", ctypes.c_int),
        ("k", ctypes.c_void_p),
        ("k_format", ctypes.c_int),
        ("k_scale", ctypes.c_void_p),
        ("scale_dtype", ctypes.c_int),
        ("scale_kind", ctypes.c_int),
        ("k_residual", ctypes.c_void_p),
        ("res_dtype", ctypes.c_int),
        ("v", ctypes.c_void_p),
        ("v_dtype", ctypes.c_int),
        ("seq_lens", ctypes.c_void_p),
        ("B", ctypes.c_int),
        ("T", ctypes.c_int),
        ("HQ", ctypes.c_int),
        ("HKV", ctypes.c_int),
        ("scale", ctypes.c_float),
        ("BS", ctypes.c_int),
        ("SBS", ctypes.c_int),
        ("delta", ctypes.c_float),
        ("threshold_in", ctypes.c_void_p),
        ("threshold_out", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("out_dtype", ctypes.c_int),
        ("m_buf", ctypes.c_void_p),
        ("l_buf", ctypes.c_void_p),
        ("o_buf", ctypes.c_void_p),
        ("nparts", ctypes.c_int),
        ("mask", ctypes.c_void_p),
        ("ntbs", ctypes.c_int),
        ("layout", ctypes.c_int),
        ("block_table", ctypes.c_void_p),
        ("bt_stride", ctypes.c_int),
        ("num_pages", ctypes.c_int),
        ("piece_max", ctypes.c_void_p),
        ("npieces", ctypes.c_int),
    ]


_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load the native library once; raise if it is absent (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "(hipcc --offload-arch=gfx950).  There is no CPU fallback."
            )
        L = ctypes.CDLL(str(LIB_PATH))
        vp, ci, cf = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.ffa_last_error.restype = ctypes.c_char_p
        L.ffa_version.restype = ctypes.c_char_p
        L.ffa_q2fp8_decode_nparts.argtypes = [ci, ci, ci]
        L.ffa_q2fp8_decode_pieces.argtypes = [ci, ci, ci, ci, ci]
        L.ffa_q2fp8_decode_pieces.restype = ci
        L.ffa_q2fp8_decode_nparts.restype = ci
        for name in ("ffa_q2fp8_decode", "ffa_q2fp8_decode_stage1", "ffa_q2fp8_decode_stage2",
                     "ffa_q2fp8_decode_noalloc"):
            getattr(L, name).argtypes = [ctypes.POINTER(DecodeArgs), vp]
            getattr(L, name).restype = ci
        L.ffa_v_mean_nsplit.argtypes = [ci]
        L.ffa_v_mean_nsplit.restype = ci
        L.ffa_v_mean.argtypes = [vp, ci, ci, vp, ci, ci, vp, ci, ci, ci, vp, ci, vp, ci, vp]
        L.ffa_v_mean.restype = ci
        L.ffa_kfmt_decode.argtypes = [ctypes.POINTER(KfmtArgs), vp]
        L.ffa_kfmt_decode.restype = ci
        L.ffa_q2_quantize_nsplit.argtypes = [ci]
        L.ffa_q2_quantize_nsplit.restype = ci
        L.ffa_q2_quantize_channel.argtypes = [vp, ci, ci, ci, ci, ci, vp, vp, vp, vp, ci, vp, vp]
        L.ffa_q2_append_channel.argtypes = [vp, ci, ci, ci, ci, ci, vp, ci, vp, vp, vp, vp, ci, vp]
        L.ffa_q2_append_channel.restype = ci
        L.ffa_q2_quantize_channel.restype = ci
        L.ffa_kproj_rope_q2_channel.argtypes = [vp, vp, vp, ci, vp, vp, ci, ci, ci, ci, ci, ci, vp, vp, vp, vp, vp,
                                                ci, vp, vp]
        L.ffa_kproj_rope_q2_channel.restype = ci
        L.ffa_kproj_rope_q2_append.argtypes = [vp, vp, vp, ci, vp, vp, ci, ci, ci, ci, vp, vp, ci, ci, vp, vp, vp,
                                               vp, ci, vp, vp, ci, vp]
        L.ffa_kproj_rope_q2_append.restype = ci
        L.ffa_q2_quantize_g32_append.argtypes = [vp, ci, ci, ci, ci, vp, vp, ci, ci, vp, vp, vp, vp, ci, vp, vp, vp]
        L.ffa_q2_quantize_g32_append.restype = ci
        L.ffa_q2_paged_dequant.argtypes = [vp, vp, vp, vp, ci, vp, ci, vp, ci, ci, vp, ci, ci, ci, vp, vp, ci, vp]
        L.ffa_q2_paged_dequant.restype = ci
        L.ffa_kproj_rope.argtypes = [vp, vp, vp, ci, vp, vp, ci, ci, ci, ci, ci, ci, vp, vp]
        L.ffa_kproj_rope.restype = ci
        L.ffa_fp8fp8_quantize.argtypes = [vp, ci, ctypes.c_size_t, vp, vp, ci, vp]
        L.ffa_fp8fp8_quantize.restype = ci
        L.ffa_fp8_scaled_quantize.argtypes = [vp, ci, ctypes.c_size_t, ci, vp, vp, vp, ci, vp]
        L.ffa_fp8_scaled_quantize.restype = ci
        L.ffa_nvfp4_quantize.argtypes = [vp, ci, ci, ci, ci, ci, ci, vp, vp, vp, ci, vp]
        L.ffa_nvfp4_quantize.restype = ci
        L.ffa_nf4_quantize_nsplit.argtypes = [ci]
        L.ffa_nf4_quantize_nsplit.restype = ci
        L.ffa_nf4_quantize.argtypes = [vp, ci, ci, ci, ci, ci, vp, vp, vp, ci, vp, vp]
        L.ffa_nf4_quantize.restype = ci
        for name in ("ffa_nvfp4_g16_append", "ffa_nf4_g64_append"):
            getattr(L, name).argtypes = [vp, ci, ci, ci, ci, vp, vp, ci, ci, vp, vp, vp, ci, vp, vp, vp]
            getattr(L, name).restype = ci
        _lib = L
        return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().ffa_last_error().decode(errors="replace")
        if rc == -2:
            raise NotImplementedError(f"{what}: {msg}")
        if rc == -1:
            raise ValueError(f"{what}: {msg}")
        raise RuntimeError(f"{what}: {msg} (rc={rc})")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
