"""ctypes binding of ``libctmr_hip.so`` (declarations in ``include/ctmr.h``).

This is the only bridge between Python and the HIP kernels.  There is no
fallback: if the library is missing or cannot be loaded, every operator raises.
"""

from __future__ import annotations

import ctypes
import re
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libctmr_hip.so")
HEADER_PATH = Path(__file__).resolve().parent.parent / "include" / "ctmr.h"

# enum values mirrored from include/ctmr.h
OK = 0
E_INVALID, E_UNSUPPORTED, E_WORKSPACE, E_LAUNCH = -1, -2, -3, -4
MODE_PLAIN, MODE_NEAREST2X, MODE_TRILINEAR2X = 0, 1, 2
F_AFFINE, F_SILU, F_BATCH_BIAS, F_RESIDUAL, F_STREAM, F_SPLIT_WAVES = 1, 2, 4, 8, 16, 32
DT_F32, DT_BF16, DT_F16X2 = 0, 1, 2
(K_STREAM, K_STREAM_DIRECT, K_LDS, K_LDS_BF16, K_POINTWISE, K_SPLIT_WAVES, K_TAP_EXPAND, K_LDS_SMALL,
 K_SMALL_COUT, K_LDS_F16X2) = range(10)
KERNEL_NAMES = ("stream", "stream_direct", "lds", "lds_bf16", "pointwise", "split_waves", "tap_expand", "lds_small",
                "small_cout", "lds_f16x2")
AVGPOOL2, NEAREST2X, TRILINEAR2X = 0, 1, 2
ABI_VERSION = 5
NOALLOC_SCRATCH_BYTES = 256 << 20  # CTMR_NOALLOC_SCRATCH_BYTES


class ConvDesc(ctypes.Structure):
    """``ctmr_conv_desc``."""

    _fields_ = [
        (name, ctypes.c_int32)
        for name in ("n", "d", "h", "w", "cin", "cout", "ksize", "stride", "mode", "flags", "dtype", "split",
                     "cin1")
    ]


class AttnDesc(ctypes.Structure):
    """``ctmr_attn_desc``."""

    _fields_ = [(name, ctypes.c_int32) for name in ("n", "lq", "lk", "heads", "head_dim", "query_tiles")] + [
        (name, ctypes.c_int64) for name in ("ldq", "ldk", "ldv", "ldo")
    ] + [("scale", ctypes.c_float)]


_c_int, _c_i32, _c_i64 = ctypes.c_int, ctypes.c_int32, ctypes.c_int64
_vp, _sz, _f = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float
_desc_p = ctypes.POINTER(ConvDesc)

_PROTOTYPES = {
    "ctmr_abi_version": (_c_int, []),
    "ctmr_last_error": (ctypes.c_char_p, []),
    "ctmr_conv3d_output_dims": (_c_int, [_desc_p, ctypes.POINTER(_c_i32)]),
    "ctmr_packed_weight_elems": (_c_i64, [_desc_p]),
    "ctmr_conv3d_workspace_bytes": (_c_i64, [_desc_p]),
    "ctmr_conv3d_split": (_c_int, [_desc_p]),
    "ctmr_conv3d_kernel": (_c_int, [_desc_p]),
    "ctmr_pack_weight": (_c_int, [_desc_p, _vp, _vp, _vp]),
    "ctmr_pack_upsample_weight": (_c_int, [_desc_p, _vp, _vp, _vp]),
    "ctmr_conv3d": (_c_int, [_desc_p, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ctmr_conv3d_noalloc": (_c_int, [_desc_p, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ctmr_conv3d_pack": (_c_int, [_desc_p, _vp, _vp, _vp, _sz, _vp]),
    "ctmr_conv3d_gemm": (_c_int, [_desc_p, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ctmr_conv3d_stats_tiles": (_c_i32, [_desc_p, _c_i32]),
    "ctmr_conv3d_gn": (_c_int, [_desc_p, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _c_i32, _vp, _vp]),
    "ctmr_conv3d_cat": (_c_int, [_desc_p, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ctmr_conv3d_cat_gn": (_c_int, [_desc_p, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _c_i32, _vp, _vp]),
    "ctmr_gn_workspace_bytes": (_c_i64, [_c_i32, _c_i64, _c_i32]),
    "ctmr_gn_affine": (_c_int, [_c_i32, _c_i64, _c_i32, _c_i32, _f, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ctmr_gn_affine_cat": (_c_int, [_c_i32, _c_i64, _c_i32, _c_i32, _c_i32, _f, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                                    _vp]),
    "ctmr_gn_affine_from_stats": (_c_int, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i64, _f, _vp, _vp, _vp, _vp, _vp]),
    "ctmr_gn_affine_from_stats2": (_c_int, [_c_i32, _c_i32, _c_i64, _f, _vp, _c_i32, _c_i32, _c_i32, _vp, _c_i32,
                                            _c_i32, _c_i32, _vp, _vp, _vp, _vp]),
    "ctmr_add_gn_partials": (_c_int, [_c_i32, _c_i64, _c_i32, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ctmr_gn_apply": (_c_int, [_c_i32, _c_i64, _c_i32, _vp, _vp, _c_i32, _vp, _vp]),
    "ctmr_silu": (_c_int, [_c_i64, _vp, _vp, _vp]),
    "ctmr_resample": (_c_int, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _vp, _vp, _vp]),
    "ctmr_gn_avgpool": (_c_int, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _vp, _vp, _c_i32, _vp, _vp, _vp]),
    "ctmr_flash_attention": (_c_int, [ctypes.POINTER(AttnDesc), _vp, _vp, _vp, _vp, _vp]),
    "ctmr_flash_attention_f16x2_workspace_bytes": (_c_i64, [ctypes.POINTER(AttnDesc)]),
    "ctmr_flash_attention_f16x2": (_c_int, [ctypes.POINTER(AttnDesc), _vp, _vp, _vp, _vp, _vp, _c_i64, _vp]),
}

_lock = threading.Lock()
_handle: ctypes.CDLL | None = None


class CtmrError(RuntimeError):
    """A non-zero status from the HIP library."""


def header_symbols() -> list[str]:
    """Function names declared in ``include/ctmr.h``."""
    text = HEADER_PATH.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+[\s\*]+(ctmr_\w+)\s*\(", text, re.M)))


def lib() -> ctypes.CDLL:
    """Load the library once (thread-safe) and declare every prototype."""
    global _handle
    if _handle is not None:
        return _handle
    with _lock:
        if _handle is None:
            if not LIB_PATH.exists():
                raise CtmrError(
                    f"{LIB_PATH.name} is not built; run __graft_entry__.build() "
                    "(there is no non-HIP fallback)"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in _PROTOTYPES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            if handle.ctmr_abi_version() != ABI_VERSION:
                raise CtmrError("libctmr_hip.so ABI version mismatch")
            _handle = handle
    return _handle


def last_error() -> str:
    """Message of the last failing call on this thread."""
    raw = lib().ctmr_last_error()
    return raw.decode() if raw else ""


def check(status: int, what: str) -> int:
    """Raise ``CtmrError`` for a negative status, else return it."""
    if status < 0:
        raise CtmrError(f"{what} failed with status {status}: {last_error()}")
    return status


def conv_desc(
    n: int,
    d: int,
    h: int,
    w: int,
    cin: int,
    cout: int,
    *,
    ksize: int = 3,
    stride: int = 1,
    mode: int = MODE_PLAIN,
    flags: int = 0,
    dtype: int = DT_F32,
    split: int = 0,
    cin1: int = 0,
) -> ConvDesc:
    """Build a ``ctmr_conv_desc`` (``cin1``: channels of the first of two input tensors, 0 for one)."""
    return ConvDesc(n, d, h, w, cin, cout, ksize, stride, mode, flags, dtype, split, cin1)


def output_dims(desc: ConvDesc) -> tuple[int, int, int]:
    """Output spatial extent of a described conv."""
    out = (ctypes.c_int32 * 3)()
    check(lib().ctmr_conv3d_output_dims(ctypes.byref(desc), out), "ctmr_conv3d_output_dims")
    return int(out[0]), int(out[1]), int(out[2])


def packed_weight_elems(desc: ConvDesc) -> int:
    return check(lib().ctmr_packed_weight_elems(ctypes.byref(desc)), "ctmr_packed_weight_elems")


def workspace_bytes(desc: ConvDesc) -> int:
    return check(lib().ctmr_conv3d_workspace_bytes(ctypes.byref(desc)), "ctmr_conv3d_workspace_bytes")


def conv_split(desc: ConvDesc) -> int:
    return check(lib().ctmr_conv3d_split(ctypes.byref(desc)), "ctmr_conv3d_split")


def conv_kernel(desc: ConvDesc) -> str:
    """Name of the GEMM formulation ``ctmr_conv3d`` runs for ``desc`` (``ctmr_conv3d_kernel``)."""
    return KERNEL_NAMES[check(lib().ctmr_conv3d_kernel(ctypes.byref(desc)), "ctmr_conv3d_kernel")]


def gn_workspace_bytes(n: int, s: int, c: int) -> int:
    return check(lib().ctmr_gn_workspace_bytes(n, s, c), "ctmr_gn_workspace_bytes")
