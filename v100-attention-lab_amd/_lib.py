"""ctypes binding of the C ABI declared in ``include/gdn_mi355x.h``."""

from __future__ import annotations

import ctypes
import os
import threading

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "lib", "libgdn_mi355x.so")

ABI_VERSION = 5

# enum GdnDtype
DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

# enum GdnStatus (argument errors; other non-zero values are hipError_t)
GDN_OK = 0
GDN_ERR_NULL_POINTER = 1001
GDN_ERR_BAD_SHAPE = 1002
GDN_ERR_UNSUPPORTED = 1003
GDN_ERR_MISALIGNED = 1004
GDN_ERR_BAD_DTYPE = 1005
GDN_ERR_WORKSPACE = 1006
GDN_ERR_SCRATCH_LIMIT = 1007

# enum GdnFlags
FLAG_PHASED_KERNEL = 1
FLAG_FUSED_KERNEL = 2

# Every symbol the header declares; tests check the library exports them.
EXPORTED_SYMBOLS = (
    "gdn_fwd_launch",
    "gdn_fwd_workspace_size",
    "gdn_fwd_auto_block_v",
    "gdn_fwd_status_string",
    "gdn_fwd_abi_version",
    "gdn_prep_launch",
    "gdn_bwd_workspace_size",
    "gdn_bwd_workspace_size_params",
    "gdn_bwd_segment_workspace_size",
    "gdn_bwd_launch",
    "gdn_fwd_launch_noalloc",
    "gdn_fwd_scratch_bytes",
)

_I64x3 = ctypes.c_int64 * 3
_I64x4 = ctypes.c_int64 * 4


class GdnFwdParams(ctypes.Structure):
    """Mirror of ``struct GdnFwdParams`` (field order and types match)."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("g", ctypes.c_void_p),
        ("beta", ctypes.c_void_p),
        ("h0", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("final_state", ctypes.c_void_p),
        ("q_stride", _I64x3),
        ("k_stride", _I64x3),
        ("v_stride", _I64x3),
        ("g_stride", _I64x3),
        ("beta_stride", _I64x3),
        ("o_stride", _I64x3),
        ("h0_stride", _I64x4),
        ("fs_stride", _I64x4),
        ("B", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("K", ctypes.c_int32),
        ("V", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("chunk_size", ctypes.c_int32),
        ("block_v", ctypes.c_int32),
        ("qkv_dtype", ctypes.c_int32),
        ("g_dtype", ctypes.c_int32),
        ("beta_dtype", ctypes.c_int32),
        ("o_dtype", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("cu_seqlens", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_int64),
    ]


class GdnPrepParams(ctypes.Structure):
    """Mirror of ``GdnPrepParams`` in include/gdn_mi355x.h."""

    _fields_ = [
        ("q_in", ctypes.c_void_p),
        ("q_out", ctypes.c_void_p),
        ("k_in", ctypes.c_void_p),
        ("k_out", ctypes.c_void_p),
        ("beta_in", ctypes.c_void_p),
        ("beta_out", ctypes.c_void_p),
        ("g_in", ctypes.c_void_p),
        ("g_out", ctypes.c_void_p),
        ("q_in_stride", _I64x3),
        ("q_out_stride", _I64x3),
        ("k_in_stride", _I64x3),
        ("k_out_stride", _I64x3),
        ("beta_in_stride", _I64x3),
        ("beta_out_stride", _I64x3),
        ("g_in_stride", _I64x3),
        ("g_out_stride", _I64x3),
        ("B", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("K", ctypes.c_int32),
        ("qk_dtype", ctypes.c_int32),
        ("beta_in_dtype", ctypes.c_int32),
        ("beta_out_dtype", ctypes.c_int32),
        ("g_in_dtype", ctypes.c_int32),
        ("g_out_dtype", ctypes.c_int32),
        ("eps", ctypes.c_float),
    ]


class GdnBwdParams(ctypes.Structure):
    """Mirror of ``GdnBwdParams`` in include/gdn_mi355x.h."""

    _fields_ = [(n, ctypes.c_void_p) for n in (
        "q", "k", "v", "g", "beta", "h0", "d_o", "d_final_state",
        "dq", "dk", "dv", "dg", "dbeta", "dh0", "workspace")] + \
        [(n, _I64x3) for n in (
            "q_stride", "k_stride", "v_stride", "g_stride", "beta_stride", "do_stride",
            "dq_stride", "dk_stride", "dv_stride", "dg_stride", "dbeta_stride")] + \
        [(n, _I64x4) for n in ("h0_stride", "dfs_stride", "dh0_stride")] + \
        [(n, ctypes.c_int32) for n in ("B", "T", "H", "K", "V")] + \
        [("scale", ctypes.c_float)] + \
        [(n, ctypes.c_int32) for n in ("qkv_dtype", "g_dtype", "beta_dtype", "do_dtype")] + \
        [("cu_seqlens", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64)]


_lock = threading.Lock()
_lib = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the built HIP library (once).  Raises ImportError if it is missing.

    There is no fallback: without the library the GDN forward is unavailable.
    """
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise ImportError(
                f"GDN HIP library not found at {path}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` or "
                "`python v100-attention-lab_amd/build.py`")
        lib = ctypes.CDLL(path)
        lib.gdn_fwd_launch.argtypes = [ctypes.POINTER(GdnFwdParams), ctypes.c_void_p]
        lib.gdn_fwd_launch.restype = ctypes.c_int
        lib.gdn_fwd_launch_noalloc.argtypes = [ctypes.POINTER(GdnFwdParams), ctypes.c_void_p]
        lib.gdn_fwd_launch_noalloc.restype = ctypes.c_int
        lib.gdn_fwd_scratch_bytes.argtypes = []
        lib.gdn_fwd_scratch_bytes.restype = ctypes.c_int64
        lib.gdn_fwd_workspace_size.argtypes = [ctypes.POINTER(GdnFwdParams)]
        lib.gdn_fwd_workspace_size.restype = ctypes.c_int64
        lib.gdn_fwd_auto_block_v.argtypes = [ctypes.c_int] * 6
        lib.gdn_fwd_auto_block_v.restype = ctypes.c_int
        lib.gdn_fwd_status_string.argtypes = [ctypes.c_int]
        lib.gdn_fwd_status_string.restype = ctypes.c_char_p
        lib.gdn_prep_launch.argtypes = [ctypes.POINTER(GdnPrepParams), ctypes.c_void_p]
        lib.gdn_prep_launch.restype = ctypes.c_int
        lib.gdn_bwd_launch.argtypes = [ctypes.POINTER(GdnBwdParams), ctypes.c_void_p]
        lib.gdn_bwd_launch.restype = ctypes.c_int
        lib.gdn_bwd_workspace_size.argtypes = [ctypes.c_int] * 6
        lib.gdn_bwd_workspace_size.restype = ctypes.c_int64
        lib.gdn_bwd_workspace_size_params.argtypes = [ctypes.POINTER(GdnBwdParams)]
        lib.gdn_bwd_workspace_size_params.restype = ctypes.c_int64
        lib.gdn_bwd_segment_workspace_size.argtypes = [ctypes.POINTER(GdnBwdParams), ctypes.c_int]
        lib.gdn_bwd_segment_workspace_size.restype = ctypes.c_int64
        lib.gdn_fwd_abi_version.argtypes = []
        lib.gdn_fwd_abi_version.restype = ctypes.c_int
        ver = lib.gdn_fwd_abi_version()
        if ver != ABI_VERSION:
            raise ImportError(f"{path}: ABI version {ver}, expected {ABI_VERSION}; rebuild")
        _lib = lib
        return lib


def status_string(code: int) -> str:
    return load_library().gdn_fwd_status_string(int(code)).decode()
