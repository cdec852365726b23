"""ctypes binding of libqmla.so (the C ABI declared in include/qmla.h).

torch is imported first on purpose: torch ships the HIP runtime (libamdhip64.so.7) and the library
must bind to that same runtime instance so streams and device pointers are shared.
"""
from __future__ import annotations

import ctypes
import os
import pathlib

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

LIB_NAME = "libqmla.so"
LIB_PATH = pathlib.Path(__file__).resolve().parent / LIB_NAME

ABI_VERSION = 2

# error codes (include/qmla.h)
OK = 0
ERR_NULL, ERR_SHAPE, ERR_ALIGN, ERR_WORKSPACE, ERR_MODE, ERR_LAUNCH, ERR_NOKERNEL, ERR_PAGE = -1, -2, -3, -4, -5, -6, -7, -8
ERR_NAMES = {
    ERR_NULL: "QMLA_ERR_NULL (a required pointer is NULL)",
    ERR_SHAPE: "QMLA_ERR_SHAPE (unsupported or inconsistent dimension)",
    ERR_ALIGN: "QMLA_ERR_ALIGN (row, page or base address off 4-byte boundaries, or off 16-byte ones in a layout "
               "no narrow-row kernel serves)",
    ERR_WORKSPACE: "QMLA_ERR_WORKSPACE (workspace missing or too small)",
    ERR_MODE: "QMLA_ERR_MODE (unknown dtype / rms mode / split mode)",
    ERR_LAUNCH: "QMLA_ERR_LAUNCH (HIP launch failed)",
    ERR_NOKERNEL: "QMLA_ERR_NOKERNEL (no compiled kernel instance for this shape)",
    ERR_PAGE: "QMLA_ERR_PAGE (a block-table entry outside [0, num_pages))",
}

KV_BF16, KV_FP8 = 0, 1
RMS_NONE, RMS_BF16, RMS_LOG8, RMS_BF16_BYTES, RMS_E4M3 = 0, 1, 2, 3, 4
DT_BF16, DT_F32, DT_F16 = 0, 1, 2
STATIC_SCRATCH_BYTES = 64 << 20   # QMLA_STATIC_SCRATCH_BYTES


class DecodeParams(ctypes.Structure):
    """Mirror of `qmla_decode_params` (include/qmla.h); field order and types must match."""

    _fields_ = [
        ("q_nope", ctypes.c_void_p),
        ("q_nope_stride_row", ctypes.c_int64),
        ("q_nope_stride_head", ctypes.c_int64),
        ("q_pe", ctypes.c_void_p),
        ("q_pe_stride_row", ctypes.c_int64),
        ("q_pe_stride_head", ctypes.c_int64),
        ("kv_cache", ctypes.c_void_p),
        ("page_stride", ctypes.c_int64),
        ("token_stride", ctypes.c_int64),
        ("kv_dtype", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("d_c", ctypes.c_int32),
        ("rope_w", ctypes.c_int32),
        ("rms_offset", ctypes.c_int32),
        ("rms_mode", ctypes.c_int32),
        ("k_scale", ctypes.c_void_p),
        ("sm_scale", ctypes.c_float),
        ("logit_cap", ctypes.c_float),
        ("block_table", ctypes.c_void_p),
        ("bt_stride", ctypes.c_int64),
        ("seq_lens", ctypes.c_void_p),
        ("rows", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("rms_heads", ctypes.c_int32),
        ("qrows", ctypes.c_int32),
        ("groups", ctypes.c_int32),
        ("out", ctypes.c_void_p),
        ("out_stride_row", ctypes.c_int64),
        ("out_stride_head", ctypes.c_int64),
        ("out_dtype", ctypes.c_int32),
        ("lse", ctypes.c_void_p),
        ("lse_stride_row", ctypes.c_int64),
        ("lse_dtype", ctypes.c_int32),
        ("num_splits", ctypes.c_int32),
        ("split_align", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("ws_stride_row", ctypes.c_int64),
        ("ws_stride_head", ctypes.c_int64),
        ("ws_stride_split", ctypes.c_int64),
        ("num_workgroups", ctypes.c_int32),
        ("num_pages", ctypes.c_int32),
        ("status", ctypes.c_void_p),
    ]


class CacheWriteParams(ctypes.Structure):
    """Mirror of `qmla_cache_write_params` (include/qmla.h); field order and types must match."""

    _fields_ = [
        ("kv_c", ctypes.c_void_p),
        ("kv_c_stride", ctypes.c_int64),
        ("k_pe", ctypes.c_void_p),
        ("k_pe_stride", ctypes.c_int64),
        ("slots", ctypes.c_void_p),
        ("n", ctypes.c_int32),
        ("d_c", ctypes.c_int32),
        ("rope_w", ctypes.c_int32),
        ("rms_heads", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32),
        ("rms_mode", ctypes.c_int32),
        ("k_scale", ctypes.c_void_p),
        ("cache", ctypes.c_void_p),
        ("page_stride", ctypes.c_int64),
        ("token_stride", ctypes.c_int64),
        ("page_size", ctypes.c_int32),
        ("num_slots", ctypes.c_int64),
    ]


class GatherParams(ctypes.Structure):
    """Mirror of `qmla_gather_params` (include/qmla.h); field order and types must match."""

    _fields_ = [
        ("cache", ctypes.c_void_p),
        ("page_stride", ctypes.c_int64),
        ("token_stride", ctypes.c_int64),
        ("page_size", ctypes.c_int32),
        ("num_pages", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32),
        ("rms_mode", ctypes.c_int32),
        ("rms_offset", ctypes.c_int32),
        ("rms_heads", ctypes.c_int32),
        ("row_elems", ctypes.c_int32),
        ("scale", ctypes.c_void_p),
        ("block_table", ctypes.c_void_p),
        ("bt_stride", ctypes.c_int64),
        ("num_seqs", ctypes.c_int32),
        ("bt_cols", ctypes.c_int32),
        ("cu_seq_lens", ctypes.c_void_p),
        ("token_to_seq", ctypes.c_void_p),
        ("seq_starts", ctypes.c_void_p),
        ("num_tokens", ctypes.c_int32),
        ("dst", ctypes.c_void_p),
        ("dst_stride", ctypes.c_int64),
        ("dst_dtype", ctypes.c_int32),
    ]


class PrepParams(ctypes.Structure):
    """Mirror of `qmla_prep_params` (include/qmla.h); field order and types must match."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("q_token_stride", ctypes.c_int64),
        ("q_head_stride", ctypes.c_int64),
        ("latent", ctypes.c_void_p),
        ("latent_stride", ctypes.c_int64),
        ("k_rope", ctypes.c_void_p),
        ("k_rope_stride", ctypes.c_int64),
        ("k_up", ctypes.c_void_p),
        ("k_gain", ctypes.c_void_p),
        ("cos_sin", ctypes.c_void_p),
        ("cos_sin_dtype", ctypes.c_int32),
        ("max_pos", ctypes.c_int64),
        ("positions", ctypes.c_void_p),
        ("pos_row_stride", ctypes.c_int64),
        ("pos_rows", ctypes.c_int32),
        ("rope_sec", ctypes.c_void_p),
        ("n", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("rope_dim", ctypes.c_int32),
        ("kv_heads", ctypes.c_int32),
        ("d_c", ctypes.c_int32),
        ("head_offset", ctypes.c_int32),
        ("rope_group", ctypes.c_int32),
        ("rope_first", ctypes.c_int32),
        ("rope_span", ctypes.c_int32),
        ("declared_rope", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("q_out", ctypes.c_void_p),
        ("q_out_token_stride", ctypes.c_int64),
        ("q_out_head_stride", ctypes.c_int64),
        ("k_pe", ctypes.c_void_p),
        ("k_pe_stride", ctypes.c_int64),
    ]


# every function include/qmla.h declares, with its ctypes signature
_P = ctypes.POINTER(DecodeParams)
_W = ctypes.POINTER(CacheWriteParams)
_G = ctypes.POINTER(GatherParams)
_R = ctypes.POINTER(PrepParams)
SIGNATURES = {
    "qmla_version": (ctypes.c_int, []),
    "qmla_build_info": (ctypes.c_char_p, []),
    "qmla_workspace_bytes": (ctypes.c_size_t, [_P]),
    "qmla_decode": (ctypes.c_int, [_P, ctypes.c_void_p]),
    "qmla_decode_static": (ctypes.c_int, [_P, ctypes.c_void_p]),
    "qmla_plan": (ctypes.c_int, [_P, ctypes.c_void_p]),
    "qmla_decode_partial": (ctypes.c_int, [_P, ctypes.c_void_p]),
    "qmla_combine": (ctypes.c_int, [_P, ctypes.c_void_p]),
    "qmla_plan_switch_tiles": (ctypes.c_int, [_P]),
    "qmla_decode_supported": (ctypes.c_int, [_P]),
    "qmla_cache_write": (ctypes.c_int, [_W, ctypes.c_void_p]),
    "qmla_gather": (ctypes.c_int, [_G, ctypes.c_void_p]),
    "qmla_prep": (ctypes.c_int, [_R, ctypes.c_void_p]),
}

_lib = None


class QmlaError(RuntimeError):
    def __init__(self, fn: str, code: int):
        super().__init__(f"{fn} failed: {ERR_NAMES.get(code, code)}")
        self.code = code


def lib() -> ctypes.CDLL:
    """Load libqmla.so once. Raises if it has not been built: there is no fallback path."""
    global _lib
    if _lib is not None:
        return _lib
    path = os.environ.get("QMLA_LIB", str(LIB_PATH))
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build the HIP library first "
                          f"(python -c 'import __graft_entry__ as g; g.build()')")
    handle = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    ver = handle.qmla_version()
    if ver != ABI_VERSION:
        raise ImportError(f"{path}: ABI version {ver}, expected {ABI_VERSION}")
    _lib = handle
    return _lib


def check(fn: str, code: int) -> None:
    if code != OK:
        if code == ERR_NOKERNEL:
            raise NotImplementedError(f"{fn}: {ERR_NAMES[code]}")
        raise QmlaError(fn, code)
