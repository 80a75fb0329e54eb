"""Loader of the in-tree HIP library ``librq_hip.so`` (C ABI in include/rq_hip.h).

There is no CPU fallback: if the library is missing or cannot be loaded,
``lib()`` raises, and every op that needs it fails loudly.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("RQ_HIP_LIBRARY") or os.path.join(PACKAGE_DIR, "librq_hip.so")
CSRC_DIR = os.path.join(PACKAGE_DIR, "csrc")

RQ_OK, RQ_EINVAL, RQ_ENOKERNEL, RQ_ELAUNCH, RQ_ENOSPACE = 0, -1, -2, -3, -4
RQ_ATTENTION_NOALLOC_MAX_BYTES = 8 << 20

# Every symbol include/rq_hip.h declares.
EXPORTED_SYMBOLS = (
    "rq_version",
    "rq_last_error",
    "rq_page_width",
    "rq_quantize",
    "rq_attention_workspace_bytes",
    "rq_attention",
    "rq_attention_noalloc",
    "rq_packed_prefill_attention",
    "rq_dequantize",
    "rq_paged_attention_bf16",
    "rq_prefill_attention",
    "rq_prefill_workspace_bytes",
    "rq_rms_norm",
    "rq_rope_qkv",
    "rq_silu_mul",
    "rq_linear_rows",
    "rq_timing_enable",
    "rq_timing_read",
    "rq_set_split_target",
)

_lib = None


def build(jobs: int = 8, force: bool = False) -> str:
    """Compile every HIP source for gfx950 into ``librq_hip.so`` (hipcc via make).

    ``force`` recompiles every object even where make finds them up to date.
    """
    args = ["make", "-s", "-C", CSRC_DIR, f"-j{jobs}"] + (["-B"] if force else [])
    subprocess.run(args, check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"HIP library {LIB_PATH} is not built; run "
                "`python -c 'import __graft_entry__ as g; g.build()'` or `make -C residualquant_amd/csrc`")
        handle = ctypes.CDLL(LIB_PATH)
        _declare(handle)
        _lib = handle
    return _lib


def _declare(l: ctypes.CDLL) -> None:
    i32, i64, vp, sz = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t
    l.rq_version.restype = i32
    l.rq_version.argtypes = []
    l.rq_last_error.restype = ctypes.c_char_p
    l.rq_last_error.argtypes = []
    l.rq_page_width.restype = i32
    l.rq_page_width.argtypes = [i32, i32, vp, vp]
    l.rq_quantize.restype = i32
    l.rq_quantize.argtypes = [i32, vp, vp, vp, vp, i64, vp, i64, i32, i32, i32, vp, i64, i32, vp, vp,
                              vp, vp, vp, i32, i32, i32, vp]
    l.rq_attention_workspace_bytes.restype = sz
    l.rq_attention_workspace_bytes.argtypes = [i64, i32, i32, i64, i32]
    l.rq_attention.restype = i32
    l.rq_attention.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i64, i32, i32, vp, i64, i32, i32,
                               vp, vp, i64, vp, i64, i64, vp, vp, vp, i32, vp, vp, i32, i32, i32, vp,
                               sz, vp]
    l.rq_packed_prefill_attention.restype = i32
    l.rq_packed_prefill_attention.argtypes = l.rq_attention.argtypes
    l.rq_attention_noalloc.restype = i32
    l.rq_attention_noalloc.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i64, i32, i32, vp, i64, i32, i32,
                                       vp, vp, i64, vp, i64, i64, vp, vp, vp, i32, vp, vp, i32, i32, i32, vp]
    l.rq_dequantize.restype = i32
    l.rq_dequantize.argtypes = [vp, i64, i32, i32, i32, vp, i64, i32, vp, i32, vp, vp, i32, i32, i32,
                                vp, vp, vp]
    l.rq_paged_attention_bf16.restype = i32
    l.rq_paged_attention_bf16.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i64, i32, i32, vp, i64,
                                          i32, vp, vp, i64, vp, i64, i64, vp, sz, vp]
    l.rq_timing_enable.restype = None
    l.rq_prefill_attention.restype = i32
    l.rq_prefill_attention.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32, vp, vp, i64, i64,
                                       i64, ctypes.c_float, i32, vp, ctypes.c_size_t, vp]
    l.rq_prefill_workspace_bytes.restype = ctypes.c_size_t
    l.rq_prefill_workspace_bytes.argtypes = [i64, i32, i32, i64, i64, i32, i32]
    l.rq_rms_norm.restype = i32
    l.rq_rms_norm.argtypes = [vp, i64, vp, vp, i64, vp, i64, vp, vp, i64, i64, i32, ctypes.c_float, vp]
    l.rq_rope_qkv.restype = i32
    l.rq_rope_qkv.argtypes = [vp, i64, vp, vp, vp, i64, i32, i32, i64, vp, i64, vp, i64, vp, vp, i64, vp]
    l.rq_silu_mul.restype = i32
    l.rq_silu_mul.argtypes = [vp, i64, vp, i64, i64, i32, vp]
    l.rq_linear_rows.restype = i32
    l.rq_linear_rows.argtypes = [vp, i64, vp, vp, i64, i64, i64, i64, vp]
    l.rq_timing_enable.argtypes = [i32]
    l.rq_timing_read.restype = i32
    l.rq_timing_read.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64)]
    l.rq_set_split_target.restype = None
    l.rq_set_split_target.argtypes = [i32]


def check(status: int) -> None:
    """Raise RuntimeError with the library's message for a failed call."""
    if status != RQ_OK:
        message = lib().rq_last_error().decode(errors="replace")
        raise RuntimeError(message or f"librq_hip call failed with status {status}")
