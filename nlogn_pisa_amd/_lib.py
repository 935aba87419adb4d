"""ctypes binding of ``libpisa_hip.so`` (declared in ``include/pisa_hip.h``).

The library is loaded lazily on first use; a missing library is an error, never
a fallback.  Build it with ``python -m nlogn_pisa_amd.build``.
"""

from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(HERE, "libpisa_hip.so")

PISA_OK = 0
PISA_ERR_INVALID = -1
PISA_ERR_UNSUPPORTED = -2
PISA_ERR_WORKSPACE = -3
PISA_ERR_LAUNCH = -4

PISA_F32, PISA_F16, PISA_BF16 = 0, 1, 2
METHODS = {"pisa1": 0, "pisa2": 1, "pisa": 2}
SCHEDULES = {"grouped": 0, "fused": 1}
MAX_LEVELS = 32

# Every exported entry point of include/pisa_hip.h.
EXPORTS = (
    "pisa_last_error", "pisa_abi_version", "pisa_routing_geometry", "pisa_pyramid_layout",
    "pisa_mean_pool", "pisa_build_pyramid", "pisa_pyramid_append", "pisa_rotary", "pisa_select_workspace_size", "pisa_select",
    "pisa_leaf_workspace_size", "pisa_leaf_scores", "pisa_bsa_workspace_size", "pisa_bsa_select", "pisa_attention_workspace_size", "pisa_attention_block_limit", "pisa_sparse_attention_fwd",
    "pisa_sparse_attention_bwd", "pisa_noalloc_scratch_bytes", "pisa_sparse_attention_fwd_noalloc",
    "pisa_profile_begin", "pisa_profile_end",
)


class QkDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32), ("query_tokens", ctypes.c_int32),
        ("query_heads", ctypes.c_int32), ("key_tokens", ctypes.c_int32),
        ("key_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("q_stride_batch", ctypes.c_int64), ("q_stride_token", ctypes.c_int64),
        ("k_stride_batch", ctypes.c_int64), ("k_stride_token", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
    ]


class PyramidDesc(ctypes.Structure):
    _fields_ = [
        ("storage", ctypes.c_void_p), ("stride_batch", ctypes.c_int64),
        ("levels", ctypes.c_int32),
        ("offsets", ctypes.c_int32 * MAX_LEVELS), ("lengths", ctypes.c_int32 * MAX_LEVELS),
    ]


class SelectParams(ctypes.Structure):
    _fields_ = [
        ("method", ctypes.c_int32), ("block_size", ctypes.c_int32),
        ("branching", ctypes.c_int32), ("topk", ctypes.c_int32),
        ("force_first", ctypes.c_int32), ("force_recent", ctypes.c_int32),
        ("top", ctypes.c_int32), ("first_width", ctypes.c_int32),
        ("schedule", ctypes.c_int32), ("scale", ctypes.c_float),
    ]


class AttnDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32), ("query_tokens", ctypes.c_int32),
        ("query_heads", ctypes.c_int32), ("key_tokens", ctypes.c_int32),
        ("key_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("value_dim", ctypes.c_int32),
        ("q_stride_batch", ctypes.c_int64), ("q_stride_token", ctypes.c_int64),
        ("k_stride_batch", ctypes.c_int64), ("k_stride_token", ctypes.c_int64),
        ("v_stride_batch", ctypes.c_int64), ("v_stride_token", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("topk", ctypes.c_int32), ("index_bits", ctypes.c_int32),
        ("block_size", ctypes.c_int32), ("causal", ctypes.c_int32), ("scale", ctypes.c_float),
        ("block_key_start", ctypes.c_void_p), ("block_key_rows", ctypes.c_void_p),
        ("blocks", ctypes.c_int32),
    ]


class KernelTime(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 48), ("launches", ctypes.c_int32),
                ("total_ms", ctypes.c_double)]


_lock = threading.Lock()
_lib = None

P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64
SZ = ctypes.c_size_t


def _declare(lib):
    sig = {
        "pisa_last_error": (ctypes.c_char_p, []),
        "pisa_abi_version": (I32, []),
        "pisa_routing_geometry": (I32, [I32, I32, I32, ctypes.POINTER(I32), ctypes.POINTER(I32)]),
        "pisa_pyramid_layout": (I32, [I32, I32, I32, I32, ctypes.POINTER(I32),
                                      ctypes.POINTER(I32), ctypes.POINTER(I32)]),
        "pisa_mean_pool": (I32, [P, I64, I64, I32, I32, I32, I32, I32, P, I64, I64, I32, P]),
        "pisa_build_pyramid": (I32, [P, I64, I64, I32, I32, I32, I32, I32, I32, I32, P, I64, I32, P]),
        "pisa_pyramid_append": (I32, [P, I64, I64, I32, I32, I32, I32, I32, I32, I32, I32,
                                      ctypes.POINTER(I32), P, I64, I32, P]),
        "pisa_rotary": (I32, [P, I64, I64, P, I64, I64, I32, I32, I32, I32, P, P, I64, I32, I32, P]),
        "pisa_select_workspace_size": (SZ, [ctypes.POINTER(QkDesc), ctypes.POINTER(SelectParams)]),
        "pisa_select": (I32, [ctypes.POINTER(QkDesc), ctypes.POINTER(SelectParams), P, P,
                              ctypes.POINTER(PyramidDesc), P, I64, P, P, P, SZ, P]),
        "pisa_leaf_workspace_size": (SZ, [ctypes.POINTER(QkDesc), I32, I32]),
        "pisa_bsa_workspace_size": (SZ, [ctypes.POINTER(QkDesc), I32]),
        "pisa_bsa_select": (I32, [ctypes.POINTER(QkDesc), I32, I32, I32, I32, P, P, P, I64, P, P,
                                  SZ, P]),
        "pisa_leaf_scores": (I32, [ctypes.POINTER(QkDesc), ctypes.POINTER(SelectParams), P, P, P,
                                   I64, P, I32, P, I64, P, P, SZ, P]),
        "pisa_attention_workspace_size": (SZ, [ctypes.POINTER(AttnDesc), I32]),
        "pisa_attention_block_limit": (I32, [I32, I32, I32, I32]),
        "pisa_sparse_attention_fwd": (I32, [ctypes.POINTER(AttnDesc), P, P, P, P, P, I64, P, P, P,
                                            P, SZ, P]),
        "pisa_sparse_attention_bwd": (I32, [ctypes.POINTER(AttnDesc), P, P, P, P, P, I64, P, P, P,
                                            P, P, P, P, P, SZ, P]),
        "pisa_noalloc_scratch_bytes": (SZ, []),
        "pisa_sparse_attention_fwd_noalloc": (I32, [ctypes.POINTER(AttnDesc), P, P, P, P, P, I64, P,
                                                    P, P, P]),
        "pisa_profile_begin": (I32, []),
        "pisa_profile_end": (I32, [ctypes.POINTER(KernelTime), I32, ctypes.POINTER(I32)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def library():
    """Load (once) and return the ctypes handle of libpisa_hip.so.

    ``PISA_HIP_LIBRARY`` names another build of the same library (e.g. one
    compiled with other hipcc options) to load instead.
    """
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = os.environ.get("PISA_HIP_LIBRARY") or LIBRARY_PATH
            if not os.path.exists(path):
                raise RuntimeError(
                    f"{path} is missing: build it with `python -m nlogn_pisa_amd.build` "
                    "(hipcc, gfx950); there is no fallback implementation")
            lib = ctypes.CDLL(path)
            _declare(lib)
            _lib = lib
    return _lib


class PisaError(RuntimeError):
    """A non-zero status from libpisa_hip.so."""


def check(status):
    if status == PISA_OK:
        return
    message = library().pisa_last_error().decode(errors="replace")
    if status == PISA_ERR_INVALID:
        raise ValueError(message)
    raise PisaError(f"libpisa_hip status {status}: {message}")


def profile_begin():
    """Start timing every kernel launch of the library (HIP events on its stream)."""
    check(library().pisa_profile_begin())


def profile_end():
    """Stop timing; {kernel name: (launches, total milliseconds)}."""
    cap = 64
    buf = (KernelTime * cap)()
    count = ctypes.c_int32()
    check(library().pisa_profile_end(buf, cap, ctypes.byref(count)))
    return {buf[i].name.decode(): (buf[i].launches, buf[i].total_ms)
            for i in range(min(cap, count.value))}
