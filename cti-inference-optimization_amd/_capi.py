"""ctypes binding of libcti_ebag.so (the C ABI declared in include/cti_ebag.h).

The library is loaded after ``import torch`` so that it binds to the HIP runtime torch already
loaded (both carry the soname ``libamdhip64.so.7``); one process then has one HIP runtime, and
torch's device pointers and streams are valid handles for the library.

There is no fallback: if the library is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the dlopen below, see module docstring)

LIB_NAME = "libcti_ebag.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

ABI_VERSION = 5

F32, BF16, F16, I8 = 0, 1, 2, 3
I64, I32 = 0, 1
SUM, MEAN = 0, 1

OK = 0
EINVAL = -1
EUNSUPPORTED = -2
EHIP = -3
EWORKSPACE = -4

_STATUS_NAMES = {EINVAL: "EINVAL", EUNSUPPORTED: "EUNSUPPORTED", EHIP: "EHIP", EWORKSPACE: "EWORKSPACE"}

_DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}
_INDEX_CODE = {torch.int64: I64, torch.int32: I32}
_POOL_CODE = {"sum": SUM, "mean": MEAN}


class EbagError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[{_STATUS_NAMES.get(status, status)}] {message}")
        self.status = status


class Table(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("rows", ctypes.c_int64),
        ("row_stride", ctypes.c_int64),
        ("dim", ctypes.c_int32),
        ("out_col", ctypes.c_int32),
        ("row_scale", ctypes.c_void_p),
    ]


class Options(ctypes.Structure):
    _fields_ = [
        ("long_threshold", ctypes.c_int32),
        ("use_bins", ctypes.c_int32),
        ("block_threshold", ctypes.c_int32),
        ("split_threshold", ctypes.c_int32),
        ("tile_order", ctypes.c_void_p),
        ("next_order", ctypes.c_void_p),
        ("next_offsets", ctypes.c_void_p),
        ("order_bytes", ctypes.c_int64),
    ]


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_PP = ctypes.POINTER(ctypes.c_void_p)
_PI64 = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); the exported surface of include/cti_ebag.h
SIGNATURES = {
    "cti_ebag_abi_version": (ctypes.c_int, []),
    "cti_ebag_last_error": (ctypes.c_char_p, []),
    "cti_ebag_fused_all_slots": (
        ctypes.c_int,
        [_P, _P, _P, _P, _I32, _P, _I64, _I32, _I32, _I64, _I64, _P],
    ),
    "cti_ebag_forward": (
        ctypes.c_int,
        [_P, _I32, _I64, _P, _I64, _I32, ctypes.POINTER(Table), _I32, _I32, _P, _I32, _I64, _P, _I64,
         ctypes.POINTER(Options), _P],
    ),
    "cti_ebag_forward_static": (
        ctypes.c_int,
        [_P, _I32, _I64, _P, _I64, _I32, ctypes.POINTER(Table), _I32, _I32, _P, _I32, _I64,
         ctypes.POINTER(Options), _P],
    ),
    "cti_ebag_workspace_bytes": (ctypes.c_int64, [_I64, _I32]),
    "cti_ebag_order_bytes": (ctypes.c_int64, [_I64, _I32]),
    "cti_ebag_pack_slots": (ctypes.c_int, [_PP, _PP, _PI64, _I32, _I64, _P, _P, _P, _P, _P]),
    "cti_ebag_merge_batches": (
        ctypes.c_int,
        [_PP, _PP, _PP, _PI64, _PI64, _I32, _I32, _P, _P, _P, _P, _P],
    ),
    "cti_ebag_merge_batches_int32": (
        ctypes.c_int,
        [_PP, _PP, _PP, _PI64, _PI64, _I32, _I32, _P, _P, _P, _P, _P],
    ),
    "cti_ebag_layernorm": (
        ctypes.c_int,
        [_P, _P, _I64, _I64, _I32, _P, _P, _I32, ctypes.c_float, _P, _P, _P],
    ),
    "cti_ebag_layernorm_linear": (
        ctypes.c_int,
        [_P, _I64, _I32, _P, _P, _P, _P, _I32, _P, _I32, _P, _I32, _P, _I32, _P, _I64, _P],
    ),
    "cti_ebag_layernorm_linear_workspace_bytes": (ctypes.c_int64, [_I64, _I32, _I32]),
    "cti_ebag_fused_all_slots_int8": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, _I32, _I64, _I32, _I32, _I64, _I64, _P],
    ),
    "cti_ebag_quantize_int8": (ctypes.c_int, [_P, _I32, _I64, _I64, _I64, _P, _P, _P]),
    "cti_ebag_narrow_ids": (ctypes.c_int, [_P, _I64, _P, _I32]),
    "cti_ebag_fused_all_slots_layernorm": (
        ctypes.c_int,
        [_P, _I32, _P, _P, _I32, _P, _I32, _P, _I64, _I32, _I32, _I64, _I64, _I32, _P, _P, _I32, ctypes.c_float, _P],
    ),
    "cti_ebag_stage_copy": (
        ctypes.c_int,
        [_PP, ctypes.POINTER(ctypes.c_int32), _PI64, _I32, _I32, _P, _I64, _P, _I32, _P],
    ),
    "cti_ebag_stage_offset": (ctypes.c_int64, [_PI64, _I32, _I32, _I32]),
    "cti_ebag_order_host": (ctypes.c_int, [_P, _I32, _I64, _I64, _I32, _I32, _I32, _P, _I64, _I32]),
    "cti_ebag_fused_all_slots_ordered": (
        ctypes.c_int,
        [_P, _I32, _P, _P, _I32, _P, _I32, _P, _P, _I32, _I64, _I32, _I32, _I64, _I64, _P, _I64, _P],
    ),
    "cti_ebag_fused_all_slots_typed": (
        ctypes.c_int,
        [_P, _I32, _P, _P, _I32, _P, _I32, _P, _P, _I32, _I64, _I32, _I32, _I64, _I64, _P],
    ),
}

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it is missing or incompatible."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; build it with `make -C <package>/csrc` "
                "(or __graft_entry__.build())"
            )
        handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        ver = handle.cti_ebag_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI version {ver}, expected {ABI_VERSION}")
        _lib = handle
        return _lib


def last_error() -> str:
    msg = lib().cti_ebag_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(status: int) -> None:
    if status != OK:
        raise EbagError(status, last_error())


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise TypeError(f"unsupported element type {dt}; expected float32, bfloat16 or float16") from None


def index_code(dt: torch.dtype) -> int:
    try:
        return _INDEX_CODE[dt]
    except KeyError:
        raise TypeError(f"unsupported index type {dt}; expected int64 or int32") from None


def pooling_code(mode: str) -> int:
    try:
        return _POOL_CODE[mode]
    except KeyError:
        raise ValueError(f"unsupported pooling {mode!r}; expected 'sum' or 'mean'") from None


def current_stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream
