"""ctypes binding of libcame8.so, the HIP library behind the C ABI in ``include/came8.h``.

The library is built in-tree (``came_amd/lib/libcame8.so``, see
``came_amd/build.py``).  There is no fallback: if the library is missing or
fails to load, every entry point that needs it raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libcame8.so")

CAME8_F32, CAME8_BF16, CAME8_F16 = 0, 1, 2
CAME8_OK, CAME8_EINVAL, CAME8_ESPACE, CAME8_EHIP = 0, -1, -2, -3
ABI_VERSION = 5  # include/came8.h: CAME8_ABI_VERSION
CAME8_FLAG_REFERENCE_NORM = 1  # the default (accepted for callers of ABI 3)
CAME8_FLAG_EXACT_NORM = 2
CAME8_FLAG_PLAN_ONLY = 4
CAME8_FLAG_FP16_UPDATE = 8
CAME8_TENSOR_FP16_UPDATE = 1  # came8_tensor.tensor_flags
CAME8_STATE_Q8 = 0
CAME8_STATE_FP32 = 1
CAME8_STATE_8BIT2D = 2
CAME8_STATE_Q8_MATRIX = 3  # the reference CUDA N-D path's per-matrix blocks

# every symbol include/came8.h declares
EXPORTED_SYMBOLS = (
    "came8_version",
    "came8_abi_version",
    "came8_last_error",
    "came8_workspace_size",
    "came8_release_workspace",
    "came8_step",
    "came8_step_static",
    "came8_profile_enable",
    "came8_profile_read",
    "came8_read_clip",
    "came8_side_stream_count",
    "came8_quantize_blockwise",
    "came8_dequantize_blockwise",
)


class Came8Tensor(ctypes.Structure):
    """Mirror of ``came8_tensor`` (include/came8.h)."""

    _fields_ = [
        ("param", ctypes.c_void_p),
        ("grad", ctypes.c_void_p),
        ("exp_avg_q", ctypes.c_void_p),
        ("exp_avg_absmax", ctypes.c_void_p),
        ("row_q", ctypes.c_void_p),
        ("row_absmax", ctypes.c_void_p),
        ("col_q", ctypes.c_void_p),
        ("col_absmax", ctypes.c_void_p),
        ("prefix", ctypes.c_int64),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("param_dtype", ctypes.c_int32),
        ("grad_dtype", ctypes.c_int32),
        ("factored", ctypes.c_int32),
        ("state_kind", ctypes.c_int32),
        ("res_row_q", ctypes.c_void_p),
        ("res_row_absmax", ctypes.c_void_p),
        ("res_col_q", ctypes.c_void_p),
        ("res_col_absmax", ctypes.c_void_p),
        ("res_row_partial", ctypes.c_void_p),
        ("res_col_partial", ctypes.c_void_p),
        ("tensor_flags", ctypes.c_uint32),
        ("reserved", ctypes.c_int32),
    ]


class Came8HParams(ctypes.Structure):
    """Mirror of ``came8_hparams`` (include/came8.h)."""

    _fields_ = [
        ("lr", ctypes.c_double),
        ("beta1", ctypes.c_double),
        ("beta2", ctypes.c_double),
        ("beta3", ctypes.c_double),
        ("eps0", ctypes.c_double),
        ("eps1", ctypes.c_double),
        ("clip_threshold", ctypes.c_double),
        ("weight_decay", ctypes.c_double),
        ("block_size", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
    ]


class Came8PhaseStat(ctypes.Structure):
    """Mirror of ``came8_phase_stat`` (include/came8.h)."""

    _fields_ = [
        ("name", ctypes.c_char * 32),
        ("launches", ctypes.c_int64),
        ("total_ms", ctypes.c_double),
        ("alg_bytes", ctypes.c_double),
    ]


_lib = None
_lock = threading.Lock()
_tag_lock = threading.Lock()
_next_tag = [0]


def new_workspace_tag() -> int:
    """A process-unique nonzero tag for one workspace allocation (came8_step's workspace_tag)."""
    with _tag_lock:
        _next_tag[0] += 1
        return _next_tag[0]


def lib_path() -> str:
    return LIB_PATH


def load(path: str | None = None) -> ctypes.CDLL:
    """Load libcame8.so once; raise RuntimeError if it is missing (no fallback path exists)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise RuntimeError(
                f"came_amd: HIP library not found at {p}; build it with `python -c \"import came_amd.build as b; b.build()\"`"
            )
        lib = ctypes.CDLL(p)
        vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t
        lib.came8_version.restype = ctypes.c_char_p
        lib.came8_version.argtypes = []
        lib.came8_abi_version.restype = ctypes.c_int
        lib.came8_abi_version.argtypes = []
        lib.came8_last_error.restype = ctypes.c_char_p
        lib.came8_last_error.argtypes = []
        lib.came8_workspace_size.restype = ctypes.c_int
        lib.came8_workspace_size.argtypes = [ctypes.POINTER(Came8Tensor), i32, i32, ctypes.POINTER(sz)]
        lib.came8_release_workspace.restype = ctypes.c_int
        lib.came8_release_workspace.argtypes = [vp]
        lib.came8_step.restype = ctypes.c_int
        lib.came8_step.argtypes = [ctypes.POINTER(Came8Tensor), i32, ctypes.POINTER(Came8HParams), vp, sz,
                                   ctypes.c_uint64, vp]
        lib.came8_step_static.restype = ctypes.c_int
        lib.came8_step_static.argtypes = [ctypes.POINTER(Came8Tensor), i32, ctypes.POINTER(Came8HParams), vp]
        lib.came8_profile_enable.restype = ctypes.c_int
        lib.came8_side_stream_count.restype = ctypes.c_int
        lib.came8_side_stream_count.argtypes = []
        lib.came8_profile_enable.argtypes = [i32]
        lib.came8_profile_read.restype = ctypes.c_int
        lib.came8_profile_read.argtypes = [ctypes.POINTER(Came8PhaseStat), i32, ctypes.POINTER(i32), i32]
        lib.came8_read_clip.restype = ctypes.c_int
        lib.came8_read_clip.argtypes = [vp, ctypes.c_uint64, i32, ctypes.POINTER(ctypes.c_float), vp]
        lib.came8_quantize_blockwise.restype = ctypes.c_int
        lib.came8_quantize_blockwise.argtypes = [vp, i64, i32, i32, vp, vp, vp]
        lib.came8_dequantize_blockwise.restype = ctypes.c_int
        lib.came8_dequantize_blockwise.argtypes = [vp, vp, i64, i32, i32, vp, vp]
        if lib.came8_abi_version() != ABI_VERSION:
            raise RuntimeError(f"came_amd: {p} has ABI {lib.came8_abi_version()}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != CAME8_OK:
        msg = load().came8_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def profile_enable(on: bool = True) -> None:
    """Start/stop per-kernel device timing of came8_step (HIP events on the launch stream)."""
    check(load().came8_profile_enable(1 if on else 0), "came8_profile_enable")


def profile_read(reset: bool = True) -> dict:
    """{phase: (launches, total_ms, alg_bytes)} for the launches recorded since the last reset."""
    lib = load()
    arr = (Came8PhaseStat * 32)()
    n = ctypes.c_int32(0)
    check(lib.came8_profile_read(arr, 32, ctypes.byref(n), 1 if reset else 0), "came8_profile_read")
    return {arr[i].name.decode(): (arr[i].launches, arr[i].total_ms, arr[i].alg_bytes) for i in range(n.value)}
