"""ctypes binding of ``libslipstream_hip.so`` (declared in ``include/slipstream_hip.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime torch
already loaded (same soname), i.e. one runtime, one set of device pointers and
streams. A missing library is an error, never a silent fallback.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (must be imported before the HIP library, see above)

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libslipstream_hip.so"

SS_OK = 0
SS_ERR_INVALID = 1
SS_ERR_UNSUPPORTED = 2
SS_ERR_LAUNCH = 3
SS_ERR_WORKSPACE = 4

SS_STATUS_QUERY_TOO_LONG = 1
SS_STATUS_STREAM_OVERRUN = 2
SS_STATUS_PREFIX_SHORT = 4

SS_DTYPE_F16 = 0
SS_DTYPE_BF16 = 1
SS_DTYPE_F32 = 2

# Every exported function: name -> (restype, argtypes). Kept in the order of the header.
_c_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "ss_status_string": (ctypes.c_char_p, [_i32]),
    "ss_last_error": (ctypes.c_char_p, []),
    "ss_version": (_i32, []),
    "ss_reshape_and_cache": (
        _i32,
        [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i64, _c_i64p, _c_i64p, _c_i64p, _i32, _vp],
    ),
    "ss_paged_attention_workspace_size": (_i32, [_i64, _i32, _i32, _i32, _i32, _i32, _c_i64p]),
    "ss_paged_attention": (
        _i32,
        [
            _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i64,
            _c_i64p, _c_i64p, _c_i64p, _i64, ctypes.c_float, _i32, _vp, _i64, _vp,
        ],
    ),
    "ss_attention_status": (_i32, [ctypes.POINTER(ctypes.c_int), _i32, _vp]),
    "ss_paged_attention_shared_prefix_workspace_size": (_i32, [_i64, _i32, _i32, _i32, _i32, _i32, _i32, _c_i64p]),
    "ss_paged_attention_shared_prefix": (
        _i32,
        [
            _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _i64, _i32,
            _c_i64p, _c_i64p, _c_i64p, _i64, ctypes.c_float, _i32, _vp, _i64, _vp,
        ],
    ),
    "ss_paged_attention_varlen": (
        _i32,
        [
            _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i64,
            _c_i64p, _c_i64p, _c_i64p, _i64, ctypes.c_float, _i32, _vp, _i64, _vp,
        ],
    ),
    "ss_paged_attention_varlen_noalloc": (
        _i32,
        [
            _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i64,
            _c_i64p, _c_i64p, _c_i64p, _i64, ctypes.c_float, _i32, _vp,
        ],
    ),
    "ss_w4a16_workspace_size": (_i32, [_i64, _i64, _i64, _i32, _i32, _c_i64p]),
    "ss_w4a16_gemm": (
        _i32,
        [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i64, _i64, _i32, _i32, _vp, _i64, _vp],
    ),
    "ss_copy_blocks": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp]),
    "ss_build_step_metadata": (_i32, [_vp, _i64, _i32, _vp, _vp, _i32, _i32, _vp, _vp, _vp, _i64, _vp]),
    "ss_rmsnorm": (_i32, [_vp, _vp, _vp, _vp, _i64, _i32, _i64, _i64, _i64, ctypes.c_float, _i32, _vp]),
    "ss_swiglu": (_i32, [_vp, _vp, _vp, _i64, _i32, _i64, _i64, _i64, _i32, _vp]),
    "ss_rope_and_cache": (
        _i32,
        [
            _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i32, _i64,
            _c_i64p, _c_i64p, _c_i64p, _c_i64p, _c_i64p, _c_i64p, _c_i64p, _i32, _vp,
        ],
    ),
}

_lib: ctypes.CDLL | None = None
_lock = threading.Lock()


class KernelError(RuntimeError):
    """A HIP entry point returned an error status (unsupported tile, launch failure)."""


def lib() -> ctypes.CDLL:
    """Load the library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"slipstream_amd HIP library missing at {LIB_PATH}; build it with "
                    "`python -m slipstream_amd.build` (hipcc, gfx950)"
                )
            handle = ctypes.CDLL(os.fspath(LIB_PATH), mode=ctypes.RTLD_LOCAL)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def i64_array(values) -> ctypes.Array:
    vals = [int(v) for v in values]
    return (ctypes.c_int64 * len(vals))(*vals)


_I64x2 = ctypes.c_int64 * 2
_I64x3 = ctypes.c_int64 * 3


def i64x2(a: int, b: int) -> ctypes.Array:
    return _I64x2(a, b)


def i64x3(a: int, b: int, c: int) -> ctypes.Array:
    return _I64x3(a, b, c)


def check(status: int, what: str) -> None:
    """Map a C status to the reference's exception classes."""
    if status == SS_OK:
        return
    l = lib()
    detail = (l.ss_last_error() or b"").decode(errors="replace")
    name = (l.ss_status_string(status) or b"").decode(errors="replace")
    msg = f"{what}: {name}: {detail}"
    if status == SS_ERR_INVALID:
        raise ValueError(msg)
    raise KernelError(msg)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device) -> int:
    """Raw ``hipStream_t`` of torch's current stream on ``device`` (torch's own raw
    accessor when it has one: a tenth of the cost of building the stream object, which
    matters for the microsecond-scale launches of a decode step)."""
    if _raw_stream is not None:
        idx = device.index
        return _raw_stream(torch.cuda.current_device() if idx is None else idx)
    return int(torch.cuda.current_stream(device).cuda_stream)


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return SS_DTYPE_BF16
    if dtype == torch.float16:
        return SS_DTYPE_F16
    if dtype == torch.float32:
        return SS_DTYPE_F32
    raise KernelError(f"dtype {dtype} not supported by the HIP kernels")
