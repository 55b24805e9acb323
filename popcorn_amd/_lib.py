"""ctypes binding of `libpopcorn_amd.so` (declared in include/popcorn_amd.h).

The library is loaded on first use and never replaced by anything else: a
missing or stale library raises, there is no fallback path.
"""

from __future__ import annotations

import contextlib
import ctypes
import threading
from pathlib import Path

import torch

LIBRARY = Path(__file__).resolve().parent / "libpopcorn_amd.so"
ABI_VERSION = 5

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP = 0, 1, 2, 3
F32, BF16, F16 = 0, 1, 2

DTYPE_CODES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/popcorn_amd.h
SIGNATURES = {
    "pk_version": (_int, []),
    "pk_last_error": (ctypes.c_char_p, []),
    "pk_swiglu_fwd": (_int, [_p, _p, _p, _i64, _int, _p]),
    "pk_swiglu_bwd": (_int, [_p, _p, _p, _p, _p, _i64, _int, _p]),
    "pk_rmsnorm_fwd": (_int, [_p, _p, _p, _p, _p, _i64, _i64, _f32, _int, _int, _p]),
    "pk_rmsnorm_bwd_workspace": (_i64, [_i64, _i64, _int]),
    "pk_rmsnorm_bwd": (_int, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _int, _int, _p]),
    "pk_rmsnorm_bwd_noalloc": (_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _int, _int, _p]),
    "pk_add_rmsnorm_fwd": (_int, [_p, _p, _p, _p, _p, _p, _i64, _i64, _f32, _f32, _int, _int, _p]),
    "pk_add_rmsnorm_bwd": (_int, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _f32, _int, _int, _p]),
    "pk_rotary": (_int, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _int, _int, _int, _int, _p]),
    "pk_rope": (_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _int, _int, _int, _int, _p]),
    "pk_qk_norm_rope_fwd": (_int, [_p] * 10 + [_p, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _int, _int, _int, _int, _p]),
    "pk_qk_norm_rope_bwd_workspace": (_i64, [_i64, _i64, _i64, _i64, _i64, _int]),
    "pk_qk_norm_rope_bwd": (_int, [_p] * 14 + [_i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _int, _int, _int, _int, _p]),
    "pk_attn_fwd": (_int, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _int, _int, _p]),
    "pk_attn_bwd_workspace": (_i64, [_i64] * 5),
    "pk_attn_bwd": (_int, [_p] * 7 + [_i64] + [_p] * 4 + [_i64] * 5 + [_f32, _int, _int, _p]),
    "pk_attn_varlen_bwd_workspace": (_i64, [_i64] * 6),
    "pk_attn_varlen_bwd": (_int, [_p] * 7 + [_i64] + [_p] * 5 + [_i64] * 6 + [_f32, _int, _int, _p]),
    "pk_attn_varlen_fwd": (_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _int, _int, _p]),
    "pk_probe_mfma": (_int, [_int, _int, _int, _p, _p]),
    "pk_probe_stream": (_int, [_p, _p, _p, _i64, _int, _p]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class KernelError(RuntimeError):
    """A popcorn_amd entry point returned a non-zero status."""


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load (once) and type the library; raises if it is missing or mismatched."""
    global _lib
    if _lib is not None and path is None:  # the per-call path: no lock once loaded
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        target = Path(path) if path is not None else LIBRARY
        if not target.exists():
            raise RuntimeError(
                f"popcorn_amd: HIP kernel library {target} is not built; run `python -m popcorn_amd.build` "
                "(or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(str(target))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.pk_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"popcorn_amd: library ABI {version}, bindings expect {ABI_VERSION}; rebuild")
        if path is None:
            _lib = lib
        return lib


def check(status: int, lib: ctypes.CDLL | None = None) -> None:
    if status != OK:
        lib = lib or load()
        message = lib.pk_last_error().decode(errors="replace")
        raise KernelError(f"popcorn_amd: {message or f'status {status}'}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device`.

    torch's raw-stream query skips building a Stream object (about 2 us per
    call); the public `current_stream` is the path where it is absent.
    """
    if _raw_stream is not None and device.index is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


_get_device = getattr(torch._C, "_cuda_getDevice", None)
_NO_SWITCH = contextlib.nullcontext()


def on_device(device: torch.device):
    """A context in which `device` is the current HIP device: a no-op when it already is.

    Kernels launch on the current device, and stream handle 0 (torch's default
    stream) names that device's null stream, so a call whose tensors live on
    another device makes theirs current around the launch and restores the
    caller's afterwards, as torch's own operators do.
    """
    index = device.index
    if index is None or index == (_get_device() if _get_device is not None else torch.cuda.current_device()):
        return _NO_SWITCH
    return torch.cuda.device(index)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"popcorn_amd: unsupported dtype {dtype}") from None
