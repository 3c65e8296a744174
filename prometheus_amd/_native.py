"""ctypes binding of ``libpmdelta.so`` (the C ABI in ``include/pm_delta.h``).

The library is built in-tree by ``prometheus_amd.build``. Loading fails
loudly when it is missing: there is no CPU or PyTorch fallback.

``torch`` is imported first on purpose: the HIP runtime torch ships carries
the same SONAME as ``/opt/rocm``'s, so loading it first makes this library
bind to the very runtime that owns torch's device memory and streams.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (see module docstring: must precede CDLL)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpmdelta.so")

ABI_VERSION = 13
DTYPE_F32 = 0
DTYPE_BF16 = 1
MAX_D = 256
MAX_D_BWD = 256
NOALLOC_SCRATCH_BYTES = 64 << 20

E_NULL, E_SHAPE, E_DTYPE, E_ALIGN, E_WORKSPACE, E_UNSUPPORTED = -1, -2, -3, -4, -5, -6

# every symbol include/pm_delta.h declares
EXPORTS = (
    "pm_delta_fwd",
    "pm_delta_fwd_varlen",
    "pm_delta_step",
    "pm_delta_step_slots",
    "pm_gated_delta_fwd",
    "pm_gated_delta_step",
    "pm_linear_attention",
    "pm_linear_attention_ws",
    "pm_linear_attention_workspace_bytes",
    "pm_delta_workspace_bytes",
    "pm_delta_varlen_workspace_bytes",
    "pm_delta_bwd",
    "pm_delta_bwd_workspace_bytes",
    "pm_delta_bwd_noalloc",
    "pm_last_error",
    "pm_abi_version",
    "pm_delta_set_path",
    "pm_delta_set_tile",
    "pm_varlen_check",
    "pm_gated_delta_bwd",
    "pm_gated_delta_bwd_workspace_bytes",
    "pm_kda_delta_fwd",
    "pm_kda_delta_workspace_bytes",
    "pm_kda_delta_step",
    "pm_kda_delta_bwd",
    "pm_kda_delta_bwd_workspace_bytes",
)

_lib = None
_lock = threading.Lock()


class NativeError(RuntimeError):
    """A nonzero return from libpmdelta.so; ``code`` is the return value."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"libpmdelta error {code}: {msg}")
        self.code = code


def lib() -> ctypes.CDLL:
    """The loaded library (loaded once); raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m prometheus_amd.build` "
                "(the delta-rule path has no fallback)"
            )
        L = ctypes.CDLL(LIB_PATH)
        vp, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        L.pm_delta_fwd.argtypes = [vp, vp, vp, vp, vp, vp, vp, i, i, i, i, i, i, i, vp, sz, vp]
        L.pm_delta_fwd.restype = i
        L.pm_delta_fwd_varlen.argtypes = [vp, vp, vp, vp, vp, i, i, vp, vp, vp, i, i, i, i, i,
                                          vp, sz, vp]
        L.pm_delta_fwd_varlen.restype = i
        L.pm_delta_step.argtypes = [vp, vp, vp, vp, vp, vp, i, i, i, i, vp]
        L.pm_delta_step.restype = i
        L.pm_gated_delta_fwd.argtypes = [vp] * 8 + [i] * 6 + [vp]
        L.pm_gated_delta_fwd.restype = i
        L.pm_gated_delta_step.argtypes = [vp] * 7 + [i] * 4 + [vp]
        L.pm_gated_delta_step.restype = i
        L.pm_kda_delta_fwd.argtypes = [vp] * 8 + [i] * 6 + [vp, sz, vp]
        L.pm_kda_delta_workspace_bytes.argtypes = [i] * 5
        L.pm_kda_delta_workspace_bytes.restype = sz
        L.pm_kda_delta_fwd.restype = i
        L.pm_kda_delta_step.argtypes = [vp] * 7 + [i] * 4 + [vp]
        L.pm_kda_delta_step.restype = i
        L.pm_delta_step_slots.argtypes = [vp, vp, i, vp, vp, vp, vp, vp, i, i, i, i, vp]
        L.pm_delta_step_slots.restype = i
        L.pm_linear_attention.argtypes = [vp, vp, vp, vp, vp, vp, i, i, i, i, i, i, vp]
        L.pm_linear_attention.restype = i
        L.pm_linear_attention_ws.argtypes = [vp, vp, vp, vp, vp, vp, i, i, i, i, i, i, vp, sz, vp]
        L.pm_linear_attention_ws.restype = i
        L.pm_linear_attention_workspace_bytes.argtypes = [i] * 5
        L.pm_linear_attention_workspace_bytes.restype = sz
        L.pm_delta_workspace_bytes.argtypes = [i, i, i, i, i]
        L.pm_delta_workspace_bytes.restype = sz
        L.pm_delta_varlen_workspace_bytes.argtypes = [i, i, i, i, i]
        L.pm_delta_varlen_workspace_bytes.restype = sz
        L.pm_delta_bwd.argtypes = [vp] * 12 + [i] * 5 + [vp, sz, vp]
        L.pm_delta_bwd.restype = i
        L.pm_delta_bwd_workspace_bytes.argtypes = [i, i, i, i, i]
        L.pm_delta_bwd_workspace_bytes.restype = sz
        L.pm_delta_bwd_noalloc.argtypes = [vp] * 12 + [i] * 5 + [vp]
        L.pm_delta_bwd_noalloc.restype = i
        L.pm_last_error.argtypes = []
        L.pm_last_error.restype = ctypes.c_char_p
        L.pm_abi_version.argtypes = []
        L.pm_abi_version.restype = i
        L.pm_delta_set_path.argtypes = [i]
        L.pm_delta_set_path.restype = i
        L.pm_delta_set_tile.argtypes = [i]
        L.pm_delta_set_tile.restype = i
        L.pm_varlen_check.argtypes = [vp, i, i, vp, vp]
        L.pm_varlen_check.restype = i
        L.pm_gated_delta_bwd.argtypes = [vp] * 14 + [i] * 5 + [vp, sz, vp]
        L.pm_gated_delta_bwd.restype = i
        L.pm_gated_delta_bwd_workspace_bytes.argtypes = [i] * 5
        L.pm_gated_delta_bwd_workspace_bytes.restype = sz
        L.pm_kda_delta_bwd.argtypes = [vp] * 14 + [i] * 5 + [vp, sz, vp]
        L.pm_kda_delta_bwd.restype = i
        L.pm_kda_delta_bwd_workspace_bytes.argtypes = [i] * 5
        L.pm_kda_delta_bwd_workspace_bytes.restype = sz
        got = L.pm_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI version {got}, expected {ABI_VERSION}")
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        msg = lib().pm_last_error()
        raise NativeError(rc, msg.decode(errors="replace") if msg else "")


def set_path(path: int) -> int:
    """0 automatic, 1 per-token kernel, 2 chunked kernel required; returns old value."""
    old = lib().pm_delta_set_path(int(path))
    if old < 0:
        check(old)
    return old


def set_tile(dv_tile: int) -> int:
    """Chunked kernel d_v tile width (0 auto, 16, 32; 64 runs as 32); returns old value."""
    old = lib().pm_delta_set_tile(int(dv_tile))
    if old < 0:
        check(old)
    return old


def knobs() -> tuple[int, int]:
    """The calling thread's (path, tile) selection.  Both knobs are per thread in the
    library, so code that launches on another thread (torch autograd runs a CUDA
    backward on its device thread) carries them over with ``use_knobs``."""
    path = set_path(0)
    set_path(path)
    tile = set_tile(0)
    set_tile(tile)
    return path, tile


class use_knobs:
    """Context manager: this thread's path and tile set to ``(path, tile)`` inside the
    block, restored after it."""

    def __init__(self, path: int, tile: int):
        self.path, self.tile = int(path), int(tile)

    def __enter__(self):
        self.old = (set_path(self.path), set_tile(self.tile))
        return self

    def __exit__(self, *exc):
        set_path(self.old[0])
        set_tile(self.old[1])
        return False
