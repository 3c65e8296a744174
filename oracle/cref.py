"""ctypes binding of ``libdelta_oracle.so`` (the C restatement).

Test infrastructure / CPU baseline only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

from oracle.build import LIB, build

_lib = None


def load(rebuild_if_missing: bool = True):
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB):
        if not rebuild_if_missing:
            raise FileNotFoundError(LIB)
        build()
    lib = ctypes.CDLL(LIB)
    vp, fp, i = ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int
    lib.oracle_delta_fwd.argtypes = [vp, vp, vp, fp, fp, fp, fp, i, i, i, i, i, i]
    lib.oracle_delta_fwd.restype = i
    lib.oracle_delta_step.argtypes = [fp, vp, vp, vp, fp, fp, i, i, i, i, i]
    lib.oracle_delta_step.restype = i
    lib.oracle_max_threads.restype = i
    _lib = lib
    return lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _in(x):
    """fp32 array, or a bf16 bit-pattern array given as uint16."""
    x = np.ascontiguousarray(x)
    if x.dtype == np.uint16:
        return x, 1
    return np.ascontiguousarray(x, dtype=np.float32), 0


def delta_fwd(q, k, v, beta, state=None, threads: int = 0):
    """(O fp32, S fp32) for (B, T, H, D) inputs; uint16 inputs are bf16 bits."""
    lib = load()
    q, bf = _in(q)
    k, _ = _in(k)
    v, _ = _in(v)
    beta = np.ascontiguousarray(beta, dtype=np.float32)
    b, t, h, d = q.shape
    o = np.empty((b, t, h, d), dtype=np.float32)
    s = np.empty((b, h, d, d), dtype=np.float32)
    s0 = None if state is None else np.ascontiguousarray(state, dtype=np.float32)
    rc = lib.oracle_delta_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(beta), _ptr(s0), _ptr(o), _ptr(s),
                              b, t, h, d, bf, int(threads))
    if rc != 0:
        raise ValueError(f"oracle_delta_fwd rc={rc}")
    return o, s


def delta_step(state, q, k, v, beta, threads: int = 0):
    """In-place step on ``state`` (B, H, D, D) fp32; returns o (B, H, D)."""
    lib = load()
    assert state.dtype == np.float32 and state.flags.c_contiguous
    q, bf = _in(q)
    k, _ = _in(k)
    v, _ = _in(v)
    beta = np.ascontiguousarray(beta, dtype=np.float32)
    b, h, d = q.shape
    o = np.empty((b, h, d), dtype=np.float32)
    rc = lib.oracle_delta_step(_ptr(state), _ptr(q), _ptr(k), _ptr(v), _ptr(beta), _ptr(o),
                               b, h, d, bf, int(threads))
    if rc != 0:
        raise ValueError(f"oracle_delta_step rc={rc}")
    return o


def max_threads() -> int:
    return int(load().oracle_max_threads())
