"""Seeded synthetic inputs for the delta-rule configurations (tests and bench).

Distributions (one ``numpy.random.default_rng(seed)`` per case, draws in
the order q, k, v, beta, then S0, then sequence lengths):

* q, k ~ N(0, 1), L2-normalised per (b, t, h) vector as
  ``x / max(||x||, 1e-6)`` (the reference's ``_l2_normalize``,
  ``model/__init__.py:203-205``), then cast to the input dtype
  (bf16 by round-to-nearest-even);
* v ~ N(0, 1) (cast likewise);
* beta = sigmoid(N(0, 1)), fp32;
* S0 ~ N(0, s0_std) fp32 when requested.

The fp32 values the reference would consume are the cast values upcast
back to fp32 (``kernels/__init__.py:344-347``); ``FwdInputs`` carries both.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

# The BASELINE configurations (index = config number).
CONFIGS = {
    0: dict(B=1, H=4, T=256, D=64, dtype="fp32", s0_std=None),
    1: dict(B=4, H=16, T=4096, D=128, dtype="bf16", s0_std=None),
    2: dict(total=16384, H=16, D=128, dtype="bf16", lo=64, hi=4096),
    3: dict(B=1, H=32, T=32768, D=128, dtype="bf16", s0_std=0.02),
    4: dict(B=256, H=32, D=128, dtype="bf16", steps=64, s0_std=0.02),
}


def l2_normalize(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    n = np.linalg.norm(x, axis=-1, keepdims=True)
    return (x / np.maximum(n, np.float32(eps))).astype(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    # finite inputs only: the largest finite pattern plus the bias stays below 2**32
    u = (u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))) >> np.uint32(16)
    return u.astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def sigmoid(x: np.ndarray) -> np.ndarray:
    return (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)


@dataclass
class FwdInputs:
    """q/k/v in the input dtype (``*_bits`` uint16 for bf16) and as fp32 values."""

    q: np.ndarray  # fp32 values the reference consumes
    k: np.ndarray
    v: np.ndarray
    beta: np.ndarray
    s0: np.ndarray | None
    dtype: str
    q_bits: np.ndarray | None = None
    k_bits: np.ndarray | None = None
    v_bits: np.ndarray | None = None


def _cast(x: np.ndarray, dtype: str):
    if dtype == "bf16":
        bits = bf16_bits(x)
        return bf16_to_f32(bits), bits
    if dtype == "fp32":
        return x.astype(np.float32), None
    raise ValueError(dtype)


def fwd_inputs(shape, seed: int, dtype: str = "bf16", s0_std: float | None = None,
               normalize: bool = True) -> FwdInputs:
    """Inputs of shape (..., D) for q, k, v and (...) for beta; S0 (B, H, D, D).

    ``shape`` is (B, T, H, D) for the padded layout or (N, H, D) for packed.
    """
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(shape, dtype=np.float32)
    k = rng.standard_normal(shape, dtype=np.float32)
    v = rng.standard_normal(shape, dtype=np.float32)
    beta = sigmoid(rng.standard_normal(shape[:-1], dtype=np.float32))
    if normalize:
        q, k = l2_normalize(q), l2_normalize(k)
    s0 = None
    if s0_std is not None:
        if len(shape) != 4:
            raise ValueError("s0 needs the (B, T, H, D) layout")
        b, _, h, d = shape
        s0 = rng.normal(0.0, s0_std, (b, h, d, d)).astype(np.float32)
    qf, qb = _cast(q, dtype)
    kf, kb = _cast(k, dtype)
    vf, vb = _cast(v, dtype)
    return FwdInputs(qf, kf, vf, beta, s0, dtype, qb, kb, vb)


def varlen_lengths(total: int, lo: int, hi: int, seed: int) -> np.ndarray:
    """Lengths drawn from U[lo, hi] until they reach ``total``; the last is clipped."""
    rng = np.random.default_rng(seed)
    out = []
    acc = 0
    while acc < total:
        n = int(rng.integers(lo, hi + 1))
        n = min(n, total - acc)
        out.append(n)
        acc += n
    return np.asarray(out, dtype=np.int64)


def cu_seqlens(lengths: np.ndarray) -> np.ndarray:
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)


def reference_test_inputs(rng: np.random.Generator, batch=2, seq=5, heads=2, dim=4):
    """The reference tests' distribution (tests/test_kernels.py:77-82):
    unnormalised N(0, 1) q, k, v and beta = 0.35 + 0.30 U[0, 1)."""
    q = rng.standard_normal((batch, seq, heads, dim)).astype(np.float32)
    k = rng.standard_normal((batch, seq, heads, dim)).astype(np.float32)
    v = rng.standard_normal((batch, seq, heads, dim)).astype(np.float32)
    beta = (0.35 + 0.30 * rng.random((batch, seq, heads))).astype(np.float32)
    return q, k, v, beta
