"""NumPy restatement of the model's linear attention (test infrastructure).

Not the product: only ``tests/`` uses this module, as the checker.

The reference's ``model.linear_attention`` (``model/__init__.py:393-432``)
and its NumPy restatement (``tests/reference/model.py:254-292``): q and k
are L2-normalised per (token, head) as ``x / max(||x||, 1e-6)``
(``model/__init__.py:203-205``), and the delta rule runs with beta = 1:

    S_t = (I - k^_t k^_t^T) S_{t-1} + k^_t v_t^T,    o_t = q^_t S_t

``_linear_attn`` (``model/__init__.py:726-734``) wraps it in the head
projections W_q, W_k, W_v (d_model, heads, d_head) and W_o (heads, d_head,
d_model).

Pinned (tests/test_oracle_model.py) by: equality with the independently
pinned delta-rule oracle on normalised inputs with beta = 1, the one-token
closed form, invariance under positive rescaling of q and k, the zero-vector
case of the eps guard, and the reference's own causality, state-carry and
3-D squeeze tests run on this restatement.
"""

from __future__ import annotations

import numpy as np

EPS = 1e-6


def l2_normalize(x, eps: float = EPS, dtype=np.float32):
    """``x / max(||x||_2, eps)`` over the last axis (``model/__init__.py:203-205``)."""
    x = np.asarray(x, dtype=dtype)
    n = np.sqrt(np.sum(x * x, axis=-1, keepdims=True))
    return x / np.maximum(n, dtype(eps))


def _ensure_heads(x, dtype):
    """3-D (B, S, D) gets a unit heads axis (``model/__init__.py:383-390``)."""
    x = np.asarray(x, dtype=dtype)
    if x.ndim == 3:
        return x[:, :, None, :], True
    if x.ndim == 4:
        return x, False
    raise ValueError(f"expected 3-D or 4-D tensor, got shape {x.shape}")


def linear_attention(q, k, v, state=None, dtype=np.float32):
    """Per-token loop of ``tests/reference/model.py:254-292``; returns (out, state)."""
    q, squeeze = _ensure_heads(q, dtype)
    k, _ = _ensure_heads(k, dtype)
    v, _ = _ensure_heads(v, dtype)
    if q.shape != k.shape or q.shape[:3] != v.shape[:3] or q.shape[-1] != v.shape[-1]:
        raise ValueError("q, k, v must share batch/seq/heads and key/value dim")
    b, t, h, d = q.shape
    qn = l2_normalize(q, dtype=dtype)
    kn = l2_normalize(k, dtype=dtype)
    if state is None:
        s = np.zeros((b, h, d, d), dtype=dtype)
    else:
        s = np.array(state, dtype=dtype)
        if s.ndim == 3:
            s = s[:, None, :, :]
        if s.shape != (b, h, d, d):
            raise ValueError(f"state shape {s.shape} != {(b, h, d, d)}")
    out = np.zeros((b, t, h, d), dtype=dtype)
    eye = np.eye(d, dtype=dtype)
    for i in range(t):
        kt, vt, qt = kn[:, i], v[:, i], qn[:, i]
        decay = eye[None, None] - np.einsum("bhd,bhe->bhde", kt, kt)
        s = np.einsum("bhij,bhjk->bhik", decay, s) + np.einsum("bhd,bhe->bhde", kt, vt)
        out[:, i] = np.einsum("bhd,bhde->bhe", qt, s)
    if squeeze:
        return out[:, :, 0, :], s[:, 0]
    return out, s


def linear_attn_layer(x, layer, state=None, dtype=np.float32):
    """``_linear_attn`` (``model/__init__.py:726-734``): projections around linear_attention."""
    x = np.asarray(x, dtype=dtype)
    w = {n: np.asarray(layer[n], dtype=dtype) for n in ("W_q", "W_k", "W_v", "W_o")}
    q = np.einsum("bsd,dhe->bshe", x, w["W_q"])
    k = np.einsum("bsd,dhe->bshe", x, w["W_k"])
    v = np.einsum("bsd,dhe->bshe", x, w["W_v"])
    y, s = linear_attention(q, k, v, state, dtype=dtype)
    return np.einsum("bshe,hed->bsd", y, w["W_o"]), s
