"""NumPy restatement of the reference delta-rule forward (test infrastructure).

Not the product: only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg use this module, as the checker.

Recurrence (reference contract, ``tests/reference/kernels.py:9-24``)::

    S_t = (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T
    o_t = q_t S_t

q, k, v: (B, T, H, D); beta: (B, T, H); state: (B, H, D, D) as [d_k][d_v].
"""

from __future__ import annotations

import numpy as np


def _as(x, dtype):
    return np.asarray(x, dtype=dtype)


def _check(q, k, v, beta, state):
    if q.ndim != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k, v must all have shape (B, S, H, D)")
    b, t, h, d = q.shape
    if beta.shape != (b, t, h):
        raise ValueError(f"beta shape {beta.shape} != {(b, t, h)}")
    if state is not None and state.shape != (b, h, d, d):
        raise ValueError(f"state shape {state.shape} != {(b, h, d, d)}")


def gated_delta_rule(q, k, v, beta, state=None, dtype=np.float32):
    """Explicit per-timestep recurrence with the (I - beta k k^T) matrix.

    Follows ``tests/reference/kernels.py:134-171`` (the reference's NumPy
    oracle): inputs cast to ``dtype``, ``state=None`` means zeros, every
    step forms ``decay = I - beta k k^T`` and left-multiplies the state.
    """
    q, k, v, beta = (_as(x, dtype) for x in (q, k, v, beta))
    st = None if state is None else _as(state, dtype)
    _check(q, k, v, beta, st)
    b, t, h, d = q.shape
    s = np.zeros((b, h, d, d), dtype=dtype) if st is None else st.copy()
    eye = np.eye(d, dtype=dtype)
    out = np.zeros((b, t, h, d), dtype=dtype)
    for i in range(t):
        kt, vt, qt = k[:, i], v[:, i], q[:, i]
        bt = beta[:, i, :, None, None]
        decay = eye[None, None] - bt * np.einsum("bhd,bhe->bhde", kt, kt)
        s = np.einsum("bhij,bhjk->bhik", decay, s)
        s = s + bt * np.einsum("bhd,bhe->bhde", kt, vt)
        out[:, i] = np.einsum("bhd,bhde->bhe", qt, s)
    return out, s


def delta_step(s, q, k, v, beta):
    """One rank-1 step on (B, H, D) tokens; returns (S', o).

    Follows ``kernels/__init__.py:357-366``: ``kS = k^T S``,
    ``S' = S - beta k kS^T + beta k v^T``, ``o = q S'``.
    """
    bt = beta[..., None, None]
    k_s = np.einsum("bhd,bhde->bhe", k, s)
    s_new = s - bt * np.einsum("bhd,bhe->bhde", k, k_s) + bt * np.einsum("bhd,bhe->bhde", k, v)
    o = np.einsum("bhd,bhde->bhe", q, s_new)
    return s_new, o


def chunked_fwd_rank1(q, k, v, beta, state=None, chunk=64, dtype=np.float32):
    """The reference's traversal: chunks, then timesteps, rank-1 steps.

    Follows ``kernels/__init__.py:379-395`` (NumPy path) and the order of
    ``:421-458`` (JAX path, including the remainder chunk and ``T == 0``).
    """
    if chunk < 1:
        raise ValueError(f"chunk must be >= 1, got {chunk}")
    q, k, v, beta = (_as(x, dtype) for x in (q, k, v, beta))
    st = None if state is None else _as(state, dtype)
    _check(q, k, v, beta, st)
    b, t, h, d = q.shape
    s = np.zeros((b, h, d, d), dtype=dtype) if st is None else st.copy()
    out = np.empty((b, t, h, d), dtype=dtype)
    for start in range(0, t, chunk):
        for i in range(start, min(start + chunk, t)):
            s, out[:, i] = delta_step(s, q[:, i], k[:, i], v[:, i], beta[:, i])
    return out, s


def wy_chunked_fwd(q, k, v, beta, state=None, chunk=64, dtype=np.float64):
    """Chunked WY/UT form (the GPU kernel's algorithm), fp64 by default.

    Not in the reference (its chunking is only a traversal order,
    ``kernels/__init__.py:471``); it is the exact algebraic restatement of
    the same recurrence (DeltaNet chunk form, Yang et al. 2024). Per chunk
    with start state S, rows K, V, Q, beta:

        A = strict_lower(diag(beta) K K^T)
        T = (I + A)^-1                     (unit lower triangular)
        U = T diag(beta) (V - K S)         (u_t = beta_t (v_t - S_{t-1}^T k_t))
        O = Q S + lower_incl_diag(Q K^T) U
        S <- S + K^T U
    """
    if chunk < 1:
        raise ValueError(f"chunk must be >= 1, got {chunk}")
    q, k, v, beta = (_as(x, dtype) for x in (q, k, v, beta))
    st = None if state is None else _as(state, dtype)
    _check(q, k, v, beta, st)
    b, t, h, d = q.shape
    s = np.zeros((b, h, d, d), dtype=dtype) if st is None else st.copy()
    out = np.zeros((b, t, h, d), dtype=dtype)
    # (B, H, T, D) views
    qh, kh, vh = (np.moveaxis(x, 2, 1) for x in (q, k, v))
    bh = np.moveaxis(beta, 2, 1)
    for start in range(0, t, chunk):
        end = min(start + chunk, t)
        c = end - start
        kc, vc, qc = kh[:, :, start:end], vh[:, :, start:end], qh[:, :, start:end]
        bc = bh[:, :, start:end]
        gram = np.einsum("bhid,bhjd->bhij", kc, kc)
        a = np.tril(bc[..., :, None] * gram, -1)
        tinv = np.linalg.inv(np.eye(c, dtype=dtype) + a)
        r = bc[..., None] * (vc - np.einsum("bhtd,bhde->bhte", kc, s))
        u = np.einsum("bhts,bhse->bhte", tinv, r)
        p = np.tril(np.einsum("bhid,bhjd->bhij", qc, kc))
        o = np.einsum("bhtd,bhde->bhte", qc, s) + np.einsum("bhts,bhse->bhte", p, u)
        out[:, start:end] = np.moveaxis(o, 2, 1)
        s = s + np.einsum("bhtd,bhte->bhde", kc, u)
    return out, s


def varlen_fwd(q, k, v, beta, cu_seqlens, state=None, dtype=np.float32):
    """Packed batch: independent sequences with the state reset per segment.

    q, k, v: (N, H, D); beta (N, H); cu_seqlens int (n+1,); state None or
    (n, H, D, D). Reduces to ``gated_delta_rule`` with B=1 on each segment
    (no reference counterpart exists; the reference equivalent is n
    separate ``chunked_delta_rule`` calls, ``kernels/__init__.py:591-619``).
    """
    q, k, v, beta = (_as(x, dtype) for x in (q, k, v, beta))
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    n = cu.size - 1
    _, h, d = q.shape
    out = np.zeros(q.shape, dtype=dtype)
    states = np.zeros((n, h, d, d), dtype=dtype)
    for i in range(n):
        a, z = int(cu[i]), int(cu[i + 1])
        s0 = None if state is None else _as(state, dtype)[i : i + 1]
        o, s = gated_delta_rule(q[None, a:z], k[None, a:z], v[None, a:z], beta[None, a:z], s0, dtype)
        out[a:z] = o[0]
        states[i] = s[0]
    return out, states


def delta_vjp(q, k, v, beta, go, gs, state=None, dtype=np.float64):
    """Reverse mode of the recurrence with the full state history.

    Follows the reference's ``_delta_vjp_np`` (``kernels/__init__.py:460-527``)
    and its oracle ``gated_delta_rule_vjp`` (``tests/reference/kernels.py:174-251``):
    a forward pass keeps every S_t, then a reverse pass per token

        gq_t = S_t go_t             g_S += q_t go_t^T
        g_A  = g_S S_{t-1}^T        gv_t = beta_t g_S^T k_t
        gk_t = beta_t (g_S v_t - g_A k_t - g_A^T k_t)
        gbeta_t = k_t^T g_S v_t - k_t^T g_A k_t
        g_S <- (I - beta_t k_t k_t^T) g_S

    ``go`` is dL/dO (B, T, H, D), ``gs`` dL/dS_T (B, H, D, D), either may be
    None (zeros).  Returns (gq, gk, gv, gbeta, gstate0).
    """
    q, k, v, beta = (_as(x, dtype) for x in (q, k, v, beta))
    st = None if state is None else _as(state, dtype)
    _check(q, k, v, beta, st)
    b, t, h, d = q.shape
    go = np.zeros((b, t, h, d), dtype) if go is None else _as(go, dtype)
    g_s = np.zeros((b, h, d, d), dtype) if gs is None else _as(gs, dtype).copy()
    s = np.zeros((b, h, d, d), dtype=dtype) if st is None else st.copy()
    eye = np.eye(d, dtype=dtype)
    hist = [s]
    for i in range(t):
        bt = beta[:, i, :, None, None]
        decay = eye[None, None] - bt * np.einsum("bhd,bhe->bhde", k[:, i], k[:, i])
        s = np.einsum("bhij,bhjk->bhik", decay, s) + bt * np.einsum("bhd,bhe->bhde", k[:, i], v[:, i])
        hist.append(s)
    gq, gk, gv = (np.zeros((b, t, h, d), dtype) for _ in range(3))
    gbeta = np.zeros((b, t, h), dtype)
    for i in range(t - 1, -1, -1):
        qt, kt, vt, bt, g_o = q[:, i], k[:, i], v[:, i], beta[:, i], go[:, i]
        s_t, s_prev = hist[i + 1], hist[i]
        gq[:, i] = np.einsum("bhe,bhde->bhd", g_o, s_t)
        g_s = g_s + np.einsum("bhd,bhe->bhde", qt, g_o)
        g_a = np.einsum("bhik,bhjk->bhij", g_s, s_prev)
        gv[:, i] = np.einsum("bhde,bhd->bhe", g_s, kt) * bt[..., None]
        gk[:, i] = bt[..., None] * (np.einsum("bhde,bhe->bhd", g_s, vt)
                                    - np.einsum("bhde,bhe->bhd", g_a, kt)
                                    - np.einsum("bhed,bhe->bhd", g_a, kt))
        gbeta[:, i] = (np.einsum("bhde,bhd,bhe->bh", g_s, kt, vt)
                       - np.einsum("bhde,bhd,bhe->bh", g_a, kt, kt))
        a_t = eye[None, None] - bt[..., None, None] * np.einsum("bhd,bhe->bhde", kt, kt)
        g_s = np.einsum("bhij,bhik->bhjk", a_t, g_s)
    return gq, gk, gv, gbeta, g_s


def delta_vjp_downdate(q, k, v, beta, go, gs, state=None, ckpt=64, dtype=np.float64):
    """The same gradients in the form the GPU backward computes them.

    Not in the reference: a restatement that keeps no state history.  A
    forward pass stores u_t = v_t - S_{t-1}^T k_t per token and the state at
    the end of every ``ckpt`` tokens; the reverse pass restarts from those
    checkpoints and walks the state back exactly, S_{t-1} = S_t - beta_t k_t
    u_t^T, with (w_t = g_S^T k_t after g_S += q_t go_t^T)

        gq_t = S_t go_t          gv_t = beta_t w_t
        gk_t = beta_t (g_S u_t - S_{t-1} w_t)      gbeta_t = k_t^T g_S u_t
        g_S <- g_S - beta_t k_t w_t^T

    (g_A k_t = g_S S_{t-1}^T k_t = g_S (v_t - u_t) folds the reference's
    three k-terms into these two.)
    """
    q, k, v, beta = (_as(x, dtype) for x in (q, k, v, beta))
    st = None if state is None else _as(state, dtype)
    _check(q, k, v, beta, st)
    b, t, h, d = q.shape
    go = np.zeros((b, t, h, d), dtype) if go is None else _as(go, dtype)
    g_s = np.zeros((b, h, d, d), dtype) if gs is None else _as(gs, dtype).copy()
    s = np.zeros((b, h, d, d), dtype=dtype) if st is None else st.copy()
    u = np.zeros((b, t, h, d), dtype)
    ends = {}
    for i in range(t):
        u[:, i] = v[:, i] - np.einsum("bhd,bhde->bhe", k[:, i], s)
        s = s + beta[:, i, :, None, None] * np.einsum("bhd,bhe->bhde", k[:, i], u[:, i])
        if (i + 1) % ckpt == 0 or i + 1 == t:
            ends[i] = s.copy()
    gq, gk, gv = (np.zeros((b, t, h, d), dtype) for _ in range(3))
    gbeta = np.zeros((b, t, h), dtype)
    for i in range(t - 1, -1, -1):
        if i in ends:
            s = ends[i].copy()
        kt, bt, g_o = k[:, i], beta[:, i], go[:, i]
        gq[:, i] = np.einsum("bhde,bhe->bhd", s, g_o)
        g_s = g_s + np.einsum("bhd,bhe->bhde", q[:, i], g_o)
        w = np.einsum("bhde,bhd->bhe", g_s, kt)
        x = np.einsum("bhde,bhe->bhd", g_s, u[:, i])
        s = s - bt[..., None, None] * np.einsum("bhd,bhe->bhde", kt, u[:, i])
        y = np.einsum("bhde,bhe->bhd", s, w)
        gv[:, i] = bt[..., None] * w
        gk[:, i] = bt[..., None] * (x - y)
        gbeta[:, i] = np.einsum("bhd,bhd->bh", kt, x)
        g_s = g_s - bt[..., None, None] * np.einsum("bhd,bhe->bhde", kt, w)
    return gq, gk, gv, gbeta, g_s


def rel_l2(got, exp) -> float:
    """||got - exp||_2 / ||exp||_2 over all elements (0/0 -> 0)."""
    got = np.asarray(got, dtype=np.float64)
    exp = np.asarray(exp, dtype=np.float64)
    num = float(np.linalg.norm((got - exp).ravel()))
    den = float(np.linalg.norm(exp.ravel()))
    if den == 0.0:
        return num
    return num / den
