"""NumPy restatement of the gated delta rule (test infrastructure).

Not the product: only ``tests/`` uses this module, as the checker.

The reference names the gated variant as its model's intent (Gated
DeltaNet / KDA, ``spec/03-model.md:12``) and as known missing
(``PROGRESS.md:109``); it has no code or oracle for it. This restates the
published recurrence (Yang, Kautz, Hatamizadeh, "Gated Delta Networks:
Improving Mamba2 with Delta Rule", ICLR 2025) in this build's state
convention ([d_k][d_v], ``o_t = q_t S_t``) with a scalar log-gate per
(token, head), ``alpha_t = exp(g_t)``:

    S_t = alpha_t (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T
    o_t = q_t S_t

With ``g = 0`` it is the delta rule of ``delta_oracle.gated_delta_rule``.

Pinned (tests/test_oracle_gated.py) by: reduction to the pinned delta-rule
oracle at g = 0; the closed forms at beta = 0 (pure decay: S_T = prod(alpha)
S_0) and for one token; linearity in (v, S_0); agreement of the per-token
form with the independent chunked (WY) restatement below at several chunk
sizes; and planted mistakes (gate applied after the update, gate on the
rank-1 term only, exp of the wrong sign) that these checks catch.
"""

from __future__ import annotations

import numpy as np


def gated_delta_rule(q, k, v, beta, g, state=None, dtype=np.float64):
    """Per-token recurrence; q, k, v (B, T, H, D), beta and g (B, T, H), state (B, H, D, D)."""
    q, k, v, beta, g = (np.asarray(x, dtype=dtype) for x in (q, k, v, beta, g))
    b, t, h, d = q.shape
    s = np.zeros((b, h, d, d), dtype=dtype) if state is None else np.array(state, dtype=dtype)
    out = np.zeros((b, t, h, d), dtype=dtype)
    for i in range(t):
        kt, vt, qt = k[:, i], v[:, i], q[:, i]
        bt = beta[:, i][..., None, None]
        at = np.exp(g[:, i])[..., None, None]
        ks = np.einsum("bhd,bhde->bhe", kt, s)
        s = at * (s - bt * np.einsum("bhd,bhe->bhde", kt, ks)) + bt * np.einsum("bhd,bhe->bhde", kt, vt)
        out[:, i] = np.einsum("bhd,bhde->bhe", qt, s)
    return out, s


def gated_wy_chunked(q, k, v, beta, g, state=None, chunk=64, dtype=np.float64):
    """The chunked (WY/UT) form with in-chunk decays, independent of the loop above.

    Per chunk, with G the cumulative log-gate inside the chunk and
    Gam[t, s] = exp(G_t - G_s) (t >= s; every factor <= 1 when g <= 0):
        A = strict_lower(diag(beta) (Gam * K K^T)),  T = (I + A)^-1
        U = T diag(beta) (V - diag(exp G) K S)
        O = diag(exp G) Q S + (Gam * lower_incl(Q K^T)) U
        S <- exp(G_C) S + K^T diag(exp(G_C - G)) U
    """
    q, k, v, beta, g = (np.asarray(x, dtype=dtype) for x in (q, k, v, beta, g))
    b, t, h, d = q.shape
    s_all = np.zeros((b, h, d, d), dtype=dtype) if state is None else np.array(state, dtype=dtype)
    out = np.zeros((b, t, h, d), dtype=dtype)
    for bi in range(b):
        for hi in range(h):
            s = s_all[bi, hi]
            for c0 in range(0, t, chunk):
                sl = slice(c0, min(t, c0 + chunk))
                K, Q, V = k[bi, sl, hi], q[bi, sl, hi], v[bi, sl, hi]
                be, G = beta[bi, sl, hi], np.cumsum(g[bi, sl, hi])
                n = K.shape[0]
                # exponents above the diagonal are positive (and can overflow): mask them first
                low = np.tril(np.ones((n, n), dtype=bool))
                gam = np.exp(np.where(low, G[:, None] - G[None, :], -np.inf))
                A = np.tril(be[:, None] * gam * (K @ K.T), -1)
                T = np.linalg.inv(np.eye(n) + A)
                U = T @ (be[:, None] * (V - np.exp(G)[:, None] * (K @ s)))
                out[bi, sl, hi] = np.exp(G)[:, None] * (Q @ s) + (gam * (Q @ K.T)) @ U
                s = np.exp(G[-1]) * s + K.T @ (np.exp(G[-1] - G)[:, None] * U)
            s_all[bi, hi] = s
    return out, s_all


def gated_step(s, q, k, v, beta, g):
    """One token for (B, H, D) inputs, beta and g (B, H); returns (o, new state)."""
    o, s1 = gated_delta_rule(np.asarray(q)[:, None], np.asarray(k)[:, None], np.asarray(v)[:, None],
                             np.asarray(beta)[:, None], np.asarray(g)[:, None], s)
    return o[:, 0], s1


def gated_vjp(q, k, v, beta, g, go, gs, state=None, dtype=np.float64):
    """Reverse mode of ``gated_delta_rule`` with the full state history.

    With P_t = alpha_t S_{t-1} (the decayed state) the step is S_t = P_t + beta_t k_t u_t^T,
    u_t = v_t - P_t^T k_t, and per token in reverse (G = dL/dS_t after G += q_t go_t^T):

        w = G^T k_t      x = G u_t      y = P_t w
        gq_t = S_t go_t  gv_t = beta_t w   gbeta_t = k_t . x   gk_t = beta_t (x - y)
        G_P = G - beta_t k_t w^T       gg_t = <G_P, P_t>  (dL/dg_t = alpha_t dL/dalpha_t)
        G <- alpha_t G_P

    ``go`` (B, T, H, D) and ``gs`` (B, H, D, D) may be None (zeros).
    Returns (gq, gk, gv, gbeta, gg, gstate0). With g = 0 the first four and gstate0 are
    ``delta_oracle.delta_vjp``'s.
    """
    q, k, v, beta, g = (np.asarray(x, dtype=dtype) for x in (q, k, v, beta, g))
    b, t, h, d = q.shape
    go = np.zeros((b, t, h, d), dtype) if go is None else np.asarray(go, dtype=dtype)
    G = np.zeros((b, h, d, d), dtype) if gs is None else np.array(gs, dtype=dtype)
    s = np.zeros((b, h, d, d), dtype=dtype) if state is None else np.array(state, dtype=dtype)
    hist = [s]
    us = []
    for i in range(t):
        a = np.exp(g[:, i])[..., None, None]
        p = a * s
        u = v[:, i] - np.einsum("bhd,bhde->bhe", k[:, i], p)
        s = p + beta[:, i][..., None, None] * np.einsum("bhd,bhe->bhde", k[:, i], u)
        hist.append(s)
        us.append(u)
    gq, gk, gv = (np.zeros((b, t, h, d), dtype) for _ in range(3))
    gbeta, gg = np.zeros((b, t, h), dtype), np.zeros((b, t, h), dtype)
    for i in range(t - 1, -1, -1):
        kt, bt, a = k[:, i], beta[:, i], np.exp(g[:, i])
        s_t, p = hist[i + 1], a[..., None, None] * hist[i]
        gq[:, i] = np.einsum("bhe,bhde->bhd", go[:, i], s_t)
        G = G + np.einsum("bhd,bhe->bhde", q[:, i], go[:, i])
        w = np.einsum("bhde,bhd->bhe", G, kt)
        x = np.einsum("bhde,bhe->bhd", G, us[i])
        y = np.einsum("bhde,bhe->bhd", p, w)
        gv[:, i] = bt[..., None] * w
        gbeta[:, i] = np.einsum("bhd,bhd->bh", kt, x)
        gk[:, i] = bt[..., None] * (x - y)
        G = G - bt[..., None, None] * np.einsum("bhd,bhe->bhde", kt, w)
        gg[:, i] = np.einsum("bhde,bhde->bh", G, p)
        G = a[..., None, None] * G
    return gq, gk, gv, gbeta, gg, G


# --- KDA: a log-gate per key channel (Kimi Delta Attention) ---


def kda_delta_rule(q, k, v, beta, g, state=None, dtype=np.float64):
    """Per-token recurrence with a decay per key channel: g (B, T, H, D) log-gates,
    alpha_t = exp(g_t) a d_k-vector, and (Kimi Linear's KDA, the reference's "KDA
    family" of spec/03-model.md:12)

        S_t = (I - beta_t k_t k_t^T) Diag(alpha_t) S_{t-1} + beta_t k_t v_t^T,   o_t = q_t S_t

    With g constant along d it is ``gated_delta_rule`` (Diag(alpha) = alpha I commutes)."""
    q, k, v, beta, g = (np.asarray(x, dtype=dtype) for x in (q, k, v, beta, g))
    b, t, h, d = q.shape
    s = np.zeros((b, h, d, d), dtype=dtype) if state is None else np.array(state, dtype=dtype)
    out = np.zeros((b, t, h, d), dtype=dtype)
    for i in range(t):
        kt, vt, qt = k[:, i], v[:, i], q[:, i]
        bt = beta[:, i][..., None, None]
        s = np.exp(g[:, i])[..., None] * s  # rows (key channels) decay
        ks = np.einsum("bhd,bhde->bhe", kt, s)
        s = s - bt * np.einsum("bhd,bhe->bhde", kt, ks) + bt * np.einsum("bhd,bhe->bhde", kt, vt)
        out[:, i] = np.einsum("bhd,bhde->bhe", qt, s)
    return out, s


def kda_wy_chunked(q, k, v, beta, g, state=None, chunk=16, dtype=np.float64):
    """The chunked (WY/UT) form of ``kda_delta_rule``, independent of the loop above.

    Per chunk, with G_t the cumulative log-gates inside the chunk (a d_k-vector per token),
    K^ = K * exp(G) and K~ = K * exp(-G) (row-wise), Q^ = Q * exp(G):
        A = strict_lower(diag(beta) K^ K~^T),  U = (I + A)^-1 diag(beta) (V - K^ S)
        O = Q^ S + lower_incl(Q^ K~^T) U,      S <- Diag(exp(G_C)) S + (K * exp(G_C - G))^T U
    (exp(-G) grows along the chunk, so the chunk is kept short for the test inputs.)"""
    q, k, v, beta, g = (np.asarray(x, dtype=dtype) for x in (q, k, v, beta, g))
    b, t, h, d = q.shape
    s_all = np.zeros((b, h, d, d), dtype=dtype) if state is None else np.array(state, dtype=dtype)
    out = np.zeros((b, t, h, d), dtype=dtype)
    for bi in range(b):
        for hi in range(h):
            s = s_all[bi, hi]
            for c0 in range(0, t, chunk):
                sl = slice(c0, min(t, c0 + chunk))
                K, Q, V = k[bi, sl, hi], q[bi, sl, hi], v[bi, sl, hi]
                be, G = beta[bi, sl, hi], np.cumsum(g[bi, sl, hi], axis=0)
                n = K.shape[0]
                Kh, Kt, Qh = K * np.exp(G), K * np.exp(-G), Q * np.exp(G)
                A = np.tril(be[:, None] * (Kh @ Kt.T), -1)
                U = np.linalg.solve(np.eye(n) + A, be[:, None] * (V - Kh @ s))
                out[bi, sl, hi] = Qh @ s + np.tril(Qh @ Kt.T) @ U
                s = np.exp(G[-1])[:, None] * s + (K * np.exp(G[-1] - G)).T @ U
            s_all[bi, hi] = s
    return out, s_all


def kda_step(s, q, k, v, beta, g):
    """One KDA token for (B, H, D) inputs, beta (B, H), g (B, H, D); returns (o, new state)."""
    o, s1 = kda_delta_rule(np.asarray(q)[:, None], np.asarray(k)[:, None], np.asarray(v)[:, None],
                           np.asarray(beta)[:, None], np.asarray(g)[:, None], s)
    return o[:, 0], s1


def kda_vjp(q, k, v, beta, g, go, gs, state=None, dtype=np.float64):
    """Reverse mode of ``kda_delta_rule`` with the full state history.

    With P_t = Diag(alpha_t) S_{t-1} (each key channel's row decayed) the step is
    S_t = P_t + beta_t k_t u_t^T, u_t = v_t - P_t^T k_t, and per token in reverse
    (G = dL/dS_t after G += q_t go_t^T) everything is ``gated_vjp``'s except the gate:

        G_P = G - beta_t k_t w^T      gg_t[d] = <G_P[d, :], P_t[d, :]>      G <- Diag(alpha_t) G_P

    g (B, T, H, D); returns (gq, gk, gv, gbeta, gg (B, T, H, D), gstate0). With g constant
    along D, gg summed over D is ``gated_vjp``'s gg and the rest equals it.
    """
    q, k, v, beta, g = (np.asarray(x, dtype=dtype) for x in (q, k, v, beta, g))
    b, t, h, d = q.shape
    go = np.zeros((b, t, h, d), dtype) if go is None else np.asarray(go, dtype=dtype)
    G = np.zeros((b, h, d, d), dtype) if gs is None else np.array(gs, dtype=dtype)
    s = np.zeros((b, h, d, d), dtype=dtype) if state is None else np.array(state, dtype=dtype)
    hist, us = [s], []
    for i in range(t):
        p = np.exp(g[:, i])[..., None] * s
        u = v[:, i] - np.einsum("bhd,bhde->bhe", k[:, i], p)
        s = p + beta[:, i][..., None, None] * np.einsum("bhd,bhe->bhde", k[:, i], u)
        hist.append(s)
        us.append(u)
    gq, gk, gv, gg = (np.zeros((b, t, h, d), dtype) for _ in range(4))
    gbeta = np.zeros((b, t, h), dtype)
    for i in range(t - 1, -1, -1):
        kt, bt, a = k[:, i], beta[:, i], np.exp(g[:, i])
        s_t, p = hist[i + 1], a[..., None] * hist[i]
        gq[:, i] = np.einsum("bhe,bhde->bhd", go[:, i], s_t)
        G = G + np.einsum("bhd,bhe->bhde", q[:, i], go[:, i])
        w = np.einsum("bhde,bhd->bhe", G, kt)
        x = np.einsum("bhde,bhe->bhd", G, us[i])
        y = np.einsum("bhde,bhe->bhd", p, w)
        gv[:, i] = bt[..., None] * w
        gbeta[:, i] = np.einsum("bhd,bhd->bh", kt, x)
        gk[:, i] = bt[..., None] * (x - y)
        G = G - bt[..., None, None] * np.einsum("bhd,bhe->bhde", kt, w)
        gg[:, i] = np.einsum("bhde,bhde->bhd", G, p)
        G = a[..., None] * G
    return gq, gk, gv, gbeta, gg, G
