"""CPU tests that pin the gated delta-rule oracle (oracle/gated_oracle.py),
for which the reference holds no code or oracle (spec/03-model.md:12 names
the variant; PROGRESS.md:109 lists it as missing). Pinned by mathematics:
reduction to the pinned delta-rule oracle at g = 0, closed forms, linearity,
agreement of two independent formulations, and planted mistakes.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import delta_oracle as dref
from oracle import gated_oracle as gref


def _problem(rng, shape, gate_scale=0.3):
    b, t, h, d = shape
    q = rng.standard_normal(shape)
    k = rng.standard_normal(shape)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal(shape)
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((b, t, h))))
    g = -gate_scale * np.abs(rng.standard_normal((b, t, h)))  # log-gates <= 0
    s0 = rng.standard_normal((b, h, d, d)) * 0.1
    return q, k, v, beta, g, s0


def test_zero_gate_is_the_delta_rule():
    rng = np.random.default_rng(1)
    q, k, v, beta, _, s0 = _problem(rng, (2, 9, 2, 5))
    o, s = gref.gated_delta_rule(q, k, v, beta, np.zeros(beta.shape), s0)
    o2, s2 = dref.gated_delta_rule(q, k, v, beta, s0, dtype=np.float64)
    np.testing.assert_allclose(o, o2, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(s, s2, rtol=1e-12, atol=1e-12)


def test_pure_decay_closed_form():
    """beta = 0: S_t = (prod_{s<=t} alpha_s) S_0 and o_t = q_t S_t."""
    rng = np.random.default_rng(2)
    q, k, v, _, g, s0 = _problem(rng, (1, 7, 2, 4))
    o, s = gref.gated_delta_rule(q, k, v, np.zeros(g.shape), g, s0)
    cum = np.exp(np.cumsum(g, axis=1))  # (B, T, H)
    np.testing.assert_allclose(s, cum[:, -1, :, None, None] * s0, rtol=1e-12)
    want = cum[..., None] * np.einsum("bthd,bhde->bthe", q, s0)
    np.testing.assert_allclose(o, want, rtol=1e-12, atol=1e-14)


def test_one_token_closed_form():
    rng = np.random.default_rng(3)
    q, k, v, beta, g, s0 = _problem(rng, (1, 1, 1, 6))
    o, s = gref.gated_delta_rule(q, k, v, beta, g, s0)
    a, b_ = np.exp(g[0, 0, 0]), beta[0, 0, 0]
    kk, vv, qq, S0 = k[0, 0, 0], v[0, 0, 0], q[0, 0, 0], s0[0, 0]
    s1 = a * (S0 - b_ * np.outer(kk, kk @ S0)) + b_ * np.outer(kk, vv)
    np.testing.assert_allclose(s[0, 0], s1, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(o[0, 0, 0], qq @ s1, rtol=1e-12, atol=1e-14)


def test_linear_in_values_and_state():
    rng = np.random.default_rng(4)
    q, k, v, beta, g, s0 = _problem(rng, (1, 11, 2, 4))
    _, _, v2, _, _, s02 = _problem(rng, (1, 11, 2, 4))
    a = gref.gated_delta_rule(q, k, v, beta, g, s0)
    b = gref.gated_delta_rule(q, k, v2, beta, g, s02)
    c = gref.gated_delta_rule(q, k, 2.0 * v - 3.0 * v2, beta, g, 2.0 * s0 - 3.0 * s02)
    for x, y, z in zip(a, b, c):
        np.testing.assert_allclose(z, 2.0 * x - 3.0 * y, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("chunk", [1, 4, 16, 64])
def test_chunked_form_agrees(chunk):
    rng = np.random.default_rng(5)
    for shape, scale in [((2, 70, 2, 8), 0.3), ((1, 130, 1, 16), 2.0), ((1, 33, 2, 4), 0.0)]:
        q, k, v, beta, g, s0 = _problem(rng, shape, scale)
        a = gref.gated_delta_rule(q, k, v, beta, g, s0)
        b = gref.gated_wy_chunked(q, k, v, beta, g, s0, chunk=chunk)
        for x, y in zip(a, b):
            np.testing.assert_allclose(y, x, rtol=1e-9, atol=1e-11)


def test_strong_decay_stays_finite():
    """Log-gates of -20 per token: every factor of the chunked form stays <= 1."""
    rng = np.random.default_rng(6)
    q, k, v, beta, _, s0 = _problem(rng, (1, 64, 1, 8))
    g = np.full(beta.shape, -20.0)
    a = gref.gated_delta_rule(q, k, v, beta, g, s0)
    b = gref.gated_wy_chunked(q, k, v, beta, g, s0, chunk=64)
    for x, y in zip(a, b):
        assert np.all(np.isfinite(y))
        np.testing.assert_allclose(y, x, rtol=1e-9, atol=1e-11)


def _planted(kind):
    def f(q, k, v, beta, g, s0):
        b, t, h, d = q.shape
        s = np.array(s0, dtype=np.float64)
        out = np.zeros((b, t, h, d))
        for i in range(t):
            kt, vt, qt = k[:, i], v[:, i], q[:, i]
            bt = beta[:, i][..., None, None]
            at = np.exp(g[:, i])[..., None, None]
            if kind == "gate_after_update":
                ks = np.einsum("bhd,bhde->bhe", kt, s)
                s = at * (s - bt * np.einsum("bhd,bhe->bhde", kt, ks) + bt * np.einsum("bhd,bhe->bhde", kt, vt))
            elif kind == "gate_on_rank1_only":
                ks = np.einsum("bhd,bhde->bhe", kt, s)
                s = s - at * bt * np.einsum("bhd,bhe->bhde", kt, ks) + bt * np.einsum("bhd,bhe->bhde", kt, vt)
            elif kind == "wrong_sign":
                at = np.exp(-g[:, i])[..., None, None]
                ks = np.einsum("bhd,bhde->bhe", kt, s)
                s = at * (s - bt * np.einsum("bhd,bhe->bhde", kt, ks)) + bt * np.einsum("bhd,bhe->bhde", kt, vt)
            out[:, i] = np.einsum("bhd,bhde->bhe", qt, s)
        return out, s
    return f


@pytest.mark.parametrize("kind", ["gate_after_update", "gate_on_rank1_only", "wrong_sign"])
def test_planted_mistakes_are_caught(kind):
    rng = np.random.default_rng(7)
    q, k, v, beta, g, s0 = _problem(rng, (1, 1, 1, 6))
    wrong = _planted(kind)
    o, s = wrong(q, k, v, beta, g, s0)
    a, b_ = np.exp(g[0, 0, 0]), beta[0, 0, 0]
    kk, vv, S0 = k[0, 0, 0], v[0, 0, 0], s0[0, 0]
    s1 = a * (S0 - b_ * np.outer(kk, kk @ S0)) + b_ * np.outer(kk, vv)
    assert not np.allclose(s[0, 0], s1, rtol=1e-9)


# --- the reverse mode (gated_vjp) ---


def _loss(q, k, v, beta, g, s0, go, gs):
    o, s = gref.gated_delta_rule(q, k, v, beta, g, s0)
    return float(np.sum(o * go) + np.sum(s * gs))


def test_vjp_zero_gate_is_the_delta_rule_vjp():
    """g = 0: the five ungated gradients are the pinned delta_vjp's."""
    rng = np.random.default_rng(11)
    q, k, v, beta, _, s0 = _problem(rng, (2, 9, 2, 5))
    go = rng.standard_normal(q.shape)
    gs = rng.standard_normal(s0.shape) * 0.1
    got = gref.gated_vjp(q, k, v, beta, np.zeros(beta.shape), go, gs, s0)
    want = dref.delta_vjp(q, k, v, beta, go, gs, s0)
    for name, a, b in zip(("gq", "gk", "gv", "gbeta", "gs0"), got[:4] + got[5:], want):
        np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12, err_msg=name)


@pytest.mark.parametrize("gate_scale", [0.05, 0.3, 2.0])
def test_vjp_finite_differences(gate_scale):
    """Every gradient, g's included, against central differences of the fp64 forward
    along random directions (strong decay at gate_scale 2: alpha down to ~0.01)."""
    rng = np.random.default_rng(int(gate_scale * 100))
    q, k, v, beta, g, s0 = _problem(rng, (1, 7, 2, 4), gate_scale)
    go = rng.standard_normal(q.shape)
    gs = rng.standard_normal(s0.shape)
    grads = gref.gated_vjp(q, k, v, beta, g, go, gs, s0)
    args = {"q": q, "k": k, "v": v, "beta": beta, "g": g, "s0": s0}
    eps = 1e-6
    for name, gx in zip(("q", "k", "v", "beta", "g", "s0"), grads):
        d = rng.standard_normal(args[name].shape)
        plus, minus = dict(args), dict(args)
        plus[name], minus[name] = args[name] + eps * d, args[name] - eps * d
        fd = (_loss(**plus, go=go, gs=gs) - _loss(**minus, go=go, gs=gs)) / (2 * eps)
        np.testing.assert_allclose(np.sum(gx * d), fd, rtol=1e-6, atol=1e-8, err_msg=name)


def test_vjp_pure_decay_closed_form():
    """beta = 0, go = 0: S_T = exp(sum g) S_0, so dL/dg_t = <gs, S_T> for every t and
    dL/dS_0 = exp(sum g) gs."""
    rng = np.random.default_rng(12)
    q, k, v, _, g, s0 = _problem(rng, (1, 6, 2, 3))
    gs = rng.standard_normal(s0.shape)
    _, _, _, _, gg, gs0 = gref.gated_vjp(q, k, v, np.zeros(g.shape), g, None, gs, s0)
    s_t = np.exp(g.sum(axis=1))[..., None, None] * s0
    want = np.einsum("bhde,bhde->bh", gs, s_t)
    np.testing.assert_allclose(gg, np.repeat(want[:, None], g.shape[1], axis=1), rtol=1e-12)
    np.testing.assert_allclose(gs0, np.exp(g.sum(axis=1))[..., None, None] * gs, rtol=1e-12)


def test_vjp_planted_mistakes_are_caught():
    """Restatements with a plausible mistake each (the gate gradient taken against S_{t-1}
    instead of alpha S_{t-1}; G not scaled by alpha; the gate's gradient taken before the
    rank-1 downdate) differ from finite differences."""
    rng = np.random.default_rng(13)
    q, k, v, beta, g, s0 = _problem(rng, (1, 5, 1, 4), 0.5)
    go = rng.standard_normal(q.shape)
    gs = rng.standard_normal(s0.shape)
    eps = 1e-6
    d = rng.standard_normal(g.shape)
    fd = (_loss(q, k, v, beta, g + eps * d, s0, go, gs) - _loss(q, k, v, beta, g - eps * d, s0, go, gs)) / (2 * eps)

    def mutant(kind):
        b, t, h, dd = q.shape
        G = gs.copy()
        s = s0.copy()
        hist, us = [s], []
        for i in range(t):
            a = np.exp(g[:, i])[..., None, None]
            p = a * s
            u = v[:, i] - np.einsum("bhd,bhde->bhe", k[:, i], p)
            s = p + beta[:, i][..., None, None] * np.einsum("bhd,bhe->bhde", k[:, i], u)
            hist.append(s)
            us.append(u)
        gg = np.zeros(g.shape)
        for i in range(t - 1, -1, -1):
            a = np.exp(g[:, i])
            p = a[..., None, None] * hist[i]
            G = G + np.einsum("bhd,bhe->bhde", q[:, i], go[:, i])
            w = np.einsum("bhde,bhd->bhe", G, k[:, i])
            if kind == "before_downdate":
                gg[:, i] = np.einsum("bhde,bhde->bh", G, p)
            G = G - beta[:, i][..., None, None] * np.einsum("bhd,bhe->bhde", k[:, i], w)
            if kind == "no_alpha_in_gate":
                gg[:, i] = np.einsum("bhde,bhde->bh", G, hist[i])
            elif kind != "before_downdate":
                gg[:, i] = np.einsum("bhde,bhde->bh", G, p)
            if kind != "G_not_scaled":
                G = a[..., None, None] * G
        return float(np.sum(gg * d))

    for kind in ("no_alpha_in_gate", "G_not_scaled", "before_downdate"):
        assert abs(mutant(kind) - fd) > 1e-4 * max(1.0, abs(fd)), kind
    assert abs(mutant("correct") - fd) < 1e-6 * max(1.0, abs(fd))


# --- KDA (per-channel decay) ---


def _kda_problem(rng, shape, gate_scale=0.2):
    q, k, v, beta, _, s0 = _problem(rng, shape)
    g = -gate_scale * np.abs(rng.standard_normal(shape))  # a log-gate per key channel
    return q, k, v, beta, g, s0


def test_kda_channel_constant_gate_is_the_scalar_gate():
    rng = np.random.default_rng(21)
    q, k, v, beta, g, s0 = _problem(rng, (2, 9, 2, 5))
    gch = np.repeat(g[..., None], 5, axis=-1)
    o, s = gref.kda_delta_rule(q, k, v, beta, gch, s0)
    o2, s2 = gref.gated_delta_rule(q, k, v, beta, g, s0)
    np.testing.assert_allclose(o, o2, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(s, s2, rtol=1e-12, atol=1e-12)


def test_kda_pure_decay_closed_form():
    """beta = 0: row d of S decays by exp(sum of g[.., d]), and o_t = q_t Diag(exp G_t) S_0."""
    rng = np.random.default_rng(22)
    q, k, v, _, g, s0 = _kda_problem(rng, (1, 6, 2, 4))
    o, s = gref.kda_delta_rule(q, k, v, np.zeros(g.shape[:3]), g, s0)
    G = np.cumsum(g, axis=1)  # (B, T, H, D)
    np.testing.assert_allclose(s, np.exp(G[:, -1])[..., None] * s0, rtol=1e-12)
    want = np.einsum("bthd,bhde->bthe", q * np.exp(G), s0)
    np.testing.assert_allclose(o, want, rtol=1e-12, atol=1e-14)


def test_kda_one_token_closed_form():
    rng = np.random.default_rng(23)
    q, k, v, beta, g, s0 = _kda_problem(rng, (1, 1, 1, 6))
    o, s = gref.kda_delta_rule(q, k, v, beta, g, s0)
    a, b_ = np.exp(g[0, 0, 0]), beta[0, 0, 0]
    kk, vv, qq, S0 = k[0, 0, 0], v[0, 0, 0], q[0, 0, 0], s0[0, 0]
    ds = a[:, None] * S0
    s1 = ds - b_ * np.outer(kk, kk @ ds) + b_ * np.outer(kk, vv)
    np.testing.assert_allclose(s[0, 0], s1, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(o[0, 0, 0], qq @ s1, rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("chunk", [1, 3, 8, 16])
def test_kda_chunked_form_agrees(chunk):
    rng = np.random.default_rng(24 + chunk)
    q, k, v, beta, g, s0 = _kda_problem(rng, (2, 21, 2, 6))
    o, s = gref.kda_delta_rule(q, k, v, beta, g, s0)
    o2, s2 = gref.kda_wy_chunked(q, k, v, beta, g, s0, chunk=chunk)
    np.testing.assert_allclose(o2, o, rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(s2, s, rtol=1e-9, atol=1e-10)


def test_kda_planted_mistakes_are_caught():
    """Decay on the columns instead of the rows, decay after the rank-1 update, and the
    opposite sign of the exponent each differ from the recurrence."""
    rng = np.random.default_rng(25)
    q, k, v, beta, g, s0 = _kda_problem(rng, (1, 8, 1, 5), 0.5)
    o, s = gref.kda_delta_rule(q, k, v, beta, g, s0)

    def mutant(kind):
        st = s0[0, 0].copy()
        outs = []
        for i in range(q.shape[1]):
            a = np.exp(-g[0, i, 0] if kind == "sign" else g[0, i, 0])
            kk, vv, bb = k[0, i, 0], v[0, i, 0], beta[0, i, 0]
            if kind == "columns":
                st = st * a[None, :]
            elif kind != "after":
                st = a[:, None] * st
            st = st - bb * np.outer(kk, kk @ st) + bb * np.outer(kk, vv)
            if kind == "after":
                st = a[:, None] * st
            outs.append(q[0, i, 0] @ st)
        return np.array(outs)

    for kind in ("columns", "after", "sign"):
        assert np.abs(mutant(kind) - o[0, :, 0]).max() > 1e-3, kind
    np.testing.assert_allclose(mutant("correct"), o[0, :, 0], rtol=1e-12, atol=1e-12)


# --- the KDA reverse mode (kda_vjp) ---


def _kda_loss(q, k, v, beta, g, s0, go, gs):
    o, s = gref.kda_delta_rule(q, k, v, beta, g, s0)
    return float(np.sum(o * go) + np.sum(s * gs))


def test_kda_vjp_channel_constant_gate_is_the_gated_vjp():
    """g constant along D: gq, gk, gv, gbeta and gstate0 are gated_vjp's, and gg summed
    over the channels is gated_vjp's gg."""
    rng = np.random.default_rng(31)
    q, k, v, beta, g, s0 = _problem(rng, (2, 8, 2, 5))
    go = rng.standard_normal(q.shape)
    gs = rng.standard_normal(s0.shape) * 0.1
    got = gref.kda_vjp(q, k, v, beta, np.repeat(g[..., None], 5, axis=-1), go, gs, s0)
    want = gref.gated_vjp(q, k, v, beta, g, go, gs, s0)
    for name, a, b in zip(("gq", "gk", "gv", "gbeta", "gs0"), got[:4] + got[5:], want[:4] + want[5:]):
        np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12, err_msg=name)
    np.testing.assert_allclose(got[4].sum(axis=-1), want[4], rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("gate_scale", [0.05, 0.5, 2.0])
def test_kda_vjp_finite_differences(gate_scale):
    rng = np.random.default_rng(40 + int(gate_scale * 10))
    q, k, v, beta, g, s0 = _kda_problem(rng, (1, 6, 2, 4), gate_scale)
    go = rng.standard_normal(q.shape)
    gs = rng.standard_normal(s0.shape)
    grads = gref.kda_vjp(q, k, v, beta, g, go, gs, s0)
    args = {"q": q, "k": k, "v": v, "beta": beta, "g": g, "s0": s0}
    eps = 1e-6
    for name, gx in zip(("q", "k", "v", "beta", "g", "s0"), grads):
        d = rng.standard_normal(args[name].shape)
        plus, minus = dict(args), dict(args)
        plus[name], minus[name] = args[name] + eps * d, args[name] - eps * d
        fd = (_kda_loss(**plus, go=go, gs=gs) - _kda_loss(**minus, go=go, gs=gs)) / (2 * eps)
        np.testing.assert_allclose(np.sum(gx * d), fd, rtol=1e-6, atol=1e-8, err_msg=name)


def test_kda_vjp_pure_decay_closed_form():
    """beta = 0, go = 0: S_T = Diag(exp(sum_t g_t)) S_0, so dL/dg_t[d] = <gs[d, :], S_T[d, :]>
    for every t and dL/dS_0 = Diag(exp(sum_t g_t)) gs."""
    rng = np.random.default_rng(32)
    q, k, v, _, g, s0 = _kda_problem(rng, (1, 5, 2, 3))
    gs = rng.standard_normal(s0.shape)
    _, _, _, _, gg, gs0 = gref.kda_vjp(q, k, v, np.zeros(g.shape[:3]), g, None, gs, s0)
    dec = np.exp(g.sum(axis=1))[..., None]  # (B, H, D, 1)
    want = np.einsum("bhde,bhde->bhd", gs, dec * s0)
    np.testing.assert_allclose(gg, np.repeat(want[:, None], g.shape[1], axis=1), rtol=1e-12)
    np.testing.assert_allclose(gs0, dec * gs, rtol=1e-12)


def test_kda_vjp_planted_mistakes_are_caught():
    """The channel gradient summed over the wrong axis (columns instead of rows), G
    scaled along its columns, and the gate's gradient taken before the downdate each
    differ from finite differences."""
    rng = np.random.default_rng(33)
    q, k, v, beta, g, s0 = _kda_problem(rng, (1, 5, 1, 4), 0.5)
    go = rng.standard_normal(q.shape)
    gs = rng.standard_normal(s0.shape)
    eps = 1e-6
    d = rng.standard_normal(g.shape)
    fd = (_kda_loss(q, k, v, beta, g + eps * d, s0, go, gs)
          - _kda_loss(q, k, v, beta, g - eps * d, s0, go, gs)) / (2 * eps)

    def mutant(kind):
        t = q.shape[1]
        G, s = gs.copy(), s0.copy()
        hist, us = [s], []
        for i in range(t):
            p = np.exp(g[:, i])[..., None] * s
            u = v[:, i] - np.einsum("bhd,bhde->bhe", k[:, i], p)
            s = p + beta[:, i][..., None, None] * np.einsum("bhd,bhe->bhde", k[:, i], u)
            hist.append(s)
            us.append(u)
        gg = np.zeros(g.shape)
        for i in range(t - 1, -1, -1):
            a = np.exp(g[:, i])
            p = a[..., None] * hist[i]
            G = G + np.einsum("bhd,bhe->bhde", q[:, i], go[:, i])
            w = np.einsum("bhde,bhd->bhe", G, k[:, i])
            if kind == "before_downdate":
                gg[:, i] = np.einsum("bhde,bhde->bhd", G, p)
            G = G - beta[:, i][..., None, None] * np.einsum("bhd,bhe->bhde", k[:, i], w)
            if kind == "column_sums":
                gg[:, i] = np.einsum("bhde,bhde->bhe", G, p)
            elif kind != "before_downdate":
                gg[:, i] = np.einsum("bhde,bhde->bhd", G, p)
            G = a[..., None, :] * G if kind == "scaled_columns" else a[..., None] * G
        return float(np.sum(gg * d))

    for kind in ("column_sums", "scaled_columns", "before_downdate"):
        assert abs(mutant(kind) - fd) > 1e-4 * max(1.0, abs(fd)), kind
    assert abs(mutant("correct") - fd) < 1e-6 * max(1.0, abs(fd))
