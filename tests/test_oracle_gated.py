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
