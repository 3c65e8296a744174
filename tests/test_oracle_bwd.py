"""CPU tests that pin the backward oracle (oracle/delta_oracle.py: delta_vjp,
delta_vjp_downdate) before it is trusted as the checker of the GPU backward.

The gradients are fixed by the forward, which is pinned on its own: central
differences of L = <go, O> + <gs, S_T> in fp64 along random directions, the
reference's own finite-difference test (tests/test_kernels.py:409-432, seed
18), closed forms for one token, agreement of the two independent
formulations (state history vs checkpoints with exact downdating), and
planted mistakes that the checks must catch.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import delta_oracle as ref
from prometheus_amd import synth
from tests.golden.make_golden import reference_cases


def _loss(q, k, v, beta, s0, go, gs):
    o, s = ref.gated_delta_rule(q, k, v, beta, s0, dtype=np.float64)
    return float(np.sum(go * o) + np.sum(gs * s))


def _random_problem(rng, shape, with_state=True):
    b, t, h, d = shape
    q = rng.standard_normal(shape)
    k = rng.standard_normal(shape)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal(shape)
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((b, t, h))))
    s0 = rng.standard_normal((b, h, d, d)) * 0.1 if with_state else None
    go = rng.standard_normal(shape)
    gs = rng.standard_normal((b, h, d, d)) * 0.1
    return q, k, v, beta, s0, go, gs


def _fd_check(vjp, q, k, v, beta, s0, go, gs, rng, eps=1e-6, rtol=1e-7):
    grads = vjp(q, k, v, beta, go, gs, s0)
    args = {"q": q, "k": k, "v": v, "beta": beta, "s0": s0}
    for i, name in enumerate(["q", "k", "v", "beta", "s0"]):
        x = args[name]
        if x is None:
            continue
        d = rng.standard_normal(x.shape)
        plus, minus = dict(args), dict(args)
        plus[name], minus[name] = x + eps * d, x - eps * d
        fd = (_loss(**plus, go=go, gs=gs) - _loss(**minus, go=go, gs=gs)) / (2 * eps)
        an = float(np.sum(grads[i] * d))
        assert abs(fd - an) <= rtol * max(1.0, abs(an)) + 1e-9, (name, fd, an)


VJPS = {
    "history": lambda q, k, v, b, go, gs, s0: ref.delta_vjp(q, k, v, b, go, gs, s0),
    "downdate": lambda q, k, v, b, go, gs, s0: ref.delta_vjp_downdate(q, k, v, b, go, gs, s0, ckpt=4),
}


@pytest.mark.parametrize("form", sorted(VJPS))
@pytest.mark.parametrize("shape", [(1, 1, 1, 3), (2, 5, 2, 3), (1, 9, 2, 4)])
def test_finite_differences_fp64(form, shape):
    rng = np.random.default_rng(hash((form, shape)) % 2**32)
    q, k, v, beta, s0, go, gs = _random_problem(rng, shape)
    _fd_check(VJPS[form], q, k, v, beta, s0, go, gs, rng)


@pytest.mark.parametrize("form", sorted(VJPS))
def test_reference_fd_case_seed18(form):
    """tests/test_kernels.py:409-432: seed 18, (1, 3, 2, 3), go = ones, gs = zeros,
    unit directions drawn after the inputs; tolerance 1e-3 there."""
    rng = np.random.default_rng(18)
    q, k, v, beta = synth.reference_test_inputs(rng, batch=1, seq=3, heads=2, dim=3)
    go = np.ones((1, 3, 2, 3), dtype=np.float32)
    gs = np.zeros((1, 2, 3, 3), dtype=np.float32)
    gq, gk, gv, gbeta, _ = VJPS[form](q, k, v, beta, go, gs, None)
    eps = 1e-3

    def prod_sum(qq, kk, vv, bb):
        o, _ = ref.gated_delta_rule(qq, kk, vv, bb, None, dtype=np.float64)
        return float(np.sum(o))

    for name, x, gx in (("q", q, gq), ("k", k, gk), ("v", v, gv), ("beta", beta, gbeta)):
        d = rng.standard_normal(x.shape).astype(np.float32)
        d /= np.linalg.norm(d) + 1e-12
        xs = {"q": q, "k": k, "v": v, "beta": beta}
        plus, minus = dict(xs), dict(xs)
        plus[name], minus[name] = x + eps * d, x - eps * d
        fd = (prod_sum(plus["q"], plus["k"], plus["v"], plus["beta"])
              - prod_sum(minus["q"], minus["k"], minus["v"], minus["beta"])) / (2 * eps)
        np.testing.assert_allclose(fd, float(np.sum(gx * d)), rtol=1e-3, atol=1e-3, err_msg=name)


def test_single_token_closed_forms():
    """T = 1, gs = 0: with u = v - S_0^T k, S_1 = S_0 + b k u^T and
    o = S_1^T q = S_0^T q + b (k.q) u, so gq = S_1 go, gv = b (k.q) go,
    gk = b (u.go) q - b (k.q) S_0 go, gbeta = (k.q)(u.go) and
    gS_0 = (I - b k k^T) q go^T."""
    rng = np.random.default_rng(5)
    d = 4
    q, k, v, go = (rng.standard_normal((1, 1, 1, d)) for _ in range(4))
    b = np.array([[[0.7]]])
    s0 = rng.standard_normal((1, 1, d, d))
    gq, gk, gv, gbeta, gs0 = ref.delta_vjp(q, k, v, b, go, None, s0)
    qv, kv, vv, gov, S0 = q[0, 0, 0], k[0, 0, 0], v[0, 0, 0], go[0, 0, 0], s0[0, 0]
    bb = 0.7
    u = vv - S0.T @ kv
    S1 = S0 + bb * np.outer(kv, u)
    np.testing.assert_allclose(gq[0, 0, 0], S1 @ gov, rtol=1e-12)
    np.testing.assert_allclose(gv[0, 0, 0], bb * (kv @ qv) * gov, rtol=1e-12)
    # o = S0^T q + b (k.q) u: d/dk = b (u.go) q + b (k.q) d(u.go)/dk, u = v - S0^T k
    np.testing.assert_allclose(gk[0, 0, 0], bb * (u @ gov) * qv - bb * (kv @ qv) * (S0 @ gov),
                               rtol=1e-12)
    np.testing.assert_allclose(gbeta[0, 0, 0], (kv @ qv) * (u @ gov), rtol=1e-12)
    np.testing.assert_allclose(gs0[0, 0], (np.eye(d) - bb * np.outer(kv, kv)) @ np.outer(qv, gov),
                               rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("ckpt", [1, 3, 64])
def test_formulations_agree(ckpt):
    rng = np.random.default_rng(7)
    for shape in [(2, 7, 2, 5), (1, 70, 1, 8)]:
        q, k, v, beta, s0, go, gs = _random_problem(rng, shape)
        a = ref.delta_vjp(q, k, v, beta, go, gs, s0)
        b = ref.delta_vjp_downdate(q, k, v, beta, go, gs, s0, ckpt=ckpt)
        for x, y in zip(a, b):
            np.testing.assert_allclose(y, x, rtol=1e-10, atol=1e-12)


def test_reference_cases_run_and_agree():
    rng = np.random.default_rng(105)
    for name, q, k, v, b, s0, chunk in reference_cases():
        go = rng.standard_normal(q.shape)
        gs = rng.standard_normal((q.shape[0], q.shape[2], q.shape[3], q.shape[3])) * 0.05
        a = ref.delta_vjp(q, k, v, b, go, gs, s0)
        c = ref.delta_vjp_downdate(q, k, v, b, go, gs, s0, ckpt=chunk)
        for x, y in zip(a, c):
            np.testing.assert_allclose(y, x, rtol=1e-10, atol=1e-12, err_msg=name)


def _planted(kind):
    """A copy of delta_vjp with one plausible mistake (test-only)."""

    def vjp(q, k, v, beta, go, gs, s0):
        gq, gk, gv, gb, g0 = ref.delta_vjp(q, k, v, beta, go, gs, s0)
        if kind == "gk_drops_transpose_term":
            # recompute gk without the g_A^T k term
            b, t, h, d = q.shape
            s = np.zeros((b, h, d, d)) if s0 is None else s0.copy()
            hist = [s]
            for i in range(t):
                u = v[:, i] - np.einsum("bhd,bhde->bhe", k[:, i], s)
                s = s + beta[:, i, :, None, None] * np.einsum("bhd,bhe->bhde", k[:, i], u)
                hist.append(s)
            g_s = gs.copy()
            gk2 = np.zeros_like(gk)
            for i in range(t - 1, -1, -1):
                g_s = g_s + np.einsum("bhd,bhe->bhde", q[:, i], go[:, i])
                g_a = np.einsum("bhik,bhjk->bhij", g_s, hist[i])
                bt = beta[:, i]
                gk2[:, i] = bt[..., None] * (np.einsum("bhde,bhe->bhd", g_s, v[:, i])
                                             - np.einsum("bhde,bhe->bhd", g_a, k[:, i]))
                w = np.einsum("bhde,bhd->bhe", g_s, k[:, i])
                g_s = g_s - bt[..., None, None] * np.einsum("bhd,bhe->bhde", k[:, i], w)
            return gq, gk2, gv, gb, g0
        if kind == "gbeta_sign":
            return gq, gk, gv, -gb, g0
        if kind == "gs0_untransposed":
            return gq, gk, gv, gb, np.swapaxes(g0, -1, -2)
        raise AssertionError(kind)

    return vjp


@pytest.mark.parametrize("kind", ["gk_drops_transpose_term", "gbeta_sign", "gs0_untransposed"])
def test_planted_mistakes_are_caught(kind):
    rng = np.random.default_rng(11)
    q, k, v, beta, s0, go, gs = _random_problem(rng, (1, 6, 1, 4))
    with pytest.raises(AssertionError):
        _fd_check(_planted(kind), q, k, v, beta, s0, go, gs, rng)
