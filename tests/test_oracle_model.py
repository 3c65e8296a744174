"""CPU tests that pin the linear-attention oracle (oracle/model_oracle.py)
before it checks the GPU path, and the host-side validation of
prometheus_amd.model (which fails before any GPU work).

The oracle restates model.linear_attention (model/__init__.py:393-432,
tests/reference/model.py:254-292). What pins it: equality with the
delta-rule oracle (itself pinned to the reference's goldens) on normalised
q, k with beta = 1; the one-token closed form; invariance of the output
under positive rescaling of q and k (the normalisation); the eps guard on a
zero vector; the reference's causality, state-carry and 3-D tests
(tests/test_model.py:353-406) run on the restatement; and planted mistakes
that these checks catch.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import delta_oracle as dref
from oracle import model_oracle as mref
from prometheus_amd import model

TOL = dict(rtol=1e-5, atol=1e-5)  # tests/test_model.py:43


def _rand(rng, shape):
    return rng.standard_normal(shape).astype(np.float32)


def test_equals_delta_rule_with_unit_beta_on_normalised_inputs():
    rng = np.random.default_rng(1)
    for shape in [(2, 5, 3, 8), (1, 17, 2, 4), (1, 3, 1, 16)]:
        q, k, v = (_rand(rng, shape) for _ in range(3))
        s0 = _rand(rng, (shape[0], shape[2], shape[3], shape[3])) * 0.1
        out, s = mref.linear_attention(q, k, v, s0, dtype=np.float64)
        qn, kn = mref.l2_normalize(q, dtype=np.float64), mref.l2_normalize(k, dtype=np.float64)
        o2, s2 = dref.gated_delta_rule(qn, kn, v, np.ones(shape[:3]), s0, dtype=np.float64)
        np.testing.assert_allclose(out, o2, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(s, s2, rtol=1e-12, atol=1e-12)


def test_one_token_closed_form():
    """S_1 = (I - k^ k^^T) S_0 + k^ v^T and o = q^ S_1 with unit vectors q^, k^."""
    rng = np.random.default_rng(2)
    d = 6
    q, k, v = (rng.standard_normal((1, 1, 1, d)) for _ in range(3))
    s0 = rng.standard_normal((1, 1, d, d))
    out, s = mref.linear_attention(q, k, v, s0, dtype=np.float64)
    kh = k[0, 0, 0] / np.linalg.norm(k[0, 0, 0])
    qh = q[0, 0, 0] / np.linalg.norm(q[0, 0, 0])
    s1 = s0[0, 0] - np.outer(kh, kh @ s0[0, 0]) + np.outer(kh, v[0, 0, 0])
    np.testing.assert_allclose(s[0, 0], s1, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(out[0, 0, 0], qh @ s1, rtol=1e-12, atol=1e-12)


def test_rescaling_q_and_k_changes_nothing():
    rng = np.random.default_rng(3)
    q, k, v = (_rand(rng, (2, 7, 2, 8)) for _ in range(3))
    a = mref.linear_attention(q, k, v, dtype=np.float64)
    scale = rng.uniform(0.1, 10.0, size=(2, 7, 2, 1))
    b = mref.linear_attention(q * scale, k * scale[:, ::-1], v, dtype=np.float64)
    for x, y in zip(a, b):
        np.testing.assert_allclose(x, y, rtol=1e-10, atol=1e-12)


def test_zero_vectors_use_the_eps_guard():
    """x / max(||x||, 1e-6): a zero q gives a zero output row, a zero k leaves S unchanged."""
    rng = np.random.default_rng(4)
    q, k, v = (_rand(rng, (1, 4, 1, 4)) for _ in range(3))
    q[0, 1] = 0.0
    k[0, 2] = 0.0
    out, _ = mref.linear_attention(q, k, v, dtype=np.float64)
    assert np.all(out[0, 1] == 0.0)
    _, s_before = mref.linear_attention(q[:, :2], k[:, :2], v[:, :2], dtype=np.float64)
    _, s_after = mref.linear_attention(q[:, 2:3], k[:, 2:3], v[:, 2:3], s_before, dtype=np.float64)
    np.testing.assert_array_equal(s_after, s_before)
    # a tiny k is scaled up to unit length only down to the eps floor
    tiny = np.zeros((1, 1, 1, 4))
    tiny[..., 0] = 1e-8
    np.testing.assert_allclose(mref.l2_normalize(tiny, dtype=np.float64)[..., 0], 1e-2)


def test_reference_tests_on_the_restatement():
    """tests/test_model.py:367-406 (seeds 8, 9, 10) run on the oracle itself."""
    rng = np.random.default_rng(8)
    q, k, v = (_rand(rng, (1, 6, 2, 4)) for _ in range(3))
    out, _ = mref.linear_attention(q, k, v)
    q2, k2, v2 = q.copy(), k.copy(), v.copy()
    for x in (q2, k2, v2):
        x[:, -1] += 1.5
    out2, _ = mref.linear_attention(q2, k2, v2)
    np.testing.assert_allclose(out[:, :-1], out2[:, :-1], **TOL)
    rng = np.random.default_rng(9)
    q, k, v = (_rand(rng, (2, 6, 2, 4)) for _ in range(3))
    full, st_full = mref.linear_attention(q, k, v)
    a, st = mref.linear_attention(q[:, :2], k[:, :2], v[:, :2])
    b, st2 = mref.linear_attention(q[:, 2:], k[:, 2:], v[:, 2:], state=st)
    np.testing.assert_allclose(np.concatenate([a, b], axis=1), full, **TOL)
    np.testing.assert_allclose(st2, st_full, **TOL)
    rng = np.random.default_rng(10)
    q, k, v = (_rand(rng, (2, 4, 8)) for _ in range(3))
    out, st = mref.linear_attention(q, k, v)
    assert out.shape == q.shape and st.shape == (2, 8, 8)
    o4, s4 = mref.linear_attention(q[:, :, None], k[:, :, None], v[:, :, None])
    np.testing.assert_array_equal(out, o4[:, :, 0])
    np.testing.assert_array_equal(st, s4[:, 0])


def test_layer_projections():
    rng = np.random.default_rng(5)
    b, s, d, h, e = 2, 5, 12, 3, 4
    x = _rand(rng, (b, s, d))
    layer = {"W_q": _rand(rng, (d, h, e)), "W_k": _rand(rng, (d, h, e)),
             "W_v": _rand(rng, (d, h, e)), "W_o": _rand(rng, (h, e, d))}
    y, st = mref.linear_attn_layer(x, layer, dtype=np.float64)
    q = (x.astype(np.float64).reshape(b * s, d) @ layer["W_q"].reshape(d, h * e)).reshape(b, s, h, e)
    k = (x.astype(np.float64).reshape(b * s, d) @ layer["W_k"].reshape(d, h * e)).reshape(b, s, h, e)
    v = (x.astype(np.float64).reshape(b * s, d) @ layer["W_v"].reshape(d, h * e)).reshape(b, s, h, e)
    o, st2 = mref.linear_attention(q, k, v, dtype=np.float64)
    y2 = o.reshape(b * s, h * e) @ layer["W_o"].astype(np.float64).reshape(h * e, d)
    np.testing.assert_allclose(y, y2.reshape(b, s, d), rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(st, st2, rtol=1e-12)


def _planted(kind):
    def la(q, k, v, state=None, dtype=np.float64):
        if kind == "k_not_normalised":
            qn = mref.l2_normalize(q, dtype=dtype)
            o, s = dref.gated_delta_rule(qn, k, v, np.ones(np.shape(q)[:3]), state, dtype=dtype)
            return o, s
        if kind == "eps_added":
            def nrm(x):
                x = np.asarray(x, dtype=dtype)
                return x / (np.linalg.norm(x, axis=-1, keepdims=True) + 1e-2)
            return dref.gated_delta_rule(nrm(q), nrm(k), v, np.ones(np.shape(q)[:3]), state, dtype=dtype)
        if kind == "decay_plus":
            qn, kn = mref.l2_normalize(q, dtype=dtype), mref.l2_normalize(k, dtype=dtype)
            b, t, h, d = np.shape(q)
            s = np.zeros((b, h, d, d)) if state is None else np.array(state, dtype=dtype)
            out = np.zeros((b, t, h, d))
            for i in range(t):
                kk = np.einsum("bhd,bhe->bhde", kn[:, i], kn[:, i])
                s = np.einsum("bhij,bhjk->bhik", np.eye(d) + kk, s) + np.einsum("bhd,bhe->bhde", kn[:, i], v[:, i])
                out[:, i] = np.einsum("bhd,bhde->bhe", qn[:, i], s)
            return out, s
        raise AssertionError(kind)
    return la


@pytest.mark.parametrize("kind", ["k_not_normalised", "eps_added", "decay_plus"])
def test_planted_mistakes_are_caught(kind):
    """Each plausible slip fails the closed form or the rescaling check."""
    wrong = _planted(kind)
    rng = np.random.default_rng(6)
    q, k, v = (rng.standard_normal((1, 3, 1, 4)) for _ in range(3))
    s0 = rng.standard_normal((1, 1, 4, 4))
    caught = False
    try:
        out, s = wrong(q[:, :1], k[:, :1], v[:, :1], s0)
        kh = k[0, 0, 0] / np.linalg.norm(k[0, 0, 0])
        qh = q[0, 0, 0] / np.linalg.norm(q[0, 0, 0])
        s1 = s0[0, 0] - np.outer(kh, kh @ s0[0, 0]) + np.outer(kh, v[0, 0, 0])
        np.testing.assert_allclose(out[0, 0, 0], qh @ s1, rtol=1e-9)
        a = wrong(q, k, v)
        b = wrong(q * 3.0, k * 0.2, v)
        np.testing.assert_allclose(a[0], b[0], rtol=1e-9)
    except AssertionError:
        caught = True
    assert caught, kind


def test_model_host_validation_without_gpu():
    """Shape errors are ValueErrors raised before any GPU work (model/__init__.py:397-411)."""
    z3 = np.zeros((2, 4, 8), np.float32)
    z4 = np.zeros((2, 4, 3, 8), np.float32)
    with pytest.raises(ValueError):
        model.linear_attention(np.zeros((2, 8), np.float32), z3, z3)
    with pytest.raises(ValueError):
        model.linear_attention(z4, z4[:, :3], z4)
    with pytest.raises(ValueError):
        model.linear_attention(z4, z4, z4[..., :4])
    with pytest.raises(ValueError):
        model.linear_attention(z4, z4, z4, state=np.zeros((2, 3, 8, 4), np.float32))
    with pytest.raises(ValueError):
        model.linear_attention(z3, z3, z3, state=np.zeros((2, 2, 8, 8), np.float32))
    layer = {"W_q": np.zeros((6, 2, 4)), "W_k": np.zeros((6, 2, 4)), "W_v": np.zeros((6, 2, 4)),
             "W_o": np.zeros((2, 4, 5))}
    with pytest.raises(ValueError):
        model._linear_attn(np.zeros((1, 3, 6), np.float32), layer)
