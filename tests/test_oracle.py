"""CPU tests that pin the oracle (oracle/) before it is trusted as the checker.

Each formulation is checked against what the reference itself fixes (its
closed-form goldens, tests/test_kernels.py:279-316, and invariants,
:319-406), against the other, independent formulations (explicit
(I - beta k k^T) matrix, rank-1 step, WY/UT chunk form), against special
cases the mathematics fixes, and against planted mistakes that a weak check
would let through.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import delta_oracle as ref
from prometheus_amd import synth
from tests.golden.make_golden import expected, reference_cases, sha
from tests.parity import assert_f32_parity

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TOL = dict(rtol=1e-5, atol=1e-5)

FORMS = {
    "explicit": lambda q, k, v, b, s=None, chunk=64, dtype=np.float32:
        ref.gated_delta_rule(q, k, v, b, s, dtype=dtype),
    "rank1": lambda q, k, v, b, s=None, chunk=64, dtype=np.float32:
        ref.chunked_fwd_rank1(q, k, v, b, s, chunk=chunk, dtype=dtype),
    "wy": lambda q, k, v, b, s=None, chunk=64, dtype=np.float64:
        ref.wy_chunked_fwd(q, k, v, b, s, chunk=chunk, dtype=dtype),
}

# --- the reference's three closed-form goldens (tests/test_kernels.py:279-316) ---

G_Q = np.array([[[[1.0, 0.0]], [[0.0, 1.0]]]], dtype=np.float32)
G_K = np.array([[[[1.0, 0.0]], [[0.0, 1.0]]]], dtype=np.float32)
G_V = np.array([[[[1.0, 2.0]], [[3.0, 4.0]]]], dtype=np.float32)
G_B = np.array([[[1.0], [1.0]]], dtype=np.float32)


@pytest.mark.parametrize("form", sorted(FORMS))
@pytest.mark.parametrize("chunk", [1, 2, 64])
def test_golden_orthogonal_keys(form, chunk):
    out, st = FORMS[form](G_Q, G_K, G_V, G_B, None, chunk)
    np.testing.assert_allclose(out, G_V, **TOL)
    np.testing.assert_allclose(st, np.array([[[[1.0, 2.0], [3.0, 4.0]]]]), **TOL)


@pytest.mark.parametrize("form", sorted(FORMS))
def test_golden_beta_half(form):
    q = np.array([[[[1.0, 0.0]]]], dtype=np.float32)
    v = np.array([[[[2.0, 4.0]]]], dtype=np.float32)
    b = np.array([[[0.5]]], dtype=np.float32)
    out, st = FORMS[form](q, q, v, b)
    np.testing.assert_allclose(out, np.array([[[[1.0, 2.0]]]]), **TOL)
    np.testing.assert_allclose(st, np.array([[[[1.0, 2.0], [0.0, 0.0]]]]), **TOL)


@pytest.mark.parametrize("form", sorted(FORMS))
def test_golden_nonzero_initial_state(form):
    s0 = np.eye(2, dtype=np.float32)[None, None]
    q = np.array([[[[1.0, 0.0]]]], dtype=np.float32)
    k = np.array([[[[0.0, 1.0]]]], dtype=np.float32)
    v = np.zeros((1, 1, 1, 2), dtype=np.float32)
    b = np.array([[[1.0]]], dtype=np.float32)
    out, st = FORMS[form](q, k, v, b, s0)
    np.testing.assert_allclose(out, np.array([[[[1.0, 0.0]]]]), **TOL)
    np.testing.assert_allclose(st, np.array([[[[1.0, 0.0], [0.0, 0.0]]]]), **TOL)


# --- independent formulations agree (fp64) ---


@pytest.mark.parametrize("case", reference_cases(), ids=lambda c: c[0])
def test_formulations_agree_reference_cases(case):
    _, q, k, v, b, s0, chunk = case
    o1, s1 = ref.gated_delta_rule(q, k, v, b, s0, dtype=np.float64)
    for form in ("rank1", "wy"):
        o2, s2 = FORMS[form](q, k, v, b, s0, chunk, np.float64)
        np.testing.assert_allclose(o2, o1, rtol=1e-10, atol=1e-10)
        np.testing.assert_allclose(s2, s1, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("chunk", [1, 3, 7, 16, 64])
def test_formulations_agree_normalised_inputs(chunk):
    x = synth.fwd_inputs((2, 150, 3, 16), seed=3, dtype="fp32", s0_std=0.1)
    o1, s1 = ref.gated_delta_rule(x.q, x.k, x.v, x.beta, x.s0, dtype=np.float64)
    for form in ("rank1", "wy"):
        o2, s2 = FORMS[form](x.q, x.k, x.v, x.beta, x.s0, chunk, np.float64)
        np.testing.assert_allclose(o2, o1, rtol=1e-11, atol=1e-11)
        np.testing.assert_allclose(s2, s1, rtol=1e-11, atol=1e-11)


# --- special cases the mathematics fixes ---


@pytest.mark.parametrize("form", sorted(FORMS))
def test_single_token_from_zero_state(form):
    rng = np.random.default_rng(5)
    q, k, v = (rng.standard_normal((2, 1, 3, 6)).astype(np.float32) for _ in range(3))
    b = rng.random((2, 1, 3)).astype(np.float32)
    out, st = FORMS[form](q, k, v, b)
    exp_s = b[:, 0, :, None, None] * np.einsum("bhd,bhe->bhde", k[:, 0], v[:, 0])
    exp_o = (b[:, 0, :, None] * np.einsum("bhd,bhd->bh", q[:, 0], k[:, 0])[..., None]) * v[:, 0]
    np.testing.assert_allclose(st, exp_s, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out[:, 0], exp_o, rtol=1e-5, atol=1e-6)


def test_orthonormal_key_permutation_overwrites_rows():
    # beta=1 and k_t = e_{pi(t)}: S row pi(t) becomes v_t, so o_t = v_t for q_t = k_t
    d = 5
    perm = [3, 0, 4, 1, 2]
    k = np.eye(d, dtype=np.float32)[perm][None, :, None, :]
    rng = np.random.default_rng(6)
    v = rng.standard_normal((1, d, 1, d)).astype(np.float32)
    s0 = rng.standard_normal((1, 1, d, d)).astype(np.float32)
    b = np.ones((1, d, 1), dtype=np.float32)
    for form in sorted(FORMS):
        out, st = FORMS[form](k, k, v, b, s0, 2)
        np.testing.assert_allclose(out, v, **TOL)
        np.testing.assert_allclose(st[0, 0][perm], v[0, :, 0], **TOL)


def test_step_matches_one_token_forward():
    rng = np.random.default_rng(7)
    q, k, v = (rng.standard_normal((3, 2, 5)) for _ in range(3))
    b = rng.random((3, 2))
    s = rng.standard_normal((3, 2, 5, 5))
    s_new, o = ref.delta_step(s, q, k, v, b)
    o2, s2 = ref.gated_delta_rule(q[:, None], k[:, None], v[:, None], b[:, None], s,
                                  dtype=np.float64)
    np.testing.assert_allclose(o, o2[:, 0], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(s_new, s2, rtol=1e-12, atol=1e-12)


# --- the reference's invariants (tests/test_kernels.py:319-406) on the oracle ---


def test_invariants():
    rng = np.random.default_rng(11)
    q, k, v, b = synth.reference_test_inputs(rng, seq=6)
    out, _ = ref.gated_delta_rule(q, k, v, b)
    q2, k2, v2, b2 = q.copy(), k.copy(), v.copy(), b.copy()
    q2[:, 3:] += 3.0
    k2[:, 3:] -= 1.5
    v2[:, 3:] += 4.0
    b2[:, 3:] = 0.9
    out2, _ = ref.gated_delta_rule(q2, k2, v2, b2)
    np.testing.assert_allclose(out[:, :3], out2[:, :3], **TOL)  # causality

    rng = np.random.default_rng(12)
    q, k, v, b = synth.reference_test_inputs(rng, seq=7)
    oa, sa = ref.gated_delta_rule(q[:, :3], k[:, :3], v[:, :3], b[:, :3])
    ob, sb = ref.gated_delta_rule(q[:, 3:], k[:, 3:], v[:, 3:], b[:, 3:], sa)
    of, sf = ref.gated_delta_rule(q, k, v, b)
    np.testing.assert_allclose(np.concatenate([oa, ob], 1), of, **TOL)  # state carry
    np.testing.assert_allclose(sb, sf, **TOL)

    rng = np.random.default_rng(17)
    q, k, v, b = synth.reference_test_inputs(rng, batch=1, seq=4, heads=1, dim=3)
    o1, s1 = ref.gated_delta_rule(q, k, v, b)
    o2, s2 = ref.gated_delta_rule(q, k, 2.0 * v, b)
    np.testing.assert_allclose(o2, 2.0 * o1, **TOL)  # linear in v
    np.testing.assert_allclose(s2, 2.0 * s1, **TOL)
    _, sq = ref.gated_delta_rule(q + 1.25, k, v, b)
    np.testing.assert_allclose(sq, s1, **TOL)  # S independent of q
    zeros = np.zeros((1, 1, 3, 3), dtype=np.float32)
    oz, sz = ref.gated_delta_rule(q, k, v, b, zeros)
    np.testing.assert_allclose(oz, o1, **TOL)  # None == zeros
    np.testing.assert_allclose(sz, s1, **TOL)


def test_empty_sequence_passes_state_through():
    q = np.zeros((2, 0, 3, 4), dtype=np.float32)
    b = np.zeros((2, 0, 3), dtype=np.float32)
    s0 = np.arange(2 * 3 * 16, dtype=np.float32).reshape(2, 3, 4, 4)
    for form in sorted(FORMS):
        out, st = FORMS[form](q, q, q, b, s0)
        assert out.shape == (2, 0, 3, 4)
        np.testing.assert_array_equal(st, s0)


def test_varlen_is_per_segment():
    x = synth.fwd_inputs((40, 2, 8), seed=9, dtype="fp32")
    cu = np.array([0, 7, 7, 30, 40])
    o, s = ref.varlen_fwd(x.q, x.k, x.v, x.beta, cu)
    for i in range(4):
        a, z = cu[i], cu[i + 1]
        oi, si = ref.gated_delta_rule(x.q[None, a:z], x.k[None, a:z], x.v[None, a:z],
                                      x.beta[None, a:z])
        np.testing.assert_array_equal(o[a:z], oi[0])
        np.testing.assert_array_equal(s[i], si[0])
    np.testing.assert_array_equal(s[1], 0.0)  # empty segment keeps the zero state


# --- planted mistakes must be caught by the checks above ---


def _mutant(kind):
    def f(q, k, v, b, s=None):
        q, k, v, b = (np.asarray(x, np.float64) for x in (q, k, v, b))
        bb, t, h, d = q.shape
        st = np.zeros((bb, h, d, d)) if s is None else np.array(s, np.float64)
        out = np.zeros((bb, t, h, d))
        for i in range(t):
            kt, vt, qt, bt = k[:, i], v[:, i], q[:, i], b[:, i, :, None, None]
            sign = -1.0 if kind == "sign" else 1.0
            decay = np.eye(d) - sign * bt * np.einsum("bhd,bhe->bhde", kt, kt)
            prev = st
            st = np.einsum("bhij,bhjk->bhik", decay, st) + bt * np.einsum("bhd,bhe->bhde", kt, vt)
            if kind == "transpose":
                out[:, i] = np.einsum("bhd,bhed->bhe", qt, st)
            elif kind == "stale_state":
                out[:, i] = np.einsum("bhd,bhde->bhe", qt, prev)
            else:
                out[:, i] = np.einsum("bhd,bhde->bhe", qt, st)
        return out, st
    return f


@pytest.mark.parametrize("kind", ["sign", "transpose", "stale_state"])
def test_planted_mistakes_are_caught(kind):
    bad = _mutant(kind)
    assert _mutant("none")(G_Q, G_K, G_V, G_B)[0] == pytest.approx(G_V)
    caught = False
    try:
        out, st = bad(G_Q, G_K, G_V, G_B)
        np.testing.assert_allclose(out, G_V, **TOL)
        q = np.array([[[[1.0, 0.0]]]], dtype=np.float32)
        v = np.array([[[[2.0, 4.0]]]], dtype=np.float32)
        out, st = bad(q, q, v, np.array([[[0.5]]], dtype=np.float32))
        np.testing.assert_allclose(out, np.array([[[[1.0, 2.0]]]]), **TOL)
        case = reference_cases()[0]
        o1, _ = ref.gated_delta_rule(*case[1:6], dtype=np.float64)
        o2, _ = bad(*case[1:6])
        np.testing.assert_allclose(o2, o1, rtol=1e-6, atol=1e-6)
    except AssertionError:
        caught = True
    assert caught, f"planted mistake {kind!r} was not caught"


# --- committed fixtures (regression against the pinned oracle) ---


def test_reference_case_fixtures():
    data = np.load(os.path.join(GOLDEN, "reference_cases.npz"))
    for name, q, k, v, b, s0, chunk in reference_cases():
        assert str(data[f"{name}/sha"]) == sha(q, k, v, b, s0), f"{name}: input generator drifted"
        o, s = expected(q, k, v, b, s0, chunk)
        np.testing.assert_allclose(o, data[f"{name}/o"], rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(s, data[f"{name}/s"], rtol=1e-6, atol=1e-6)
        o32, s32 = ref.gated_delta_rule(q, k, v, b, s0)
        assert_f32_parity(o32, data[f"{name}/o"], name, scaled=True)
        assert_f32_parity(s32, data[f"{name}/s"], name, scaled=True)


def test_cfg0_fixture():
    c = synth.CONFIGS[0]
    x = synth.fwd_inputs((c["B"], c["T"], c["H"], c["D"]), seed=0, dtype="fp32")
    data = np.load(os.path.join(GOLDEN, "cfg0.npz"))
    assert str(data["sha"]) == sha(x.q, x.k, x.v, x.beta)
    o, s = ref.chunked_fwd_rank1(x.q, x.k, x.v, x.beta, None, 64)  # fp32 oracle
    assert ref.rel_l2(o, data["o"]) < 1e-5 and float(np.abs(o - data["o"]).max()) < 1e-4
    assert ref.rel_l2(s, data["s"]) < 1e-5 and float(np.abs(s - data["s"]).max()) < 1e-4


# --- the C restatement (CPU baseline) agrees with the NumPy oracle ---


@pytest.fixture(scope="module")
def cref():
    from oracle import cref as c

    c.load()
    return c


def test_c_restatement_reference_cases(cref):
    for name, q, k, v, b, s0, _ in reference_cases():
        o, s = cref.delta_fwd(q, k, v, b, s0, threads=2)
        e_o, e_s = ref.gated_delta_rule(q, k, v, b, s0, dtype=np.float64)
        assert_f32_parity(o, e_o, name, scaled=True)
        assert_f32_parity(s, e_s, name, scaled=True)


def test_c_restatement_bf16_bits_and_step(cref):
    x = synth.fwd_inputs((2, 70, 3, 32), seed=4, dtype="bf16", s0_std=0.02)
    o, s = cref.delta_fwd(x.q_bits, x.k_bits, x.v_bits, x.beta, x.s0, threads=2)
    e_o, e_s = ref.chunked_fwd_rank1(x.q, x.k, x.v, x.beta, x.s0, 64, dtype=np.float64)
    assert ref.rel_l2(o, e_o) < 1e-5 and ref.rel_l2(s, e_s) < 1e-5
    st = x.s0.copy()
    o_step = cref.delta_step(st, x.q_bits[:, 0], x.k_bits[:, 0], x.v_bits[:, 0], x.beta[:, 0])
    e_s1, e_o1 = ref.delta_step(x.s0.astype(np.float64), x.q[:, 0], x.k[:, 0], x.v[:, 0],
                                x.beta[:, 0])
    np.testing.assert_allclose(o_step, e_o1, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(st, e_s1, rtol=1e-5, atol=1e-6)


def test_bf16_rounding_matches_torch():
    import torch

    x = np.random.default_rng(1).standard_normal(10000).astype(np.float32) * 3
    x[:4] = [1.0 + 2**-8, 1.0 + 3 * 2**-8, -(1.0 + 2**-8), 0.0]  # ties to even
    got = synth.bf16_bits(x)
    exp = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, exp)
