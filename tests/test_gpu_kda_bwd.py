"""GPU tests of the KDA backward (pm_kda_delta_bwd, chunked_kda_rule_bwd and autograd
through chunked_kda_rule) against the fp64 KDA VJP oracle (oracle/gated_oracle.kda_vjp,
pinned on the CPU by its reduction to the scalar-gate VJP, finite differences, a
closed form and planted mistakes).

The reference has no KDA code (spec/03-model.md:12 names the family); the bounds are
the fp32 ones of the other backwards (rel-L2 <= 1e-5, max-abs <= 1e-4 scaled by the
gradient's size, tests/parity.py).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gated_oracle as gref
from prometheus_amd import _native, kernels, synth
from tests.parity import assert_f32_parity

pytestmark = pytest.mark.gpu

NAMES = ("gq", "gk", "gv", "gbeta", "gg", "gstate")


def _np(x):
    return x.detach().cpu().numpy() if isinstance(x, torch.Tensor) else np.asarray(x)


def _dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()


def _case(shape, seed, gate_scale, state):
    x = synth.fwd_inputs(shape, seed=seed, dtype="fp32", s0_std=0.05 if state else None)
    rng = np.random.default_rng(seed + 1)
    b, t, h, d = shape
    g = (-gate_scale * np.abs(rng.standard_normal(shape))).astype(np.float32)
    go = rng.standard_normal(shape).astype(np.float32)
    gs = (rng.standard_normal((b, h, d, d)) * 0.05).astype(np.float32)
    return x, g, go, gs


def _gpu_bwd(q, k, v, beta, g, s0, go, gs):
    d = q.shape[-1]
    s0d = _dev(s0) if s0 is not None else torch.zeros((q.shape[0], q.shape[2], d, d), device="cuda")
    res = kernels._GatedDeltaResidual(q=_dev(q), k=_dev(k), v=_dev(v), beta=_dev(beta), g=_dev(g),
                                      state0=s0d, chunk=64)
    return kernels.chunked_kda_rule_bwd(res, (_dev(go), _dev(gs)))


@pytest.mark.parametrize("shape", [(1, 1, 1, 8), (2, 37, 2, 16), (1, 64, 2, 32), (2, 100, 2, 64),
                                   (1, 130, 2, 128), (1, 33, 1, 160), (1, 20, 1, 256)])
@pytest.mark.parametrize("state", [True, False])
def test_against_the_oracle(shape, state):
    x, g, go, gs = _case(shape, sum(shape) + state, 0.3, state)
    got = _gpu_bwd(x.q, x.k, x.v, x.beta, g, x.s0, go, gs)
    exp = gref.kda_vjp(x.q, x.k, x.v, x.beta, g, go, gs, x.s0)
    for name, a, e in zip(NAMES, got, exp):
        assert _np(a).dtype == np.float32
        assert_f32_parity(_np(a), e, f"{shape} {name}", scaled=True)


@pytest.mark.parametrize("gate_scale", [0.02, 1.0, 4.0])
def test_gate_strengths(gate_scale):
    shape = (2, 90, 2, 64)
    x, g, go, gs = _case(shape, 41, gate_scale, True)
    got = _gpu_bwd(x.q, x.k, x.v, x.beta, g, x.s0, go, gs)
    exp = gref.kda_vjp(x.q, x.k, x.v, x.beta, g, go, gs, x.s0)
    for name, a, e in zip(NAMES, got, exp):
        assert_f32_parity(_np(a), e, f"scale {gate_scale} {name}", scaled=True)


def test_channel_constant_gate_matches_the_gated_backward():
    """g constant along D: the five other gradients within the fp32 bounds of the
    scalar-gated backward, and gg summed over D against its gg."""
    shape = (2, 70, 2, 64)
    x, _, go, gs = _case(shape, 43, 0.0, True)
    g1 = (-0.3 * np.abs(np.random.default_rng(44).standard_normal(shape[:3]))).astype(np.float32)
    got = _gpu_bwd(x.q, x.k, x.v, x.beta, np.repeat(g1[..., None], 64, axis=-1), x.s0, go, gs)
    res = kernels._GatedDeltaResidual(q=_dev(x.q), k=_dev(x.k), v=_dev(x.v), beta=_dev(x.beta), g=_dev(g1),
                                      state0=_dev(x.s0), chunk=64)
    ref = kernels.chunked_gated_delta_rule_bwd(res, (_dev(go), _dev(gs)))
    for name, a, e in zip(("gq", "gk", "gv", "gbeta", "gstate"), got[:4] + got[5:], ref[:4] + ref[5:]):
        assert_f32_parity(_np(a), _np(e), f"constant gate {name}", scaled=True)
    assert_f32_parity(_np(got[4]).sum(axis=-1), _np(ref[4]), "constant gate gg", scaled=True)


def test_missing_cotangents_and_empty_sequence():
    shape = (1, 20, 2, 32)
    x, g, go, _ = _case(shape, 47, 0.3, True)
    got = _gpu_bwd(x.q, x.k, x.v, x.beta, g, x.s0, go, None)
    exp = gref.kda_vjp(x.q, x.k, x.v, x.beta, g, go, None, x.s0)
    for name, a, e in zip(NAMES, got, exp):
        assert_f32_parity(_np(a), e, f"gs None {name}", scaled=True)
    z = np.zeros((1, 0, 2, 32), np.float32)
    gs = np.ones((1, 2, 32, 32), np.float32)
    out = _gpu_bwd(z, z, z, np.zeros((1, 0, 2), np.float32), z, x.s0, None, gs)
    assert _np(out[4]).shape == (1, 0, 2, 32)
    np.testing.assert_array_equal(_np(out[5]), gs)


def test_bf16_inputs_run_the_fp32_reverse_kernels():
    shape = (2, 75, 2, 128)
    x = synth.fwd_inputs(shape, seed=51, dtype="bf16", s0_std=0.02)
    rng = np.random.default_rng(52)
    g = (-0.2 * np.abs(rng.standard_normal(shape))).astype(np.float32)
    go = rng.standard_normal(shape).astype(np.float32)
    gs = (rng.standard_normal((2, 2, 128, 128)) * 0.05).astype(np.float32)
    bf = lambda b: torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).cuda()
    res = kernels._GatedDeltaResidual(q=bf(x.q_bits), k=bf(x.k_bits), v=bf(x.v_bits), beta=_dev(x.beta),
                                      g=_dev(g), state0=_dev(x.s0), chunk=64)
    got = kernels.chunked_kda_rule_bwd(res, (_dev(go), _dev(gs)))
    exp = gref.kda_vjp(x.q, x.k, x.v, x.beta, g, go, gs, x.s0)
    for name, a, e in zip(NAMES, got, exp):
        assert_f32_parity(_np(a), e, f"bf16 {name}", scaled=True)


def test_autograd_through_the_kda_forward():
    """torch.autograd.grad through chunked_kda_rule gives chunked_kda_rule_bwd's bits for
    all six leaves, the gates included; the explicit fwd/bwd pair gives the same."""
    shape = (2, 50, 2, 48)
    x, g, go, gs = _case(shape, 61, 0.4, True)
    leaves = [torch.from_numpy(a).cuda().requires_grad_(True) for a in (x.q, x.k, x.v, x.beta, g, x.s0)]
    y, ns = kernels.chunked_kda_rule(*leaves)
    assert y.requires_grad and ns.requires_grad
    grads = torch.autograd.grad((y, ns), leaves, (_dev(go), _dev(gs)))
    (y2, ns2), res = kernels.chunked_kda_rule_fwd(*(l.detach() for l in leaves), kernels.LinearAttnConfig())
    assert torch.equal(y2, y) and torch.equal(ns2, ns)
    direct = kernels.chunked_kda_rule_bwd(res, (_dev(go), _dev(gs)))
    exp = gref.kda_vjp(x.q, x.k, x.v, x.beta, g, go, gs, x.s0)
    for name, a, d, e in zip(NAMES, grads, direct, exp):
        assert torch.equal(a, d), name
        assert_f32_parity(_np(a), e, f"autograd {name}", scaled=True)


def test_finite_differences_of_the_gpu_forward():
    """The per-channel gate gradient against central differences of the GPU's own fp32
    forward along random directions."""
    shape = (1, 12, 2, 8)
    x, g, _, _ = _case(shape, 71, 0.5, True)
    rng = np.random.default_rng(72)
    go = np.ones(shape, np.float32)
    got = _gpu_bwd(x.q, x.k, x.v, x.beta, g, x.s0, go, None)

    def loss(gg):
        o, _ = kernels.chunked_kda_rule(x.q, x.k, x.v, x.beta, gg, x.s0)
        return float(np.sum(np.asarray(o, np.float64)))

    eps = 1e-2
    d = rng.standard_normal(g.shape).astype(np.float32)
    d /= np.linalg.norm(d)
    fd = (loss(g + eps * d) - loss(g - eps * d)) / (2 * eps)
    np.testing.assert_allclose(float(np.sum(_np(got[4]) * d)), fd, rtol=2e-3, atol=2e-3)


def test_chunked_path_is_refused():
    shape = (1, 8, 1, 64)
    x, g, go, gs = _case(shape, 81, 0.3, False)
    with _native.use_knobs(2, 0), pytest.raises(_native.NativeError) as ei:
        _gpu_bwd(x.q, x.k, x.v, x.beta, g, None, go, gs)
    assert ei.value.code == _native.E_UNSUPPORTED
