"""GPU parity tests of the backward (K5, ``chunked_delta_rule_bwd``) against
the pinned CPU oracle (``oracle/delta_oracle.py: delta_vjp``, the
reference's ``_delta_vjp_np``, kernels/__init__.py:460-527).

Mirrors the reference's backward tests: the seeded fwd->bwd cases with
random go / gs (tests/test_kernels_delta_fwd_jit.py:284-347, seeds 105 and
106), the finite-difference test of the gradients (tests/test_kernels.py:
409-432, seed 18), plus the shapes this build adds: head dimensions up to
128 with padded row slices and ragged 32-column tiles of the state,
sequences across several checkpoint blocks, head dimensions 129-256 on 16-column
tiles, bf16 q/k/v, missing cotangents, T = 0 and repeatability.

Tolerance: fp32 (tests/parity.py), rel-L2 <= 1e-5 and max-abs <= 1e-4
(scaled), against the fp64 oracle on the same (for bf16: bf16-rounded)
inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import delta_oracle as ref
from prometheus_amd import _native, kernels, synth
from tests.golden.make_golden import reference_cases
from tests.parity import assert_f32_parity

pytestmark = pytest.mark.gpu

NAMES = ("gq", "gk", "gv", "gbeta", "gstate")


def _np(x):
    return x.detach().cpu().numpy() if isinstance(x, torch.Tensor) else np.asarray(x)


def _dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()


def _residual(q, k, v, beta, s0):
    d = q.shape[-1]
    s0d = _dev(s0) if s0 is not None else torch.zeros((q.shape[0], q.shape[2], d, d),
                                                       dtype=torch.float32, device="cuda")
    return kernels._DeltaResidual(q=_dev(q), k=_dev(k), v=_dev(v), beta=_dev(beta), state0=s0d,
                                  chunk=64)


def _check(got, exp, what):
    for name, g, e in zip(NAMES, got, exp):
        g = _np(g)
        assert g.dtype == np.float32, f"{what} {name}"
        assert_f32_parity(g, e, f"{what} {name}", scaled=True)


def test_reference_cases_with_random_cotangents():
    """tests/test_kernels_delta_fwd_jit.py:284-317 (seed 105 over the fwd cases)."""
    rng = np.random.default_rng(105)
    for name, q, k, v, b, s0, _ in reference_cases():
        go = rng.standard_normal(q.shape).astype(np.float32)
        gs = (rng.standard_normal((q.shape[0], q.shape[2], q.shape[3], q.shape[3])) * 0.05
              ).astype(np.float32)
        got = kernels.chunked_delta_rule_bwd(_residual(q, k, v, b, s0), (_dev(go), _dev(gs)))
        _check(got, ref.delta_vjp(q, k, v, b, go, gs, s0), name)


def test_fwd_residual_feeds_bwd():
    """tests/test_kernels_delta_fwd_jit.py:320-347 (seed 106, chunk 2, state0)."""
    rng = np.random.default_rng(106)
    q, k, v, beta = synth.reference_test_inputs(rng, batch=2, seq=5, heads=2, dim=3)
    state0 = (rng.standard_normal((2, 2, 3, 3)) * 0.05).astype(np.float32)
    cfg = kernels.LinearAttnConfig(chunk=2)
    (out, ns), res = kernels.chunked_delta_rule_fwd(_dev(q), _dev(k), _dev(v), _dev(beta),
                                                    _dev(state0), cfg)
    go = rng.standard_normal(_np(out).shape).astype(np.float32)
    gs = (rng.standard_normal(_np(ns).shape) * 0.05).astype(np.float32)
    got = kernels.chunked_delta_rule_bwd(res, (_dev(go), _dev(gs)))
    assert len(got) == 5
    _check(got, ref.delta_vjp(q, k, v, beta, go, gs, state0), "rng106")
    # NumPy residual (the reference's host path) gives NumPy gradients
    (_, _), res_np = kernels.chunked_delta_rule_fwd(q, k, v, beta, state0, cfg)
    got_np = kernels.chunked_delta_rule_bwd(res_np, (go, gs))
    assert all(isinstance(g, np.ndarray) for g in got_np)
    _check(got_np, ref.delta_vjp(q, k, v, beta, go, gs, state0), "rng106 numpy")


def test_finite_differences_of_the_gpu_forward():
    """tests/test_kernels.py:409-432: seed 18, go = ones, gs = zeros, unit directions;
    the analytic gradients against central differences of the GPU forward."""
    rng = np.random.default_rng(18)
    q, k, v, beta = synth.reference_test_inputs(rng, batch=1, seq=3, heads=2, dim=3)
    go = np.ones((1, 3, 2, 3), dtype=np.float32)
    gs = np.zeros((1, 2, 3, 3), dtype=np.float32)
    gq, gk, gv, gbeta, _ = (_np(x) for x in kernels.chunked_delta_rule_bwd(
        _residual(q, k, v, beta, None), (_dev(go), _dev(gs))))
    eps = 1e-3

    def prod_sum(qq, kk, vv, bb):
        o, _ = kernels.chunked_delta_rule(_dev(qq), _dev(kk), _dev(vv), _dev(bb))
        return float(np.sum(_np(o).astype(np.float64)))

    for name, x, gx in (("q", q, gq), ("k", k, gk), ("v", v, gv), ("beta", beta, gbeta)):
        d = rng.standard_normal(x.shape).astype(np.float32)
        d /= np.linalg.norm(d) + 1e-12
        xs = {"q": q, "k": k, "v": v, "beta": beta}
        plus, minus = dict(xs), dict(xs)
        plus[name], minus[name] = x + eps * d, x - eps * d
        fd = (prod_sum(plus["q"], plus["k"], plus["v"], plus["beta"])
              - prod_sum(minus["q"], minus["k"], minus["v"], minus["beta"])) / (2 * eps)
        np.testing.assert_allclose(fd, float(np.sum(gx * d)), rtol=1e-3, atol=1e-3, err_msg=name)


@pytest.mark.parametrize("shape", [(1, 1, 1, 8), (2, 63, 2, 16), (1, 41, 2, 24), (2, 9, 3, 32),
                                   (1, 65, 2, 48), (1, 200, 2, 64), (2, 130, 1, 128), (1, 17, 2, 33),
                                   (1, 20, 1, 100)])
@pytest.mark.parametrize("state", [True, False])
def test_shapes_across_checkpoint_blocks(shape, state):
    x = synth.fwd_inputs(shape, seed=sum(shape) + state, dtype="fp32",
                         s0_std=0.02 if state else None)
    rng = np.random.default_rng(sum(shape))
    b, t, h, d = shape
    go = rng.standard_normal(shape).astype(np.float32)
    gs = (rng.standard_normal((b, h, d, d)) * 0.05).astype(np.float32)
    got = kernels.chunked_delta_rule_bwd(_residual(x.q, x.k, x.v, x.beta, x.s0),
                                         (_dev(go), _dev(gs)))
    _check(got, ref.delta_vjp(x.q, x.k, x.v, x.beta, go, gs, x.s0), str(shape))


@pytest.mark.parametrize("shape", [(1, 20, 2, 160), (1, 17, 1, 256), (2, 9, 1, 129), (1, 33, 1, 200)])
@pytest.mark.parametrize("state", [True, False])
def test_head_dims_above_128(shape, state):
    """Head dimensions the forward serves above 128 (up to 256): 16-column tiles of
    the state, 32 row slices per column."""
    x = synth.fwd_inputs(shape, seed=sum(shape) + state, dtype="fp32",
                         s0_std=0.02 if state else None)
    rng = np.random.default_rng(sum(shape))
    b, t, h, d = shape
    go = rng.standard_normal(shape).astype(np.float32)
    gs = (rng.standard_normal((b, h, d, d)) * 0.05).astype(np.float32)
    got = kernels.chunked_delta_rule_bwd(_residual(x.q, x.k, x.v, x.beta, x.s0),
                                         (_dev(go), _dev(gs)))
    _check(got, ref.delta_vjp(x.q, x.k, x.v, x.beta, go, gs, x.s0), str(shape))


def test_bf16_inputs_d256_against_rounded_values():
    x = synth.fwd_inputs((1, 24, 2, 256), seed=11, dtype="bf16", s0_std=0.02)
    rng = np.random.default_rng(11)
    go = rng.standard_normal(x.q.shape).astype(np.float32)

    def bf(bits):
        return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()

    res = kernels._DeltaResidual(q=bf(x.q_bits), k=bf(x.k_bits), v=bf(x.v_bits), beta=_dev(x.beta),
                                 state0=_dev(x.s0), chunk=64)
    got = kernels.chunked_delta_rule_bwd(res, (_dev(go), None))
    _check(got, ref.delta_vjp(x.q, x.k, x.v, x.beta, go, None, x.s0), "bf16 D256")


def test_bf16_inputs_against_rounded_values():
    """The per-token kernel (path 1) reading bf16 q/k/v: fp32 parity on the
    rounded values. (The automatic choice for bf16 and D = 64 is the chunked
    kernel, tests/test_gpu_bwd_chunked.py.)"""
    x = synth.fwd_inputs((2, 100, 2, 64), seed=9, dtype="bf16", s0_std=0.02)
    rng = np.random.default_rng(9)
    go = rng.standard_normal(x.q.shape).astype(np.float32)
    gs = (rng.standard_normal((2, 2, 64, 64)) * 0.05).astype(np.float32)

    def bf(bits):
        return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()

    res = kernels._DeltaResidual(q=bf(x.q_bits), k=bf(x.k_bits), v=bf(x.v_bits), beta=_dev(x.beta),
                                 state0=_dev(x.s0), chunk=64)
    old = _native.set_path(1)
    try:
        got = kernels.chunked_delta_rule_bwd(res, (_dev(go), _dev(gs)))
    finally:
        _native.set_path(old)
    # x.q, x.k, x.v are the bf16-rounded values in fp32
    _check(got, ref.delta_vjp(x.q, x.k, x.v, x.beta, go, gs, x.s0), "bf16")


def test_missing_cotangents_are_zeros():
    x = synth.fwd_inputs((1, 40, 2, 16), seed=3, dtype="fp32", s0_std=0.02)
    rng = np.random.default_rng(3)
    go = rng.standard_normal(x.q.shape).astype(np.float32)
    gs = (rng.standard_normal((1, 2, 16, 16)) * 0.05).astype(np.float32)
    res = _residual(x.q, x.k, x.v, x.beta, x.s0)
    _check(kernels.chunked_delta_rule_bwd(res, (None, _dev(gs))),
           ref.delta_vjp(x.q, x.k, x.v, x.beta, None, gs, x.s0), "go None")
    _check(kernels.chunked_delta_rule_bwd(res, (_dev(go), None)),
           ref.delta_vjp(x.q, x.k, x.v, x.beta, go, None, x.s0), "gs None")


def test_empty_sequence_passes_gs_through():
    z = np.zeros((2, 0, 3, 8), np.float32)
    gs = np.random.default_rng(4).standard_normal((2, 3, 8, 8)).astype(np.float32)
    res = _residual(z, z, z, np.zeros((2, 0, 3), np.float32), None)
    gq, gk, gv, gb, g0 = kernels.chunked_delta_rule_bwd(res, (None, _dev(gs)))
    assert _np(gq).shape == (2, 0, 3, 8) and _np(gb).shape == (2, 0, 3)
    np.testing.assert_array_equal(_np(g0), gs)


def test_repeat_calls_are_bitwise_identical():
    x = synth.fwd_inputs((2, 150, 2, 32), seed=8, dtype="fp32", s0_std=0.02)
    rng = np.random.default_rng(8)
    go = _dev(rng.standard_normal(x.q.shape).astype(np.float32))
    res = _residual(x.q, x.k, x.v, x.beta, x.s0)
    a = [_np(g) for g in kernels.chunked_delta_rule_bwd(res, (go, None))]
    b = [_np(g) for g in kernels.chunked_delta_rule_bwd(res, (go, None))]
    for name, x1, x2 in zip(NAMES, a, b):
        np.testing.assert_array_equal(x1, x2, err_msg=name)
