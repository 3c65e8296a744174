"""GPU parity tests of the gated delta rule (kernels.chunked_gated_delta_rule,
kernels.gated_delta_rule_step) against the pinned gated oracle
(oracle/gated_oracle.py: the Gated DeltaNet recurrence, reduced to the
reference's delta rule at g = 0).

* bf16 q/k/v with D in {64, 128}: the chunked MFMA kernel with the in-chunk
  decays folded in, at the bf16 bound (rel-L2 <= 2e-2) against the fp64
  oracle on the same rounded inputs: one token, partial and ragged chunks,
  with and without S0, moderate and strong decay, slightly positive gates.
* fp32 inputs: the per-token kernel at the fp32 bounds.
* g = 0 reproduces the ungated kernels.
* (2, 1000, 4, 128): chunked against the per-token kernel on the same bf16
  inputs, bitwise repeatable.
* The gated step (K3 for D in {32, 64, 128}, else the per-token kernel), and
  a chunked prefill continued by gated steps, against the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gated_oracle as gref
from prometheus_amd import _native, kernels, synth
from tests.parity import assert_bf16_parity, assert_f32_parity

pytestmark = pytest.mark.gpu


def _bits(b):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).cuda()


def _gates(rng, shape, scale):
    return (-scale * np.abs(rng.standard_normal(shape))).astype(np.float32)


def _bf16_problem(shape, seed, scale, state):
    x = synth.fwd_inputs(shape, seed=seed, dtype="bf16", s0_std=0.02 if state else None)
    g = _gates(np.random.default_rng(seed + 1), shape[:3], scale)
    return x, g


@pytest.mark.parametrize("shape", [(1, 1, 1, 64), (2, 77, 3, 64), (1, 200, 2, 128), (2, 130, 1, 128)])
@pytest.mark.parametrize("state", [False, True])
@pytest.mark.parametrize("scale", [0.1, 3.0])
def test_chunked_against_oracle(shape, state, scale):
    x, g = _bf16_problem(shape, sum(shape) + 3 * state, scale, state)
    o, s = kernels.chunked_gated_delta_rule(_bits(x.q_bits), _bits(x.k_bits), _bits(x.v_bits),
                                            torch.from_numpy(x.beta).cuda(), torch.from_numpy(g).cuda(),
                                            None if x.s0 is None else torch.from_numpy(x.s0).cuda())
    o_r, s_r = gref.gated_delta_rule(x.q, x.k, x.v, x.beta, g, x.s0)
    assert_bf16_parity(o.cpu().numpy(), o_r, f"{shape} O")
    assert_bf16_parity(s.cpu().numpy(), s_r, f"{shape} S")


def test_chunked_slightly_positive_gates():
    """g > 0 (a growing state) is outside the usual range but exact in the kernel."""
    x = synth.fwd_inputs((1, 150, 2, 64), seed=3, dtype="bf16")
    g = np.full((1, 150, 2), 0.01, np.float32)
    o, s = kernels.chunked_gated_delta_rule(_bits(x.q_bits), _bits(x.k_bits), _bits(x.v_bits),
                                            torch.from_numpy(x.beta).cuda(), torch.from_numpy(g).cuda())
    o_r, s_r = gref.gated_delta_rule(x.q, x.k, x.v, x.beta, g)
    assert_bf16_parity(o.cpu().numpy(), o_r, "O")
    assert_bf16_parity(s.cpu().numpy(), s_r, "S")


@pytest.mark.parametrize("shape", [(2, 50, 2, 32), (1, 100, 2, 64), (1, 40, 3, 128)])
def test_fp32_per_token_against_oracle(shape):
    x = synth.fwd_inputs(shape, seed=sum(shape), dtype="fp32", s0_std=0.02)
    g = _gates(np.random.default_rng(5), shape[:3], 0.5)
    o, s = kernels.chunked_gated_delta_rule(x.q, x.k, x.v, x.beta, g, x.s0)
    o_r, s_r = gref.gated_delta_rule(x.q, x.k, x.v, x.beta, g, x.s0)
    assert_f32_parity(o, o_r, f"{shape} O")
    assert_f32_parity(s, s_r, f"{shape} S")


def test_zero_gate_reproduces_the_ungated_kernels():
    x = synth.fwd_inputs((2, 150, 2, 128), seed=9, dtype="bf16", s0_std=0.02)
    z = torch.zeros((2, 150, 2), device="cuda")
    args = (_bits(x.q_bits), _bits(x.k_bits), _bits(x.v_bits), torch.from_numpy(x.beta).cuda())
    s0 = torch.from_numpy(x.s0).cuda()
    og, sg = kernels.chunked_gated_delta_rule(*args, z, s0)
    # the ungated single-stage form (path 2): by default this shape runs the split form,
    # which rounds differently
    old = _native.set_path(2)
    try:
        ou, su = kernels.chunked_delta_rule(*args, s0)
    finally:
        _native.set_path(old)
    np.testing.assert_allclose(og.cpu().numpy(), ou.cpu().numpy(), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(sg.cpu().numpy(), su.cpu().numpy(), rtol=1e-6, atol=1e-6)
    # the per-token kernel multiplies by exp(0) = 1 exactly: bitwise
    xf = synth.fwd_inputs((1, 60, 2, 48), seed=10, dtype="fp32")
    og, sg = kernels.chunked_gated_delta_rule(xf.q, xf.k, xf.v, xf.beta, np.zeros((1, 60, 2), np.float32))
    ou, su = kernels.chunked_delta_rule(xf.q, xf.k, xf.v, xf.beta)
    np.testing.assert_array_equal(og, ou)
    np.testing.assert_array_equal(sg, su)


def test_large_against_per_token_and_repeatable():
    shape = (2, 1000, 4, 128)
    x, g = _bf16_problem(shape, 11, 0.2, True)
    args = (_bits(x.q_bits), _bits(x.k_bits), _bits(x.v_bits), torch.from_numpy(x.beta).cuda(),
            torch.from_numpy(g).cuda(), torch.from_numpy(x.s0).cuda())
    a = kernels.chunked_gated_delta_rule(*args)
    old = _native.set_path(1)
    try:
        exact = kernels.chunked_gated_delta_rule(*args)
    finally:
        _native.set_path(old)
    for got, want, n in zip(a, exact, ("O", "S")):
        assert_bf16_parity(got.cpu().numpy(), want.cpu().numpy(), n)
    b = kernels.chunked_gated_delta_rule(*args)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("d", [32, 64, 128, 48])
def test_gated_step(d):
    rng = np.random.default_rng(d)
    b, h = 5, 3
    x = synth.fwd_inputs((b, 1, h, d), seed=d, dtype="fp32", s0_std=0.05)
    g = _gates(rng, (b, h), 1.0)
    state = torch.from_numpy(x.s0.copy()).cuda()
    o = kernels.gated_delta_rule_step(torch.from_numpy(x.q[:, 0]).cuda(), torch.from_numpy(x.k[:, 0]).cuda(),
                                      torch.from_numpy(x.v[:, 0]).cuda(), torch.from_numpy(x.beta[:, 0]).cuda(),
                                      torch.from_numpy(g).cuda(), state)
    o_r, s_r = gref.gated_step(x.s0, x.q[:, 0], x.k[:, 0], x.v[:, 0], x.beta[:, 0], g)
    assert_f32_parity(o.cpu().numpy(), o_r, f"D{d} o")
    assert_f32_parity(state.cpu().numpy(), s_r, f"D{d} S")


def test_chunked_prefill_then_gated_steps():
    rng = np.random.default_rng(21)
    t_pre, n_dec, shape = 130, 5, (2, 135, 2, 128)
    x, g = _bf16_problem(shape, 21, 0.3, False)
    qb, kb, vb = _bits(x.q_bits), _bits(x.k_bits), _bits(x.v_bits)
    beta, gg = torch.from_numpy(x.beta).cuda(), torch.from_numpy(g).cuda()
    o_pre, s = kernels.chunked_gated_delta_rule(qb[:, :t_pre].contiguous(), kb[:, :t_pre].contiguous(),
                                                vb[:, :t_pre].contiguous(), beta[:, :t_pre].contiguous(),
                                                gg[:, :t_pre].contiguous())
    outs = [kernels.gated_delta_rule_step(qb[:, t].contiguous(), kb[:, t].contiguous(), vb[:, t].contiguous(),
                                          beta[:, t].contiguous(), gg[:, t].contiguous(), s)
            for t in range(t_pre, shape[1])]
    o = torch.cat([o_pre, torch.stack(outs, dim=1)], dim=1).cpu().numpy()
    o_r, s_r = gref.gated_delta_rule(x.q, x.k, x.v, x.beta, g)
    assert_bf16_parity(o, o_r, "O")
    assert_bf16_parity(s.cpu().numpy(), s_r, "S")
