"""GPU tests of the differentiable forms: ``kernels.chunked_delta_rule`` and
``model.linear_attention`` under torch autograd.

The reference makes ``chunked_delta_rule`` a ``jax.custom_vjp`` whose
gradient is the fused reverse-state kernel, and tests that ``jax.vjp``
through it equals ``chunked_delta_rule_bwd`` and the NumPy VJP
(``tests/test_kernels.py:520-560``, GPU form ``:1551-1581``). These tests
mirror them with ``torch.autograd``: gradients through ``(output,
next_state)`` equal ``chunked_delta_rule_bwd`` on the forward's residual
(bit for bit: the same kernels on the same inputs) and the fp64 oracle
``delta_vjp`` at the fp32 bounds (bf16 bound for bf16 inputs).

``model.linear_attention`` (the reference differentiates it by JAX autodiff
of its scan, ``model/__init__.py:393-432``) is checked against torch
autograd of an independent fp64 CPU recurrence with the same normalisation.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import delta_oracle as ref
from prometheus_amd import _native, kernels, model, synth
from tests.parity import assert_bf16_parity, assert_f32_parity

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-5, atol=1e-5)


def _np(x):
    return x.detach().cpu().numpy()


def _leaf(x, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dtype).cuda().requires_grad_(True)


def test_autograd_is_the_bwd_kernel_fp32():
    """tests/test_kernels.py:520-560: rng(61), (2, 5, 2, 3), state x 0.05, chunk 2."""
    rng = np.random.default_rng(61)
    q, k, v, beta = synth.reference_test_inputs(rng, 2, 5, 2, 3)
    state = rng.standard_normal((2, 2, 3, 3)).astype(np.float32) * 0.05
    cfg = kernels.LinearAttnConfig(chunk=2)
    (y_fwd, ns_fwd), residual = kernels.chunked_delta_rule_fwd(q, k, v, beta, state, cfg)
    go = rng.standard_normal(y_fwd.shape).astype(np.float32)
    gs = rng.standard_normal(ns_fwd.shape).astype(np.float32) * 0.05
    bwd = kernels.chunked_delta_rule_bwd(residual, (go, gs))

    leaves = [_leaf(x) for x in (q, k, v, beta, state)]
    y, ns = kernels.chunked_delta_rule(*leaves, config=cfg)
    assert y.requires_grad and ns.requires_grad
    np.testing.assert_allclose(_np(y), y_fwd, **TOL)
    np.testing.assert_allclose(_np(ns), ns_fwd, **TOL)
    grads = torch.autograd.grad((y, ns), leaves, (torch.from_numpy(go).cuda(), torch.from_numpy(gs).cuda()))
    exp = ref.delta_vjp(q, k, v, beta, go, gs, state)
    for name, got, e_bwd, e_ref, leaf in zip(("gq", "gk", "gv", "gbeta", "gstate"), grads, bwd, exp, leaves):
        assert got.shape == leaf.shape and got.dtype == torch.float32, name
        np.testing.assert_allclose(_np(got), e_bwd, **TOL, err_msg=name)
        assert_f32_parity(_np(got), e_ref, f"autograd {name} vs delta_vjp", scaled=True)


def test_autograd_head_dim_160_fp32():
    """A head dimension above 128: the per-token forward and backward (16-column tiles)."""
    x = synth.fwd_inputs((1, 40, 2, 160), seed=160, dtype="fp32", s0_std=0.02)
    rng = np.random.default_rng(160)
    go = rng.standard_normal(x.q.shape).astype(np.float32)
    gs = rng.standard_normal(x.s0.shape).astype(np.float32) * 0.05
    leaves = [_leaf(a) for a in (x.q, x.k, x.v, x.beta, x.s0)]
    y, ns = kernels.chunked_delta_rule(*leaves)
    grads = torch.autograd.grad((y, ns), leaves, (torch.from_numpy(go).cuda(), torch.from_numpy(gs).cuda()))
    exp = ref.delta_vjp(x.q, x.k, x.v, x.beta, go, gs, x.s0)
    for name, got, e_ref in zip(("gq", "gk", "gv", "gbeta", "gstate"), grads, exp):
        assert_f32_parity(_np(got), e_ref, f"autograd D160 {name} vs delta_vjp", scaled=True)


def test_autograd_gpu_v1_case():
    """tests/test_kernels.py:1551-1581: rng(64), (2, 8, 2, 4), chunk 64, against the
    bwd entry point and the NumPy-style VJP."""
    rng = np.random.default_rng(64)
    q, k, v, beta = synth.reference_test_inputs(rng, 2, 8, 2, 4)
    state = rng.standard_normal((2, 2, 4, 4)).astype(np.float32) * 0.05
    cfg = kernels.LinearAttnConfig(chunk=64)
    (y_fwd, ns_fwd), residual = kernels.chunked_delta_rule_fwd(q, k, v, beta, state, cfg)
    go = rng.standard_normal(y_fwd.shape).astype(np.float32)
    gs = rng.standard_normal(ns_fwd.shape).astype(np.float32) * 0.05
    bwd = kernels.chunked_delta_rule_bwd(residual, (go, gs))
    exp = ref.delta_vjp(q, k, v, beta, go, gs, state)
    leaves = [_leaf(x) for x in (q, k, v, beta, state)]
    y, ns = kernels.chunked_delta_rule(*leaves, config=cfg)
    (y * torch.from_numpy(go).cuda()).sum().add((ns * torch.from_numpy(gs).cuda()).sum()).backward()
    for got, e_bwd, e_ref in zip((x.grad for x in leaves), bwd, exp):
        np.testing.assert_allclose(_np(got), e_bwd, **TOL)
        np.testing.assert_allclose(_np(got), e_ref, **TOL)


def test_autograd_partial_inputs_and_no_state():
    """Only the leaves that require grad get one; state=None has no gradient; a
    loss on the output alone gives the bwd kernel's result with gs = 0."""
    rng = np.random.default_rng(65)
    q, k, v, beta = synth.reference_test_inputs(rng, 1, 7, 3, 5)
    qd, kd = _leaf(q), torch.from_numpy(k).cuda()
    vd, bd = _leaf(v), torch.from_numpy(beta).cuda()
    y, ns = kernels.chunked_delta_rule(qd, kd, vd, bd)
    go = torch.from_numpy(rng.standard_normal(y.shape).astype(np.float32)).cuda()
    gq, gv = torch.autograd.grad(y, (qd, vd), go)
    (_, _), res = kernels.chunked_delta_rule_fwd(q, k, v, beta, None, kernels.LinearAttnConfig())
    e = kernels.chunked_delta_rule_bwd(res, (_np(go), None))
    np.testing.assert_allclose(_np(gq), e[0], **TOL)
    np.testing.assert_allclose(_np(gv), e[2], **TOL)
    with torch.no_grad():
        y2, _ = kernels.chunked_delta_rule(qd, kd, vd, bd)
    assert not y2.requires_grad


def test_autograd_bf16_chunked_kernel():
    """bf16 q/k/v at D = 128 with a carried-in state: gradients are the chunked bwd
    kernel's bits, in the inputs' dtypes, and within the bf16 bound of delta_vjp."""
    x = synth.fwd_inputs((2, 150, 2, 128), seed=7, dtype="bf16", s0_std=0.02)

    def bf(bits):
        return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda().requires_grad_(True)

    q, k, v = bf(x.q_bits), bf(x.k_bits), bf(x.v_bits)
    beta, s0 = _leaf(x.beta), _leaf(x.s0)
    y, ns = kernels.chunked_delta_rule(q, k, v, beta, s0)
    rng = np.random.default_rng(8)
    go = torch.from_numpy(rng.standard_normal(y.shape).astype(np.float32)).cuda()
    gs = torch.from_numpy(rng.standard_normal(ns.shape).astype(np.float32) * 0.05).cuda()
    grads = torch.autograd.grad((y, ns), (q, k, v, beta, s0), (go, gs))
    assert [g.dtype for g in grads] == [torch.bfloat16] * 3 + [torch.float32] * 2
    res = kernels._DeltaResidual(q=q.detach(), k=k.detach(), v=v.detach(), beta=beta.detach(),
                                 state0=s0.detach(), chunk=64)
    direct = kernels.chunked_delta_rule_bwd(res, (go, gs))
    for got, d in zip(grads, direct):
        assert torch.equal(got, d.to(got.dtype))
    exp = ref.delta_vjp(x.q, x.k, x.v, x.beta, _np(go), _np(gs), x.s0)
    for name, got, e in zip(("gq", "gk", "gv", "gbeta", "gstate"), direct, exp):
        assert_bf16_parity(_np(got), e, f"bf16 autograd {name}")


def test_autograd_backward_runs_under_the_callers_path():
    """The path and tile knobs are per thread, and torch autograd runs a CUDA backward on
    its device thread: the backward must still run the kernels the caller selected. With
    path 1 (per-token kernels) around the forward, the gradients are the per-token fp32
    backward's bits, not the chunked bf16 backward's (which differ from them)."""
    x = synth.fwd_inputs((1, 100, 2, 128), seed=17, dtype="bf16", s0_std=0.02)

    def bf(bits):
        return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda().requires_grad_(True)

    q, k, v = bf(x.q_bits), bf(x.k_bits), bf(x.v_bits)
    beta, s0 = _leaf(x.beta), _leaf(x.s0)
    rng = np.random.default_rng(18)
    go = torch.from_numpy(rng.standard_normal(q.shape).astype(np.float32)).cuda()
    gs = torch.from_numpy(rng.standard_normal(x.s0.shape).astype(np.float32) * 0.05).cuda()
    res = kernels._DeltaResidual(q=q.detach(), k=k.detach(), v=v.detach(), beta=beta.detach(),
                                 state0=s0.detach(), chunk=64)
    chunked = kernels.chunked_delta_rule_bwd(res, (go, gs))
    old = _native.set_path(1)
    try:
        per_token = kernels.chunked_delta_rule_bwd(res, (go, gs))
        y, ns = kernels.chunked_delta_rule(q, k, v, beta, s0)
        grads = torch.autograd.grad((y, ns), (q, k, v, beta, s0), (go, gs))
        assert _native.knobs()[0] == 1
    finally:
        _native.set_path(old)
    assert not torch.equal(chunked[1], per_token[1]), "the two backwards should round differently"
    for got, d in zip(grads, per_token):
        assert torch.equal(got, d.to(got.dtype))


# ---------------------------------------------------------------------------
# model.linear_attention
# ---------------------------------------------------------------------------


def _torch_linear_attention_f64(q, k, v, state):
    """Independent CPU restatement: beta = 1 delta rule on x / max(||x||, 1e-6)."""
    qn = q / torch.clamp_min(torch.linalg.vector_norm(q, dim=-1, keepdim=True), 1e-6)
    kn = k / torch.clamp_min(torch.linalg.vector_norm(k, dim=-1, keepdim=True), 1e-6)
    s = state
    outs = []
    for t in range(q.shape[1]):
        kt, vt, qt = kn[:, t], v[:, t], qn[:, t]                      # (B, H, D)
        ks = torch.einsum("bhd,bhde->bhe", kt, s)
        s = s - torch.einsum("bhd,bhe->bhde", kt, ks) + torch.einsum("bhd,bhe->bhde", kt, vt)
        outs.append(torch.einsum("bhd,bhde->bhe", qt, s))
    return torch.stack(outs, dim=1), s


@pytest.mark.parametrize("dim", [8, 64])
def test_linear_attention_autograd_fp32(dim):
    rng = np.random.default_rng(70 + dim)
    shape = (2, 9, 2, dim)
    q, k, v = (rng.standard_normal(shape).astype(np.float32) for _ in range(3))
    state = rng.standard_normal((2, 2, dim, dim)).astype(np.float32) * 0.05
    go = rng.standard_normal(shape).astype(np.float32)
    gs = rng.standard_normal((2, 2, dim, dim)).astype(np.float32) * 0.05
    leaves = [_leaf(x) for x in (q, k, v, state)]
    y, ns = model.linear_attention(*leaves)
    grads = torch.autograd.grad((y, ns), leaves, (torch.from_numpy(go).cuda(), torch.from_numpy(gs).cuda()))
    cpu = [torch.from_numpy(x).double().requires_grad_(True) for x in (q, k, v, state)]
    ey, es = _torch_linear_attention_f64(*cpu)
    assert_f32_parity(_np(y), ey.detach().numpy(), "linear_attention O")
    assert_f32_parity(_np(ns), es.detach().numpy(), "linear_attention S")
    egrads = torch.autograd.grad((ey, es), cpu, (torch.from_numpy(go).double(), torch.from_numpy(gs).double()))
    for name, got, e in zip(("gq", "gk", "gv", "gstate"), grads, egrads):
        assert_f32_parity(_np(got), e.numpy(), f"linear_attention {name}", scaled=True)


def test_linear_attention_autograd_bf16_heads_squeezed():
    """bf16 3-D inputs (one head, squeezed): the chunked kernels both ways, within the
    bf16 bound of the fp64 reference's gradients."""
    rng = np.random.default_rng(80)
    shape = (2, 130, 64)
    q, k, v = (synth.bf16_to_f32(synth.bf16_bits(rng.standard_normal(shape).astype(np.float32))) for _ in range(3))
    go = rng.standard_normal(shape).astype(np.float32)
    leaves = [_leaf(x, torch.bfloat16) for x in (q, k, v)]
    y, ns = model.linear_attention(*leaves)
    assert y.shape == shape and ns.shape == (2, 64, 64)
    grads = torch.autograd.grad(y, leaves, torch.from_numpy(go).cuda())
    cpu = [torch.from_numpy(x[:, :, None, :]).double().requires_grad_(True) for x in (q, k, v)]
    ey, _ = _torch_linear_attention_f64(*cpu, torch.zeros((2, 1, 64, 64), dtype=torch.float64))
    egrads = torch.autograd.grad(ey, cpu, torch.from_numpy(go[:, :, None, :]).double())
    for name, got, e in zip(("gq", "gk", "gv"), grads, egrads):
        assert got.dtype == torch.bfloat16
        assert_bf16_parity(_np(got.float()), e.numpy()[:, :, 0], f"bf16 linear_attention {name}")
