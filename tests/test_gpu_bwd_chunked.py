"""GPU parity tests of the chunked backward (bf16 q/k/v, D in {64, 128}):
``chunked_delta_rule_bwd`` on bf16 inputs runs the chunked reverse-mode
kernels on bf16 MFMA.

Checked against the pinned fp64 oracle (``oracle/delta_oracle.py:
delta_vjp``, the reference's ``_delta_vjp_np``, kernels/__init__.py:460-527)
on the same bf16-rounded inputs, at the north_star's bf16 tolerance
(rel-L2 <= 2e-2 against the fp32 reference), for every gradient: sequences
of one token, of a partial chunk, of several chunks with a ragged tail,
with and without an initial state, with either cotangent missing. At larger
sizes the per-token fp32 backward (path 1) on the same bf16 inputs is the
reference, and the results must be bitwise repeatable.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import delta_oracle as ref
from prometheus_amd import _native, kernels, synth
from tests.parity import assert_bf16_parity

pytestmark = pytest.mark.gpu

NAMES = ("gq", "gk", "gv", "gbeta", "gstate")


def _np(x):
    return x.detach().cpu().numpy() if isinstance(x, torch.Tensor) else np.asarray(x)


def _dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()


def _bf(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def _problem(shape, seed, state):
    x = synth.fwd_inputs(shape, seed=seed, dtype="bf16", s0_std=0.02 if state else None)
    b, t, h, d = shape
    rng = np.random.default_rng(seed + 1000)
    go = rng.standard_normal(shape).astype(np.float32)
    gs = (rng.standard_normal((b, h, d, d)) * 0.05).astype(np.float32)
    s0 = x.s0 if state else np.zeros((b, h, d, d), np.float32)
    res = kernels._DeltaResidual(q=_bf(x.q_bits), k=_bf(x.k_bits), v=_bf(x.v_bits),
                                 beta=_dev(x.beta), state0=_dev(s0), chunk=64)
    return x, go, gs, res


def _check(got, exp, what):
    for name, g, e in zip(NAMES, got, exp):
        g = _np(g)
        assert g.dtype == np.float32, f"{what} {name}"
        assert_bf16_parity(g, e, f"{what} {name}")


# chunk counts 1 to 5 (the reverse sweep's first and last iterations take their own
# branches of its copy and build schedule), full and ragged last chunks, D = 64 and 128
@pytest.mark.parametrize("shape", [(1, 1, 1, 64), (1, 37, 2, 64), (2, 64, 1, 64), (2, 150, 2, 64),
                                   (1, 63, 1, 128), (2, 130, 3, 128), (1, 257, 1, 128),
                                   (1, 128, 2, 128), (1, 192, 1, 64), (2, 200, 1, 128)])
@pytest.mark.parametrize("state", [True, False])
def test_against_oracle(shape, state):
    x, go, gs, res = _problem(shape, seed=sum(shape) + 7 * state, state=state)
    got = kernels.chunked_delta_rule_bwd(res, (_dev(go), _dev(gs)))
    # x.q, x.k, x.v hold the bf16-rounded values in fp32
    _check(got, ref.delta_vjp(x.q, x.k, x.v, x.beta, go, gs, x.s0 if state else None), str(shape))


def test_missing_cotangents():
    x, go, gs, res = _problem((1, 100, 2, 128), seed=21, state=True)
    _check(kernels.chunked_delta_rule_bwd(res, (None, _dev(gs))),
           ref.delta_vjp(x.q, x.k, x.v, x.beta, None, gs, x.s0), "go None")
    _check(kernels.chunked_delta_rule_bwd(res, (_dev(go), None)),
           ref.delta_vjp(x.q, x.k, x.v, x.beta, go, None, x.s0), "gs None")


def test_empty_sequence_passes_gs_through():
    z = torch.zeros((2, 0, 3, 64), dtype=torch.bfloat16, device="cuda")
    gs = np.random.default_rng(4).standard_normal((2, 3, 64, 64)).astype(np.float32)
    res = kernels._DeltaResidual(q=z, k=z, v=z, beta=torch.zeros((2, 0, 3), device="cuda"),
                                 state0=torch.zeros((2, 3, 64, 64), device="cuda"), chunk=64)
    gq, _, _, gb, g0 = kernels.chunked_delta_rule_bwd(res, (None, _dev(gs)))
    assert _np(gq).shape == (2, 0, 3, 64) and _np(gb).shape == (2, 0, 3)
    np.testing.assert_array_equal(_np(g0), gs)


# The last two have 1920 and 768 chunks, more than the 256 CUs: each workgroup of the
# persistent gradient kernel then walks several chunks, ragged ones (40 tokens) among them,
# with the next chunk's inputs fetched during the current one.
@pytest.mark.parametrize("shape", [(2, 1000, 4, 128), (3, 700, 2, 64), (3, 1000, 40, 64), (2, 1000, 24, 128)])
def test_against_per_token_kernel_and_repeatable(shape):
    """Larger sizes: the per-token fp32 backward on the same bf16 inputs is
    the reference (itself pinned to the oracle at fp32 tolerance)."""
    _, go, gs, res = _problem(shape, seed=31, state=True)
    god, gsd = _dev(go), _dev(gs)
    a = [_np(g) for g in kernels.chunked_delta_rule_bwd(res, (god, gsd))]
    old = _native.set_path(1)
    try:
        exact = [_np(g) for g in kernels.chunked_delta_rule_bwd(res, (god, gsd))]
    finally:
        _native.set_path(old)
    for name, g, e in zip(NAMES, a, exact):
        assert_bf16_parity(g, e, f"{shape} {name}")
    b = [_np(g) for g in kernels.chunked_delta_rule_bwd(res, (god, gsd))]
    for name, x1, x2 in zip(NAMES, a, b):
        np.testing.assert_array_equal(x1, x2, err_msg=name)


def test_path_two_requires_the_chunked_kernel():
    x, go, gs, res = _problem((1, 40, 1, 64), seed=3, state=False)
    old = _native.set_path(2)
    try:
        got = kernels.chunked_delta_rule_bwd(res, (_dev(go), _dev(gs)))
        _check(got, ref.delta_vjp(x.q, x.k, x.v, x.beta, go, gs, None), "path 2")
        # fp32 q/k/v with D = 48: no chunked backward serves it (fp32 D in {64, 128} runs the
        # fp32 chunked one, tests/test_gpu_bwd_f32_chunked.py)
        x48, go48, _, _ = _problem((1, 40, 1, 48), seed=3, state=False)
        r32 = kernels._DeltaResidual(q=_dev(x48.q), k=_dev(x48.k), v=_dev(x48.v), beta=_dev(x48.beta),
                                     state0=_dev(np.zeros((1, 1, 48, 48), np.float32)), chunk=64)
        with pytest.raises(_native.NativeError):
            kernels.chunked_delta_rule_bwd(r32, (_dev(go48), None))
    finally:
        _native.set_path(old)
