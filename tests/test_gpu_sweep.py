"""Seeded randomized parity sweep over the product entry points.

The other GPU tests pin chosen shapes and edge cases. This file draws shapes at random
(seeded, so every run checks the same cases): batch 1-3, 1-600 tokens (ragged against
the 64-token chunks and the 16-token and 256-token spans of the fp32 paths), 1-4 heads,
head dimension 64 or 128, with and without an initial state. Each case runs one entry
point through ``prometheus_amd.kernels`` (and so the C ABI and the gfx950 kernels the
default routing picks) and compares with the fp64 oracle on the same inputs, at the
bounds of tests/parity.py: bf16 q/k/v rel-L2 <= 2e-2 against the recurrence on the
bf16-rounded values; fp32 q/k/v rel-L2 <= 1e-5 and max-abs <= 1e-4 (gradients: the
max-abs bound scaled by their size, as in every backward test).

Oracles: ``oracle/delta_oracle.py`` (``wy_chunked_fwd``, the chunk form of the
reference's recurrence, kernels/__init__.py:421-458; ``delta_vjp``, its VJP,
:460-527) and ``oracle/gated_oracle.py`` (``gated_delta_rule``, ``kda_delta_rule``), each
pinned by the CPU tests.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import delta_oracle as ref
from oracle import gated_oracle as gref
from prometheus_amd import kernels, synth
from tests.parity import assert_bf16_parity, assert_f32_parity

pytestmark = pytest.mark.gpu

SEEDS = list(range(12))


def _shape(seed):
    rng = np.random.default_rng(1000 + seed)
    b = int(rng.integers(1, 4))
    t = int(rng.choice([int(rng.integers(1, 70)), int(rng.integers(1, 601))]))
    h = int(rng.integers(1, 5))
    d = int(rng.choice([64, 128]))
    return (b, t, h, d), bool(rng.integers(0, 2))


def _bits(b):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).cuda()


def _dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()


def _np(x):
    return x.detach().cpu().numpy()


@pytest.mark.parametrize("seed", SEEDS)
def test_bf16_forward(seed):
    shape, state = _shape(seed)
    x = synth.fwd_inputs(shape, seed=seed, dtype="bf16", s0_std=0.02 if state else None)
    for odt in (None, torch.bfloat16):
        o, s = kernels.chunked_delta_rule(_bits(x.q_bits), _bits(x.k_bits), _bits(x.v_bits), _dev(x.beta),
                                          _dev(x.s0), out_dtype=odt)
        e_o, e_s = ref.wy_chunked_fwd(x.q, x.k, x.v, x.beta, x.s0)
        what = f"seed {seed} {shape} state {state} out {odt}"
        assert_bf16_parity(_np(o.float()), e_o, what + " O")
        assert_bf16_parity(_np(s), e_s, what + " S")


@pytest.mark.parametrize("seed", SEEDS)
def test_fp32_forward(seed):
    shape, state = _shape(seed)
    x = synth.fwd_inputs(shape, seed=seed, dtype="fp32", s0_std=0.02 if state else None)
    o, s = kernels.chunked_delta_rule(_dev(x.q), _dev(x.k), _dev(x.v), _dev(x.beta), _dev(x.s0))
    e_o, e_s = ref.wy_chunked_fwd(x.q, x.k, x.v, x.beta, x.s0)
    what = f"seed {seed} {shape} state {state}"
    assert_f32_parity(_np(o), e_o, what + " O")
    assert_f32_parity(_np(s), e_s, what + " S")


@pytest.mark.parametrize("seed", SEEDS)
@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_backward(seed, dtype):
    shape, state = _shape(seed)
    b, t, h, d = shape
    x = synth.fwd_inputs(shape, seed=seed, dtype=dtype, s0_std=0.05 if state else None)
    rng = np.random.default_rng(seed + 99)
    go = rng.standard_normal(shape).astype(np.float32)
    gs = (0.05 * rng.standard_normal((b, h, d, d))).astype(np.float32)
    s0 = x.s0 if x.s0 is not None else np.zeros((b, h, d, d), np.float32)
    if dtype == "bf16":
        q, k, v = _bits(x.q_bits), _bits(x.k_bits), _bits(x.v_bits)
    else:
        q, k, v = _dev(x.q), _dev(x.k), _dev(x.v)
    res = kernels._DeltaResidual(q=q, k=k, v=v, beta=_dev(x.beta), state0=_dev(s0), chunk=64)
    got = kernels.chunked_delta_rule_bwd(res, (_dev(go), _dev(gs)))
    exp = ref.delta_vjp(x.q, x.k, x.v, x.beta, go, gs, s0)
    for name, g_, e_ in zip(("gq", "gk", "gv", "gbeta", "gstate"), got, exp):
        what = f"seed {seed} {shape} {dtype} state {state} {name}"
        if dtype == "bf16":
            assert_bf16_parity(_np(g_), e_, what)
        else:
            assert_f32_parity(_np(g_), e_, what, scaled=True)


@pytest.mark.parametrize("seed", SEEDS[:8])
def test_gated_and_kda_forward(seed):
    shape, state = _shape(seed)
    x = synth.fwd_inputs(shape, seed=seed, dtype="bf16", s0_std=0.02 if state else None)
    rng = np.random.default_rng(seed + 5)
    scale = float(rng.choice([0.05, 0.5, 2.0]))
    g = (-scale * np.abs(rng.standard_normal(shape[:3]))).astype(np.float32)
    gk = (-scale * np.abs(rng.standard_normal(shape))).astype(np.float32)
    q, k, v = _bits(x.q_bits), _bits(x.k_bits), _bits(x.v_bits)
    what = f"seed {seed} {shape} state {state} gate scale {scale}"
    o, s = kernels.chunked_gated_delta_rule(q, k, v, _dev(x.beta), _dev(g), _dev(x.s0))
    e_o, e_s = gref.gated_delta_rule(x.q, x.k, x.v, x.beta, g, x.s0)
    assert_bf16_parity(_np(o), e_o, what + " gated O")
    assert_bf16_parity(_np(s), e_s, what + " gated S")
    o, s = kernels.chunked_kda_rule(q, k, v, _dev(x.beta), _dev(gk), _dev(x.s0))
    e_o, e_s = gref.kda_delta_rule(x.q, x.k, x.v, x.beta, gk, x.s0)
    assert_bf16_parity(_np(o), e_o, what + " KDA O")
    assert_bf16_parity(_np(s), e_s, what + " KDA S")


@pytest.mark.parametrize("seed", SEEDS[:6])
def test_varlen_forward(seed):
    rng = np.random.default_rng(2000 + seed)
    h, d = int(rng.integers(1, 5)), int(rng.choice([64, 128]))
    lens = rng.integers(0, 400, size=int(rng.integers(1, 12)))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    n = int(cu[-1])
    if n == 0:
        lens[0], cu = 1, np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        n = int(cu[-1])
    x = synth.fwd_inputs((n, h, d), seed=seed, dtype="bf16")
    o, s = kernels.chunked_delta_rule_varlen(_bits(x.q_bits), _bits(x.k_bits), _bits(x.v_bits), _dev(x.beta),
                                             torch.from_numpy(cu).cuda())
    o, s = _np(o), _np(s)
    for i in range(lens.size):
        a, z = int(cu[i]), int(cu[i + 1])
        e_o, e_s = ref.wy_chunked_fwd(x.q[None, a:z], x.k[None, a:z], x.v[None, a:z], x.beta[None, a:z])
        what = f"seed {seed} H{h} D{d} segment {i} [{a}, {z})"
        if z > a:
            assert_bf16_parity(o[a:z], e_o[0], what + " O")
        assert_bf16_parity(s[i], e_s[0], what + " S")
