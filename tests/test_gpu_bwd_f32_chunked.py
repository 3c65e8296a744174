"""GPU parity tests of the fp32 chunked backward (K9: fp32 q/k/v with D in {64, 128},
``chunked_delta_rule_bwd``) against the pinned fp64 oracle ``oracle/delta_oracle.py:
delta_vjp`` (the reference's ``_delta_vjp_np``, kernels/__init__.py:460-527) and against
the per-token fp32 backward (K5, path 1).

The cases cover what the chunk form has to get right: a single token, ragged 16-token
chunks, sequences ending on and just past a 256-token span (the state and its gradient
are kept per span), several spans, tokens with beta = 0, missing cotangents, and the
cfg1 shape. Tolerance: the fp32 bounds of tests/parity.py (rel-L2 <= 1e-5, max-abs <=
1e-4 scaled by the gradient's size, as for every backward test).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import delta_oracle as ref
from prometheus_amd import _native, kernels, synth
from tests.parity import assert_f32_parity

pytestmark = pytest.mark.gpu

NAMES = ("gq", "gk", "gv", "gbeta", "gstate")


def _np(x):
    return x.detach().cpu().numpy() if isinstance(x, torch.Tensor) else np.asarray(x)


def _dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()


def _case(shape, seed, state=True):
    x = synth.fwd_inputs(shape, seed=seed, dtype="fp32", s0_std=0.05 if state else None)
    rng = np.random.default_rng(seed + 7)
    b, t, h, d = shape
    go = rng.standard_normal(shape).astype(np.float32)
    gs = (rng.standard_normal((b, h, d, d)) * 0.05).astype(np.float32)
    return x, go, gs


def _bwd(x, go, gs, path=0, beta=None):
    b, t, h, d = x.q.shape
    s0 = x.s0 if x.s0 is not None else np.zeros((b, h, d, d), np.float32)
    res = kernels._DeltaResidual(q=_dev(x.q), k=_dev(x.k), v=_dev(x.v),
                                 beta=_dev(x.beta if beta is None else beta), state0=_dev(s0), chunk=64)
    with _native.use_knobs(path, 0):
        return [_np(g) for g in kernels.chunked_delta_rule_bwd(res, (_dev(go), _dev(gs)))]


def _check(got, exp, what):
    for name, g, e in zip(NAMES, got, exp):
        assert g.dtype == np.float32, f"{what} {name}"
        assert_f32_parity(g, e, f"{what} {name}", scaled=True)


@pytest.mark.parametrize("shape", [(1, 1, 1, 64), (1, 15, 2, 64), (2, 16, 1, 128), (1, 17, 2, 64),
                                   (1, 255, 1, 128), (2, 256, 2, 64), (1, 257, 2, 128), (2, 300, 2, 64),
                                   (1, 520, 1, 128)])
@pytest.mark.parametrize("state", [True, False])
def test_against_the_oracle(shape, state):
    x, go, gs = _case(shape, sum(shape) + state, state)
    got = _bwd(x, go, gs, path=2)  # path 2: the chunked kernels or an error, never a fallback
    _check(got, ref.delta_vjp(x.q, x.k, x.v, x.beta, go, gs, x.s0), str(shape))


def test_zero_betas_and_missing_cotangents():
    shape = (2, 150, 2, 64)
    x, go, gs = _case(shape, 5)
    beta = x.beta.copy()
    beta[:, ::7] = 0.0  # dL/dbeta of a token with beta = 0 is still W . (v - S^T k)
    got = _bwd(x, go, gs, beta=beta)
    _check(got, ref.delta_vjp(x.q, x.k, x.v, beta, go, gs, x.s0), "beta zeros")
    _check(_bwd(x, None, gs), ref.delta_vjp(x.q, x.k, x.v, x.beta, None, gs, x.s0), "go None")
    _check(_bwd(x, go, None), ref.delta_vjp(x.q, x.k, x.v, x.beta, go, None, x.s0), "gs None")


@pytest.mark.parametrize("shape", [(2, 1000, 4, 128), (3, 700, 2, 64)])
def test_against_the_per_token_backward_and_repeatable(shape):
    """Several spans per sequence (4 and 3), both head dimensions: K9 against K5 (path 1)
    on the same inputs within the fp32 bounds, and bitwise repeatable."""
    x, go, gs = _case(shape, 11)
    a = _bwd(x, go, gs)
    k5 = _bwd(x, go, gs, path=1)
    for name, g, e in zip(NAMES, a, k5):
        assert_f32_parity(g, e.astype(np.float64), f"{shape} vs K5 {name}", scaled=True)
    b = _bwd(x, go, gs)
    for name, x1, x2 in zip(NAMES, a, b):
        np.testing.assert_array_equal(x1, x2, err_msg=name)


def test_cfg1_shape_against_the_per_token_backward():
    """The cfg1 shape (B4 T4096 H16 D128, 16 spans per sequence) against K5: the size-
    independent check at full size (the fp64 oracle would take minutes here)."""
    shape = (4, 4096, 16, 128)
    x = synth.fwd_inputs(shape, seed=1, dtype="fp32", s0_std=0.02)
    rng = np.random.default_rng(2)
    go = (rng.standard_normal(shape) * 0.1).astype(np.float32)
    gs = (rng.standard_normal((4, 16, 128, 128)) * 0.01).astype(np.float32)
    a = _bwd(x, go, gs)
    k5 = _bwd(x, go, gs, path=1)
    for name, g, e in zip(NAMES, a, k5):
        assert_f32_parity(g, e.astype(np.float64), f"cfg1 vs K5 {name}", scaled=True)


def test_unsupported_shapes_keep_the_per_token_kernel():
    """D outside {64, 128}: the automatic path runs K5; path 2 refuses."""
    x, go, gs = _case((1, 40, 1, 48), 21)
    _check(_bwd(x, go, gs), ref.delta_vjp(x.q, x.k, x.v, x.beta, go, gs, x.s0), "D48")
    with pytest.raises(_native.NativeError) as ei:
        _bwd(x, go, gs, path=2)
    assert ei.value.code == _native.E_UNSUPPORTED


def test_graph_capture_replays():
    """The three launches captured in a HIP graph: every replay (with eager work and
    synchronisations between them) gives the eager call's bits."""
    shape = (2, 300, 2, 64)
    x, go, gs = _case(shape, 31)
    b, t, h, d = shape
    q, k, v, beta, s0, god, gsd = (_dev(a) for a in (x.q, x.k, x.v, x.beta, x.s0, go, gs))
    outs = [torch.empty_like(q) for _ in range(3)] + [torch.empty_like(beta), torch.empty_like(s0)]
    L = _native.lib()
    nb = L.pm_delta_bwd_workspace_bytes(b, t, h, d, _native.DTYPE_F32)
    ws = torch.empty((nb,), dtype=torch.uint8, device="cuda")
    ptrs = [z.data_ptr() for z in (q, k, v, beta, s0, god, gsd, *outs)]
    stream = torch.cuda.Stream()

    def call():
        _native.check(L.pm_delta_bwd(*ptrs, b, t, h, d, _native.DTYPE_F32, ws.data_ptr(), nb, stream.cuda_stream))

    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        call()
    stream.synchronize()
    eager = [o.clone() for o in outs]
    _check([_np(o) for o in eager], ref.delta_vjp(x.q, x.k, x.v, x.beta, go, gs, x.s0), "eager")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        call()
    for _ in range(3):
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, o, e in zip(NAMES, outs, eager):
            assert torch.equal(o, e), name
