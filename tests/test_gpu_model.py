"""GPU parity tests of the model-side caller (prometheus_amd.model) against
the pinned oracle (oracle/model_oracle.py), following the reference's own
tests of model.linear_attention (tests/test_model.py:353-406, seeds 7-10,
rtol = atol = 1e-5 there) and adding: head dimensions up to 128 over
several hundred tokens, zero and tiny vectors (the eps guard), a 3-D state,
torch tensors in place, the projection layer _linear_attn
(model/__init__.py:726-734), and bf16 inputs on the chunked MFMA kernel with
the norms folded in (rel-L2 <= 2e-2, the bf16 bound).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import model_oracle as mref
from prometheus_amd import _native, model
from tests.parity import assert_bf16_parity, assert_f32_parity

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-5, atol=1e-5)  # tests/test_model.py:43


def _rand(rng, shape):
    return rng.standard_normal(shape).astype(np.float32)


def test_linear_attention_matches_reference():
    """tests/test_model.py:353-364."""
    rng = np.random.default_rng(7)
    q, k, v = (_rand(rng, (2, 5, 3, 8)) for _ in range(3))
    out_m, st_m = model.linear_attention(q, k, v)
    out_r, st_r = mref.linear_attention(q, k, v)
    np.testing.assert_allclose(out_m, out_r, **TOL)
    np.testing.assert_allclose(st_m, st_r, **TOL)
    assert out_m.shape == q.shape and st_m.shape == (2, 3, 8, 8) and out_m.dtype == np.float32


def test_linear_attention_is_causal():
    """tests/test_model.py:367-380."""
    rng = np.random.default_rng(8)
    q, k, v = (_rand(rng, (1, 6, 2, 4)) for _ in range(3))
    out, _ = model.linear_attention(q, k, v)
    q2, k2, v2 = q.copy(), k.copy(), v.copy()
    for x in (q2, k2, v2):
        x[:, -1] += 1.5
    out2, _ = model.linear_attention(q2, k2, v2)
    np.testing.assert_allclose(out[:, :-1], out2[:, :-1], **TOL)


def test_linear_attention_state_chunks_match_full():
    """tests/test_model.py:383-395."""
    rng = np.random.default_rng(9)
    q, k, v = (_rand(rng, (2, 6, 2, 4)) for _ in range(3))
    full, st_full = model.linear_attention(q, k, v)
    a, st = model.linear_attention(q[:, :2], k[:, :2], v[:, :2])
    b, st2 = model.linear_attention(q[:, 2:], k[:, 2:], v[:, 2:], state=st)
    np.testing.assert_allclose(np.concatenate([a, b], axis=1), full, **TOL)
    np.testing.assert_allclose(st2, st_full, **TOL)


def test_linear_attention_3d_squeezes_heads():
    """tests/test_model.py:398-406, plus a 3-D state carried between calls."""
    rng = np.random.default_rng(10)
    q, k, v = (_rand(rng, (2, 4, 8)) for _ in range(3))
    out, st = model.linear_attention(q, k, v)
    assert out.shape == q.shape and st.shape == (2, 8, 8)
    out_r, st_r = mref.linear_attention(q, k, v)
    np.testing.assert_allclose(out, out_r, **TOL)
    np.testing.assert_allclose(st, st_r, **TOL)
    o2, s2 = model.linear_attention(q, k, v, state=st)
    o2r, s2r = mref.linear_attention(q, k, v, state=st_r)
    np.testing.assert_allclose(o2, o2r, **TOL)
    np.testing.assert_allclose(s2, s2r, **TOL)


@pytest.mark.parametrize("shape", [(1, 300, 2, 64), (2, 130, 2, 128), (1, 77, 3, 33)])
def test_larger_shapes(shape):
    rng = np.random.default_rng(sum(shape))
    q, k, v = (_rand(rng, shape) for _ in range(3))
    s0 = _rand(rng, (shape[0], shape[2], shape[3], shape[3])) * 0.05
    out, st = model.linear_attention(q, k, v, state=s0)
    out_r, st_r = mref.linear_attention(q, k, v, s0, dtype=np.float64)
    assert_f32_parity(out, out_r, f"{shape} out")
    assert_f32_parity(st, st_r, f"{shape} state")


def test_zero_and_tiny_vectors():
    rng = np.random.default_rng(11)
    q, k, v = (_rand(rng, (1, 8, 2, 16)) for _ in range(3))
    q[0, 2, 0] = 0.0
    k[0, 3, 1] = 0.0
    k[0, 5, 0] = 1e-9
    out, st = model.linear_attention(q, k, v)
    out_r, st_r = mref.linear_attention(q, k, v, dtype=np.float64)
    assert np.all(out[0, 2, 0] == 0.0)
    np.testing.assert_allclose(out, out_r, **TOL)
    np.testing.assert_allclose(st, st_r, **TOL)


def _bf16(rng, shape):
    x = torch.from_numpy(_rand(rng, shape)).to(torch.bfloat16).cuda()
    return x, x.float().cpu().numpy()


def test_bf16_and_torch_tensors_in_place():
    """bf16 tensors, used in place: the chunked kernel (bf16 parity) by default,
    the per-token kernel (fp32 parity on the rounded values) under path 1."""
    rng = np.random.default_rng(12)
    (qb, q), (kb, k), (vb, v) = (_bf16(rng, (2, 50, 2, 64)) for _ in range(3))
    out_r, st_r = mref.linear_attention(q, k, v, dtype=np.float64)
    out, st = model.linear_attention(qb, kb, vb)
    assert isinstance(out, torch.Tensor) and out.is_cuda and out.dtype == torch.float32
    assert_bf16_parity(out.cpu().numpy(), out_r, "chunked out")
    assert_bf16_parity(st.cpu().numpy(), st_r, "chunked state")
    old = _native.set_path(1)
    try:
        out1, st1 = model.linear_attention(qb, kb, vb)
    finally:
        _native.set_path(old)
    assert_f32_parity(out1.cpu().numpy(), out_r, "per-token out")
    assert_f32_parity(st1.cpu().numpy(), st_r, "per-token state")


@pytest.mark.parametrize("shape", [(1, 1, 1, 64), (2, 77, 3, 64), (1, 200, 2, 128), (2, 64, 1, 128)])
@pytest.mark.parametrize("state", [False, True])
def test_chunked_kernel_against_oracle(shape, state):
    """bf16 q/k/v, D in {64, 128}: the chunked kernel folding the norms into its tiles."""
    rng = np.random.default_rng(sum(shape) + state)
    (qb, q), (kb, k), (vb, v) = (_bf16(rng, shape) for _ in range(3))
    s0 = (_rand(rng, (shape[0], shape[2], shape[3], shape[3])) * 0.05) if state else None
    out, st = model.linear_attention(qb, kb, vb, state=None if s0 is None else torch.from_numpy(s0).cuda())
    out_r, st_r = mref.linear_attention(q, k, v, s0, dtype=np.float64)
    assert_bf16_parity(out.cpu().numpy(), out_r, f"{shape} out")
    assert_bf16_parity(st.cpu().numpy(), st_r, f"{shape} state")


def test_chunked_kernel_large_zero_rows_and_repeatable():
    """(2, 1000, 4, 128) against the per-token kernel on the same bf16 inputs, with
    zero and tiny q/k rows (the eps guard), and bitwise repeatable."""
    rng = np.random.default_rng(13)
    shape = (2, 1000, 4, 128)
    (qb, _), (kb, _), (vb, _) = (_bf16(rng, shape) for _ in range(3))
    qb[0, 10, 1] = 0
    kb[1, 500, 2] = 0
    kb[0, 65, 0] = 1e-9
    a = model.linear_attention(qb, kb, vb)
    old = _native.set_path(1)
    try:
        exact = model.linear_attention(qb, kb, vb)
    finally:
        _native.set_path(old)
    for x, e, n in zip(a, exact, ("out", "state")):
        assert_bf16_parity(x.cpu().numpy(), e.cpu().numpy(), n)
    assert torch.all(a[0][0, 10, 1] == 0)
    b = model.linear_attention(qb, kb, vb)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("shape", [(1, 1, 1, 64), (2, 77, 3, 64), (1, 200, 2, 128), (2, 64, 1, 128)])
@pytest.mark.parametrize("state", [False, True])
def test_fp32_chunked_kernel_against_oracle(shape, state):
    """fp32 q/k/v, D in {64, 128}: the fp32 chunked forward in its normalised mode
    (fp32 MFMA), at the fp32 bounds."""
    rng = np.random.default_rng(100 + sum(shape) + state)
    q, k, v = (_rand(rng, shape) for _ in range(3))
    s0 = (_rand(rng, (shape[0], shape[2], shape[3], shape[3])) * 0.05) if state else None
    lib = _native.lib()
    assert lib.pm_linear_attention_workspace_bytes(shape[0], shape[1], shape[2], shape[3],
                                                   _native.DTYPE_F32) > 0
    qd, kd, vd = (torch.from_numpy(x).cuda() for x in (q, k, v))
    out, st = model.linear_attention(qd, kd, vd, state=None if s0 is None else torch.from_numpy(s0).cuda())
    out_r, st_r = mref.linear_attention(q, k, v, s0, dtype=np.float64)
    assert_f32_parity(out.cpu().numpy(), out_r, f"{shape} out")
    assert_f32_parity(st.cpu().numpy(), st_r, f"{shape} state")


def test_fp32_chunked_kernel_large_zero_rows_and_repeatable():
    """(2, 1000, 4, 128) fp32 against the per-token kernel, with zero and tiny q/k
    rows (the eps guard), and bitwise repeatable."""
    rng = np.random.default_rng(14)
    shape = (2, 1000, 4, 128)
    q, k, v = (torch.from_numpy(_rand(rng, shape)).cuda() for _ in range(3))
    q[0, 10, 1] = 0
    k[1, 500, 2] = 0
    k[0, 65, 0] = 1e-9
    a = model.linear_attention(q, k, v)
    old = _native.set_path(1)
    try:
        exact = model.linear_attention(q, k, v)
    finally:
        _native.set_path(old)
    for x, e, n in zip(a, exact, ("out", "state")):
        assert_f32_parity(x.cpu().numpy(), e.cpu().numpy(), n)
    assert torch.all(a[0][0, 10, 1] == 0)
    b = model.linear_attention(q, k, v)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_empty_sequence_passes_state_through():
    s0 = np.random.default_rng(13).standard_normal((2, 3, 8, 8)).astype(np.float32)
    z = np.zeros((2, 0, 3, 8), np.float32)
    out, st = model.linear_attention(z, z, z, state=s0)
    assert out.shape == (2, 0, 3, 8)
    np.testing.assert_array_equal(st, s0)


def test_linear_attn_layer():
    rng = np.random.default_rng(14)
    b, s, d, h, e = 2, 40, 96, 3, 32
    x = _rand(rng, (b, s, d))
    layer = {"W_q": _rand(rng, (d, h, e)) * 0.1, "W_k": _rand(rng, (d, h, e)) * 0.1,
             "W_v": _rand(rng, (d, h, e)) * 0.1, "W_o": _rand(rng, (h, e, d)) * 0.1}
    y, st = model._linear_attn(x, layer)
    y_r, st_r = mref.linear_attn_layer(x, layer, dtype=np.float64)
    assert y.shape == (b, s, d) and st.shape == (b, h, e, e)
    assert_f32_parity(y, y_r, "layer y")
    assert_f32_parity(st, st_r, "layer state")
    # the state carries across calls as in model._linear_attn's decode use
    y2, st2 = model._linear_attn(x[:, :7], layer)
    y3, st3 = model._linear_attn(x[:, 7:], layer, st2)
    assert_f32_parity(np.concatenate([y2, y3], axis=1), y_r, "layer split y")
    assert_f32_parity(st3, st_r, "layer split state")
