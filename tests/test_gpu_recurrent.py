"""GPU parity tests of the per-token recurrence (K4, csrc/delta_recurrent.hip)
across its geometries and load paths, against the pinned fp64 oracle
(oracle/delta_oracle.py, oracle/model_oracle.py, oracle/gated_oracle.py).

K4 splits each (sequence, head) into column groups; a thread holds 8 rows
of a column up to D = 128 and 16 rows above, and the RS row slices of a
column (RS = 1, 2, 4, 8 or 16) are summed with DPP. q/k rows are read
four elements at a time when D % 4 == 0 and the pointers are aligned
(16 bytes for fp32, 8 for bf16), else element by element. These tests
take every geometry and both load paths, partial token blocks (T not a
multiple of 16), pair counts that are not a multiple of 8, and the
model (L2-normalised) and gated modes, at the fp32 bounds.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import delta_oracle as ref
from oracle import gated_oracle as gref
from oracle import model_oracle as mref
from prometheus_amd import _native, kernels, model, synth
from tests.parity import assert_f32_parity

pytestmark = pytest.mark.gpu


def _misaligned(x: np.ndarray, dtype: torch.dtype, offset: int = 1) -> torch.Tensor:
    """x on the GPU as a contiguous view whose data starts `offset` elements into its buffer."""
    flat = torch.empty(x.size + offset, dtype=dtype, device="cuda")
    view = flat[offset:].view(x.shape)
    view.copy_(torch.from_numpy(np.ascontiguousarray(x)).to(dtype))
    return view


# (B, T, H, D): every (RPT, RS) geometry of K4, with D % 4 == 0 and != 0
GEOMETRIES = [
    (2, 17, 3, 1),     # RS 1
    (1, 33, 2, 8),     # RS 1, full slice
    (2, 15, 2, 12),    # RS 2
    (1, 40, 1, 17),    # RS 4, scalar loads
    (2, 31, 2, 48),    # RS 8
    (1, 50, 2, 100),   # RS 16
    (1, 20, 2, 129),   # RPT 16, RS 16, scalar loads
    (1, 18, 1, 160),   # RPT 16
    (1, 17, 2, 256),   # RPT 16, the largest D
]


@pytest.mark.parametrize("shape", GEOMETRIES, ids=lambda s: "x".join(map(str, s)))
def test_fp32_geometries_against_oracle(shape):
    x = synth.fwd_inputs(shape, seed=sum(shape), dtype="fp32", s0_std=0.05)
    out, st = kernels.chunked_delta_rule(x.q, x.k, x.v, x.beta, state=x.s0)
    o_r, s_r = ref.gated_delta_rule(x.q, x.k, x.v, x.beta, x.s0, dtype=np.float64)
    assert_f32_parity(out, o_r, f"{shape} O")
    assert_f32_parity(st, s_r, f"{shape} S")


@pytest.mark.parametrize("shape", [(2, 37, 2, 33), (1, 45, 3, 48), (1, 21, 2, 200)],
                         ids=lambda s: "x".join(map(str, s)))
def test_bf16_inputs_on_both_load_paths(shape):
    """bf16 q/k/v with D outside {64, 128}: K4 in fp32 arithmetic on the rounded values
    (D = 33: element loads; 48, 200: 8-byte loads)."""
    x = synth.fwd_inputs(shape, seed=7 + sum(shape), dtype="bf16", s0_std=0.02)
    bf = lambda bits: torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()  # noqa: E731
    out, st = kernels.chunked_delta_rule(bf(x.q_bits), bf(x.k_bits), bf(x.v_bits), torch.from_numpy(x.beta).cuda(),
                                         torch.from_numpy(x.s0).cuda())
    o_r, s_r = ref.gated_delta_rule(x.q, x.k, x.v, x.beta, x.s0, dtype=np.float64)
    assert_f32_parity(out.cpu().numpy(), o_r, f"{shape} O")
    assert_f32_parity(st.cpu().numpy(), s_r, f"{shape} S")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_misaligned_pointers_take_element_loads(dtype):
    """q/k/v one element into their buffers (4- or 2-byte aligned): element loads,
    same results as the aligned call (bitwise) and the oracle."""
    shape = (2, 70, 2, 64)
    x = synth.fwd_inputs(shape, seed=61, dtype="fp32")
    if dtype == torch.bfloat16:
        q, k, v = (torch.from_numpy(a).to(torch.bfloat16).float().numpy() for a in (x.q, x.k, x.v))
    else:
        q, k, v = x.q, x.k, x.v
    beta = torch.from_numpy(x.beta).cuda()
    mq, mk, mv = (_misaligned(a, dtype) for a in (q, k, v))
    assert mq.data_ptr() % 8 != 0
    old = _native.set_path(1)  # bf16 at D = 64 would otherwise fall back only when misaligned
    try:
        out_m, st_m = kernels.chunked_delta_rule(mq, mk, mv, beta)
        aq, ak, av = (torch.from_numpy(a).to(dtype).cuda() for a in (q, k, v))
        out_a, st_a = kernels.chunked_delta_rule(aq, ak, av, beta)
    finally:
        _native.set_path(old)
    assert torch.equal(out_m, out_a) and torch.equal(st_m, st_a)
    o_r, s_r = ref.gated_delta_rule(q, k, v, x.beta, None, dtype=np.float64)
    assert_f32_parity(out_m.cpu().numpy(), o_r, "O")
    assert_f32_parity(st_m.cpu().numpy(), s_r, "S")


def test_many_pairs_not_a_multiple_of_eight():
    """B*H = 303: the last slot of 8 pairs is partly empty."""
    shape = (101, 9, 3, 8)
    x = synth.fwd_inputs(shape, seed=5, dtype="fp32", s0_std=0.1)
    out, st = kernels.chunked_delta_rule(x.q, x.k, x.v, x.beta, state=x.s0)
    o_r, s_r = ref.gated_delta_rule(x.q, x.k, x.v, x.beta, x.s0, dtype=np.float64)
    assert_f32_parity(out, o_r, "O")
    assert_f32_parity(st, s_r, "S")


@pytest.mark.parametrize("d", [17, 160])
def test_model_normalisation_on_other_geometries(d):
    """pm_linear_attention on K4 (fp32): unnormalised rows, D with scalar loads and RPT 16."""
    rng = np.random.default_rng(d)
    q, k, v = (rng.standard_normal((2, 40, 2, d)).astype(np.float32) for _ in range(3))
    k[0, 3, 1] = 0.0  # the eps guard
    out, st = model.linear_attention(q, k, v)
    o_r, s_r = mref.linear_attention(q, k, v, dtype=np.float64)
    assert_f32_parity(out, o_r, f"D{d} out")
    assert_f32_parity(st, s_r, f"D{d} state")


def test_gated_on_rpt16_geometry():
    shape = (1, 37, 2, 160)
    x = synth.fwd_inputs(shape, seed=17, dtype="fp32", s0_std=0.05)
    g = (-0.3 * np.abs(np.random.default_rng(3).standard_normal(shape[:3]))).astype(np.float32)
    out, st = kernels.chunked_gated_delta_rule(x.q, x.k, x.v, x.beta, g, x.s0)
    o_r, s_r = gref.gated_delta_rule(x.q, x.k, x.v, x.beta, g, x.s0)
    assert_f32_parity(out, o_r, "O")
    assert_f32_parity(st, s_r, "S")


def test_varlen_with_empty_segments_on_k4():
    lens = [0, 19, 1, 0, 40, 16]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    x = synth.fwd_inputs((int(cu[-1]), 2, 100), seed=23, dtype="fp32")
    s0 = (np.random.default_rng(2).standard_normal((len(lens), 2, 100, 100)) * 0.02).astype(np.float32)
    out, st = kernels.chunked_delta_rule_varlen(x.q, x.k, x.v, x.beta, cu, s0)
    o_r, s_r = ref.varlen_fwd(x.q, x.k, x.v, x.beta, cu, s0, dtype=np.float64)
    assert_f32_parity(out, o_r, "packed O")
    assert_f32_parity(st, s_r, "packed S")
    np.testing.assert_array_equal(st[0], s0[0])  # empty segments pass their state through
    np.testing.assert_array_equal(st[3], s0[3])


def test_repeatable_bitwise():
    x = synth.fwd_inputs((3, 90, 4, 100), seed=29, dtype="fp32", s0_std=0.02)
    args = tuple(torch.from_numpy(a).cuda() for a in (x.q, x.k, x.v, x.beta, x.s0))
    o1, s1 = kernels.chunked_delta_rule(*args)
    o2, s2 = kernels.chunked_delta_rule(*args)
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
