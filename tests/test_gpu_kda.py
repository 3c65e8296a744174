"""GPU parity tests of the per-channel gated delta rule (KDA: kernels.chunked_kda_rule,
kernels.kda_delta_rule_step) against the pinned KDA oracle (oracle/gated_oracle.py:
kda_delta_rule, pinned by its reduction to the scalar gate, closed forms, an
independent chunked form and planted mistakes).

* fp32 inputs on the benchmark distribution: the per-token kernel at the fp32
  bounds, D from 2 to 256, with and without S0, weak to strong decay.
* bf16 inputs (fp32 and bf16 outputs): the bf16 bound on the same rounded inputs.
* g = 0 is bitwise the ungated per-token kernel (alpha = 1 scales exactly); g
  constant along D matches the scalar-gated kernel at the fp32 bounds.
* The KDA step (K3 for D in {32, 64, 128}, else the per-token kernel) run token by
  token against the oracle and against the per-token forward; T = 0, misaligned
  gates, path 2 and scalar-gate shapes refused.
* The chunked WY form (bf16 q/k/v, D in {64, 128}): against the oracle at the bf16
  bound (one token, partial and ragged chunks, with and without S0, weak and strong
  decay, channels decayed to nothing next to undecayed ones, slightly positive gates,
  bf16 O), against the per-token kernel on the same inputs over long sequences,
  bitwise repeatable, and g constant along D against the scalar-gated chunked kernel.
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


def _gates(seed, shape, scale):
    return (-scale * np.abs(np.random.default_rng(seed).standard_normal(shape))).astype(np.float32)


@pytest.mark.parametrize("shape", [(1, 1, 1, 2), (2, 37, 2, 8), (1, 50, 3, 32), (2, 40, 2, 64),
                                   (1, 33, 2, 100), (1, 45, 2, 128), (1, 20, 1, 256)])
@pytest.mark.parametrize("state", [False, True])
@pytest.mark.parametrize("scale", [0.05, 1.0])
def test_fp32_against_oracle(shape, state, scale):
    x = synth.fwd_inputs(shape, seed=sum(shape) + state, dtype="fp32", s0_std=0.02 if state else None)
    g = _gates(sum(shape) + 7, shape, scale)
    o, s = kernels.chunked_kda_rule(x.q, x.k, x.v, x.beta, g, x.s0)
    o_r, s_r = gref.kda_delta_rule(x.q, x.k, x.v, x.beta, g, x.s0)
    assert_f32_parity(o, o_r, f"{shape} O")
    assert_f32_parity(s, s_r, f"{shape} S")


@pytest.mark.parametrize("shape", [(2, 70, 2, 64), (1, 129, 2, 128)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_bf16_inputs_against_oracle(shape, out_dtype):
    x = synth.fwd_inputs(shape, seed=11, dtype="bf16", s0_std=0.02)
    g = torch.from_numpy(_gates(12, shape, 0.3)).cuda()
    o, s = kernels.chunked_kda_rule(_bits(x.q_bits), _bits(x.k_bits), _bits(x.v_bits),
                                    torch.from_numpy(x.beta).cuda(), g, torch.from_numpy(x.s0).cuda(),
                                    out_dtype=out_dtype)
    assert o.dtype == out_dtype
    o_r, s_r = gref.kda_delta_rule(x.q, x.k, x.v, x.beta, g.cpu().numpy(), x.s0)
    assert_bf16_parity(o.float().cpu().numpy(), o_r, f"{shape} O")
    assert_bf16_parity(s.cpu().numpy(), s_r, f"{shape} S")


def test_zero_gate_is_bitwise_the_ungated_per_token_kernel():
    shape = (2, 90, 2, 128)
    x = synth.fwd_inputs(shape, seed=13, dtype="fp32", s0_std=0.02)
    o, s = kernels.chunked_kda_rule(x.q, x.k, x.v, x.beta, np.zeros(shape, np.float32), x.s0)
    with _native.use_knobs(1, 0):  # the per-token kernel
        o2, s2 = kernels.chunked_delta_rule(x.q, x.k, x.v, x.beta, x.s0)
    assert np.array_equal(o, o2) and np.array_equal(s, s2)


@pytest.mark.parametrize("dim", [16, 64, 128])
def test_channel_constant_gate_is_the_scalar_gate(dim):
    shape = (2, 60, 2, dim)
    x = synth.fwd_inputs(shape, seed=dim, dtype="fp32", s0_std=0.02)
    g = _gates(dim + 1, shape[:3], 0.5)
    o, s = kernels.chunked_kda_rule(x.q, x.k, x.v, x.beta, np.repeat(g[..., None], dim, axis=-1), x.s0)
    o2, s2 = kernels.chunked_gated_delta_rule(x.q, x.k, x.v, x.beta, g, x.s0)
    assert_f32_parity(o, o2, "O")
    assert_f32_parity(s, s2, "S")


def test_strong_and_uneven_decay_stays_finite():
    """Channels from no decay (g = 0) to g = -30 (alpha ~ 1e-13) in one head."""
    shape = (1, 64, 2, 64)
    x = synth.fwd_inputs(shape, seed=21, dtype="fp32", s0_std=0.02)
    g = np.zeros(shape, np.float32)
    g[..., ::2] = -30.0
    g[..., 1::4] = -0.01
    o, s = kernels.chunked_kda_rule(x.q, x.k, x.v, x.beta, g, x.s0)
    o_r, s_r = gref.kda_delta_rule(x.q, x.k, x.v, x.beta, g, x.s0)
    assert_f32_parity(o, o_r, "O")
    assert_f32_parity(s, s_r, "S")


def test_misaligned_gates_take_the_element_loads():
    """A g view 4 bytes past a 16-byte boundary: the kernel's 16-byte row loads are off."""
    shape = (1, 40, 2, 64)
    x = synth.fwd_inputs(shape, seed=22, dtype="fp32", s0_std=0.02)
    g_np = _gates(23, shape, 0.4)
    buf = torch.empty(g_np.size + 1, dtype=torch.float32, device="cuda")
    g = buf[1:].view(shape)
    g.copy_(torch.from_numpy(g_np))
    assert g.data_ptr() % 16 != 0
    dev = [torch.from_numpy(a).cuda() for a in (x.q, x.k, x.v, x.beta, x.s0)]
    o, s = kernels.chunked_kda_rule(dev[0], dev[1], dev[2], dev[3], g, dev[4])
    o2, s2 = kernels.chunked_kda_rule(dev[0], dev[1], dev[2], dev[3], g.contiguous().clone(), dev[4])
    assert torch.equal(o, o2) and torch.equal(s, s2)
    o_r, s_r = gref.kda_delta_rule(x.q, x.k, x.v, x.beta, g_np, x.s0)
    assert_f32_parity(o.cpu().numpy(), o_r, "O")
    assert_f32_parity(s.cpu().numpy(), s_r, "S")


@pytest.mark.parametrize("dim", [32, 64, 128, 48, 256])
@pytest.mark.parametrize("in_dtype", ["fp32", "bf16"])
def test_step_against_oracle_and_forward(dim, in_dtype):
    """T steps from S0 (K3 for D in {32, 64, 128}, the per-token kernel otherwise)
    against the oracle, and against the forward on the same tokens."""
    b, t, h = 2, 12, 3
    x = synth.fwd_inputs((b, t, h, dim), seed=dim, dtype=in_dtype, s0_std=0.02)
    g = _gates(dim + 3, (b, t, h, dim), 0.3)
    if in_dtype == "bf16":
        q, k, v = _bits(x.q_bits), _bits(x.k_bits), _bits(x.v_bits)
    else:
        q, k, v = (torch.from_numpy(a).cuda() for a in (x.q, x.k, x.v))
    beta, gd = torch.from_numpy(x.beta).cuda(), torch.from_numpy(g).cuda()
    state = torch.from_numpy(x.s0).cuda().clone()
    outs = []
    for i in range(t):
        outs.append(kernels.kda_delta_rule_step(q[:, i].contiguous(), k[:, i].contiguous(), v[:, i].contiguous(),
                                                beta[:, i].contiguous(), gd[:, i].contiguous(), state))
    o = torch.stack(outs, dim=1).cpu().numpy()
    o_r, s_r = gref.kda_delta_rule(x.q, x.k, x.v, x.beta, g, x.s0)
    assert_f32_parity(o, o_r, "steps O")
    assert_f32_parity(state.cpu().numpy(), s_r, "steps S")
    with _native.use_knobs(1, 0):  # the per-token forward: the steps' arithmetic
        of, sf = kernels.chunked_kda_rule(q, k, v, beta, gd, torch.from_numpy(x.s0).cuda())
    assert_f32_parity(o, of.cpu().numpy(), "steps vs forward O")
    assert_f32_parity(state.cpu().numpy(), sf.cpu().numpy(), "steps vs forward S")


def test_no_tokens_passes_the_state_through():
    x = synth.fwd_inputs((2, 0, 2, 64), seed=1, dtype="fp32", s0_std=0.02)
    o, s = kernels.chunked_kda_rule(x.q, x.k, x.v, x.beta, np.zeros((2, 0, 2, 64), np.float32), x.s0)
    assert o.shape == (2, 0, 2, 64)
    assert np.array_equal(s, x.s0)


def test_path_2_and_bad_gate_shapes_are_refused():
    """Path 2 requires the chunked form, which takes bf16 q/k/v with D in {64, 128}."""
    x = synth.fwd_inputs((1, 8, 1, 64), seed=2, dtype="bf16")
    g = torch.zeros((1, 8, 1, 64), device="cuda")
    args = (_bits(x.q_bits), _bits(x.k_bits), _bits(x.v_bits), torch.from_numpy(x.beta).cuda(), g)
    xf = [torch.from_numpy(a).cuda() for a in (x.q, x.k, x.v)]
    with _native.use_knobs(2, 0), pytest.raises(_native.NativeError, match="needs bf16") as ei:
        kernels.chunked_kda_rule(*xf, args[3], g)
    assert ei.value.code == _native.E_UNSUPPORTED
    with _native.use_knobs(2, 0):
        o, _ = kernels.chunked_kda_rule(*args)  # bf16 D = 64: the chunked form
    assert torch.isfinite(o).all()
    with pytest.raises(kernels.KernelError, match="g shape"):
        kernels.chunked_kda_rule(*args[:4], g[..., :32])


# --- the chunked WY form (bf16 q/k/v, D in {64, 128}) ---


def _bf16_kda(shape, seed, scale, state, positive=None):
    x = synth.fwd_inputs(shape, seed=seed, dtype="bf16", s0_std=0.02 if state else None)
    g = _gates(seed + 1, shape, scale) if positive is None else np.full(shape, positive, np.float32)
    return x, g


def _run_chunked(x, g, out_dtype=None):
    return kernels.chunked_kda_rule(_bits(x.q_bits), _bits(x.k_bits), _bits(x.v_bits),
                                    torch.from_numpy(x.beta).cuda(), torch.from_numpy(g).cuda(),
                                    None if x.s0 is None else torch.from_numpy(x.s0).cuda(), out_dtype=out_dtype)


@pytest.mark.parametrize("shape", [(1, 1, 1, 64), (2, 77, 3, 64), (1, 200, 2, 128), (2, 130, 1, 128),
                                   (1, 64, 2, 128)])
@pytest.mark.parametrize("state", [False, True])
@pytest.mark.parametrize("scale", [0.1, 3.0])
def test_chunked_against_oracle(shape, state, scale):
    x, g = _bf16_kda(shape, sum(shape) + 3 * state, scale, state)
    o, s = _run_chunked(x, g)
    o_r, s_r = gref.kda_delta_rule(x.q, x.k, x.v, x.beta, g, x.s0)
    assert_bf16_parity(o.cpu().numpy(), o_r, f"{shape} O")
    assert_bf16_parity(s.cpu().numpy(), s_r, f"{shape} S")


def test_chunked_strong_and_uneven_decay():
    """Channels at g = -30 (beyond the chunked form's clamp at -10) next to undecayed
    ones and mild ones: within the bf16 bound of the unclamped oracle."""
    shape = (2, 190, 2, 128)
    x = synth.fwd_inputs(shape, seed=31, dtype="bf16", s0_std=0.02)
    g = np.zeros(shape, np.float32)
    g[..., ::2] = -30.0
    g[..., 1::4] = -0.01
    g[:, 100:110] = -12.0
    o, s = _run_chunked(x, g)
    o_r, s_r = gref.kda_delta_rule(x.q, x.k, x.v, x.beta, g, x.s0)
    assert_bf16_parity(o.cpu().numpy(), o_r, "O")
    assert_bf16_parity(s.cpu().numpy(), s_r, "S")


def test_chunked_slightly_positive_gates():
    x, g = _bf16_kda((1, 150, 2, 64), 32, 0.0, True, positive=0.01)
    o, s = _run_chunked(x, g)
    o_r, s_r = gref.kda_delta_rule(x.q, x.k, x.v, x.beta, g, x.s0)
    assert_bf16_parity(o.cpu().numpy(), o_r, "O")
    assert_bf16_parity(s.cpu().numpy(), s_r, "S")


@pytest.mark.parametrize("shape", [(2, 1000, 4, 128), (3, 700, 2, 64)])
def test_chunked_against_the_per_token_kernel(shape):
    """Long sequences: chunked against the per-token kernel on the same bf16 inputs (the
    fp32 recurrence), and bitwise repeatable."""
    x, g = _bf16_kda(shape, 33, 0.2, True)
    o, s = _run_chunked(x, g)
    o2, s2 = _run_chunked(x, g)
    assert torch.equal(o, o2) and torch.equal(s, s2)
    with _native.use_knobs(1, 0):
        o1, s1 = _run_chunked(x, g)
    assert_bf16_parity(o.cpu().numpy(), o1.cpu().numpy(), "O vs per-token")
    assert_bf16_parity(s.cpu().numpy(), s1.cpu().numpy(), "S vs per-token")


def test_chunked_channel_constant_gate_matches_the_scalar_gated_kernel():
    shape = (2, 300, 2, 128)
    x = synth.fwd_inputs(shape, seed=34, dtype="bf16", s0_std=0.02)
    g1 = _gates(35, shape[:3], 0.3)
    o, s = _run_chunked(x, np.repeat(g1[..., None], 128, axis=-1))
    o2, s2 = kernels.chunked_gated_delta_rule(_bits(x.q_bits), _bits(x.k_bits), _bits(x.v_bits),
                                              torch.from_numpy(x.beta).cuda(), torch.from_numpy(g1).cuda(),
                                              torch.from_numpy(x.s0).cuda())
    assert_bf16_parity(o.cpu().numpy(), o2.cpu().numpy(), "O")
    assert_bf16_parity(s.cpu().numpy(), s2.cpu().numpy(), "S")


def test_chunked_bf16_output():
    x, g = _bf16_kda((2, 150, 2, 128), 36, 0.3, True)
    o, s = _run_chunked(x, g, out_dtype=torch.bfloat16)
    o32, s32 = _run_chunked(x, g)
    assert o.dtype == torch.bfloat16
    assert torch.equal(o, o32.to(torch.bfloat16)) and torch.equal(s, s32)
