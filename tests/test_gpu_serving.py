"""GPU tests of the serving-side state cache (prometheus_amd.serving) and its
slot-indexed decode step (pm_delta_step_slots).

* A decode over slots equals the plain decode step (pm_delta_step,
  kernels/__init__.py:357-376) on the gathered states, bitwise, and leaves
  every other slot bitwise untouched.
* Padding slots (negative or >= n_slots) read and write nothing, and
  give zero outputs.
* Prefill then decode, per request, equals the pinned oracle's forward
  over the whole sequence: the prompt (fixed-length and packed/varlen),
  then the decoded tokens.
* swap_out / swap_in is bitwise, and decoding resumes identically.
* A HIP-graph-captured decode, replayed with new inputs and a new slot
  table written in place between replays, matches eager decode on every
  replay.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import delta_oracle as ref
from prometheus_amd import kernels, serving, synth
from tests.parity import assert_bf16_parity, assert_f32_parity

pytestmark = pytest.mark.gpu


def _bf(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(torch.bfloat16).cuda()


def _tok(rng, b, h, d, dtype):
    q = synth.l2_normalize(rng.standard_normal((b, h, d)).astype(np.float32))
    k = synth.l2_normalize(rng.standard_normal((b, h, d)).astype(np.float32))
    v = rng.standard_normal((b, h, d)).astype(np.float32)
    beta = (1.0 / (1.0 + np.exp(-rng.standard_normal((b, h))))).astype(np.float32)
    t = (lambda x: _bf(x)) if dtype == "bf16" else (lambda x: torch.from_numpy(x).cuda())
    return t(q), t(k), t(v), torch.from_numpy(beta).cuda()


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_decode_over_slots_equals_plain_step(d, dtype):
    rng = np.random.default_rng(d)
    h, n_slots = 3, 10
    cache = serving.LinearStateCache(2, n_slots, h, d)
    cache.pool.copy_(torch.from_numpy(rng.standard_normal(cache.pool.shape).astype(np.float32) * 0.1))
    before = cache.pool.clone()
    slots = torch.tensor([7, 2, 9, 4], dtype=torch.int32, device="cuda")
    q, k, v, beta = _tok(rng, 4, h, d, dtype)
    o = cache.decode(1, slots, q, k, v, beta)
    s = before[1, slots.long()].clone()
    o_ref = kernels.delta_rule_step(q, k, v, beta, s)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref)
    assert torch.equal(cache.pool[1, slots.long()], s)
    mask = torch.ones(n_slots, dtype=torch.bool)
    mask[slots.long().cpu()] = False
    assert torch.equal(cache.pool[1][mask.cuda()], before[1][mask.cuda()])
    assert torch.equal(cache.pool[0], before[0])


def test_padding_slots_are_skipped():
    rng = np.random.default_rng(3)
    h, d, n_slots = 2, 64, 4
    cache = serving.LinearStateCache(1, n_slots, h, d)
    cache.pool.copy_(torch.from_numpy(rng.standard_normal(cache.pool.shape).astype(np.float32)))
    before = cache.pool.clone()
    slots = torch.tensor([-1, 1, n_slots, 12345], dtype=torch.int32, device="cuda")
    q, k, v, beta = _tok(rng, 4, h, d, "bf16")
    o = torch.full((4, h, d), 7.0, device="cuda")
    cache.decode(0, slots, q, k, v, beta, out=o)
    torch.cuda.synchronize()
    assert torch.all(o[[0, 2, 3]] == 0)
    assert torch.any(o[1] != 0)
    keep = torch.tensor([True, False, True, True], device="cuda")
    assert torch.equal(cache.pool[0][keep], before[0][keep])


@pytest.mark.parametrize("dtype,d", [("bf16", 128), ("bf16", 64), ("fp32", 64)])
def test_prefill_then_decode_matches_the_oracle(dtype, d):
    rng = np.random.default_rng(11 + d)
    n, t_prompt, n_dec, h = 3, 150, 6, 2
    x = synth.fwd_inputs((n, t_prompt + n_dec, h, d), seed=5 + d, dtype=dtype)
    cache = serving.LinearStateCache(1, 8, h, d)
    slots = cache.alloc(n)
    to = (lambda bits: torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()) \
        if dtype == "bf16" else (lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda())
    q = to(x.q_bits if dtype == "bf16" else x.q)
    k = to(x.k_bits if dtype == "bf16" else x.k)
    v = to(x.v_bits if dtype == "bf16" else x.v)
    beta = torch.from_numpy(x.beta).cuda()
    o_pre = cache.prefill(0, slots, q[:, :t_prompt].contiguous(), k[:, :t_prompt].contiguous(),
                          v[:, :t_prompt].contiguous(), beta[:, :t_prompt].contiguous())
    st = torch.tensor(slots, dtype=torch.int32, device="cuda")
    outs = [cache.decode(0, st, q[:, t].contiguous(), k[:, t].contiguous(), v[:, t].contiguous(),
                         beta[:, t].contiguous()) for t in range(t_prompt, t_prompt + n_dec)]
    o = torch.cat([o_pre, torch.stack(outs, dim=1)], dim=1).cpu().numpy()
    o_ref, s_ref = ref.gated_delta_rule(x.q, x.k, x.v, x.beta, None, dtype=np.float64)
    check = assert_bf16_parity if dtype == "bf16" else assert_f32_parity
    check(o, o_ref, "outputs")
    check(cache.pool[0, slots].cpu().numpy(), s_ref, "states")


def test_packed_prefill_into_slots():
    rng = np.random.default_rng(21)
    h, d = 2, 128
    lens = [70, 5, 130]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    x = synth.fwd_inputs((1, int(cu[-1]), h, d), seed=21, dtype="bf16")
    cache = serving.LinearStateCache(1, 6, h, d)
    slots = cache.alloc(3)
    s0 = (rng.standard_normal((3, h, d, d)) * 0.02).astype(np.float32)
    cache.pool[0, torch.tensor(slots).cuda()] = torch.from_numpy(s0).cuda()
    bf = lambda bits: torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()
    o = cache.prefill(0, slots, bf(x.q_bits), bf(x.k_bits), bf(x.v_bits), torch.from_numpy(x.beta).cuda(),
                      cu_seqlens=torch.from_numpy(cu).cuda())
    o_ref, s_ref = ref.varlen_fwd(x.q[0], x.k[0], x.v[0], x.beta[0], cu, s0, dtype=np.float64)
    assert o.shape == (1, int(cu[-1]), h, d)
    assert_bf16_parity(o[0].cpu().numpy(), o_ref, "packed outputs")
    assert_bf16_parity(cache.pool[0, slots].cpu().numpy(), s_ref, "packed states")


def test_swap_out_and_in_resume_identically():
    rng = np.random.default_rng(31)
    h, d = 2, 64
    cache = serving.LinearStateCache(3, 5, h, d)
    slots = cache.alloc(2)
    cache.pool.copy_(torch.from_numpy(rng.standard_normal(cache.pool.shape).astype(np.float32) * 0.1))
    saved = cache.swap_out(slots)
    assert saved.device.type == "cpu" and saved.is_pinned()
    st = torch.tensor(slots, dtype=torch.int32, device="cuda")
    q, k, v, beta = _tok(rng, 2, h, d, "bf16")
    o1 = cache.decode(2, st, q, k, v, beta).clone()
    after1 = cache.pool[:, slots].clone()
    cache.reset(slots)
    assert torch.count_nonzero(cache.pool[:, slots]) == 0
    cache.swap_in(slots, saved)
    o2 = cache.decode(2, st, q, k, v, beta)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert torch.equal(cache.pool[:, slots], after1)


def test_graph_captured_decode_replays():
    rng = np.random.default_rng(41)
    h, d, n_slots, b = 4, 128, 12, 6
    cache = serving.LinearStateCache(1, n_slots, h, d)
    cache.pool.copy_(torch.from_numpy(rng.standard_normal(cache.pool.shape).astype(np.float32) * 0.05))
    slots = torch.tensor([0, 3, 5, -1, 8, 11], dtype=torch.int32, device="cuda")
    q, k, v, beta = _tok(rng, b, h, d, "bf16")
    out = torch.empty((b, h, d), device="cuda")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        cache.decode(0, slots, q, k, v, beta, out=out)  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        cache.decode(0, slots, q, k, v, beta, out=out)
    for rep in range(4):
        # new tokens and a new slot table, written in place
        nq, nk, nv, nb = _tok(rng, b, h, d, "bf16")
        q.copy_(nq), k.copy_(nk), v.copy_(nv), beta.copy_(nb)
        perm = rng.permutation(n_slots)[:b].astype(np.int32)
        perm[rep % b] = -1
        slots.copy_(torch.from_numpy(perm).cuda())
        pool_before = cache.pool.clone()
        graph.replay()
        torch.cuda.synchronize()
        got_out, got_pool = out.clone(), cache.pool.clone()
        cache.pool.copy_(pool_before)
        want = cache.decode(0, slots, q, k, v, beta)
        torch.cuda.synchronize()
        assert torch.equal(got_out, want), rep
        assert torch.equal(got_pool, cache.pool), rep


def test_graph_captured_packed_prefill_replays():
    """prefill with GPU slots and GPU cu_seqlens under HIP graph capture: nothing in it
    synchronises with the host (the offsets are checked on the device), and every replay,
    with new tokens, offsets and slots written in place between replays, equals the eager
    prefill of the same inputs bit for bit (outputs and the whole pool)."""
    rng = np.random.default_rng(51)
    h, d, n_slots, n_tok = 2, 128, 8, 400
    cache = serving.LinearStateCache(1, n_slots, h, d)
    cache.pool.copy_(torch.from_numpy(rng.standard_normal(cache.pool.shape).astype(np.float32) * 0.02))
    slots = torch.tensor([1, 4, 6], dtype=torch.int64, device="cuda")
    cu = torch.tensor([0, 150, 151, n_tok], dtype=torch.int32, device="cuda")

    def tokens(seed):
        x = synth.fwd_inputs((1, n_tok, h, d), seed=seed, dtype="bf16")
        bf = lambda b: torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).cuda()
        return bf(x.q_bits), bf(x.k_bits), bf(x.v_bits), torch.from_numpy(x.beta).cuda()

    q, k, v, beta = tokens(51)
    kernels.check_varlen()  # the device flag word exists before capture
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        cache.prefill(0, slots, q, k, v, beta, cu_seqlens=cu)  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        o_graph = cache.prefill(0, slots, q, k, v, beta, cu_seqlens=cu)
    for rep in range(4):
        nq, nk, nv, nb = tokens(60 + rep)
        q.copy_(nq), k.copy_(nk), v.copy_(nv), beta.copy_(nb)
        a = int(rng.integers(0, n_tok))
        z = int(rng.integers(a, n_tok + 1))
        cu.copy_(torch.tensor([0, a, z, n_tok], dtype=torch.int32))
        slots.copy_(torch.from_numpy(rng.permutation(n_slots)[:3].astype(np.int64)))
        pool_before = cache.pool.clone()
        graph.replay()
        torch.cuda.synchronize()
        got_o, got_pool = o_graph.clone(), cache.pool.clone()
        cache.pool.copy_(pool_before)
        want = cache.prefill(0, slots, q, k, v, beta, cu_seqlens=cu)
        torch.cuda.synchronize()
        assert torch.equal(got_o, want), rep
        assert torch.equal(got_pool, cache.pool), rep
    kernels.check_varlen()
    cache.check_slots()


def test_device_offsets_and_slots_are_checked_lazily():
    """A malformed GPU cu_seqlens is reported by check_varlen (then cleared); an out-of-range
    GPU slot computes into the spare slot, leaves every pool slot but the valid ones
    untouched, and is reported by check_slots."""
    rng = np.random.default_rng(52)
    h, d, n_slots, n_tok = 2, 64, 6, 200
    cache = serving.LinearStateCache(1, n_slots, h, d)
    cache.pool.copy_(torch.from_numpy(rng.standard_normal(cache.pool.shape).astype(np.float32) * 0.02))
    x = synth.fwd_inputs((1, n_tok, h, d), seed=52, dtype="bf16")
    bf = lambda b: torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).cuda()
    q, k, v, beta = bf(x.q_bits), bf(x.k_bits), bf(x.v_bits), torch.from_numpy(x.beta).cuda()
    kernels.check_varlen()
    cache.check_slots()
    for bad, what in (([0, 120, 80, n_tok], "decreasing"), ([5, 80, 120, n_tok], r"cu_seqlens\[0\]"),
                      ([0, 80, 120, n_tok - 1], r"cu_seqlens\[-1\]"), ([0, -3, 120, n_tok], "outside")):
        cache.prefill(0, [0, 1, 2], q, k, v, beta,
                      cu_seqlens=torch.tensor(bad, dtype=torch.int32, device="cuda"))
        with pytest.raises(kernels.KernelError, match=what):
            kernels.check_varlen()
        kernels.check_varlen()  # cleared
    good = torch.tensor([0, 70, 71, n_tok], dtype=torch.int32, device="cuda")
    before = cache.pool.clone()
    cache.prefill(0, torch.tensor([3, 99, 5], device="cuda"), q, k, v, beta, cu_seqlens=good)
    with pytest.raises(ValueError, match="outside"):
        cache.check_slots()
    cache.check_slots()  # cleared
    changed = {i for i in range(n_slots) if not torch.equal(before[0, i], cache.pool[0, i])}
    assert changed == {3, 5}
