"""GPU test of pm_delta_bwd_noalloc, the backward with the library's fixed scratch.

Called through the C ABI and compared with pm_delta_bwd (caller workspace) on
the same inputs: the kernels are the same, so the five gradients must be
equal bit for bit. Two calls in a row, the second with a smaller problem,
for the chunked bf16 backward and for the per-token fp32 one; the scratch
keeps the previous call's contents, which the kernels must not depend on.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from prometheus_amd import _native, synth

pytestmark = pytest.mark.gpu


def _grads(entry, x, dtype, B, T, H, D, side_stream=None):
    dev = torch.device("cuda", 0)
    f32 = torch.float32
    if dtype == _native.DTYPE_BF16:
        q, k, v = (torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).to(dev) for b in (x.q_bits, x.k_bits, x.v_bits))
    else:
        q, k, v = (torch.from_numpy(a).to(dev) for a in (x.q, x.k, x.v))
    beta = torch.from_numpy(x.beta).to(dev)
    s0 = torch.from_numpy(x.s0).to(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(B * 1000 + T)
    go = torch.randn((B, T, H, D), generator=g, device=dev)
    gs = torch.randn((B, H, D, D), generator=g, device=dev) * 0.05
    gq, gk, gv = (torch.full((B, T, H, D), float("nan"), device=dev) for _ in range(3))
    gb = torch.full((B, T, H), float("nan"), device=dev)
    gs0 = torch.full((B, H, D, D), float("nan"), device=dev)
    L = _native.lib()
    stream = torch.cuda.current_stream(dev) if side_stream is None else side_stream
    st = stream.cuda_stream
    ptrs = [t.data_ptr() for t in (q, k, v, beta, s0, go, gs, gq, gk, gv, gb, gs0)]
    if side_stream is not None:
        side_stream.wait_stream(torch.cuda.current_stream(dev))  # inputs written on the default stream
    if entry == "noalloc":
        rc = L.pm_delta_bwd_noalloc(*ptrs, B, T, H, D, dtype, st)
    else:
        nbytes = L.pm_delta_bwd_workspace_bytes(B, T, H, D, dtype)
        ws = torch.empty(((nbytes + 3) // 4,), dtype=f32, device=dev)
        rc = L.pm_delta_bwd(*ptrs, B, T, H, D, dtype, ws.data_ptr(), nbytes, st)
    _native.check(rc)
    torch.cuda.synchronize()
    return [t.cpu() for t in (gq, gk, gv, gb, gs0)]


@pytest.mark.parametrize("dtype,shapes", [
    (_native.DTYPE_BF16, [(2, 300, 3, 128), (1, 70, 2, 64)]),
    (_native.DTYPE_F32, [(2, 130, 2, 64), (1, 40, 1, 16)]),
])
def test_noalloc_backward_equals_the_workspace_entry_point(dtype, shapes):
    L = _native.lib()
    for B, T, H, D in shapes:  # the second call is smaller than the first
        need = L.pm_delta_bwd_workspace_bytes(B, T, H, D, dtype)
        assert 0 < need <= _native.NOALLOC_SCRATCH_BYTES
        x = synth.fwd_inputs((B, T, H, D), seed=B + T + D, dtype="bf16" if dtype else "fp32", s0_std=0.02)
        ref = _grads("workspace", x, dtype, B, T, H, D)
        got = _grads("noalloc", x, dtype, B, T, H, D)
        for name, a, b in zip(("gq", "gk", "gv", "gbeta", "gs0"), got, ref):
            assert torch.isfinite(a).all(), name
            assert torch.equal(a, b), (name, (B, T, H, D))


def test_noalloc_on_a_side_stream():
    """The cached scratch address serves a call on a stream other than the current one."""
    B, T, H, D = 1, 200, 2, 128
    x = synth.fwd_inputs((B, T, H, D), seed=5, dtype="bf16", s0_std=0.02)
    ref = _grads("workspace", x, _native.DTYPE_BF16, B, T, H, D)
    side = torch.cuda.Stream()
    got = _grads("noalloc", x, _native.DTYPE_BF16, B, T, H, D, side_stream=side)
    for name, a, b in zip(("gq", "gk", "gv", "gbeta", "gs0"), got, ref):
        assert torch.equal(a, b), name


def test_noalloc_refuses_problems_beyond_its_scratch():
    """cfg1's chunked backward needs about 411 MB of workspace: the no-allocation entry point
    returns E_WORKSPACE before launching anything, and the outputs keep their contents.
    (The buffers are full-size, so nothing could reach beyond them in any case.)"""
    B, T, H, D = 4, 4096, 16, 128
    L = _native.lib()
    need = L.pm_delta_bwd_workspace_bytes(B, T, H, D, _native.DTYPE_BF16)
    assert need > _native.NOALLOC_SCRATCH_BYTES
    dev = torch.device("cuda", 0)
    q, k, v = (torch.zeros((B, T, H, D), dtype=torch.bfloat16, device=dev) for _ in range(3))
    beta = torch.full((B, T, H), 0.5, device=dev)
    go = torch.zeros((B, T, H, D), device=dev)
    gs = torch.zeros((B, H, D, D), device=dev)
    outs = [torch.full((B, T, H, D), 7.0, device=dev) for _ in range(3)]
    gb = torch.full((B, T, H), 7.0, device=dev)
    gs0 = torch.full((B, H, D, D), 7.0, device=dev)
    torch.cuda.synchronize()
    rc = L.pm_delta_bwd_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), None,
                                go.data_ptr(), gs.data_ptr(), *(t.data_ptr() for t in outs),
                                gb.data_ptr(), gs0.data_ptr(), B, T, H, D, _native.DTYPE_BF16,
                                torch.cuda.current_stream(dev).cuda_stream)
    assert rc == _native.E_WORKSPACE
    assert b"workspace" in L.pm_last_error()
    torch.cuda.synchronize()
    for t in (*outs, gb, gs0):
        assert bool((t == 7.0).all())
