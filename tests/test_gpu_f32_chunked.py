"""GPU parity tests of the fp32 chunked forward (fp32 q/k/v, D in {64, 128}: a
parallel pass building each 16-token chunk's T and P, then the chunk
recurrence on fp32 MFMA).

Against the fp32 oracle at the fp32 bounds (rel-L2 <= 1e-5, max-abs <= 1e-4,
tests/parity.py): the NumPy oracle on small shapes, the C restatement at the
full cfg1 shape, and the per-token kernel (path 1) on the same inputs.  Bit for
bit: repeats, the two tile widths (each 16 state columns run the same
arithmetic), a varlen batch against its segments run alone, and graph replay.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import delta_oracle as ref
from prometheus_amd import _native, kernels, synth
from tests.parity import assert_f32_parity

pytestmark = pytest.mark.gpu

CPU_THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


def _np(x):
    return x.detach().cpu().numpy()


def _dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()


class _path:
    def __init__(self, path, tile=0):
        self.path, self.tile = path, tile

    def __enter__(self):
        self.old = _native.set_path(self.path)
        self.old_tile = _native.set_tile(self.tile)

    def __exit__(self, *exc):
        _native.set_path(self.old)
        _native.set_tile(self.old_tile)


def _case(shape, seed, s0_std=None):
    x = synth.fwd_inputs(shape, seed=seed, dtype="fp32", s0_std=s0_std)
    return x, (_dev(x.q), _dev(x.k), _dev(x.v), _dev(x.beta), _dev(x.s0))


@pytest.mark.parametrize("shape", [(1, 256, 4, 64), (2, 300, 3, 128), (1, 17, 2, 128), (1, 5, 1, 64),
                                   (2, 1000, 4, 64), (1, 64, 1, 128), (3, 33, 2, 64)])
@pytest.mark.parametrize("state", [False, True])
def test_f32_chunked_vs_oracle(shape, state):
    x, (q, k, v, b, s0) = _case(shape, seed=sum(shape) + state, s0_std=0.02 if state else None)
    with _path(2):  # the fp32 chunked forward, required
        o, s = kernels.chunked_delta_rule(q, k, v, b, s0)
    e_o, e_s = ref.chunked_fwd_rank1(x.q, x.k, x.v, x.beta, x.s0, 64, dtype=np.float64)
    assert_f32_parity(_np(o), e_o, f"{shape} O")
    assert_f32_parity(_np(s), e_s, f"{shape} S")


def test_f32_chunked_is_the_default_and_matches_the_per_token_kernel():
    x, (q, k, v, b, s0) = _case((2, 700, 4, 128), seed=5, s0_std=0.02)
    o_d, s_d = kernels.chunked_delta_rule(q, k, v, b, s0)
    with _path(2):
        o_c, s_c = kernels.chunked_delta_rule(q, k, v, b, s0)
    with _path(1):
        o_r, s_r = kernels.chunked_delta_rule(q, k, v, b, s0)
    assert torch.equal(o_d, o_c) and torch.equal(s_d, s_c)
    assert_f32_parity(_np(o_c), _np(o_r), "chunked vs per-token O")
    assert_f32_parity(_np(s_c), _np(s_r), "chunked vs per-token S")


@pytest.mark.parametrize("d", [64, 128])
def test_f32_chunked_tiles_and_repeats_are_bitwise(d):
    _, (q, k, v, b, s0) = _case((2, 150, 2, d), seed=d, s0_std=0.02)
    with _path(2, 16):
        o16, s16 = kernels.chunked_delta_rule(q, k, v, b, s0)
        o16b, s16b = kernels.chunked_delta_rule(q, k, v, b, s0)
    with _path(2, 32):
        o32, s32 = kernels.chunked_delta_rule(q, k, v, b, s0)
    assert torch.equal(o16, o16b) and torch.equal(s16, s16b)
    assert torch.equal(o16, o32) and torch.equal(s16, s32)


def test_f32_chunked_bf16_output():
    x, (q, k, v, b, _) = _case((1, 200, 2, 128), seed=3)
    with _path(2):
        o32, s32 = kernels.chunked_delta_rule(q, k, v, b)
        o16, s16 = kernels.chunked_delta_rule(q, k, v, b, out_dtype=torch.bfloat16)
    assert o16.dtype == torch.bfloat16 and torch.equal(s16, s32)
    assert torch.equal(o16, o32.to(torch.bfloat16))


def test_f32_chunked_cfg1_shape_vs_c_oracle():
    from oracle import cref

    x, (q, k, v, b, _) = _case((4, 4096, 16, 128), seed=41)
    o, s = kernels.chunked_delta_rule(q, k, v, b)
    e_o, e_s = cref.delta_fwd(x.q, x.k, x.v, x.beta, None, threads=CPU_THREADS)
    assert_f32_parity(_np(o), e_o, "cfg1 fp32 O")
    assert_f32_parity(_np(s), e_s, "cfg1 fp32 S")


def test_f32_chunked_varlen_segments_and_oracle():
    lens = [16, 1, 0, 130, 700, 33, 257]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    n = int(cu[-1])
    x = synth.fwd_inputs((1, n, 3, 128), seed=77, dtype="fp32")
    q, k, v, b = (_dev(a) for a in (x.q, x.k, x.v, x.beta))
    cu_d = torch.from_numpy(cu).cuda()
    o, s = kernels.chunked_delta_rule_varlen(q, k, v, b, cu_d)
    o, s = _np(o), _np(s)
    for i, (a, z) in enumerate(zip(cu[:-1], cu[1:])):
        if z == a:
            np.testing.assert_array_equal(s[i], 0.0)
            continue
        o1, s1 = kernels.chunked_delta_rule(q[:, a:z].contiguous(), k[:, a:z].contiguous(),
                                            v[:, a:z].contiguous(), b[:, a:z].contiguous())
        np.testing.assert_array_equal(o[:, a:z], _np(o1), err_msg=f"segment {i} O")
        np.testing.assert_array_equal(s[i], _np(s1)[0], err_msg=f"segment {i} S")
        if i in (0, 3, 6):
            e_o, e_s = ref.chunked_fwd_rank1(x.q[:, a:z], x.k[:, a:z], x.v[:, a:z], x.beta[:, a:z], None, 64,
                                              dtype=np.float64)
            assert_f32_parity(o[:, a:z], e_o, f"segment {i} O")
            assert_f32_parity(s[i], e_s[0], f"segment {i} S")


def test_f32_chunked_graph_replay_is_bitwise():
    B, T, H, D = 2, 256, 4, 128
    _, (q, k, v, b, s0) = _case((B, T, H, D), seed=12, s0_std=0.02)
    lib = _native.lib()
    nb = lib.pm_delta_workspace_bytes(B, T, H, D, _native.DTYPE_F32)
    assert nb == B * H * (T // 16) * 1024
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
    o = torch.empty((B, T, H, D), device="cuda")
    s = torch.empty((B, H, D, D), device="cuda")
    st = torch.cuda.Stream()

    def launch():
        rc = lib.pm_delta_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), b.data_ptr(), s0.data_ptr(),
                              o.data_ptr(), s.data_ptr(), B, T, H, D, _native.DTYPE_F32, _native.DTYPE_F32,
                              64, ctypes.c_void_p(ws.data_ptr()), nb, ctypes.c_void_p(st.cuda_stream))
        assert rc == 0

    with torch.cuda.stream(st):
        launch()
    torch.cuda.synchronize()
    o1, s1 = o.clone(), s.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        launch()
    for _ in range(3):
        o.zero_()
        s.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, o1) and torch.equal(s, s1)


def test_f32_chunked_t0_and_empty_batch():
    _, (q, k, v, b, s0) = _case((2, 0, 2, 64), seed=1, s0_std=0.02)
    with _path(2):
        o, s = kernels.chunked_delta_rule(q, k, v, b, s0)
    assert o.shape == (2, 0, 2, 64)
    assert torch.equal(s, s0)
