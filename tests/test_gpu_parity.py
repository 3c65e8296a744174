"""GPU parity tests: the HIP kernels against the pinned CPU oracle.

Every test runs the product path (``prometheus_amd.kernels`` -> the C ABI
of ``libpmdelta.so`` -> gfx950 kernels) and compares with ``oracle/`` on the
same seeded inputs, at the BASELINE tolerances (``tests/parity.py``):
fp32 inputs rel-L2 <= 1e-5 / max-abs <= 1e-4, bf16 inputs rel-L2 <= 2e-2
against the fp32 recurrence on the bf16-rounded inputs. Integer work
(cu_seqlens segmentation, state carry at chunk-aligned splits, graph
replay, repeated calls) is checked bit for bit.

The reference's own hot-path tests (tests/test_kernels.py:265-481,
:1537-1548; tests/test_kernels_delta_fwd_jit.py:246-420) are mirrored
against the build's API.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import delta_oracle as ref
from prometheus_amd import _native, kernels, synth
from tests.golden.make_golden import reference_cases
from tests.parity import assert_bf16_parity, assert_f32_parity, rel_l2

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TOL = dict(rtol=1e-5, atol=1e-5)
CPU_THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


def _np(x):
    return x.detach().cpu().numpy() if isinstance(x, torch.Tensor) else np.asarray(x)


def _bf16_dev(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def _dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _bf16_case(shape, seed, s0_std=None):
    x = synth.fwd_inputs(shape, seed=seed, dtype="bf16", s0_std=s0_std)
    dev = (_bf16_dev(x.q_bits), _bf16_dev(x.k_bits), _bf16_dev(x.v_bits), _dev(x.beta),
           _dev(x.s0))
    return x, dev


class _path:
    """Forces the C ABI's kernel choice (and chunked tile width) inside a block."""

    def __init__(self, path, tile=0):
        self.path, self.tile = path, tile

    def __enter__(self):
        self.old = _native.set_path(self.path)
        self.old_tile = _native.set_tile(self.tile)

    def __exit__(self, *exc):
        _native.set_path(self.old)
        _native.set_tile(self.old_tile)


# ---------------------------------------------------------------------------
# MFMA lane layouts the chunked kernel assumes
# ---------------------------------------------------------------------------


def test_mfma_layout_probe():
    lib = ctypes.CDLL(os.path.join(os.path.dirname(__file__), "hip", "libmfma_probe.so"))
    rng = np.random.default_rng(0)
    a32 = synth.bf16_bits(rng.standard_normal((16, 32)).astype(np.float32))
    b32 = synth.bf16_bits(rng.standard_normal((32, 16)).astype(np.float32))
    a16 = synth.bf16_bits(rng.standard_normal((16, 16)).astype(np.float32))
    b16 = synth.bf16_bits(rng.standard_normal((16, 16)).astype(np.float32))
    da32, db32, da16, db16 = (_bf16_dev(x) for x in (a32, b32, a16, b16))
    c32 = torch.zeros((16, 16), dtype=torch.float32, device="cuda")
    c16 = torch.zeros((16, 16), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    rc = lib.mfma_probe(ctypes.c_void_p(da32.data_ptr()), ctypes.c_void_p(db32.data_ptr()),
                        ctypes.c_void_p(c32.data_ptr()), ctypes.c_void_p(da16.data_ptr()),
                        ctypes.c_void_p(db16.data_ptr()), ctypes.c_void_p(c16.data_ptr()))
    assert rc == 0
    e32 = synth.bf16_to_f32(a32).astype(np.float64) @ synth.bf16_to_f32(b32)
    e16 = synth.bf16_to_f32(a16).astype(np.float64) @ synth.bf16_to_f32(b16)
    np.testing.assert_allclose(_np(c32), e32, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(_np(c16), e16, rtol=1e-5, atol=1e-5)


def test_mfma_f32_layout_probe():
    """v_mfma_f32_16x16x4f32's lane layout, which the fp32 chunked forward assumes."""
    lib = ctypes.CDLL(os.path.join(os.path.dirname(__file__), "hip", "libmfma_probe.so"))
    rng = np.random.default_rng(1)
    a = rng.standard_normal((16, 4)).astype(np.float32)
    b = rng.standard_normal((4, 16)).astype(np.float32)
    c = torch.zeros((16, 16), dtype=torch.float32, device="cuda")
    da, db = _dev(a), _dev(b)
    torch.cuda.synchronize()
    assert lib.mfma_probe_f32(ctypes.c_void_p(da.data_ptr()), ctypes.c_void_p(db.data_ptr()),
                              ctypes.c_void_p(c.data_ptr())) == 0
    np.testing.assert_allclose(_np(c), a.astype(np.float64) @ b, rtol=1e-6, atol=1e-6)


def test_dpp_lane_reductions_probe():
    """The DPP reductions the kernels use (gate scan, row and wave sums, lane-group
    sums), on one wave: against NumPy, and every lane of a group with the same bits."""
    lib = ctypes.CDLL(os.path.join(os.path.dirname(__file__), "hip", "libmfma_probe.so"))
    x = np.random.default_rng(3).standard_normal(64).astype(np.float32)
    dx = torch.from_numpy(x).cuda()
    out = torch.full((9, 64), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    assert lib.dpp_probe(ctypes.c_void_p(dx.data_ptr()), ctypes.c_void_p(out.data_ptr())) == 0
    r = _np(out)
    x64 = x.astype(np.float64)
    np.testing.assert_allclose(r[0], np.cumsum(x64), rtol=1e-5, atol=1e-5)
    rows = np.repeat(x64.reshape(4, 16).sum(axis=1), 16)
    np.testing.assert_allclose(r[1], rows, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(r[2][48:], np.full(16, x64.sum()), rtol=1e-5, atol=1e-5)
    for j, n in enumerate((2, 4, 8, 16, 32, 64), start=3):
        groups = r[j].reshape(64 // n, n)
        np.testing.assert_allclose(groups[:, 0], x64.reshape(64 // n, n).sum(axis=1), rtol=1e-5, atol=1e-5)
        assert (groups == groups[:, :1]).all(), f"lane_sum<{n}>: lanes of a group differ"
    r1 = r[1].reshape(4, 16)
    assert (r1 == r1[:, :1]).all(), "row16_sum: lanes of a row differ"


# ---------------------------------------------------------------------------
# the reference's own cases (fp32 -> per-token kernel)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("case", reference_cases(), ids=lambda c: c[0])
def test_reference_cases_match_fixtures(case):
    name, q, k, v, b, s0, chunk = case
    data = np.load(os.path.join(GOLDEN, "reference_cases.npz"))
    cfg = kernels.LinearAttnConfig(chunk=chunk)
    out, st = kernels.chunked_delta_rule(q, k, v, b, state=s0, config=cfg)
    assert isinstance(out, np.ndarray) and out.dtype == np.float32
    assert_f32_parity(out, data[f"{name}/o"], name, scaled=True)
    assert_f32_parity(st, data[f"{name}/s"], name, scaled=True)
    if np.abs(data[f"{name}/o"]).max() < 100:  # the reference's element-wise 1e-5
        np.testing.assert_allclose(out, data[f"{name}/o"], **TOL)
        np.testing.assert_allclose(st, data[f"{name}/s"], **TOL)
    # device tensors in, device tensors out
    dq, dk, dv, db, ds = (_dev(x) for x in (q, k, v, b, s0))
    dout, dst = kernels.chunked_delta_rule(dq, dk, dv, db, ds, cfg)
    assert dout.is_cuda and dst.is_cuda
    np.testing.assert_array_equal(_np(dout), out)
    np.testing.assert_array_equal(_np(dst), st)


def test_reference_goldens():
    q = np.array([[[[1.0, 0.0]], [[0.0, 1.0]]]], dtype=np.float32)
    v = np.array([[[[1.0, 2.0]], [[3.0, 4.0]]]], dtype=np.float32)
    b = np.array([[[1.0], [1.0]]], dtype=np.float32)
    (out, st), res = kernels.chunked_delta_rule_fwd(q, q, v, b, None, kernels.LinearAttnConfig(2))
    np.testing.assert_allclose(out, v, **TOL)
    np.testing.assert_allclose(st, np.array([[[[1.0, 2.0], [3.0, 4.0]]]]), **TOL)
    assert type(res.chunk) is int and res.chunk == 2
    np.testing.assert_array_equal(res.state0, np.zeros((1, 1, 2, 2), np.float32))

    q1 = np.array([[[[1.0, 0.0]]]], dtype=np.float32)
    out, st = kernels.chunked_delta_rule(q1, q1, np.array([[[[2.0, 4.0]]]], np.float32),
                                         np.array([[[0.5]]], np.float32))
    np.testing.assert_allclose(out, np.array([[[[1.0, 2.0]]]]), **TOL)
    np.testing.assert_allclose(st, np.array([[[[1.0, 2.0], [0.0, 0.0]]]]), **TOL)

    out, st = kernels.chunked_delta_rule(q1, np.array([[[[0.0, 1.0]]]], np.float32),
                                         np.zeros((1, 1, 1, 2), np.float32),
                                         np.array([[[1.0]]], np.float32),
                                         state=np.eye(2, dtype=np.float32)[None, None])
    np.testing.assert_allclose(out, np.array([[[[1.0, 0.0]]]]), **TOL)
    np.testing.assert_allclose(st, np.array([[[[1.0, 0.0], [0.0, 0.0]]]]), **TOL)


def test_reference_invariants():
    inp = synth.reference_test_inputs
    rng = np.random.default_rng(11)
    q, k, v, b = inp(rng, seq=6)
    out, _ = kernels.chunked_delta_rule(q, k, v, b)
    q2, k2, v2, b2 = q.copy(), k.copy(), v.copy(), b.copy()
    q2[:, 3:] += 3.0
    k2[:, 3:] -= 1.5
    v2[:, 3:] += 4.0
    b2[:, 3:] = 0.9
    out2, _ = kernels.chunked_delta_rule(q2, k2, v2, b2)
    np.testing.assert_allclose(out[:, :3], out2[:, :3], **TOL)

    rng = np.random.default_rng(12)
    q, k, v, b = inp(rng, seq=7)
    oa, sa = kernels.chunked_delta_rule(q[:, :3], k[:, :3], v[:, :3], b[:, :3])
    ob, sb = kernels.chunked_delta_rule(q[:, 3:], k[:, 3:], v[:, 3:], b[:, 3:], state=sa)
    of, sf = kernels.chunked_delta_rule(q, k, v, b)
    np.testing.assert_allclose(np.concatenate([oa, ob], axis=1), of, **TOL)
    np.testing.assert_allclose(sb, sf, **TOL)

    rng = np.random.default_rng(13)
    q, k, v, b = inp(rng, seq=10, dim=3)
    e_o, e_s = ref.gated_delta_rule(q, k, v, b, dtype=np.float64)
    for chunk in (4, 7):
        o, s = kernels.chunked_delta_rule(q, k, v, b, config=kernels.LinearAttnConfig(chunk))
        np.testing.assert_allclose(o, e_o, **TOL)
        np.testing.assert_allclose(s, e_s, **TOL)

    rng = np.random.default_rng(15)
    q, k, v, b = inp(rng, batch=3, seq=4, heads=2, dim=5)
    o, s = kernels.chunked_delta_rule(q, k, v, b)
    assert o.shape == (3, 4, 2, 5) and s.shape == (3, 2, 5, 5)
    assert o.dtype == np.float32 and s.dtype == np.float32

    rng = np.random.default_rng(16)
    q, k, v, b = inp(rng, batch=1, seq=3, heads=1, dim=3)
    oa, sa = kernels.chunked_delta_rule(q, k, v, b, state=None)
    ob, sb = kernels.chunked_delta_rule(q, k, v, b, state=np.zeros((1, 1, 3, 3), np.float32))
    np.testing.assert_allclose(oa, ob, **TOL)
    np.testing.assert_allclose(sa, sb, **TOL)

    rng = np.random.default_rng(17)
    q, k, v, b = inp(rng, batch=1, seq=4, heads=1, dim=3)
    o1, s1 = kernels.chunked_delta_rule(q, k, v, b)
    o2, s2 = kernels.chunked_delta_rule(q, k, 2.0 * v, b)
    np.testing.assert_allclose(o2, 2.0 * o1, **TOL)
    np.testing.assert_allclose(s2, 2.0 * s1, **TOL)
    _, sq = kernels.chunked_delta_rule(q + 1.25, k, v, b)
    np.testing.assert_allclose(sq, s1, **TOL)


def test_fwd_residual_and_numpy_path():
    rng = np.random.default_rng(101)
    q, k, v, b = synth.reference_test_inputs(rng)
    s0 = rng.standard_normal((2, 2, 4, 4)).astype(np.float32) * 0.05
    cfg = kernels.LinearAttnConfig(chunk=2)
    (out, ns), res = kernels.chunked_delta_rule_fwd(q, k, v, b, s0, cfg)
    assert type(res) is kernels._DeltaResidual and type(res.chunk) is int and res.chunk == 2
    for got, exp in ((res.q, q), (res.k, k), (res.v, v), (res.beta, b), (res.state0, s0)):
        np.testing.assert_array_equal(got, exp)
    e_o, e_s = ref.gated_delta_rule(q, k, v, b, s0, dtype=np.float64)
    np.testing.assert_allclose(out, e_o, **TOL)
    np.testing.assert_allclose(ns, e_s, **TOL)
    dq, dk, dv, db, ds = (_dev(x) for x in (q, k, v, b, s0))
    (dout, dns), dres = kernels.chunked_delta_rule_fwd(dq, dk, dv, db, ds, cfg)
    assert dres.q is dq and dres.state0.is_cuda and dres.state0.dtype == torch.float32
    np.testing.assert_array_equal(_np(dout), out)


def test_cfg0_fp32():
    c = synth.CONFIGS[0]
    x = synth.fwd_inputs((c["B"], c["T"], c["H"], c["D"]), seed=0, dtype="fp32")
    data = np.load(os.path.join(GOLDEN, "cfg0.npz"))
    out, st = kernels.chunked_delta_rule(_dev(x.q), _dev(x.k), _dev(x.v), _dev(x.beta))
    assert_f32_parity(_np(out), data["o"], "cfg0 O")
    assert_f32_parity(_np(st), data["s"], "cfg0 S")


def test_empty_and_degenerate_sizes():
    s0 = np.arange(2 * 3 * 16, dtype=np.float32).reshape(2, 3, 4, 4)
    z = np.zeros((2, 0, 3, 4), np.float32)
    out, st = kernels.chunked_delta_rule(z, z, z, np.zeros((2, 0, 3), np.float32), state=s0)
    assert out.shape == (2, 0, 3, 4)
    np.testing.assert_array_equal(st, s0)
    out, st = kernels.chunked_delta_rule(z, z, z, np.zeros((2, 0, 3), np.float32))
    np.testing.assert_array_equal(st, 0.0)
    e = np.zeros((0, 5, 2, 4), np.float32)
    out, st = kernels.chunked_delta_rule(e, e, e, np.zeros((0, 5, 2), np.float32))
    assert out.shape == (0, 5, 2, 4) and st.shape == (0, 2, 4, 4)


# ---------------------------------------------------------------------------
# chunked MFMA kernel (bf16)
# ---------------------------------------------------------------------------

BF16_SHAPES = [
    ((1, 64, 1, 128), None),
    ((2, 200, 3, 128), 0.05),
    ((1, 1, 2, 128), 0.05),
    ((1, 130, 2, 64), None),
    ((3, 256, 2, 64), 0.05),
]


@pytest.mark.parametrize("tile", [16, 32, 64])
@pytest.mark.parametrize("shape,s0_std", BF16_SHAPES, ids=lambda s: str(s))
def test_chunked_bf16_vs_oracle(shape, s0_std, tile):
    x, (q, k, v, b, s0) = _bf16_case(shape, seed=sum(shape) + tile, s0_std=s0_std)
    with _path(2, tile):
        out, st = kernels.chunked_delta_rule(q, k, v, b, s0)
    e_o, e_s = ref.wy_chunked_fwd(x.q, x.k, x.v, x.beta, x.s0, chunk=64, dtype=np.float64)
    ro = assert_bf16_parity(_np(out), e_o, f"O {shape}")
    rs = assert_bf16_parity(_np(st), e_s, f"S {shape}")
    print(f"{shape} tile {tile}: rel-L2 O {ro:.2e} S {rs:.2e}")


def test_chunked_tiles_and_recurrent_agree():
    x, (q, k, v, b, s0) = _bf16_case((2, 300, 2, 128), seed=5, s0_std=0.02)
    outs = []
    for tile in (16, 32, 64):
        with _path(2, tile):
            outs.append(kernels.chunked_delta_rule(q, k, v, b, s0))
    with _path(1):
        o_rec, s_rec = kernels.chunked_delta_rule(q, k, v, b, s0)
    for o, s in outs:  # per-column arithmetic does not depend on the tile width
        assert torch.equal(o, outs[0][0]) and torch.equal(s, outs[0][1])
        assert rel_l2(_np(o), _np(o_rec)) < 1e-2
        assert rel_l2(_np(s), _np(s_rec)) < 1e-2
    # the per-token kernel on bf16 inputs is exact fp32 arithmetic
    e_o, e_s = ref.chunked_fwd_rank1(x.q, x.k, x.v, x.beta, x.s0, 64, dtype=np.float64)
    assert_f32_parity(_np(o_rec), e_o, "recurrent bf16-in O")
    assert_f32_parity(_np(s_rec), e_s, "recurrent bf16-in S")


def test_chunked_bf16_output_mode():
    _, (q, k, v, b, s0) = _bf16_case((1, 192, 2, 128), seed=8, s0_std=0.02)
    o32, s32 = kernels.chunked_delta_rule(q, k, v, b, s0)
    o16, s16 = kernels.chunked_delta_rule(q, k, v, b, s0, out_dtype=torch.bfloat16)
    assert o16.dtype == torch.bfloat16 and s16.dtype == torch.float32
    np.testing.assert_array_equal(_np(s16), _np(s32))
    np.testing.assert_array_equal(_np(o16.float()), _np(o32.to(torch.bfloat16).float()))


@pytest.mark.parametrize("tile", [16, 32])
def test_chunked_bf16_output_tiles_ragged_and_varlen(tile):
    # 32-column tiles stage bf16 O in LDS and store whole rows from the loader wave;
    # 16-column tiles store from the chain wave: both round the fp32 result once
    _, (q, k, v, b, s0) = _bf16_case((2, 200, 2, 128), seed=18, s0_std=0.02)
    with _path(2, tile):
        o32, s32 = kernels.chunked_delta_rule(q, k, v, b, s0)
        o16, s16 = kernels.chunked_delta_rule(q, k, v, b, s0, out_dtype=torch.bfloat16)
    np.testing.assert_array_equal(_np(s16), _np(s32))
    np.testing.assert_array_equal(_np(o16.float()), _np(o32.to(torch.bfloat16).float()))
    _, (qv, kv, vv, bv), cu = _varlen_case(700, 2, 128, seed=19, lo=1, hi=300)
    with _path(2, tile):
        ov32, sv32 = kernels.chunked_delta_rule_varlen(qv, kv, vv, bv, cu)
        ov16, sv16 = kernels.chunked_delta_rule_varlen(qv, kv, vv, bv, cu, out_dtype=torch.bfloat16)
    np.testing.assert_array_equal(_np(sv16), _np(sv32))
    np.testing.assert_array_equal(_np(ov16.float()), _np(ov32.to(torch.bfloat16).float()))


def test_chunked_state_carry_is_bitwise_at_chunk_boundaries():
    _, (q, k, v, b, s0) = _bf16_case((2, 640, 2, 128), seed=9, s0_std=0.02)
    of, sf = kernels.chunked_delta_rule(q, k, v, b, s0)
    cut = 384
    oa, sa = kernels.chunked_delta_rule(q[:, :cut].contiguous(), k[:, :cut].contiguous(),
                                        v[:, :cut].contiguous(), b[:, :cut].contiguous(), s0)
    ob, sb = kernels.chunked_delta_rule(q[:, cut:].contiguous(), k[:, cut:].contiguous(),
                                        v[:, cut:].contiguous(), b[:, cut:].contiguous(), sa)
    assert torch.equal(torch.cat([oa, ob], dim=1), of)
    assert torch.equal(sb, sf)


def test_chunked_repeat_and_graph_replay_are_bitwise():
    _, (q, k, v, b, s0) = _bf16_case((2, 256, 4, 128), seed=10, s0_std=0.02)
    with _path(2):  # the single-stage form (this shape's default is the split form)
        o1, s1 = kernels.chunked_delta_rule(q, k, v, b, s0)
        o2, s2 = kernels.chunked_delta_rule(q, k, v, b, s0)
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    lib = _native.lib()
    o = torch.empty_like(o1)
    s = torch.empty_like(s1)

    def launch():
        st = torch.cuda.current_stream().cuda_stream
        rc = lib.pm_delta_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), b.data_ptr(),
                              s0.data_ptr(), o.data_ptr(), s.data_ptr(), 2, 256, 4, 128,
                              _native.DTYPE_BF16, _native.DTYPE_F32, 64, None, 0, st)
        _native.check(rc)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch()  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch()
    for _ in range(3):
        o.zero_()
        s.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, o1) and torch.equal(s, s1)
        kernels.chunked_delta_rule(q, k, v, b, s0)  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("path", [0, 3])
def test_cfg1_full_size_vs_c_oracle(path):
    from oracle import cref

    c = synth.CONFIGS[1]
    x, (q, k, v, b, _) = _bf16_case((c["B"], c["T"], c["H"], c["D"]), seed=1)
    with _path(path):
        out, st = kernels.chunked_delta_rule(q, k, v, b)
    e_o, e_s = cref.delta_fwd(x.q_bits, x.k_bits, x.v_bits, x.beta, None, threads=CPU_THREADS)
    ro = assert_bf16_parity(_np(out), e_o, "cfg1 O")
    rs = assert_bf16_parity(_np(st), e_s, "cfg1 S")
    print(f"cfg1: rel-L2 O {ro:.2e} S {rs:.2e}")


def test_cfg3_full_size_vs_c_oracle_and_carry():
    from oracle import cref

    c = synth.CONFIGS[3]
    x, (q, k, v, b, s0) = _bf16_case((c["B"], c["T"], c["H"], c["D"]), seed=3,
                                     s0_std=c["s0_std"])
    out, st = kernels.chunked_delta_rule(q, k, v, b, s0)
    e_o, e_s = cref.delta_fwd(x.q_bits, x.k_bits, x.v_bits, x.beta, x.s0, threads=CPU_THREADS)
    ro = assert_bf16_parity(_np(out), e_o, "cfg3 O")
    rs = assert_bf16_parity(_np(st), e_s, "cfg3 S")
    print(f"cfg3: rel-L2 O {ro:.2e} S {rs:.2e}")
    half = c["T"] // 2
    oa, sa = kernels.chunked_delta_rule(q[:, :half].contiguous(), k[:, :half].contiguous(),
                                        v[:, :half].contiguous(), b[:, :half].contiguous(), s0)
    ob, sb = kernels.chunked_delta_rule(q[:, half:].contiguous(), k[:, half:].contiguous(),
                                        v[:, half:].contiguous(), b[:, half:].contiguous(), sa)
    assert torch.equal(torch.cat([oa, ob], dim=1), out) and torch.equal(sb, st)


# ---------------------------------------------------------------------------
# packed variable-length batch (cu_seqlens)
# ---------------------------------------------------------------------------


def _varlen_case(total, heads, dim, seed, lo=64, hi=4096):
    lens = synth.varlen_lengths(total, lo, hi, seed)
    cu = synth.cu_seqlens(lens)
    x = synth.fwd_inputs((total, heads, dim), seed=seed, dtype="bf16")
    dev = (_bf16_dev(x.q_bits), _bf16_dev(x.k_bits), _bf16_dev(x.v_bits), _dev(x.beta))
    return x, dev, cu


@pytest.mark.parametrize("path", [0, 1, 2, 3])
def test_varlen_segments_bitwise_equal_standalone(path):
    """With the kernel form fixed (path 1 per-token, 2 single-stage chunked, 3 split form),
    each varlen segment equals its standalone call bit for bit. At H = 2 the default path
    takes the split form for both calls, so path 0 is bitwise here too."""
    x, (q, k, v, b), cu = _varlen_case(3000, 2, 128, seed=12, lo=1, hi=700)
    cu = np.concatenate([cu[:2], cu[1:2], cu[2:]]).astype(np.int32)  # add an empty segment
    with _path(path):
        out, st = kernels.chunked_delta_rule_varlen(q, k, v, b, cu)
        assert out.shape == q.shape and st.shape == (cu.size - 1, 2, 128, 128)
        for i in range(cu.size - 1):
            a, z = int(cu[i]), int(cu[i + 1])
            oi, si = kernels.chunked_delta_rule(q[None, a:z], k[None, a:z], v[None, a:z],
                                                b[None, a:z])
            assert torch.equal(out[a:z], oi[0]), f"segment {i} [{a}, {z})"
            assert torch.equal(st[i], si[0]), f"segment {i} state"


def test_cfg2_default_path_segments_vs_standalone():
    """cfg2 (10 sequences x 16 heads) under the default path. The form is chosen per call
    from its (sequence, head) count: the varlen call (160 pairs, 32-column tiles) runs the
    single-stage kernel, while each standalone segment (16 pairs) runs the split form.
    The two forms round differently, so the segments agree within the bf16 bound, not
    bitwise; with the single-stage form forced (path 2) they agree bit for bit."""
    c = synth.CONFIGS[2]
    x, (q, k, v, b), cu = _varlen_case(c["total"], c["H"], c["D"], seed=2, lo=c["lo"], hi=c["hi"])
    cu_d = torch.from_numpy(cu).cuda()
    out0, st0 = kernels.chunked_delta_rule_varlen(q, k, v, b, cu_d)
    with _path(2):
        out2, st2 = kernels.chunked_delta_rule_varlen(q, k, v, b, cu_d)
    assert torch.equal(out0, out2) and torch.equal(st0, st2), "default varlen call is the single-stage form"
    for i in range(cu.size - 1):
        a, z = int(cu[i]), int(cu[i + 1])
        seg = (q[None, a:z], k[None, a:z], v[None, a:z], b[None, a:z])
        oi, si = kernels.chunked_delta_rule(*seg)
        assert_bf16_parity(_np(oi[0]), _np(out0[a:z]), f"segment {i} O, default path")
        assert_bf16_parity(_np(si[0]), _np(st0[i]), f"segment {i} S, default path")
        with _path(2):
            oi2, si2 = kernels.chunked_delta_rule(*seg)
        assert torch.equal(oi2[0], out2[a:z]) and torch.equal(si2[0], st2[i]), f"segment {i}, path 2"


def test_cfg2_varlen_vs_c_oracle():
    from oracle import cref

    c = synth.CONFIGS[2]
    x, (q, k, v, b), cu = _varlen_case(c["total"], c["H"], c["D"], seed=2, lo=c["lo"], hi=c["hi"])
    out, st = kernels.chunked_delta_rule_varlen(q, k, v, b, torch.from_numpy(cu).cuda())
    o_np, s_np = _np(out), _np(st)
    for i in range(cu.size - 1):
        a, z = int(cu[i]), int(cu[i + 1])
        e_o, e_s = cref.delta_fwd(x.q_bits[None, a:z], x.k_bits[None, a:z], x.v_bits[None, a:z],
                                  x.beta[None, a:z], None, threads=CPU_THREADS)
        assert_bf16_parity(o_np[a:z], e_o[0], f"cfg2 segment {i} O")
        assert_bf16_parity(s_np[i], e_s[0], f"cfg2 segment {i} S")


def _varlen_abi(q, k, v, b, cu_d, n_seqs, s0, ws=None, nws=0):
    n, H, D = q.shape
    o = torch.full((n, H, D), float("nan"), device="cuda")
    s = torch.full((n_seqs, H, D, D), float("nan"), device="cuda")
    rc = _native.lib().pm_delta_fwd_varlen(q.data_ptr(), k.data_ptr(), v.data_ptr(), b.data_ptr(), cu_d.data_ptr(),
                                           n_seqs, n, s0.data_ptr(), o.data_ptr(), s.data_ptr(), H, D,
                                           _native.DTYPE_BF16, _native.DTYPE_F32, 64,
                                           None if ws is None else ws.data_ptr(), nws,
                                           torch.cuda.current_stream().cuda_stream)
    _native.check(rc)
    return o, s


def _varlen_lens_case(lens, seed):
    lens = np.array(lens)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    n, H, D = int(cu[-1]), 2, 128
    x, (q, k, v, b, _) = _bf16_case((n, H, D), seed=seed)
    rng = np.random.default_rng(seed + 1)
    s0 = torch.from_numpy((0.02 * rng.standard_normal((lens.size, H, D, D))).astype(np.float32)).cuda()
    return lens, cu, x, (q, k, v, b), s0


@pytest.mark.parametrize("lens", [
    [3, 64, 0, 65, 700, 64, 130, 4000],             # longest last, ties (64 and 3: one chunk each), an empty one
    [4000, 700, 130, 65, 64, 3, 0],                 # already longest first
    [1] * 40 + [300] * 23 + [900],                  # 64 sequences, the most the kernel ranks itself
])
def test_varlen_longest_first_in_kernel_rank(lens):
    """Up to 64 sequences the single-stage varlen forward ranks them inside the kernel
    (longest first): no workspace is asked for, and every sequence's O rows and final state
    equal a standalone single-stage call on it (with its own initial state) bit for bit, so
    each workgroup found its own sequence; the longest and the shortest also against the
    oracle."""
    lens, cu, x, (q, k, v, b), s0 = _varlen_lens_case(lens, seed=44)
    n, H, D = q.shape
    with _path(2):  # the single-stage form at any shape
        assert _native.lib().pm_delta_varlen_workspace_bytes(lens.size, n, H, D, _native.DTYPE_BF16) == 0
        o, s = _varlen_abi(q, k, v, b, torch.from_numpy(cu).cuda(), lens.size, s0)
        for i in range(lens.size):
            a, z = int(cu[i]), int(cu[i + 1])
            oi, si = kernels.chunked_delta_rule(q[None, a:z], k[None, a:z], v[None, a:z], b[None, a:z], s0[i:i + 1])
            assert torch.equal(o[a:z], oi[0]), f"sequence {i} [{a}, {z}) O"
            assert torch.equal(s[i], si[0]), f"sequence {i} state"
    o_np, s_np = _np(o), _np(s)
    for i in (int(np.argmax(lens)), int(np.argmin(lens))):
        a, z = int(cu[i]), int(cu[i + 1])
        e_o, e_s = ref.wy_chunked_fwd(x.q[None, a:z], x.k[None, a:z], x.v[None, a:z], x.beta[None, a:z],
                                      _np(s0[i:i + 1]), chunk=64, dtype=np.float64)
        if z > a:
            assert_bf16_parity(o_np[a:z], e_o[0], f"ordered varlen sequence {i} O")
        assert_bf16_parity(s_np[i], e_s[0], f"ordered varlen sequence {i} S")


def _expected_order(cu, total):
    """Sequences by chunk count, largest first, ties in index order (offsets clamped as the
    kernels clamp them)."""
    a = np.clip(cu[:-1], 0, total)
    z = np.maximum(np.clip(cu[1:], 0, total), a)
    nc = (z - a + 63) // 64
    return np.array(sorted(range(len(nc)), key=lambda i: (-nc[i], i)), dtype=np.int32)


@pytest.mark.parametrize("lens", [
    [1] * 40 + [300] * 24 + [900],                  # 65 sequences: the order through the workspace
    [200] * 5 + [1] * 300 + [2000],                 # 306 sequences: two workgroups of the rank kernel
])
def test_varlen_longest_first_order_table(lens):
    """Beyond 64 sequences the order comes from the rank kernel through the workspace
    (pm_delta_varlen_workspace_bytes): the workspace then holds the expected permutation,
    and O and every final state equal the call without a workspace (cu_seqlens order) bit
    for bit, with an initial state per sequence."""
    lens, cu, x, (q, k, v, b), s0 = _varlen_lens_case(lens, seed=46)
    n, H, D = q.shape
    cu_d = torch.from_numpy(cu).cuda()
    with _path(2):
        nws = _native.lib().pm_delta_varlen_workspace_bytes(lens.size, n, H, D, _native.DTYPE_BF16)
        assert nws == 4 * lens.size
        ws = torch.full((nws // 4,), -7, dtype=torch.int32, device="cuda")
        o0, s0_ = _varlen_abi(q, k, v, b, cu_d, lens.size, s0)
        o1, s1_ = _varlen_abi(q, k, v, b, cu_d, lens.size, s0, ws, nws)
        torch.cuda.synchronize()
    assert np.array_equal(ws.cpu().numpy(), _expected_order(cu, n))
    assert not torch.isnan(o0).any() and not torch.isnan(s0_).any()
    assert torch.equal(o0, o1) and torch.equal(s0_, s1_)
    i = int(np.argmax(lens))
    a, z = int(cu[i]), int(cu[i + 1])
    e_o, e_s = ref.wy_chunked_fwd(x.q[None, a:z], x.k[None, a:z], x.v[None, a:z], x.beta[None, a:z],
                                  _np(s0[i:i + 1]), chunk=64, dtype=np.float64)
    assert_bf16_parity(_np(o1)[a:z], e_o[0], f"ordered varlen sequence {i} O")
    assert_bf16_parity(_np(s1_)[i], e_s[0], f"ordered varlen sequence {i} S")


# ---------------------------------------------------------------------------
# decode step
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dim", [128, 64, 32, 8])
def test_step_matches_forward_with_state(dim):
    rng = np.random.default_rng(30 + dim)
    q, k, v = (rng.standard_normal((3, 2, dim)).astype(np.float32) / np.sqrt(dim) for _ in range(3))
    b = rng.random((3, 2)).astype(np.float32)
    s = rng.standard_normal((3, 2, dim, dim)).astype(np.float32) * 0.05
    e_s, e_o = ref.delta_step(s.astype(np.float64), q, k, v, b)
    sd = _dev(s)
    o = kernels.delta_rule_step(_dev(q), _dev(k), _dev(v), _dev(b), sd)
    assert_f32_parity(_np(o), e_o, "step o")
    assert_f32_parity(_np(sd), e_s, "step S")
    o_f, s_f = kernels.chunked_delta_rule(q[:, None], k[:, None], v[:, None], b[:, None], state=s)
    assert_f32_parity(_np(o), o_f[:, 0], "step vs T=1 forward")
    assert_f32_parity(_np(sd), s_f, "step vs T=1 forward state")
    # NumPy state is updated in place through a copy
    s_host = s.copy()
    o_h = kernels.delta_rule_step(q, k, v, b, s_host)
    np.testing.assert_array_equal(o_h, _np(o))
    np.testing.assert_array_equal(s_host, _np(sd))


def test_cfg4_decode_steps_vs_c_oracle():
    """BASELINE cfg4 in full: B256 H32 D128, 64 consecutive in-place steps, o checked
    at every step and the state after the last one."""
    from oracle import cref

    c = synth.CONFIGS[4]
    bsz, heads, dim, steps = c["B"], c["H"], c["D"], c["steps"]
    assert steps == 64
    rng = np.random.default_rng(4)
    s0 = rng.normal(0.0, c["s0_std"], (bsz, heads, dim, dim)).astype(np.float32)
    s_dev = _dev(s0)
    s_cpu = s0.copy()
    for t in range(steps):
        x = synth.fwd_inputs((bsz, heads, dim), seed=100 + t, dtype="bf16")
        o = kernels.delta_rule_step(_bf16_dev(x.q_bits), _bf16_dev(x.k_bits), _bf16_dev(x.v_bits),
                                    _dev(x.beta), s_dev)
        e_o = cref.delta_step(s_cpu, x.q_bits, x.k_bits, x.v_bits, x.beta, threads=CPU_THREADS)
        assert_f32_parity(_np(o), e_o, f"cfg4 step {t} o")
    assert_f32_parity(_np(s_dev), s_cpu, "cfg4 final S")


@pytest.mark.parametrize("shape,tile,s0_std,out16", [
    ((1, 64, 1, 128), 0, None, False), ((2, 150, 2, 128), 0, 0.02, False), ((1, 1, 3, 128), 32, None, False),
    ((2, 257, 3, 64), 0, 0.02, False), ((3, 300, 2, 128), 16, 0.02, True), ((1, 130, 4, 64), 32, None, True),
    ((1, 700, 2, 128), 32, 0.02, False),
])
def test_split_form_vs_oracle(shape, tile, s0_std, out16):
    """pm_delta_set_path(3): the plain forward in split form (T diag(beta) built by a parallel
    pass into the workspace, then the chunk recurrence), against the fp64 chunked oracle at
    the bf16 bound, and against the single-stage kernel (path 2) over tails, D 64/128, both
    tile widths, S0 and bf16 O."""
    x, (q, k, v, b, s0) = _bf16_case(shape, seed=sum(shape) + tile + 7, s0_std=s0_std)
    odt = torch.bfloat16 if out16 else None
    with _path(3, tile):
        o3, s3 = kernels.chunked_delta_rule(q, k, v, b, s0, out_dtype=odt)
    with _path(2, tile):
        o2, s2 = kernels.chunked_delta_rule(q, k, v, b, s0, out_dtype=odt)
    torch.cuda.synchronize()
    e_o, e_s = ref.wy_chunked_fwd(x.q, x.k, x.v, x.beta, x.s0, chunk=64, dtype=np.float64)
    ro = assert_bf16_parity(_np(o3.float()), e_o, f"split O {shape}")
    rs = assert_bf16_parity(_np(s3), e_s, f"split S {shape}")
    assert rel_l2(_np(o3.float()), _np(o2.float())) < 2e-2 and rel_l2(_np(s3), _np(s2)) < 2e-2
    print(f"{shape} tile {tile}: split rel-L2 O {ro:.2e} S {rs:.2e}")


def test_split_form_default_choice_and_repeat():
    """By default the split form runs where the chunked kernel takes 16-column tiles (here
    B*H*(D/32) = 8 < 256): the default call equals the path-3 call bit for bit, repeats
    bitwise, and state carry at a chunk boundary is bitwise."""
    x, (q, k, v, b, s0) = _bf16_case((1, 640, 2, 128), seed=33, s0_std=0.02)
    assert _native.lib().pm_delta_workspace_bytes(1, 640, 2, 128, _native.DTYPE_BF16) > 0
    o0, s0_ = kernels.chunked_delta_rule(q, k, v, b, s0)
    with _path(3):
        o3, s3 = kernels.chunked_delta_rule(q, k, v, b, s0)
    o1, s1 = kernels.chunked_delta_rule(q, k, v, b, s0)
    assert torch.equal(o0, o3) and torch.equal(s0_, s3)
    assert torch.equal(o0, o1) and torch.equal(s0_, s1)
    oa, sa = kernels.chunked_delta_rule(q[:, :384].contiguous(), k[:, :384].contiguous(),
                                        v[:, :384].contiguous(), b[:, :384].contiguous(), s0)
    ob, sb = kernels.chunked_delta_rule(q[:, 384:].contiguous(), k[:, 384:].contiguous(),
                                        v[:, 384:].contiguous(), b[:, 384:].contiguous(), sa)
    assert torch.equal(torch.cat([oa, ob], dim=1), o0) and torch.equal(sb, s0_)


def test_split_form_graph_replay_is_bitwise():
    _, (q, k, v, b, s0) = _bf16_case((2, 256, 4, 128), seed=34, s0_std=0.02)
    lib = _native.lib()
    with _path(3):
        o1, s1 = kernels.chunked_delta_rule(q, k, v, b, s0)
        nb = lib.pm_delta_workspace_bytes(2, 256, 4, 128, _native.DTYPE_BF16)
    assert nb == 8 * 4 * 6 * 1024
    ws = torch.empty(nb, dtype=torch.uint8, device=q.device)
    o = torch.empty_like(o1)
    s = torch.empty_like(s1)

    def launch():
        st = torch.cuda.current_stream().cuda_stream
        old = _native.set_path(3)
        try:
            rc = lib.pm_delta_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), b.data_ptr(),
                                  s0.data_ptr(), o.data_ptr(), s.data_ptr(), 2, 256, 4, 128,
                                  _native.DTYPE_BF16, _native.DTYPE_F32, 64, ws.data_ptr(), nb, st)
        finally:
            _native.set_path(old)
        _native.check(rc)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch()
    for _ in range(3):
        o.zero_()
        s.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, o1) and torch.equal(s, s1)
        kernels.chunked_delta_rule(q, k, v, b, s0)
        torch.cuda.synchronize()


def test_split_form_varlen_segments_and_oracle():
    """Varlen in split form: each segment (empty, 1-token and multi-chunk ones included)
    equals its standalone split-form call bit for bit, and matches the oracle."""
    lens = np.array([64, 1, 0, 130, 700, 3000, 257])
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    n = int(cu[-1])
    x, (q, k, v, b, _) = _bf16_case((n, 4, 128), seed=91)
    for tile in (0, 16):
        with _path(3, tile):
            o3, s3 = kernels.chunked_delta_rule_varlen(q, k, v, b, cu)
            for i in range(cu.size - 1):
                a, z = int(cu[i]), int(cu[i + 1])
                oi, si = kernels.chunked_delta_rule(q[None, a:z], k[None, a:z], v[None, a:z], b[None, a:z])
                assert torch.equal(o3[a:z], oi[0]), f"segment {i} [{a}, {z}) tile {tile}"
                assert torch.equal(s3[i], si[0]), f"segment {i} state tile {tile}"
    o_np, s_np = _np(o3), _np(s3)
    for i in (0, 3, 6):
        a, z = int(cu[i]), int(cu[i + 1])
        e_o, e_s = ref.wy_chunked_fwd(x.q[None, a:z], x.k[None, a:z], x.v[None, a:z], x.beta[None, a:z],
                                      None, chunk=64, dtype=np.float64)
        assert_bf16_parity(o_np[a:z], e_o[0], f"split varlen segment {i} O")
        assert_bf16_parity(s_np[i], e_s[0], f"split varlen segment {i} S")
