"""CPU tests of the host side: the reference call surface, its checks, and the C ABI.

Nothing here launches a kernel: the checks mirrored from the reference
(kernels/__init__.py:308-338, :613-614, :676-677; tests/test_kernels.py:
218-241, :464-481) all fire before any device work, and the C ABI's
argument validation returns before touching the GPU.
"""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

from prometheus_amd import _native, kernels, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _inputs(rng, batch=2, seq=5, heads=2, dim=4):
    return synth.reference_test_inputs(rng, batch, seq, heads, dim)


# --- constants and dataclasses (tests/test_kernels.py:218-241) ---


def test_default_chunk_is_64():
    assert kernels.DEFAULT_CHUNK == 64


def test_linear_attn_config_defaults():
    cfg = kernels.LinearAttnConfig()
    assert cfg.chunk == 64
    assert cfg.eps == pytest.approx(1e-6)
    with pytest.raises(Exception):
        cfg.chunk = 3  # frozen


def test_kernel_error_is_value_error():
    assert issubclass(kernels.KernelError, ValueError)
    assert isinstance(kernels.KernelError("shape"), ValueError)


def test_delta_residual_fields():
    fields = [f for f in kernels._DeltaResidual.__dataclass_fields__]
    assert fields == ["q", "k", "v", "beta", "state0", "chunk"]


# --- KernelError before any device work (tests/test_kernels.py:464-481) ---


def test_bad_shapes_raise_kernel_error():
    q, k, v, beta = _inputs(np.random.default_rng(21), batch=1, seq=3, heads=1, dim=4)
    with pytest.raises(kernels.KernelError):
        kernels.chunked_delta_rule(q[:, :, :, :3], k, v, beta)
    with pytest.raises(kernels.KernelError):
        kernels.chunked_delta_rule(q, k, v, beta[:, :2])
    with pytest.raises(kernels.KernelError):
        kernels.chunked_delta_rule(q, k, v, beta, state=np.zeros((1, 1, 3, 3), np.float32))
    with pytest.raises(kernels.KernelError):
        kernels.chunked_delta_rule(q[0], k[0], v[0], beta[0])


def test_negative_beta_raises_kernel_error():
    q, k, v, beta = _inputs(np.random.default_rng(22), batch=1, seq=2, heads=1, dim=2)
    beta = beta.copy()
    beta[0, 0, 0] = -0.1
    with pytest.raises(kernels.KernelError):
        kernels.chunked_delta_rule(q, k, v, beta)
    with pytest.raises(kernels.KernelError):
        kernels.chunked_delta_rule_fwd(q, k, v, beta, None, kernels.LinearAttnConfig())


def test_chunk_below_one_raises_kernel_error():
    q, k, v, beta = _inputs(np.random.default_rng(23))
    with pytest.raises(kernels.KernelError):
        kernels.chunked_delta_rule(q, k, v, beta, config=kernels.LinearAttnConfig(chunk=0))
    with pytest.raises(kernels.KernelError):
        kernels.chunked_delta_rule_fwd(q, k, v, beta, None, kernels.LinearAttnConfig(chunk=-2))


def test_head_dim_limit_raises_kernel_error():
    z = np.zeros((1, 1, 1, 257), np.float32)
    with pytest.raises(kernels.KernelError):
        kernels.chunked_delta_rule(z, z, z, np.zeros((1, 1, 1), np.float32))


def _residual(b=1, t=3, h=2, d=4, state=True):
    z = np.zeros((b, t, h, d), np.float32)
    s0 = np.zeros((b, h, d, d), np.float32)
    return kernels._DeltaResidual(q=z, k=z, v=z, beta=np.zeros((b, t, h), np.float32),
                                  state0=s0 if state else None, chunk=64)


def test_bwd_shape_checks_raise_before_any_device_work():
    r = _residual()
    with pytest.raises(kernels.KernelError):
        kernels.chunked_delta_rule_bwd(r, (np.zeros((1, 3, 2, 5), np.float32), None))
    with pytest.raises(kernels.KernelError):
        kernels.chunked_delta_rule_bwd(r, (None, np.zeros((1, 2, 4, 3), np.float32)))
    big = _residual(d=257)
    with pytest.raises(kernels.KernelError):
        kernels.chunked_delta_rule_bwd(big, (None, None))


def _per_token_ws(b, t, h, d):
    n_ck, n_tiles = -(-t // 8), -(-d // (32 if d <= 128 else 16))
    part = n_tiles * t * (2 * d + 1) if n_tiles > 1 else 0
    return 4 * b * h * (t * d + n_ck * d * d + part)


def _chunked_ws(b, t, h, d):
    return 2 * b * h * (-(-t // 64)) * (2 * d * d + 64 * d + 3072)


def _f32_chunked_ws(b, t, h, d):
    # (T'')^T and the T / K K^T / beta / P record per 16-token chunk, S at every 256-token span
    # start and at the end, G at every span end, W and U per token; each region 256-byte aligned
    n_ch = -(-t // 16)
    n_span = -(-n_ch // 16)
    n = b * h
    al = lambda x: -(-x // 256) * 256
    size = al(n * n_ch * 256 * 4)
    size = al(size + n * n_ch * 784 * 4)
    size = al(size + n * (n_span + 1) * d * d * 4)
    size = al(size + n * n_span * d * d * 4)
    size = al(size + n * t * d * 4)
    return al(size + n * t * d * 4)


def test_bwd_workspace_bytes():
    lib = _native.lib()
    f32, bf16 = _native.DTYPE_F32, _native.DTYPE_BF16
    for b, t, h, d in [(1, 1, 1, 3), (2, 130, 3, 64), (4, 4096, 16, 128), (1, 0, 2, 8), (1, 70, 2, 48)]:
        want = _f32_chunked_ws(b, t, h, d) if d in (64, 128) else _per_token_ws(b, t, h, d)
        assert lib.pm_delta_bwd_workspace_bytes(b, t, h, d, f32) == want
        want = _chunked_ws(b, t, h, d) if d in (64, 128) else _per_token_ws(b, t, h, d)
        assert lib.pm_delta_bwd_workspace_bytes(b, t, h, d, bf16) == want
    # the cfg1 shape's fp32 chunked workspace stays under 0.5 GB
    assert lib.pm_delta_bwd_workspace_bytes(4, 4096, 16, 128, f32) < 500_000_000
    # path 1 (per-token kernel) applies to the backward as well
    old = _native.set_path(1)
    try:
        assert lib.pm_delta_bwd_workspace_bytes(2, 130, 3, 64, bf16) == _per_token_ws(2, 130, 3, 64)
        assert lib.pm_delta_bwd_workspace_bytes(2, 130, 3, 64, f32) == _per_token_ws(2, 130, 3, 64)
    finally:
        _native.set_path(old)
    assert lib.pm_delta_bwd_workspace_bytes(1, 4, 1, 257, f32) == 0
    # D above 128: 16-column tiles
    assert lib.pm_delta_bwd_workspace_bytes(1, 20, 2, 160, f32) == _per_token_ws(1, 20, 2, 160)
    assert lib.pm_delta_bwd_workspace_bytes(1, 20, 2, 256, bf16) == _per_token_ws(1, 20, 2, 256)
    assert lib.pm_delta_bwd_workspace_bytes(1, 4, 1, 0, f32) == 0
    assert lib.pm_delta_bwd_workspace_bytes(1, 4, 1, 8, 3) == 0


def test_bwd_abi_argument_validation_without_gpu():
    lib = _native.lib()
    f = lib.pm_delta_bwd
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first

    def call(b, t, h, d, dt, ws, nbytes, *, ptrs=None, gs0=p):
        q = ptrs if ptrs is not None else [p, p, p, p, None, None, None, p, p, p, p]
        return f(*q, gs0, b, t, h, d, dt, ws, nbytes, None)

    assert call(1, 4, 1, 0, 0, p, 1 << 20) == _native.E_SHAPE
    assert call(1, 4, 1, 257, 0, p, 1 << 20) == _native.E_SHAPE
    assert b"backward D" in lib.pm_last_error()
    assert call(-1, 4, 1, 8, 0, p, 1 << 20) == _native.E_SHAPE
    assert call(1, 4, 1, 8, 3, p, 1 << 20) == _native.E_DTYPE
    assert call(1, 4, 1, 8, 0, p, 1 << 20, gs0=None) == _native.E_NULL
    assert call(1, 4, 1, 8, 0, p, 1 << 20, ptrs=[None] + [p] * 3 + [None] * 3 + [p] * 4) == _native.E_NULL
    need = lib.pm_delta_bwd_workspace_bytes(1, 4, 1, 8, 0)
    assert call(1, 4, 1, 8, 0, p, need - 4) == _native.E_WORKSPACE
    assert call(1, 4, 1, 8, 0, None, need) == _native.E_WORKSPACE
    assert call(1, 4, 1, 8, 0, ctypes.c_void_p(18), need) == _native.E_ALIGN
    # chunked backward (bf16, D = 64): 16-byte alignment of q, k, v, go, workspace
    need = lib.pm_delta_bwd_workspace_bytes(1, 4, 1, 64, 1)
    odd = ctypes.c_void_p(24)
    assert call(1, 4, 1, 64, 1, p, need, ptrs=[odd, p, p, p, None, None, None, p, p, p, p]) == _native.E_ALIGN
    assert call(1, 4, 1, 64, 1, odd, need) == _native.E_ALIGN
    # path 2 (chunked required) refuses what only the per-token kernel serves
    old = _native.set_path(2)
    try:
        assert call(1, 4, 1, 8, 0, p, 1 << 20) == _native.E_UNSUPPORTED
        assert call(1, 4, 1, 48, 1, p, 1 << 20) == _native.E_UNSUPPORTED
    finally:
        _native.set_path(old)
    # nothing to do: B*H == 0
    assert call(0, 4, 1, 8, 0, None, 0) == 0


def test_varlen_checks():
    q = np.zeros((10, 2, 4), np.float32)
    b = np.zeros((10, 2), np.float32)
    for cu in ([0, 5, 9], [1, 5, 10], [0, 6, 5, 10], [0.0, 10.0]):
        with pytest.raises(kernels.KernelError):
            kernels.chunked_delta_rule_varlen(q, q, q, b, np.asarray(cu))
    with pytest.raises(kernels.KernelError):
        kernels.chunked_delta_rule_varlen(q, q, q, b[:5], np.array([0, 10]))
    with pytest.raises(kernels.KernelError):
        kernels.chunked_delta_rule_varlen(q, q, q, b, np.array([0, 4, 10]),
                                          state=np.zeros((3, 2, 4, 4), np.float32))


def test_step_checks():
    q = np.zeros((2, 3, 4), np.float32)
    b = np.zeros((2, 3), np.float32)
    with pytest.raises(kernels.KernelError):
        kernels.delta_rule_step(q, q, q, b, np.zeros((2, 3, 4, 5), np.float32))
    with pytest.raises(kernels.KernelError):
        kernels.delta_rule_step(q, q, q, b, np.zeros((2, 3, 4, 4), np.float64))
    with pytest.raises(kernels.KernelError):
        kernels.delta_rule_step(q, q, q, b[:1], np.zeros((2, 3, 4, 4), np.float32))


def test_out_dtype_check():
    q, k, v, beta = _inputs(np.random.default_rng(24))
    with pytest.raises(kernels.KernelError):
        kernels.chunked_delta_rule(q, k, v, beta, out_dtype="fp16")


# --- the C ABI library: loads, exports what include/pm_delta.h declares ---


def _header_functions():
    text = open(os.path.join(ROOT, "include", "pm_delta.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pm_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    declared = _header_functions()
    assert declared == sorted(_native.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.pm_abi_version() == _native.ABI_VERSION


def test_abi_argument_validation_without_gpu():
    lib = _native.lib()
    f = lib.pm_delta_fwd
    dummy = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    # D out of range
    assert f(dummy, dummy, dummy, dummy, None, dummy, dummy, 1, 4, 1, 0, 0, 0, 64, None, 0,
             None) == _native.E_SHAPE
    assert b"D must be" in lib.pm_last_error()
    assert f(dummy, dummy, dummy, dummy, None, dummy, dummy, 1, 4, 1, 300, 0, 0, 64, None, 0,
             None) == _native.E_SHAPE
    # chunk < 1
    assert f(dummy, dummy, dummy, dummy, None, dummy, dummy, 1, 4, 1, 8, 0, 0, 0, None, 0,
             None) == _native.E_SHAPE
    # dtype
    assert f(dummy, dummy, dummy, dummy, None, dummy, dummy, 1, 4, 1, 8, 7, 0, 64, None, 0,
             None) == _native.E_DTYPE
    assert f(dummy, dummy, dummy, dummy, None, dummy, dummy, 1, 4, 1, 8, 0, 5, 64, None, 0,
             None) == _native.E_DTYPE
    # NULL inputs with tokens to process
    assert f(None, dummy, dummy, dummy, None, dummy, dummy, 1, 4, 1, 8, 0, 0, 64, None, 0,
             None) == _native.E_NULL
    assert f(dummy, dummy, dummy, dummy, None, dummy, None, 1, 4, 1, 8, 0, 0, 64, None, 0,
             None) == _native.E_NULL
    # negative sizes
    assert f(dummy, dummy, dummy, dummy, None, dummy, dummy, -1, 4, 1, 8, 0, 0, 64, None, 0,
             None) == _native.E_SHAPE
    # nothing to do: B*H == 0 returns success without touching anything
    assert f(None, None, None, None, None, None, None, 0, 4, 3, 8, 0, 0, 64, None, 0, None) == 0
    # varlen: NULL cu_seqlens, misaligned cu_seqlens
    g = lib.pm_delta_fwd_varlen
    assert g(dummy, dummy, dummy, dummy, None, 2, 10, None, dummy, dummy, 1, 8, 0, 0, 64, None, 0,
             None) == _native.E_NULL
    assert g(dummy, dummy, dummy, dummy, ctypes.c_void_p(18), 2, 10, None, dummy, dummy, 1, 8, 0,
             0, 64, None, 0, None) == _native.E_ALIGN
    # step
    h = lib.pm_delta_step
    assert h(None, dummy, dummy, dummy, dummy, dummy, 2, 2, 8, 0, None) == _native.E_NULL
    assert h(dummy, dummy, dummy, dummy, dummy, dummy, 2, 2, 0, 0, None) == _native.E_SHAPE
    assert h(dummy, dummy, dummy, dummy, dummy, dummy, 2, 2, 8, 3, None) == _native.E_DTYPE
    assert lib.pm_delta_workspace_bytes(4, 4096, 16, 128, 1) == 0


def test_forward_workspace_sizes_and_checks():
    """The split form's T workspace (6 KiB per (b, h) and chunk) is asked for exactly where
    the forward would run that form: by default where even 16-column tiles give fewer than
    256 workgroups (pairs * D / 16 < 256), always under path 3."""
    lib = _native.lib()
    bf16, f32 = _native.DTYPE_BF16, _native.DTYPE_F32
    per = 6 * 1024
    assert lib.pm_delta_workspace_bytes(1, 32768, 32, 128, bf16) == 0  # cfg3: 256 workgroups
    assert lib.pm_delta_workspace_bytes(1, 32768, 31, 128, bf16) == 31 * 512 * per  # 248
    assert lib.pm_delta_workspace_bytes(1, 4096, 16, 128, bf16) == 16 * 64 * per
    assert lib.pm_delta_workspace_bytes(4, 4096, 16, 64, bf16) == 0  # 256 workgroups at D = 64
    assert lib.pm_delta_workspace_bytes(1, 130, 2, 64, bf16) == 2 * 3 * per
    assert lib.pm_delta_workspace_bytes(4, 4096, 16, 128, bf16) == 0  # cfg1: 32-col tiles
    assert lib.pm_delta_workspace_bytes(1, 4096, 16, 256, bf16) == 0
    # fp32 q/k/v at D in {64, 128}: the fp32 chunked forward's 2 KiB per (b, h) and 16-token chunk
    assert lib.pm_delta_workspace_bytes(1, 4096, 16, 128, f32) == 16 * 256 * 1024
    assert lib.pm_delta_workspace_bytes(2, 17, 3, 64, f32) == 6 * 2 * 1024
    assert lib.pm_delta_workspace_bytes(2, 17, 3, 48, f32) == 0  # per-token kernel
    assert lib.pm_delta_varlen_workspace_bytes(3, 100, 2, 128, f32) == 2 * (7 + 3) * 1024
    # varlen: H x (ceil(total / 64) + n_seqs) slots
    assert lib.pm_delta_varlen_workspace_bytes(3, 1000, 4, 128, bf16) == 4 * (16 + 3) * per
    # the single-stage kernel on a packed batch: the sequence order (4 bytes per sequence)
    # for 65 to 8192 sequences; up to 64 the kernel ranks them itself
    assert lib.pm_delta_varlen_workspace_bytes(8, 16384, 16, 128, bf16) == 0  # cfg2: 32-col tiles
    assert lib.pm_delta_varlen_workspace_bytes(64, 16384, 16, 128, bf16) == 0
    assert lib.pm_delta_varlen_workspace_bytes(65, 16384, 16, 128, bf16) == 65 * 4
    assert lib.pm_delta_varlen_workspace_bytes(8192, 16384, 16, 128, bf16) == 8192 * 4
    assert lib.pm_delta_varlen_workspace_bytes(8193, 16384, 16, 128, bf16) == 0
    assert lib.pm_delta_workspace_bytes(8, 2048, 16, 128, bf16) == 0  # fixed length: no order
    old = _native.set_path(3)
    try:
        assert lib.pm_delta_workspace_bytes(4, 4096, 16, 128, bf16) == 64 * 64 * per
        assert lib.pm_delta_varlen_workspace_bytes(8, 16384, 16, 128, bf16) == 16 * (256 + 8) * per
        # path 3 refuses to run without the workspace (checked before any launch)
        p = ctypes.c_void_p(256)
        rc = lib.pm_delta_fwd(p, p, p, p, None, p, p, 1, 64, 1, 128, bf16, f32, 64, None, 0, None)
        assert rc == _native.E_WORKSPACE and b"workspace" in lib.pm_last_error()
        rc = lib.pm_delta_fwd(p, p, p, p, None, p, p, 1, 64, 1, 128, bf16, f32, 64, p, per - 16, None)
        assert rc == _native.E_WORKSPACE
    finally:
        _native.set_path(old)
    old = _native.set_path(1)
    try:
        assert lib.pm_delta_workspace_bytes(1, 32768, 32, 128, bf16) == 0
        assert lib.pm_delta_workspace_bytes(1, 4096, 16, 128, f32) == 0
    finally:
        _native.set_path(old)
    old = _native.set_path(2)
    try:
        # path 2 with fp32 inputs: the fp32 chunked forward, which needs its workspace
        p = ctypes.c_void_p(256)
        rc = lib.pm_delta_fwd(p, p, p, p, None, p, p, 1, 64, 1, 128, f32, f32, 64, None, 0, None)
        assert rc == _native.E_WORKSPACE and b"fp32 chunked" in lib.pm_last_error()
        rc = lib.pm_delta_fwd(p, p, p, p, None, p, p, 1, 64, 1, 48, f32, f32, 64, None, 0, None)
        assert rc == _native.E_UNSUPPORTED
    finally:
        _native.set_path(old)
    old = _native.set_tile(32)
    try:
        assert lib.pm_delta_workspace_bytes(1, 32768, 32, 128, bf16) == 0
    finally:
        _native.set_tile(old)


def test_path_and_tile_switches():
    old = _native.set_path(1)
    try:
        assert _native.set_path(2) == 1
        assert _native.set_path(3) == 2
    finally:
        _native.set_path(old)
    with pytest.raises(_native.NativeError):
        _native.set_path(4)
    old = _native.set_tile(32)
    try:
        assert _native.set_tile(16) == 32
    finally:
        _native.set_tile(old)
    with pytest.raises(_native.NativeError):
        _native.set_tile(48)


def test_synth_configs_and_lengths():
    c = synth.CONFIGS[2]
    lens = synth.varlen_lengths(c["total"], c["lo"], c["hi"], seed=0)
    assert int(lens.sum()) == c["total"]
    assert np.all(lens[:-1] >= 64) and np.all(lens <= 4096)
    cu = synth.cu_seqlens(lens)
    assert cu.dtype == np.int32 and cu[0] == 0 and cu[-1] == c["total"]
    x = synth.fwd_inputs((1, 8, 2, 16), seed=1, dtype="bf16", s0_std=0.02)
    np.testing.assert_allclose(np.linalg.norm(x.q, axis=-1), 1.0, atol=1e-2)
    assert x.q_bits.dtype == np.uint16 and x.s0.shape == (1, 2, 16, 16)
    assert np.all((x.beta > 0) & (x.beta < 1))


def test_state_cache_bookkeeping_without_gpu():
    from prometheus_amd import serving

    cache = serving.LinearStateCache(2, 4, 1, 8, device="cpu")
    a = cache.alloc(3)
    assert a == [0, 1, 2] and cache.n_free == 1
    cache.pool[:, a] = 1.0
    cache.free([1])
    assert cache.alloc(1) == [1]  # freed slots come back zeroed
    assert float(cache.pool[:, 1].abs().sum()) == 0.0
    with pytest.raises(RuntimeError):
        cache.alloc(2)
    with pytest.raises(ValueError):
        cache.free([3])  # never allocated
    with pytest.raises(ValueError):
        cache.reset([4])  # outside the pool
    # the lowest free slots come first, whatever the order they were freed in
    big = serving.LinearStateCache(1, 8, 1, 8, device="cpu")
    assert big.alloc(6) == [0, 1, 2, 3, 4, 5]
    big.free([4, 1, 3])
    assert big.alloc(2) == [1, 3] and big.alloc(2) == [4, 6]
    with pytest.raises(RuntimeError):  # computing needs the GPU: no host fallback
        cache.decode(0, None, None, None, None, None)


def test_slot_decode_abi_validation_without_gpu():
    lib = _native.lib()
    p = ctypes.c_void_p(256)  # never dereferenced: validation fails first

    def call(n_slots, b, h, d, dt=1, pool=p, slots=p, o=p):
        return lib.pm_delta_step_slots(pool, slots, n_slots, p, p, p, p, o, b, h, d, dt, None)

    assert call(4, 2, 2, 48) == _native.E_UNSUPPORTED
    assert call(4, 2, 2, 64, dt=5) == _native.E_DTYPE
    assert call(-1, 2, 2, 64) == _native.E_SHAPE
    assert call(4, 2, 2, 64, slots=None) == _native.E_NULL
    assert call(4, 2, 2, 64, pool=None) == _native.E_NULL
    assert call(4, 2, 2, 64, pool=ctypes.c_void_p(8)) == _native.E_ALIGN
    assert call(4, 2, 2, 64, o=ctypes.c_void_p(8)) == _native.E_ALIGN
    assert call(4, 0, 2, 64) == 0  # nothing to do


def test_gated_validation_without_gpu():
    q = np.zeros((1, 4, 2, 8), np.float32)
    b = np.zeros((1, 4, 2), np.float32)
    with pytest.raises(kernels.KernelError):
        kernels.chunked_gated_delta_rule(q, q, q, b, np.zeros((1, 4, 3), np.float32))
    with pytest.raises(kernels.KernelError):
        kernels.gated_delta_rule_step(q[:, 0], q[:, 0], q[:, 0], b[:, 0], np.zeros((1, 3), np.float32),
                                      np.zeros((1, 2, 8, 8), np.float32))
    lib = _native.lib()
    p = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    assert lib.pm_gated_delta_fwd(p, p, p, p, None, None, p, p, 1, 4, 2, 8, 0, 0, None) == _native.E_NULL
    assert lib.pm_gated_delta_fwd(p, p, p, p, ctypes.c_void_p(2), None, p, p, 1, 4, 2, 8, 0, 0,
                                  None) == _native.E_ALIGN
    assert lib.pm_gated_delta_fwd(p, p, p, p, p, None, p, p, 1, 4, 2, 300, 0, 0, None) == _native.E_SHAPE
    assert lib.pm_gated_delta_step(p, p, p, p, p, None, p, 1, 2, 8, 0, None) == _native.E_NULL


def test_kda_validation_without_gpu():
    """The per-channel gates are (B, T, H, D) for the forward and (B, H, D) for the step;
    the scalar-gate shapes are refused, as are NULL, misaligned and oversized inputs."""
    q = np.zeros((1, 4, 2, 8), np.float32)
    b = np.zeros((1, 4, 2), np.float32)
    with pytest.raises(kernels.KernelError, match="g shape"):
        kernels.chunked_kda_rule(q, q, q, b, b)
    with pytest.raises(kernels.KernelError):
        kernels.kda_delta_rule_step(q[:, 0], q[:, 0], q[:, 0], b[:, 0], b[:, 0],
                                    np.zeros((1, 2, 8, 8), np.float32))
    lib = _native.lib()
    p = ctypes.c_void_p(256)
    assert lib.pm_kda_delta_fwd(p, p, p, p, None, None, p, p, 1, 4, 2, 8, 0, 0, None, 0, None) == _native.E_NULL
    assert lib.pm_kda_delta_fwd(p, p, p, p, ctypes.c_void_p(2), None, p, p, 1, 4, 2, 8, 0, 0,
                                None, 0, None) == _native.E_ALIGN
    assert lib.pm_kda_delta_fwd(p, p, p, p, p, None, p, p, 1, 4, 2, 300, 0, 0, None, 0, None) == _native.E_SHAPE
    assert lib.pm_kda_delta_fwd(p, p, p, p, p, None, p, p, 1, 4, 2, 8, 0, 7, None, 0, None) == _native.E_DTYPE
    assert lib.pm_kda_delta_step(p, p, p, p, p, None, p, 1, 2, 8, 0, None) == _native.E_NULL
    assert lib.pm_kda_delta_step(p, p, p, p, p, p, p, 1, 2, 300, 0, None) == _native.E_SHAPE
    # the chunked form's workspace: 61 KiB (D = 128) or 37 KiB (D = 64) per chunk, bf16 only
    bf16 = _native.DTYPE_BF16
    for b, t, h, d, per in [(4, 4096, 16, 128, 61), (2, 130, 3, 64, 37), (1, 1, 1, 128, 61)]:
        assert lib.pm_kda_delta_workspace_bytes(b, t, h, d, bf16) == b * h * (-(-t // 64)) * per * 1024
    assert lib.pm_kda_delta_workspace_bytes(1, 64, 1, 128, _native.DTYPE_F32) == 0
    assert lib.pm_kda_delta_workspace_bytes(1, 64, 1, 48, bf16) == 0
    with _native.use_knobs(1, 0):
        assert lib.pm_kda_delta_workspace_bytes(1, 64, 1, 128, bf16) == 0
    # path 2: the chunked form required; fp32 inputs refused, a missing workspace too
    al = ctypes.c_void_p(1 << 20)
    with _native.use_knobs(2, 0):
        assert lib.pm_kda_delta_fwd(al, al, al, al, al, None, al, al, 1, 4, 2, 64, 0, 0, None, 0,
                                    None) == _native.E_UNSUPPORTED
        assert lib.pm_kda_delta_fwd(al, al, al, al, al, None, al, al, 1, 4, 2, 64, 1, 0, None, 0,
                                    None) == _native.E_WORKSPACE


def test_selection_knobs_are_per_thread():
    """pm_delta_set_path / pm_delta_set_tile act on the calling thread only, so a
    workspace-size query and the call it sizes agree whatever another thread
    selects meanwhile (no GPU needed: both calls are host-only)."""
    import threading

    L = _native.lib()
    B, T, H, D = 2, 300, 4, 128
    bf16 = _native.DTYPE_BF16
    chunked = L.pm_delta_bwd_workspace_bytes(B, T, H, D, bf16)
    L.pm_delta_set_path(1)
    try:
        per_token = L.pm_delta_bwd_workspace_bytes(B, T, H, D, bf16)
    finally:
        L.pm_delta_set_path(0)
    assert chunked != per_token and chunked > 0 and per_token > 0

    barrier = threading.Barrier(2)
    seen = {}

    def worker(path, key):
        L.pm_delta_set_path(path)
        barrier.wait()  # both threads have selected before either queries
        sizes = [L.pm_delta_bwd_workspace_bytes(B, T, H, D, bf16) for _ in range(200)]
        barrier.wait()
        seen[key] = (L.pm_delta_set_path(0), set(sizes))

    threads = [threading.Thread(target=worker, args=(1, "a")), threading.Thread(target=worker, args=(2, "b"))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert seen["a"] == (1, {per_token})
    assert seen["b"] == (2, {chunked})
    assert L.pm_delta_set_path(0) == 0  # this thread never selected anything


def test_no_unprefixed_exports():
    """The library exports exactly the pm_* entry points of include/pm_delta.h (no
    internal helper leaks as an unprefixed C symbol)."""
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", _native.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    names = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    c_names = {n for n in names if not n.startswith("_Z")}
    assert c_names - {"_init", "_fini"} == set(_native.EXPORTS), sorted(c_names)


def test_noalloc_backward_rejects_sizes_beyond_its_scratch():
    """pm_delta_bwd_noalloc refuses (PM_E_WORKSPACE, before any device work) a call
    whose workspace would exceed the library's fixed scratch, and validates its
    arguments like pm_delta_bwd."""
    L = _native.lib()
    p = ctypes.c_void_p(16)  # never dereferenced
    ptrs = [p] * 12
    B, T, H, D = 4, 4096, 16, 128
    assert L.pm_delta_bwd_workspace_bytes(B, T, H, D, _native.DTYPE_BF16) > _native.NOALLOC_SCRATCH_BYTES
    assert L.pm_delta_bwd_noalloc(*ptrs, B, T, H, D, _native.DTYPE_BF16, None) == _native.E_WORKSPACE
    assert b"no-allocation" in L.pm_last_error()
    assert L.pm_delta_bwd_noalloc(*ptrs, 1, 8, 1, 257, _native.DTYPE_F32, None) == _native.E_SHAPE
    assert L.pm_delta_bwd_noalloc(*ptrs, 1, 8, 1, 8, 7, None) == _native.E_DTYPE
    # nothing to do: B*H == 0 returns before any device work
    assert L.pm_delta_bwd_noalloc(*([None] * 12), 0, 8, 1, 8, _native.DTYPE_F32, None) == 0


def test_knobs_read_and_scoped_set():
    """knobs() reads this thread's (path, tile) without changing them; use_knobs sets both
    for a block and restores them, also when the block raises; another thread keeps its own."""
    import threading

    base = _native.knobs()
    assert _native.knobs() == base
    with _native.use_knobs(2, 16):
        assert _native.knobs() == (2, 16)
        seen = []
        t = threading.Thread(target=lambda: seen.append(_native.knobs()))
        t.start()
        t.join()
        assert seen == [(0, 0)]  # a fresh thread starts at the defaults
    assert _native.knobs() == base
    try:
        with _native.use_knobs(1, 32):
            raise KeyError("inside")
    except KeyError:
        pass
    assert _native.knobs() == base


def test_kda_backward_workspace_and_checks():
    """pm_kda_delta_bwd_workspace_bytes: the per-token backward's workspace plus, with
    several column tiles (D > 32), a partial sum of dL/dg per channel and tile; null
    gates are refused before any launch, and so is path 2."""
    lib = _native.lib()
    f32, bf16 = _native.DTYPE_F32, _native.DTYPE_BF16
    for b, t, h, d in [(1, 1, 1, 3), (2, 130, 3, 64), (4, 4096, 16, 128), (1, 70, 2, 48), (1, 20, 2, 160)]:
        base = _per_token_ws(b, t, h, d)
        n_tiles = 1 if d <= 32 else ((d + 31) // 32 if d <= 128 else (d + 15) // 16)
        extra = 4 * b * t * h * d * n_tiles if n_tiles > 1 else 0
        for dt in (f32, bf16):
            assert lib.pm_kda_delta_bwd_workspace_bytes(b, t, h, d, dt) == base + extra
    assert lib.pm_kda_delta_bwd_workspace_bytes(1, 4, 1, 257, f32) == 0
    p = ctypes.c_void_p(256)
    rc = lib.pm_kda_delta_bwd(p, p, p, p, None, None, p, p, p, p, p, p, p, p, 1, 4, 1, 8, f32, p, 1 << 20, None)
    assert rc == _native.E_NULL and b"g and gg" in lib.pm_last_error()
    old = _native.set_path(2)
    try:
        rc = lib.pm_kda_delta_bwd(p, p, p, p, p, None, p, p, p, p, p, p, p, p, 1, 4, 1, 64, bf16, p, 1 << 24, None)
        assert rc == _native.E_UNSUPPORTED and b"per-token" in lib.pm_last_error()
    finally:
        _native.set_path(old)


def test_gated_backward_workspace_and_checks():
    """pm_gated_delta_bwd_workspace_bytes: the per-token backward's workspace plus the
    partial sums of dL/dg over column tiles (D > 32), for bf16 inputs as well (the gated
    backward has no chunked form); null gates are refused before any launch."""
    lib = _native.lib()
    f32, bf16 = _native.DTYPE_F32, _native.DTYPE_BF16
    for b, t, h, d in [(1, 1, 1, 3), (2, 130, 3, 64), (4, 4096, 16, 128), (1, 70, 2, 48), (1, 20, 2, 160)]:
        base = _per_token_ws(b, t, h, d)
        n_tiles = 1 if d <= 32 else ((d + 31) // 32 if d <= 128 else (d + 15) // 16)
        extra = 4 * b * t * h * n_tiles if n_tiles > 1 else 0
        for dt in (f32, bf16):
            assert lib.pm_gated_delta_bwd_workspace_bytes(b, t, h, d, dt) == base + extra
    assert lib.pm_gated_delta_bwd_workspace_bytes(1, 4, 1, 257, f32) == 0
    assert lib.pm_gated_delta_bwd_workspace_bytes(1, 4, 1, 8, 3) == 0
    p = ctypes.c_void_p(256)
    rc = lib.pm_gated_delta_bwd(p, p, p, p, None, None, p, p, p, p, p, p, p, p, 1, 4, 1, 8, f32, p, 1 << 20, None)
    assert rc == _native.E_NULL and b"g and gg" in lib.pm_last_error()
    rc = lib.pm_gated_delta_bwd(p, p, p, p, p, None, p, p, p, p, p, p, None, p, 1, 4, 1, 8, f32, p, 1 << 20, None)
    assert rc == _native.E_NULL
    old = _native.set_path(2)
    try:
        rc = lib.pm_gated_delta_bwd(p, p, p, p, p, None, p, p, p, p, p, p, p, p, 1, 4, 1, 64, bf16, p, 1 << 24, None)
        assert rc == _native.E_UNSUPPORTED and b"per-token" in lib.pm_last_error()
    finally:
        _native.set_path(old)
