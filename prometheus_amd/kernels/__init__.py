"""Delta-rule linear attention on MI355X — the reference's ``kernels`` call surface.

Drop-in for the delta-rule forward of teddytennant/prometheus
(``kernels/__init__.py``): same names, same positional order
``(q, k, v, beta, state, config)``, same shapes, fp32 outputs, the same
``_DeltaResidual`` fields and the same ``KernelError`` checks. The work runs
in hand-written HIP kernels for gfx950 behind the C ABI of
``include/pm_delta.h`` (``libpmdelta.so``); torch tensors are only device
buffers and streams. There is no CPU fallback: without the built library
or a GPU every call that reaches compute raises.

Recurrence (decay gate 1), per batch b and head h::

    S_t = (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T,    o_t = q_t S_t

Inputs may be torch tensors (any device; CUDA/HIP tensors are used in
place, CPU tensors are copied over and results copied back) or NumPy arrays
(the reference's NumPy path: copied to the GPU, results returned as NumPy).
bf16 q/k/v run the chunked MFMA kernel; every other dtype is cast to fp32,
as the reference does (``kernels/__init__.py:344-347``), and runs the fp32
per-token kernel.

Beyond the reference surface: ``chunked_delta_rule_varlen`` (packed batch
with ``cu_seqlens``), ``delta_rule_step`` (public single-token decode step)
and the keyword ``out_dtype`` (bf16 output, opt-in; fp32 by default).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import numpy as np
import torch

from prometheus_amd import _native

Array = Any  # torch.Tensor or numpy.ndarray

# Chunk width for the delta-rule tiling (kernels/__init__.py:80).
DEFAULT_CHUNK = 64


class KernelError(ValueError):
    """Shape, dtype, or routing invariant failed before the kernel ran.

    Same class as ``kernels/__init__.py:68-69``.
    """


@dataclass(frozen=True)
class LinearAttnConfig:
    """Chunked delta-rule knobs. ``chunk`` does not change the mathematical result.

    Same fields and defaults as ``kernels/__init__.py:90-95``; ``eps`` is
    unused there and here. The GPU kernel tiles by 64 tokens whatever
    ``chunk`` says; ``chunk`` is validated (>= 1) and kept in the residual.
    """

    chunk: int = DEFAULT_CHUNK
    eps: float = 1e-6


@dataclass(frozen=True)
class _DeltaResidual:
    """Residual of ``chunked_delta_rule_fwd`` (``kernels/__init__.py:148-163``).

    ``q, k, v, beta, state0`` are the arrays the kernel consumed (not
    copied: bf16 inputs stay bf16, a documented difference from the
    reference's fp32 copies); ``state0`` is fp32, zeros when ``state`` was
    None; ``chunk`` is a Python int.
    """

    q: Array
    k: Array
    v: Array
    beta: Array
    state0: Array
    chunk: int


# ---------------------------------------------------------------------------
# argument normalisation
# ---------------------------------------------------------------------------


def _on_host(*xs) -> bool:
    """True when no argument is a GPU tensor (the reference's host-array path)."""
    return not any(isinstance(x, torch.Tensor) and x.device.type == "cuda" for x in xs)


def _shape(x) -> tuple:
    return tuple(x.shape) if hasattr(x, "shape") else tuple(np.shape(x))


def _check_chunk(config: LinearAttnConfig) -> int:
    if config.chunk < 1:
        raise KernelError(f"chunk must be >= 1, got {config.chunk}")
    return int(config.chunk)


def _validate(q, k, v, beta, state) -> tuple[int, int, int, int]:
    """Shape checks of ``kernels/__init__.py:308-338`` on any array type."""
    qs, ks, vs, bs = _shape(q), _shape(k), _shape(v), _shape(beta)
    if len(qs) != 4 or ks != qs or vs != qs:
        raise KernelError(f"q, k, v must all have shape (B, S, H, D); got {qs}")
    batch, seq, heads, dim = qs
    if bs != (batch, seq, heads):
        raise KernelError(f"beta shape {bs} != {(batch, seq, heads)}")
    if state is not None and _shape(state) != (batch, heads, dim, dim):
        raise KernelError(f"state shape {_shape(state)} != {(batch, heads, dim, dim)}")
    if dim > _native.MAX_D:
        raise KernelError(f"head dimension {dim} exceeds the supported maximum {_native.MAX_D}")
    return batch, seq, heads, dim


def _check_beta_host(beta) -> None:
    """``beta < 0`` check of the reference's host path (kernels/__init__.py:317-318)."""
    if isinstance(beta, torch.Tensor):
        b = beta.detach().cpu().float().numpy()
    else:
        b = np.asarray(beta, dtype=np.float32)
    if np.any(b < 0):
        raise KernelError("beta must be in (0, 1]")


def _device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("prometheus_amd.kernels needs a HIP GPU; none is visible")
    return torch.device("cuda", torch.cuda.current_device())


class _Call:
    """Moves a call's arrays onto one GPU and remembers how to give results back."""

    def __init__(self, *xs):
        tensors = [x for x in xs if isinstance(x, torch.Tensor)]
        dev_tensors = [t for t in tensors if t.device.type == "cuda"]
        self.host_numpy = not tensors
        self.host_torch = bool(tensors) and not dev_tensors
        if dev_tensors:
            self.device = dev_tensors[0].device
            for t in dev_tensors:
                if t.device != self.device:
                    raise KernelError("all tensors must be on the same device")
        else:
            self.device = _device()

    def dev(self, x, dtype=None):
        if x is None:
            return None
        if isinstance(x, torch.Tensor):
            t = x
        else:
            t = torch.from_numpy(np.ascontiguousarray(np.asarray(x, dtype=np.float32)))
        if dtype is not None and t.dtype != dtype:
            t = t.to(dtype)
        return t.to(self.device, non_blocking=False).contiguous()

    def out(self, t):
        if self.host_numpy:
            return t.cpu().numpy()
        if self.host_torch:
            return t.cpu()
        return t


def _qkv_dtype(q, k, v) -> torch.dtype:
    dts = {x.dtype for x in (q, k, v) if isinstance(x, torch.Tensor)}
    if dts == {torch.bfloat16} and all(isinstance(x, torch.Tensor) for x in (q, k, v)):
        return torch.bfloat16
    return torch.float32


def _out_dtype(out_dtype) -> torch.dtype:
    if out_dtype is None or out_dtype in (torch.float32, np.float32, "fp32", "float32"):
        return torch.float32
    if out_dtype in (torch.bfloat16, "bf16", "bfloat16"):
        return torch.bfloat16
    raise KernelError(f"out_dtype must be fp32 (default) or bf16, got {out_dtype!r}")


def _code(dt: torch.dtype) -> int:
    return _native.DTYPE_BF16 if dt == torch.bfloat16 else _native.DTYPE_F32


def _ptr(t) -> int | None:
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _aligned16(t):
    return t if t is None or t.numel() == 0 or t.data_ptr() % 16 == 0 else t.clone()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


# ---------------------------------------------------------------------------
# forward
# ---------------------------------------------------------------------------


def _forward(q, k, v, beta, state, chunk: int, out_dtype):
    batch, seq, heads, dim = _validate(q, k, v, beta, state)
    odt = _out_dtype(out_dtype)
    if _on_host(q, k, v, beta, state):
        _check_beta_host(beta)
    call = _Call(q, k, v, beta, state)
    cdt = _qkv_dtype(q, k, v)
    with torch.cuda.device(call.device):
        qd, kd, vd = call.dev(q, cdt), call.dev(k, cdt), call.dev(v, cdt)
        bd = call.dev(beta, torch.float32)
        sd = call.dev(state, torch.float32)
        o = torch.empty((batch, seq, heads, dim), dtype=odt, device=call.device)
        s_out = torch.empty((batch, heads, dim, dim), dtype=torch.float32, device=call.device)
        # the split form's T workspace, where the C ABI would use it (torch's caching allocator)
        nbytes = _native.lib().pm_delta_workspace_bytes(batch, seq, heads, dim, _code(cdt))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=call.device) if nbytes else None
        rc = _native.lib().pm_delta_fwd(
            _ptr(qd), _ptr(kd), _ptr(vd), _ptr(bd), _ptr(sd), _ptr(o), _ptr(s_out),
            batch, seq, heads, dim, _code(cdt), _code(odt), chunk, _ptr(ws), nbytes,
            _stream(call.device),
        )
        _native.check(rc)
        if sd is None:
            sd = torch.zeros((batch, heads, dim, dim), dtype=torch.float32, device=call.device)
    return call, (qd, kd, vd, bd, sd), o, s_out


def _wants_grad(*xs) -> bool:
    return torch.is_grad_enabled() and any(isinstance(x, torch.Tensor) and x.requires_grad for x in xs)


class _ChunkedDeltaRule(torch.autograd.Function):
    """``chunked_delta_rule`` as a differentiable op: the forward kernel, and
    ``chunked_delta_rule_bwd`` (pm_delta_bwd) as its backward -- the torch form of
    the reference's ``jax.custom_vjp`` (kernels/__init__.py:591-658).  The config
    is not differentiated; a ``state=None`` input has no gradient.  Gradients
    come back in each input's dtype and device (autograd's contract); they are
    computed in fp32 as the backward's outputs are."""

    @staticmethod
    def forward(ctx, q, k, v, beta, state, chunk, out_dtype):
        call, (qd, kd, vd, bd, sd), o, s = _forward(q, k, v, beta, state, chunk, out_dtype)
        ctx.save_for_backward(qd, kd, vd, bd, sd)
        ctx.chunk = chunk
        ctx.like = [(x.dtype, x.device) if isinstance(x, torch.Tensor) else None
                    for x in (q, k, v, beta, state)]
        # the library's kernel knobs are per thread and autograd may run the backward on
        # another thread: the backward runs under the forward caller's selection
        ctx.knobs = _native.knobs()
        return call.out(o), call.out(s)

    @staticmethod
    def backward(ctx, go, gs):
        qd, kd, vd, bd, sd = ctx.saved_tensors
        res = _DeltaResidual(q=qd, k=kd, v=vd, beta=bd, state0=sd, chunk=ctx.chunk)
        with _native.use_knobs(*ctx.knobs):
            grads = chunked_delta_rule_bwd(res, (go, gs))
        out = []
        for g, like, need in zip(grads, ctx.like, ctx.needs_input_grad[:5]):
            out.append(g.to(device=like[1], dtype=like[0]) if (like is not None and need) else None)
        return (*out, None, None)


def chunked_delta_rule(q, k, v, beta, state=None, config=None, *, out_dtype=None):
    """Gated delta-rule linear attention (``kernels/__init__.py:591-619``).

    q, k, v: (batch, seq, heads, dim). beta: (batch, seq, heads) gate in (0, 1].
    state: (batch, heads, dim, dim) recurrent state, zeros if None.
    Returns ``(output, next_state)``; output shaped like v (fp32 unless
    ``out_dtype`` asks for bf16), next_state fp32.

    Differentiable like the reference's ``custom_vjp``: when autograd records
    and a torch input requires grad, ``torch.autograd.grad`` / ``backward``
    through ``(output, next_state)`` runs ``chunked_delta_rule_bwd`` (the
    fused reverse kernels), never an unrolled graph of the recurrence.
    """
    cfg = LinearAttnConfig() if config is None else config
    chunk = _check_chunk(cfg)
    if _wants_grad(q, k, v, beta, state):
        _validate(q, k, v, beta, state)
        return _ChunkedDeltaRule.apply(q, k, v, beta, state, chunk, out_dtype)
    call, _, o, s = _forward(q, k, v, beta, state, chunk, out_dtype)
    return call.out(o), call.out(s)


def chunked_delta_rule_fwd(q, k, v, beta, state, config, *, out_dtype=None):
    """Explicit forward of the VJP pair (``kernels/__init__.py:661-689``).

    Returns ``((output, next_state), _DeltaResidual)``.
    """
    chunk = _check_chunk(config)
    call, (qd, kd, vd, bd, sd), o, s = _forward(q, k, v, beta, state, chunk, out_dtype)
    if call.host_numpy:
        residual = _DeltaResidual(
            q=np.asarray(q, dtype=np.float32), k=np.asarray(k, dtype=np.float32),
            v=np.asarray(v, dtype=np.float32), beta=np.asarray(beta, dtype=np.float32),
            state0=sd.cpu().numpy(), chunk=chunk,
        )
    else:
        residual = _DeltaResidual(q=call.out(qd), k=call.out(kd), v=call.out(vd),
                                  beta=call.out(bd), state0=call.out(sd), chunk=chunk)
    return (call.out(o), call.out(s)), residual


def chunked_delta_rule_bwd(residual: _DeltaResidual, grads):
    """Backward of the VJP pair (``kernels/__init__.py:692-719``).

    ``grads = (go, gs)``: dL/dO (B, T, H, D) and dL/dS_T (B, H, D, D), either
    may be None (zeros, as the custom-VJP rule treats missing cotangents,
    ``:638-653``). Returns ``(gq, gk, gv, gbeta, gstate)``, all fp32, shaped
    like ``q, k, v, beta, state0``: the gradients of the reference's
    ``_delta_vjp_np`` / ``_delta_vjp_jax`` (``:460-588``). Head dimension up
    to 256. As in the forward, head dimension 64 or 128 runs a chunked
    backward: on bf16 MFMA for bf16 q/k/v (bf16 parity), on fp32 MFMA for
    fp32 q/k/v (fp32 parity); everything else runs the fp32 per-token
    reverse-mode kernel with state checkpoints (fp32 parity). None keeps the
    reference's per-token state history.
    """
    go, gs = grads
    q, k, v, beta, s0 = residual.q, residual.k, residual.v, residual.beta, residual.state0
    batch, seq, heads, dim = _validate(q, k, v, beta, s0)
    if dim > _native.MAX_D_BWD:
        raise KernelError(f"backward head dimension {dim} exceeds {_native.MAX_D_BWD}")
    if go is not None and _shape(go) != (batch, seq, heads, dim):
        raise KernelError(f"grad of output shape {_shape(go)} != {(batch, seq, heads, dim)}")
    if gs is not None and _shape(gs) != (batch, heads, dim, dim):
        raise KernelError(f"grad of state shape {_shape(gs)} != {(batch, heads, dim, dim)}")
    call = _Call(q, k, v, beta, s0, go, gs)
    cdt = _qkv_dtype(q, k, v)
    f32 = torch.float32
    with torch.cuda.device(call.device):
        qd, kd, vd = call.dev(q, cdt), call.dev(k, cdt), call.dev(v, cdt)
        bd, sd = call.dev(beta, f32), call.dev(s0, f32)
        god, gsd = call.dev(go, f32), call.dev(gs, f32)
        # the chunked backward reads q, k, v and dO with 16-byte vector loads: a view at an
        # odd offset is copied to a fresh (aligned) buffer rather than refused
        qd, kd, vd, god = (_aligned16(x) for x in (qd, kd, vd, god))
        gq = torch.empty((batch, seq, heads, dim), dtype=f32, device=call.device)
        gk, gv = torch.empty_like(gq), torch.empty_like(gq)
        gb = torch.empty((batch, seq, heads), dtype=f32, device=call.device)
        gs0 = torch.empty((batch, heads, dim, dim), dtype=f32, device=call.device)
        L = _native.lib()
        nbytes = L.pm_delta_bwd_workspace_bytes(batch, seq, heads, dim, _code(cdt))
        ws = torch.empty(((nbytes + 3) // 4,), dtype=f32, device=call.device) if nbytes else None
        rc = L.pm_delta_bwd(
            _ptr(qd), _ptr(kd), _ptr(vd), _ptr(bd), _ptr(sd), _ptr(god), _ptr(gsd),
            _ptr(gq), _ptr(gk), _ptr(gv), _ptr(gb), _ptr(gs0),
            batch, seq, heads, dim, _code(cdt), _ptr(ws), nbytes, _stream(call.device),
        )
        _native.check(rc)
    return tuple(call.out(x) for x in (gq, gk, gv, gb, gs0))


# ---------------------------------------------------------------------------
# packed variable-length forward (no reference counterpart)
# ---------------------------------------------------------------------------


def _validate_cu(cu_host: np.ndarray, total: int) -> None:
    if cu_host.ndim != 1 or cu_host.size < 1:
        raise KernelError("cu_seqlens must be a 1-D array of n_seqs + 1 offsets")
    if cu_host[0] != 0 or cu_host[-1] != total:
        raise KernelError(f"cu_seqlens must start at 0 and end at {total}; got "
                          f"{int(cu_host[0])}..{int(cu_host[-1])}")
    if np.any(np.diff(cu_host) < 0):
        raise KernelError("cu_seqlens must be non-decreasing")


# Per-device flag words of the device-side cu_seqlens check (pm_varlen_check).
_VARLEN_FLAGS: dict = {}
_VARLEN_BITS = {1: "cu_seqlens[0] != 0", 2: "cu_seqlens[-1] != N", 4: "decreasing offsets",
                8: "an offset outside [0, N]"}


def _varlen_flag(device) -> torch.Tensor:
    flag = _VARLEN_FLAGS.get(device)
    if flag is None:
        if torch.cuda.is_current_stream_capturing():
            raise KernelError("the device-side cu_seqlens check keeps one flag word per device: run "
                              "check_varlen(device) (or one varlen call) there before capturing a graph")
        flag = torch.zeros(1, dtype=torch.int32, device=device)
        _VARLEN_FLAGS[device] = flag
    return flag


def check_varlen(device=None) -> None:
    """Surface what the device-side checks of ``chunked_delta_rule_varlen`` found.

    A ``cu_seqlens`` tensor already on the GPU is checked by a kernel on the call's
    stream (no host copy, no synchronisation; graph-capturable), which records any
    malformed offsets in a per-device flag word. This synchronises with the device,
    clears the flag and raises ``KernelError`` naming what was found since the last
    check. (The forward kernels clamp every segment into [0, N] themselves, so bad
    offsets never reach outside the buffers.)
    """
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    flag = _varlen_flag(dev)
    bits = int(flag.item())
    if bits:
        flag.zero_()
        found = ", ".join(msg for b, msg in _VARLEN_BITS.items() if bits & b)
        raise KernelError(f"a device cu_seqlens passed to chunked_delta_rule_varlen was malformed: {found}")


def chunked_delta_rule_varlen(q, k, v, beta, cu_seqlens, state=None, config=None, *,
                              out_dtype=None):
    """Packed batch of independent sequences, state reset at every boundary.

    q, k, v: (N, H, D) or (1, N, H, D); beta: (N, H) or (1, N, H);
    cu_seqlens: int32 (n_seqs + 1,) exclusive prefix, 0 .. N;
    state: None (zeros) or (n_seqs, H, D, D) initial states.
    Returns ``(output, final_states)`` with output shaped like q and
    final_states (n_seqs, H, D, D) fp32. Each segment equals a B=1
    ``chunked_delta_rule`` call on that segment alone, bit for bit, when both
    calls run the same kernel form (``pm_delta_set_path`` 1, 2 or 3; the default
    picks the form from a call's (sequence, head) count, and two forms agree within
    the bf16 bound).

    ``cu_seqlens`` on the host (NumPy, a CPU tensor) is validated here before any
    device work. A GPU tensor (int32, or int64 converted on the device) is never
    copied to the host: a kernel on the call's stream checks it and records what it
    finds for ``check_varlen`` to report, so the call stays free of synchronisation
    and can be captured in a graph.
    """
    cfg = LinearAttnConfig() if config is None else config
    chunk = _check_chunk(cfg)
    qs = _shape(q)
    lead4 = len(qs) == 4
    if lead4:
        if qs[0] != 1:
            raise KernelError(f"packed q must be (N, H, D) or (1, N, H, D); got {qs}")
        qs = qs[1:]
    if len(qs) != 3 or _shape(k)[-3:] != qs or _shape(v)[-3:] != qs:
        raise KernelError(f"q, k, v must all have shape (N, H, D); got {_shape(q)}")
    n_tok, heads, dim = qs
    bs = _shape(beta)
    if bs not in ((n_tok, heads), (1, n_tok, heads)):
        raise KernelError(f"beta shape {bs} != {(n_tok, heads)}")
    if dim > _native.MAX_D:
        raise KernelError(f"head dimension {dim} exceeds the supported maximum {_native.MAX_D}")
    cu_on_dev = isinstance(cu_seqlens, torch.Tensor) and cu_seqlens.device.type == "cuda"
    if cu_on_dev:
        if cu_seqlens.dim() != 1 or cu_seqlens.numel() < 1:
            raise KernelError("cu_seqlens must be a 1-D array of n_seqs + 1 offsets")
        if cu_seqlens.dtype not in (torch.int32, torch.int64):
            raise KernelError(f"cu_seqlens must be an integer array, got {cu_seqlens.dtype}")
        if n_tok >= 2**31:
            raise KernelError("cu_seqlens exceeds int32")
        n_seqs = cu_seqlens.numel() - 1
    else:
        if isinstance(cu_seqlens, torch.Tensor):
            cu_host = cu_seqlens.detach().numpy()
        else:
            cu_host = np.asarray(cu_seqlens)
        if not np.issubdtype(cu_host.dtype, np.integer):
            raise KernelError(f"cu_seqlens must be an integer array, got {cu_host.dtype}")
        cu_host = cu_host.astype(np.int64)
        _validate_cu(cu_host, n_tok)
        if cu_host[-1] >= 2**31:
            raise KernelError("cu_seqlens exceeds int32")
        n_seqs = cu_host.size - 1
    if state is not None and _shape(state) != (n_seqs, heads, dim, dim):
        raise KernelError(f"state shape {_shape(state)} != {(n_seqs, heads, dim, dim)}")

    odt = _out_dtype(out_dtype)
    if _on_host(q, k, v, beta, state):
        _check_beta_host(beta)
    call = _Call(q, k, v, beta, state, cu_seqlens)
    cdt = _qkv_dtype(q, k, v)
    with torch.cuda.device(call.device):
        qd = call.dev(q, cdt).reshape(n_tok, heads, dim)
        kd = call.dev(k, cdt).reshape(n_tok, heads, dim)
        vd = call.dev(v, cdt).reshape(n_tok, heads, dim)
        bd = call.dev(beta, torch.float32).reshape(n_tok, heads)
        sd = call.dev(state, torch.float32)
        if cu_on_dev:
            cu = cu_seqlens.to(torch.int32).contiguous()
            _native.check(_native.lib().pm_varlen_check(_ptr(cu), n_seqs, n_tok,
                                                        _varlen_flag(call.device).data_ptr(),
                                                        _stream(call.device)))
        else:
            cu = torch.from_numpy(cu_host.astype(np.int32)).to(call.device)
        o = torch.empty((n_tok, heads, dim), dtype=odt, device=call.device)
        s_out = torch.empty((n_seqs, heads, dim, dim), dtype=torch.float32, device=call.device)
        nbytes = _native.lib().pm_delta_varlen_workspace_bytes(n_seqs, n_tok, heads, dim, _code(cdt))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=call.device) if nbytes else None
        rc = _native.lib().pm_delta_fwd_varlen(
            _ptr(qd), _ptr(kd), _ptr(vd), _ptr(bd), _ptr(cu), n_seqs, n_tok, _ptr(sd),
            _ptr(o), _ptr(s_out), heads, dim, _code(cdt), _code(odt), chunk, _ptr(ws), nbytes,
            _stream(call.device),
        )
        _native.check(rc)
    if lead4:
        o = o.reshape(1, n_tok, heads, dim)
    return call.out(o), call.out(s_out)


# ---------------------------------------------------------------------------
# single-token decode step (public form of kernels/__init__.py:357-376)
# ---------------------------------------------------------------------------


def delta_rule_step(q, k, v, beta, state):
    """One recurrent step for (B, H, D) tokens; ``state`` (B, H, D, D) updated in place.

    Same algebra as ``_delta_step_np`` / ``_delta_step_jax``
    (``kernels/__init__.py:357-376``): ``S' = S - beta k (k^T S) + beta k v^T``
    and ``o = q S'``. ``state`` must be fp32: a contiguous GPU tensor is
    updated on the device, a NumPy array or CPU tensor is updated through a
    copy. Returns o (B, H, D) fp32.
    """
    qs = _shape(q)
    if len(qs) != 3 or _shape(k) != qs or _shape(v) != qs:
        raise KernelError(f"q, k, v must all have shape (B, H, D); got {qs}")
    batch, heads, dim = qs
    if _shape(beta) != (batch, heads):
        raise KernelError(f"beta shape {_shape(beta)} != {(batch, heads)}")
    if state is None or _shape(state) != (batch, heads, dim, dim):
        raise KernelError(f"state shape {_shape(state) if state is not None else None} != "
                          f"{(batch, heads, dim, dim)}")
    if dim > _native.MAX_D:
        raise KernelError(f"head dimension {dim} exceeds the supported maximum {_native.MAX_D}")
    in_place = isinstance(state, torch.Tensor) and state.device.type == "cuda"
    if in_place and (state.dtype != torch.float32 or not state.is_contiguous()):
        raise KernelError("state must be a contiguous fp32 tensor to be updated in place")
    if isinstance(state, np.ndarray) and state.dtype != np.float32:
        raise KernelError("state must be fp32 to be updated in place")
    if _on_host(q, k, v, beta, state):
        _check_beta_host(beta)
    call = _Call(q, k, v, beta, state)
    cdt = _qkv_dtype(q, k, v)
    with torch.cuda.device(call.device):
        qd, kd, vd = call.dev(q, cdt), call.dev(k, cdt), call.dev(v, cdt)
        bd = call.dev(beta, torch.float32)
        sd = state if in_place else call.dev(state, torch.float32)
        o = torch.empty((batch, heads, dim), dtype=torch.float32, device=call.device)
        rc = _native.lib().pm_delta_step(_ptr(sd), _ptr(qd), _ptr(kd), _ptr(vd), _ptr(bd),
                                         _ptr(o), batch, heads, dim, _code(cdt),
                                         _stream(call.device))
        _native.check(rc)
        if not in_place:
            host = sd.cpu()
            if isinstance(state, np.ndarray):
                state[...] = host.numpy()
            else:
                state.copy_(host)
    return call.out(o)


# ---------------------------------------------------------------------------
# gated variant (no reference code: the model's intent, spec/03-model.md:12)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class _GatedDeltaResidual:
    """Residual of ``chunked_gated_delta_rule_fwd``: ``_DeltaResidual``'s fields plus the
    log-gates ``g`` (the arrays the kernel consumed, not copied)."""

    q: Array
    k: Array
    v: Array
    beta: Array
    g: Array
    state0: Array
    chunk: int


def _gated_forward(q, k, v, beta, g, state, out_dtype, per_channel=False):
    batch, seq, heads, dim = _validate(q, k, v, beta, state)
    gshape = (batch, seq, heads, dim) if per_channel else (batch, seq, heads)
    if _shape(g) != gshape:
        raise KernelError(f"g shape {_shape(g)} != {gshape}")
    odt = _out_dtype(out_dtype)
    if _on_host(q, k, v, beta, state):
        _check_beta_host(beta)
    call = _Call(q, k, v, beta, g, state)
    cdt = _qkv_dtype(q, k, v)
    with torch.cuda.device(call.device):
        qd, kd, vd = call.dev(q, cdt), call.dev(k, cdt), call.dev(v, cdt)
        bd, gd = call.dev(beta, torch.float32), call.dev(g, torch.float32)
        sd = call.dev(state, torch.float32)
        o = torch.empty((batch, seq, heads, dim), dtype=odt, device=call.device)
        s_out = torch.empty((batch, heads, dim, dim), dtype=torch.float32, device=call.device)
        L = _native.lib()
        if per_channel:
            nbytes = L.pm_kda_delta_workspace_bytes(batch, seq, heads, dim, _code(cdt))
            ws = torch.empty((nbytes,), dtype=torch.uint8, device=call.device) if nbytes else None
            rc = L.pm_kda_delta_fwd(
                _ptr(qd), _ptr(kd), _ptr(vd), _ptr(bd), _ptr(gd), _ptr(sd), _ptr(o), _ptr(s_out),
                batch, seq, heads, dim, _code(cdt), _code(odt), _ptr(ws), nbytes, _stream(call.device),
            )
        else:
            rc = L.pm_gated_delta_fwd(
                _ptr(qd), _ptr(kd), _ptr(vd), _ptr(bd), _ptr(gd), _ptr(sd), _ptr(o), _ptr(s_out),
                batch, seq, heads, dim, _code(cdt), _code(odt), _stream(call.device),
            )
        _native.check(rc)
        if sd is None:
            sd = torch.zeros((batch, heads, dim, dim), dtype=torch.float32, device=call.device)
    return call, (qd, kd, vd, bd, gd, sd), o, s_out


def chunked_gated_delta_rule_bwd(residual: _GatedDeltaResidual, grads):
    """Backward of the gated VJP pair: ``grads = (go, gs)`` as ``chunked_delta_rule_bwd``
    (either may be None). Returns ``(gq, gk, gv, gbeta, gg, gstate)``, fp32, shaped like
    ``q, k, v, beta, g, state0``. Runs the per-token fp32 reverse-mode kernels
    (``pm_gated_delta_bwd``) for every dtype and head dimension up to 256: with P_t =
    exp(g_t) S_{t-1}, dL/dg_t = <G - beta_t k_t w^T, P_t> and G <- exp(g_t) (G - beta_t
    k_t w^T), the other gradients as in the ungated backward."""
    return _gated_bwd(residual, grads, per_channel=False)


def chunked_kda_rule_bwd(residual: _GatedDeltaResidual, grads):
    """Backward of ``chunked_kda_rule_fwd``: as ``chunked_gated_delta_rule_bwd`` with g
    and gg (batch, seq, heads, dim). With P_t = Diag(exp(g_t)) S_{t-1}, dL/dg_t[d] =
    <G_P[d, :], P_t[d, :]> (G_P = G - beta_t k_t w^T) and G <- Diag(exp(g_t)) G_P
    (``pm_kda_delta_bwd``, the per-token fp32 kernels, head dimension up to 256)."""
    return _gated_bwd(residual, grads, per_channel=True)


def _gated_bwd(residual, grads, per_channel):
    go, gs = grads
    q, k, v, beta, g, s0 = residual.q, residual.k, residual.v, residual.beta, residual.g, residual.state0
    batch, seq, heads, dim = _validate(q, k, v, beta, s0)
    gshape = (batch, seq, heads, dim) if per_channel else (batch, seq, heads)
    if _shape(g) != gshape:
        raise KernelError(f"g shape {_shape(g)} != {gshape}")
    if dim > _native.MAX_D_BWD:
        raise KernelError(f"backward head dimension {dim} exceeds {_native.MAX_D_BWD}")
    if go is not None and _shape(go) != (batch, seq, heads, dim):
        raise KernelError(f"grad of output shape {_shape(go)} != {(batch, seq, heads, dim)}")
    if gs is not None and _shape(gs) != (batch, heads, dim, dim):
        raise KernelError(f"grad of state shape {_shape(gs)} != {(batch, heads, dim, dim)}")
    call = _Call(q, k, v, beta, g, s0, go, gs)
    cdt = _qkv_dtype(q, k, v)
    f32 = torch.float32
    with torch.cuda.device(call.device):
        qd, kd, vd = call.dev(q, cdt), call.dev(k, cdt), call.dev(v, cdt)
        bd, gd, sd = call.dev(beta, f32), call.dev(g, f32), call.dev(s0, f32)
        god, gsd = call.dev(go, f32), call.dev(gs, f32)
        gq = torch.empty((batch, seq, heads, dim), dtype=f32, device=call.device)
        gk, gv = torch.empty_like(gq), torch.empty_like(gq)
        gb = torch.empty((batch, seq, heads), dtype=f32, device=call.device)
        gg = torch.empty(gshape, dtype=f32, device=call.device)
        gs0 = torch.empty((batch, heads, dim, dim), dtype=f32, device=call.device)
        L = _native.lib()
        wsf = L.pm_kda_delta_bwd_workspace_bytes if per_channel else L.pm_gated_delta_bwd_workspace_bytes
        nbytes = wsf(batch, seq, heads, dim, _code(cdt))
        ws = torch.empty(((nbytes + 3) // 4,), dtype=f32, device=call.device) if nbytes else None
        rc = (L.pm_kda_delta_bwd if per_channel else L.pm_gated_delta_bwd)(
            _ptr(qd), _ptr(kd), _ptr(vd), _ptr(bd), _ptr(gd), _ptr(sd), _ptr(god), _ptr(gsd),
            _ptr(gq), _ptr(gk), _ptr(gv), _ptr(gb), _ptr(gg), _ptr(gs0),
            batch, seq, heads, dim, _code(cdt), _ptr(ws), nbytes, _stream(call.device),
        )
        _native.check(rc)
    return tuple(call.out(x) for x in (gq, gk, gv, gb, gg, gs0))


class _ChunkedGatedDeltaRule(torch.autograd.Function):
    """``chunked_gated_delta_rule`` (``per_channel``: ``chunked_kda_rule``) as a
    differentiable op: the gated forward kernel and ``chunked_gated_delta_rule_bwd``
    (``chunked_kda_rule_bwd``) as its backward (gradients for q, k, v, beta, g and the
    state, in each input's dtype and device)."""

    @staticmethod
    def forward(ctx, q, k, v, beta, g, state, chunk, out_dtype, per_channel=False):
        call, (qd, kd, vd, bd, gd, sd), o, s = _gated_forward(q, k, v, beta, g, state, out_dtype, per_channel)
        ctx.save_for_backward(qd, kd, vd, bd, gd, sd)
        ctx.chunk = chunk
        ctx.per_channel = per_channel
        ctx.like = [(x.dtype, x.device) if isinstance(x, torch.Tensor) else None
                    for x in (q, k, v, beta, g, state)]
        ctx.knobs = _native.knobs()
        return call.out(o), call.out(s)

    @staticmethod
    def backward(ctx, go, gs):
        qd, kd, vd, bd, gd, sd = ctx.saved_tensors
        res = _GatedDeltaResidual(q=qd, k=kd, v=vd, beta=bd, g=gd, state0=sd, chunk=ctx.chunk)
        with _native.use_knobs(*ctx.knobs):
            grads = _gated_bwd(res, (go, gs), ctx.per_channel)
        out = []
        for gr, like, need in zip(grads, ctx.like, ctx.needs_input_grad[:6]):
            out.append(gr.to(device=like[1], dtype=like[0]) if (like is not None and need) else None)
        return (*out, None, None, None)


def chunked_gated_delta_rule(q, k, v, beta, g, state=None, config=None, *, out_dtype=None):
    """Gated delta rule (Gated DeltaNet) with a log-gate per token and head.

    ``S_t = exp(g_t) (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T``,
    ``o_t = q_t S_t``. q, k, v, beta, state and the return value as
    ``chunked_delta_rule``; g: (batch, seq, heads) fp32 log-gates (g = 0 gives
    ``chunked_delta_rule``). bf16 q/k/v with dim 64 or 128 run the chunked
    MFMA kernel with the in-chunk decays folded into its tiles; other inputs
    run the fp32 per-token kernel. Differentiable: when autograd records and a
    torch input (the gates included) requires grad, the backward runs
    ``chunked_gated_delta_rule_bwd``.
    """
    cfg = LinearAttnConfig() if config is None else config
    chunk = _check_chunk(cfg)
    if _wants_grad(q, k, v, beta, g, state):
        _validate(q, k, v, beta, state)
        return _ChunkedGatedDeltaRule.apply(q, k, v, beta, g, state, chunk, out_dtype)
    call, _, o, s = _gated_forward(q, k, v, beta, g, state, out_dtype)
    return call.out(o), call.out(s)


def chunked_gated_delta_rule_fwd(q, k, v, beta, g, state, config, *, out_dtype=None):
    """Explicit forward of the gated VJP pair: ``((output, next_state), _GatedDeltaResidual)``."""
    return _gated_fwd_pair(q, k, v, beta, g, state, config, out_dtype, per_channel=False)


def _gated_fwd_pair(q, k, v, beta, g, state, config, out_dtype, per_channel):
    chunk = _check_chunk(config)
    call, (qd, kd, vd, bd, gd, sd), o, s = _gated_forward(q, k, v, beta, g, state, out_dtype, per_channel)
    if call.host_numpy:
        residual = _GatedDeltaResidual(
            q=np.asarray(q, dtype=np.float32), k=np.asarray(k, dtype=np.float32),
            v=np.asarray(v, dtype=np.float32), beta=np.asarray(beta, dtype=np.float32),
            g=np.asarray(g, dtype=np.float32), state0=sd.cpu().numpy(), chunk=chunk)
    else:
        residual = _GatedDeltaResidual(q=call.out(qd), k=call.out(kd), v=call.out(vd), beta=call.out(bd),
                                       g=call.out(gd), state0=call.out(sd), chunk=chunk)
    return (call.out(o), call.out(s)), residual


def chunked_kda_rule(q, k, v, beta, g, state=None, config=None, *, out_dtype=None):
    """The delta rule with a decay per key channel (KDA, Kimi Delta Attention).

    ``S_t = (I - beta_t k_t k_t^T) Diag(exp(g_t)) S_{t-1} + beta_t k_t v_t^T``,
    ``o_t = q_t S_t``. q, k, v, beta, state and the return value as
    ``chunked_delta_rule``; g: (batch, seq, heads, dim) fp32 log-gates, one per
    key channel (g constant along dim gives ``chunked_gated_delta_rule``). bf16 q/k/v
    with dim 64 or 128 run the chunked WY form on bf16 MFMA (``pm_kda_delta_fwd`` with
    a workspace; log-gates clamped into [-10, 1] there); other inputs run the fp32
    per-token kernel for every dim up to 256.
    Differentiable: when autograd records and a torch input (the gates included)
    requires grad, the backward runs ``chunked_kda_rule_bwd``.
    """
    cfg = LinearAttnConfig() if config is None else config
    chunk = _check_chunk(cfg)
    if _wants_grad(q, k, v, beta, g, state):
        _validate(q, k, v, beta, state)
        return _ChunkedGatedDeltaRule.apply(q, k, v, beta, g, state, chunk, out_dtype, True)
    call, _, o, s = _gated_forward(q, k, v, beta, g, state, out_dtype, per_channel=True)
    return call.out(o), call.out(s)


def chunked_kda_rule_fwd(q, k, v, beta, g, state, config, *, out_dtype=None):
    """Explicit forward of the KDA VJP pair: ``((output, next_state), residual)`` for
    ``chunked_kda_rule_bwd``."""
    return _gated_fwd_pair(q, k, v, beta, g, state, config, out_dtype, per_channel=True)


def gated_delta_rule_step(q, k, v, beta, g, state):
    """One gated step for (B, H, D) tokens, g (B, H); ``state`` updated in place as in
    ``delta_rule_step``: ``S' = exp(g) (S - beta k (k^T S)) + beta k v^T``, ``o = q S'``."""
    return _gated_step(q, k, v, beta, g, state, per_channel=False)


def kda_delta_rule_step(q, k, v, beta, g, state):
    """One KDA step for (B, H, D) tokens, g (B, H, D) log-gates per key channel;
    ``state`` updated in place: ``S' = (I - beta k k^T) Diag(exp(g)) S + beta k v^T``,
    ``o = q S'``."""
    return _gated_step(q, k, v, beta, g, state, per_channel=True)


def _gated_step(q, k, v, beta, g, state, per_channel):
    qs = _shape(q)
    if len(qs) != 3 or _shape(k) != qs or _shape(v) != qs:
        raise KernelError(f"q, k, v must all have shape (B, H, D); got {qs}")
    batch, heads, dim = qs
    gshape = (batch, heads, dim) if per_channel else (batch, heads)
    if _shape(beta) != (batch, heads) or _shape(g) != gshape:
        raise KernelError(f"beta must be {(batch, heads)} and g {gshape}; got {_shape(beta)}, {_shape(g)}")
    if state is None or _shape(state) != (batch, heads, dim, dim):
        raise KernelError(f"state shape {_shape(state) if state is not None else None} != "
                          f"{(batch, heads, dim, dim)}")
    if dim > _native.MAX_D:
        raise KernelError(f"head dimension {dim} exceeds the supported maximum {_native.MAX_D}")
    if not (isinstance(state, torch.Tensor) and state.device.type == "cuda"
            and state.dtype == torch.float32 and state.is_contiguous()):
        raise KernelError("state must be a contiguous fp32 GPU tensor (updated in place)")
    call = _Call(q, k, v, beta, g, state)
    cdt = _qkv_dtype(q, k, v)
    with torch.cuda.device(call.device):
        qd, kd, vd = call.dev(q, cdt), call.dev(k, cdt), call.dev(v, cdt)
        bd, gd = call.dev(beta, torch.float32), call.dev(g, torch.float32)
        o = torch.empty((batch, heads, dim), dtype=torch.float32, device=call.device)
        stepf = _native.lib().pm_kda_delta_step if per_channel else _native.lib().pm_gated_delta_step
        rc = stepf(_ptr(state), _ptr(qd), _ptr(kd), _ptr(vd), _ptr(bd), _ptr(gd), _ptr(o), batch, heads,
                   dim, _code(cdt), _stream(call.device))
        _native.check(rc)
    return call.out(o)


__all__ = [
    "DEFAULT_CHUNK",
    "KernelError",
    "LinearAttnConfig",
    "_DeltaResidual",
    "chunked_delta_rule",
    "chunked_delta_rule_fwd",
    "chunked_delta_rule_bwd",
    "chunked_delta_rule_varlen",
    "check_varlen",
    "chunked_kda_rule",
    "chunked_kda_rule_fwd",
    "chunked_kda_rule_bwd",
    "kda_delta_rule_step",
    "delta_rule_step",
    "chunked_gated_delta_rule",
    "chunked_gated_delta_rule_fwd",
    "chunked_gated_delta_rule_bwd",
    "gated_delta_rule_step",
]
