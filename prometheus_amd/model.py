"""The model-side caller of the delta rule on MI355X — the reference's
``model.linear_attention`` and ``model._linear_attn`` call surface.

``linear_attention(q, k, v, state=None)`` (``model/__init__.py:393-432``):
the Gated DeltaNet / KDA-family recurrence with beta = 1 on L2-normalised
q and k (``x / max(||x||, 1e-6)``, ``:203-205``). q, k, v are (batch, seq,
heads, dim) or (batch, seq, dim) (a single head, squeezed again on output);
state is (batch, heads, dim, dim) or (batch, dim, dim), zeros when None.
Returns ``(output, next_state)``, fp32. The normalisation and the unit gate
run inside the HIP kernel as it loads q and k (``pm_linear_attention``); no
normalised copies are written.

``_linear_attn(x, layer, state)`` (``:726-734``): the head projections
``W_q, W_k, W_v`` (d_model, heads, d_head) and ``W_o`` (heads, d_head,
d_model) around it, as fp32 GEMMs on the GPU (torch / hipBLASLt).

Inputs may be NumPy arrays (results come back as NumPy, the reference's
host path) or torch tensors (GPU tensors are used in place). bf16 tensors
are read as bf16 by the kernel, which equals the reference's cast to fp32.
There is no CPU fallback.
"""

from __future__ import annotations

import numpy as np
import torch

from prometheus_amd import _native
from prometheus_amd.kernels import _Call, _code, _DeltaResidual, _ptr, _stream, chunked_delta_rule_bwd

__all__ = ["linear_attention", "_linear_attn"]


def _shape(x) -> tuple:
    return tuple(x.shape)


def _heads(x) -> tuple[tuple, bool]:
    """Shape with a heads axis, and whether one was added (``model/__init__.py:383-390``)."""
    s = _shape(x)
    if len(s) == 3:
        return (s[0], s[1], 1, s[2]), True
    if len(s) == 4:
        return s, False
    raise ValueError(f"expected 3-D or 4-D tensor, got shape {s}")


def _dtype(q, k, v) -> torch.dtype:
    if all(isinstance(x, torch.Tensor) and x.dtype == torch.bfloat16 for x in (q, k, v)):
        return torch.bfloat16
    return torch.float32


def _l2n(x):
    """``x / max(||x||, 1e-6)`` over the last axis (model/__init__.py:203-205)."""
    return x / torch.clamp_min(torch.linalg.vector_norm(x, dim=-1, keepdim=True), 1e-6)


def _run_linear_attention(qd, kd, vd, sd, cdt, device):
    batch, seq, heads, dim = qd.shape
    o = torch.empty(qd.shape, dtype=torch.float32, device=device)
    s_out = torch.empty((batch, heads, dim, dim), dtype=torch.float32, device=device)
    lib = _native.lib()
    nbytes = lib.pm_linear_attention_workspace_bytes(batch, seq, heads, dim, _code(cdt))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device) if nbytes else None
    rc = lib.pm_linear_attention_ws(
        _ptr(qd), _ptr(kd), _ptr(vd), _ptr(sd), _ptr(o), _ptr(s_out),
        batch, seq, heads, dim, _code(cdt), _native.DTYPE_F32, _ptr(ws), nbytes, _stream(device),
    )
    _native.check(rc)
    return o, s_out


class _LinearAttention(torch.autograd.Function):
    """The fused kernel forward; the backward runs ``chunked_delta_rule_bwd`` (the
    reverse kernels) on the normalised rows with beta = 1, then differentiates the
    normalisation ``x / max(||x||, 1e-6)`` with torch.  bf16 q/k run the chunked
    bf16 backward on bf16-rounded normalised rows; fp32 q/k the fp32 backward."""

    @staticmethod
    def forward(ctx, qd, kd, vd, sd, cdt):
        o, s_out = _run_linear_attention(qd, kd, vd, sd, cdt, qd.device)
        ctx.save_for_backward(qd, kd, vd, sd)
        ctx.cdt = cdt
        # the library's kernel knobs are per thread and autograd may run the backward on
        # another thread: the backward runs under the forward caller's selection
        ctx.knobs = _native.knobs()
        return o, s_out

    @staticmethod
    def backward(ctx, go, gs):
        qd, kd, vd, sd = ctx.saved_tensors
        with torch.enable_grad():
            qf = qd.detach().float().requires_grad_(True)
            kf = kd.detach().float().requires_grad_(True)
            qn, kn = _l2n(qf), _l2n(kf)
        ones = torch.ones(qd.shape[:3], dtype=torch.float32, device=qd.device)
        s0 = sd if sd is not None else torch.zeros(
            (qd.shape[0], qd.shape[2], qd.shape[3], qd.shape[3]), dtype=torch.float32, device=qd.device)
        res = _DeltaResidual(q=qn.detach().to(ctx.cdt), k=kn.detach().to(ctx.cdt), v=vd, beta=ones,
                             state0=s0, chunk=64)
        with _native.use_knobs(*ctx.knobs):
            gqn, gkn, gv, _, gs0 = chunked_delta_rule_bwd(res, (go, gs))
        gq, gk = torch.autograd.grad((qn, kn), (qf, kf), (gqn, gkn))
        need = ctx.needs_input_grad
        return (gq.to(qd.dtype) if need[0] else None, gk.to(kd.dtype) if need[1] else None,
                gv.to(vd.dtype) if need[2] else None, gs0 if (sd is not None and need[3]) else None, None)


def linear_attention(q, k, v, state=None):
    """Causal delta rule with beta = 1 on L2-normalised q, k; returns (output, next_state).

    Differentiable when autograd records and a torch input requires grad (the
    reference differentiates it with JAX autodiff through its scan).
    """
    qs, squeeze = _heads(q)
    ks, _ = _heads(k)
    vs, _ = _heads(v)
    if qs != ks or qs[:3] != vs[:3] or qs[-1] != vs[-1]:
        raise ValueError("q, k, v must share batch/seq/heads and key/value dim")
    batch, seq, heads, dim = qs
    if state is not None:
        ss = _shape(state)
        if len(ss) == 3:
            ss = (ss[0], 1, ss[1], ss[2])
        if ss != (batch, heads, dim, dim):
            raise ValueError(f"state shape {ss} != {(batch, heads, dim, dim)}")
    if dim < 1 or dim > 256:
        raise ValueError(f"head dimension {dim} not in [1, 256]")
    call = _Call(q, k, v, state)
    cdt = _dtype(q, k, v)
    grad = torch.is_grad_enabled() and any(isinstance(x, torch.Tensor) and x.requires_grad
                                           for x in (q, k, v, state))
    with torch.cuda.device(call.device):
        qd, kd, vd = (call.dev(x, cdt).reshape(qs) for x in (q, k, v))
        sd = None if state is None else call.dev(state, torch.float32).reshape(batch, heads, dim, dim)
        if grad:
            o, s_out = _LinearAttention.apply(qd, kd, vd, sd, cdt)
        else:
            o, s_out = _run_linear_attention(qd, kd, vd, sd, cdt, call.device)
    if squeeze:
        o, s_out = o[:, :, 0, :], s_out[:, 0]
    return call.out(o), call.out(s_out)


def _linear_attn(x, layer, state=None):
    """Linear-attention layer: x (batch, seq, d_model) -> (y, next_state)."""
    xs = _shape(x)
    if len(xs) != 3:
        raise ValueError(f"x must be (batch, seq, d_model), got {xs}")
    b, s, d = xs
    w_shapes = {n: _shape(layer[n]) for n in ("W_q", "W_k", "W_v", "W_o")}
    dq = w_shapes["W_q"]
    if len(dq) != 3 or dq[0] != d or w_shapes["W_k"] != dq or w_shapes["W_v"] != dq:
        raise ValueError(f"W_q, W_k, W_v must be (d_model, heads, d_head) with d_model {d}")
    h, e = dq[1], dq[2]
    if w_shapes["W_o"] != (h, e, d):
        raise ValueError(f"W_o shape {w_shapes['W_o']} != {(h, e, d)}")
    call = _Call(x, layer["W_q"], layer["W_k"], layer["W_v"], layer["W_o"], state)
    f32 = torch.float32
    with torch.cuda.device(call.device):
        xd = call.dev(x, f32).reshape(b * s, d)
        # einsum("bsd,dhe->bshe") as one (b*s, d) x (d, h*e) GEMM per projection
        q, k, v = (torch.matmul(xd, call.dev(layer[n], f32).reshape(d, h * e)).reshape(b, s, h, e)
                   for n in ("W_q", "W_k", "W_v"))
        sd = None if state is None else call.dev(state, f32)
        y, s_out = linear_attention(q, k, v, sd)
        # einsum("bshe,hed->bsd")
        out = torch.matmul(y.reshape(b * s, h * e), call.dev(layer["W_o"], f32).reshape(h * e, d))
        out = out.reshape(b, s, d)
    return call.out(out), call.out(s_out)
