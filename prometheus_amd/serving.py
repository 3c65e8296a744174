"""Serving-side state cache of the linear-attention layers on MI355X.

The reference's serving spec (``spec/13-serving.md`` item 4) and its SGLang
fork (``sglang-fork/sglang_fork/model_def.py``, layer kinds only) describe
the consumer of the decode step: every linear-attention layer keeps one
fixed-size state per request (``(H, D, D)`` fp32, as ``kernels/__init__.py``
carries it), so a serving engine holds those states in a pool and decodes a
batch of requests through a slot table, and parks idle sessions' states in
host memory. ``LinearStateCache`` is that pool on one GPU:

* ``pool``: ``(n_layers, n_slots, H, D, D)`` fp32 in HBM (64 KiB per slot and
  layer at H = 1, D = 128);
* ``alloc`` / ``free`` / ``reset``: slot bookkeeping on the host;
* ``prefill``: runs a prompt through the forward (the chunked MFMA kernel for
  bf16 with D in {64, 128}), starting from and ending in the requests' slots;
  with the slots and ``cu_seqlens`` as GPU tensors it never synchronises with
  the host, so it can be captured in a HIP graph (an out-of-range device slot
  computes from a zero state into a spare slot past the pool's end, leaves the
  pool untouched, and is reported by ``check_slots``);
* ``decode``: one token per request, in place, through ``pm_delta_step_slots``
  (allocation-free with ``out=``, no host synchronisation, so it can be
  captured in a HIP graph with a fixed slot tensor whose contents change
  between replays; slots outside ``[0, n_slots)`` are padding);
* ``swap_out`` / ``swap_in``: park states in pinned host memory and restore
  them (the spec's tier-2 parking of long sessions).
"""

from __future__ import annotations

import heapq

import torch

from prometheus_amd import _native, kernels

__all__ = ["LinearStateCache"]


class LinearStateCache:
    """Per-request recurrent states of ``n_layers`` linear-attention layers."""

    def __init__(self, n_layers: int, n_slots: int, heads: int, dim: int, device=None):
        if n_layers < 1 or n_slots < 1 or heads < 1 or dim < 1:
            raise ValueError("n_layers, n_slots, heads and dim must be >= 1")
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.n_layers, self.n_slots, self.heads, self.dim = n_layers, n_slots, heads, dim
        # one spare slot past the end: out-of-range device slot indices land there
        self._pool = torch.zeros((n_layers, n_slots + 1, heads, dim, dim), dtype=torch.float32,
                                 device=device)
        self.pool = self._pool[:, :n_slots]
        self._bad_slot = torch.zeros(1, dtype=torch.int32, device=device)
        # a min-heap: alloc hands out the lowest free slots, so that a batch admitted in
        # order decodes through an increasing slot table, which walks the pool in address
        # order (at cfg4, 0.71 of HBM against 0.69 for a random table)
        self._free = list(range(n_slots))
        self._used: set[int] = set()

    # ---- bookkeeping ----
    @property
    def n_free(self) -> int:
        return len(self._free)

    def alloc(self, n: int = 1) -> list[int]:
        """Take ``n`` free slots; their states are zero (a fresh request)."""
        if n < 0 or n > len(self._free):
            raise RuntimeError(f"cannot allocate {n} slots ({len(self._free)} free)")
        got = [heapq.heappop(self._free) for _ in range(n)]
        self._used.update(got)
        if got:
            self.reset(got)
        return got

    def free(self, slots) -> None:
        for s in self._ids(slots):
            if s not in self._used:
                raise ValueError(f"slot {s} is not allocated")
            self._used.remove(s)
            heapq.heappush(self._free, s)

    def reset(self, slots) -> None:
        idx = self._index(slots)
        self._pool[:, idx] = 0.0

    # ---- compute ----
    def prefill(self, layer: int, slots, q, k, v, beta, cu_seqlens=None, config=None):
        """Run prompts through the forward from the slots' states into them.

        Fixed length: q, k, v ``(n, T, H, D)``, beta ``(n, T, H)``, one request per
        row. Packed: q, k, v ``(1, N, H, D)`` with ``cu_seqlens`` ``(n + 1,)``.
        Returns the output ``(.., H, D)`` fp32. ``slots`` may be a list of ints or a
        GPU int tensor; with GPU ``slots`` and ``cu_seqlens`` nothing here waits for
        the device (see ``check_slots`` and ``kernels.check_varlen``).
        """
        self._check_layer(layer)
        idx = self._index(slots)
        self._check_cuda(q, k, v, beta)
        self._pool[layer, self.n_slots].zero_()  # the spare slot: a fresh state
        s0 = self._pool[layer, idx]  # gathered copy (n, H, D, D)
        if cu_seqlens is None:
            o, s = kernels.chunked_delta_rule(q, k, v, beta, s0, config)
        else:
            o, s = kernels.chunked_delta_rule_varlen(q, k, v, beta, cu_seqlens, s0, config)
        self._pool[layer, idx] = s
        return o

    def check_slots(self) -> None:
        """Raise ``ValueError`` if a GPU slot tensor given to ``prefill`` or ``reset`` since
        the last check held an index outside ``[0, n_slots)`` (synchronises; clears)."""
        if int(self._bad_slot.item()):
            self._bad_slot.zero_()
            raise ValueError(f"a device slot index was outside [0, {self.n_slots})")

    def decode(self, layer: int, slots: torch.Tensor, q, k, v, beta, out=None):
        """One token per request: q, k, v ``(B, H, D)``, beta ``(B, H)``, ``slots``
        an int32 GPU tensor ``(B,)``. Updates the states in place and returns
        ``out`` ``(B, H, D)`` fp32 (allocated when None)."""
        self._check_layer(layer)
        self._check_cuda(q, k, v, beta, slots)
        b = slots.shape[0] if slots.dim() == 1 else -1
        if b < 0 or slots.dtype != torch.int32 or not slots.is_contiguous():
            raise ValueError("slots must be a contiguous int32 tensor of shape (B,)")
        want = (b, self.heads, self.dim)
        for name, x in (("q", q), ("k", k), ("v", v)):
            if tuple(x.shape) != want or not x.is_contiguous():
                raise ValueError(f"{name} must be contiguous {want}, got {tuple(x.shape)}")
        if q.dtype != k.dtype or q.dtype != v.dtype or q.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("q, k, v must share one dtype, fp32 or bf16")
        if tuple(beta.shape) != (b, self.heads) or beta.dtype != torch.float32 or not beta.is_contiguous():
            raise ValueError(f"beta must be contiguous fp32 {(b, self.heads)}")
        if out is None:
            out = torch.empty(want, dtype=torch.float32, device=q.device)
        elif tuple(out.shape) != want or out.dtype != torch.float32 or not out.is_contiguous():
            raise ValueError(f"out must be contiguous fp32 {want}")
        rc = _native.lib().pm_delta_step_slots(
            self.pool[layer].data_ptr(), slots.data_ptr(), self.n_slots, q.data_ptr(), k.data_ptr(),
            v.data_ptr(), beta.data_ptr(), out.data_ptr(), b, self.heads, self.dim,
            _native.DTYPE_BF16 if q.dtype == torch.bfloat16 else _native.DTYPE_F32,
            torch.cuda.current_stream(q.device).cuda_stream,
        )
        _native.check(rc)
        return out

    # ---- tiering ----
    def swap_out(self, slots) -> torch.Tensor:
        """The slots' states of every layer, copied to pinned host memory:
        ``(n_layers, n, H, D, D)``. The slots stay allocated."""
        idx = self._index(slots)
        host = torch.empty((self.n_layers, len(idx), self.heads, self.dim, self.dim),
                           dtype=torch.float32, pin_memory=True)
        host.copy_(self._pool[:, idx])
        return host

    def swap_in(self, slots, saved: torch.Tensor) -> None:
        idx = self._index(slots)
        want = (self.n_layers, len(idx), self.heads, self.dim, self.dim)
        if tuple(saved.shape) != want:
            raise ValueError(f"saved states {tuple(saved.shape)} != {want}")
        self._pool[:, idx] = saved.to(self._pool.device, dtype=torch.float32)

    # ---- helpers ----
    def _ids(self, slots) -> list[int]:
        ids = [int(s) for s in (slots.tolist() if isinstance(slots, torch.Tensor) else slots)]
        for s in ids:
            if not 0 <= s < self.n_slots:
                raise ValueError(f"slot {s} outside [0, {self.n_slots})")
        return ids

    def _index(self, slots) -> torch.Tensor:
        if isinstance(slots, torch.Tensor) and slots.device.type == "cuda":
            # checked on the device: an index outside [0, n_slots) becomes the spare slot
            if slots.dim() != 1 or slots.dtype not in (torch.int32, torch.int64):
                raise ValueError("a GPU slot tensor must be 1-D int32 or int64")
            if slots.device != self._pool.device:
                raise ValueError("slots must be on the pool's device")
            idx = slots.long()
            bad = (idx < 0) | (idx >= self.n_slots)
            self._bad_slot.bitwise_or_(bad.any().to(torch.int32))
            return torch.where(bad, torch.full_like(idx, self.n_slots), idx)
        return torch.tensor(self._ids(slots), dtype=torch.long, device=self._pool.device)

    def _check_layer(self, layer: int) -> None:
        if not 0 <= layer < self.n_layers:
            raise ValueError(f"layer {layer} outside [0, {self.n_layers})")

    def _check_cuda(self, *xs) -> None:
        if self.pool.device.type != "cuda":
            raise RuntimeError("the state cache computes on a HIP GPU; this pool is on the host")
        for x in xs:
            if not (isinstance(x, torch.Tensor) and x.device == self.pool.device):
                raise ValueError("inputs must be tensors on the pool's device")
