"""Benchmark: delta-rule forward on one MI355X (BASELINE cfg1), plus the decode step.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A "step" is one call of the forward (``pm_delta_fwd``, the C ABI behind
``prometheus_amd.kernels.chunked_delta_rule``) over the cfg1 batch:
B=4 H=16 T=4096 d_k=d_v=128, bf16 q/k/v (q, k L2-normalised), fp32 beta,
zero initial state, fp32 O and final S, chunk 64. Inputs are resident in
HBM before timing starts; two input sets alternate so that consecutive
steps never find their 201 MB of inputs in the 256 MB Infinity Cache.
The shader clock ramps up over the first ~150 calls after the GPU idles, so
the default warm-up (200 steps) and each later leg's own warm-up run past
it, and the CPU work (the baseline and the parity replays) runs after every
GPU leg, from host copies of the outputs it checks.

Prints ONE JSON line (the driver's contract) with ``roofline`` for the
forward kernel (HBM-bound at this shape: 340.8 MB vs 47.6 GFLOP) and
``cpu_baseline`` (the C restatement of the reference's per-token CPU
algorithm, OpenMP over the 64 (b, h) sequences, on this host). The decode
step (cfg4: B=256 H=32 D=128, fp32 state updated in place) is measured in
the same run and reported under ``decode`` (with the same batch through a
serving state cache under ``decode.state_cache``), the backward at cfg1
under ``backward``, the model's linear attention at the cfg1 shape
under ``model_linear_attention``, the cfg1 forward with fp32 q/k/v (the
fp32 chunked forward, and the per-token kernel beside it) under ``fp32_forward``, the gated variant at cfg1
under ``gated``, and KDA (a log-gate per key channel: the chunked form, and the per-token
kernel beside it) at cfg1 under ``kda``.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, vendor figure
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, vendor figure
FP32_VALU_PEAK_TFLOPS = 157.3  # MI355X fp32 vector, vendor figure (packed FMA; half without)
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 MFMA, vendor figure
CHUNK = 64
WARM_CALLS = 5  # untimed calls before each later leg's timed ones (fresh output buffers)
CALIB_COPY_BYTES = 1 << 30  # bytes read (and written) by one calibration copy launch
CPU_SAMPLE_S = 10.0  # seconds of CPU work timed for cpu_baseline (whole cfg1 batches)


def fwd_flops(B, T, H, D, chunk=CHUNK) -> float:
    """Algorithmic flops of the chunked form: 10 c^2 D + 6 c D^2 + c^3/3 per (b, h) chunk."""
    n_full, rem = divmod(T, chunk)
    per = lambda c: 10 * c * c * D + 6 * c * D * D + c ** 3 / 3.0  # noqa: E731
    return B * H * (n_full * per(chunk) + (per(rem) if rem else 0.0))


def bwd32_flops(B, T, H, D, chunk=16) -> float:
    """Algorithmic flops of the fp32 chunked backward in 16-token chunks: per (b, h) chunk
    8 products of D x D size (the forward state K S and K^T U; the gradient sweep K G,
    Q^T dO and K^T diag(beta) W; dO S^T, U G^T and diag(beta) W S^T over d_v), 2 c D^2 each,
    and 11 of chunk size (K K^T, T'' X, Q K^T, P^T dO, T^T dU, dO U^T, W U^T, dP K, dP^T Q,
    dA K, dA^T K), 2 c^2 D each: 16 c D^2 + 22 c^2 D.  What the kernels recompute (the
    span's forward, S rebuilt backwards, the G recurrence inside each span) is not counted."""
    n_full, rem = divmod(T, chunk)
    per = lambda c: 16 * c * D * D + 22 * c * c * D  # noqa: E731
    return B * H * (n_full * per(chunk) + (per(rem) if rem else 0.0))


def fwd_bytes(B, T, H, D, s_in=2, s_out=4, s0=False) -> float:
    """Algorithmic HBM bytes: q, k, v in + beta + O out + S out (+ S0 in)."""
    E = B * T * H * D
    S = 4 * B * H * D * D
    return 3 * E * s_in + 4 * B * T * H + E * s_out + S + (S if s0 else 0)


def bwd_bytes(B, T, H, D, s_in=2) -> float:
    """Backward: q, k, v, beta, S0, go, gS in; gq, gk, gv, gbeta, gS0 out (fp32 grads)."""
    E = B * T * H * D
    S = 4 * B * H * D * D
    return 3 * E * s_in + 4 * E + 3 * 4 * E + 2 * 4 * B * T * H + 3 * S


def step_bytes(B, H, D, s_in=2) -> float:
    """Decode step: S read + written, q, k, v in, beta in, o out."""
    S = 4 * B * H * D * D
    return 2 * S + 3 * B * H * D * s_in + 4 * B * H + 4 * B * H * D


def make_inputs(torch, B, T, H, D, seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(seed)

    def unit(shape):
        x = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
        x = x / torch.clamp(torch.linalg.vector_norm(x, dim=-1, keepdim=True), min=1e-6)
        return x.to(torch.bfloat16).contiguous()

    q = unit((B, T, H, D))
    k = unit((B, T, H, D))
    v = torch.randn((B, T, H, D), generator=g, device=device).to(torch.bfloat16).contiguous()
    beta = torch.sigmoid(torch.randn((B, T, H), generator=g, device=device)).contiguous()
    return q, k, v, beta


def bits(t) -> np.ndarray:
    return t.detach().cpu().contiguous().view(dtype=__import__("torch").int16).numpy().view(np.uint16)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_threads() -> int:
    """Threads for the CPU baseline: OMP_NUM_THREADS when the environment sets it (the
    GPU box sets it to its CPU share), else every CPU this process may run on."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    return max(1, len(os.sched_getaffinity(0)))


def time_launches(stream, fn, n):
    """Mean ms per call of fn(0..n-1), launched back to back on `stream` between one
    pair of events (no event between the launches)."""
    import torch

    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(n):
        fn(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n


def _time_calls(torch, stream, f, calls):
    """Mean ms per call over `calls` back-to-back calls (one event pair), after 2 untimed."""
    for i in range(2):
        f(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(calls):
        f(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / calls


def _time_rounds(torch, stream, fns, calls, rounds=3):
    """Median ms per call of each of `fns`, timed in `rounds` interleaved rounds (each fn
    `calls` back-to-back calls per round, after 2 untimed), so that clock and cache
    warm-up fall on every candidate alike."""
    res = [[] for _ in fns]
    for _ in range(rounds):
        for j, f in enumerate(fns):
            res[j].append(_time_calls(torch, stream, f, calls))
    return [sorted(r)[len(r) // 2] for r in res]


SPLIT_SWEEP_SHAPES = [(4, 4096, 16, 128), (2, 4096, 16, 128), (1, 4096, 16, 128), (1, 32768, 32, 128),
                      (2, 8192, 8, 128), (1, 1024, 4, 128), (4, 4096, 16, 64), (1, 8192, 16, 64),
                      (8, 2048, 16, 128), (16, 512, 16, 128)]


def split_sweep(torch, lib, _native, dev, stream, calls=10):
    """The forward's two chunked forms (single-stage: pm_delta_set_path 2; split: 3) at the
    shapes of SPLIT_SWEEP_SHAPES, bf16 q/k/v, fp32 O, in interleaved rounds; and which form
    path 0 takes there (it takes the split form exactly when it asks for a workspace).
    One JSON line per shape."""
    for (B, T, H, D) in SPLIT_SWEEP_SHAPES:
        sets = [make_inputs(torch, B, T, H, D, seed, dev) for seed in (1, 2)]
        o = torch.empty((B, T, H, D), dtype=torch.float32, device=dev)
        s = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
        auto_ws = lib.pm_delta_workspace_bytes(B, T, H, D, _native.DTYPE_BF16)
        old = _native.set_path(3)
        nws = lib.pm_delta_workspace_bytes(B, T, H, D, _native.DTYPE_BF16)
        _native.set_path(old)
        ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev)

        def run(path):
            def f(i):
                q, k, v, beta = sets[i % 2]
                old = _native.set_path(path)
                try:
                    _native.check(lib.pm_delta_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), None,
                                                   o.data_ptr(), s.data_ptr(), B, T, H, D, _native.DTYPE_BF16,
                                                   _native.DTYPE_F32, CHUNK, ws.data_ptr(), nws, stream.cuda_stream))
                finally:
                    _native.set_path(old)
            return f

        single, split = _time_rounds(torch, stream, [run(2), run(3)], calls)
        tile = 16 if B * H * (D // 32) < 256 else 32
        print(json.dumps({"shape": {"B": B, "T": T, "H": H, "D": D}, "d_v_tile": tile,
                          "single_stage_us": single * 1e3, "split_us": split * 1e3, "split_over_single": split / single,
                          "path0_takes": "split" if auto_ws else "single-stage"}), flush=True)
        del sets, o, s, ws


def _roofline(nbytes, ms):
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS}


def time_cfg3(torch, lib, _native, dev, stream, calls=4):
    """cfg3, the long-context single-GPU share: B1 H32 T32768 D128 bf16 with S0 ~ N(0, 0.02).
    The default path (with the workspace the Python layer passes) and the single-stage
    kernel forced (path 2), in interleaved rounds; two input sets alternate."""
    B, T, H, D = 1, 32768, 32, 128
    print(f"[bench] cfg3 B{B} T{T} H{H} D{D}", file=sys.stderr, flush=True)
    sets = [make_inputs(torch, B, T, H, D, seed, dev) for seed in (31, 32)]
    g = torch.Generator(device=dev)
    g.manual_seed(33)
    s0 = (torch.randn((B, H, D, D), generator=g, device=dev) * 0.02).contiguous()
    o = torch.empty((B, T, H, D), dtype=torch.float32, device=dev)
    s = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
    nws = lib.pm_delta_workspace_bytes(B, T, H, D, _native.DTYPE_BF16)
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev)

    def f(i, use_ws=True):
        q, k, v, beta = sets[i % 2]
        rc = lib.pm_delta_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), s0.data_ptr(),
                              o.data_ptr(), s.data_ptr(), B, T, H, D, _native.DTYPE_BF16, _native.DTYPE_F32,
                              CHUNK, ws.data_ptr() if use_ws and nws else None, nws if use_ws else 0,
                              stream.cuda_stream)
        _native.check(rc)

    def single(i):
        old = _native.set_path(2)
        try:
            f(i, False)
        finally:
            _native.set_path(old)

    ms_default, ms_single = _time_rounds(torch, stream, [f, single], calls)
    nb = fwd_bytes(B, T, H, D, s0=True)
    tile = 16 if B * H * (D // 32) < 256 else 32  # the chunked kernel's d_v tile rule
    return {
        "workload": "cfg3 forward: B1 H32 T32768 D128 bf16, S0 ~ N(0, 0.02), fp32 O and S",
        "calls": calls,
        "kernel_us": ms_default * 1e3,
        "path": "split form (T by a parallel pass into the workspace, then the recurrence)" if nws
                else "single-stage chunked kernel",
        "d_v_tile": tile,
        "tokens_per_s": B * T / (ms_default * 1e-3),
        "algorithmic_bytes": nb,
        "roofline": _roofline(nb, ms_default),
        "single_stage": {"kernel_us": ms_single * 1e3, "roofline": _roofline(nb, ms_single)},
    }


def time_cfg2(torch, lib, _native, synth, dev, stream, calls=10):
    """cfg2, the packed variable-length batch: 16384 tokens, H16 D128 bf16, lengths drawn
    from U[64, 4096] (seed 2) and concatenated through cu_seqlens (on the device)."""
    c = synth.CONFIGS[2]
    N, H, D = c["total"], c["H"], c["D"]
    lens = synth.varlen_lengths(N, c["lo"], c["hi"], seed=2)
    cu = torch.from_numpy(synth.cu_seqlens(lens)).to(dev)
    n_seqs = len(lens)
    print(f"[bench] cfg2 varlen N{N} H{H} D{D}, {n_seqs} sequences", file=sys.stderr, flush=True)
    sets = [make_inputs(torch, 1, N, H, D, seed, dev) for seed in (21, 22)]
    o = torch.empty((1, N, H, D), dtype=torch.float32, device=dev)
    s = torch.empty((n_seqs, H, D, D), dtype=torch.float32, device=dev)
    nws = lib.pm_delta_varlen_workspace_bytes(n_seqs, N, H, D, _native.DTYPE_BF16)
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev)

    def call(i, use_ws):
        q, k, v, beta = sets[i % 2]
        w = use_ws and nws > 0
        rc = lib.pm_delta_fwd_varlen(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), cu.data_ptr(),
                                     n_seqs, N, None, o.data_ptr(), s.data_ptr(), H, D, _native.DTYPE_BF16,
                                     _native.DTYPE_F32, CHUNK, ws.data_ptr() if w else None, nws if w else 0,
                                     stream.cuda_stream)
        _native.check(rc)

    # the default call (with the workspace pm_delta_varlen_workspace_bytes asks for, none
    # at cfg2), medians of three rounds
    ms = statistics.median(_time_calls(torch, stream, lambda i: call(i, True), calls) for _ in range(3))
    # the schedule: one batch of 60 x 192 tokens and one 4096-token sequence, packed with the
    # long sequence first and with it last; the forward takes sequences longest first, so
    # the two orders should time the same (in cu_seqlens order the late long sequence
    # starts only when the short ones have freed CUs)
    sched = {}
    for name, sl in (("long_first", [4096] + [192] * 60), ("long_last", [192] * 60 + [4096])):
        cu2 = torch.from_numpy(synth.cu_seqlens(np.array(sl))).to(dev)
        n2, N2 = len(sl), sum(sl)
        assert N2 <= N
        q2, k2, v2, b2 = (x[:, :N2].contiguous() for x in sets[0])
        o2 = torch.empty((1, N2, H, D), dtype=torch.float32, device=dev)
        s2 = torch.empty((n2, H, D, D), dtype=torch.float32, device=dev)

        def call2(i):
            rc = lib.pm_delta_fwd_varlen(q2.data_ptr(), k2.data_ptr(), v2.data_ptr(), b2.data_ptr(), cu2.data_ptr(),
                                         n2, N2, None, o2.data_ptr(), s2.data_ptr(), H, D, _native.DTYPE_BF16,
                                         _native.DTYPE_F32, CHUNK, None, 0, stream.cuda_stream)
            _native.check(rc)

        sched[name + "_us"] = statistics.median(_time_calls(torch, stream, call2, calls) for _ in range(3)) * 1e3
    E = N * H * D
    nb = 3 * E * 2 + 4 * N * H + 4 * E + 4 * n_seqs * H * D * D + 4 * (n_seqs + 1)
    return {
        "workload": f"cfg2 varlen forward: {N} packed tokens, H16 D128 bf16, {n_seqs} sequences "
                    f"(lengths U[64, 4096], seed 2), cu_seqlens int32 on the device",
        "calls": calls,
        "kernel_us": ms * 1e3,
        "path": ("split form" if nws > 4 * n_seqs else
                 "single-stage chunked kernel, sequences longest first"
                 + (" (order from the rank kernel)" if nws else " (ranked in the kernel)")),
        "lengths": [int(x) for x in lens],
        "longest": int(max(lens)),
        "tokens_per_s": N / (ms * 1e-3),
        "algorithmic_bytes": nb,
        "roofline": _roofline(nb, ms),
        "rounds": 3,
        "schedule": {"batch": "60 x 192 tokens and one of 4096, H16 D128 bf16, packed with the long "
                              "sequence first or last", **sched},
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # the shader clock ramps up over the first ~150 calls after idle (measured: rounds of 10
    # calls at 128-137 us, settling at 109-110 us), so the default warm-up covers the ramp
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--decode-steps", type=int, default=64)
    ap.add_argument("--gated-calls", type=int, default=10,
                    help="timed pm_gated_delta_fwd and pm_kda_delta_fwd calls at cfg1 (0 skips)")
    ap.add_argument("--model-calls", type=int, default=2,
                    help="timed pm_linear_attention calls at the cfg1 shape (0 skips)")
    ap.add_argument("--bwd-steps", type=int, default=10,
                    help="timed calls of the backward at cfg1 (0 skips it)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-long-configs", dest="long_configs", action="store_false",
                    help="skip the cfg3 (B1 H32 T32768, S0) and cfg2 (varlen) forward legs")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "traffic_cfg1.json"),
                    help="JSON with measured HBM bytes per launch (from rocprofv3 --pmc)")
    ap.add_argument("--mfma-counters", default=os.path.join(ROOT, "profiles", "mfma_cfg1.json"),
                    help="JSON with rocprofv3 MfmaUtil / MfmaFlopsBF16 for the forward kernel")
    ap.add_argument("--decode-traffic", default=os.path.join(ROOT, "profiles", "traffic_cfg4_decode.json"),
                    help="JSON with measured HBM bytes per decode-step launch (rocprofv3 --pmc)")
    ap.add_argument("--tile", type=int, default=0, help="d_v tile of the chunked kernel (0 auto)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run 3 launches of a plain 1 GiB fp32 elementwise copy (torch.neg, "
                         "4 GiB read+written in all) so that rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE "
                         "runs can be scaled to bytes")
    ap.add_argument("--split-sweep", action="store_true",
                    help="only time the forward's single-stage and split forms at a list of shapes "
                         "(one JSON line per shape) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for "
              f"--gpus {args.gpus}); the forward shards over (b, h) with no exchange", file=sys.stderr)
        sys.exit(2)

    import torch

    from prometheus_amd import _native, synth

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    lib = _native.lib()
    if args.tile:
        _native.set_tile(args.tile)
    if args.split_sweep:
        split_sweep(torch, lib, _native, dev, torch.cuda.current_stream(dev))
        return

    B, T, H, D = 4, 4096, 16, 128
    print(f"[bench] cfg1 inputs B{B} T{T} H{H} D{D}", file=sys.stderr, flush=True)
    sets = [make_inputs(torch, B, T, H, D, seed, dev) for seed in (1, 2)]
    o = torch.empty((B, T, H, D), dtype=torch.float32, device=dev)
    s = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)

    def launch(i):
        q, k, v, beta = sets[i % 2]
        rc = lib.pm_delta_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), None,
                              o.data_ptr(), s.data_ptr(), B, T, H, D, _native.DTYPE_BF16,
                              _native.DTYPE_F32, CHUNK, None, 0, stream.cuda_stream)
        _native.check(rc)

    for i in range(args.warmup):
        launch(i)
    torch.cuda.synchronize()
    print(f"[bench] warmup {args.warmup} done; timing {args.steps} steps", file=sys.stderr,
          flush=True)
    # one event pair on the launch stream over the whole timed region: the launches run
    # back to back, and no event sits between them
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(args.steps):
        launch(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern_ms = ev0.elapsed_time(ev1) / args.steps
    ms_per_step = wall * 1e3 / args.steps
    last = (args.steps - 1) % 2

    def spin_up(ms=25.0):
        """Untimed forward calls for about `ms` of GPU time before a leg: the shader clock
        drops while the GPU waits on host work (copies, allocations) and ramps up again
        over ~150 calls."""
        w0, w1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        w0.record(stream)
        n = 0
        while True:
            for _ in range(10):
                launch(n)
                n += 1
            w1.record(stream)
            w1.synchronize()
            if w0.elapsed_time(w1) >= ms:
                return

    tokens = B * T
    flops = fwd_flops(B, T, H, D)
    nbytes = fwd_bytes(B, T, H, D)
    achieved_gbs = nbytes / (kern_ms * 1e-3) / 1e9
    tflops = flops / (kern_ms * 1e-3) / 1e12
    traffic = None
    if os.path.exists(args.traffic):
        with open(args.traffic) as f:
            traffic = json.load(f).get("bytes_per_launch")
    # MFMA counters of the same kernel and workload, from a rocprofv3 --pmc run (the file
    # records the command): busy fraction of the MFMA pipes and executed bf16 MFMA flops
    mfma_counters = None
    if os.path.exists(args.mfma_counters):
        with open(args.mfma_counters) as f:
            mc = json.load(f)
        mfma_counters = {"mfma_util_pct": mc.get("mfma_util_pct"),
                         "executed_bf16_mfma_flop": mc.get("executed_bf16_mfma_flop"),
                         "executed_over_algorithmic": mc.get("executed_over_algorithmic")}

    def time_fwd(out_code, out_t, calls=20, ws=None):
        n = [0]

        def f():  # the two input sets alternate, as in the headline loop
            q, k, v, beta = sets[n[0] % 2]
            n[0] += 1
            rc = lib.pm_delta_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), None,
                                  out_t.data_ptr(), s.data_ptr(), B, T, H, D, _native.DTYPE_BF16,
                                  out_code, CHUNK, None if ws is None else ws.data_ptr(),
                                  0 if ws is None else ws.numel(), stream.cuda_stream)
            _native.check(rc)

        for _ in range(3):  # first touches of a fresh output buffer are slower
            f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(calls):
            f()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / calls

    # the opt-in bf16 output (out_dtype=bf16): 273.7 MB instead of 340.8 MB per call. The
    # shader clock of these boxes depends on the power the work draws and drifts between
    # runs, so bf16 O is timed in rounds interleaved with fp32 O calls (medians over rounds)
    o16 = torch.empty((B, T, H, D), dtype=torch.bfloat16, device=dev)
    rounds_16, rounds_32 = [], []
    for _ in range(5):
        rounds_32.append(time_fwd(_native.DTYPE_F32, o, calls=10))
        rounds_16.append(time_fwd(_native.DTYPE_BF16, o16, calls=10))
    b16_ms = float(np.median(rounds_16))
    f32_ms_interleaved = float(np.median(rounds_32))
    b16_bytes = fwd_bytes(B, T, H, D, s_out=2)
    bf16_out = {
        "workload": "cfg1 forward, bf16 O (pm_delta_fwd out_dtype bf16)",
        "timing": "5 rounds of 10 calls, each round right after 10 fp32-O calls; medians",
        "kernel_us": b16_ms * 1e3,
        "fp32_out_kernel_us_same_rounds": f32_ms_interleaved * 1e3,
        "bf16_over_fp32": b16_ms / f32_ms_interleaved,
        "tokens_per_s": tokens / (b16_ms * 1e-3),
        "algorithmic_bytes": b16_bytes,
        "roofline": {"bound": "hbm", "achieved": b16_bytes / (b16_ms * 1e-3) / 1e9,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": b16_bytes / (b16_ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
        "mfma": {"achieved_tflops": flops / (b16_ms * 1e-3) / 1e12, "peak_tflops": BF16_PEAK_TFLOPS,
                 "frac": flops / (b16_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS},
    }
    del o16
    # the split form of the chunked kernel (T diag(beta) by a parallel pass into a workspace,
    # then the chunk recurrence), forced at cfg1 with pm_delta_set_path(3); by default it runs
    # only where the chunked kernel takes 16-column tiles, where it is the faster form
    old_path = _native.set_path(3)
    try:
        ws_split = torch.empty(lib.pm_delta_workspace_bytes(B, T, H, D, _native.DTYPE_BF16),
                               dtype=torch.uint8, device=dev)
        split_ms = time_fwd(_native.DTYPE_F32, o, ws=ws_split)
    finally:
        _native.set_path(old_path)
    del ws_split
    split_form = {"workload": "cfg1 forward, chunked kernel in split form (path 3, prep + recurrence)",
                  "kernel_us": split_ms * 1e3,
                  "roofline_frac": nbytes / (split_ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
    cfg3 = cfg2 = None
    if args.long_configs:
        cfg3 = time_cfg3(torch, lib, _native, dev, stream)
        cfg2 = time_cfg2(torch, lib, _native, synth, dev, stream)
    launch(last)  # the output the parity check reads
    torch.cuda.synchronize()
    # host copies for the CPU baseline and its parity check, which run after every GPU leg
    # (an idle GPU drops its clock, and the legs after a long CPU phase would time the ramp)
    host_o = host_s = None
    if not args.no_cpu_baseline:
        host_o, host_s = o.cpu().numpy(), s.cpu().numpy()
        host_in = tuple(bits(x) for x in sets[last][:3]) + (sets[last][3].cpu().numpy(),)

    # The gated and KDA forwards run next to the other bf16 forward legs: after the heavy
    # fp32 legs the same calls took 3-25% longer for a while (0.118-0.142 ms for a gated
    # call that takes 0.114-0.115 ms in a steady loop)
    g = torch.Generator(device=dev)
    # the gated delta rule at cfg1 (pm_gated_delta_fwd): cfg1's inputs plus log-gates
    # -0.1 |N(0, 1)| per token and head, on the chunked kernel
    gated = None
    if args.gated_calls > 0:
        spin_up()
        g.manual_seed(8)
        gates = -0.1 * torch.randn((B, T, H), generator=g, device=dev).abs()
        og = torch.empty((B, T, H, D), device=dev)
        sg = torch.empty((B, H, D, D), device=dev)

        def gfwd(i=0):  # the two input sets alternate, as in the headline loop
            q, k, v, beta = sets[i % 2]
            rc = lib.pm_gated_delta_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(),
                                        gates.data_ptr(), None, og.data_ptr(), sg.data_ptr(), B, T, H,
                                        D, _native.DTYPE_BF16, _native.DTYPE_F32, stream.cuda_stream)
            _native.check(rc)

        # after the heavy fp32 legs, 20 untimed calls, then the median of 5 rounds
        for i in range(20):
            gfwd(i)
        g_ms = float(np.median([time_launches(stream, gfwd, args.gated_calls) for _ in range(5)]))
        gb = fwd_bytes(B, T, H, D) + 4 * B * T * H
        gated = {
            "workload": "cfg1 gated delta rule (log-gates -0.1|N(0,1)|), bf16 q/k/v, chunked kernel",
            "calls": args.gated_calls,
            "timing": "median of 5 rounds of the calls, after 20 untimed",
            "ms_per_call": g_ms,
            "tokens_per_s": tokens / (g_ms * 1e-3),
            "roofline": {"bound": "hbm", "achieved": gb / (g_ms * 1e-3) / 1e9,
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gb / (g_ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
        }
        del og, sg, gates

    # KDA at cfg1 (pm_kda_delta_fwd): cfg1's inputs plus log-gates -0.1 |N(0, 1)| per token,
    # head and key channel; the chunked form (prepass + recurrence) and the per-token kernel
    kda = None
    if args.gated_calls > 0:
        spin_up()
        g.manual_seed(9)
        gates = -0.1 * torch.randn((B, T, H, D), generator=g, device=dev).abs()
        ok_ = torch.empty((B, T, H, D), device=dev)
        sk_ = torch.empty((B, H, D, D), device=dev)
        kws_bytes = lib.pm_kda_delta_workspace_bytes(B, T, H, D, _native.DTYPE_BF16)
        kws = torch.empty((kws_bytes,), dtype=torch.uint8, device=dev)

        def kfwd(i=0, ws=True):
            q, k, v, beta = sets[i % 2]
            rc = lib.pm_kda_delta_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(),
                                      gates.data_ptr(), None, ok_.data_ptr(), sk_.data_ptr(), B, T, H, D,
                                      _native.DTYPE_BF16, _native.DTYPE_F32, kws.data_ptr() if ws else None,
                                      kws_bytes if ws else 0, stream.cuda_stream)
            _native.check(rc)

        def time_kda(ws, calls):
            # as for the gated leg: untimed calls, then the median of rounds (one round for
            # the slow per-token kernel)
            for i in range(20 if ws else 1):
                kfwd(i, ws)
            return float(np.median([time_launches(stream, lambda i: kfwd(i, ws), calls)
                                    for _ in range(5 if ws else 1)]))

        k_ms = time_kda(True, args.gated_calls)
        o_chunk = ok_.clone()
        kp_ms = time_kda(False, max(1, args.gated_calls // 5))
        kfwd(args.gated_calls - 1, False)  # the per-token result on the chunked call's inputs
        torch.cuda.synchronize()
        rel = float(torch.linalg.vector_norm(o_chunk - ok_) / torch.linalg.vector_norm(ok_))
        kb_ = fwd_bytes(B, T, H, D) + 4 * B * T * H * D
        kda = {
            "workload": "cfg1 KDA (log-gates -0.1|N(0,1)| per key channel), bf16 q/k/v, fp32 O",
            "calls": args.gated_calls,
            "timing": "median of 5 rounds of the calls, after 20 untimed",
            "ms_per_call": k_ms,
            "tokens_per_s": tokens / (k_ms * 1e-3),
            "workspace_bytes": kws_bytes,
            "algorithmic_bytes": kb_,
            "roofline": {"bound": "hbm", "achieved": kb_ / (k_ms * 1e-3) / 1e9,
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": kb_ / (k_ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
            "per_token": {"ms_per_call": kp_ms, "tokens_per_s": tokens / (kp_ms * 1e-3)},
            "chunked_vs_per_token_rel_l2": rel,
        }
        del ok_, sk_, gates, kws, o_chunk

    # decode step, cfg4: B256 H32 D128, fp32 state updated in place, 64 steps
    Bd, Hd = 256, 32
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    state = (torch.randn((Bd, Hd, D, D), generator=g, device=dev) * 0.02).contiguous()
    toks = []
    for _ in range(2):
        qd = torch.randn((Bd, Hd, D), generator=g, device=dev)
        qd = (qd / qd.norm(dim=-1, keepdim=True)).to(torch.bfloat16)
        kd = torch.randn((Bd, Hd, D), generator=g, device=dev)
        kd = (kd / kd.norm(dim=-1, keepdim=True)).to(torch.bfloat16)
        vd = torch.randn((Bd, Hd, D), generator=g, device=dev).to(torch.bfloat16)
        bd = torch.sigmoid(torch.randn((Bd, Hd), generator=g, device=dev))
        toks.append((qd, kd, vd, bd))
    od = torch.empty((Bd, Hd, D), dtype=torch.float32, device=dev)

    def step(i):
        qd, kd, vd, bd = toks[i % 2]
        rc = lib.pm_delta_step(state.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                               bd.data_ptr(), od.data_ptr(), Bd, Hd, D, _native.DTYPE_BF16,
                               stream.cuda_stream)
        _native.check(rc)

    # the state before any step, for the parity check of the whole in-place sequence
    state0_host = state.cpu().numpy() if not args.no_cpu_baseline else None
    spin_up()
    for i in range(4):
        step(i)
    torch.cuda.synchronize()
    # one event pair around the back-to-back steps (as for the forward's roofline)
    step_ms = time_launches(stream, step, args.decode_steps)
    dbytes = step_bytes(Bd, Hd, D)
    dtraffic = None
    if os.path.exists(args.decode_traffic):
        with open(args.decode_traffic) as f:
            dtraffic = json.load(f).get("bytes_per_launch")
    decode = {
        "workload": "cfg4 decode step B256 H32 D128, bf16 token, fp32 state in place",
        "steps": args.decode_steps,
        "us_per_step": step_ms * 1e3,
        "tokens_per_s": Bd / (step_ms * 1e-3),
        "roofline": {"bound": "hbm", "achieved": dbytes / (step_ms * 1e-3) / 1e9,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": dbytes / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                     "traffic": dtraffic},
    }
    decode_host = None
    if state0_host is not None:  # replayed on the C restatement after every GPU leg
        decode_host = (state0_host, [(bits(a), bits(b_), bits(c_), d_.cpu().numpy()) for a, b_, c_, d_ in toks],
                       state.cpu().numpy(), od.cpu().numpy())

    # the same decode through a serving state cache: a pool of 2*B slots, the batch's
    # requests on a random half of them (pm_delta_step_slots)
    pool = (torch.randn((2 * Bd, Hd, D, D), generator=g, device=dev) * 0.02).contiguous()
    perm = torch.randperm(2 * Bd, generator=torch.Generator().manual_seed(6))[:Bd]
    slots = perm.to(torch.int32).to(dev)

    def step_slots(i):
        qd, kd, vd, bd = toks[i % 2]
        rc = lib.pm_delta_step_slots(pool.data_ptr(), slots.data_ptr(), 2 * Bd, qd.data_ptr(),
                                     kd.data_ptr(), vd.data_ptr(), bd.data_ptr(), od.data_ptr(),
                                     Bd, Hd, D, _native.DTYPE_BF16, stream.cuda_stream)
        _native.check(rc)

    spin_up()
    for i in range(4):
        step_slots(i)
    torch.cuda.synchronize()
    slot_ms = time_launches(stream, step_slots, args.decode_steps)
    # the same slots with the table in increasing order (the batch rows still map to the
    # same states): the order in which the workgroups walk the pool
    slots.copy_(torch.sort(slots).values)
    for i in range(4):
        step_slots(i)
    torch.cuda.synchronize()
    sorted_ms = time_launches(stream, step_slots, args.decode_steps)
    decode["state_cache"] = {
        "workload": "cfg4 decode through a 512-slot state cache (pm_delta_step_slots), the batch on a "
                    "random half of the slots",
        "us_per_step": slot_ms * 1e3,
        "roofline": {"bound": "hbm", "achieved": dbytes / (slot_ms * 1e-3) / 1e9,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": dbytes / (slot_ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
        "sorted_table": {"us_per_step": sorted_ms * 1e3,
                         "frac": dbytes / (sorted_ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
    }
    del pool, state

    # What a plain read-modify-write stream reaches on this HBM: torch's in-place
    # elementwise multiply over a 512 MiB fp32 buffer (the bytes one decode step
    # reads and writes back).
    buf = torch.ones((Bd * Hd * D * D,), dtype=torch.float32, device=dev)
    rmw_ms = time_launches(stream, lambda i: buf.mul_(0.9999999), args.decode_steps)
    rmw_gbs = 2 * buf.numel() * 4 / (rmw_ms * 1e-3) / 1e9
    decode["rmw_ceiling"] = {"kernel": "torch in-place mul_ over 512 MiB fp32", "achieved": rmw_gbs,
                             "unit": "GB/s", "frac": rmw_gbs / HBM_PEAK_GBS,
                             "decode_over_rmw": decode["roofline"]["achieved"] / rmw_gbs}
    del buf

    # the model's linear attention (pm_linear_attention_ws: q/k L2-normalised inside the
    # kernel, beta = 1) at the cfg1 shape: bf16 q/k/v on the chunked kernel, fp32 (the
    # reference model's dtype) on the fp32 chunked forward, with the per-token kernel beside
    model_la = None
    if args.model_calls > 0:
        spin_up()
        model_la = {"workload": "cfg1 shape, model.linear_attention (beta 1, L2-normalised q/k)"}
        g.manual_seed(7)
        om = torch.empty((B, T, H, D), device=dev)
        sm = torch.empty((B, H, D, D), device=dev)
        for name, dt, code, s_in in (("bf16", torch.bfloat16, _native.DTYPE_BF16, 2),
                                     ("fp32", torch.float32, _native.DTYPE_F32, 4)):
            qm, km, vm = (torch.randn((B, T, H, D), generator=g, device=dev).to(dt) for _ in range(3))
            nbl = lib.pm_linear_attention_workspace_bytes(B, T, H, D, code)
            wsl = torch.empty(nbl, dtype=torch.uint8, device=dev) if nbl else None

            def la(i, ws=wsl, nb=nbl):
                rc = lib.pm_linear_attention_ws(qm.data_ptr(), km.data_ptr(), vm.data_ptr(), None,
                                                om.data_ptr(), sm.data_ptr(), B, T, H, D, code,
                                                _native.DTYPE_F32, None if ws is None else ws.data_ptr(), nb,
                                                stream.cuda_stream)
                _native.check(rc)

            for i in range(WARM_CALLS):  # first touches of fresh output buffers are slower
                la(i)
            calls = args.model_calls * (10 if name == "bf16" else 5)
            la_ms = time_launches(stream, la, calls)
            lb = fwd_bytes(B, T, H, D, s_in=s_in, s_out=4) - 4 * B * T * H  # no beta array
            model_la[name] = {
                "kernel": "chunked MFMA, norms folded in" if name == "bf16"
                          else "fp32 chunked forward on fp32 MFMA, norms folded in",
                "calls": calls,
                "ms_per_call": la_ms,
                "tokens_per_s": tokens / (la_ms * 1e-3),
                "roofline": {"bound": "hbm", "achieved": lb / (la_ms * 1e-3) / 1e9,
                             "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": lb / (la_ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
            }
            if name == "fp32":
                la(0, None, 0)
                model_la[name]["per_token_ms_per_call"] = time_launches(
                    stream, lambda i: la(i, None, 0), args.model_calls * 2)
            del qm, km, vm, wsl
        del om, sm

    # the same cfg1 forward with fp32 q/k/v (the reference's dtype): the per-token kernel
    fp32_fwd = None
    if args.model_calls > 0:
        fsets = [tuple(x.float() for x in st_) for st_ in sets]  # both input sets, alternating
        of = torch.empty((B, T, H, D), device=dev)
        sf = torch.empty((B, H, D, D), device=dev)
        nbf = lib.pm_delta_workspace_bytes(B, T, H, D, _native.DTYPE_F32)
        wsf = torch.empty(nbf, dtype=torch.uint8, device=dev) if nbf else None

        def ffwd(ws, i=0):
            q, k, v, beta = fsets[i % 2]
            rc = lib.pm_delta_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), None,
                                  of.data_ptr(), sf.data_ptr(), B, T, H, D, _native.DTYPE_F32,
                                  _native.DTYPE_F32, CHUNK, None if ws is None else ws.data_ptr(),
                                  0 if ws is None else ws.numel(), stream.cuda_stream)
            _native.check(rc)

        def time_ffwd(ws, calls):
            for i in range(WARM_CALLS if ws is not None else 1):  # first touches of fresh output buffers are slower
                ffwd(ws, i)
            return time_launches(stream, lambda i: ffwd(ws, i), calls)

        calls = args.model_calls * 5
        f_ms = time_ffwd(wsf, calls)  # the default: the fp32 chunked forward on fp32 MFMA
        old_path = _native.set_path(1)
        try:
            r_ms = time_ffwd(None, args.model_calls * 2)  # the per-token VALU kernel
        finally:
            _native.set_path(old_path)
        fb = fwd_bytes(B, T, H, D, s_in=4, s_out=4)
        cflop = fwd_flops(B, T, H, D, chunk=16)  # the chunked form at 16-token chunks
        rflop = 6 * B * T * H * D * D  # per token: k.S, q.S and the rank-1 update, 2 flops per FMA
        fp32_fwd = {
            "workload": "cfg1 forward with fp32 q/k/v (pm_delta_fwd, fp32 chunked forward on fp32 MFMA)",
            "calls": calls,
            "ms_per_call": f_ms,
            "tokens_per_s": tokens / (f_ms * 1e-3),
            "workspace_bytes": nbf,
            "roofline": {"bound": "mfma", "achieved": cflop / (f_ms * 1e-3) / 1e12,
                         "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": cflop / (f_ms * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS,
                         "algorithmic_gflop": cflop / 1e9},
            "hbm_gbs": fb / (f_ms * 1e-3) / 1e9,
            "per_token": {
                "kernel": "per-token fp32 VALU kernel (pm_delta_set_path 1)",
                "ms_per_call": r_ms,
                "roofline": {"bound": "valu", "achieved": rflop / (r_ms * 1e-3) / 1e12,
                             "peak": FP32_VALU_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": rflop / (r_ms * 1e-3) / 1e12 / FP32_VALU_PEAK_TFLOPS},
            },
        }
        del fsets, of, sf, wsf

    # backward at cfg1 (chunked_delta_rule_bwd through the C ABI): bf16 q/k/v, zero S0,
    # random go and gS, fp32 gradients
    backward = None
    if args.bwd_steps > 0:
        spin_up()
        q, k, v, beta = sets[last]
        g.manual_seed(5)
        go = torch.randn((B, T, H, D), generator=g, device=dev)
        gs = torch.randn((B, H, D, D), generator=g, device=dev) * 0.05
        gq, gk, gv = (torch.empty((B, T, H, D), device=dev) for _ in range(3))
        gb = torch.empty((B, T, H), device=dev)
        gs0 = torch.empty((B, H, D, D), device=dev)
        ws_bytes = lib.pm_delta_bwd_workspace_bytes(B, T, H, D, _native.DTYPE_BF16)
        ws = torch.empty(((ws_bytes + 3) // 4,), device=dev)

        def bwd():
            rc = lib.pm_delta_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), None,
                                  go.data_ptr(), gs.data_ptr(), gq.data_ptr(), gk.data_ptr(),
                                  gv.data_ptr(), gb.data_ptr(), gs0.data_ptr(), B, T, H, D,
                                  _native.DTYPE_BF16, ws.data_ptr(), ws_bytes, stream.cuda_stream)
            _native.check(rc)

        for _ in range(60):  # warm-up: about 25 ms of calls, past the clock's ramp
            bwd()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.bwd_steps):
            bwd()
        e1.record(stream)
        torch.cuda.synchronize()
        bwd_ms = e0.elapsed_time(e1) / args.bwd_steps
        bb = bwd_bytes(B, T, H, D)
        backward = {
            "workload": "cfg1 backward (chunked_delta_rule_bwd), bf16 q/k/v, fp32 grads",
            "calls": args.bwd_steps,
            "ms_per_call": bwd_ms,
            "tokens_per_s": tokens / (bwd_ms * 1e-3),
            "workspace_bytes": ws_bytes,
            "roofline": {"bound": "hbm", "achieved": bb / (bwd_ms * 1e-3) / 1e9,
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": bb / (bwd_ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
        }
        del ws
        # the same backward with fp32 q/k/v (the reference's dtype): the fp32 chunked backward
        # on fp32 MFMA, and the per-token kernel (path 1) beside it
        q, k, v = (x.float() for x in (q, k, v))
        ws_bytes = lib.pm_delta_bwd_workspace_bytes(B, T, H, D, _native.DTYPE_F32)
        ws = torch.empty(((ws_bytes + 3) // 4,), device=dev)

        def bwd32():
            rc = lib.pm_delta_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), None,
                                  go.data_ptr(), gs.data_ptr(), gq.data_ptr(), gk.data_ptr(),
                                  gv.data_ptr(), gb.data_ptr(), gs0.data_ptr(), B, T, H, D,
                                  _native.DTYPE_F32, ws.data_ptr(), ws_bytes, stream.cuda_stream)
            _native.check(rc)

        for _ in range(20):  # warm-up, as above
            bwd32()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(args.bwd_steps):
            bwd32()
        e1.record(stream)
        torch.cuda.synchronize()
        b32_ms = e0.elapsed_time(e1) / args.bwd_steps
        f32 = bwd32_flops(B, T, H, D)
        backward["fp32"] = {
            "workload": "cfg1 backward with fp32 q/k/v (fp32 chunked backward on fp32 MFMA)",
            "calls": args.bwd_steps,
            "ms_per_call": b32_ms,
            "tokens_per_s": tokens / (b32_ms * 1e-3),
            "workspace_bytes": ws_bytes,
            "roofline": {"bound": "mfma", "achieved": f32 / (b32_ms * 1e-3) / 1e12,
                         "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": f32 / (b32_ms * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS,
                         "flops": f32},
        }
        del ws
        with _native.use_knobs(1, 0):
            ws_bytes = lib.pm_delta_bwd_workspace_bytes(B, T, H, D, _native.DTYPE_F32)
            ws = torch.empty(((ws_bytes + 3) // 4,), device=dev)
            bwd32()
            torch.cuda.synchronize()
            e0.record(stream)
            for _ in range(max(1, args.bwd_steps // 2)):
                bwd32()
            e1.record(stream)
            torch.cuda.synchronize()
        backward["fp32"]["per_token_ms_per_call"] = e0.elapsed_time(e1) / max(1, args.bwd_steps // 2)
        backward["fp32"]["per_token_workspace_bytes"] = ws_bytes
        del go, gs, gq, gk, gv, gb, gs0, ws, q, k, v

    if args.calib_copy:
        n = CALIB_COPY_BYTES // 4
        x = torch.randn(n, device=dev)
        y = torch.empty_like(x)
        for _ in range(3):
            torch.neg(x, out=y)
        torch.cuda.synchronize()
        del x, y

    # parity of the timed output against the C restatement (which is also the CPU baseline)
    cpu = None
    parity = None
    if not args.no_cpu_baseline:
        from oracle import cref

        hq, hk, hv, hb = host_in
        threads = cpu_threads()
        print(f"[bench] CPU baseline on {threads} threads", file=sys.stderr, flush=True)
        cref.delta_fwd(hq[:, :64], hk[:, :64], hv[:, :64], hb[:, :64], None, threads=threads)
        # the full batch, repeated for about CPU_SAMPLE_S seconds of CPU work
        t1 = time.perf_counter()
        e_o, e_s = cref.delta_fwd(hq, hk, hv, hb, None, threads=threads)
        reps = 1
        while time.perf_counter() - t1 < CPU_SAMPLE_S and reps < 1000:
            cref.delta_fwd(hq, hk, hv, hb, None, threads=threads)
            reps += 1
        cpu_s = (time.perf_counter() - t1) / reps
        got_o, got_s = host_o, host_s
        rel = lambda a, b: float(np.linalg.norm((a - b).ravel()) / np.linalg.norm(b.ravel()))  # noqa
        parity = {"rel_l2_o": rel(got_o, e_o), "rel_l2_s": rel(got_s, e_s), "bound": 2e-2}
        parity["ok"] = parity["rel_l2_o"] <= 2e-2 and parity["rel_l2_s"] <= 2e-2
        cpu = {"value": tokens / cpu_s, "unit": "tokens/s", "cores": threads, "kind": "port",
               "sample": f"full cfg1 batch (B4 T4096 H16 D128, bf16 inputs upcast to fp32), "
                         f"{reps} repeats, {cpu_s:.3f} s each; C restatement of the reference's per-token rank-1 "
                         f"recurrence (oracle/delta_ref.c), OpenMP over 64 (b,h) sequences",
               "cpu_model": cpu_model(),
               "affinity_cpus": len(os.sched_getaffinity(0)),
               "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS"),
               "threads_used": threads,
               "threads_rule": "OMP_NUM_THREADS when set (the box's CPU share), else the affinity count"}
        # the other BASELINE configurations on the same CPU path, per call / per step
        x0 = synth.fwd_inputs((1, 256, 4, 64), seed=0, dtype="fp32")
        t1 = time.perf_counter()
        reps0 = 0
        while time.perf_counter() - t1 < 1.0:
            cref.delta_fwd(x0.q, x0.k, x0.v, x0.beta, None, threads=threads)
            reps0 += 1
        cpu["cfg0_ms_per_call"] = (time.perf_counter() - t1) * 1e3 / reps0
        cpu["cfg0_tokens_per_s"] = 256 / ((time.perf_counter() - t1) / reps0)

    if decode_host is not None:
        # every decode step the GPU ran (4 untimed + the timed ones), replayed on the C
        # restatement
        from oracle import cref

        threads = cpu_threads()
        s_ref, htoks, got_state, got_od = decode_host
        n_all = 4 + args.decode_steps
        t1 = time.perf_counter()
        for i in range(n_all):
            e_od = cref.delta_step(s_ref, *htoks[i % 2], threads=threads)
        cpu_step_s = (time.perf_counter() - t1) / n_all
        rel = lambda a, b: float(np.linalg.norm((a - b).ravel()) / np.linalg.norm(b.ravel()))  # noqa
        decode["parity"] = {"steps_checked": n_all, "rel_l2_final_state": rel(got_state, s_ref),
                            "rel_l2_last_o": rel(got_od, e_od), "bound": 1e-5}
        decode["parity"]["ok"] = (decode["parity"]["rel_l2_final_state"] <= 1e-5
                                  and decode["parity"]["rel_l2_last_o"] <= 1e-5)
        if cpu is not None:
            cpu["cfg4_ms_per_step"] = cpu_step_s * 1e3
            cpu["cfg4_tokens_per_s"] = Bd / cpu_step_s
        del s_ref

    line = {
        "metric": "delta-rule fwd tokens/s + % MFMA/HBM roofline, B4·H16·T4096·d128 bf16",
        "value": tokens / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded torch RNG: q,k L2-normalised N(0,1), v N(0,1), "
                "beta sigmoid(N(0,1)); two input sets alternate)",
        "config": {"workload": "cfg1 delta-rule forward", "B": B, "T": T, "H": H, "d_k": D,
                   "d_v": D, "chunk": CHUNK, "in_dtype": "bf16", "out_dtype": "fp32",
                   "state0": "zeros"},
        "roofline": {"bound": "hbm", "achieved": achieved_gbs, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved_gbs / HBM_PEAK_GBS, "traffic": traffic},
        "mfma": {"achieved_tflops": tflops, "peak_tflops": BF16_PEAK_TFLOPS,
                 "frac": tflops / BF16_PEAK_TFLOPS, "algorithmic_gflop": flops / 1e9,
                 "counters": mfma_counters},
        "attainable_roofline_frac": max(flops / (BF16_PEAK_TFLOPS * 1e12),
                                        nbytes / (HBM_PEAK_GBS * 1e9)) / (kern_ms * 1e-3),
        "kernel_us": kern_ms * 1e3,
        "algorithmic_bytes": nbytes,
        "cpu_baseline": cpu,
        "parity": parity,
        "decode": decode,
        "bf16_out": bf16_out,
        "split_form": split_form,
        "cfg3": cfg3,
        "cfg2": cfg2,
        "model_linear_attention": model_la,
        "fp32_forward": fp32_fwd,
        "gated": gated,
        "kda": kda,
        "backward": backward,
    }
    print(json.dumps(line), flush=True)
    if parity is not None and not parity["ok"]:
        sys.exit(3)
    if decode.get("parity") is not None and not decode["parity"]["ok"]:
        sys.exit(3)


if __name__ == "__main__":
    main()
