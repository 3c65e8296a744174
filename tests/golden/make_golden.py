"""Write the golden fixtures under tests/golden/ (run from the repo root).

    python tests/golden/make_golden.py

Fixtures hold expected outputs computed in fp64 by the oracle (two
independent formulations that must agree to 1e-10 before anything is
written) on seeded inputs; the inputs themselves are regenerated from the
seeds with ``prometheus_amd.synth`` and pinned by a SHA-256 of their bytes.
No reference code is imported or run: the seeded cases mirror the inputs of
the reference's own tests (tests/test_kernels.py, tests/test_kernels_delta_fwd_jit.py)
and the BASELINE cfg0 distribution.
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import delta_oracle as ref  # noqa: E402
from prometheus_amd import synth  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def reference_cases():
    """(name, q, k, v, beta, state, chunk) mirroring the reference tests' seeds."""
    cases = []
    r = np.random.default_rng(10)
    cases.append(("rng10", *synth.reference_test_inputs(r), None, 64))
    r = np.random.default_rng(12)
    cases.append(("rng12_seq7", *synth.reference_test_inputs(r, seq=7), None, 64))
    r = np.random.default_rng(13)
    cases.append(("rng13_seq10_d3", *synth.reference_test_inputs(r, seq=10, dim=3), None, 4))
    r = np.random.default_rng(14)
    cases.append(("rng14_seq20_h1_d3", *synth.reference_test_inputs(r, seq=20, heads=1, dim=3),
                  None, 64))
    r = np.random.default_rng(19)
    cases.append(("rng19_seq6", *synth.reference_test_inputs(r, seq=6), None, 64))
    r = np.random.default_rng(101)
    q, k, v, b = synth.reference_test_inputs(r, batch=2, seq=5, heads=2, dim=4)
    s0 = (r.standard_normal((2, 2, 4, 4)).astype(np.float32) * 0.05)
    cases.append(("rng101_chunk2_state", q, k, v, b, s0, 2))
    cases.append(("rng101_chunk4_none", q, k, v, b, None, 4))
    q1, k1, v1, b1 = synth.reference_test_inputs(r, batch=1, seq=3, heads=1, dim=3)
    cases.append(("rng101_default", q1, k1, v1, b1, None, 64))
    r = np.random.default_rng(106)
    q, k, v, b = synth.reference_test_inputs(r, batch=2, seq=5, heads=2, dim=3)
    s0 = r.standard_normal((2, 2, 3, 3)).astype(np.float32) * 0.05
    cases.append(("rng106_state_d3", q, k, v, b, s0, 2))
    r = np.random.default_rng(107)
    q, k, v, b = synth.reference_test_inputs(r, batch=2, seq=5, heads=2, dim=4)
    s0 = r.standard_normal((2, 2, 4, 4)).astype(np.float32) * 0.05
    cases.append(("rng107_state", q, k, v, b, s0, 2))
    r = np.random.default_rng(50)
    cases.append(("rng50_gpu_2x16x2x8",
                  *synth.reference_test_inputs(r, batch=2, seq=16, heads=2, dim=8), None, 64))
    return cases


def expected(q, k, v, b, s0, chunk):
    o1, s1 = ref.gated_delta_rule(q, k, v, b, s0, dtype=np.float64)
    o2, s2 = ref.wy_chunked_fwd(q, k, v, b, s0, chunk=chunk, dtype=np.float64)
    o3, s3 = ref.chunked_fwd_rank1(q, k, v, b, s0, chunk=chunk, dtype=np.float64)
    scale = max(1.0, float(np.abs(o1).max()), float(np.abs(s1).max()))
    for a, c in ((o1, o2), (o1, o3), (s1, s2), (s1, s3)):
        err = float(np.abs(a - c).max()) / scale
        assert err < 1e-10, f"oracle formulations disagree: {err}"
    return o1.astype(np.float32), s1.astype(np.float32)


def main():
    out = {}
    for name, q, k, v, b, s0, chunk in reference_cases():
        o, s = expected(q, k, v, b, s0, chunk)
        out[f"{name}/sha"] = np.array(sha(q, k, v, b, s0))
        out[f"{name}/chunk"] = np.array(chunk)
        out[f"{name}/o"] = o
        out[f"{name}/s"] = s
    np.savez_compressed(os.path.join(HERE, "reference_cases.npz"), **out)

    # BASELINE cfg0: B1 H4 T256 D64 fp32, seed 0, chunk 64, S0 = 0
    c = synth.CONFIGS[0]
    x = synth.fwd_inputs((c["B"], c["T"], c["H"], c["D"]), seed=0, dtype="fp32")
    o_r, s_r = ref.chunked_fwd_rank1(x.q, x.k, x.v, x.beta, None, 64, dtype=np.float64)
    o_w, s_w = ref.wy_chunked_fwd(x.q, x.k, x.v, x.beta, None, 64, dtype=np.float64)
    assert np.abs(o_r - o_w).max() < 1e-10 and np.abs(s_r - s_w).max() < 1e-10
    np.savez_compressed(os.path.join(HERE, "cfg0.npz"), sha=np.array(sha(x.q, x.k, x.v, x.beta)),
                        o=o_r.astype(np.float32), s=s_r.astype(np.float32))
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
