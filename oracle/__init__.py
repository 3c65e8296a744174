"""CPU oracle for the delta-rule forward — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import, call or link anything here, and only as the checker
(or the timed CPU baseline). The product path (``prometheus_amd``) never
imports this package and has no CPU fallback.

Contents
--------
``delta_oracle.py``
    NumPy restatements:
      * ``gated_delta_rule`` — explicit per-token recurrence with the
        (I - beta k k^T) matrix, after the reference's NumPy oracle
        ``tests/reference/kernels.py:134-171``;
      * ``delta_step`` — the rank-1 single-token step,
        ``kernels/__init__.py:357-376``;
      * ``chunked_fwd_rank1`` — the reference's chunk traversal
        ``kernels/__init__.py:379-395`` / ``:421-458``;
      * ``wy_chunked_fwd`` — the chunked WY/UT form the GPU kernel uses,
        an independent formulation (not in the reference), fp64;
      * ``varlen_fwd`` — packed cu_seqlens batch as independent per-segment
        calls (no reference counterpart; reduces to ``gated_delta_rule``).
``delta_ref.c`` (built to ``oracle/libdelta_oracle.so`` by ``build.py``)
    C restatement of the same per-token rank-1 recurrence, fp32, OpenMP over
    the B*H independent sequences: the CPU baseline ``bench.py`` times.

Pinning (each function is checked by ``tests/test_oracle.py``):
    * the reference's three closed-form goldens
      (``tests/test_kernels.py:279-316``),
    * its invariants (causality, state carry, chunk independence, linearity
      in v, S independent of q, None == zeros: ``tests/test_kernels.py:319-406``),
    * agreement between the three independent formulations (explicit
      matrix, rank-1, WY/UT) in fp64,
    * special cases the mathematics fixes (T=1 from zero state:
      S = beta k v^T, o = beta (q.k) v; orthonormal keys with beta=1 give
      o_t = v_t; a planted sign/index error must be caught).
"""
