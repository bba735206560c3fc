"""TEST INFRASTRUCTURE — CPU oracle for Theorem's four hot kernels.

Not product code: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import anything here, and only as the checker (or, in
bench.py, as the timed CPU baseline).  The product path (theorem_amd) never
imports this package.

  conv.py      causal conv: NumPy restatement of scripts/cpu_reference.py:40-63,
               the C restatement in conv1d.c (ctypes), and a brute-force loop.
  deltanet.py  NumPy restatements of chunk_fwd_h (reference and delta forms),
               chunk_fwd_o, recompute_w_u and the A builder, plus a token-level
               gated delta rule used to pin the chunked chain.

How each function is pinned (closed forms, library routines, brute force) is
listed in the tests under tests/test_oracle_*.py.  No function here is left
unpinned.
"""
