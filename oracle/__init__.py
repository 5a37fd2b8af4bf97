"""CPU oracle for vectra::rbf_attention -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or, for bench.py, the timed CPU
baseline).  The product (vectra_amd) never imports it: the device path runs
the HIP library or fails.

Contents (oracle/rbf.py), each a restatement of a reference formulation:

  direct_fp64     sum_d (q - k)^2 in float64 (reference.py:46-58 at fp64)
  expanded_fp64   Euclidean expansion in float64 (reference.py:61-76)
  eager_fp32      the eager operator chain in torch fp32 (reference.py:46-58)
  tiled           the kernel's online-softmax tile loop (reference.py:102-161)

Pins (tests/test_oracle.py): brute-force pure-Python loops on tiny inputs,
the committed brute-force fixtures in tests/golden/, torch's
scaled_dot_product_attention and cdist identities, closed-form special cases
(one live key, fully masked rows, zero scale, a single key), and planted
mistakes that each pin must catch.  No function here is "parity unpinned".

The reference is Python + Triton; there is no C/C++ source on this path, so
there is no oracle/_ref build.
"""
