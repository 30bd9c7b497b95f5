"""CPU oracle for the quantized decode hot path -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's pure-array ``reference_*`` path of
manishklach/mlx-metal-kernels (the MLX ops the reference runs; MLX itself is
not installable here).  Each function cites the reference file:line it
follows.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker /
the timed CPU baseline -- the product path (the ``mk`` package and
``libmk_hip.so``) never calls it.

Pinning (tests/test_oracle.py): every function is checked against the
reference tests' known answers where they exist, and otherwise against
closed forms, invariants and brute-force loops that mirror the reference's
scalar Metal kernels on tiny inputs.  Functions whose check is only a
tolerance-level match to textbook math say so in their docstring.
"""
