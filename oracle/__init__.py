"""CPU oracle for the eager nanoGPT hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (float64 unless noted), the arithmetic the
reference computes on its hot path.  Only `tests/`, `__graft_entry__.smoke()`
and `bench.py`'s `cpu_baseline` leg may import it, and only as the checker
or the CPU baseline: the product path (`torch_mojo_backend`) never imports,
calls or falls back to anything here.

The reference's own oracle for these ops is stock PyTorch CPU ATen in f32
(torch_mojo_backend/testing.py:186-229; tests/test_eager_kernels.py:
10083-10094; tests/test_eager_optimizer_ops.py:65-435).  Each function in
`ops.py` cites the reference file:line whose semantics it follows and is
pinned in tests/test_oracle.py against (a) PyTorch CPU on seeded inputs,
(b) the committed golden vectors in tests/golden/, and (c) properties the
mathematics fixes (closed forms, invariants, finite differences, brute
force on tiny inputs).
"""
