"""CPU oracle for the continuous-depth-batching decode step.

TEST INFRASTRUCTURE ONLY. This package restates, in numpy, the reference's
algorithms for the CDB decode step (paged decode attention with KV append,
RoPE, RMSNorm, the exit gates, slot mapping and block tables, and the
scheduler's refill order). It exists to check the HIP kernels and the engine:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker. The product path
(``continuous_depth_batching_amd``) never imports it and has no CPU fallback.

Each function cites the reference file:line it restates. How each one is
pinned (golden vectors, closed forms, invariants, library routines) is stated
in its module docstring.
"""
