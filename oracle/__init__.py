"""CPU oracle for the weight-quantized matmul path. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this package, and only
as the checker (or, for the baseline, as the CPU path that is timed). The product (``mojo-adreno_amd/aq``) never
imports it and has no CPU fallback.
"""
