"""TEST INFRASTRUCTURE — the CPU oracle of the decode hot path.

This package restates, on the CPU, the algorithms of proof-carrying-kernels that the HIP
library must reproduce: the GEMV summation-tree models, the CPU blocked checker, the exact
threshold of the GPU checker and the token-membership check.  Each function cites the
reference file:line it follows.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
anything from here, and only as the checker (or, for the bench, as the CPU baseline that is
timed beside the GPU).  The product package `pck` never imports this package: its GPU entry
points fail loudly when the HIP library is missing instead of falling back to these models.
"""
