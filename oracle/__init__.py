"""CPU oracle for the NF4 decode hot path - TEST INFRASTRUCTURE.

Only the tests, `__graft_entry__.smoke()` and the CPU-baseline leg of
`bench.py` import this package, and only as the checker (or the timed CPU
baseline); the product (`ttspipe_amd`) never does.
"""
