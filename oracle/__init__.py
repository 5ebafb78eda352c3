"""CPU oracle for parity tests — test infrastructure, never part of the product path.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s cpu_baseline leg may import it.
"""
