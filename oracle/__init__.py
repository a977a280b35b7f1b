"""Test infrastructure only: CPU restatement of the reference's Pi0 decoder path.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s CPU-baseline leg may
import this package, and only as the checker. The product path never calls it.
"""
