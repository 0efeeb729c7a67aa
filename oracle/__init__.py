"""CPU oracle for the quantized-linear hot path (test infrastructure only).

Imported only by tests, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py``; the product never uses it.
"""
