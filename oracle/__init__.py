"""CPU oracle for the AWQ W4A16 path: test infrastructure only.

Imported by tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg,
as the checker; the product package never imports it.
"""
