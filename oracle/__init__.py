"""CPU oracle for the fused residual + dropout + LayerNorm - TEST INFRASTRUCTURE ONLY.

Imported only by tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of bench.py, and only as the checker; the product never uses it.
"""
