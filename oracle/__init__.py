"""CPU oracle of the sparse-KV residency hot path - test infrastructure only.

Imported by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg
to verify the HIP kernels' results; never by the product package.
"""
