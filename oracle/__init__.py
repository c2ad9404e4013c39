"""CPU oracle of the sparse-KV residency hot path - test infrastructure only.

Imported by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg
as the checker of the HIP kernels; never by the product package.
"""
