"""Sparse-KV residency hot path: resident lookup, Top-K gather, migration.

Mirrors the reference package adaptive_sparse: resident_lookup,
sparse_read, migration, migration_budget, minimax_vmm (PhysicalPages).
"""
