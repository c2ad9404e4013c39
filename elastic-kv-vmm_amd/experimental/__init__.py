"""Fixed-position virtual layout, resident arena and row gather.

Mirrors the reference package experimental: virtual_layout, resident_arena,
sparse_read.
"""
