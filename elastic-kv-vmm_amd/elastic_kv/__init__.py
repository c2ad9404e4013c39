"""HIP VMM backing of a demand-backed KV range (MI355X / gfx950).

Mirrors the reference package elastic_kv: backing.Backing, slots.FreeSlots,
adapter.PlaneProjection.
"""
