"""Host-side data layout producers (packing)."""
