"""Launch and memory planning for the MI355X hot path (CPU-only math, testable without a GPU)."""
