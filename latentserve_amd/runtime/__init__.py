"""Host-side runtime around the HIP decode path: the paged cache's
bookkeeping, a Qwen2.5-1.5B-geometry decoder for full-step runs, and the
HIP-graph bucket runner."""
