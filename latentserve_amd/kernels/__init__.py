"""Kernel front ends: ``gqa.paged_decode`` (the dispatch API) and ``hip`` (the backend)."""
