"""Serving-framework integration of the packed paged hot path (reference:
turboquant/integration/).  paged_backend holds the per-layer state, the boundary-layer policy
and a decode attention implementation in vLLM's shape; vLLM itself is not required."""
