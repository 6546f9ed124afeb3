"""Paged-decode runtime: paged KV cache and the dense attention backend."""
