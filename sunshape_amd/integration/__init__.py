"""Serving-runtime integration points (vLLM runtime state)."""
