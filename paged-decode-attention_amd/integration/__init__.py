"""Serving-engine integration of the HIP paged decode (vLLM V1)."""
