"""Minimal stand-in for the parts of vLLM the GRINQH plugin imports, so the
plugin's config / linear-method surface can be exercised on a CPU-only host.
Test infrastructure only; a real deployment imports the real vLLM."""
