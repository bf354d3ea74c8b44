"""Stand-in package tree for the ROCm install-hook tests (not vLLM code)."""
