"""Benchmark scripts (run as modules)."""
