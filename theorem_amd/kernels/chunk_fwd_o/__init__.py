"""Gated DeltaNet chunkwise output (forward, o) on MI355X (gfx950 HIP)."""
from .kernel import custom_kernel
from .reference import _build_inputs, generate_input, ref_kernel

__all__ = ["custom_kernel", "ref_kernel", "generate_input", "_build_inputs"]
