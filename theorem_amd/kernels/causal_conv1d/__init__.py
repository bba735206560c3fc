"""Depthwise causal 1-D convolution on MI355X (gfx950 HIP)."""
from .kernel import custom_kernel
from .reference import generate_input, ref_kernel

__all__ = ["custom_kernel", "ref_kernel", "generate_input"]
