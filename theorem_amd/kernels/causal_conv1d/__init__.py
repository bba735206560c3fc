"""Depthwise causal 1-D convolution on MI355X (gfx950 HIP)."""
from .kernel import causal_conv1d_update, custom_kernel
from .reference import generate_input, ref_kernel

__all__ = ["custom_kernel", "causal_conv1d_update", "ref_kernel", "generate_input"]
