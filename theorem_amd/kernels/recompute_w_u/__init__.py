"""Gated DeltaNet WY recompute of (w, u) on MI355X (gfx950 HIP).

Exports:
    custom_kernel(data) -> (w, u)   HIP implementation
    ref_kernel(data)    -> (w, u)   eager PyTorch reference
"""
from .kernel import SHAPE_CONFIGS, SHAPE_LIST, custom_kernel
from .reference import BT, Data, generate_data, generate_input, ref_kernel

__all__ = ["custom_kernel", "ref_kernel", "generate_data", "generate_input", "Data", "BT",
           "SHAPE_CONFIGS", "SHAPE_LIST"]
