"""Gated DeltaNet WY recompute of (w, u) on MI355X (gfx950 HIP).

Exports:
    custom_kernel(data) -> (w, u)   HIP implementation
    ref_kernel(data)    -> (w, u)   eager PyTorch reference
    build_A(k, beta, g, sign)       HIP WY matrix (the step before recompute_w_u)
"""
from .kernel import SHAPE_CONFIGS, SHAPE_LIST, build_A, custom_kernel
from .reference import BT, Data, generate_data, generate_input, ref_kernel

__all__ = ["custom_kernel", "build_A", "ref_kernel", "generate_data", "generate_input", "Data", "BT",
           "SHAPE_CONFIGS", "SHAPE_LIST"]
