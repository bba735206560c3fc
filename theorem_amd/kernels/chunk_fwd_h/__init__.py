"""chunk_fwd_h: Gated DeltaNet inter-chunk state recurrence on MI355X (gfx950 HIP)."""
from .kernel import custom_kernel
from .reference import generate_input, ref_kernel, ref_kernel_delta

__all__ = ["custom_kernel", "ref_kernel", "ref_kernel_delta", "generate_input"]
