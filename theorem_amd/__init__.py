"""theorem_amd — MI355X (gfx950) HIP implementation of Theorem's four hot kernels.

Layout mirrors the reference project root, so the reference's harness idioms
work unchanged with this package directory as the project root:

  kernels/<name>/      drop-in packages: custom_kernel, ref_kernel, generate_input, task.yml
  kernels/_capi.py     ctypes binding of lib/libtheorem_mi355x.so (the C ABI in include/)
  utils.py, eval.py    harness helpers and the test/benchmark driver
  benchmarks/          PyTorch eager / torch.compile comparison
  chain.py             Gated DeltaNet chunk forward composed from the three ops
  configs.py           seeded generators for the BASELINE configurations
  csrc/                HIP sources; build.py compiles them with hipcc
"""
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
