"""Build libtheorem_mi355x.so (gfx950 HIP kernels + C ABI) in-tree with hipcc.

Usage: python -m theorem_amd.build [-v]

Objects go to theorem_amd/_build/, the shared library to
theorem_amd/lib/libtheorem_mi355x.so (loaded by theorem_amd.kernels._capi).
A second library, theorem_amd/lib/libtheorem_floors.so (csrc/floors.hip),
holds the memory-only pattern kernels bench.py times as each kernel's floor;
it is measurement tooling, not part of the C ABI.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ_DIR = PKG / "_build"
LIB_DIR = PKG / "lib"
LIB_NAME = "libtheorem_mi355x.so"
LIB_PATH = LIB_DIR / LIB_NAME

SOURCES = [
    "capi.cpp",
    "causal_conv1d.hip",
    "causal_conv1d_ext.hip",
    "recompute_w_u.hip",
    "chunk_fwd_h.hip",
    "chunk_fwd_h_f32.hip",
    "chunk_fwd_o.hip",
    "chunk_fwd_fused.hip",
    "wy_build_A.hip",
    "wy_fwd.hip",
    "gates.hip",
]

# Per-unit code generation.  Forcing MFMA accumulators into VGPRs (no AGPR
# copies) measured faster for these units (recompute_w_u bf16 275.1 -> 271.6 us,
# the bf16 register chunk_fwd_h at config 3 25.5 -> 24.4 us, config 4
# bit-identical outputs) and slower for the fp32 register chunk_fwd_h and the
# fp32 chunk_fwd_o (775 -> 884 and 883 -> 927 us), so it is not global.
MFMA_VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
UNIT_FLAGS = {
    "recompute_w_u.hip": MFMA_VGPR_FORM,
    "chunk_fwd_h.hip": MFMA_VGPR_FORM,
}

FLOORS_SRC = "floors.hip"
FLOORS_LIB = LIB_DIR / "libtheorem_floors.so"

# Host fast path of the custom_kernel wrappers: a pybind11 module over torch
# tensors, linked against the C-ABI library (theorem_amd/kernels/_capi.py
# loads it when present; the wrappers' ctypes path is the same kernels).
FAST_SRC = "host/fastpath.cpp"
FAST_NAME = "_fastpath"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed-fp32 VALU ops are disabled for all device code; the host pass warns
# that it does not know the feature, which is harmless.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line for line in (r.stdout + r.stderr).splitlines()
        if "is not a recognized feature for this target" not in line
    )
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip() and verbose:
        print(out)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source for gfx950 and link the shared library; return its path."""
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    missing = [s for s in SOURCES + [FLOORS_SRC, FAST_SRC] if not (CSRC / s).exists()]
    if missing:
        raise RuntimeError(f"missing sources in {CSRC}: {', '.join(missing)}")
    srcs = [CSRC / s for s in SOURCES]
    objs = [OBJ_DIR / (s.name + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [
            ex.submit(_run, [HIPCC, *COMMON_FLAGS, *UNIT_FLAGS.get(s.name, []), "-c", str(s), "-o", str(o)], verbose)
            for s, o in zip(srcs, objs)
        ]
        for f in futs:
            f.result()
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,-soname,{LIB_NAME}", "-o", str(tmp),
          *map(str, objs)], verbose)
    os.replace(tmp, LIB_PATH)
    ftmp = LIB_DIR / (FLOORS_LIB.name + ".tmp")
    _run([HIPCC, *COMMON_FLAGS, "-shared", "-o", str(ftmp), str(CSRC / FLOORS_SRC)], verbose)
    os.replace(ftmp, FLOORS_LIB)
    build_fastpath(verbose)
    return LIB_PATH


def fastpath_path() -> Path:
    import sysconfig

    return LIB_DIR / (FAST_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def build_fastpath(verbose: bool = False) -> Path:
    """g++ the pybind11 fast-path module against torch's headers and libraries
    and the C-ABI library (rpath $ORIGIN: both live in theorem_amd/lib)."""
    import sysconfig

    import torch.utils.cpp_extension as ce

    out = fastpath_path()
    tmp = out.with_name(out.name + ".tmp")
    torch_lib = ce.library_paths()[0]
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__",
           "-DTORCH_EXTENSION_NAME=" + FAST_NAME, "-DTORCH_API_INCLUDE_EXTENSION_H",
           "-I/opt/rocm/include", f"-I{PKG.parent / 'include'}",
           *(f"-I{p}" for p in ce.include_paths()), f"-I{sysconfig.get_paths()['include']}",
           str(CSRC / FAST_SRC), "-o", str(tmp),
           f"-L{LIB_DIR}", "-ltheorem_mi355x", f"-L{torch_lib}",
           "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    p = build(verbose="-v" in sys.argv)
    print(p)
