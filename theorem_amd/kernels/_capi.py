"""ctypes binding of libtheorem_mi355x.so, the C ABI declared in include/theorem_mi355x.h.

The library is loaded from the package's lib/ directory (built in-tree by
``python -m theorem_amd.build``).  There is no fallback: if the library is
missing, every kernel call raises.  Tensors cross the boundary as raw device
pointers; the launch goes onto torch's current stream of the tensors' device.

Status handling mirrors the C ABI: a negative status (argument rejected on the
host, nothing launched) raises ``ValueError``; a positive status (a HIP launch
error) raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent.parent / "lib" / "libtheorem_mi355x.so"
ABI_VERSION = 1

THM_DTYPE = {torch.float32: 0, torch.bfloat16: 1}
THM_ACT_NONE = 0
THM_ACT_SILU = 1
THM_H_DELTA = 1

_c_vp = ctypes.c_void_p
_c_i64 = ctypes.c_int64
_c_i32 = ctypes.c_int32

# name -> argtypes (restype is c_int unless listed in _RESTYPES)
SIGNATURES = {
    "thm_abi_version": [],
    "thm_status_string": [ctypes.c_int],
    "thm_causal_conv1d_fwd": [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i32,
                              _c_i32, _c_i32, _c_i32, _c_vp],
    "thm_causal_conv1d_fwd_channels_last": [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,
                                            _c_i32, _c_i32, _c_i32, _c_i32, _c_vp],
    "thm_causal_conv1d_update": [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64,
                                 _c_i32, _c_i32, _c_i32, _c_i32, _c_vp],
    "thm_recompute_w_u_fwd": [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                              _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_vp],
    "thm_chunk_fwd_h": [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_vp],
    "thm_chunk_fwd_o": [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, ctypes.c_float,
                        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_vp],
    "thm_chunk_gated_delta_fwd": [_c_vp] * 9 + [ctypes.c_float] + [_c_i64] * 5 + [_c_i32, _c_i32, _c_vp],
    "thm_chunk_gated_delta_fwd_a": [_c_vp] * 10 + [ctypes.c_float] + [_c_i64] * 5 + [_c_i32, _c_i32, _c_vp],
    "thm_wy_build_A": [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64,
                       _c_i32, _c_i32, _c_i32, _c_vp],
    "thm_chunk_local_cumsum": [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_vp],
    "thm_wy_fwd": [_c_vp] * 6 + [_c_i64] * 5 + [_c_i32, _c_i32, _c_i32, _c_vp],
}
_RESTYPES = {"thm_status_string": ctypes.c_char_p}

_lib = None
_lock = threading.Lock()


def load_library(path: Path | str | None = None) -> ctypes.CDLL:
    """Load (once) and type the shared library; raise if it is absent or mismatched."""
    global _lib
    if path is None and _lib is not None:  # the per-call fast path: no lock once loaded
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"{p} is not built: run `python -m theorem_amd.build` (hipcc, gfx950). "
                "There is no CPU fallback for these kernels."
            )
        lib = ctypes.CDLL(str(p))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        got = lib.thm_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"{p}: ABI version {got}, expected {ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


_fast = None


def fastpath():
    """The host fast-path module of the wrappers (``theorem_amd/lib/_fastpath*.so``,
    built by theorem_amd.build: argument checks, output allocation and the C-ABI
    launch of a call in C++), or None when it is not built or does not load.
    Its functions return None for any call outside the common case; the
    wrappers then take their ctypes path to the same kernels.  A nonzero C
    status comes back as an int, which the wrappers raise (``fast_result``)."""
    global _fast
    if _fast is None:
        _fast = False
        try:
            import importlib.machinery
            import importlib.util

            from ..build import fastpath_path

            p = fastpath_path()
            if p.exists():
                load_library()  # the C-ABI library first: the module links against it by soname
                loader = importlib.machinery.ExtensionFileLoader("_fastpath", str(p))
                spec = importlib.util.spec_from_file_location("_fastpath", str(p), loader=loader)
                mod = importlib.util.module_from_spec(spec)
                loader.exec_module(mod)
                _fast = mod
        except (ImportError, OSError):
            _fast = False
    return _fast or None


def fast_result(r, what: str):
    """A fast-path function's result: None (take the Python path), an int
    (the C ABI's nonzero status: raised here, nothing is launched again) or
    the outputs."""
    if isinstance(r, int):
        check(r, what)
    return r


def status_string(status: int) -> str:
    return load_library().thm_status_string(int(status)).decode()


def check(status: int, what: str) -> None:
    if status == 0:
        return
    msg = f"{what}: {status_string(status)} (status {status})"
    if status < 0:
        raise ValueError(msg)
    raise RuntimeError(msg)


def dtype_code(t: torch.Tensor, what: str) -> int:
    code = THM_DTYPE.get(t.dtype)
    if code is None:
        raise AssertionError(f"{what}: dtype {t.dtype} not supported (float32 or bfloat16)")
    return code


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# torch's current-stream handle of a device.  The raw accessor returns the same
# hipStream_t as torch.cuda.current_stream(device).cuda_stream without building
# a Stream object (~0.1 against ~1.9 µs per call, which matters at the small
# task.yml shapes where the host side of a call is most of its latency).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def dev_ptrs(*ts: torch.Tensor | None) -> tuple[list, list | None]:
    """Device pointers of the given tensors (None stays None) for the C ABI.

    Every tensor must be on one GPU.  A tensor that is not dense row-major or
    not 16-byte aligned is copied first (the kernels use fixed 16-byte vector
    addressing); the copies are returned as the second item, to be kept alive
    until the launch has been enqueued.  This is the per-call host path of
    every wrapper, so it uses the cheapest tensor queries (is_cuda,
    get_device, is_contiguous, data_ptr: ~0.25 us per tensor)."""
    dev = -1
    out = []
    keep = None
    for t in ts:
        if t is None:
            out.append(None)
            continue
        if not t.is_cuda:
            raise AssertionError("all inputs must be on the MI355X device (torch 'cuda')")
        d = t.get_device()
        if dev < 0:
            dev = d
        elif d != dev:
            raise AssertionError(f"inputs on different devices: cuda:{dev} and cuda:{d}")
        if not t.is_contiguous():
            t = t.contiguous()
            keep = (keep or []) + [t]
        p = t.data_ptr()
        if p & 15:
            t = t.clone()
            keep = (keep or []) + [t]
            p = t.data_ptr()
        out.append(p)
    return out, keep


_devices: dict = {}


def device_of(t: torch.Tensor) -> torch.device:
    """t's torch.device, from a per-index cache (t.device builds a new object)."""
    i = t.get_device()
    d = _devices.get(i)
    if d is None:
        d = _devices[i] = t.device
    return d


def require_device(*ts: torch.Tensor | None) -> torch.device:
    """All given tensors must live on one GPU; return it."""
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise AssertionError("all inputs must be on the MI355X device (torch 'cuda')")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise AssertionError(f"inputs on different devices: {dev} and {t.device}")
    return dev


def prep(t: torch.Tensor | None, what: str) -> torch.Tensor | None:
    """Dense row-major and 16-byte aligned (a copy only when the input is not)."""
    if t is None:
        return None
    if not t.is_contiguous():
        t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def require_f32(t: torch.Tensor | None, what: str) -> None:
    if t is not None and t.dtype != torch.float32:
        raise AssertionError(f"{what} must be float32, got {t.dtype}")
