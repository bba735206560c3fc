"""The C++ host fast path of the four custom_kernel wrappers
(theorem_amd/csrc/host/fastpath.cpp) against their ctypes path: the same
kernels, so every output must be bit-identical; calls outside the fast path's
common case (a non-contiguous input, an unsupported option) must fall back to
the ctypes path and give the same result; and the module must be built and
loaded, so that the fast path is the one the bench and the harness time."""
from __future__ import annotations

import pytest
import torch

from theorem_amd import configs
from theorem_amd.kernels import _capi, causal_conv1d, chunk_fwd_h, chunk_fwd_o, recompute_w_u

pytestmark = pytest.mark.gpu


def _both(fn):
    """fn() through the fast path, then through the ctypes path."""
    assert _capi.fastpath() is not None, "the fast-path module is not built or does not load"
    fast = fn()
    saved = _capi._fast
    _capi._fast = False
    try:
        slow = fn()
    finally:
        _capi._fast = saved
    return fast, slow


def _equal(a, b):
    if isinstance(a, tuple):
        assert isinstance(b, tuple) and len(a) == len(b)
        for x, y in zip(a, b):
            _equal(x, y)
    elif a is None:
        assert b is None
    else:
        assert a.dtype == b.dtype and a.shape == b.shape and torch.equal(a, b)


def test_fastpath_loaded(dev):
    fp = _capi.fastpath()
    assert fp is not None and all(hasattr(fp, n) for n in ("conv1d", "wu", "h", "o"))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("act", [None, "silu"])
def test_conv_fast_equals_ctypes(dev, dtype, act):
    x, w, b = configs.make_conv_inputs(2, 96, 200, 4, dtype=dtype, seed=1, device=dev)
    _equal(*_both(lambda: causal_conv1d.custom_kernel((x, w, b), activation=act)))
    _equal(*_both(lambda: causal_conv1d.custom_kernel((x, w, None), activation=act)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_wu_fast_equals_ctypes(dev, dtype):
    d = configs.make_wu_inputs(2, 256, 3, 64, 128, seed=2, device=dev, dtype=dtype)
    data = recompute_w_u.Data(**d, B=2, T=256, H=3, K=64, V=128)
    _equal(*_both(lambda: recompute_w_u.custom_kernel(data)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("form", ["delta", "reference"])
def test_h_fast_equals_ctypes(dev, dtype, form):
    d = configs.make_h_inputs(2, 320, 3, 64, 64, seed=3, device=dev, dtype=dtype, gate="mild", h0_std=0.1)
    if form == "delta":
        for extra in ({}, {"initial_state": d["h0"], "output_final_state": True},
                      {"save_new_value": False, "output_final_state": True}):
            data = dict(k=d["k"], w=d["w"], u=d["u"], g=d["g"], **extra)
            _equal(*_both(lambda: chunk_fwd_h.custom_kernel(data)))
    else:
        for extra in ({}, {"output_final_state": True}):
            data = dict(k=d["k"], v=d["u"], g=d["g"], **extra)
            _equal(*_both(lambda: chunk_fwd_h.custom_kernel(data)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_o_fast_equals_ctypes(dev, dtype):
    d = configs.make_o_inputs(2, 256, 3, 64, 128, seed=4, device=dev, dtype=dtype)
    data = dict(q=d["q"], k=d["k"], v=d["v"], g=d["g"], h=d["h"], scale=d["scale"])
    _equal(*_both(lambda: chunk_fwd_o.custom_kernel(data)))
    data["g"] = None
    _equal(*_both(lambda: chunk_fwd_o.custom_kernel(data)))


def test_fastpath_declines_outside_common_case(dev):
    """A strided input and a wrong dtype: the fast path returns None (the
    wrapper then copies the input, or raises the reference's error)."""
    fp = _capi.fastpath()
    d = configs.make_o_inputs(1, 128, 2, 64, 64, seed=5, device=dev)
    q_strided = torch.empty(1, 128, 2, 128, dtype=d["q"].dtype, device=dev)[..., :64]
    q_strided.copy_(d["q"])
    assert fp.o(q_strided, d["k"], d["v"], d["g"], d["h"], d["scale"]) is None
    data = dict(q=q_strided, k=d["k"], v=d["v"], g=d["g"], h=d["h"], scale=d["scale"])
    ref = chunk_fwd_o.custom_kernel(dict(data, q=d["q"]))
    assert torch.equal(chunk_fwd_o.custom_kernel(data), ref)
    assert fp.o(d["q"], d["k"], d["v"], d["g"], d["h"].half(), d["scale"]) is None
    with pytest.raises(AssertionError):
        chunk_fwd_o.custom_kernel(dict(data, h=d["h"].half()))
    x, w, b = configs.make_conv_inputs(1, 64, 100, 4, seed=6, device=dev)
    assert fp.conv1d(x.transpose(1, 2).contiguous().transpose(1, 2), w, b, 0) is None


def test_fastpath_raises_host_rejection_once(dev, monkeypatch):
    """An argument the fast path's checks pass but the C ABI rejects on the
    host (an unsupported K or W): the C status comes back from the fast path
    and the wrapper raises ValueError at once, without entering its ctypes
    path (which would validate and call the C ABI a second time)."""
    assert _capi.fastpath() is not None

    def no_ctypes_path(*a, **k):
        raise AssertionError("the ctypes path ran after the fast path's status")

    monkeypatch.setattr(_capi, "dev_ptrs", no_ctypes_path)
    monkeypatch.setattr(_capi, "require_device", no_ctypes_path)
    d = configs.make_o_inputs(1, 128, 2, 64, 64, seed=7, device=dev)
    q = d["q"][..., :32].contiguous()
    k = d["k"][..., :32].contiguous()
    h = d["h"][:, :, :, :32].contiguous()
    with pytest.raises(ValueError, match="thm_chunk_fwd_o"):
        chunk_fwd_o.custom_kernel(dict(q=q, k=k, v=d["v"], g=d["g"], h=h, scale=d["scale"]))
    with pytest.raises(ValueError, match="thm_chunk_fwd_h"):
        chunk_fwd_h.custom_kernel(dict(k=k, v=d["v"], g=d["g"]))
    wd = configs.make_wu_inputs(1, 128, 2, 64, 64, seed=8, device=dev)
    with pytest.raises(ValueError, match="thm_recompute_w_u_fwd"):
        recompute_w_u.custom_kernel(recompute_w_u.Data(**dict(wd, k=wd["k"][..., :32].contiguous()),
                                                       B=1, T=128, H=2, K=32, V=64))
    x, w, b = configs.make_conv_inputs(1, 64, 100, 4, seed=9, device=dev)
    w9 = torch.zeros(64, 9, dtype=w.dtype, device=dev)
    with pytest.raises(ValueError, match="thm_causal_conv1d_fwd"):
        causal_conv1d.custom_kernel((x, w9, b))
