"""GPU parity of the three Gated DeltaNet kernels (through the drop-in
custom_kernel wrappers) against the CPU oracle (float64).

Tolerances: rtol = atol = 1e-2 for bf16 inputs (the reference's task.yml
tolerance and BASELINE.json's bar); fp32 inputs are also held to 1e-3, since
their products run as bf16 hi/lo splits at ~2^-16 relative accuracy.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import deltanet as odn
from tests.helpers import assert_close
from theorem_amd import configs
from theorem_amd.kernels import chunk_fwd_h, chunk_fwd_o, recompute_w_u

pytestmark = pytest.mark.gpu

TASK_SHAPES = {
    "recompute_w_u": [(1, 64, 2, 64, 64, 4242), (2, 128, 4, 64, 64, 5236), (1, 256, 4, 64, 128, 1001)],
    "other": [(1, 64, 1, 64, 64, 4242), (2, 128, 4, 64, 64, 5236), (1, 256, 4, 64, 128, 1001)],
}
KV = [(64, 64), (64, 128), (128, 64), (128, 128)]


def np_(t):
    return None if t is None else t.detach().double().cpu().numpy()


def sync():
    torch.cuda.synchronize()


# --------------------------------------------------------------------------- recompute_w_u

@pytest.mark.parametrize("B,T,H,K,V,seed", TASK_SHAPES["recompute_w_u"])
def test_wu_task_shapes_fp32(dev, B, T, H, K, V, seed):
    data = recompute_w_u.generate_data(B, T, H, K, V, seed, device="cuda")
    w, u = recompute_w_u.custom_kernel(data)
    sync()
    assert w.dtype == torch.float32 and u.dtype == torch.float32
    ew, eu = odn.recompute_w_u_ref(*(np_(t) for t in (data.k, data.v, data.beta, data.A, data.g)))
    assert_close(w, ew, 1e-3, 1e-5, "w")
    assert_close(u, eu, 1e-3, 1e-5, "u")
    # The harness reference agrees too (dtype and values).
    rw, ru = recompute_w_u.ref_kernel(data)
    assert_close(w, rw, 1e-2, 1e-2, "w vs ref_kernel")


@pytest.mark.parametrize("K,V", KV)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_wu_config_inputs(dev, K, V, dtype):
    d = configs.make_wu_inputs(2, 512, 3, K, V, seed=1, device=dev, dtype=dtype)
    w, u = recompute_w_u.custom_kernel(recompute_w_u.Data(**d, B=2, T=512, H=3, K=K, V=V))
    sync()
    assert w.dtype == dtype
    ew, eu = odn.recompute_w_u_ref(*(np_(d[n]) for n in ("k", "v", "beta", "A", "g")))
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-3
    assert_close(w, ew, tol, tol, f"w K={K} V={V} {dtype}")
    assert_close(u, eu, tol, tol, f"u K={K} V={V} {dtype}")


def test_wu_identity_A_and_no_gate(dev):
    # A = I  =>  w = k beta e^g, u = v beta (closed form); g = None => e^g = 1.
    d = configs.make_wu_inputs(1, 128, 2, 64, 64, seed=2, device=dev, dtype=torch.float32)
    eye = torch.eye(64, device=dev).repeat(2, 1).reshape(1, 128, 1, 64).expand(1, 128, 2, 64).contiguous()
    w, u = recompute_w_u.custom_kernel(recompute_w_u.Data(d["k"], d["v"], d["beta"], eye, d["g"], 1, 128, 2, 64, 64))
    w0, u0 = recompute_w_u.custom_kernel(recompute_w_u.Data(d["k"], d["v"], d["beta"], eye, None, 1, 128, 2, 64, 64))
    sync()
    b = d["beta"].unsqueeze(-1)
    # fp32 operands run as bf16 hi/lo splits (~2^-16 relative per product).
    assert_close(w, d["k"] * b * torch.exp(d["g"]).unsqueeze(-1), 1e-4, 1e-6, "A=I w")
    assert_close(u, d["v"] * b, 1e-4, 1e-6, "A=I u")
    assert_close(w0, d["k"] * b, 1e-4, 1e-6, "A=I, g=None w")
    assert_close(u0, u, 0, 0, "u independent of g")


# --------------------------------------------------------------------------- chunk_fwd_o

@pytest.mark.parametrize("B,T,H,K,V,seed", TASK_SHAPES["other"])
def test_o_task_shapes_fp32(dev, B, T, H, K, V, seed):
    data = chunk_fwd_o.generate_input(B, T, H, K, V, seed, device="cuda")
    o = chunk_fwd_o.custom_kernel(data)
    sync()
    assert o.dtype == torch.float32 and o.shape == (B, T, H, V)
    e = odn.chunk_fwd_o_ref(*(np_(data[n]) for n in ("q", "k", "v", "g", "h")), data["scale"])
    assert_close(o, e, 1e-3, 1e-3, "o")
    assert_close(o, chunk_fwd_o.ref_kernel(data), 1e-2, 1e-2, "o vs ref_kernel")


@pytest.mark.parametrize("K,V", KV)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("gate", ["logsigmoid", "mild"])
def test_o_config_inputs(dev, K, V, dtype, gate):
    d = configs.make_o_inputs(2, 512, 3, K, V, seed=3, device=dev, dtype=dtype, gate=gate)
    o = chunk_fwd_o.custom_kernel(d)
    sync()
    assert o.dtype == dtype
    e = odn.chunk_fwd_o_diff(*(np_(d[n]) for n in ("q", "k", "v", "g", "h")), d["scale"])
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-3
    assert_close(o, e, tol, tol, f"o K={K} V={V} {dtype} {gate}")


# bf16 grids with at least 2 tiles per persistent workgroup (2 per CU) run the
# software-pipelined kernel; these shapes (1024+ tiles) force it at every K, V.
@pytest.mark.parametrize("K,V", KV)
@pytest.mark.parametrize("gate", ["logsigmoid", None])
def test_o_pipelined_path(dev, K, V, gate):
    B, T, H = 2, 2048, 17
    d = configs.make_o_inputs(B, T, H, K, V, seed=13, device=dev, dtype=torch.bfloat16, gate=gate or "zero")
    g = d["g"] if gate else None
    o = chunk_fwd_o.custom_kernel(dict(q=d["q"], k=d["k"], v=d["v"], g=g, h=d["h"], scale=d["scale"]))
    sync()
    e = odn.chunk_fwd_o_diff(np_(d["q"]), np_(d["k"]), np_(d["v"]), np_(g) if g is not None else None,
                             np_(d["h"]), d["scale"])
    assert_close(o, e, 1e-2, 1e-2, f"o K={K} V={V} gate={gate}")


def test_o_pipelined_handout_across_launches_and_streams(dev):
    # The pipelined kernel hands out its tiles at run time from a counter slot
    # that the launch's last workgroup resets; the slots rotate per launch.
    # 300 launches in a row (more than the 256 slots, so every slot is reused
    # after its reset) and launches alternating between two streams with no
    # synchronisation between them must all give the first launch's output bit
    # for bit, and that output must match the oracle.
    K = V = 64
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    B, H = 1, 32
    T = 64 * max(2, -(-6 * cus // H))  # 3 tiles per persistent workgroup (2 per CU)
    d = configs.make_o_inputs(B, T, H, K, V, seed=21, device=dev, dtype=torch.bfloat16)
    args = dict(q=d["q"], k=d["k"], v=d["v"], g=d["g"], h=d["h"], scale=d["scale"])
    o0 = chunk_fwd_o.custom_kernel(args)
    sync()
    e = odn.chunk_fwd_o_diff(np_(d["q"]), np_(d["k"]), np_(d["v"]), np_(d["g"]), np_(d["h"]), d["scale"])
    assert_close(o0, e, 1e-2, 1e-2, "o pipelined")
    outs = [chunk_fwd_o.custom_kernel(args) for _ in range(300)]
    sync()
    bad = [i for i, o in enumerate(outs) if not torch.equal(o, o0)]
    assert not bad, f"launches {bad[:8]} differ from the first"
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    cur = torch.cuda.current_stream()
    for s in streams:
        s.wait_stream(cur)
    outs = []
    for i in range(16):
        with torch.cuda.stream(streams[i % 2]):
            outs.append(chunk_fwd_o.custom_kernel(args))
    sync()
    bad = [i for i, o in enumerate(outs) if not torch.equal(o, o0)]
    assert not bad, f"two-stream launches {bad} differ from the first"
    # A smaller pipelined shape right after (2 tiles per workgroup instead of 3,
    # the same slots).
    H2 = H // 2
    T2 = 64 * max(2, -(-4 * cus // H2))
    assert B * (T2 // 64) * H2 < B * (T // 64) * H
    d2 = configs.make_o_inputs(B, T2, H2, K, V, seed=22, device=dev, dtype=torch.bfloat16)
    o2 = chunk_fwd_o.custom_kernel(dict(q=d2["q"], k=d2["k"], v=d2["v"], g=d2["g"], h=d2["h"], scale=d2["scale"]))
    sync()
    e2 = odn.chunk_fwd_o_diff(np_(d2["q"]), np_(d2["k"]), np_(d2["v"]), np_(d2["g"]), np_(d2["h"]), d2["scale"])
    assert_close(o2, e2, 1e-2, 1e-2, "o pipelined, smaller shape after")


def test_o_closed_forms(dev):
    d = configs.make_o_inputs(1, 128, 2, 64, 64, seed=4, device=dev, dtype=torch.float32)
    q, k, v, h = d["q"], d["k"], d["v"], d["h"]
    # h = 0, g = None: o = scale tril_incl(q k^T) v per chunk.
    o = chunk_fwd_o.custom_kernel(dict(q=q, k=k, v=v, g=None, h=torch.zeros_like(h), scale=0.5))
    # v = 0: o = scale e^g q h[c].
    o2 = chunk_fwd_o.custom_kernel(dict(q=q, k=k, v=torch.zeros_like(v), g=d["g"], h=h, scale=0.5))
    sync()
    qc = q.double().reshape(1, 2, 64, 2, 64).permute(0, 1, 3, 2, 4)
    kc = k.double().reshape(1, 2, 64, 2, 64).permute(0, 1, 3, 2, 4)
    vc = v.double().reshape(1, 2, 64, 2, 64).permute(0, 1, 3, 2, 4)
    e = 0.5 * (torch.tril(qc @ kc.transpose(-1, -2)) @ vc)
    assert_close(o, e.permute(0, 1, 3, 2, 4).reshape(1, 128, 2, 64), 1e-4, 1e-4, "h=0,g=0")
    gc = d["g"].double().reshape(1, 2, 64, 2).permute(0, 1, 3, 2)
    e2 = 0.5 * (qc * torch.exp(gc).unsqueeze(-1)) @ h.double()
    assert_close(o2, e2.permute(0, 1, 3, 2, 4).reshape(1, 128, 2, 64), 1e-4, 1e-4, "v=0")


# --------------------------------------------------------------------------- chunk_fwd_h

@pytest.mark.parametrize("B,T,H,K,V,seed", TASK_SHAPES["other"])
def test_h_task_shapes_fp32(dev, B, T, H, K, V, seed):
    data = chunk_fwd_h.generate_input(B, T, H, K, V, seed, device="cuda:0")
    h = chunk_fwd_h.custom_kernel(data)
    sync()
    assert h.dtype == torch.float32 and h.shape == (B, T // 64, H, K, V)
    e = odn.chunk_fwd_h_ref(np_(data["k"]), np_(data["v"]), np_(data["g"]))
    assert_close(h, e, 1e-3, 1e-3, "h")
    assert_close(h, chunk_fwd_h.ref_kernel(data), 1e-2, 1e-2, "h vs ref_kernel")


@pytest.mark.parametrize("K,V", KV)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("gate", ["logsigmoid", "mild", "zero"])
def test_h_delta_config_inputs(dev, K, V, dtype, gate):
    T = 1024 if gate != "zero" else 256
    d = configs.make_h_inputs(2, T, 3, K, V, seed=5, device=dev, dtype=dtype, gate=gate, h0_std=0.1)
    h, vn, ht = chunk_fwd_h.custom_kernel(dict(k=d["k"], w=d["w"], u=d["u"], g=d["g"],
                                               initial_state=d["h0"], output_final_state=True))
    sync()
    assert h.dtype == torch.float32 and vn.dtype == dtype and ht.dtype == torch.float32
    eh, evn, eht = odn.chunk_fwd_h_delta(np_(d["k"]), np_(d["w"]), np_(d["u"]), np_(d["g"]), h0=np_(d["h0"]))
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-3
    assert_close(h, eh, tol, tol, f"h K={K} V={V} {dtype} {gate}")
    assert_close(vn, evn, tol, tol, f"v_new K={K} V={V} {dtype} {gate}")
    assert_close(ht, eht, tol, tol, f"final K={K} V={V} {dtype} {gate}")


def test_h_delta_cfg3_zero_state(dev):
    # BASELINE config 3 exactly: B=2, T=1024, H=3, K=V=64, bf16, zero initial state.
    d = configs.make_h_inputs(2, 1024, 3, 64, 64, seed=0, device=dev)
    h, vn, ht = chunk_fwd_h.custom_kernel(dict(k=d["k"], w=d["w"], u=d["u"], g=d["g"], output_final_state=True))
    sync()
    eh, evn, eht = odn.chunk_fwd_h_delta(np_(d["k"]), np_(d["w"]), np_(d["u"]), np_(d["g"]))
    assert np.abs(np_(h[:, 0])).max() == 0.0  # h[0] is the (zero) initial state
    assert_close(h, eh, 1e-2, 1e-2, "h")
    assert_close(vn, evn, 1e-2, 1e-2, "v_new")
    assert_close(ht, eht, 1e-2, 1e-2, "final")


def test_h_reference_form_extras(dev):
    # Reference form with initial / final state; w = 0 in the delta form gives the
    # same states shifted by one chunk (pre- vs post-update storage).
    d = configs.make_h_inputs(1, 256, 2, 64, 64, seed=6, device=dev, dtype=torch.float32, gate="mild", h0_std=0.2)
    h_ref, ht_ref = chunk_fwd_h.custom_kernel(dict(k=d["k"], v=d["u"], g=d["g"], initial_state=d["h0"],
                                                   output_final_state=True))
    h_del, vn, ht_del = chunk_fwd_h.custom_kernel(dict(k=d["k"], w=torch.zeros_like(d["w"]), u=d["u"], g=d["g"],
                                                       initial_state=d["h0"], output_final_state=True))
    sync()
    assert_close(h_del[:, 1:], h_ref[:, :-1], 1e-5, 1e-5, "shifted states")
    assert_close(h_del[:, 0], d["h0"], 0, 0, "h[0] = h0")
    assert_close(ht_del, ht_ref, 1e-5, 1e-5, "final states")
    assert_close(vn, d["u"], 0, 0, "v_new = u when w = 0")
    assert_close(ht_ref, h_ref[:, -1], 0, 0, "final = last post-update state")


@pytest.mark.parametrize("K,V", KV)
@pytest.mark.parametrize("gate", ["logsigmoid", None])
def test_h_reference_form_bf16(dev, K, V, gate):
    # bf16 reference form (v used as is, h stored after each chunk), with an
    # initial and a final state; NT = 5 exercises a ring of stages that does
    # not divide the chunk count.
    d = configs.make_h_inputs(2, 320, 3, K, V, seed=8, device=dev, dtype=torch.bfloat16,
                              gate=gate or "zero", h0_std=0.1)
    g = d["g"] if gate else None
    h, ht = chunk_fwd_h.custom_kernel(dict(k=d["k"], v=d["u"], g=g, initial_state=d["h0"],
                                           output_final_state=True))
    sync()
    gk = np_(g) if g is not None else None
    # With an initial state the reference form is the delta form with w = 0,
    # stored one chunk later (after instead of before each chunk's update).
    eh_pre, _, eht = odn.chunk_fwd_h_delta(np_(d["k"]), np.zeros_like(np_(d["w"])), np_(d["u"]), gk,
                                           h0=np_(d["h0"]))
    eh_post = np.concatenate([eh_pre[:, 1:], eht[:, None]], axis=1)
    assert_close(h, eh_post, 1e-2, 1e-2, f"h K={K} V={V} gate={gate}")
    assert_close(ht, eht, 1e-2, 1e-2, f"final K={K} V={V} gate={gate}")
    # Without one it is the oracle's reference form directly.
    h_z = chunk_fwd_h.custom_kernel(dict(k=d["k"], v=d["u"], g=g))
    sync()
    g0 = gk if gk is not None else np.zeros(d["k"].shape[:3])
    assert_close(h_z, odn.chunk_fwd_h_ref(np_(d["k"]), np_(d["u"]), g0), 1e-2, 1e-2, f"h0=0 K={K} V={V}")


@pytest.mark.parametrize("K,V", [(64, 64), (128, 128)])
def test_h_delta_bf16_without_v_new_and_gate(dev, K, V):
    # save_new_value=False (no v_new output) and no gate; single chunk and odd chunk counts.
    for T in (64, 192):
        d = configs.make_h_inputs(1, T, 2, K, V, seed=9, device=dev, dtype=torch.bfloat16, h0_std=0.1)
        h, vn, ht = chunk_fwd_h.custom_kernel(dict(k=d["k"], w=d["w"], u=d["u"], g=None, initial_state=d["h0"],
                                                   output_final_state=True, save_new_value=False))
        sync()
        assert vn is None
        eh, _, eht = odn.chunk_fwd_h_delta(np_(d["k"]), np_(d["w"]), np_(d["u"]), None, h0=np_(d["h0"]))
        assert_close(h, eh, 1e-2, 1e-2, f"h K={K} V={V} T={T}")
        assert_close(ht, eht, 1e-2, 1e-2, f"final K={K} V={V} T={T}")


# bf16 grids of at least 256 workgroups (B * H * V / 64) run the DMA pipeline
# kernel; smaller ones the register-prefetch kernel.  These shapes force the
# former at every K, V and flag combination.
@pytest.mark.parametrize("K,V", KV)
@pytest.mark.parametrize("form", ["delta", "delta_plain", "reference", "reference_plain"])
def test_h_dma_pipeline_forms(dev, K, V, form):
    B, H = 4, (64 if V == 64 else 32)
    assert B * H * (V // 64) >= 256
    for T in (192, 64):
        d = configs.make_h_inputs(B, T, H, K, V, seed=10, device=dev, dtype=torch.bfloat16, h0_std=0.1)
        plain = form.endswith("plain")
        g = None if plain else d["g"]
        h0 = None if plain else d["h0"]
        gk = np_(g) if g is not None else None
        h0k = np_(h0) if h0 is not None else None
        if form.startswith("delta"):
            h, vn, ht = chunk_fwd_h.custom_kernel(dict(k=d["k"], w=d["w"], u=d["u"], g=g, initial_state=h0,
                                                       output_final_state=True, save_new_value=not plain))
            sync()
            eh, evn, eht = odn.chunk_fwd_h_delta(np_(d["k"]), np_(d["w"]), np_(d["u"]), gk, h0=h0k)
            if not plain:
                assert_close(vn, evn, 1e-2, 1e-2, f"v_new {form} K={K} V={V} T={T}")
            else:
                assert vn is None
        else:
            h, ht = chunk_fwd_h.custom_kernel(dict(k=d["k"], v=d["u"], g=g, initial_state=h0,
                                                   output_final_state=True))
            sync()
            pre, _, eht = odn.chunk_fwd_h_delta(np_(d["k"]), np.zeros_like(np_(d["w"])), np_(d["u"]), gk, h0=h0k)
            eh = np.concatenate([pre[:, 1:], eht[:, None]], axis=1)
        assert_close(h, eh, 1e-2, 1e-2, f"h {form} K={K} V={V} T={T}")
        assert_close(ht, eht, 1e-2, 1e-2, f"final {form} K={K} V={V} T={T}")


# fp32 grids of at least 256 workgroups run the register kernel with its
# two-chunks-ahead prefetch (two register sets); T = 64 * (1, 2, 3, 4) covers
# the odd / even chunk counts of its two-chunk loop.
@pytest.mark.parametrize("K,V", KV)
@pytest.mark.parametrize("form", ["delta", "reference_plain"])
def test_h_fp32_deep_prefetch(dev, K, V, form):
    B, H = 4, (64 if V == 64 else 32)
    assert B * H * (V // 64) >= 256
    for T in (64, 128, 192, 256):
        d = configs.make_h_inputs(B, T, H, K, V, seed=13, device=dev, dtype=torch.float32, h0_std=0.1)
        plain = form.endswith("plain")
        g = None if plain else d["g"]
        h0 = None if plain else d["h0"]
        gk = np_(g) if g is not None else None
        h0k = np_(h0) if h0 is not None else None
        if form == "delta":
            h, vn, ht = chunk_fwd_h.custom_kernel(dict(k=d["k"], w=d["w"], u=d["u"], g=g, initial_state=h0,
                                                       output_final_state=True))
            sync()
            eh, evn, eht = odn.chunk_fwd_h_delta(np_(d["k"]), np_(d["w"]), np_(d["u"]), gk, h0=h0k)
            assert_close(vn, evn, 1e-3, 1e-3, f"v_new fp32 K={K} V={V} T={T}")
        else:
            h, ht = chunk_fwd_h.custom_kernel(dict(k=d["k"], v=d["u"], g=g, initial_state=h0,
                                                   output_final_state=True))
            sync()
            pre, _, eht = odn.chunk_fwd_h_delta(np_(d["k"]), np.zeros_like(np_(d["w"])), np_(d["u"]), gk, h0=h0k)
            eh = np.concatenate([pre[:, 1:], eht[:, None]], axis=1)
        assert_close(h, eh, 1e-3, 1e-3, f"h fp32 {form} K={K} V={V} T={T}")
        assert_close(ht, eht, 1e-3, 1e-3, f"final fp32 {form} K={K} V={V} T={T}")


# fp32 grids under 256 workgroups run the role-split small-grid kernel where
# its stages fit in LDS (all but K = 128 in the delta form).  The reference
# form at every K, V, with and without gates and initial state;
# T = 64 * (1 .. 5) covers the odd / even chunk counts of its memory waves'
# two-chunk loop and the one-chunk case.
@pytest.mark.parametrize("K,V", KV)
@pytest.mark.parametrize("form", ["reference", "reference_plain"])
def test_h_fp32_small_grid_reference_form(dev, K, V, form):
    B, H = 2, 3
    assert B * H * (V // 64) < 256
    for T in (64, 128, 192, 256, 320):
        d = configs.make_h_inputs(B, T, H, K, V, seed=14, device=dev, dtype=torch.float32, h0_std=0.1)
        plain = form.endswith("plain")
        g = None if plain else d["g"]
        h0 = None if plain else d["h0"]
        gk = np_(g) if g is not None else None
        h0k = np_(h0) if h0 is not None else None
        h, ht = chunk_fwd_h.custom_kernel(dict(k=d["k"], v=d["u"], g=g, initial_state=h0, output_final_state=True))
        sync()
        pre, _, eht = odn.chunk_fwd_h_delta(np_(d["k"]), np.zeros_like(np_(d["w"])), np_(d["u"]), gk, h0=h0k)
        eh = np.concatenate([pre[:, 1:], eht[:, None]], axis=1)
        assert_close(h, eh, 1e-4, 1e-4, f"h fp32 {form} K={K} V={V} T={T}")
        assert_close(ht, eht, 1e-4, 1e-4, f"final fp32 {form} K={K} V={V} T={T}")


def test_h_dma_pipeline_unaligned_head_count_and_empty(dev):
    # B * H not a multiple of 8 (the plain block mapping) and T = 0 on the DMA path.
    B, T, H, K, V = 1, 128, 260, 64, 64
    d = configs.make_h_inputs(B, T, H, K, V, seed=12, device=dev, dtype=torch.bfloat16, h0_std=0.1)
    h, vn, ht = chunk_fwd_h.custom_kernel(dict(k=d["k"], w=d["w"], u=d["u"], g=d["g"], initial_state=d["h0"],
                                               output_final_state=True))
    sync()
    eh, evn, eht = odn.chunk_fwd_h_delta(np_(d["k"]), np_(d["w"]), np_(d["u"]), np_(d["g"]), h0=np_(d["h0"]))
    assert_close(h, eh, 1e-2, 1e-2, "h")
    assert_close(vn, evn, 1e-2, 1e-2, "v_new")
    assert_close(ht, eht, 1e-2, 1e-2, "final")
    k0 = torch.empty(B, 0, H, K, device=dev, dtype=torch.bfloat16)
    h, vn, ht = chunk_fwd_h.custom_kernel(dict(k=k0, w=k0, u=torch.empty(B, 0, H, V, device=dev, dtype=torch.bfloat16),
                                               g=None, initial_state=d["h0"], output_final_state=True))
    sync()
    assert h.shape == (B, 0, H, K, V)
    assert_close(ht, d["h0"], 0, 0, "T=0 final state")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_h_empty_sequence_final_state(dev, dtype):
    k = torch.empty(1, 0, 2, 64, device=dev, dtype=dtype)
    h0 = torch.randn(1, 2, 64, 64, device=dev)
    h, ht = chunk_fwd_h.custom_kernel(dict(k=k, v=torch.empty(1, 0, 2, 64, device=dev, dtype=dtype), g=None,
                                           initial_state=h0, output_final_state=True))
    sync()
    assert h.shape == (1, 0, 2, 64, 64)
    assert_close(ht, h0, 0, 0, "T=0 final state")


# --------------------------------------------------------------------------- full chain

@pytest.mark.parametrize("K,V", [(64, 64), (128, 128)])
@pytest.mark.parametrize("gate", ["logsigmoid", "mild"])
def test_chain_matches_token_recurrence(dev, K, V, gate):
    from theorem_amd.chain import chunk_gated_delta_rule_fwd
    gen = torch.Generator().manual_seed(11)
    B, T, H = 1, 256, 2
    q = configs.l2norm(torch.randn(B, T, H, K, generator=gen)).to(torch.bfloat16)
    k = configs.l2norm(torch.randn(B, T, H, K, generator=gen)).to(torch.bfloat16)
    v = torch.randn(B, T, H, V, generator=gen).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    if gate == "logsigmoid":
        a = torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=gen))
    else:
        a = -0.05 * torch.rand(B, T, H, generator=gen) - 0.005
    g = configs.chunk_local_cumsum(a)
    scale = K ** -0.5
    o, ht = chunk_gated_delta_rule_fwd(q.to(dev), k.to(dev), v.to(dev), beta.to(dev), g.to(dev), scale,
                                       output_final_state=True)
    sync()
    eo, eS = odn.gated_delta_rule_tokens(np_(q), np_(k), np_(v), np_(beta), np_(a), scale)
    assert_close(o, eo, 1e-2, 1e-2, f"chain o {gate}")
    assert_close(ht, eS, 1e-2, 1e-2, f"chain final state {gate}")


# --------------------------------------------------------------------------- strided and offset views

def _strided(t):
    """A non-contiguous view holding t's values: every other element along the
    last dimension of a tensor twice as wide."""
    wide = torch.zeros(*t.shape[:-1], 2 * t.shape[-1], dtype=t.dtype, device=t.device)
    wide[..., ::2] = t
    return wide[..., ::2]


def _offset(t):
    """A contiguous view holding t's values whose data pointer sits 4 bytes past
    a 16-byte boundary."""
    n, e = t.numel(), 4 // t.element_size()
    flat = torch.zeros(n + 16, dtype=t.dtype, device=t.device)
    assert flat.data_ptr() % 16 == 0
    flat[e:e + n] = t.reshape(-1)
    return flat[e:e + n].view(t.shape)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("view", [_strided, _offset])
def test_wrappers_take_strided_and_offset_views(dev, dtype, view):
    """The three wrappers accept non-contiguous and misaligned inputs (copied to
    dense 16-byte aligned tensors before the C ABI call) and return exactly
    what the dense inputs give."""
    d = configs.make_wu_inputs(1, 128, 2, 64, 64, seed=3, device=dev, dtype=dtype)
    vw = {n: view(t) for n, t in d.items()}
    assert not vw["k"].is_contiguous() or vw["k"].data_ptr() % 16
    ref = recompute_w_u.custom_kernel(recompute_w_u.Data(**d, B=1, T=128, H=2, K=64, V=64))
    got = recompute_w_u.custom_kernel(recompute_w_u.Data(**vw, B=1, T=128, H=2, K=64, V=64))
    sync()
    assert all(torch.equal(a, b) for a, b in zip(ref, got)), "recompute_w_u"

    d = configs.make_o_inputs(1, 128, 2, 64, 128, seed=4, device=dev, dtype=dtype)
    ref = chunk_fwd_o.custom_kernel(d)
    got = chunk_fwd_o.custom_kernel({**{n: view(d[n]) for n in ("q", "k", "v", "g", "h")}, "scale": d["scale"]})
    sync()
    assert torch.equal(ref, got), "chunk_fwd_o"

    d = configs.make_h_inputs(1, 256, 2, 64, 64, seed=5, device=dev, dtype=dtype, h0_std=0.1)
    keys = dict(k="k", w="w", u="u", g="g", initial_state="h0")
    ref = chunk_fwd_h.custom_kernel({**{a: d[b] for a, b in keys.items()}, "output_final_state": True})
    got = chunk_fwd_h.custom_kernel({**{a: view(d[b]) for a, b in keys.items()}, "output_final_state": True})
    sync()
    assert all(torch.equal(a, b) for a, b in zip(ref, got)), "chunk_fwd_h"
