"""Lane-layout checks of the single gfx950 instructions the kernels are built on
(tests/csrc/probe.hip): MFMA operand/accumulator layouts, the LDS transpose
read, the DPP whole-wave shift, the fp32 -> bf16 conversion and the quad
transpose used before the 16-byte state stores."""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "_build" / "libthm_probe.so"


@pytest.fixture(scope="module")
def probe():
    assert LIB.exists(), "tests/_build/libthm_probe.so not built (run __graft_entry__.build())"
    return ctypes.CDLL(str(LIB))


def P(t):
    return ctypes.c_void_p(t.data_ptr())


def S():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ab(seed):
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(-4, 5, (64, 8), generator=g).to(torch.bfloat16)
    b = torch.randint(-4, 5, (64, 8), generator=g).to(torch.bfloat16)
    return a, b


def test_mfma_16x16x32_layout(probe, dev):
    a, b = _ab(1)
    c = torch.zeros(64, 4, device=dev)
    assert probe.probe_mfma_16x16x32_bf16(P(a.to(dev)), P(b.to(dev)), P(c), S()) == 0
    A = np.zeros((16, 32)); B = np.zeros((32, 16))
    for l in range(64):
        for i in range(8):
            A[l % 16, 8 * (l // 16) + i] = a[l, i]
            B[8 * (l // 16) + i, l % 16] = b[l, i]
    D = A @ B
    exp = np.array([[D[4 * (l // 16) + r, l % 16] for r in range(4)] for l in range(64)])
    assert np.array_equal(c.cpu().numpy(), exp)


def test_mfma_32x32x16_layout(probe, dev):
    a, b = _ab(2)
    c = torch.zeros(64, 16, device=dev)
    assert probe.probe_mfma_32x32x16_bf16(P(a.to(dev)), P(b.to(dev)), P(c), S()) == 0
    A = np.zeros((32, 16)); B = np.zeros((16, 32))
    for l in range(64):
        for i in range(8):
            A[l % 32, 8 * (l // 32) + i] = a[l, i]
            B[8 * (l // 32) + i, l % 32] = b[l, i]
    D = A @ B
    exp = np.array([[D[8 * (r // 4) + 4 * (l // 32) + r % 4, l % 32] for r in range(16)] for l in range(64)])
    assert np.array_equal(c.cpu().numpy(), exp)


@pytest.mark.parametrize("pattern", ["lin", "rows", "paired"])
def test_ds_read_tr16_b64(probe, dev, pattern):
    # LDS holds lds[i] = i.  Model: in each 16-lane group, output lane j element r
    # is element (j % 4) of the 8 bytes addressed by source lane 4r + j // 4.
    if pattern == "lin":
        adr = [4 * l for l in range(64)]
    elif pattern == "rows":   # row-major tile, pitch 32: natural-order fragment addressing
        adr = [((8 * (l // 16)) + (l % 16) // 4) * 32 + 4 * (l % 4) for l in range(64)]
    else:                     # pitch 24: paired-order addressing (second half)
        adr = [((4 * (l // 16)) + 16 + (l % 16) // 4) * 24 + 4 * (l % 4) for l in range(64)]
    assert max(adr) <= 1020  # the probe clamps addresses to its 1024-entry LDS array
    adr = [a - a % 4 for a in adr]
    ai = torch.tensor(adr, dtype=torch.int32, device=dev)
    out = torch.zeros(64, 4, dtype=torch.int16, device=dev)
    assert probe.probe_ds_read_tr16_b64(P(ai), P(out), S()) == 0
    exp = np.array([[adr[16 * (l // 16) + 4 * r + (l % 16) // 4] + (l % 16) % 4 for r in range(4)] for l in range(64)])
    assert np.array_equal(out.cpu().numpy().astype(np.int64), exp)


def test_dpp_wave_shr1(probe, dev):
    src = torch.arange(64, dtype=torch.int32, device=dev) + 100
    old = torch.arange(64, dtype=torch.int32, device=dev) + 1000
    out = torch.zeros(64, dtype=torch.int32, device=dev)
    assert probe.probe_dpp_wave_shr1(P(src), P(old), P(out), S()) == 0
    exp = np.concatenate([[1000], np.arange(63) + 100])
    assert np.array_equal(out.cpu().numpy(), exp)


def test_bf16_conversion_is_rne(probe, dev):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(4096, generator=g) * 3
    x[:8] = torch.tensor([1.0 + 2**-8, 1.0 + 3 * 2**-8, 1.0 + 2**-9, -1.0 - 2**-8, 65504.0, 1e-40,
                          float("inf"), float("nan")])
    y = torch.zeros(4096, dtype=torch.bfloat16, device=dev)
    assert probe.probe_cvt_bf16(P(x.to(dev)), P(y), 4096, S()) == 0
    ref = x.to(torch.bfloat16)
    yy = y.cpu()
    same = (yy.view(torch.int16) == ref.view(torch.int16)) | (torch.isnan(yy) & torch.isnan(ref))
    assert bool(same.all())


def test_quad_transpose(probe, dev):
    # Lane 4m + q holds row q of a 4x4 block in x[lane][0..3]; afterwards it
    # must hold column q: y[4m + q][i] = x[4m + i][q].
    x = (torch.arange(256, dtype=torch.float32).reshape(64, 4) * 1.5 - 7).to(dev)
    y = torch.empty_like(x)
    assert probe.probe_quad_transpose(P(x), P(y), S()) == 0
    torch.cuda.synchronize()
    xc, yc = x.cpu().numpy(), y.cpu().numpy()
    exp = np.empty_like(xc)
    for lane in range(64):
        for i in range(4):
            exp[lane, i] = xc[(lane & ~3) + i, lane & 3]
    np.testing.assert_array_equal(yc, exp)


def test_mfma_16x16x4_f32_layout(probe, dev):
    # v_mfma_f32_16x16x4_f32: lane l holds A[m = l % 16][k = l // 16] and
    # B[k = l // 16][n = l % 16]; the result D[m = 4 (l // 16) + r][n = l % 16]
    # lands in c[l][r].  Integer-valued inputs make the products exact.
    g = torch.Generator().manual_seed(5)
    A = torch.randint(-8, 9, (16, 4), generator=g).float()
    Bm = torch.randint(-8, 9, (4, 16), generator=g).float()
    lanes = torch.arange(64)
    a = A[lanes % 16, lanes // 16].contiguous().to(dev)
    b = Bm[lanes // 16, lanes % 16].contiguous().to(dev)
    c = torch.empty(64, 4, device=dev)
    assert probe.probe_mfma_16x16x4_f32(P(a), P(b), P(c), S()) == 0
    torch.cuda.synchronize()
    D = A @ Bm
    exp = torch.stack([D[4 * (lanes // 16) + r, lanes % 16] for r in range(4)], dim=1)
    assert torch.equal(c.cpu(), exp)
