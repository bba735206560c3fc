"""chunk_fwd_o's persistent kernel and its run-time tile hand-out under HIP
graph capture and with many launches in flight on several streams.

The pipelined bf16 kernel (csrc/chunk_fwd_o.hip, grids of >= 2 workgroups per
CU over at least twice as many tiles) hands tiles out at run time from
counters in a static device array (csrc/handout.h).  The reference's launcher
is stateless (kernels/chunk_fwd_o/kernel.py:183-187), so this build must be
too, observably:
  * a launch captured into a graph takes the fixed walk and holds no state:
    its replays, repeated, interleaved with eager launches and run on two
    streams at once, all give the eager output bit for bit (the tile order
    does not change the arithmetic of a tile), which matches the oracle;
  * eager launches queued far beyond the slot count on two streams never
    share a slot (each slot's previous launch must have completed first), so
    every one of them gives the same output.
The captured region allocates its output from the graph's pool and launches
one kernel; it records no memset.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import deltanet as odn
from theorem_amd import configs
from theorem_amd.kernels import chunk_fwd_o

from tests.helpers import assert_close

pytestmark = pytest.mark.gpu

# 2 x 64 chunks x 8 heads = 1024 tiles: at least 2 x (2 workgroups per CU x 256
# CUs), so the pipelined kernel with the hand-out runs.
SHAPE = dict(B=2, T=4096, H=8, K=64, V=64)


def _inputs(dev, seed):
    d = configs.make_o_inputs(**SHAPE, seed=seed, device=dev)
    return dict(q=d["q"], k=d["k"], v=d["v"], g=d["g"], h=d["h"], scale=d["scale"])


def _pipelined(dev) -> bool:
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    tiles = SHAPE["B"] * (SHAPE["T"] // 64) * SHAPE["H"]
    return tiles >= 2 * 2 * cus


def test_o_graph_capture_replays(dev):
    assert _pipelined(dev), "the test shape no longer selects the pipelined kernel"
    data = _inputs(dev, seed=21)
    eager = chunk_fwd_o.custom_kernel(data)
    torch.cuda.synchronize()
    print("capture: eager output computed", flush=True)
    exp = odn.chunk_fwd_o_diff(*(data[n].float().cpu().numpy() for n in ("q", "k", "v", "g", "h")), data["scale"])
    assert_close(eager, exp, 1e-2, 1e-2, "eager chunk_fwd_o")

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on a side stream before capture
        chunk_fwd_o.custom_kernel(data)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graphs, outs = [], []
    for _ in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs.append(chunk_fwd_o.custom_kernel(data))
        graphs.append(g)
    torch.cuda.synchronize()
    print("capture: two graphs captured", flush=True)

    # Replays one after another, each after the output was overwritten, with
    # eager launches (which use the hand-out slots) between them.
    for r in range(4):
        outs[0].fill_(float("nan"))
        torch.cuda.synchronize()
        graphs[0].replay()
        extra = chunk_fwd_o.custom_kernel(data)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], eager), f"replay {r} differs from the eager output"
        assert torch.equal(extra, eager), f"eager launch after replay {r} differs"

    # Concurrent: graph 0 on two streams at once (both write the same values
    # into its one output), graph 1 and eager launches on a third stream.
    s1, s2, s3 = torch.cuda.Stream(), torch.cuda.Stream(), torch.cuda.Stream()
    for s in (s1, s2, s3):
        s.wait_stream(torch.cuda.current_stream())
    outs[0].fill_(float("nan"))
    outs[1].fill_(float("nan"))
    torch.cuda.synchronize()
    eagers = []
    for _ in range(3):
        with torch.cuda.stream(s1):
            graphs[0].replay()
        with torch.cuda.stream(s2):
            graphs[0].replay()
            graphs[1].replay()
        with torch.cuda.stream(s3):
            eagers.append(chunk_fwd_o.custom_kernel(data))
    torch.cuda.synchronize()
    print("capture: concurrent replays done", flush=True)
    assert torch.equal(outs[0], eager), "graph 0 replayed on two streams differs"
    assert torch.equal(outs[1], eager), "graph 1 replayed beside graph 0 differs"
    for i, e in enumerate(eagers):
        assert torch.equal(e, eager), f"eager launch {i} beside the replays differs"


def test_o_handout_many_in_flight(dev):
    """320 eager launches (more than the 256 hand-out slots) queued on two
    streams without a synchronisation: the slot table gives a slot only to a
    launch whose slot's previous launch has completed (else the fixed walk),
    so every output equals the first launch's."""
    assert _pipelined(dev)
    data = _inputs(dev, seed=22)
    ref = chunk_fwd_o.custom_kernel(data)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = []
    for i in range(320):
        with torch.cuda.stream(streams[i % 2]):
            outs.append(chunk_fwd_o.custom_kernel(data))
    torch.cuda.synchronize()
    print("many in flight: 320 launches done", flush=True)
    bad = [i for i, o in enumerate(outs) if not torch.equal(o, ref)]
    assert not bad, f"{len(bad)} of 320 launches differ from the first (first: {bad[:8]})"
    assert np.isfinite(ref.float().cpu().numpy()).all()
