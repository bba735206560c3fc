"""Benchmark of the MI355X hot path: one step = causal_conv1d + the Gated
DeltaNet chunk forward (recompute_w_u -> chunk_fwd_h -> chunk_fwd_o) at
BASELINE.json config 4 (the largest single-GPU configuration), bf16.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-shapes] [--small]

Prints ONE JSON line (rank 0).  ``value`` is microseconds per step (all four
kernels, inputs resident in HBM, outputs preallocated by the caching
allocator).  Per-kernel durations come from HIP events recorded on the stream
the kernels are launched on (torch's current stream), averaged over the timed
steps.  ``roofline`` is for the kernel with the largest share of the step:
algorithmic bytes per launch / its average duration vs 8 TB/s.  ``traffic``
is read from profiles/traffic_cfg4.json when that summary of rocprofv3
FETCH_SIZE / WRITE_SIZE runs exists and was recorded from the kernel sources
built now (else null, with the reason in ``traffic_note``). ``cpu_baseline`` times the CPU
oracle on a bounded sample (batch elements of the same workload, as many as
fit in about 12 s) and scales to a full step. ``floors`` times memory-only
kernels that move each step kernel's algorithmic bytes in its own tile pattern
with no compute (theorem_amd/csrc/floors.hip): the fastest this box moves
those bytes in that pattern, reported per kernel as ``floor_us`` and
``of_floor`` (floor / kernel time) beside the 8 TB/s roofline.  Each floor
also gives the same pattern with tiles of 2 and 4 adjacent heads
(``heads2_us``, ``heads4_us``: 512 B and 1 KB contiguous row runs) and a
contiguous ceiling, the kernel's read and write bytes as one contiguous
stream each in the same ratio (``ceiling_us``; per kernel ``of_ceiling``).
``measured_peaks`` gives the box's copy rate and bf16 MFMA throughput (a
register-only MFMA loop); each kernel's ``mfma_frac_of_measured`` is its flop
rate against the latter. ``shapes`` gives each kernel's latency at configs
0-3 (bf16 where the configs ask for it; chunk_fwd_h in the delta form);
``shapes_reference`` is the like-for-like leg: fp32 inputs from each package's
generate_input, the reference's semantics, at the 12 shapes of the
reference's results/baseline_compare.csv, timed with the reference's
protocol, beside the reference's published MI300X numbers; ``extensions`` times the
kernels beyond the four (WY matrix, gate cumsum, channels-last conv, conv
decode step, fused WY, fused h + o, the whole chunked forward) and the four
step kernels in fp32, the reference's dtype, at config-4 sizes.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK = 8.0e12        # B/s, MI355X published
MFMA_BF16_PEAK = 2.5e15  # flop/s, dense bf16, MI355X published
METRIC = "µs/call and % of roofline (HBM GB/s or bf16 MFMA) per kernel, 1×MI355X"

CFG4 = dict(B=8, T=8192, H=16, K=128, V=128)
CFG4_CONV = dict(B=8, D=4096, S=8192, W=4)


# --------------------------------------------------------------------------- algorithmic work

def work_conv(B, D, S, W, eb=2, ebw=2):
    return 2 * B * D * S * eb + D * (W + 1) * ebw, 2 * W * B * D * S


def work_wu(B, T, H, K, V, eb=2):
    N = B * T * H
    NC = N // 64
    return N * (K + V) * eb + N * 8 + N * 64 * 4 + N * (K + V) * eb, NC * 2 * 64 * 64 * (K + V)


def work_h(B, T, H, K, V, eb=2, final=True):
    N = B * T * H
    NC = N // 64
    by = N * (2 * K + V) * eb + 4 * N + NC * K * V * 4 + N * V * eb + (B * H * K * V * 4 if final else 0)
    return by, NC * 4 * 64 * K * V


def work_o(B, T, H, K, V, eb=2):
    N = B * T * H
    NC = N // 64
    by = N * (2 * K + V) * eb + 4 * N + NC * K * V * 4 + N * V * eb
    return by, NC * (2 * 64 * 64 * (K + V) + 2 * 64 * K * V)


# --------------------------------------------------------------------------- measured traffic

def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from profiles/traffic_cfg4.json (two
    rocprofv3 counter passes, FETCH_SIZE and WRITE_SIZE, calibrated against a
    plain copy), or None when the summary is missing or was recorded from
    other kernel sources than the ones built now (theorem_amd.profiling
    source_digest of the kernel's unit and its headers)."""
    from theorem_amd.profiling import UNITS, source_digest

    tpath = ROOT / "profiles" / "traffic_cfg4.json"
    try:
        rec = json.loads(tpath.read_text()).get(kernel)
    except (OSError, ValueError):
        return None, "no counter summary"
    if not rec:
        return None, "kernel not in the counter summary"
    if rec.get("source_digest") != source_digest(UNITS[kernel]):
        return None, "stale: the kernel's sources changed after the counter run"
    return rec["hbm_bytes_per_launch"], (f"profiles/traffic_cfg4.json, ratio {rec['ratio']} of the algorithmic "
                                         f"{rec['algorithmic_bytes']} B")


def settle(torch, fn, min_s: float, batch: int = 4) -> float:
    """Run ``fn`` (untimed) in batches until ``min_s`` seconds of wall time have
    passed, synchronising after each batch; return the seconds spent.

    The GPU comes out of an idle period (input generation, host work between
    phases) at a lowered clock and takes tens of milliseconds of continuous work
    to reach its steady clock (``--ramp-probe``): on MI355X the fused h + o
    kernel runs its first ~10 ms after even 20 ms of idle at 395-425 us per
    call, against ~345 us after ~35 ms, and the config-4 step at 1367-1387
    against ~1287 us.  The step and the extension kernels are timed
    after such a settle run of the same work, so their numbers are steady-state
    rates; the per-shape latencies keep the reference's protocol (a
    synchronised call at a time)."""
    t0 = time.perf_counter()
    while True:
        for _ in range(batch):
            fn()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= min_s:
            return time.perf_counter() - t0


# --------------------------------------------------------------------------- CPU baseline

def cpu_baseline(torch, inputs, conv_inputs, target_s: float = 12.0):
    """Time the CPU oracle on a bounded sample of the same workload and scale to a full step.

    One batch element is timed first; the sample then grows to as many batch
    elements (and repetitions) as fit in about ``target_s`` seconds, and the
    median per-element time is scaled to the full batch."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import conv as oconv
    from oracle import deltanet as odn

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    Bfull = inputs["q"].shape[0]
    x, w, bias = conv_inputs
    wn, bn = w.float().cpu().numpy(), bias.float().cpu().numpy()

    def host(nb):
        f = lambda t: t[:nb].float().cpu().numpy()  # noqa: E731
        return tuple(f(inputs[k]) for k in ("q", "k", "v", "beta", "g", "A")) + (x[:nb].float().cpu().numpy(),)

    def run(arrs):
        q, k, v, beta, g, A, xs = arrs
        t0 = time.perf_counter()
        oconv.causal_conv1d_c(xs, wn, bn)
        t1 = time.perf_counter()
        ww, uu = odn.recompute_w_u_ref(k, v, beta, A, g, dtype=np.float32)
        h, vn, _ = odn.chunk_fwd_h_delta(k, ww, uu, g, dtype=np.float32)
        odn.chunk_fwd_o_diff(q, k, vn, g, h, inputs["scale"], dtype=np.float32)
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1

    with threadpool_limits(limits=n):
        one = host(1)
        # warm-up on a tiny slice (library load, first-touch page faults)
        oconv.causal_conv1d_c(one[6][:, :8], wn[:8], bn[:8])
        odn.recompute_w_u_ref(*(a[:, :64, :1] for a in (one[1], one[2], one[3], one[5], one[4])), dtype=np.float32)
        c1, d1 = run(one)
        per_elem = c1 + d1
        nb = int(max(1, min(Bfull, target_s / 3 / max(per_elem, 1e-3))))
        reps = int(max(1, min(5, target_s / max(per_elem * nb, 1e-3))))
        arrs = one if nb == 1 else host(nb)
        times = [run(arrs) for _ in range(reps)]
    conv_s = sorted(t[0] for t in times)[len(times) // 2] / nb
    chain_s = sorted(t[1] for t in times)[len(times) // 2] / nb
    us = (conv_s + chain_s) * Bfull * 1e6
    # torch-CPU F.conv1d over all the cores, on the same sample (a library
    # leg beside the single-threaded restatement of scripts/cpu_reference.py).
    xt = torch.from_numpy(arrs[6])
    wt = torch.from_numpy(wn).unsqueeze(1)
    bt = torch.from_numpy(bn)
    Wd = wn.shape[1]

    def tconv():
        t0 = time.perf_counter()
        torch.nn.functional.conv1d(torch.nn.functional.pad(xt, (Wd - 1, 0)), wt, bt, groups=wt.shape[0])
        return time.perf_counter() - t0

    tconv()
    tconv_s = sorted(tconv() for _ in range(max(3, reps)))[max(3, reps) // 2] / nb
    return {"value": round(us, 1), "unit": "µs/call", "cores": n, "kind": "port",
            "sample": (f"oracle/ (C conv single-threaded; NumPy fp32 recompute_w_u/chunk_fwd_h/chunk_fwd_o, "
                       f"BLAS threads={n}) on batch elements 0..{nb - 1} of config 4, median of {reps} runs, "
                       f"scaled x{Bfull / nb:g} to the full step; per batch element: conv {1e3 * conv_s:.0f} ms, "
                       f"chain {1e3 * chain_s:.0f} ms"),
            "legs_us": {"conv_oracle_c_1_thread": round(conv_s * Bfull * 1e6, 1),
                        f"conv_torch_cpu_{n}_threads": round(tconv_s * Bfull * 1e6, 1),
                        f"chain_oracle_numpy_{n}_threads": round(chain_s * Bfull * 1e6, 1)},
            "host": _cpu_model()}


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# --------------------------------------------------------------------------- per-shape latency

def shape_latencies(torch, dev, warmup: int = 5, iters: int = 50, batched: int = 200):
    """Latency of each kernel at BASELINE.json configs 0-3 (the reference's
    published shapes), three ways:
      us_ref       the reference's protocol (benchmarks/pytorch_baseline.py:72-96):
                   min over ``iters`` calls, each an event pair around
                   ``custom_kernel`` on an idle GPU, so the host-side launch
                   (Python wrapper + ctypes + HIP launch) is inside the bracket;
      us_cold_*    min / p50 with a 512 MiB write before each call: the start
                   event runs after that write, by which time the launch is
                   queued, so this is the kernel on cold caches;
      us_batched   ``batched`` back-to-back calls under one event pair, per call
                   (bounded below by the host launch rate for tiny kernels);
      us_kernel    median with a spin kernel (torch.cuda._sleep) queued ahead of
                   the start event: the kernel alone on warm caches;
      host_us      host wall time per call of ``batched`` back-to-back calls
                   queued behind a spin kernel: the host side of a call (Python
                   wrapper, output allocation, ctypes, HIP launch; the launch
                   alone is ~2.3 us through any HIP launch API on the box).
    On ROCm the event pair of us_ref does not open before the kernel's own
    dispatch, so us_ref is close to us_kernel and host_us is the host cost."""
    from theorem_amd import configs
    from theorem_amd.kernels import causal_conv1d, chunk_fwd_h, chunk_fwd_o, recompute_w_u

    flush = torch.empty(1 << 27, dtype=torch.float32, device=dev)
    c0 = configs.make_conv_inputs(1, 2560, 4096, 4, dtype=torch.float32, seed=0, device=dev)
    w1 = configs.make_wu_inputs(2, 512, 3, 64, 64, seed=0, device=dev)
    o2 = configs.make_o_inputs(2, 512, 3, 64, 64, seed=0, device=dev)
    h3 = configs.make_h_inputs(2, 1024, 3, 64, 64, seed=0, device=dev)
    wu_data = recompute_w_u.Data(**w1, B=2, T=512, H=3, K=64, V=64)
    cases = [
        ("cfg0", "causal_conv1d", "(1,2560,4096,W=4) fp32", lambda: causal_conv1d.custom_kernel(c0),
         work_conv(1, 2560, 4096, 4, eb=4, ebw=4)),
        ("cfg1", "recompute_w_u", "(2,512,3,64,64) bf16", lambda: recompute_w_u.custom_kernel(wu_data),
         work_wu(2, 512, 3, 64, 64)),
        ("cfg2", "chunk_fwd_o", "(2,512,3,64,64) bf16",
         lambda: chunk_fwd_o.custom_kernel(dict(q=o2["q"], k=o2["k"], v=o2["v"], g=o2["g"], h=o2["h"],
                                                scale=o2["scale"])),
         work_o(2, 512, 3, 64, 64)),
        ("cfg3", "chunk_fwd_h", "(2,1024,3,64,64) bf16 delta form, h0 = 0",
         lambda: chunk_fwd_h.custom_kernel(dict(k=h3["k"], w=h3["w"], u=h3["u"], g=h3["g"],
                                                output_final_state=True)),
         work_h(2, 1024, 3, 64, 64)),
    ]
    out = {}
    for cfg, name, shape, fn, (by, fl) in cases:
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        def timed(pre):
            ts = []
            for _ in range(iters):
                if pre is not None:
                    pre()
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                fn()
                e.record()
                torch.cuda.synchronize()
                ts.append(s.elapsed_time(e) * 1e3)
            return sorted(ts)
        ref = timed(None)
        cold = timed(flush.zero_)
        # Kernel alone on warm caches: a spin kernel ahead of the start event
        # keeps the GPU busy while the host enqueues the call, so the event
        # pair brackets the kernel only; us_ref - us_kernel is the host side.
        warm = timed(lambda: torch.cuda._sleep(200000))
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(batched):
            fn()
        e.record()
        torch.cuda.synchronize()
        bat = s.elapsed_time(e) * 1e3 / batched
        # Host side of a call: wall time per call of back-to-back calls with
        # the GPU kept busy ahead of them (the launches only queue).
        torch.cuda._sleep(20000000)
        t0 = time.perf_counter()
        for _ in range(batched):
            fn()
        host = (time.perf_counter() - t0) * 1e6 / batched
        torch.cuda.synchronize()
        out[cfg] = {"kernel": name, "shape": shape, "us_ref": round(ref[0], 2),
                    "us_kernel": round(warm[len(warm) // 2], 2), "host_us": round(host, 2),
                    "us_cold_min": round(cold[0], 2), "us_cold_p50": round(cold[len(cold) // 2], 2),
                    "us_batched": round(bat, 2), "bytes": by, "flops": fl,
                    "hbm_frac_cold_min": round(by / (cold[0] * 1e-6) / HBM_PEAK, 4)}
    del flush
    return out


# The reference's published Triton numbers (MI300X, fp32, min over 50
# event-bracketed calls after 5 warm-up calls, host-inclusive) at its task.yml
# benchmark shapes: results/baseline_compare.csv:2-13 of the reference,
# column triton_min_us.
REF_PUBLISHED_US = {
    ("causal_conv1d", "B=1,D=1536,S=2048,W=4"): 24.78,
    ("causal_conv1d", "B=1,D=2560,S=2048,W=4"): 32.96,
    ("causal_conv1d", "B=1,D=2560,S=4096,W=4"): 46.83,
    ("chunk_fwd_h", "B=1,T=64,H=1,K=64,V=64"): 28.74,
    ("chunk_fwd_h", "B=2,T=512,H=3,K=64,V=64"): 37.40,
    ("chunk_fwd_h", "B=2,T=1024,H=3,K=64,V=64"): 49.11,
    ("chunk_fwd_o", "B=1,T=64,H=1,K=64,V=64"): 36.56,
    ("chunk_fwd_o", "B=2,T=512,H=3,K=64,V=64"): 42.54,
    ("chunk_fwd_o", "B=2,T=1024,H=3,K=64,V=64"): 33.11,
    ("recompute_w_u", "B=1,T=64,H=1,K=64,V=64"): 39.93,
    ("recompute_w_u", "B=2,T=512,H=3,K=64,V=64"): 38.93,
    ("recompute_w_u", "B=2,T=1024,H=3,K=64,V=64"): 38.45,
}


def shapes_reference(torch, compile_: bool = False, batched: int = 200):
    """Like for like with the reference's published numbers: each kernel at
    its task.yml benchmark shapes (the rows of the reference's
    results/baseline_compare.csv), fp32 inputs from the package's own
    generate_input with the task.yml seed, the reference's semantics
    (chunk_fwd_h as (k, v, g) -> h, the state after each chunk), timed with
    the reference's protocol (benchmarks/pytorch_baseline.py:72-96: 5 warm-up
    calls, min over 50 calls each bracketed by an event pair and a
    synchronize; theorem_amd.benchmarks.pytorch_baseline._time_callable).
    ``us_min`` is that figure; ``us_batched`` is ``batched`` back-to-back
    calls under one event pair, per call; ``eager_min_us`` the vectorised
    PyTorch eager form on the same inputs; ``compiled_min_us`` torch.compile
    of it (only with ``compile_``); ``ref_published_us`` the reference's
    number on MI300X."""
    import yaml

    from theorem_amd.benchmarks import pytorch_baseline as pb

    rows = []
    for kname in ("causal_conv1d", "chunk_fwd_h", "chunk_fwd_o", "recompute_w_u"):
        spec = yaml.safe_load((ROOT / "theorem_amd" / "kernels" / kname / "task.yml").read_text())
        for shape in spec["shapes"]["benchmarks"]:
            label = ",".join(f"{k}={v}" for k, v in shape.items() if k != "seed")
            run_hip, run_eager, run_comp = pb._stage(kname, shape, compile_)
            t = pb._time_callable(run_hip)
            e = pb._time_callable(run_eager)
            c = pb._safe_time("compiled", shape, run_comp) if run_comp else None
            s, ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(batched):
                run_hip()
            ev.record()
            torch.cuda.synchronize()
            pub = REF_PUBLISHED_US.get((kname, label))
            rows.append({"kernel": kname, "shape": label, "dtype": "fp32", "us_min": round(t, 2),
                         "us_batched": round(s.elapsed_time(ev) * 1e3 / batched, 2),
                         "eager_min_us": round(e, 2),
                         "compiled_min_us": None if c is None or c != c else round(c, 2),
                         "ref_published_us": pub,
                         "speedup_vs_ref_published": round(pub / t, 2) if pub else None})
            torch.cuda.empty_cache()
    return rows


# --------------------------------------------------------------------------- extensions

def pattern_floors(torch, inp, conv_in, reps: int = 5):
    """Memory-only floor of each step kernel's access pattern (libtheorem_floors.so,
    csrc/floors.hip): the same algorithmic bytes moved in the same tile pattern
    with no compute, min over ``reps`` launches (HIP events on the current stream).
    The conv's floor is a streaming copy of x into a buffer of its size."""
    import ctypes

    from theorem_amd.build import FLOORS_LIB

    if not FLOORS_LIB.exists():
        return None
    lib = ctypes.CDLL(str(FLOORS_LIB))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    stream = vp(torch.cuda.current_stream().cuda_stream)
    P = lambda t: vp(t.data_ptr())  # noqa: E731
    q, k, v, beta, g, A = (inp[n] for n in ("q", "k", "v", "beta", "g", "A"))
    B, T, H, K = k.shape
    if K != 128 or v.shape[-1] != 128:
        return None
    x = conv_in[0]
    xo = torch.empty_like(x)
    w2, u2, vn2, o2 = (torch.empty_like(k) for _ in range(4))
    h2 = torch.empty(B, T // 64, H, K, K, device=k.device, dtype=torch.float32)
    N = B * T * H
    runs = {
        "causal_conv1d": (lambda: lib.thm_floor_copy(P(x), P(xo), i64(x.numel() * x.element_size()), stream),
                          2 * x.numel() * x.element_size()),
        "recompute_w_u": (lambda: lib.thm_floor_wu(P(k), P(v), P(A), P(beta), P(g), P(w2), P(u2), i64(B), i64(T),
                                                   i64(H), stream), N * (4 * 256 + 8 + 256)),
        "chunk_fwd_h": (lambda: lib.thm_floor_h(P(k), P(w2), P(u2), P(g), P(h2), P(vn2), i64(B), i64(T), i64(H),
                                                stream), N * (4 * 256 + 4) + (N // 64) * 65536),
        "chunk_fwd_o": (lambda: lib.thm_floor_o(P(q), P(k), P(v), P(h2), P(g), P(o2), i64(B), i64(T), i64(H),
                                                stream), N * (4 * 256 + 4) + (N // 64) * 65536),
        # extension kernels: the fused WY forward and the fused h + o
        "wy_fwd": (lambda: lib.thm_floor_wy(P(k), P(v), P(beta), P(g), P(w2), P(u2), i64(B), i64(T), i64(H), stream),
                   N * (4 * 256 + 8)),
        "chunk_gated_delta_fwd": (lambda: lib.thm_floor_ho(P(q), P(k), P(w2), P(u2), P(g), P(o2), i64(B), i64(T),
                                                           i64(H), stream), N * (5 * 256 + 4)),
    }
    # Multi-head variants of the tile floors: tiles of 2 and 4 adjacent heads,
    # so each token row of a tensor is one 512 B or 1 KB contiguous run.
    heads = {
        "recompute_w_u": lambda nh: lib.thm_floor_wu_heads(P(k), P(v), P(A), P(beta), P(g), P(w2), P(u2), i64(B),
                                                           i64(T), i64(H), ctypes.c_int32(nh), stream),
        "chunk_fwd_h": lambda nh: lib.thm_floor_h_heads(P(k), P(w2), P(u2), P(g), P(h2), P(vn2), i64(B), i64(T),
                                                        i64(H), ctypes.c_int32(nh), stream),
        "chunk_fwd_o": lambda nh: lib.thm_floor_o_heads(P(q), P(k), P(v), P(h2), P(g), P(o2), i64(B), i64(T), i64(H),
                                                        ctypes.c_int32(nh), stream),
    }
    # Contiguous ceilings: each kernel's read and write bytes as one
    # contiguous stream per direction, in the kernel's read : write ratio.
    NC = N // 64
    mix = {
        "causal_conv1d": (x.numel() * x.element_size(), x.numel() * x.element_size()),
        "recompute_w_u": (N * (3 * 256 + 8), N * 2 * 256),
        "chunk_fwd_h": (N * (3 * 256 + 4), N * 256 + NC * 65536),
        "chunk_fwd_o": (N * (3 * 256 + 4) + NC * 65536, N * 256),
        "wy_fwd": (N * (2 * 256 + 8), N * 2 * 256),
        "chunk_gated_delta_fwd": (N * (4 * 256 + 4), N * 256),
        "chunk_gated_delta_fwd_a": (N * (4 * 256 + 8), N * 256),
    }
    src = torch.empty(max(r for r, _ in mix.values()), dtype=torch.uint8, device=k.device)
    dst = torch.empty(max(w for _, w in mix.values()), dtype=torch.uint8, device=k.device)

    def best_of(fn):
        if fn() != 0:
            return None
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            best = min(best, e0.elapsed_time(e1) * 1e3)
        return best

    out = {}
    for name, (fn, by) in runs.items():
        best = best_of(fn)
        if best is None:
            return None
        out[name] = {"us": round(best, 2), "bytes": by, "GBps": round(by / best / 1e3, 1)}
        for nh in (2, 4):
            if name in heads and H % nh == 0:
                t = best_of(lambda: heads[name](nh))
                if t is not None:
                    out[name][f"heads{nh}_us"] = round(t, 2)
        rd, wr = mix[name]
        t = best_of(lambda: lib.thm_floor_mix(P(src), i64(rd), P(dst), i64(wr), stream))
        if t is not None:
            out[name]["ceiling_us"] = round(t, 2)
            out[name]["ceiling_GBps"] = round((rd + wr) / t / 1e3, 1)
    for name in mix.keys() - runs.keys():  # a ceiling only (the A form shares the w / u form's floor)
        rd, wr = mix[name]
        t = best_of(lambda: lib.thm_floor_mix(P(src), i64(rd), P(dst), i64(wr), stream))
        if t is not None:
            out[name] = {"ceiling_us": round(t, 2), "ceiling_GBps": round((rd + wr) / t / 1e3, 1)}
    del src, dst
    return out


def measured_peaks(torch, dev, floors, reps: int = 5):
    """Peaks taken on this box beside the published ones: the streaming-copy
    rate (the conv's floor, a copy of x) and the bf16 MFMA throughput of
    floor_mfma_kernel (libtheorem_floors.so: v_mfma_f32_16x16x32_bf16 on register
    operands, no memory traffic; 8 workgroups of 4 waves per CU, 16 independent
    accumulator chains per wave), min over ``reps`` launches."""
    import ctypes

    from theorem_amd.build import FLOORS_LIB

    if not FLOORS_LIB.exists():
        return None
    lib = ctypes.CDLL(str(FLOORS_LIB))
    nblocks = 8 * torch.cuda.get_device_properties(dev).multi_processor_count
    iters, chains = 2048, 16
    out = torch.empty(nblocks * 256, device=dev, dtype=torch.float32)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def run():
        return lib.thm_floor_mfma(ctypes.c_void_p(out.data_ptr()), ctypes.c_int64(nblocks), ctypes.c_int64(iters),
                                  stream)

    if run() != 0:
        return None
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        run()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3)
    flops = nblocks * 4 * iters * chains * 16384
    res = {"mfma_bf16_TFLOPs": round(flops / best / 1e6, 1),
           "mfma_of_published": round(flops / (best * 1e-6) / MFMA_BF16_PEAK, 3)}
    if floors and "causal_conv1d" in floors:
        res["copy_GBps"] = floors["causal_conv1d"]["GBps"]
        res["copy_of_published"] = round(floors["causal_conv1d"]["GBps"] * 1e9 / HBM_PEAK, 3)
    return res


def work_build_A(B, T, H, K, eb=2):
    N = B * T * H
    return N * K * eb + N * 8 + N * 64 * 4


def extension_timings(torch, inp, conv_in, iters: int = 10, settle_s: float = 0.05):
    """The kernels beyond the four (WY matrix, gate cumsum, channels-last conv,
    conv decode step, fused WY, fused h + o, the whole chunked forward) and the
    four in fp32 (the reference's dtype), at config-4 sizes: HIP events around
    ``iters`` back-to-back launches after a ``settle_s`` settle run of the same
    call."""
    from theorem_amd import chain
    from theorem_amd.kernels import causal_conv1d, recompute_w_u

    B, T, H, K = inp["k"].shape
    x, w, b = conv_in
    Bc, D, S = x.shape
    xcl = x.transpose(1, 2).contiguous().transpose(1, 2)
    a = torch.randn(B, T, H, device=x.device)
    state = torch.zeros(Bc, D, w.shape[1] - 1, dtype=x.dtype, device=x.device)
    xt = x[:, :, 0].contiguous()
    cases = {
        "wy_build_A": (lambda: recompute_w_u.build_A(inp["k"], inp["beta"], inp["g"], sign=+1),
                       work_build_A(B, T, H, K), f"({B},{T},{H},K={K}) bf16 k, sign +1"),
        "chunk_local_cumsum": (lambda: chain.chunk_local_cumsum(a, logsigmoid=True), B * T * H * 8,
                               f"({B},{T},{H}) fp32, logsigmoid"),
        "causal_conv1d_channels_last": (lambda: causal_conv1d.custom_kernel((xcl, w, b)),
                                        work_conv(Bc, D, S, w.shape[1])[0], f"({Bc},{S},{D}) bf16 [B,S,D]"),
        "causal_conv1d_update": (lambda: causal_conv1d.causal_conv1d_update(xt, state, w, b),
                                 Bc * D * (2 * 2 + 2 * (w.shape[1] - 1) * 2), f"({Bc},{D}) bf16, one token"),
    }
    V = inp["v"].shape[-1]
    ww, uu = recompute_w_u.custom_kernel(recompute_w_u.Data(
        k=inp["k"], v=inp["v"], beta=inp["beta"], A=inp["A"], g=inp["g"], B=B, T=T, H=H, K=K, V=V))
    N = B * T * H
    cases["wy_fwd"] = (
        lambda: chain.wy_fwd(inp["k"], inp["v"], inp["beta"], inp["g"], sign=+1),
        N * (K * 2 + V * 2 + 8) + N * (K * 2 + V * 2),
        f"({B},{T},{H},{K},{V}) bf16: A-builder + recompute_w_u fused, A kept on chip")
    cases["chunk_gated_delta_fwd"] = (
        lambda: chain.chunk_fwd_fused(inp["q"], inp["k"], ww, uu, inp["g"], inp["scale"], None, True),
        N * (3 * K * 2 + V * 2 + 4) + N * V * 2 + B * H * K * V * 4,
        f"({B},{T},{H},{K},{V}) bf16: chunk_fwd_h + chunk_fwd_o fused, final state out")
    cases["chunk_gated_delta_fwd_a"] = (
        lambda: chain.chunk_fwd_fused_a(inp["q"], inp["k"], inp["v"], inp["beta"], inp["A"], inp["g"], inp["scale"],
                                        None, True),
        N * (2 * K * 2 + V * 2 + 64 * 4 + 8) + N * V * 2 + B * H * K * V * 4,
        f"({B},{T},{H},{K},{V}) bf16: recompute_w_u + chunk_fwd_h + chunk_fwd_o fused from A, final state out")
    cases["chunk_gated_delta_rule_fwd"] = (
        lambda: chain.chunk_gated_delta_rule_fwd(inp["q"], inp["k"], inp["v"], inp["beta"], inp["g"], inp["scale"],
                                                 output_final_state=True),
        N * (K * 2 + 8) + N * 64 * 4 + N * (2 * K * 2 + V * 2 + 64 * 4 + 8) + N * V * 2 + B * H * K * V * 4,
        "the whole chunked forward from (q, k, v, beta, g): A-builder, then the fused forward from A")
    cases["chunk_gated_delta_rule_fwd_wy"] = (
        lambda: chain.chunk_gated_delta_rule_fwd(inp["q"], inp["k"], inp["v"], inp["beta"], inp["g"], inp["scale"],
                                                 output_final_state=True, fused_form="wy"),
        N * (K * 2 + V * 2 + 8) + N * (K * 2 + V * 2) + N * (3 * K * 2 + V * 2 + 4) + N * V * 2 + B * H * K * V * 4,
        "the same through w and u: fused WY (A, w, u), fused h + o")
    # The reference's own dtype (fp32; kernel.py asserts it) at config-4 sizes.
    from theorem_amd.kernels import chunk_fwd_h, chunk_fwd_o
    k32, v32, q32 = inp["k"].float(), inp["v"].float(), inp["q"].float()
    w32, u32 = ww.float(), uu.float()
    h32 = torch.zeros(B, T // 64, H, K, V, device=k32.device)
    x32, w32c, b32 = x.float(), w.float(), b.float()
    g, beta, A, scale = inp["g"], inp["beta"], inp["A"], inp["scale"]
    cases["fp32_causal_conv1d"] = (lambda: causal_conv1d.custom_kernel((x32, w32c, b32)),
                                   work_conv(Bc, D, S, w.shape[1], eb=4, ebw=4)[0], f"({Bc},{D},{S},W=4) fp32")
    cases["fp32_recompute_w_u"] = (
        lambda: recompute_w_u.custom_kernel(recompute_w_u.Data(k=k32, v=v32, beta=beta, A=A, g=g, B=B, T=T, H=H,
                                                               K=K, V=V)),
        work_wu(B, T, H, K, V, eb=4)[0], f"({B},{T},{H},{K},{V}) fp32")
    cases["fp32_chunk_fwd_h"] = (
        lambda: chunk_fwd_h.custom_kernel(dict(k=k32, w=w32, u=u32, g=g, output_final_state=True)),
        work_h(B, T, H, K, V, eb=4)[0], f"({B},{T},{H},{K},{V}) fp32, delta form")
    cases["fp32_chunk_fwd_h_reference_form"] = (
        lambda: chunk_fwd_h.custom_kernel(dict(k=k32, v=v32, g=g)),
        N * (K + V) * 4 + 4 * N + (N // 64) * K * V * 4, f"({B},{T},{H},{K},{V}) fp32, the reference's (k, v, g) -> h")
    cases["fp32_chunk_fwd_o"] = (
        lambda: chunk_fwd_o.custom_kernel(dict(q=q32, k=k32, v=v32, g=g, h=h32, scale=scale)),
        work_o(B, T, H, K, V, eb=4)[0], f"({B},{T},{H},{K},{V}) fp32")
    out = {}
    for name, (fn, by, shape) in cases.items():
        settle(torch, fn, settle_s)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / iters
        out[name] = {"us": round(us, 2), "shape": shape, "bytes": by, "GBps": round(by / us / 1e3, 1),
                     "hbm_frac": round(by / (us * 1e-6) / HBM_PEAK, 4)}
    return out


# --------------------------------------------------------------------------- order probe

def order_probe(torch, step_fns: dict, reps: int = 12) -> dict:
    """recompute_w_u and chunk_fwd_o times after different preceding kernels
    (HIP events per kernel, medians over ``reps`` rounds): alone back to back,
    after a 1 GiB write (torch fill_, ordinary stores), after a 1 GiB read
    (torch sum), after a 1 GiB copy, and inside the config-4 step.  The
    kernels' own code and inputs are the same in every case."""
    import statistics

    dev = torch.device("cuda:0")
    big = torch.empty(1 << 28, device=dev)
    big2 = torch.empty_like(big)
    pre = {"alone": None, "after 1 GiB fill": lambda: big.fill_(1.0), "after 1 GiB sum": lambda: big.sum(),
           "after 1 GiB copy": lambda: big2.copy_(big)}
    out = {}
    for kname in ("recompute_w_u", "chunk_fwd_o"):
        fn = step_fns[kname]
        for label, p in pre.items():
            seq = ([p] if p else []) + [fn]
            for _ in range(3):
                for f in seq:
                    f()
            torch.cuda.synchronize()
            ts = []
            for _ in range(reps):
                if p:
                    p()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                fn()
                e1.record()
                torch.cuda.synchronize()
                ts.append(e0.elapsed_time(e1) * 1e3)
            out.setdefault(kname, {})[label] = round(statistics.median(ts), 1)
    # inside the step: per-kernel events around each launch
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(reps)]
    order = ["causal_conv1d", "recompute_w_u", "chunk_fwd_h", "chunk_fwd_o"]
    for _ in range(2):
        for n in order:
            step_fns[n]()
    torch.cuda.synchronize()
    for r in range(reps):
        evs[r][0].record()
        for i, n in enumerate(order):
            step_fns[n]()
            evs[r][i + 1].record()
    torch.cuda.synchronize()
    for i, n in enumerate(order):
        if n in out:
            out[n]["in the step"] = round(statistics.median(evs[r][i].elapsed_time(evs[r][i + 1]) * 1e3
                                                            for r in range(reps)), 1)
    return out


# --------------------------------------------------------------------------- clock ramp probe

def ramp_probe(torch, calls: dict, batches: int = 25) -> dict:
    """Per-call time of each entry of ``calls`` (name -> (fn, calls per batch))
    in consecutive batches after the GPU has been idle for 2 s, 0.2 s and
    0.02 s (HIP events around each batch, a synchronize after it): how long the
    clock takes to come out of idle, which sets the settle run before timing."""
    out = {}
    for name, (fn, per) in calls.items():
        fn()
        torch.cuda.synchronize()
        for idle in (2.0, 0.2, 0.02):
            time.sleep(idle)
            ts = []
            for _ in range(batches):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(per):
                    fn()
                e1.record()
                torch.cuda.synchronize()
                ts.append(round(e0.elapsed_time(e1) * 1e3 / per, 1))
            out.setdefault(name, {})[f"after {idle} s idle"] = ts
    return out


# --------------------------------------------------------------------------- main

def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--settle", type=float, default=0.25,
                    help="seconds of untimed steps before the warm-up, to bring the GPU clock out of idle (0: none)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline")
    ap.add_argument("--no-shapes", action="store_true", help="skip the per-shape latencies of configs 0-3")
    ap.add_argument("--no-ref-shapes", action="store_true",
                    help="skip the like-for-like fp32 timings at the reference's published shapes")
    ap.add_argument("--compile", action="store_true",
                    help="add the torch.compile column to the reference-shape timings (slow: compiles 12 graphs)")
    ap.add_argument("--no-ext", action="store_true", help="skip the extension kernels (A-builder, gate cumsum, ...)")
    ap.add_argument("--small", action="store_true", help="1/8-size workload (quick check)")
    ap.add_argument("--only", choices=["causal_conv1d", "recompute_w_u", "chunk_fwd_h", "chunk_fwd_o", "wy_build_A",
                                        "chunk_gated_delta_fwd", "chunk_gated_delta_fwd_a", "wy_fwd"],
                    help="run only this kernel of the step (for per-kernel rocprofv3 counter runs)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="run a plain 1 GiB device-to-device copy (rocprofv3 counter calibration)")
    ap.add_argument("--ramp-probe", action="store_true",
                    help="per-call times of the fused h + o kernel and of the step in batches after idle periods, "
                         "then exit")
    ap.add_argument("--order-probe", action="store_true",
                    help="time recompute_w_u and chunk_fwd_o after different preceding kernels, then exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (the hot-path kernels are single-device; "
              "multi-GPU sharding is designed but not launched). Use --gpus 1.",
              file=sys.stderr)
        return 2

    import torch

    if args.copy_calib:
        # A plain copy kernel of known size: FETCH_SIZE / WRITE_SIZE per dispatch
        # should read 1 GiB each; the ratio calibrates the counters.
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes": src.numel() * 4, "launches": args.warmup + args.steps}))
        return 0

    from theorem_amd import chain, configs
    from theorem_amd.kernels import causal_conv1d, chunk_fwd_h, chunk_fwd_o, recompute_w_u

    dev = torch.device("cuda:0")
    shp = dict(CFG4)
    cshp = dict(CFG4_CONV)
    if args.small:
        shp["B"], cshp["B"] = 1, 1
    t_gen = time.perf_counter()
    inp = configs.make_chain_inputs(**shp, seed=0, device=dev)
    conv_in = configs.make_conv_inputs(**cshp, dtype=torch.bfloat16, seed=0, device=dev)
    torch.cuda.synchronize()
    print(f"[bench] inputs ready in {time.perf_counter() - t_gen:.1f}s", file=sys.stderr, flush=True)

    B, T, H, K, V = (shp[n] for n in ("B", "T", "H", "K", "V"))
    q, k, v, beta, g, A, scale = (inp[n] for n in ("q", "k", "v", "beta", "g", "A", "scale"))
    names = ["causal_conv1d", "recompute_w_u", "chunk_fwd_h", "chunk_fwd_o"]

    def step(ev=None):
        def mark(i):
            if ev is not None:
                ev[i].record()
        mark(0)
        y = causal_conv1d.custom_kernel(conv_in)
        mark(1)
        w, u = recompute_w_u.custom_kernel(recompute_w_u.Data(k=k, v=v, beta=beta, A=A, g=g, B=B, T=T, H=H, K=K, V=V))
        mark(2)
        h, vn, ht = chunk_fwd_h.custom_kernel(dict(k=k, w=w, u=u, g=g, output_final_state=True))
        mark(3)
        o = chunk_fwd_o.custom_kernel(dict(q=q, k=k, v=vn, g=g, h=h, scale=scale))
        mark(4)
        return y, o, ht

    if args.order_probe:
        st = {}

        def _wu():
            st["w"], st["u"] = recompute_w_u.custom_kernel(
                recompute_w_u.Data(k=k, v=v, beta=beta, A=A, g=g, B=B, T=T, H=H, K=K, V=V))

        def _h():
            st["h"], st["vn"], _ = chunk_fwd_h.custom_kernel(dict(k=k, w=st["w"], u=st["u"], g=g,
                                                                  output_final_state=True))

        fns = {"causal_conv1d": lambda: causal_conv1d.custom_kernel(conv_in), "recompute_w_u": _wu,
               "chunk_fwd_h": _h,
               "chunk_fwd_o": lambda: chunk_fwd_o.custom_kernel(dict(q=q, k=k, v=st["vn"], g=g, h=st["h"],
                                                                     scale=scale))}
        _wu()
        _h()
        print(json.dumps({"order_probe_us": order_probe(torch, fns)}))
        return 0

    if args.ramp_probe:
        w0, u0 = recompute_w_u.custom_kernel(recompute_w_u.Data(k=k, v=v, beta=beta, A=A, g=g, B=B, T=T, H=H, K=K,
                                                                V=V))
        calls = {"chunk_gated_delta_fwd": (lambda: chain.chunk_fwd_fused(q, k, w0, u0, g, scale, None, True), 10),
                 "step": (step, 5)}
        print(json.dumps({"ramp_probe_us_per_call": ramp_probe(torch, calls)}))
        return 0

    if args.only:
        # One kernel, W + K launches on inputs from one full step (counter runs).
        y, o, ht = step()
        w, u = recompute_w_u.custom_kernel(recompute_w_u.Data(k=k, v=v, beta=beta, A=A, g=g, B=B, T=T, H=H, K=K, V=V))
        h, vn, _ = chunk_fwd_h.custom_kernel(dict(k=k, w=w, u=u, g=g, output_final_state=True))
        torch.cuda.synchronize()
        run = {
            "causal_conv1d": lambda: causal_conv1d.custom_kernel(conv_in),
            "recompute_w_u": lambda: recompute_w_u.custom_kernel(
                recompute_w_u.Data(k=k, v=v, beta=beta, A=A, g=g, B=B, T=T, H=H, K=K, V=V)),
            "chunk_fwd_h": lambda: chunk_fwd_h.custom_kernel(dict(k=k, w=w, u=u, g=g, output_final_state=True)),
            "chunk_fwd_o": lambda: chunk_fwd_o.custom_kernel(dict(q=q, k=k, v=vn, g=g, h=h, scale=scale)),
            "wy_build_A": lambda: recompute_w_u.build_A(k, beta, g, sign=+1),
            "chunk_gated_delta_fwd": lambda: chain.chunk_fwd_fused(q, k, w, u, g, scale, None, True),
            "chunk_gated_delta_fwd_a": lambda: chain.chunk_fwd_fused_a(q, k, v, beta, A, g, scale, None, True),
            "wy_fwd": lambda: chain.wy_fwd(k, v, beta, g, sign=+1),
        }[args.only]
        for _ in range(args.warmup + args.steps):
            run()
        torch.cuda.synchronize()
        print(json.dumps({"only": args.only, "launches": args.warmup + args.steps + 1}))
        return 0

    settled_s = settle(torch, step, args.settle) if args.settle > 0 else 0.0
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    per = {n: sum(e[j].elapsed_time(e[j + 1]) for e in evs) * 1e3 / args.steps for j, n in enumerate(names)}

    works = {
        "causal_conv1d": work_conv(**cshp),
        "recompute_w_u": work_wu(B, T, H, K, V),
        "chunk_fwd_h": work_h(B, T, H, K, V),
        "chunk_fwd_o": work_o(B, T, H, K, V),
    }
    kernels = {}
    for n in names:
        by, fl = works[n]
        us = per[n]
        kernels[n] = {"us": round(us, 2), "bytes": by, "flops": fl,
                      "GBps": round(by / us / 1e3, 1), "TFLOPs": round(fl / us / 1e6, 2),
                      "hbm_frac": round(by / (us * 1e-6) / HBM_PEAK, 4),
                      "mfma_frac": round(fl / (us * 1e-6) / MFMA_BF16_PEAK, 4)}
    dom = max(names, key=lambda n: per[n])
    traffic, traffic_note = measured_traffic(dom) if not args.small else (None, "not measured at --small")
    by, _ = works[dom]
    achieved = by / (per[dom] * 1e-6) / 1e9
    roofline = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK / 1e9,
                "unit": "GB/s", "frac": round(achieved * 1e9 / HBM_PEAK, 4), "traffic": traffic,
                "traffic_note": traffic_note}

    floors = peaks = None
    if not args.small:
        print("[bench] memory-only pattern floors", file=sys.stderr, flush=True)
        floors = pattern_floors(torch, inp, conv_in)
        if floors:
            for n in names:
                kernels[n]["floor_us"] = floors[n]["us"]
                kernels[n]["of_floor"] = round(floors[n]["us"] / kernels[n]["us"], 3)
                if "ceiling_us" in floors[n]:
                    kernels[n]["ceiling_us"] = floors[n]["ceiling_us"]
                    kernels[n]["of_ceiling"] = round(floors[n]["ceiling_us"] / kernels[n]["us"], 3)
        print("[bench] measured peaks (copy, bf16 MFMA)", file=sys.stderr, flush=True)
        peaks = measured_peaks(torch, inp["k"].device, floors)
        if peaks:
            for n in names:
                _, fl = works[n]
                kernels[n]["mfma_frac_of_measured"] = round(
                    fl / (kernels[n]["us"] * 1e-6) / (peaks["mfma_bf16_TFLOPs"] * 1e12), 4)

    shapes = None
    if not args.no_shapes:
        print("[bench] per-shape latencies (configs 0-3)", file=sys.stderr, flush=True)
        shapes = shape_latencies(torch, dev)

    ref_shapes = None
    if not args.no_ref_shapes:
        print("[bench] like-for-like fp32 timings at the reference's published shapes", file=sys.stderr, flush=True)
        ref_shapes = shapes_reference(torch, compile_=args.compile)

    ext = None
    if not args.no_ext and not args.small:
        print("[bench] extension kernels", file=sys.stderr, flush=True)
        ext = extension_timings(torch, inp, conv_in)
        # The A form's floor is the w / u form's pattern floor (the same tiles:
        # A rows are 256 bytes like w's at K = 128; its 4 more bytes of beta
        # per token-head are 0.3 % of the bytes); its ceiling is its own mix.
        for n, fn in (("wy_fwd", "wy_fwd"), ("chunk_gated_delta_fwd", "chunk_gated_delta_fwd"),
                      ("chunk_gated_delta_fwd_a", "chunk_gated_delta_fwd")):
            if floors and fn in floors and n in ext:
                ext[n]["floor_us"] = floors[fn]["us"]
                ext[n]["of_floor"] = round(floors[fn]["us"] / ext[n]["us"], 3)
                ceil = floors.get(n, {}).get("ceiling_us", floors[fn].get("ceiling_us"))
                if ceil is not None:
                    ext[n]["ceiling_us"] = ceil
                    ext[n]["of_ceiling"] = round(ceil / ext[n]["us"], 3)

    cpu = None
    if not args.no_cpu:
        print("[bench] timing the CPU oracle sample", file=sys.stderr, flush=True)
        cpu = cpu_baseline(torch, inp, conv_in)

    workload = (f"cfg4: causal_conv1d ({cshp['B']},{cshp['D']},{cshp['S']},W={cshp['W']}) bf16 + Gated DeltaNet "
                f"chunk fwd recompute_w_u->chunk_fwd_h->chunk_fwd_o B={B},T={T},H={H},K={K},V={V},BT=64 bf16")
    line = {
        "metric": METRIC, "value": round(ms_per_step * 1e3, 2), "unit": "µs/call", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "settle_s": round(settled_s, 3),
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded torch CPU generator; BASELINE.json config-4 distributions)",
        "config": {"workload": workload, "parallelism": "single GPU"},
        "kernels": kernels, "roofline": roofline, "cpu_baseline": cpu, "floors": floors, "measured_peaks": peaks,
        "shapes": shapes,
        "shapes_reference": ref_shapes,
        "extensions": ext,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
