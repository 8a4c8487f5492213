"""Measurement helpers for the projection path: MI355X peaks, algorithmic work per call, and GPU timing.

Algorithmic work per call (fp32 partials and workspace are not counted):
    flops   = 2 M N K                       (gate-up: N = 2I, the SiLU.mul flops are ignored)
    bytes   plain     2 (M K + N K + M N)
            gate-up   2 (M K + N K + M N / 2)
            residual  2 (M K + N K) + 2 M N (residual read) + 2 M N (h write) [+ 2 M N if hn is written]
Roofline time t = max(bytes / HBM peak, flops / MFMA peak); fraction = t / measured.
"""
import time

import torch

HBM_PEAK = 8.0e12         # B/s, MI355X HBM3E
MFMA_BF16_PEAK = 2.5e15   # flop/s, dense bf16 MFMA (no sparsity)

# projection shapes (N, K) of the 27B hybrid forward; gate-up N is the packed 2 I
SHAPES = {
    "qkv": (14336, 5120, "plain"),
    "gate_up": (34816, 5120, "silu"),
    "down": (5120, 17408, "residual"),
    "o_proj": (5120, 6144, "residual"),
    "lin_in": (16384, 5120, "plain"),
}
M_SWEEP = (1, 7, 16, 64, 128, 288, 539, 1024, 2048)


def work(M, N, K, kind, hn=True):
    flops = 2.0 * M * N * K
    if kind == "plain":
        b = 2.0 * (M * K + N * K + M * N)
    elif kind == "silu":
        b = 2.0 * (M * K + N * K + M * N / 2)
    else:
        b = 2.0 * (M * K + N * K) + 4.0 * M * N + (2.0 * M * N if hn else 0.0)
    return flops, b


def roofline(M, N, K, kind, seconds, hn=True):
    flops, b = work(M, N, K, kind, hn)
    t_hbm, t_mfma = b / HBM_PEAK, flops / MFMA_BF16_PEAK
    t_roof = max(t_hbm, t_mfma)
    return {
        "us": seconds * 1e6,
        "tflops": flops / seconds / 1e12,
        "gbs": b / seconds / 1e9,
        "bound": "hbm" if t_hbm >= t_mfma else "mfma",
        "roof_us": t_roof * 1e6,
        "frac": t_roof / seconds,
    }


def gpu_time(fns, iters=20, reps=5, warmup=2, graph=True, settle=0.2):
    """Average seconds per call of fns[i % len(fns)] (fns rotate over weight copies so each call streams its
    weights from HBM rather than the 256 MB Infinity Cache). Calls are captured in a HIP graph of `iters` calls
    (as bench/lt_search.py:14-27 does) and timed over `reps` replays with events on the current stream, after
    `settle` seconds of untimed replays (a GPU that was idle runs its first replays at lower clocks: measured
    up to 8% slower on the gate-up at M = 288)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(warmup * len(fns)):
            fns[i % len(fns)]()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(iters):
                fns[i % len(fns)]()
        g.replay()
        torch.cuda.synchronize()
        run = g.replay
    else:
        def run():
            for i in range(iters):
                fns[i % len(fns)]()
    t_end = time.perf_counter() + settle
    while time.perf_counter() < t_end:
        run()
        torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        run()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e-3 / (reps * iters)


def copies_for(nbytes, cache=256 << 20, minimum=2):
    """Number of rotating weight copies so that the rotation set exceeds the Infinity Cache twice over."""
    return max(minimum, int(-(-2 * cache // max(nbytes, 1))))
