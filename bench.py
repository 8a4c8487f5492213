"""Benchmark of the MI355X projection path (one GPU).

Default run (the driver's contract): the BASELINE configs[1] workload — the fused gate-up projection with the
SiLU.mul epilogue, x [288, 5120] bf16 ~ N(0,1), W_gu [2 x 17408, 5120] ~ N(0, 0.02^2), out [288, 17408] bf16 —
as W untimed warm-up steps and then exactly K timed steps, captured in one HIP graph; the graph is replayed --reps
times, each replay between two synchronizations, and the median replay gives the step time. A step is one call of the fused projection over the batch; the weights rotate over two
copies (712 MB), more than the 256 MB Infinity Cache, so every step streams its weights from HBM.

Prints ONE JSON line with the metric, the roofline of the dominant kernel (HIP events on the launch stream), the
CPU baseline (the oracle's torch CPU path on a bounded sample of the same workload, on this host's cores) and the
per-shape table at M = 7 / 64 / 288 / 539 / 2048 for the five projection shapes, and the BASELINE configs[4]
64-layer projection stack at M = 539 (`stack_ms`, `stack_frac`: one graph replay per forward, packed weights).

Other modes (each prints its own JSON lines): --sweep (full M sweep, every shape), --stack (
the 64-layer projection stack at M = 539 in one graph replay), --head (the scoring head GEMV), --vs-hipblaslt
(each planned call against torch F.linear on the same box), --prep (the full-attention in-projection with its prep:
two launches against the fused epilogue).
"""
import argparse
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "bf16 proj GEMM TFLOP/s + HBM GB/s, % roofline, at M=7/288/539 on 1 MI355X"
SHAPE_MS = (7, 64, 288, 539, 2048)   # the north star's M set for the per-shape table


def load():
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    from importlib import import_module
    return pkg, import_module("open_jev_fast_amd.ext"), import_module("open_jev_fast_amd.perf")


PACKED = True   # weights in the library's load-time packed layout (ext.pack_weight); --rowmajor turns it off


def make_weights(N, K, copies, std=0.02, seed=0, dev="cuda"):
    """Seeded weights [N, K], in the packed layout when PACKED (the layout FastProjections loads weights in)."""
    from importlib import import_module
    ext = import_module("open_jev_fast_amd.ext")
    g = torch.Generator(device=dev).manual_seed(seed)
    ws = [(torch.randn(N, K, generator=g, device=dev) * std).bfloat16() for _ in range(copies)]
    return [ext.pack_weight(w) for w in ws] if PACKED else ws


def shape_call(ext, kind, x, w, res=None, w1=None):
    if kind == "plain":
        return lambda: ext.mm(x, w)
    if kind == "silu":
        return lambda: ext.mm_silu_mul(x, w)
    return lambda: ext.mm_residual_rmsnorm(res, x, w, w1, None, 1e-6)


def measure_shape(ext, perf, name, M, iters=20, reps=5):
    N, K, kind = perf.SHAPES[name]
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(M)
    x = torch.randn(M, K, generator=g, device=dev).bfloat16()
    ws = make_weights(N, K, perf.copies_for(N * K * 2), seed=M + 1)
    res = torch.randn(M, N, generator=g, device=dev).bfloat16() if kind == "residual" else None
    w1 = torch.ones(N, device=dev) if kind == "residual" else None
    fns = [shape_call(ext, kind, x, w, res, w1) for w in ws]
    t = perf.gpu_time(fns, iters=iters, reps=reps)
    r = perf.roofline(M, N, K, kind, t)
    del ws
    return r


def cpu_baseline(M, I, K, budget_s=15.0):
    """The oracle's CPU path (the reported CPU baseline: torch.matmul on bf16 CPU tensors + the same SiLU.mul
    epilogue) on a row slice of W_gu sized to about `budget_s` seconds; median of 5 after 2 warm-ups."""
    from oracle import proj_oracle as O
    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(M, K, generator=g).bfloat16()

    def run(rows):
        wg = (torch.randn(rows, K, generator=g) * 0.02).bfloat16()
        wu = (torch.randn(rows, K, generator=g) * 0.02).bfloat16()
        w = torch.cat([wg, wu], 0)
        fn = lambda: O.silu_mul(torch.matmul(x, w.t()))   # noqa: E731
        return fn

    probe_rows = 512
    fn = run(probe_rows)
    fn()
    t0 = time.perf_counter()
    fn()
    t_probe = time.perf_counter() - t0
    rows = int(min(I, max(probe_rows, probe_rows * (budget_s / 7.0) / max(t_probe, 1e-6))))
    rows -= rows % 8
    fn = run(rows)
    for _ in range(2):
        fn()
    ts = []
    for _ in range(5):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    flops = 2.0 * M * (2 * rows) * K
    return {"value": round(flops / t / 1e12, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"gate-up+SiLU.mul M={M} K={K}, {rows} of {I} gate/up row pairs "
                      f"({2 * rows} of {2 * I} W_gu rows), torch CPU bf16 matmul, median of 5 after 2 warm-ups "
                      f"({t * 1e3:.1f} ms per call; os.cpu_count()={os.cpu_count()})"}


def main_default(args, pkg, ext, perf):
    M, I, K = 288, 17408, 5120
    N = 2 * I
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn(M, K, generator=g, device=dev).bfloat16()
    ws = make_weights(N, K, 2, seed=2)
    plan = pkg._lib.plan(M, N, K, pkg._lib.KIND_SILU_MUL | (pkg._lib.KIND_PACKED if PACKED else 0))
    fns = [lambda w=w: ext.mm_silu_mul(x, w) for w in ws]

    # warm-up (untimed), then one graph of exactly K steps
    for i in range(args.warmup):
        fns[i % 2]()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            for i in range(args.steps):
                fns[i % 2]()
    torch.cuda.synchronize()
    graph.replay()  # upload / first replay (untimed)
    torch.cuda.synchronize()
    # untimed replays until the GPU has run the workload for half a second: the clocks settle (the first timed
    # replays of a cold GPU were measured up to 25% slower than the steady state)
    t_end = time.perf_counter() + 0.5
    while time.perf_counter() < t_end:
        graph.replay()
        torch.cuda.synchronize()
    # The K steps are timed REPS times (one replay of the K-step graph each, bracketed by synchronizations); the
    # reported step time is the median replay divided by K. Every replay is reported in `replays_ms`.
    cur = torch.cuda.current_stream()
    reps = []
    for _ in range(max(1, args.reps)):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(cur)
        graph.replay()
        b.record(cur)
        torch.cuda.synchronize()
        reps.append(a.elapsed_time(b))
    ms = statistics.median(reps) / args.steps
    r = perf.roofline(M, N, K, "silu", ms * 1e-3)
    flops, nbytes = perf.work(M, N, K, "silu")

    # Per-launch duration of the dominant kernel: the GEMM launch over the plan's main rows (all W rows but the
    # tail, when the plan has one), timed with HIP events on the stream it is launched on. It is launched alone
    # through the C-ABI with the same tile, split and grid as inside the call: with split-K that is the fp32
    # partial pass (ojx_gemm_splitk_f32), otherwise the GEMM with the fused SiLU.mul epilogue on those rows. For the
    # persistent stream-K family the call is the GEMM plus the launch that sums the split tiles' pieces; the two
    # are timed together (the GEMM cannot be launched without its fixup through the C-ABI), which understates the
    # GEMM's own rate by the fixup's share.
    cur = torch.cuda.current_stream()
    n1 = N - plan.tail_rows
    fam = pkg._lib.tile_info(plan.tile)["family"]
    if plan.splitk > 1 and fam != 5:
        if PACKED:
            raise RuntimeError("the dominant-kernel timing of a split-K packed plan is not implemented")
        dom = [lambda w=w: ext.mm_splitk_f32(x, w[:n1], plan.splitk, tile=plan.tile) for w in ws]
        dom_name = "gemm (split-K partial pass)"
    else:
        dom = [lambda w=w: ext.mm_silu_mul(x, w if PACKED else w[:n1], cfg=(plan.tile, plan.splitk)) for w in ws]
        dom_name = ("persistent stream-K gemm (fused SiLU.mul epilogue) + split-tile fixup, one call of two "
                    "launches" if fam == 5 else "gemm (fused SiLU.mul epilogue)")
    dom_name += f", W rows 0..{n1} of {N}" if plan.tail_rows else ""
    for i in range(4):
        dom[i % 2]()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n_k = 50
    torch.cuda.synchronize()
    ev0.record(cur)
    for i in range(n_k):
        dom[i % 2]()
    ev1.record(cur)
    torch.cuda.synchronize()
    k_s = ev0.elapsed_time(ev1) * 1e-3 / n_k
    kflops, kbytes = perf.work(M, n1, K, "silu")
    bound = r["bound"]
    if bound == "hbm":
        achieved, peak, unit = kbytes / k_s / 1e9, perf.HBM_PEAK / 1e9, "GB/s"
    else:
        achieved, peak, unit = kflops / k_s / 1e12, perf.MFMA_BF16_PEAK / 1e12, "TFLOP/s"
    tkey = f"gate_up_silu_M{M}_tile{plan.tile}_s{plan.splitk}_rows{n1}" + ("_packed" if PACKED else "")
    roof = {"bound": bound, "achieved": round(achieved, 1), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic_from_profiles(tkey),
            "kernel": dom_name, "kernel_us": round(k_s * 1e6, 2), "algorithmic_bytes": kbytes,
            "algorithmic_flops": kflops}
    del ws, fns, dom, graph

    shapes = {}
    if not args.no_shapes:
        for name in perf.SHAPES:
            for m in SHAPE_MS:
                rr = measure_shape(ext, perf, name, m)
                shapes[f"{name}_M{m}"] = {k: round(v, 4) if isinstance(v, float) else v for k, v in rr.items()}
    stack = None if args.no_stack else run_stack(ext, perf, 5)
    cpu = None if args.no_cpu else cpu_baseline(M, I, K)
    line = {
        "metric": METRIC, "value": round(r["tflops"], 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "replays_ms": [round(v, 4) for v in reps], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: seeded x ~ N(0,1), W ~ N(0,0.02^2), bf16; 2 rotating weight copies"
                + ("; weights in the load-time packed layout (ojx_pack_weight)" if PACKED else "; row-major weights"),
        "config": {"workload": "gate_up_silu: BASELINE configs[1], fused gate-up + SiLU.mul, M=288 K=5120 "
                               "I=17408 (W_gu 34816x5120)", "M": M, "N": N, "K": K,
                   "weight_layout": "packed" if PACKED else "row-major",
                   "plan": {"tile": plan.tile, "splitk": plan.splitk, **pkg._lib.tile_info(plan.tile),
                            **({"tail_rows": plan.tail_rows, "tail_tile": plan.tail_tile,
                                "tail_splitk": plan.tail_splitk} if plan.tail_rows else {})}},
        "gbs": round(r["gbs"], 1), "roofline_frac": round(r["frac"], 4),
        "roofline": roof, "cpu_baseline": cpu, "shapes": shapes,
        # BASELINE configs[4] beside the headline: the whole 64-layer projection forward at M = 539
        "stack_ms": None if stack is None else stack["ms"], "stack_frac": None if stack is None else stack["frac"],
        "stack": stack,
    }
    print(json.dumps(line), flush=True)


def traffic_from_profiles(key):
    """HBM bytes per launch of the dominant kernel measured with rocprofv3 --pmc (FETCH_SIZE and WRITE_SIZE passes,
    each scaled by what the counter reads for a copy kernel of known size), recorded in profiles/traffic.json for
    the (shape, tile, split) it was measured on; None when that configuration was not measured."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(key)
    except (OSError, ValueError):
        return None
    return None if rec is None else rec.get("bytes")


def main_sweep(args, pkg, ext, perf):
    Ms = [int(m) for m in args.m.split(",")] if args.m else perf.M_SWEEP
    names = args.shapes.split(",") if args.shapes else list(perf.SHAPES)
    for name in names:
        for m in Ms:
            rr = measure_shape(ext, perf, name, m)
            N, K, kind = perf.SHAPES[name]
            c = pkg._lib.plan(m, N, K, {"plain": 0, "silu": 1, "residual": 2}[kind] | (4 if PACKED else 0))
            print(json.dumps({"shape": name, "M": m, "N": N, "K": K, "tile": c.tile, "splitk": c.splitk,
                              **{k: round(v, 4) if isinstance(v, float) else v for k, v in rr.items()}}), flush=True)


def run_stack(ext, perf, reps):
    """48 linear-attention + 16 full-attention layers, hidden 5120, MLP 17408, M = 539.
    Each layer: in-proj, out-proj + residual + RMSNorm, gate-up + SiLU.mul, down + residual + RMSNorm, back to
    back in one graph (the whole forward is one HIP graph replay; `reps` replays are timed). The attention cores
    between in-proj and out-proj are out of scope: the out-proj reads a fixed activation of the right shape.
    Returns the measurement as a dict."""
    M, H, I = 539, 5120, 17408
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(5)
    std = 0.02
    lin_in, full_in, lin_out_k, full_out_k = 16384, 14336, 6144, 6144
    layers = []
    for i in range(64):
        full = (i % 4) == 3
        n_in = full_in if full else lin_in
        layers.append(dict(
            w_in=(torch.randn(n_in, H, generator=g, device=dev) * std).bfloat16(),
            w_out=(torch.randn(H, full_out_k if full else lin_out_k, generator=g, device=dev) * std).bfloat16(),
            w_gu=(torch.randn(2 * I, H, generator=g, device=dev) * std).bfloat16(),
            w_dn=(torch.randn(H, I, generator=g, device=dev) * std).bfloat16()))
        if PACKED:
            layers[-1] = {k: ext.pack_weight(v) for k, v in layers[-1].items()}
    h0 = torch.randn(M, H, generator=g, device=dev).bfloat16()
    hn0 = torch.randn(M, H, generator=g, device=dev).bfloat16()
    y_att = torch.randn(M, lin_out_k, generator=g, device=dev).bfloat16()
    w1 = torch.ones(H, device=dev)

    def forward():
        h, hn = h0, hn0
        for d in layers:
            ext.mm(hn, d["w_in"])
            h, hn = ext.mm_residual_rmsnorm(h, y_att, d["w_out"], w1, None, 1e-6)
            m = ext.mm_silu_mul(hn, d["w_gu"])
            h, hn = ext.mm_residual_rmsnorm(h, m, d["w_dn"], w1, None, 1e-6)
        return h, hn

    t = perf.gpu_time([forward], iters=1, reps=reps, warmup=2)
    flops = nbytes = 0.0
    for i in range(64):
        full = (i % 4) == 3
        for (N, K, kind) in (((full_in if full else lin_in), H, "plain"), (H, lin_out_k, "residual"),
                             (2 * I, H, "silu"), (H, I, "residual")):
            f, b = perf.work(M, N, K, kind)
            flops += f
            nbytes += b
    t_roof = max(nbytes / perf.HBM_PEAK, flops / perf.MFMA_BF16_PEAK)
    del layers
    torch.cuda.empty_cache()
    return {"stack": "64-layer projection stack (48 lin + 16 full), one graph replay per forward", "M": M,
            "weight_layout": "packed" if PACKED else "row-major", "ms": round(t * 1e3, 3),
            "tflops": round(flops / t / 1e12, 1), "gbs": round(nbytes / t / 1e9, 1),
            "roof_ms": round(t_roof * 1e3, 3), "frac": round(t_roof / t, 4),
            "bound": "hbm" if nbytes / perf.HBM_PEAK >= flops / perf.MFMA_BF16_PEAK else "mfma"}


def main_stack(args, pkg, ext, perf):
    print(json.dumps(run_stack(ext, perf, args.steps)), flush=True)


def main_head(args, pkg, ext, perf):
    """The scoring head (src/server.py:37): scores = hn[lastidx].float() @ w + b over the stack's M = 539 rows, for
    R gathered rows. HBM-bound: algorithmic bytes R*H*2 (gathered rows) + H*4 (w) + R*4 (scores)."""
    rows, H = 539, 5120
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(7)
    hn = torch.randn(rows, H, generator=g, device=dev).bfloat16()
    w = torch.randn(H, generator=g, device=dev) * 0.02
    b = torch.zeros(1, device=dev)
    for R in (1, 16, 128, 539):
        idx = torch.randint(0, rows, (R,), generator=g, device=dev)
        t = perf.gpu_time([lambda: ext.head_scores(hn, idx, w, b)], iters=20, reps=5)
        nbytes = R * H * 2 + H * 4 + R * 4
        print(json.dumps({"head": "scoring head GEMV (gather + 5120 -> 1)", "R": R, "H": H, "us": round(t * 1e6, 2),
                          "gbs": round(nbytes / t / 1e9, 1), "roof_us": round(nbytes / perf.HBM_PEAK * 1e6, 3),
                          "frac": round(nbytes / perf.HBM_PEAK / t, 4)}), flush=True)


def main_prep(args, pkg, ext, perf):
    """The full-attention in-projection and its prep (src/fastmodel.py:412,462): the planned GEMM followed by
    ojx_fullattn_prep (two launches) against ojx_gemm_qkv_fullattn_prep (the prep in the GEMM's epilogue), HQ = 24,
    HKV = 4, D = 256, RoPE dims 64, K = 5120. Each timed as a HIP graph of 10 calls over rotating weight copies."""
    dev = "cuda"
    HQ, HKV, D, RD, K = 24, 4, 256, 64, 5120
    N = (2 * HQ + 2 * HKV) * D
    Ms = [int(m) for m in args.m.split(",")] if args.m else [7, 64, 288, 539, 2048]
    ws = make_weights(N, K, perf.copies_for(N * K * 2), seed=11)
    qw1 = torch.ones(D, device=dev)
    kw1 = torch.ones(D, device=dev)
    for M in Ms:
        x = torch.randn(M, K, device=dev).bfloat16()
        ang = torch.rand(M, RD // 2, device=dev) * 6.0
        cos = torch.cat([ang.cos(), ang.cos()], 1).bfloat16()
        sin = torch.cat([ang.sin(), ang.sin()], 1).bfloat16()
        proj = ext.mm(x, ws[0])
        two = [lambda w=w: ext.fullattn_prep2(ext.mm(x, w), qw1, kw1, cos, sin, 1, M, HQ, HKV, D, 1e-6) for w in ws]
        fused = [lambda w=w: ext.mm_fullattn_prep(x, w, qw1, kw1, cos, sin, HQ, HKV, D, 1e-6, fused=True)
                 for w in ws]
        gemm = [lambda w=w: ext.mm(x, w) for w in ws]
        prep = [lambda: ext.fullattn_prep2(proj, qw1, kw1, cos, sin, 1, M, HQ, HKV, D, 1e-6)]
        t = {k: min(perf.gpu_time(f, iters=10, reps=3), perf.gpu_time(f, iters=10, reps=3))
             for k, f in (("gemm", gemm), ("prep", prep), ("two_launch", two), ("fused", fused))}
        print(json.dumps({"prep": "full-attention in-projection + prep", "M": M, "N": N, "K": K,
                          **{k + "_us": round(v * 1e6, 1) for k, v in t.items()},
                          "prep_roof_us": round(4 * M * N / perf.HBM_PEAK * 1e6, 2)}), flush=True)
    del ws
    # linear-attention prep on a tree of S candidate paths: a shared prompt of Lr rows, then one leaf of lf rows per
    # path (the packed rows are the prompt and the leaves; every prompt row is written to S slots)
    import numpy as np
    HK, HV, HD = 16, 48, 128
    KD, VD = HK * HD, HV * HD
    C, P = 2 * KD + VD, 2 * KD + 2 * VD + 2 * HV
    for Lr, S, lf in ((200, 8, 11), (480, 8, 7), (1800, 16, 15)):
        N = -(-(Lr + S * lf) // 32) * 32
        L2 = -(-(Lr + lf) // 16) * 16
        src = np.full((S, L2), -1, np.int32)
        for c in range(S):
            src[c, :Lr] = np.arange(Lr)
            src[c, Lr:Lr + lf] = Lr + c * lf + np.arange(lf)
        flat = src.reshape(-1)
        grp = np.where(flat >= 0, flat, N)
        rep_pos = np.argsort(grp, kind="stable").astype(np.int32)
        rep_ptr = np.concatenate([[0], np.cumsum(np.bincount(grp, minlength=N + 1))]).astype(np.int32)
        hist = np.full((N + 1, 4), -1, np.int32)
        for c in range(S):
            for t_ in range(Lr + lf):
                hist[src[c, t_]] = [src[c, t_ - 3 + i] if t_ - 3 + i >= 0 else -1 for i in range(4)]
        d = lambda a: torch.as_tensor(a).to(dev).contiguous()  # noqa: E731
        proj = torch.randn(N, P, device=dev).bfloat16()
        convw = (torch.randn(C, 4, device=dev) * 0.5).bfloat16()
        A_log = torch.randn(HV, device=dev).bfloat16()
        dt_bias = torch.randn(HV, device=dev).bfloat16()
        args = (proj, d(hist), d(rep_ptr), d(rep_pos), L2, convw, A_log, dt_bias, KD, VD, HV, HK, HD, False)
        fn = [lambda: ext.linattn_prep_dedup2(*args)]
        tl = min(perf.gpu_time(fn, iters=10, reps=3), perf.gpu_time(fn, iters=10, reps=3))
        R = S * L2
        nbytes = (Lr + S * lf) * (C + 2 * HV) * 2 + C * 8 + R * (C * 2 + HV * 6)   # rows read once, slots written
        print(json.dumps({"prep": "linear-attention prep (tree layout)", "rows": Lr + S * lf, "paths": S, "slots": R,
                          "us": round(tl * 1e6, 1), "gbs": round(nbytes / tl / 1e9, 1),
                          "roof_us": round(nbytes / perf.HBM_PEAK * 1e6, 2),
                          "frac": round(nbytes / perf.HBM_PEAK / tl, 3)}), flush=True)


def main_vs_hipblaslt(args, pkg, ext, perf):
    """This build's planned call against torch F.linear (hipBLASLt) on the same box, in one process: each timed as a
    HIP graph of 10 calls over the same rotating weight copies (perf.gpu_time), best of two measurements. The ojx
    call includes its fused epilogue (SiLU.mul, or residual + RMSNorm); the hipBLASLt time is the GEMM alone, and
    for the fused shapes also the GEMM followed by this build's epilogue kernel (silu_mul / add_rmsnorm), the
    reference's own two-launch structure."""
    dev = "cuda"
    Ms = [int(m) for m in args.m.split(",")] if args.m else [7, 288, 539, 1024, 2048]
    names = args.shapes.split(",") if args.shapes else list(perf.SHAPES)
    for name in names:
        N, K, kind = perf.SHAPES[name]
        ws = [(torch.randn(N, K, device=dev) * 0.02).bfloat16() for _ in range(perf.copies_for(N * K * 2))]
        wo = [ext.pack_weight(w) for w in ws] if PACKED else ws   # the layout this build loads weights in
        for M in Ms:
            x = torch.randn(M, K, device=dev).bfloat16()
            res = torch.randn(M, N, device=dev).bfloat16()
            w1 = torch.ones(N, device=dev)
            blas = [lambda w=w: torch.nn.functional.linear(x, w) for w in ws]
            if kind == "plain":
                ours = [lambda w=w: ext.mm(x, w) for w in wo]
            elif kind == "silu":
                ours = [lambda w=w: ext.mm_silu_mul(x, w) for w in wo]
            else:
                ours = [lambda w=w: ext.mm_residual_rmsnorm(res, x, w, w1, None, 1e-6) for w in wo]
            t_b = min(perf.gpu_time(blas, iters=10, reps=3), perf.gpu_time(blas, iters=10, reps=3))
            t_o = min(perf.gpu_time(ours, iters=10, reps=3), perf.gpu_time(ours, iters=10, reps=3))
            extra = {}
            if kind != "plain":  # the same epilogue after the hipBLASLt GEMM, as the reference runs it (two launches)
                if kind == "silu":
                    full = [lambda w=w: ext.silu_mul(torch.nn.functional.linear(x, w)) for w in ws]
                else:
                    full = [lambda w=w: ext.add_rmsnorm(res, torch.nn.functional.linear(x, w), w1, None, 1e-6)
                            for w in ws]
                t_f = min(perf.gpu_time(full, iters=10, reps=3), perf.gpu_time(full, iters=10, reps=3))
                extra = {"hipblaslt_gemm_epilogue_us": round(t_f * 1e6, 1), "ratio_with_epilogue": round(t_f / t_o, 3)}
            print(json.dumps({"shape": name, "M": M, "N": N, "K": K, "epilogue": kind, "ojx_us": round(t_o * 1e6, 1),
                              "hipblaslt_gemm_us": round(t_b * 1e6, 1), "ratio": round(t_b / t_o, 3), **extra}),
                  flush=True)
        del ws, wo
        torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--reps", type=int, default=7, help="replays of the K-step graph; the median is reported")
    ap.add_argument("--sweep", action="store_true")
    ap.add_argument("--stack", action="store_true")
    ap.add_argument("--head", action="store_true")
    ap.add_argument("--vs-hipblaslt", action="store_true")
    ap.add_argument("--prep", action="store_true")
    ap.add_argument("--m", default="")
    ap.add_argument("--shapes", default="")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-shapes", action="store_true")
    ap.add_argument("--no-stack", action="store_true", help="leave out the 64-layer stack (configs[4]) keys")
    ap.add_argument("--rowmajor", action="store_true", help="row-major weights instead of the packed layout")
    args = ap.parse_args()
    ws = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or ws != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (the projections would shard as "
              "column/row tensor parallelism; see the design notes). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    pkg, ext, perf = load()
    global PACKED
    PACKED = not args.rowmajor
    if args.sweep:
        main_sweep(args, pkg, ext, perf)
    elif args.stack:
        main_stack(args, pkg, ext, perf)
    elif args.head:
        main_head(args, pkg, ext, perf)
    elif args.vs_hipblaslt:
        main_vs_hipblaslt(args, pkg, ext, perf)
    elif args.prep:
        main_prep(args, pkg, ext, perf)
    else:
        main_default(args, pkg, ext, perf)


if __name__ == "__main__":
    main()
