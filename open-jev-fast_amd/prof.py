"""Runs one projection configuration repeatedly, for rocprofv3 (kernel traces and --pmc counter passes).

    rocprofv3 --kernel-trace --stats -d /tmp/prof -- python3 open-jev-fast_amd/prof.py --shape gate_up --m 288
    rocprofv3 --pmc FETCH_SIZE -d /tmp/pmc -- python3 open-jev-fast_amd/prof.py --shape gate_up --m 288
    python3 open-jev-fast_amd/prof.py --copy-mb 512     # plain copy kernel, to calibrate FETCH_SIZE / WRITE_SIZE
    (--packed: weights in the packed layout of ext.pack_weight, the layout bench.py uses by default; --zero-w:
    all-zero weights, to see how much of a kernel's time depends on the operands' values)

Shapes are those of open_jev_fast_amd.perf.SHAPES (plus any --n/--k override); weights rotate over copies larger
than the Infinity Cache so each call streams its weights from HBM.
"""
import argparse
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--shape", default="gate_up")
    ap.add_argument("--m", type=int, default=288)
    ap.add_argument("--n", type=int, default=0)
    ap.add_argument("--k", type=int, default=0)
    ap.add_argument("--tile", type=int, default=-1)
    ap.add_argument("--splitk", type=int, default=1)
    ap.add_argument("--one-launch", type=int, default=0, help="with --tile: the one-launch split-K variant")
    ap.add_argument("--calls", type=int, default=40)
    ap.add_argument("--copy-mb", type=int, default=0)
    ap.add_argument("--packed", action="store_true", help="weights in the packed layout (ext.pack_weight)")
    ap.add_argument("--zero-w", action="store_true", help="all-zero weights: the same data movement and MFMA "
                    "count with operands that draw less power (the clock's dependence on the data)")
    args = ap.parse_args()
    if args.copy_mb:
        n = args.copy_mb << 20
        a = torch.ones(n // 4, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(args.calls):
            b.copy_(a)
        torch.cuda.synchronize()
        print(f"copied {args.copy_mb} MiB x {args.calls}", flush=True)
        return
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    from importlib import import_module
    ext = import_module("open_jev_fast_amd.ext")
    perf = import_module("open_jev_fast_amd.perf")
    N, K, kind = perf.SHAPES[args.shape]
    N, K = args.n or N, args.k or K
    M = args.m
    cfg = pkg._lib.cfg(args.tile, args.splitk, one_launch=args.one_launch) if args.tile >= 0 else None
    x = torch.randn(M, K, device="cuda").bfloat16()
    ws = [(torch.randn(N, K, device="cuda") * (0.0 if args.zero_w else 0.02)).bfloat16()
          for _ in range(perf.copies_for(N * K * 2))]
    if args.packed:
        ws = [ext.pack_weight(w) for w in ws]
    res = torch.randn(M, N, device="cuda").bfloat16()
    w1 = torch.ones(N, device="cuda")
    for i in range(args.calls):
        w = ws[i % len(ws)]
        if kind == "plain":
            ext.mm(x, w, cfg=cfg)
        elif kind == "silu":
            ext.mm_silu_mul(x, w, cfg=cfg)
        else:
            ext.mm_residual_rmsnorm(res, x, w, w1, None, 1e-6, cfg=cfg)
    torch.cuda.synchronize()
    c = cfg or pkg._lib.plan(M, N, K, {"plain": 0, "silu": 1, "residual": 2}[kind] | (4 if args.packed else 0))
    print(f"{args.shape} M={M} N={N} K={K} tile={c.tile} splitk={c.splitk} calls={args.calls}", flush=True)


if __name__ == "__main__":
    main()
