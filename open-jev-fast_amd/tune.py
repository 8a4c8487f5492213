"""Offline tuner: measures every (tile, split-K) candidate for the projection shapes on this GPU and writes the
plan table (csrc/plan_table.inc) that ojx_plan() reads. Replaces the reference's per-shape cuBLASLt searches
(_tune src/fastmodel.py:114-132, bench/lt_search.py) with a one-time offline sweep, so nothing is timed at run
time or during graph capture.

    python open-jev-fast_amd/tune.py --out /tmp/plan_table.inc [--m 7,288] [--shapes gate_up,down]

Each candidate is timed by graph replay over rotating weight copies (larger than the Infinity Cache); the winner
is checked against a torch fp32 GEMM on the GPU before it is accepted (max rel 1e-2, mean |d| <= 1e-3 RMS).
"""
import argparse
import json
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

KIND_ID = {"plain": 0, "silu": 1, "residual": 2}
TUNE_SHAPES = {  # name: (N, K, kind); gate-up N is the packed 2 I
    "qkv": (14336, 5120, "plain"),
    "lin_in": (16384, 5120, "plain"),
    "lin_in_real": (16480, 5120, "plain"),
    "c1_5120": (5120, 5120, "plain"),
    "gate_up": (34816, 5120, "silu"),
    "down": (5120, 17408, "residual"),
    "o_proj": (5120, 6144, "residual"),
}
M_DEFAULT = (1, 7, 16, 64, 128, 288, 539, 1024, 2048)


def main():
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    from importlib import import_module
    ext = import_module("open_jev_fast_amd.ext")
    perf = import_module("open_jev_fast_amd.perf")
    _lib = pkg._lib

    ap = argparse.ArgumentParser()
    ap.add_argument("--m", default="")
    ap.add_argument("--shapes", default="")
    ap.add_argument("--out", default="")
    ap.add_argument("--iters", type=int, default=10)
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--all", action="store_true", help="print every candidate's time")
    ap.add_argument("--tiles", default="", help="only these tile ids")
    ap.add_argument("--max-waves", type=float, default=16.0, help="skip candidates with more workgroups than this "
                    "many per CU")
    ap.add_argument("--no-tails", action="store_true", help="simple (tile, split-K) candidates only")
    ap.add_argument("--sk-splits", default="1,2,3,4,6,8", help="stream-K spreads tried for the persistent family")
    ap.add_argument("--packed", action="store_true", help="tune the packed-weight entry points (kind | 4; the "
                    "weights go through ojx_pack_weight, the K-interleaved family runs them)")
    args = ap.parse_args()
    Ms = [int(m) for m in args.m.split(",")] if args.m else list(M_DEFAULT)
    sk_splits = {int(v) for v in args.sk_splits.split(",")}
    names = args.shapes.split(",") if args.shapes else list(TUNE_SHAPES)
    rows = []
    dev = "cuda"
    for name in names:
        N, K, kind = TUNE_SHAPES[name]
        kid = KIND_ID[kind] | (_lib.KIND_PACKED if args.packed else 0)
        ws_rm = [(torch.randn(N, K, device=dev) * 0.02).bfloat16() for _ in range(perf.copies_for(N * K * 2))]
        ws = [ext.pack_weight(w) for w in ws_rm] if args.packed else ws_rm
        for M in Ms:
            x = torch.randn(M, K, device=dev).bfloat16()
            res = torch.randn(M, N, device=dev).bfloat16() if kind == "residual" else None
            w1 = torch.ones(N, device=dev)

            mm, mm_silu, mm_res = ((ext.mm_pk, ext.mm_silu_mul_pk, ext.mm_residual_rmsnorm_pk) if args.packed else
                                   (ext.mm, ext.mm_silu_mul, ext.mm_residual_rmsnorm))

            def call(w, c):
                if kind == "plain":
                    return lambda: mm(x, w, cfg=c)
                if kind == "silu":
                    return lambda: mm_silu(x, w, cfg=c)
                return lambda: mm_res(res, x, w, w1, None, 1e-6, cfg=c)

            results = []
            only = {int(t) for t in args.tiles.split(",")} if args.tiles else None

            def timed(key):
                try:
                    cc = _lib.cfg(*key)
                    t = perf.gpu_time([call(w, cc) for w in ws], iters=args.iters, reps=args.reps, settle=0.05)
                except RuntimeError as e:
                    print(json.dumps({"shape": name, "M": M, "cfg": key, "error": str(e)}), flush=True)
                    return
                results.append((t, key))

            for c in _lib.candidates(M, N, K, kid):
                if only is not None and c.tile not in only:
                    continue
                info = _lib.tile_info(c.tile)
                if info["family"] == 5:  # persistent: one workgroup per CU; splitk is the stream-K spread
                    if c.splitk not in sk_splits:
                        continue
                else:
                    wgs = -(-N // info["bn"]) * -(-M // info["bm"]) * c.splitk
                    if wgs > args.max_waves * 256:
                        continue
                timed((c.tile, c.splitk, 0, 1, 0, c.one_launch))
            if kind != "residual" and not args.no_tails and not args.packed:
                # tail configurations: the best simple tiles over whole rounds of 256 workgroups, the leftover
                # rows with a finer tile
                simple = sorted(results)
                mains, seen = [], []
                for t, key in simple:
                    if len(seen) == 4:
                        break
                    if key[0] not in seen and _lib.tile_info(key[0])["family"] != 5 and not key[5]:
                        seen.append(key[0])
                        mains += [(key[0], 1), (key[0], 2)]
                tails = [c for c in _lib.candidates(M, N, K, kid) if c.splitk <= 4 and (only is None or c.tile in only)
                         and _lib.tile_info(c.tile)["family"] != 5]
                for tile, S in mains:
                    info = _lib.tile_info(tile)
                    per_tile = -(-M // info["bm"]) * S
                    tiles_n = -(-N // info["bn"])
                    rounds = tiles_n * per_tile // 256
                    n1 = (rounds * 256 // per_tile) * info["bn"]
                    tr = N - n1
                    if rounds == 0 or tr <= 0 or tr % 8 or tiles_n * per_tile % 256 == 0:
                        continue
                    for c in tails:
                        ti = _lib.tile_info(c.tile)
                        if -(-tr // ti["bn"]) * -(-M // ti["bm"]) * c.splitk > 512:
                            continue
                        timed((tile, S, c.tile, c.splitk, tr, 0))
            results.sort()
            # accept the fastest candidate whose numerics pass
            ref = None
            best = None
            for t, key in results[:5]:
                cc = _lib.cfg(*key)
                w = ws[0]
                wr = ws_rm[0]
                if kind == "plain":
                    out = mm(x, w, cfg=cc).float()
                    ref = (x.float() @ wr.float().t()).bfloat16().float()
                elif kind == "silu":
                    out = mm_silu(x, w, cfg=cc).float()
                    gu = (x.float() @ wr.float().t()).view(M, N // 8, 2, 4)
                    g, u = gu[:, :, 0].reshape(M, N // 2), gu[:, :, 1].reshape(M, N // 2)
                    g, u = g.bfloat16().float(), u.bfloat16().float()
                    ref = ((g / (1 + torch.exp(-g))).bfloat16().float() * u).bfloat16().float()
                else:
                    out = mm_res(res, x, w, w1, None, 1e-6, want_hn=False, cfg=cc)[0].float()
                    ref = (res.float() + (x.float() @ wr.float().t()).bfloat16().float()).bfloat16().float()
                d = (out - ref).abs()
                ok = (d.max() / ref.abs().max() <= 1e-2) and (d.mean() <= 1e-3 * ref.pow(2).mean().sqrt())
                if bool(ok):
                    best = (t, key)
                    break
                print(json.dumps({"shape": name, "M": M, "cfg": key, "numerics": "FAIL"}), flush=True)
            top = [{"us": round(t * 1e6, 2), "tile": k[0], "splitk": k[1], **({"tail": k[2:5]} if k[4] else {}),
                    **({"one_launch": 1} if k[5] else {})}
                   for t, k in (results if args.all else results[:6])]
            if best is None:
                print(json.dumps({"shape": name, "M": M, "error": "no valid candidate", "top": top}), flush=True)
                continue
            t, key = best
            r = perf.roofline(M, N, K, kind, t)
            print(json.dumps({"shape": name, "M": M, "N": N, "K": K, "kind": kind, "tile": key[0],
                              "splitk": key[1], "tail": key[2:5], "one_launch": key[5], "us": round(t * 1e6, 2),
                              "frac": round(r["frac"], 4), "tflops": round(r["tflops"], 1),
                              "gbs": round(r["gbs"], 1), "top": top}), flush=True)
            rows.append((M, N, K, kid, key, t))
        del ws, ws_rm
        torch.cuda.empty_cache()
    if args.out:
        with open(args.out, "w") as f:
            f.write("// {M, N, K, kind, tile, splitk, tail_tile, tail_splitk, tail_rows, one_launch} measured by "
                    "open-jev-fast_amd/tune.py on MI355X (us in comment)\n")
            for M, N, K, kid, key, t in rows:
                f.write(f"{{{M}, {N}, {K}, {kid}, {', '.join(str(v) for v in key)}}},  // {t * 1e6:.1f} us\n")


if __name__ == "__main__":
    main()
