"""GPU parity of the one-launch split-K plans (ojx_cfg.one_launch, tile families 0 and 6), through the C-ABI.

one_launch = 1: the last split of each tile to finish sums the fp32 planes in split order and applies the epilogue
inside the GEMM launch (the residual kind ends with h; a second launch normalises h). one_launch = 2 (family 0,
residual): the last tile of each row block to finish also normalises the block's rows (the reference's separate
add_rmsnorm_sk2 launch, src/kernels.cu:1444-1501, src/fastmodel.py:196-203). Checked:
* y (plain), out (SiLU.mul), h and hn (residual, one_launch = 1) equal the two-launch path with the same tile and
  split bit for bit (the same sums in the same order); under one_launch = 2, hn within one bf16 rounding step (its
  sum of squares is added in another order) and mostly equal; masked rows zero;
* row-major and packed weights, ragged M / N / K (M over several M tiles too, and past 256 rows in the
  288-row tiles, whose 256 threads each take more than one row of the RMSNorm pass), splits 2 .. 16;
* back-to-back calls and HIP graph replays (the arrival counters re-arm themselves);
* the north star's tolerance against the oracle at full size (o_proj, down, QKV, gate-up at M = 1 / 7 / 16).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = dict(max_rel=1e-2, mean_abs_rms=1e-3)


def _say(*a):
    print(*a, flush=True)


def _one_launch_tiles(pkg):
    L = pkg._lib
    return [t for t in range(L.lib().ojx_num_tiles()) if L.tile_info(t)["family"] in (0, 6)]


def _close_hn(got, want, what):
    g, w = got.float().cpu(), want.float().cpu()
    err = (g - w).abs()
    bound = w.abs() * 2.0 ** -7 + 1e-30
    assert bool((err <= bound).all()), f"{what}: {(err - bound).max().item():.3e} above one step"
    assert (err == 0).float().mean().item() > 0.95, f"{what}: too few equal values"


def _inputs(M, N, K, seed, dev):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16().to(dev)
    w = (torch.randn(N, K, generator=g) * K ** -0.5).bfloat16().to(dev)
    res = torch.randn(M, N, generator=g).bfloat16().to(dev)
    w1 = (1.0 + 0.1 * torch.randn(N, generator=g)).float().to(dev)
    mask = (torch.rand(M, generator=g) > 0.3).int().to(dev)
    return x, w, res, w1, mask


_EQ_SHAPES = [(1, 1040, 640), (7, 264, 1024), (16, 528, 768), (37, 1040, 1152), (150, 1040, 1152), (300, 264, 1024)]


# packed weights need N % 16 == 0 and K % 64 == 0: the N = 264 shapes run row-major only
@pytest.mark.parametrize("M,N,K,packed", [s + (pk,) for s in _EQ_SHAPES for pk in (False, True)
                                          if not pk or (s[1] % 16 == 0 and s[2] % 64 == 0)])
def test_one_launch_equals_two_launches(pkg, ext, dev, M, N, K, packed):
    x, w, res, w1, mask = _inputs(M, N, K, M + N + K, dev)
    wu = ext.pack_weight(w) if packed else None
    mm = ext.mm_pk if packed else ext.mm
    mmr = ext.mm_residual_rmsnorm_pk if packed else ext.mm_residual_rmsnorm
    mms = ext.mm_silu_mul_pk if packed else ext.mm_silu_mul
    W = wu if packed else w
    for t in _one_launch_tiles(pkg):
        fam = pkg._lib.tile_info(t)["family"]
        for S in ((2, 3, 8, 16) if fam == 0 else (2, 3)):
            two, one = (t, S, 0, 1, 0, 0), (t, S, 0, 1, 0, 1)
            _say(f"case one-launch M={M} N={N} K={K} packed={packed} tile={t} S={S}")
            try:
                ref = mm(x, W, cfg=two)
            except RuntimeError as e:
                assert "invalid" in str(e), str(e)  # a split that leaves a K range empty (or a packed stage cut)
                with pytest.raises(RuntimeError):
                    mm(x, W, cfg=one)
                continue
            assert torch.equal(mm(x, W, cfg=one), ref), f"plain tile {t} S {S}"
            assert torch.equal(mms(x, W, cfg=one), mms(x, W, cfg=two)), f"silu tile {t} S {S}"
            for m in (None, mask):
                h2, hn2 = mmr(res, x, W, w1, m, 1e-6, cfg=two)
                h1, hn1 = mmr(res, x, W, w1, m, 1e-6, cfg=one)
                torch.cuda.synchronize()
                assert torch.equal(h1, h2) and torch.equal(hn1, hn2), f"residual tile {t} S {S}"
                h3 = mmr(res, x, W, w1, None, 1e-6, want_hn=False, cfg=one)[0]
                assert torch.equal(h3, h2 if m is None else mmr(res, x, W, w1, None, 1e-6, cfg=two)[0])
                if fam != 0:
                    continue
                fold = (t, S, 0, 1, 0, 2)
                hf, hnf = mmr(res, x, W, w1, m, 1e-6, cfg=fold)
                assert torch.equal(hf, h2), f"fold h tile {t} S {S}"
                _close_hn(hnf, hn2, f"fold hn tile {t} S {S} mask {m is not None}")
                if m is not None:
                    assert bool((hnf[m == 0] == 0).all())
        if fam == 6:  # the fold is family 0's only
            with pytest.raises(RuntimeError, match="invalid"):
                mmr(res, x, W, w1, None, 1e-6, cfg=(t, 2, 0, 1, 0, 2))


def test_one_launch_repeats_and_graph(pkg, ext, dev):
    """The counters re-arm: many calls in a row, several shapes interleaved, and graph replays all give the first
    call's bits."""
    x, w, res, w1, _ = _inputs(7, 5120, 6144, 11, dev)
    x2, w2, res2, w12, _ = _inputs(3, 1040, 1024, 12, dev)
    one = (0, 8, 0, 1, 0, 2)
    h0, hn0 = ext.mm_residual_rmsnorm(res, x, w, w1, None, 1e-6, cfg=one)
    y0 = ext.mm(x2, w2, cfg=(0, 4, 0, 1, 0, 1))
    h0, hn0, y0 = h0.clone(), hn0.clone(), y0.clone()
    for i in range(20):
        h, hn = ext.mm_residual_rmsnorm(res, x, w, w1, None, 1e-6, cfg=one)
        y = ext.mm(x2, w2, cfg=(0, 4, 0, 1, 0, 1))
        assert torch.equal(h, h0) and torch.equal(hn, hn0) and torch.equal(y, y0), f"call {i}"
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ext.mm_residual_rmsnorm(res, x, w, w1, None, 1e-6, cfg=one)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gh, ghn = ext.mm_residual_rmsnorm(res, x, w, w1, None, 1e-6, cfg=one)
        gy = ext.mm(x2, w2, cfg=(0, 4, 0, 1, 0, 1))
    for r in range(4):
        _say(f"case one-launch graph replay {r}")
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(gh, h0) and torch.equal(ghn, hn0) and torch.equal(gy, y0), f"replay {r}"
        ext.mm(x2, w2, cfg=(0, 4, 0, 1, 0, 1))  # eager work between replays
        torch.cuda.synchronize()
    del g


@pytest.mark.parametrize("shape", ["o_proj", "down", "qkv", "gate_up"])
@pytest.mark.parametrize("M", [1, 7, 16])
def test_one_launch_full_size_vs_oracle(pkg, ext, O, dev, shape, M):
    from importlib import import_module
    perf = import_module("open_jev_fast_amd.perf")
    N, K, kind = perf.SHAPES[shape]
    _say(f"case one-launch full size {shape} M={M}")
    x, w, res, w1, _ = _inputs(M, N, K, 3 * M + N, dev)
    wp = ext.pack_weight(w)
    S = 8
    one = (0, S, 0, 1, 0, 2 if kind == "residual" else 1)
    xc, wc = x.cpu(), w.cpu()
    if kind == "plain":
        got = ext.mm_pk(x, wp, cfg=one)
        ok, a, b = O.tolerance_ok(got.float().cpu(), O.linear_bf16(xc, wc).float(), **TOL)
        assert ok, (a, b)
    elif kind == "silu":
        got = ext.mm_silu_mul_pk(x, wp, cfg=one)
        assert torch.equal(got, ext.mm_silu_mul_pk(x, wp, cfg=(0, S, 0, 1, 0, 0)))
        gu = O.linear_bf16(xc, wc).float().view(M, N // 8, 2, 4)
        gate, up = gu[:, :, 0].reshape(M, N // 2), gu[:, :, 1].reshape(M, N // 2)
        ref = (torch.nn.functional.silu(gate).bfloat16().float() * up).bfloat16()
        ok, a, b = O.tolerance_ok(got.float().cpu(), ref.float(), **TOL)
        assert ok, (a, b)
    else:
        h, hn = ext.mm_residual_rmsnorm_pk(res, x, wp, w1, None, 1e-6, cfg=one)
        rh, rhn = O.residual_proj(res.cpu(), xc, wc, w1.cpu(), None, 1e-6, S=S)
        for got, ref, nm in ((h, rh, "h"), (hn, rhn, "hn")):
            ok, a, b = O.tolerance_ok(got.float().cpu(), ref.float(), **TOL)
            assert ok, (nm, a, b)


def test_one_launch_plans_on_concurrent_streams(pkg, ext, dev):
    """Four streams run one-launch plans at the same time: each stream's 24 calls are captured in a HIP graph on that
    stream, and the four graphs are replayed together, so their kernels overlap on the GPU. Each stream has its own
    set of the library's arrival counters (and ext its own workspace), so every result equals the same call run
    alone, bit for bit, on every replay. Plain (families 0 and 6) and residual with the RMSNorm fold."""
    L = pkg._lib
    shapes = [(64, 2048, 4096, 0, 0), (64, 4096, 2048, 0, 6), (128, 1024, 4096, 2, 0), (7, 3072, 3072, 0, 0)]
    calls = []
    for i, (M, N, K, kind, fam) in enumerate(shapes):
        x, w, res, w1, mask = _inputs(M, N, K, 100 + i, dev)
        ol = 2 if kind == 2 else 1
        cfg = next(c for c in L.candidates(M, N, K, kind)
                   if c.one_launch == ol and c.splitk >= 3 and L.tile_info(c.tile)["family"] == fam)
        if kind == 2:
            calls.append((f"residual {M}x{N}x{K} {cfg}",
                          lambda x=x, w=w, res=res, w1=w1, mask=mask, cfg=cfg:
                          torch.cat(ext.mm_residual_rmsnorm(res, x, w, w1, mask, 1e-6, cfg=cfg), 1)))
        else:
            calls.append((f"plain {M}x{N}x{K} {cfg}", lambda x=x, w=w, cfg=cfg: ext.mm(x, w, cfg=cfg)))
    alone = []
    for what, f in calls:
        _say(f"case streams alone {what}")
        alone.append(f())
        torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=dev) for _ in calls]
    graphs, outs = [], []
    for i, (what, f) in enumerate(calls):
        _say(f"case streams capture {what}")
        with torch.cuda.stream(streams[i]):
            f()  # eager first on this stream: its workspace exists before the capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=streams[i]):
            outs.append([f() for _ in range(24)])
        graphs.append(g)
    torch.cuda.synchronize()
    for rep in range(3):
        _say(f"case streams concurrent replay {rep}")
        for o in outs:
            for t in o:
                t.zero_()
        cur = torch.cuda.current_stream(dev)
        for i, g in enumerate(graphs):
            streams[i].wait_stream(cur)
            with torch.cuda.stream(streams[i]):
                g.replay()
        torch.cuda.synchronize()
        for i, (what, _) in enumerate(calls):
            for r, o in enumerate(outs[i]):
                assert torch.equal(o, alone[i]), f"{what}: replay {rep}, call {r} differs from the call run alone"
