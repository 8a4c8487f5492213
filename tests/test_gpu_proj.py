"""GPU parity of the projection kernels against the CPU oracle, through the C-ABI (libojx.so via ctypes).

Tolerance: max |out - ref| / max |ref| <= 1e-2 and mean |out - ref| <= 1e-3 * RMS(ref).
Integer-like invariants (gate/up merge, tile invariance, determinism, graph replays) are checked bit-exactly.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = dict(max_rel=1e-2, mean_abs_rms=1e-3)


def _say(*a):
    print(*a, flush=True)


def _tiles(pkg):  # the live tiles (a retired id reports family -1 and is never planned or launched)
    return [t for t in range(pkg._lib.lib().ojx_num_tiles()) if pkg._lib.tile_info(t)["family"] >= 0]


def _assert_tol(O, out, ref, what):
    ok, a, b = O.tolerance_ok(out.float().cpu(), ref.float().cpu(), **TOL)
    assert ok, f"{what}: max_rel {a:.3e} mean/rms {b:.3e}"


# ----------------------------------------------------------------------------------------------- plain GEMM
SMALL = [(1, 64, 64), (7, 128, 256), (16, 256, 512), (37, 200, 328), (96, 520, 640), (288, 512, 1024),
         (300, 264, 136)]


@pytest.mark.parametrize("M,N,K", SMALL)
def test_mm_every_tile_vs_oracle(pkg, ext, O, dev, M, N, K):
    x, w = O.seeded_inputs(M, N, K, seed=M + N + K)
    ref = O.linear_bf16(x, w)
    xd, wd = x.to(dev), w.to(dev)
    for t in _tiles(pkg):
        for S in (1, 3):
            _say(f"case mm M={M} N={N} K={K} tile={t} S={S}")
            y = ext.mm(xd, wd, cfg=(t, S))
            _assert_tol(O, y, ref, f"tile {t} S {S}")


@pytest.mark.parametrize("M,N,K", [(64, 256, 512), (288, 1024, 2048)])
def test_mm_planned_and_f64(pkg, ext, O, dev, M, N, K):
    _say(f"case mm planned M={M} N={N} K={K}")
    x, w = O.seeded_inputs(M, N, K, seed=1)
    y = ext.mm(x.to(dev), w.to(dev)).cpu()
    ref64 = torch.from_numpy(O.linear_f64(x, w))
    # fp32 accumulation + one bf16 rounding: within 1 bf16 ulp of the exact value (+ small fp32 slack)
    err = (y.double() - ref64).abs()
    assert bool((err <= ref64.abs() * 2.0 ** -8 + 1e-4).all()), f"max err {err.max().item():.3e}"


def test_mm_tile_invariance_and_determinism(pkg, ext, O, dev):
    """Without split-K the tiles of one MFMA shape sum K in the same order: outputs are bit-identical across those
    tiles and across runs (16x16x32 families 0 and 5; the K-interleaved family 6, which adds the sums of the even
    and odd 32-k blocks, among itself)."""
    M, N, K = 96, 512, 1024
    x, w = O.seeded_inputs(M, N, K, seed=3)
    xd, wd = x.to(dev), w.to(dev)
    _say("case tile invariance")
    base = {}
    for t in _tiles(pkg):
        fam = pkg._lib.tile_info(t)["family"]
        shape = "kx" if fam == 6 else 16
        y = ext.mm(xd, wd, cfg=(t, 1))
        if shape not in base:
            base[shape] = y
        assert torch.equal(y, base[shape]), f"tile {t}"
        assert torch.equal(y, ext.mm(xd, wd, cfg=(t, 1))), f"tile {t} not deterministic"
    assert len(base) == 2
    for S in (2, 4):
        a = ext.mm(xd, wd, cfg=(6, S))
        assert torch.equal(a, ext.mm(xd, wd, cfg=(6, S))), "split-K not deterministic"


def test_golden_vectors(pkg, ext, O, dev):
    import numpy as np, os
    path = os.path.join(os.path.dirname(__file__), "golden", "proj_golden.npz")
    z = np.load(path)
    for name in sorted({k.split("__")[0] for k in z.files}):
        x = torch.from_numpy(z[f"{name}__x"].view(np.int16)).view(torch.bfloat16)
        w = torch.from_numpy(z[f"{name}__w"].view(np.int16)).view(torch.bfloat16)
        ref = torch.from_numpy(z[f"{name}__y64"])
        _say(f"case golden {name} {tuple(x.shape)} x {tuple(w.shape)}")
        y = ext.mm(x.to(dev), w.to(dev)).cpu().double()
        err = (y - ref).abs()
        assert bool((err <= ref.abs() * 2.0 ** -8 + 1e-4).all()), f"{name}: max err {err.max().item():.3e}"


def test_mm_strided_and_errors(pkg, ext, O, dev):
    _say("case error paths")
    x, w = O.seeded_inputs(8, 64, 64)
    with pytest.raises(RuntimeError):
        ext.mm(x.to(dev), w[:, :56].contiguous().to(dev))  # K mismatch
    with pytest.raises(RuntimeError):
        ext.mm(x.to(dev), torch.zeros(60, 64, dtype=torch.bfloat16, device=dev))  # N % 8
    with pytest.raises(RuntimeError):
        ext.mm(x.to(dev), w.to(dev), cfg=(999, 1))
    with pytest.raises(RuntimeError):
        ext.mm(x.to(dev), w.to(dev), cfg=(52, 2))  # a retired tile id
    with pytest.raises(RuntimeError):
        ext.mm(x.to(dev).t(), w.to(dev))  # not contiguous
    y = ext.mm(torch.empty(0, 64, dtype=torch.bfloat16, device=dev), w.to(dev))
    assert y.shape == (0, 64)


# ----------------------------------------------------------------------------------------------- tail configs
@pytest.mark.parametrize("M", [37, 288])
def test_tail_configs(pkg, ext, O, dev, M):
    """A configuration with a tail runs the last tail_rows W rows as a second launch with its own tile and split.
    With S = 1 in both parts and tiles of one MFMA shape, the result is bit-identical to the single launch."""
    N, K = 1000, 640
    x, w = O.seeded_inputs(M, N, K, seed=M + 11)
    ref = O.linear_bf16(x, w)
    xd, wd = x.to(dev), w.to(dev)
    for key in [(6, 1, 4, 1, 232), (14, 2, 0, 3, 488), (10, 1, 2, 2, 104), (6, 1, 6, 1, 8)]:
        _say(f"case tail mm M={M} cfg={key}")
        y = ext.mm(xd, wd, cfg=key)
        _assert_tol(O, y, ref, f"cfg {key}")
        if key[1] == 1 and key[3] == 1:
            assert torch.equal(y, ext.mm(xd, wd, cfg=(key[0], 1))), f"cfg {key} not bit-identical"
    I = 264
    g = torch.Generator().manual_seed(M)
    wg = (torch.randn(I, K, generator=g) * 0.02).bfloat16()
    wu = (torch.randn(I, K, generator=g) * 0.02).bfloat16()
    ref = O.gate_up_silu(x, wg, wu)
    packed = ext.pack_gate_up(wg.to(dev), wu.to(dev))
    for key in [(6, 1, 4, 1, 144), (14, 2, 10, 2, 16), (6, 1, 6, 1, 8)]:
        _say(f"case tail silu M={M} cfg={key}")
        out = ext.mm_silu_mul(xd, packed, cfg=key)
        _assert_tol(O, out, ref, f"cfg {key}")
        if key[1] == 1 and key[3] == 1:
            assert torch.equal(out, ext.mm_silu_mul(xd, packed, cfg=(key[0], 1))), f"cfg {key}"
    for bad in [(6, 1, 6, 1, 4), (6, 1, 6, 1, N), (6, 1, 999, 1, 8), (6, 1, 6, 0, 8)]:
        with pytest.raises(RuntimeError):
            ext.mm(xd, wd, cfg=bad)
    h = torch.randn(M, N).bfloat16().to(dev)
    with pytest.raises(RuntimeError):
        ext.mm_residual_rmsnorm(h, xd, wd, torch.ones(N, device=dev), None, 1e-6, cfg=(6, 1, 6, 1, 8))


# ----------------------------------------------------------------------------------------------- gate-up
@pytest.mark.parametrize("M,I,K", [(1, 64, 128), (7, 256, 512), (64, 512, 512), (288, 264, 384)])
def test_mm_silu_mul_vs_oracle(pkg, ext, O, dev, M, I, K):
    g = torch.Generator().manual_seed(M * 7 + I)
    x = torch.randn(M, K, generator=g).bfloat16()
    wg = (torch.randn(I, K, generator=g) * 0.02).bfloat16()
    wu = (torch.randn(I, K, generator=g) * 0.02).bfloat16()
    ref = O.gate_up_silu(x, wg, wu)
    packed = ext.pack_gate_up(wg.to(dev), wu.to(dev))
    assert torch.equal(packed.cpu(), O.pack_gate_up(wg, wu))
    for t in _tiles(pkg):
        for S in (1, 2):
            _say(f"case silu M={M} I={I} K={K} tile={t} S={S}")
            out = ext.mm_silu_mul(x.to(dev), packed, cfg=(t, S))
            _assert_tol(O, out, ref, f"tile {t} S {S}")


def test_gate_up_merge_and_fusion_bitexact(pkg, ext, O, dev):
    """tests/test_correct.py:44-45: merged gate+up == two GEMMs and silu_mul == act(gate)*up, bit-exact; the fused
    epilogue equals GEMM -> bf16 -> silu_mul bit-exactly (same K order, same rounding points)."""
    M, I, K = 96, 512, 1024
    g = torch.Generator().manual_seed(11)
    x = torch.randn(M, K, generator=g).bfloat16().to(dev)
    wg = (torch.randn(I, K, generator=g) * 0.02).bfloat16().to(dev)
    wu = (torch.randn(I, K, generator=g) * 0.02).bfloat16().to(dev)
    _say("case gate-up merge")
    gu = ext.mm(x, torch.cat([wg, wu], 0).contiguous(), cfg=(6, 1))
    assert torch.equal(gu[:, :I], ext.mm(x, wg, cfg=(6, 1)))
    assert torch.equal(gu[:, I:], ext.mm(x, wu, cfg=(6, 1)))
    fused = ext.mm_silu_mul(x, ext.pack_gate_up(wg, wu), cfg=(6, 1))
    assert torch.equal(fused, ext.silu_mul(gu))
    kx = [t for t in _tiles(pkg) if pkg._lib.tile_info(t)["family"] == 6]
    for t in kx:  # the K-interleaved family has its own K order: fused == GEMM -> silu_mul with the same tile
        gu_t = ext.mm(x, torch.cat([wg, wu], 0).contiguous(), cfg=(t, 1))
        assert torch.equal(ext.mm_silu_mul(x, ext.pack_gate_up(wg, wu), cfg=(t, 1)), ext.silu_mul(gu_t)), f"tile {t}"
    tab, _ = ext.act_tables(x)
    assert torch.equal(ext.silu_mul_lut(gu, tab), ext.silu_mul(gu))


# ----------------------------------------------------------------------------------------------- residual
@pytest.mark.parametrize("M,N,K", [(7, 256, 512), (64, 512, 1024), (288, 640, 2176)])
@pytest.mark.parametrize("masked", [False, True])
def test_mm_residual_rmsnorm_vs_oracle(pkg, ext, O, dev, M, N, K, masked):
    g = torch.Generator().manual_seed(M + N)
    y = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.01).bfloat16()
    res = torch.randn(M, N, generator=g).bfloat16()
    w1 = (1.0 + 0.1 * torch.randn(N, generator=g)).float()
    mask = (torch.rand(M, generator=g) > 0.3).int() if masked else None
    eps = 1e-6
    for t in (0, 4, 6, 10):
        for S in (1, 2, 4):
            _say(f"case residual M={M} N={N} K={K} tile={t} S={S} masked={masked}")
            h, hn = ext.mm_residual_rmsnorm(res.to(dev), y.to(dev), w.to(dev), w1.to(dev),
                                            mask.to(dev) if masked else None, eps, cfg=(t, S))
            rh, rhn = O.residual_proj(res, y, w, w1, mask, eps, S=S)
            _assert_tol(O, h, rh, f"h tile {t} S {S}")
            _assert_tol(O, hn, rhn, f"hn tile {t} S {S}")
            if masked:
                assert bool((hn.cpu()[mask == 0] == 0).all())


def test_splitk_parts_match_reference_chunks(pkg, ext, O, dev):
    """mm_splitk_f32 planes equal the reference's equal-K/S chunks (K % (8 S) == 0) within fp32 noise."""
    M, N, K, S = 64, 256, 2048, 4
    x, w = O.seeded_inputs(M, N, K, seed=5)
    _say("case splitk planes")
    parts = ext.mm_splitk_f32(x.to(dev), w.to(dev), S).cpu()
    xs = x.float().view(M, S, K // S).transpose(0, 1)
    ws = w.float().view(N, S, K // S).permute(1, 2, 0)
    ref = torch.bmm(xs, ws)
    assert (parts - ref).abs().max().item() <= 1e-4 * ref.abs().max().item() + 1e-5


@pytest.mark.parametrize("N,K,S", [(200, 216, 3), (72, 64, 8), (5120, 17408, 2)])
def test_unsplit_weight_layout(pkg, ext, dev, N, K, S):
    """The reference's split-K copy wsk [S, K/S, N] (src/fastmodel.py:186-188) back to W [N, K]: every element,
    ragged blocks included; the result is kept per source tensor and remade after an in-place change."""
    _say(f"case unsplit N={N} K={K} S={S}")
    w = torch.randn(N, K, generator=torch.Generator().manual_seed(N + K), dtype=torch.float32).bfloat16().to(dev)
    wsk = w.view(N, S, K // S).permute(1, 2, 0).contiguous()
    u = ext.unsplit_weight(wsk)
    assert u.shape == (N, K) and torch.equal(u, w)
    assert ext.unsplit_weight(wsk) is u
    wsk.mul_(2)
    u2 = ext.unsplit_weight(wsk)
    assert u2 is not u and torch.equal(u2, w * 2)
    with pytest.raises(RuntimeError, match="multiples of 8"):
        ext.unsplit_weight(torch.zeros(2, 8, 12, dtype=torch.bfloat16, device=dev))
    if N * K <= 1 << 20:  # first seen inside a graph capture: made by the graph, not kept
        wsk3 = (w * 3).view(N, S, K // S).permute(1, 2, 0).contiguous()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            u3 = ext.unsplit_weight(wsk3)
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(u3, w * 3)
        assert ext.unsplit_weight(wsk3) is not u3 and torch.equal(ext.unsplit_weight(wsk3), w * 3)


# ----------------------------------------------------------------------------------------------- epilogues
def test_add_rmsnorm_variants(pkg, ext, O, dev):
    M, H = 33, 5120
    g = torch.Generator().manual_seed(2)
    x = torch.randn(M, H, generator=g).bfloat16()
    d = (torch.randn(M, H, generator=g) * 0.5).bfloat16()
    parts = torch.randn(3, M, H, generator=g).float()
    w1 = (1.0 + 0.1 * torch.randn(H, generator=g)).float()
    mask = (torch.arange(M) % 3 != 0).int()
    _say("case add_rmsnorm")
    h, hn = ext.add_rmsnorm(x.to(dev), d.to(dev), w1.to(dev), mask.to(dev), 1e-6)
    rh, rhn = O.add_rmsnorm(x, d, w1, mask, 1e-6)
    assert torch.equal(h.cpu(), rh)  # bf16(x + delta) is exact arithmetic + one rounding
    _assert_tol(O, hn, rhn, "hn")
    h0, hn0 = ext.add_rmsnorm(x.to(dev), None, w1.to(dev), None, 1e-6)
    assert h0.data_ptr() == x.to(dev).data_ptr() or torch.equal(h0.cpu(), x)
    _assert_tol(O, hn0, O.add_rmsnorm(x, None, w1, None, 1e-6)[1], "hn no delta")
    h2, hn2 = ext.add_rmsnorm_sk2(x.to(dev), parts.to(dev), w1.to(dev), None, 1e-6)
    rh2, rhn2 = O.add_rmsnorm(x, None, w1, None, 1e-6, parts=parts)
    diff = (h2.cpu().float() - rh2.float()).abs()
    assert (diff == 0).float().mean().item() > 0.999  # fp32 sum order is the same; rounding ties aside
    _assert_tol(O, hn2, rhn2, "hn sk2")
    with pytest.raises(RuntimeError):
        ext.add_rmsnorm_sk2(x.to(dev), torch.zeros(5, M, H, device=dev), w1.to(dev), None, 1e-6)


def test_silu_tables(pkg, ext, O, dev):
    _say("case act_tables")
    silu_b, sig_f = ext.act_tables(torch.empty(1, device=dev))
    rs, rg = O.act_tables()
    a, b = silu_b.cpu().view(torch.int16).int(), rs.view(torch.int16).int()
    fin = torch.isfinite(rs.float())
    close = ((a - b).abs() <= 1) | ~fin
    assert bool(close.all())
    assert (a[fin] == b[fin]).float().mean().item() > 0.999
    fin32 = torch.isfinite(rg)
    assert torch.allclose(sig_f.cpu()[fin32], rg[fin32], rtol=2e-6, atol=1e-30)


# ----------------------------------------------------------------------------------------------- graphs
def test_graph_capture_replays(pkg, ext, O, dev):
    """Capture the four projections of one layer into a graph; every replay equals the eager result."""
    M, K, N_in, I = 64, 512, 1024, 256
    g = torch.Generator().manual_seed(9)
    hn = torch.randn(M, K, generator=g).bfloat16().to(dev)
    h = torch.randn(M, K, generator=g).bfloat16().to(dev)
    w_in = (torch.randn(N_in, K, generator=g) * 0.02).bfloat16().to(dev)
    w_out = (torch.randn(K, N_in, generator=g) * 0.02).bfloat16().to(dev)
    w_gu = ext.pack_gate_up((torch.randn(I, K, generator=g) * 0.02).bfloat16().to(dev),
                            (torch.randn(I, K, generator=g) * 0.02).bfloat16().to(dev))
    w_dn = (torch.randn(K, I, generator=g) * 0.02).bfloat16().to(dev)
    w1 = torch.ones(K, device=dev)

    def body():
        proj = ext.mm(hn, w_in)
        h1, hn1 = ext.mm_residual_rmsnorm(h, proj, w_out, w1, None, 1e-6, cfg=(4, 2))
        m = ext.mm_silu_mul(hn1, w_gu, cfg=(4, 2))
        return ext.mm_residual_rmsnorm(h1, m, w_dn, w1, None, 1e-6, cfg=(4, 1))

    _say("case graph eager")
    eager = [t.clone() for t in body()]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    _say("case graph capture")
    with torch.cuda.graph(graph):
        outs = body()
    for r in range(4):
        _say(f"case graph replay {r}")
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, eager):
            assert torch.equal(a, b), f"replay {r} differs"
        junk = ext.mm(hn, w_in)  # eager work between replays
        torch.cuda.synchronize()
        del junk


# ----------------------------------------------------------------------------------------------- persistent family
def _sk_tiles(pkg):
    return [t for t in _tiles(pkg) if pkg._lib.tile_info(t)["family"] == 5]


@pytest.mark.parametrize("M,N,K", [(539, 16384, 512), (288, 4096, 2048), (64, 2048, 17408), (300, 264, 136)])
def test_stream_k_family(pkg, ext, O, dev, M, N, K):
    """Persistent tiles: whole-tile waves, then the remainder's K iterations spread over the grid (S = pieces per
    tile). Every spread matches the oracle, repeats bit-exactly (the partials are summed in K order whatever the
    arrival order), whatever the workspace held before the call (it is scratch: filled with NaN bytes here)."""
    x, w = O.seeded_inputs(M, N, K, seed=M + N + K + 1)
    ref = O.linear_bf16(x, w)
    xd, wd = x.to(dev), w.to(dev)
    for t in _sk_tiles(pkg):
        base = None
        for S in (1, 2, 8, 16):
            _say(f"case stream-K M={M} N={N} K={K} tile={t} S={S}")
            for buf, _ in ext._WS.values():
                buf.fill_(0xFF)
            y = ext.mm(xd, wd, cfg=(t, S))
            _assert_tol(O, y, ref, f"tile {t} S {S}")
            assert torch.equal(y, ext.mm(xd, wd, cfg=(t, S))), f"tile {t} S {S} not deterministic"
            if S == 1:
                base = y
        assert base is not None


def test_stream_k_epilogues_and_graph(pkg, ext, O, dev):
    """Fused SiLU.mul and residual epilogues through the persistent family with a stream-K remainder, eager and in
    a replayed graph (every replay bit-equal to the eager result)."""
    M, I, K, N = 288, 1032, 640, 1024
    g = torch.Generator().manual_seed(21)
    x = torch.randn(M, K, generator=g).bfloat16()
    wg = (torch.randn(I, K, generator=g) * 0.02).bfloat16()
    wu = (torch.randn(I, K, generator=g) * 0.02).bfloat16()
    wd = (torch.randn(N, K, generator=g) * 0.01).bfloat16()
    res = torch.randn(M, N, generator=g).bfloat16()
    w1 = (1.0 + 0.1 * torch.randn(N, generator=g)).float()
    ref_silu = O.gate_up_silu(x, wg, wu)
    rh, rhn = O.residual_proj(res, x, wd, w1, None, 1e-6, S=1)
    xd, packed = x.to(dev), ext.pack_gate_up(wg.to(dev), wu.to(dev))
    for t in _sk_tiles(pkg):
        for S in (1, 4):
            _say(f"case stream-K epilogues tile={t} S={S}")
            out = ext.mm_silu_mul(xd, packed, cfg=(t, S))
            _assert_tol(O, out, ref_silu, f"silu tile {t} S {S}")
            h, hn = ext.mm_residual_rmsnorm(res.to(dev), xd, wd.to(dev), w1.to(dev), None, 1e-6, cfg=(t, S))
            _assert_tol(O, h, rh, f"h tile {t} S {S}")
            _assert_tol(O, hn, rhn, f"hn tile {t} S {S}")
    t = _sk_tiles(pkg)[-1]
    cfg = (t, 4)
    eager = ext.mm_silu_mul(xd, packed, cfg=cfg).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ext.mm_silu_mul(xd, packed, cfg=cfg)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    _say("case stream-K graph capture")
    with torch.cuda.graph(graph):
        out = ext.mm_silu_mul(xd, packed, cfg=cfg)
    for r in range(4):
        _say(f"case stream-K graph replay {r}")
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r} differs"
        junk = ext.mm_silu_mul(xd, packed, cfg=cfg)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(junk, eager)


@pytest.mark.parametrize("M", [7, 300])
def test_stream_k_epilogues_ragged_m(pkg, ext, O, dev, M):
    """The persistent family's epilogues (staged through LDS, one pass per group of fragment columns) on row counts
    that leave a partial x tile: rows past M must be neither written nor counted in the RMSNorm."""
    I, K, N = 520, 384, 776
    g = torch.Generator().manual_seed(M + 5)
    x = torch.randn(M, K, generator=g).bfloat16()
    wg = (torch.randn(I, K, generator=g) * 0.02).bfloat16()
    wu = (torch.randn(I, K, generator=g) * 0.02).bfloat16()
    wd = (torch.randn(N, K, generator=g) * 0.01).bfloat16()
    res = torch.randn(M, N, generator=g).bfloat16()
    w1 = (1.0 + 0.1 * torch.randn(N, generator=g)).float()
    ref_silu = O.gate_up_silu(x, wg, wu)
    rh, rhn = O.residual_proj(res, x, wd, w1, None, 1e-6, S=1)
    xd, packed = x.to(dev), ext.pack_gate_up(wg.to(dev), wu.to(dev))
    for t in _sk_tiles(pkg):
        for S in (1, 2):
            _say(f"case stream-K ragged M={M} tile={t} S={S}")
            out = ext.mm_silu_mul(xd, packed, cfg=(t, S))
            assert out.shape == (M, I)
            _assert_tol(O, out, ref_silu, f"silu M {M} tile {t} S {S}")
            h, hn = ext.mm_residual_rmsnorm(res.to(dev), xd, wd.to(dev), w1.to(dev), None, 1e-6, cfg=(t, S))
            _assert_tol(O, h, rh, f"h M {M} tile {t} S {S}")
            _assert_tol(O, hn, rhn, f"hn M {M} tile {t} S {S}")


@pytest.mark.parametrize("M,N,K", [(288, 5120, 2176), (539, 1024, 640), (7, 2048, 1024)])
def test_stream_k_residual_row_pass_bitexact(pkg, ext, O, dev, M, N, K):
    """Persistent residual plans with split tiles run the GEMM and then one row pass that sums the split tiles,
    adds the residual and normalises (two launches). It must equal, bit for bit, the GEMM + split-tile pass without
    the norm followed by the standalone add_rmsnorm on h, and match the oracle."""
    g = torch.Generator().manual_seed(M + N)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    res = torch.randn(M, N, generator=g).bfloat16()
    w1 = (1.0 + 0.1 * torch.randn(N, generator=g)).float()
    mask = (torch.rand(M, generator=g) > 0.25).int()
    rh, rhn = O.residual_proj(res, x, w, w1, mask, 1e-6, S=1)
    xd, wd, rd, w1d, md = x.to(dev), w.to(dev), res.to(dev), w1.to(dev), mask.to(dev)
    for t in _sk_tiles(pkg):
        for S in (2, 4, 8):
            _say(f"case stream-K residual row pass M={M} N={N} K={K} tile={t} S={S}")
            h, hn = ext.mm_residual_rmsnorm(rd, xd, wd, w1d, md, 1e-6, cfg=(t, S))
            h0, _ = ext.mm_residual_rmsnorm(rd, xd, wd, w1d, md, 1e-6, want_hn=False, cfg=(t, S))
            _, hn0 = ext.add_rmsnorm(h0, None, w1d, md, 1e-6)
            assert torch.equal(h, h0), f"tile {t} S {S}: h differs from GEMM + split-tile pass"
            assert torch.equal(hn, hn0), f"tile {t} S {S}: hn differs from add_rmsnorm of h"
            _assert_tol(O, h, rh, f"h tile {t} S {S}")
            _assert_tol(O, hn, rhn, f"hn tile {t} S {S}")


def test_bf16_rounding_bit_patterns(ext, dev):
    """Every fp32 -> bf16 rounding in the kernels (one hardware conversion) is round-to-nearest-even, checked
    bit-exactly against torch's CPU conversion on about a million fp32 bit patterns: random words, the three
    patterns around every tie of random bf16 values, denormals, the largest finite values (and the ones that
    round to inf), infinities and NaNs. They go through the split-K RMSNorm with S = 1 and x = 0, whose h is
    bf16(0 + bf16(plane)), i.e. the rounding itself (a -0 result becomes +0)."""
    H = 5120
    rng = np.random.default_rng(7)
    rand = rng.integers(0, 2 ** 32, size=150 * H, dtype=np.uint64).astype(np.uint32)
    hi = rng.integers(0, 2 ** 16, size=16 * H, dtype=np.uint64).astype(np.uint32) << 16
    ties = np.concatenate([hi | 0x7FFF, hi | 0x8000, hi | 0x8001])
    special = np.array([0, 0x80000000, 1, 0x8000, 0x7FFFFF, 0x807FFFFF, 0x00800000, 0x7F7FFFFF, 0x7F7F8000,
                        0x7F7F7FFF, 0xFF7FFFFF, 0xFF7F8000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001,
                        0xFFFFFFFF, 0x3F808000, 0x3F818000], dtype=np.uint32)
    pat = np.concatenate([rand, ties, special])
    pat = np.concatenate([pat, np.zeros((-len(pat)) % H, dtype=np.uint32)])
    M = len(pat) // H
    vals = torch.from_numpy(pat.view(np.float32).copy()).reshape(M, H)
    _say(f"case bf16 rounding patterns M={M} H={H}")
    x = torch.zeros(M, H, dtype=torch.bfloat16, device=dev)
    h, _ = ext.add_rmsnorm_sk(x, vals.reshape(1, M, H).to(dev), torch.ones(H, device=dev), None, 1e-6)
    got = h.cpu().view(torch.int16).numpy().view(np.uint16)
    ref = vals.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).copy()
    ref[ref == 0x8000] = 0
    nan = np.isnan(vals.numpy())
    assert np.all(((got & 0x7FFF) > 0x7F80)[nan]), "NaN must stay NaN"
    bad = np.flatnonzero((got != ref) & ~nan)
    assert bad.size == 0, f"{bad.size} roundings differ, first input 0x{pat[bad[0]]:08x}: 0x{got.flat[bad[0]]:04x} vs 0x{ref.flat[bad[0]]:04x}"


# ----------------------------------------------------------------------------------------------- scoring head
@pytest.mark.parametrize("R", [1, 7, 64, 539])
def test_head_scores_vs_oracle(pkg, ext, O, dev, R):
    """Fused gather + GEMV of the scoring head against the oracle (fp32 sums in another order: rel 1e-5), one-hot
    weights exactly, deterministic, and NaN for an out-of-range index."""
    g = torch.Generator().manual_seed(R)
    rows, H = R + 50, 5120
    hn = torch.randn(rows, H, generator=g).bfloat16()
    w = torch.randn(H, generator=g) * 0.02
    b = torch.tensor([-0.5])
    idx = torch.randint(0, rows, (R,), generator=g)
    _say(f"case head R={R}")
    s = ext.head_scores(hn.to(dev), idx.to(dev), w.to(dev), b.to(dev)).cpu()
    ref = torch.from_numpy(O.head_scores_f64(hn, idx, w, b)).float()
    assert torch.allclose(s, ref, rtol=1e-5, atol=1e-5), (s - ref).abs().max()
    assert torch.equal(s, ext.head_scores(hn.to(dev), idx.to(dev), w.to(dev), b.to(dev)).cpu())
    e = torch.zeros(H)
    e[123] = 1.0
    assert torch.equal(ext.head_scores(hn.to(dev), idx.to(dev), e.to(dev)).cpu(), hn[idx, 123].float())
    bad = idx.clone()
    bad[0] = rows
    sb = ext.head_scores(hn.to(dev), bad.to(dev), w.to(dev), b.to(dev)).cpu()
    assert torch.isnan(sb[0]) and torch.equal(sb[1:], s[1:])


# ----------------------------------------------------------------------------------------------- full sizes
@pytest.mark.parametrize("M", [7, 288, 539])
def test_planned_full_size_projections(pkg, ext, O, dev, M):
    """Every projection shape of the forward at the headline M, through the plan table's own
    configuration (tails, split-K, stream-K included), against the oracle on the same seeded inputs."""
    from importlib import import_module
    perf = import_module("open_jev_fast_amd.perf")
    g = torch.Generator().manual_seed(M)
    for name, (N, K, kind) in perf.SHAPES.items():
        _say(f"case full size {name} M={M} plan={pkg._lib.plan(M, N, K, {'plain': 0, 'silu': 1, 'residual': 2}[kind])}")
        x = torch.randn(M, K, generator=g).bfloat16()
        w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
        if kind == "plain":
            out = ext.mm(x.to(dev), w.to(dev)).cpu()
            ref = O.linear_bf16(x, w)
            _assert_tol(O, out, ref, name)
        elif kind == "silu":
            I = N // 2
            out = ext.mm_silu_mul(x.to(dev), ext.pack_gate_up(w[:I].to(dev), w[I:].to(dev))).cpu()
            ref = O.gate_up_silu(x, w[:I], w[I:])
            _assert_tol(O, out, ref, name)
        else:
            res = torch.randn(M, N, generator=g).bfloat16()
            w1 = (1.0 + 0.1 * torch.randn(N, generator=g)).float()
            h, hn = ext.mm_residual_rmsnorm(res.to(dev), x.to(dev), w.to(dev), w1.to(dev), None, 1e-6)
            rh, rhn = O.residual_proj(res, x, w, w1, None, 1e-6, S=1)
            _assert_tol(O, h.cpu(), rh, name + " h")
            _assert_tol(O, hn.cpu(), rhn, name + " hn")
