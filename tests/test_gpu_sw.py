"""GPU parity of the skinny weight-streaming family (family 7: K split over the waves of one workgroup, operands
loaded straight into MFMA registers, one launch, no workspace) against the CPU oracle, through the C-ABI.

Covers every family-7 tile with each epilogue (bf16, SiLU.mul of packed gate/up rows, residual + RMSNorm, fp32
split-K planes), packed and row-major weights, grid split-K on top of the wave split, more waves than stages
(waves without work), N not a multiple of the tile, several M tiles, the refusal of partial 64-k stages, and graph
replays. Tolerance as
in the other parity tests; packed and row-major weights give the same bits (same K ranges).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = dict(max_rel=1e-2, mean_abs_rms=1e-3)


def _say(*a):
    print(*a, flush=True)


def _assert_tol(O, out, ref, what):
    ok, a, b = O.tolerance_ok(out.float().cpu(), ref.float().cpu(), **TOL)
    assert ok, f"{what}: max_rel {a:.3e} mean/rms {b:.3e}"


def _sw_tiles(pkg):
    L = pkg._lib
    return [t for t in range(L.lib().ojx_num_tiles()) if L.tile_info(t)["family"] == 7]


def test_family_present(pkg):
    assert len(_sw_tiles(pkg)) >= 4


@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (7, 272, 640), (16, 1040, 1344), (32, 96, 5120), (40, 208, 448)])
def test_sw_plain_vs_oracle(pkg, ext, O, dev, M, N, K):
    x, w = O.seeded_inputs(M, N, K, seed=M * 3 + N + K)
    ref = O.linear_bf16(x, w)
    xd, wd = x.to(dev), w.to(dev)
    wp = ext.pack_weight(wd)
    for t in _sw_tiles(pkg):
        for S in (1, 2, 3):
            _say(f"case sw mm M={M} N={N} K={K} tile={t} S={S}")
            try:
                y = ext.mm(xd, wd, cfg=(t, S))
            except RuntimeError as e:
                assert "invalid" in str(e), str(e)
                continue
            _assert_tol(O, y, ref, f"row-major tile {t} S {S}")
            assert torch.equal(y, ext.mm(xd, wd, cfg=(t, S))), f"tile {t} S {S} not deterministic"
            try:
                yp = ext.mm_pk(xd, wp, cfg=(t, S))
            except RuntimeError as e:
                assert "invalid" in str(e), str(e)
                continue
            _assert_tol(O, yp, ref, f"packed tile {t} S {S}")
            if S == 1:
                assert torch.equal(y, yp), f"tile {t}: packed != row-major"


@pytest.mark.parametrize("M,N,K", [(7, 200, 328), (13, 136, 1000)])
def test_sw_rejects_partial_stages(pkg, ext, O, dev, M, N, K):
    """The family reads whole 64-k stages: K % 64 != 0, or a split boundary inside a stage, is refused; N not a
    multiple of the tile is fine."""
    x, w = O.seeded_inputs(M, N, 640, seed=M + K)
    ref = O.linear_bf16(x, w)
    xb, _ = O.seeded_inputs(M, N, K, seed=M)
    wb = torch.zeros(N, K, dtype=torch.bfloat16)
    for t in _sw_tiles(pkg):
        _say(f"case sw refuse M={M} N={N} K={K} tile={t}")
        with pytest.raises(RuntimeError, match="invalid"):
            ext.mm(xb.to(dev), wb.to(dev), cfg=(t, 1))
        with pytest.raises(RuntimeError, match="invalid"):
            ext.mm(x.to(dev), w.to(dev), cfg=(t, 3))  # 640 / 3 -> 216-k splits
        _assert_tol(O, ext.mm(x.to(dev), w.to(dev), cfg=(t, 2)), ref, f"tile {t} S 2")


@pytest.mark.parametrize("M", [1, 7, 16])
def test_sw_epilogues(pkg, ext, O, dev, M):
    I, K, N = 264, 768, 528
    g = torch.Generator().manual_seed(M + 101)
    x = torch.randn(M, K, generator=g).bfloat16()
    wg = (torch.randn(I, K, generator=g) * 0.02).bfloat16()
    wu = (torch.randn(I, K, generator=g) * 0.02).bfloat16()
    ref_gu = O.gate_up_silu(x, wg, wu)
    xd = x.to(dev)
    gu = ext.pack_gate_up(wg.to(dev), wu.to(dev))
    gu_pk = ext.pack_weight(gu)
    w = (torch.randn(N, K, generator=g) * 0.01).bfloat16()
    res = torch.randn(M, N, generator=g).bfloat16()
    w1 = (1.0 + 0.1 * torch.randn(N, generator=g)).float()
    mask = (torch.rand(M, generator=g) > 0.3).int()
    mask[0] = 1
    wd, wp = w.to(dev), ext.pack_weight(w.to(dev))
    for t in _sw_tiles(pkg):
        for S in (1, 2):
            _say(f"case sw silu M={M} tile={t} S={S}")
            out = ext.mm_silu_mul(xd, gu, cfg=(t, S))
            _assert_tol(O, out, ref_gu, f"silu tile {t} S {S}")
            out_pk = ext.mm_silu_mul_pk(xd, gu_pk, cfg=(t, S))
            _assert_tol(O, out_pk, ref_gu, f"silu packed tile {t} S {S}")
            if S == 1:
                # the fused epilogue equals GEMM -> bf16 -> silu_mul with the same tile
                gu_rows = torch.cat([wg, wu], 0).contiguous().to(dev)  # [gate; up] rows, silu_mul's layout
                assert torch.equal(out, ext.silu_mul(ext.mm(xd, gu_rows, cfg=(t, 1)))), f"tile {t}"
                assert torch.equal(out, out_pk)
            _say(f"case sw residual M={M} tile={t} S={S}")
            rh, rhn = O.residual_proj(res, x, w, w1, mask, 1e-6, S=S)
            h, hn = ext.mm_residual_rmsnorm(res.to(dev), xd, wd, w1.to(dev), mask.to(dev), 1e-6, cfg=(t, S))
            _assert_tol(O, h, rh, f"h tile {t} S {S}")
            _assert_tol(O, hn, rhn, f"hn tile {t} S {S}")
            assert bool((hn.cpu()[mask == 0] == 0).all())
            hp, hnp = ext.mm_residual_rmsnorm_pk(res.to(dev), xd, wp, w1.to(dev), mask.to(dev), 1e-6, cfg=(t, S))
            assert torch.equal(h, hp) and torch.equal(hn, hnp), f"residual packed != row-major tile {t} S {S}"


def test_sw_splitk_planes_and_graph(pkg, ext, O, dev):
    """fp32 planes of a grid split on a family-7 tile sum to the GEMM; a captured graph replays bit-equal."""
    M, N, K, S = 7, 512, 2048, 4
    x, w = O.seeded_inputs(M, N, K, seed=9)
    xd, wd = x.to(dev), w.to(dev)
    ref = O.linear_f32(x, w)
    for t in _sw_tiles(pkg):
        _say(f"case sw planes tile={t}")
        parts = ext.mm_splitk_f32(xd, wd, S, tile=t).cpu()
        assert parts.shape == (S, M, N)
        d = (parts.sum(0) - ref).abs().max().item()
        assert d <= 1e-3 * ref.abs().max().item() + 1e-4, f"tile {t}: planes off by {d:.3e}"
    t = _sw_tiles(pkg)[0]
    wp = ext.pack_weight(wd)
    eager = ext.mm_pk(xd, wp, cfg=(t, 1))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ext.mm_pk(xd, wp, cfg=(t, 1))
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = ext.mm_pk(xd, wp, cfg=(t, 1))
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
        assert torch.equal(ext.mm_pk(xd, wp, cfg=(t, 1)), eager)
