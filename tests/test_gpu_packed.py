"""GPU parity of the packed-weight projections (ojx_pack_weight + the *_pk entry points), through the C-ABI.

* the packed layout equals the oracle's restatement bit for bit;
* every tile that reads the packed layout, with and without split-K / stream-K spread, matches the oracle on ragged
  shapes, and equals the row-major path with the same tile bit for bit wherever both cut K the same way (S = 1, and
  any spread of the persistent family);
* the fused SiLU.mul and residual + RMSNorm epilogues on packed weights.

Tolerance: max |out - ref| / max |ref| <= 1e-2 and mean |out - ref| <= 1e-3 * RMS(ref).
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


def _packed_tiles(pkg):
    L = pkg._lib
    return [t for t in range(L.lib().ojx_num_tiles()) if L.tile_info(t)["family"] in (0, 5, 6)]


def test_pack_weight_layout(ext, O, dev):
    g = torch.Generator().manual_seed(3)
    w = torch.randn(96, 320, generator=g).bfloat16()
    got = ext.pack_weight(w.to(dev)).cpu()
    assert torch.equal(got, O.pack_weight(w))
    with pytest.raises(RuntimeError):
        ext.pack_weight(torch.zeros(24, 64, dtype=torch.bfloat16, device=dev))  # N % 16
    with pytest.raises(RuntimeError):
        ext.pack_weight(torch.zeros(32, 96, dtype=torch.bfloat16, device=dev))  # K % 64


@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (7, 272, 320), (37, 528, 640), (96, 1024, 512), (300, 400, 192)])
def test_mm_pk_every_tile(pkg, ext, O, dev, M, N, K):
    x, w = O.seeded_inputs(M, N, K, seed=M + N + K + 5)
    ref = O.linear_bf16(x, w)
    xd, wd = x.to(dev), w.to(dev)
    wp = ext.pack_weight(wd)
    fam = lambda t: pkg._lib.tile_info(t)["family"]  # noqa: E731
    for t in _packed_tiles(pkg):
        for S in (1, 2, 3):
            _say(f"case mm_pk M={M} N={N} K={K} tile={t} S={S}")
            try:
                y = ext.mm_pk(xd, wp, cfg=(t, S))
            except RuntimeError as e:
                assert "invalid" in str(e), str(e)   # a split that leaves a K range empty
                continue
            _assert_tol(O, y, ref, f"tile {t} S {S}")
            same_cut = S == 1 or fam(t) == 5 or -(-(-(-K // S)) // 8) * 8 == -(-(-(-K // S)) // 64) * 64
            if same_cut:
                assert torch.equal(y, ext.mm(xd, wd, cfg=(t, S))), f"tile {t} S {S}: packed != row-major"


@pytest.mark.parametrize("M", [7, 64, 288])
def test_pk_epilogues(pkg, ext, O, dev, M):
    I, K, N = 520, 384, 1040
    g = torch.Generator().manual_seed(M + 17)
    x = torch.randn(M, K, generator=g).bfloat16()
    wg = (torch.randn(I, K, generator=g) * 0.02).bfloat16()
    wu = (torch.randn(I, K, generator=g) * 0.02).bfloat16()
    wd = (torch.randn(N, K, generator=g) * 0.01).bfloat16()
    res = torch.randn(M, N, generator=g).bfloat16()
    w1 = (1.0 + 0.1 * torch.randn(N, generator=g)).float()
    mask = (torch.rand(M, generator=g) > 0.2).int()
    ref_silu = O.gate_up_silu(x, wg, wu)
    rh, rhn = O.residual_proj(res, x, wd, w1, mask, 1e-6, S=1)
    xd = x.to(dev)
    gu = ext.pack_gate_up(wg.to(dev), wu.to(dev))
    gu_pk = ext.pack_weight(gu)
    wd_pk = ext.pack_weight(wd.to(dev))
    for t in [None] + _packed_tiles(pkg):
        for S in (1, 2):
            cfg = None if t is None else (t, S)
            if t is None and S == 2:
                continue
            _say(f"case pk epilogues M={M} cfg={cfg}")
            try:
                out = ext.mm_silu_mul_pk(xd, gu_pk, cfg=cfg)
                h, hn = ext.mm_residual_rmsnorm_pk(res.to(dev), xd, wd_pk, w1.to(dev), mask.to(dev), 1e-6, cfg=cfg)
            except RuntimeError as e:
                assert "invalid" in str(e), str(e)
                continue
            _assert_tol(O, out, ref_silu, f"silu {cfg}")
            _assert_tol(O, h, rh, f"h {cfg}")
            _assert_tol(O, hn, rhn, f"hn {cfg}")
            if cfg is not None and S == 1:
                assert torch.equal(out, ext.mm_silu_mul(xd, gu, cfg=cfg))
                h0, hn0 = ext.mm_residual_rmsnorm(res.to(dev), xd, wd.to(dev), w1.to(dev), mask.to(dev), 1e-6,
                                                  cfg=cfg)
                assert torch.equal(h, h0) and torch.equal(hn, hn0)
