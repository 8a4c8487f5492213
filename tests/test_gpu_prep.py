"""GPU parity of the full-attention prep (the consumer of the full-attention layers' QKV in-projection), through
the C-ABI.

* ojx_fullattn_prep (the reference's K.fullattn_prep2, src/kernels.cu:302-355) against the oracle's restatement:
  v and gate bit for bit; q and k within one bf16 rounding step, because the per-row sum of squares is added in a
  different order (wave butterfly vs the oracle's torch sum) and may move one rsqrt across a rounding boundary.
* ojx_gemm_qkv_fullattn_prep (the in-projection GEMM with the prep in its epilogue), row-major and packed weights:
  its projection is the kx tile's own, so it is checked against (a) the oracle chain GEMM -> prep on the north
  star's tolerance and (b) the unfused chain ext.mm with the same tile -> ojx_fullattn_prep, which must agree to
  within one rounding step (same products, same K order, only the sum-of-squares order differs).

Tolerance: max |out - ref| / max |ref| <= 1e-2 and mean |out - ref| <= 1e-3 * RMS(ref).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = dict(max_rel=1e-2, mean_abs_rms=1e-3)
EPS = 1e-6


def _say(*a):
    print(*a, flush=True)


def _assert_tol(O, out, ref, what):
    ok, a, b = O.tolerance_ok(out.float().cpu(), ref.float().cpu(), **TOL)
    assert ok, f"{what}: max_rel {a:.3e} mean/rms {b:.3e}"


def _inputs(N, HQ, HKV, D, RD, seed, K=None):
    g = torch.Generator().manual_seed(seed)
    qw1 = (1.0 + 0.1 * torch.randn(D, generator=g)).float()
    kw1 = (1.0 + 0.1 * torch.randn(D, generator=g)).float()
    ang = torch.rand(N, RD // 2, generator=g) * 6.0
    cos = torch.cat([ang.cos(), ang.cos()], 1).bfloat16()
    sin = torch.cat([ang.sin(), ang.sin()], 1).bfloat16()
    P = (2 * HQ + 2 * HKV) * D
    if K is None:
        return torch.randn(N, P, generator=g).bfloat16(), qw1, kw1, cos, sin
    x = torch.randn(N, K, generator=g).bfloat16()
    w = (torch.randn(P, K, generator=g) * K ** -0.5).bfloat16()
    return x, w, qw1, kw1, cos, sin


def _close_bf16(got, want, what):
    """Within one bf16 rounding step of the value or of the row's largest term, and mostly exact."""
    g, w = got.float().cpu(), want.float().cpu()
    err = (g - w).abs()
    # one step of a RoPE term is relative to the row's magnitude, not to the (possibly cancelled) sum
    bound = (w.abs() + w.abs().amax(-1, keepdim=True)) * 2.0 ** -7
    assert bool((err <= bound).all()), f"{what}: worst {(err - bound).max().item():.3e} above the bound"
    frac = (err == 0).float().mean().item()
    assert frac > 0.9, f"{what}: only {frac:.3f} of the values equal"


@pytest.mark.parametrize("N,HQ,HKV,RD", [(1, 24, 4, 64), (7, 24, 4, 64), (130, 3, 2, 64), (33, 2, 1, 32),
                                         (5, 1, 1, 128)])
def test_fullattn_prep_vs_oracle(ext, O, dev, N, HQ, HKV, RD):
    D = 256
    _say(f"case prep N={N} HQ={HQ} HKV={HKV} RD={RD}")
    proj, qw1, kw1, cos, sin = _inputs(N, HQ, HKV, D, RD, seed=N + HQ + RD)
    qt, kt, vt, gate = ext.fullattn_prep2(proj.to(dev), qw1.to(dev), kw1.to(dev), cos.to(dev), sin.to(dev), 1, N,
                                          HQ, HKV, D, EPS)
    torch.cuda.synchronize()
    rq, rk, rv, rg = O.fullattn_prep(proj, qw1, kw1, cos, sin, HQ, HKV, D, EPS)
    assert tuple(qt.shape) == (1, HQ, N, D) and tuple(kt.shape) == (1, HKV, N, D)
    assert tuple(vt.shape) == (1, HKV, N, D) and tuple(gate.shape) == (N, HQ * D)
    assert torch.equal(vt[0].cpu(), rv) and torch.equal(gate.cpu(), rg)
    _close_bf16(qt[0], rq, "q")
    _close_bf16(kt[0], rk, "k")


def test_fullattn_prep_rejects(ext, dev):
    proj, qw1, kw1, cos, sin = [t.to(dev) for t in _inputs(3, 2, 1, 256, 64, seed=1)]
    with pytest.raises(RuntimeError):
        ext.fullattn_prep2(proj, qw1, kw1, cos, sin, 2, 3, 2, 1, 256, EPS)  # B != 1
    with pytest.raises(RuntimeError):
        ext.fullattn_prep2(proj, qw1, kw1, cos[:, :48].contiguous(), sin[:, :48].contiguous(), 1, 3, 2, 1, 256, EPS)
    with pytest.raises(RuntimeError, match="cos and sin"):  # fewer cos rows than tokens
        ext.fullattn_prep2(proj, qw1, kw1, cos[:2].contiguous(), sin[:2].contiguous(), 1, 3, 2, 1, 256, EPS)
    with pytest.raises(RuntimeError, match="qw1 and kw1"):
        ext.fullattn_prep2(proj, qw1[:128].contiguous(), kw1, cos, sin, 1, 3, 2, 1, 256, EPS)
    empty = torch.empty(0, proj.shape[1], dtype=proj.dtype, device=dev)
    out = ext.fullattn_prep2(empty, qw1, kw1, cos[:0], sin[:0], 1, 0, 2, 1, 256, EPS)
    assert out[0].shape[2] == 0


# (M, HQ, HKV, K): the north star's full-attention in-projection is HQ = 24, HKV = 4, K = 5120 (N = 14336); smaller
# head counts and K keep the ragged-M cases quick.
@pytest.mark.parametrize("M,HQ,HKV,K", [(1, 2, 1, 256), (7, 24, 4, 5120), (64, 3, 2, 640), (65, 3, 2, 640),
                                        (200, 2, 1, 1024), (288, 24, 4, 5120)])
@pytest.mark.parametrize("packed", [False, True])
def test_gemm_qkv_fullattn_prep(pkg, ext, O, dev, M, HQ, HKV, K, packed):
    D, RD = 256, 64
    _say(f"case fused prep M={M} HQ={HQ} HKV={HKV} K={K} packed={packed}")
    x, w, qw1, kw1, cos, sin = _inputs(M, HQ, HKV, D, RD, seed=M + K + HQ, K=K)
    xd, wd = x.to(dev), w.to(dev)
    qd, kd, cd, sd = qw1.to(dev), kw1.to(dev), cos.to(dev), sin.to(dev)
    wuse = ext.pack_weight(wd) if packed else wd
    qt, kt, vt, gate = ext.mm_fullattn_prep(xd, wuse, qd, kd, cd, sd, HQ, HKV, D, EPS, fused=True)
    # (b) the unfused chain with the same tile: the projection is identical, the prep's sum order differs
    tile = 89 if M <= 64 else 88
    proj = (ext.mm_pk if packed else ext.mm)(xd, wuse, cfg=(tile, 1))
    uq, uk, uv, ug = ext.fullattn_prep2(proj, qd, kd, cd, sd, 1, M, HQ, HKV, D, EPS)
    torch.cuda.synchronize()
    assert torch.equal(vt.cpu(), uv.cpu()) and torch.equal(gate.cpu(), ug.cpu())
    _close_bf16(qt[0], uq[0], "fused q vs unfused")
    _close_bf16(kt[0], uk[0], "fused k vs unfused")
    # the default route (planned GEMM, then the prep kernel) against the same oracle chain below
    dq, dk, dv, dg = ext.mm_fullattn_prep(xd, wuse, qd, kd, cd, sd, HQ, HKV, D, EPS)
    # (a) the oracle chain on the north star's tolerance
    rq, rk, rv, rg = O.fullattn_prep(O.linear_bf16(x, w), qw1, kw1, cos, sin, HQ, HKV, D, EPS)
    for got, ref, nm in ((qt[0], rq, "q"), (kt[0], rk, "k"), (vt[0], rv, "v"), (gate, rg, "gate"),
                         (dq[0], rq, "q, two launches"), (dk[0], rk, "k, two launches"), (dv[0], rv, "v, two launches"),
                         (dg, rg, "gate, two launches")):
        _assert_tol(O, got, ref, f"{nm} M={M}")


def test_gemm_qkv_fullattn_prep_rejects(ext, dev):
    x, w, qw1, kw1, cos, sin = [t.to(dev) for t in _inputs(4, 2, 1, 256, 32, seed=2, K=256)]
    with pytest.raises(RuntimeError):  # the fused epilogue handles RD = 64 only
        ext.mm_fullattn_prep(x, w, qw1, kw1, cos, sin, 2, 1, 256, EPS, fused=True)
    with pytest.raises(RuntimeError):  # weight rows do not match the head counts
        ext.mm_fullattn_prep(x, w[:512].contiguous(), qw1, kw1, cos, sin, 2, 1, 256, EPS)


# ---------------------------------------------------------------- linear-attention prep (tree layout)
def _lin_inputs(tree, HK, HV, seed, HD=128, NB=32, PB=16):
    from oracle import linattn_oracle as LO
    lay = LO.tree_layout(*tree, NB=NB, PB=PB)
    KD, VD = HK * HD, HV * HD
    C = 2 * KD + VD
    g = torch.Generator().manual_seed(seed)
    proj = (torch.randn(lay["N"], C + VD + 2 * HV, generator=g) * 1.5).bfloat16()
    convw = (torch.randn(C, 4, generator=g) * 0.5).bfloat16()
    A_log = torch.randn(HV, generator=g).bfloat16()
    dt_bias = (torch.randn(HV, generator=g) * 4).bfloat16()
    return LO, lay, proj, convw, A_log, dt_bias, KD, VD


def _ulp_close(got, want, what, min_equal=0.99, steps=1):
    """Equal almost everywhere; elsewhere within `steps` bf16 rounding steps. The device expf and numpy's may differ
    in the last fp32 bit, which moves a SiLU output across a bf16 rounding boundary now and then (one step); a q / k
    value is rounded once more after the head norm (two steps)."""
    g, w = got.float().cpu(), want.float().cpu()
    err = (g - w).abs()
    lim = w.abs() * 2.0 ** -8 * (2 * steps)
    assert bool((err <= lim).all()), f"{what}: {(err - lim).max():.3e}"
    frac = (err == 0).float().mean().item()
    assert frac >= min_equal, f"{what}: only {frac:.4f} equal"


# (Lr, q_len, groups, l_len): the north star's lin-attn in-projection rows are ~288 packed tokens (a shared prompt,
# group continuations, candidate leaves); one tree with no padding slots at all, one with rows that no slot holds.
_TREES = {
    "m288": (200, [20, 12, 9], [0, 0, 1, 1, 2, 2, 0, 1], [5, 7, 3, 6, 2, 4, 1, 3]),
    "nopad": (10, [2], [0, 0], [4, 4]),
    "tiny": (1, [0], [0], [1]),   # two real rows on one path
}


@pytest.mark.parametrize("tree", list(_TREES))
@pytest.mark.parametrize("rep_qk", [False, True])
def test_linattn_prep_vs_oracle(ext, dev, tree, rep_qk):
    HK, HV, HD = 16, 48, 128   # Qwen3.5 linear attention: KD 2048, VD 6144, proj width 16480
    if tree == "tiny":
        HK, HV = 1, 3
    t = _TREES[tree]
    _say(f"case linattn_prep tree={tree} rep_qk={rep_qk}")
    LO, lay, proj, convw, A_log, dt_bias, KD, VD = _lin_inputs(t, HK, HV, seed=len(tree), PB=8 if tree == "nopad"
                                                               else 16)
    if tree == "nopad":
        assert lay["rep_ptr"][lay["N"]] == lay["rep_ptr"][lay["N"] + 1]   # no end-padding slot
    d = lambda a: torch.as_tensor(a).to(dev).contiguous()  # noqa: E731
    q, k, v, g, beta = ext.linattn_prep_dedup2(proj.to(dev), d(lay["hist"]), d(lay["rep_ptr"]), d(lay["rep_pos"]),
                                               lay["L2"], convw.to(dev), A_log.to(dev), dt_bias.to(dev), KD, VD, HV,
                                               HK, 128, rep_qk)
    torch.cuda.synchronize()
    rq_, rk_, rv_, rg_, rb_ = LO.linattn_prep(proj, lay["hist"], lay["rep_ptr"], lay["rep_pos"], lay["L2"], convw,
                                              A_log, dt_bias, KD, VD, HV, HK, 128, rep_qk)
    assert q.shape == rq_.shape and v.shape == rv_.shape and g.dtype == torch.float32
    _ulp_close(v, rv_, "v")
    _ulp_close(q, rq_, "q", steps=2)
    _ulp_close(k, rk_, "k", steps=2)
    _ulp_close(beta, rb_, "beta")
    assert torch.allclose(g.cpu(), rg_, rtol=2e-6, atol=0), (g.cpu() - rg_).abs().max()
    pad = torch.as_tensor(lay["src"].reshape(-1) < 0)
    for tnsr in (q, k, v, g, beta):   # padding slots are written (zeros), not left as they were
        assert bool((tnsr.cpu()[pad] == 0).all())


def test_linattn_prep_rejects(ext, dev):
    LO, lay, proj, convw, A_log, dt_bias, KD, VD = _lin_inputs(_TREES["nopad"], 2, 6, seed=1)
    d = lambda a: torch.as_tensor(a).to(dev).contiguous()  # noqa: E731
    args = [proj.to(dev), d(lay["hist"]), d(lay["rep_ptr"]), d(lay["rep_pos"]), lay["L2"], convw.to(dev),
            A_log.to(dev), dt_bias.to(dev), KD, VD, 6, 2]
    with pytest.raises(RuntimeError):
        ext.linattn_prep_dedup2(*args, 64, False)           # head_dim 64
    with pytest.raises(RuntimeError):
        ext.linattn_prep_dedup2(*args[:4], lay["L2"] + 1, *args[5:], 128, False)   # R not a multiple of L2
    with pytest.raises(RuntimeError):                       # rep_qk with HV / HK = 3 only
        a2 = list(args)
        a2[10] = 8
        ext.linattn_prep_dedup2(*a2, 128, True)


# ---------------------------------------------------------------- seeded random cases
def _random_prep_cases(n=30):
    import numpy as np
    rng = np.random.default_rng(7)
    full, lin = [], []
    for i in range(n):
        RD = int(rng.choice([16, 32, 64, 128, 256]))
        full.append((i, int(rng.integers(1, 300)), int(rng.integers(1, 9)), int(rng.integers(1, 5)), RD))
        ng = int(rng.integers(1, 4))
        nl = int(rng.integers(1, 7))
        tree = (int(rng.integers(1, 60)), [int(v) for v in rng.integers(0, 11, ng)],
                [int(v) for v in rng.integers(0, ng, nl)], [int(v) for v in rng.integers(1, 9, nl)])
        HK = int(rng.choice([1, 2, 4]))
        lin.append((i, tree, HK, bool(rng.integers(0, 2))))
    return full, lin


_RFULL, _RLIN = _random_prep_cases()


@pytest.mark.parametrize("case", _RFULL, ids=lambda c: f"f{c[0]}-N{c[1]}-q{c[2]}-kv{c[3]}-rd{c[4]}")
def test_fullattn_prep_random(ext, O, dev, case):
    i, N, HQ, HKV, RD = case
    D = 256
    _say(f"case prep random {i}: N={N} HQ={HQ} HKV={HKV} RD={RD}")
    proj, qw1, kw1, cos, sin = _inputs(N, HQ, HKV, D, RD, seed=1000 + i)
    qt, kt, vt, gate = ext.fullattn_prep2(proj.to(dev), qw1.to(dev), kw1.to(dev), cos.to(dev), sin.to(dev), 1, N,
                                          HQ, HKV, D, EPS)
    torch.cuda.synchronize()
    rq, rk, rv, rg = O.fullattn_prep(proj, qw1, kw1, cos, sin, HQ, HKV, D, EPS)
    assert torch.equal(vt[0].cpu(), rv) and torch.equal(gate.cpu(), rg)
    _close_bf16(qt[0], rq, "q")
    _close_bf16(kt[0], rk, "k")


@pytest.mark.parametrize("case", _RLIN, ids=lambda c: f"l{c[0]}-hk{c[2]}-rq{int(c[3])}")
def test_linattn_prep_random_trees(ext, dev, case):
    i, tree, HK, rep_qk = case
    HV = 3 * HK
    _say(f"case linattn_prep random {i}: tree={tree} HK={HK} rep_qk={rep_qk}")
    LO, lay, proj, convw, A_log, dt_bias, KD, VD = _lin_inputs(tree, HK, HV, seed=2000 + i)
    d = lambda a: torch.as_tensor(a).to(dev).contiguous()  # noqa: E731
    q, k, v, g, beta = ext.linattn_prep_dedup2(proj.to(dev), d(lay["hist"]), d(lay["rep_ptr"]), d(lay["rep_pos"]),
                                               lay["L2"], convw.to(dev), A_log.to(dev), dt_bias.to(dev), KD, VD, HV,
                                               HK, 128, rep_qk)
    torch.cuda.synchronize()
    rq_, rk_, rv_, rg_, rb_ = LO.linattn_prep(proj, lay["hist"], lay["rep_ptr"], lay["rep_pos"], lay["L2"], convw,
                                              A_log, dt_bias, KD, VD, HV, HK, 128, rep_qk)
    _ulp_close(v, rv_, "v", min_equal=0.98)
    _ulp_close(q, rq_, "q", steps=2, min_equal=0.98)
    _ulp_close(k, rk_, "k", steps=2, min_equal=0.98)
    _ulp_close(beta, rb_, "beta", min_equal=0.98)
    assert torch.allclose(g.cpu(), rg_, rtol=2e-6, atol=0), (g.cpu() - rg_).abs().max()
    pad = torch.as_tensor(lay["src"].reshape(-1) < 0)
    for tnsr in (q, k, v, g, beta):
        assert bool((tnsr.cpu()[pad] == 0).all())
