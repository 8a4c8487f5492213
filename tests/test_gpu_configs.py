"""GPU parity at the BASELINE configurations, through the C-ABI, against the CPU oracle.

* every row of the plan table (csrc/plan_table.inc) at its full size: BASELINE configs[3]'s M sweep on the five
  projection shapes plus the real lin-in N = 16480, and configs[0] (5120 x 5120), each with the plan's own tile,
  split-K / stream-K spread and tail. Outputs are checked against the oracle on sampled rows and columns (every
  output row of a projection depends only on its own input row, and every output column on its own weight row, so
  a sample is checked exactly as the full product would be), and every element against a second, independent
  configuration of the library (the skinny family-0 tile without split-K), within the same tolerance;
* configs[0] in full against the oracle;
* the 64-layer projection stack at M = 539 captured in one HIP graph, replays bit-equal to the eager
  run, the first layer and the last layer checked against the oracle;
* the drop-in shim (FastProjections / lt_ext) called the way src/fastmodel.py calls it;
* a graph that keeps using its workspace after an eager call grew the library's workspace.

Tolerance: max |out - ref| / max |ref| <= 1e-2 and mean |out - ref| <= 1e-3 * RMS(ref).
"""
import os
import re

import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOL = dict(max_rel=1e-2, mean_abs_rms=1e-3)
KIND = {"plain": 0, "silu": 1, "residual": 2}


def _say(*a):
    print(*a, flush=True)


def _assert_tol(O, out, ref, what):
    ok, a, b = O.tolerance_ok(out.float().cpu(), ref.float().cpu(), **TOL)
    assert ok, f"{what}: max_rel {a:.3e} mean/rms {b:.3e}"


def plan_rows():
    """(M, N, K, kind) of every row of the plan table."""
    text = open(os.path.join(ROOT, "open-jev-fast_amd", "csrc", "plan_table.inc")).read()
    rows = []
    for m in re.finditer(r"^\{(\d+), (\d+), (\d+), (\d+),", text, re.M):
        rows.append(tuple(int(v) for v in m.groups()))
    return rows


def unpack_gate_up(packed):
    """(gate, up) [I, K] from the fused layout [2I, K] (rows in blocks of 8: 4 gate rows, then the same 4 up
    rows), the inverse of proj_oracle.pack_gate_up (checked against it in test_unpack_inverts_pack)."""
    I2, K = packed.shape
    v = packed.view(I2 // 8, 2, 4, K)
    return v[:, 0].reshape(I2 // 2, K), v[:, 1].reshape(I2 // 2, K)


def sample_idx(n, k, gen, extra=()):
    """k random indices of range(n) plus the first and last 8 and the given extras (sorted, unique)."""
    base = set(range(min(8, n))) | set(range(max(0, n - 8), n)) | {e for e in extra if 0 <= e < n}
    rnd = torch.randperm(n, generator=gen)[:k].tolist()
    return torch.tensor(sorted(base | set(rnd)), dtype=torch.long)


_W = {}


def weight(N, K, dev, std=0.02):
    """One seeded weight per shape, made on the GPU and kept for the module (full-size weights are 50-360 MB)."""
    key = (N, K, std)
    if key not in _W:
        g = torch.Generator(device=dev).manual_seed(N * 7 + K)
        _W[key] = (torch.randn(N, K, generator=g, device=dev) * std).bfloat16()
    return _W[key]


def test_unpack_inverts_pack(O):
    g, u = torch.randn(16, 24).bfloat16(), torch.randn(16, 24).bfloat16()
    gg, uu = unpack_gate_up(O.pack_gate_up(g, u))
    assert torch.equal(gg, g) and torch.equal(uu, u)


# --------------------------------------------------------------------------------------- every plan-table row
@pytest.mark.parametrize("M,N,K,kind", plan_rows(), ids=lambda v: str(v))
def test_plan_table_row_full_size(pkg, ext, O, dev, M, N, K, kind):
    """Rows of kind | 4 are plans for packed weights: the call goes through the *_pk entry point. Sampled rows and
    columns are checked against the oracle on the CPU; every element against the library's family-0 tile and
    against the oracle's own arithmetic run on the GPU tensors (torch fp32 GEMM, an implementation independent of
    this library)."""
    plan = pkg._lib.plan(M, N, K, kind)
    _say(f"case plan row M={M} N={N} K={K} kind={kind} plan={plan}")
    packed = bool(kind & 4)
    kind &= 3
    mm = ext.mm_pk if packed else ext.mm
    mm_silu = ext.mm_silu_mul_pk if packed else ext.mm_silu_mul
    mm_res = ext.mm_residual_rmsnorm_pk if packed else ext.mm_residual_rmsnorm
    gen = torch.Generator().manual_seed(M * 31 + N + K)
    gx = torch.Generator(device=dev).manual_seed(M + N)
    x = torch.randn(M, K, generator=gx, device=dev).bfloat16()
    w = weight(N, K, dev)
    wk = ext.pack_weight(w) if packed else w
    mrows = sample_idx(M, 24, gen, extra=(15, 16, 31, 32, 95, 96, 143, 144, 191, 192, 255, 256, 287, 288))
    xs = x[mrows.to(dev)].cpu()
    ref_cfg = pkg._lib.cfg(0, 1)
    if kind == 0:
        y = mm(x, wk)
        cols = sample_idx(N, 384, gen, extra=(N - plan.tail_rows - 1, N - plan.tail_rows) if plan.tail_rows else ())
        ref = O.linear_bf16(xs, w[cols.to(dev)].cpu())
        _assert_tol(O, y[mrows.to(dev)][:, cols.to(dev)], ref, "sampled vs oracle")
        _assert_tol(O, y, ext.mm(x, w, cfg=ref_cfg), "every element vs the family-0 tile")
        _assert_tol(O, y, O.linear_bf16(x, w), "every element vs the oracle (its fp32 GEMM run on the GPU)")
    elif kind == 1:
        I = N // 2
        out = mm_silu(x, wk)
        tail_col = (N - plan.tail_rows) // 2
        cols = sample_idx(I, 384, gen, extra=(tail_col - 1, tail_col) if plan.tail_rows else ())
        gate, up = unpack_gate_up(w)
        ref = O.gate_up_silu(xs, gate[cols.to(dev)].cpu(), up[cols.to(dev)].cpu())
        _assert_tol(O, out[mrows.to(dev)][:, cols.to(dev)], ref, "sampled vs oracle")
        _assert_tol(O, out, ext.mm_silu_mul(x, w, cfg=ref_cfg), "every element vs the family-0 tile")
        _assert_tol(O, out, O.gate_up_silu(x, gate, up), "every element vs the oracle (on the GPU)")
    else:
        res = torch.randn(M, N, generator=gx, device=dev).bfloat16()
        w1 = (1.0 + 0.1 * torch.randn(N, generator=gx, device=dev)).float()
        mask = (torch.rand(M, generator=gx, device=dev) > 0.2).int()
        h, hn = mm_res(res, x, wk, w1, mask, 1e-6)
        rh, rhn = O.residual_proj(res[mrows.to(dev)].cpu(), xs, w.cpu(), w1.cpu(), mask[mrows.to(dev)].cpu(), 1e-6)
        _assert_tol(O, h[mrows.to(dev)], rh, "h sampled rows vs oracle")
        _assert_tol(O, hn[mrows.to(dev)], rhn, "hn sampled rows vs oracle")
        h2, hn2 = ext.mm_residual_rmsnorm(res, x, w, w1, mask, 1e-6, cfg=ref_cfg)
        _assert_tol(O, h, h2, "h every element vs the family-0 tile")
        _assert_tol(O, hn, hn2, "hn every element vs the family-0 tile")
        rh_all, rhn_all = O.residual_proj(res, x, w, w1, mask, 1e-6)
        _assert_tol(O, h, rh_all, "h every element vs the oracle (on the GPU)")
        _assert_tol(O, hn, rhn_all, "hn every element vs the oracle (on the GPU)")
        assert int(hn[mask == 0].count_nonzero()) == 0, "masked rows of hn must be zero"
    torch.cuda.synchronize()


def test_config0_single_linear_full(pkg, ext, O, dev):
    """y = x W^T, M = 288, K = N = 5120, x ~ N(0,1), W ~ N(0, 0.02^2), every element against
    the oracle."""
    M, N, K = 288, 5120, 5120
    _say(f"case configs[0] plan={pkg._lib.plan(M, N, K, 0)}")
    x, w = O.seeded_inputs(M, N, K, seed=100)
    y = ext.mm(x.to(dev), w.to(dev))
    _assert_tol(O, y, O.linear_bf16(x, w), "configs[0]")


# --------------------------------------------------------------------------------------- the 64-layer stack
def _stack_layer_oracle(O, rows, h, hn, y_att, d, w1):
    """One layer of the stack on the CPU for the given rows (each output row depends only on its input row)."""
    proj = O.linear_bf16(hn, d["w_in"])
    h1, hn1 = O.residual_proj(h, y_att, d["w_out"], w1, None, 1e-6)
    gate, up = unpack_gate_up(d["w_gu"])
    m = O.gate_up_silu(hn1, gate, up)
    h2, hn2 = O.residual_proj(h1, m, d["w_dn"], w1, None, 1e-6)
    return proj, h1, hn1, m, h2, hn2


def test_stack_64_layers_graph(pkg, ext, O, dev):
    """48 linear-attention + 16 full-attention layers (every fourth layer full), hidden 5120,
    MLP 17408, M = 539. Each layer runs in-proj, out-proj + residual + RMSNorm, gate-up + SiLU.mul and down +
    residual + RMSNorm back to back (the attention cores between in-proj and out-proj are outside the path: the
    out-proj reads a fixed activation). The whole forward is captured in one HIP graph; every replay is bit-equal to
    the eager run (with eager work in between), and the first and last layers match the oracle on sampled rows."""
    M, H, I = 539, 5120, 17408
    lin_in, full_in, out_k = 16384, 14336, 6144
    layers = []
    for i in range(64):
        g = torch.Generator(device=dev).manual_seed(1000 + i)
        n_in = full_in if i % 4 == 3 else lin_in
        layers.append({k: (torch.randn(*s, generator=g, device=dev) * 0.02).bfloat16() for k, s in
                       (("w_in", (n_in, H)), ("w_out", (H, out_k)), ("w_gu", (2 * I, H)), ("w_dn", (H, I)))})
    g = torch.Generator(device=dev).manual_seed(5)
    h0 = torch.randn(M, H, generator=g, device=dev).bfloat16()
    hn0 = torch.randn(M, H, generator=g, device=dev).bfloat16()
    y_att = torch.randn(M, out_k, generator=g, device=dev).bfloat16()
    w1 = (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).float()

    def forward(trace=None):
        h, hn = h0, hn0
        for i, d in enumerate(layers):
            proj = ext.mm(hn, d["w_in"])
            h1, hn1 = ext.mm_residual_rmsnorm(h, y_att, d["w_out"], w1, None, 1e-6)
            m = ext.mm_silu_mul(hn1, d["w_gu"])
            if trace is not None:
                trace.append((h, hn, proj, h1, hn1, m))
            h, hn = ext.mm_residual_rmsnorm(h1, m, d["w_dn"], w1, None, 1e-6)
        return h, hn

    _say("case stack eager")
    trace = []
    eh, ehn = forward(trace)
    eh, ehn = eh.clone(), ehn.clone()
    torch.cuda.synchronize()
    rows = sample_idx(M, 6, torch.Generator().manual_seed(3), extra=(538,)).to(dev)
    for li in (0, 63):
        d = {k: v.cpu() for k, v in layers[li].items()}
        h_in, hn_in = trace[li][0], trace[li][1]
        _say(f"case stack layer {li} vs oracle")
        want = _stack_layer_oracle(O, rows, h_in[rows].cpu(), hn_in[rows].cpu(), y_att[rows].cpu(), d, w1.cpu())
        h_out, hn_out = (trace[li + 1][0], trace[li + 1][1]) if li < 63 else (eh, ehn)
        got = (trace[li][2], trace[li][3], trace[li][4], trace[li][5], h_out, hn_out)
        for name, a, b in zip(("proj", "h_att", "hn_att", "m", "h", "hn"), got, want):
            _assert_tol(O, a[rows], b, f"layer {li} {name}")
    del trace

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        forward()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    _say("case stack capture")
    with torch.cuda.graph(graph):
        gh, ghn = forward()
    for r in range(3):
        _say(f"case stack replay {r}")
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gh, eh) and torch.equal(ghn, ehn), f"replay {r} differs from the eager forward"
        junk = ext.mm_silu_mul(hn0, layers[r]["w_gu"])  # eager work between replays
        torch.cuda.synchronize()
        del junk
    del graph, layers
    torch.cuda.empty_cache()


def test_stack_64_layers_packed_fastproj(pkg, ext, O, dev):
    """The same 64-layer stack (M = 539) the way a FastQwen35-shaped model runs it: weights
    merged and packed at load by FastProjections.merge_linear_attn / merge_full_attn / merge_mlp (the layout
    bench.py --stack times), and each layer driven through _mm, _res, _mm_silu and _res (src/fastmodel.py:412,
    477-481). One HIP graph of the whole forward; three replays bit-equal to the eager run, with eager work in
    between; the first and last layers against the oracle (row-major weights kept on the CPU for those two) on
    sampled rows."""
    fp, _ = _fastproj(pkg)
    M, H, I = 539, 5120, 17408
    lin_in, full_in, out_k = 16384, 14336, 6144
    P = fp.FastProjections(eps=1e-6)
    layers, keep = [], {}
    for i in range(64):
        g = torch.Generator(device=dev).manual_seed(2000 + i)
        full = i % 4 == 3
        n_in = full_in if full else lin_in
        w_in, w_out = [(torch.randn(*s, generator=g, device=dev) * 0.02).bfloat16() for s in ((n_in, H), (H, out_k))]
        gate, up, w_dn = [(torch.randn(*s, generator=g, device=dev) * 0.02).bfloat16() for s in ((I, H), (I, H), (H, I))]
        d = P.merge_mlp(gate, up, w_dn)
        if full:   # cat[q, k, v]: q + gate rows, then k, then v
            P.merge_full_attn(d, w_in[:12288], w_in[12288:13312], w_in[13312:], w_out)
        else:      # cat[qkv, z, b, a]
            P.merge_linear_attn(d, w_in[:10240], w_in[10240:16288], w_in[16288:16336], w_in[16336:], w_out)
        assert d.w_in.dim() == 4 and d.w_out.dim() == 4 and d.w_gu_packed.dim() == 4 and d.w_down.dim() == 4
        if i in (0, 63):
            keep[i] = {"w_in": w_in.cpu(), "w_out": w_out.cpu(), "w_gu": ext.pack_gate_up(gate, up).cpu(),
                       "w_dn": w_dn.cpu()}
        del w_in, w_out, gate, up, w_dn
        layers.append(d)
    g = torch.Generator(device=dev).manual_seed(6)
    h0 = torch.randn(M, H, generator=g, device=dev).bfloat16()
    hn0 = torch.randn(M, H, generator=g, device=dev).bfloat16()
    y_att = torch.randn(M, out_k, generator=g, device=dev).bfloat16()
    w1 = (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).float()

    def forward(trace=None):
        h, hn = h0, hn0
        for d in layers:
            proj = P._mm(hn, d.w_in)
            h1, hn1 = P._res(h, y_att, d.w_out_sk, d.sk_out, w1, None)
            m = P._mm_silu(hn1, d.w_gu_packed)
            if trace is not None:
                trace.append((h, hn, proj, h1, hn1, m))
            h, hn = P._res(h1, m, d.w_down_sk, d.sk_down, w1, None)
        return h, hn

    _say("case packed stack eager")
    trace = []
    eh, ehn = forward(trace)
    eh, ehn = eh.clone(), ehn.clone()
    torch.cuda.synchronize()
    rows = sample_idx(M, 6, torch.Generator().manual_seed(4), extra=(538,)).to(dev)
    for li in (0, 63):
        h_in, hn_in = trace[li][0], trace[li][1]
        _say(f"case packed stack layer {li} vs oracle")
        want = _stack_layer_oracle(O, rows, h_in[rows].cpu(), hn_in[rows].cpu(), y_att[rows].cpu(), keep[li],
                                   w1.cpu())
        h_out, hn_out = (trace[li + 1][0], trace[li + 1][1]) if li < 63 else (eh, ehn)
        got = (trace[li][2], trace[li][3], trace[li][4], trace[li][5], h_out, hn_out)
        for name, a, b in zip(("proj", "h_att", "hn_att", "m", "h", "hn"), got, want):
            _assert_tol(O, a[rows], b, f"layer {li} {name}")
    del trace, keep

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        forward()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    _say("case packed stack capture")
    with torch.cuda.graph(graph):
        gh, ghn = forward()
    for r in range(3):
        _say(f"case packed stack replay {r}")
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gh, eh) and torch.equal(ghn, ehn), f"replay {r} differs from the eager forward"
        junk = P._mm_silu(hn0, layers[r].w_gu_packed)  # eager work between replays
        torch.cuda.synchronize()
        del junk
    del graph, layers
    torch.cuda.empty_cache()


# --------------------------------------------------------------------------------------- drop-in shim
def _fastproj(pkg):
    from importlib import import_module
    return import_module("open_jev_fast_amd.fastproj"), import_module("open_jev_fast_amd.lt_ext")


def test_fastprojections_reference_call_pattern(pkg, ext, O, dev, monkeypatch):
    """One layer of forward_gtree (src/fastmodel.py:412, 477-481) through FastProjections at M = 288, with the
    reference's own per-layer state: d.sk_out = d.sk_down = 2 and d.w_*_sk = self._split(W, 2)
    (src/fastmodel.py:91-109). With no OJ_SK_* variable set, _res must run the plan table's configuration (bit-equal
    to the fused call with the plan); with OJ_SK_DOWN set, split-K 2. Both against the oracle on sampled rows."""
    for v in ("OJ_SK_LIN_OUT", "OJ_SK_FULL_OUT", "OJ_SK_DOWN"):
        monkeypatch.delenv(v, raising=False)
    fp, _ = _fastproj(pkg)
    M, H, I, n_in, k_out = 288, 5120, 17408, 16384, 6144
    P = fp.FastProjections(eps=1e-6)
    g = torch.Generator(device=dev).manual_seed(77)
    w_in = (torch.randn(n_in, H, generator=g, device=dev) * 0.02).bfloat16()
    w_out = (torch.randn(H, k_out, generator=g, device=dev) * 0.02).bfloat16()
    w_gate = (torch.randn(I, H, generator=g, device=dev) * 0.02).bfloat16()
    w_up = (torch.randn(I, H, generator=g, device=dev) * 0.02).bfloat16()
    w_down = (torch.randn(H, I, generator=g, device=dev) * 0.01).bfloat16()
    d = fp.FastProjections.merge_mlp(w_gate, w_up, w_down, keep_cat=True)
    d.sk_down, d.w_down_sk = 2, P._split(w_down, 2)
    d.sk_out, d.w_out_sk = 2, P._split(w_out, 2)
    h = torch.randn(M, H, generator=g, device=dev).bfloat16()
    hn = torch.randn(M, H, generator=g, device=dev).bfloat16()
    y = torch.randn(M, k_out, generator=g, device=dev).bfloat16()
    w1 = (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).float()
    mask = (torch.rand(M, generator=g, device=dev) > 0.1).int()

    _say("case shim layer, plan")
    proj = P._mm(hn, w_in)
    h1, hn1 = P._res(h, y, d.w_out_sk, d.sk_out, w1, None, d.w_out_sk)
    e1 = ext.mm_residual_rmsnorm(h, y, w_out, w1, None, 1e-6)
    assert torch.equal(h1, e1[0]) and torch.equal(hn1, e1[1]), "_res did not run the plan's configuration"
    m = P._silu_mul(P._mm(hn1, d.w_gu))
    m_fused = P._mm_silu(hn1, d.w_gu_packed)
    # the two paths may run tile families with different K summation orders: equal to rounding, both vs the oracle
    _assert_tol(O, m_fused, m, "fused gate-up vs GEMM -> silu_mul_lut")
    assert d.w_down.dim() == 4 and d.w_gu_packed.dim() == 4, "merge_mlp packs the weights by default"
    h2, hn2 = P._res(h1, m, d.w_down_sk, d.sk_down, w1, mask, w=d.w_down)
    e2 = ext.mm_residual_rmsnorm(h1, m, d.w_down, w1, mask, 1e-6)
    assert torch.equal(h2, e2[0]) and torch.equal(hn2, e2[1])

    rows = sample_idx(M, 8, torch.Generator().manual_seed(1)).to(dev)
    c = lambda t: t[rows].cpu()  # noqa: E731
    _assert_tol(O, c(proj), O.linear_bf16(c(hn), w_in.cpu()), "_mm in-proj")
    rh1, rhn1 = O.residual_proj(c(h), c(y), w_out.cpu(), w1.cpu(), None, 1e-6, S=2)
    _assert_tol(O, c(h1), rh1, "_res out h")
    _assert_tol(O, c(hn1), rhn1, "_res out hn")
    rm = O.gate_up_silu(c(hn1), w_gate.cpu(), w_up.cpu())
    _assert_tol(O, c(m), rm, "_silu_mul(_mm)")
    _assert_tol(O, c(m_fused), rm, "_mm_silu")
    rh2, rhn2 = O.residual_proj(c(h1), c(m), w_down.cpu(), w1.cpu(), c(mask), 1e-6, S=2)
    _assert_tol(O, c(h2), rh2, "_res down h")
    _assert_tol(O, c(hn2), rhn2, "_res down hn")

    _say("case shim layer, OJ_SK_DOWN=2")
    monkeypatch.setenv("OJ_SK_DOWN", "2")
    f2 = fp.FastProjections._forced_cfg(M, H, I, 2, packed=True)
    assert f2 is not None and f2.splitk == 2 and pkg._lib.tile_info(f2.tile)["family"] != 5
    h3, hn3 = P._res(h1, m, d.w_down_sk, d.sk_down, w1, mask, w=d.w_down)
    e3 = ext.mm_residual_rmsnorm(h1, m, d.w_down, w1, mask, 1e-6, cfg=f2)
    assert torch.equal(h3, e3[0]) and torch.equal(hn3, e3[1]), "OJ_SK_DOWN=2 not applied"
    _assert_tol(O, c(h3), rh2, "_res down h (split 2)")
    _assert_tol(O, c(hn3), rhn2, "_res down hn (split 2)")

    # the reference's own _split result [S, K/S, N] (src/fastmodel.py:186-188) is read back as W
    ref_layout = w_down.view(H, 2, I // 2).permute(1, 2, 0).contiguous()
    h4, hn4 = P._res(h1, m, ref_layout, 2, w1, mask)
    h5, hn5 = P._res(h1, m, w_down, 2, w1, mask)
    assert torch.equal(h4, h5) and torch.equal(hn4, hn5), "_res on the reference's split layout"
    _assert_tol(O, c(h4), rh2, "_res down h (reference split layout)")


@pytest.mark.parametrize("M", [7, 288, 539])
def test_fastprojections_skmm_and_lt(pkg, ext, O, dev, M):
    """_skmm (split-K fp32 planes; at M = 288 / 539 the residual plan's tile is persistent, which writes no planes,
    so the shim must hand the library -1) and the LT surface (lt_setup / lt_matmul / lt2_plan / lt2_search /
    lt2_run, src/lt.cpp:15-169) as _tune / _tune_sk drive them, on the down shape, against the oracle."""
    fp, lt_ext = _fastproj(pkg)
    H, I = 5120, 17408
    P = fp.FastProjections()
    g = torch.Generator(device=dev).manual_seed(M)
    y = torch.randn(M, I, generator=g, device=dev).bfloat16()
    w = weight(H, I, dev, std=0.01)
    rows = sample_idx(M, 8, torch.Generator().manual_seed(2)).to(dev)
    yc, wc = y[rows].cpu(), w.cpu()
    _say(f"case _skmm M={M}")
    parts = P._skmm(y, P._split(w, 2), 2)
    assert parts.shape == (2, M, H) and parts.dtype == torch.float32
    ref = O.splitk_parts(yc, wc, 2)
    for s in range(2):
        _assert_tol(O, parts[s][rows], ref[s], f"_skmm part {s}")

    LT = lt_ext.load()
    _say(f"case lt2 M={M}")
    hdl = LT.lt2_plan(M, H, I, 2, 1, 1)
    n = LT.lt2_search(hdl, 400, 3)
    assert n >= 1
    for i in sorted({0, n - 1}):
        p2 = LT.lt2_run(hdl, y, w, i)
        for s in range(2):
            _assert_tol(O, p2[s][rows], ref[s], f"lt2_run cand {i} part {s}")
    p3 = LT.lt2_run(hdl, y, w.view(H, 2, I // 2).permute(1, 2, 0).contiguous(), 0)  # the reference's layout
    assert torch.equal(p3, LT.lt2_run(hdl, y, w, 0))
    parts3 = P._skmm(y, w.view(H, 2, I // 2).permute(1, 2, 0).contiguous(), 2)
    assert torch.equal(parts3, parts)

    _say(f"case lt_matmul M={M}")
    x = y[:, :H].contiguous()
    wq = weight(14336, H, dev)
    na = LT.lt_setup(M, 14336, H, 32)
    assert 1 <= na <= 32
    refq = O.linear_bf16(x[rows].cpu(), wq.cpu())
    for i in sorted({0, na // 2, na - 1}):
        _assert_tol(O, LT.lt_matmul(x, wq, i)[rows], refq, f"lt_matmul {i}")
    _assert_tol(O, P._mm(x, wq)[rows], refq, "_mm")


# --------------------------------------------------------------------------------------- workspace lifetime
def test_graph_workspace_survives_growth(pkg, ext, O, dev):
    """A graph captured with the library's workspace keeps replaying correctly after an eager call has needed a
    larger workspace (the captured buffer must not go back to the allocator and be handed to other tensors)."""
    M, N, K = 64, 1024, 2048
    x, w = O.seeded_inputs(M, N, K, seed=4)
    xd, wd = x.to(dev), w.to(dev)
    cfg = pkg._lib.cfg(5, 4)   # split-K 4: fp32 planes in the workspace
    assert pkg._lib.workspace_bytes(M, N, K, 0, cfg) > 0
    eager = ext.mm(xd, wd, cfg=cfg).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ext.mm(xd, wd, cfg=cfg)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ext.mm(xd, wd, cfg=cfg)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, eager)
    # an eager call that needs a workspace far larger than the kept one
    Mb, Nb, Kb = 2048, 8192, 4096
    big_cfg = pkg._lib.cfg(5, 8)
    need = pkg._lib.workspace_bytes(Mb, Nb, Kb, 0, big_cfg)
    assert need > 64 << 20
    xb = torch.randn(Mb, Kb, device=dev).bfloat16()
    wb = (torch.randn(Nb, Kb, device=dev) * 0.02).bfloat16()
    ext.mm(xb, wb, cfg=big_cfg)
    torch.cuda.synchronize()
    # memory handed out now must not be the buffer the graph writes into
    fill = [torch.full((1 << 20,), 7.0, device=dev) for _ in range(64)]
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r} after growth differs"
        assert all(bool((f == 7.0).all()) for f in fill), "a replay wrote into memory owned by another tensor"
