"""ojx_gemm_residual_rmsnorm_noalloc: the residual projection + RMSNorm with its kernels' scratch in the library's
static device array (no workspace argument, no allocation). Called through the C-ABI and compared bit-exactly with
ojx_gemm_residual_rmsnorm run with the same configuration and a workspace of its own, on consecutive calls (the
second with a smaller input, so stale scratch from the first call is present), plus the oracle at the north-star
tolerance and the error for a configuration whose workspace exceeds the scratch."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

SCRATCH = 32 << 20
TOL = dict(max_rel=1e-2, mean_abs_rms=1e-3)


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _inputs(M, N, K, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=dev).bfloat16()
    w = (torch.randn(N, K, generator=g, device=dev) * 0.01).bfloat16()
    res = torch.randn(M, N, generator=g, device=dev).bfloat16()
    w1 = (1.0 + 0.1 * torch.randn(N, generator=g, device=dev)).float()
    mask = (torch.rand(M, generator=g, device=dev) > 0.2).int()
    return x, w, res, w1, mask


def _noalloc(L, x, w, res, w1, mask, cfg):
    M, K = x.shape
    N = w.shape[0]
    h, hn = torch.empty_like(res), torch.empty_like(res)
    rc = L.ojx_gemm_residual_rmsnorm_noalloc(_p(x), _p(w), _p(res), _p(w1), _p(mask), 1e-6, _p(h), _p(hn), M, N, K,
                                             ctypes.byref(cfg) if cfg is not None else None,
                                             ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    return rc, h, hn


def _with_workspace(pkg, L, x, w, res, w1, mask, cfg):
    M, K = x.shape
    N = w.shape[0]
    nws = pkg._lib.workspace_bytes(M, N, K, 2, cfg)
    ws = torch.empty(max(nws, 256), dtype=torch.uint8, device=x.device)
    h, hn = torch.empty_like(res), torch.empty_like(res)
    rc = L.ojx_gemm_residual_rmsnorm(_p(x), _p(w), _p(res), _p(w1), _p(mask), 1e-6, _p(h), _p(hn), M, N, K, _p(ws),
                                     nws, ctypes.byref(cfg), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    pkg._lib.check(rc)
    return h, hn


def _fitted_plan(pkg, M, N, K):
    """The configuration the entry point documents for cfg == NULL: the plan with its split lowered until it fits."""
    c = pkg._lib.plan(M, N, K, 2)
    while c.splitk > 1:
        n = pkg._lib.lib().ojx_workspace_bytes(M, N, K, 2, ctypes.byref(c))
        if 0 <= n <= SCRATCH:
            break
        c = pkg._lib.cfg(c.tile, c.splitk - 1)
    assert 0 <= pkg._lib.workspace_bytes(M, N, K, 2, c) <= SCRATCH
    return c


def test_noalloc_matches_workspace_entry_point(pkg, O, dev):
    L = pkg._lib.lib()
    cases = [
        # (M, N, K, cfg or None): a plan that must be lowered to fit (o_proj at M = 288), a stream-K configuration
        # with partial tiles in the scratch, then smaller calls after larger ones
        (288, 5120, 6144, None),
        (288, 5120, 17408, pkg._lib.cfg(79, 2)),
        (64, 5120, 17408, None),
        (7, 5120, 6144, None),
    ]
    for i, (M, N, K, cfg) in enumerate(cases):
        print(f"case noalloc M={M} N={N} K={K} cfg={cfg}", flush=True)
        x, w, res, w1, mask = _inputs(M, N, K, dev, seed=i + 1)
        want_cfg = cfg if cfg is not None else _fitted_plan(pkg, M, N, K)
        assert pkg._lib.workspace_bytes(M, N, K, 2, want_cfg) > 0, "case must use the scratch"
        rc, h, hn = _noalloc(L, x, w, res, w1, mask, cfg)
        pkg._lib.check(rc)
        eh, ehn = _with_workspace(pkg, L, x, w, res, w1, mask, want_cfg)
        torch.cuda.synchronize()
        assert torch.equal(h, eh) and torch.equal(hn, ehn), f"case {i}: differs from the workspace entry point"
        rows = torch.arange(0, M, max(1, M // 16), device=dev)
        rh, rhn = O.residual_proj(res[rows].cpu(), x[rows].cpu(), w.cpu(), w1.cpu(), mask[rows].cpu(), 1e-6)
        for name, a, b in (("h", h[rows], rh), ("hn", hn[rows], rhn)):
            ok, e1, e2 = O.tolerance_ok(a.cpu(), b, **TOL)
            assert ok, f"case {i} {name}: max_rel {e1:.3e} mean/rms {e2:.3e}"


def test_noalloc_rejects_oversize_cfg_and_replays_in_graph(pkg, dev):
    L = pkg._lib.lib()
    M, N, K = 288, 5120, 17408
    x, w, res, w1, mask = _inputs(M, N, K, dev, seed=9)
    big = pkg._lib.cfg(79, 8)
    assert pkg._lib.workspace_bytes(M, N, K, 2, big) > SCRATCH
    rc, _, _ = _noalloc(L, x, w, res, w1, mask, big)
    assert rc == 3 and b"static scratch" in L.ojx_last_error()
    # capture: the call allocates nothing, so it records as plain kernel launches; replays equal the eager call
    cfg = pkg._lib.cfg(79, 2)
    rc, eh, ehn = _noalloc(L, x, w, res, w1, mask, cfg)
    pkg._lib.check(rc)
    h, hn = torch.empty_like(res), torch.empty_like(res)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        rc = L.ojx_gemm_residual_rmsnorm_noalloc(_p(x), _p(w), _p(res), _p(w1), _p(mask), 1e-6, _p(h), _p(hn), M, N,
                                                 K, ctypes.byref(cfg), ctypes.c_void_p(s.cuda_stream))
    pkg._lib.check(rc)
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(h, eh) and torch.equal(hn, ehn), f"replay {r}"
        rc, _, _ = _noalloc(L, x[:7].contiguous(), w, res[:7].contiguous(), w1, mask[:7].contiguous(), None)
        pkg._lib.check(rc)  # eager use of the same scratch between replays
        torch.cuda.synchronize()
