"""Seeded random cases through the C-ABI: random shapes (ragged M, N, K), random kinds (plain, SiLU.mul, residual +
RMSNorm with a row mask), row-major or packed weights, and a random configuration drawn from the library's own
candidate list (tile, split-K count or stream-K spread, one-launch variants), or the plan. Every element is checked
against the oracle's arithmetic run on the GPU tensors (torch fp32 GEMM) within the north star's tolerance, so a
tile, split or epilogue combination that the fixed-shape tests do not reach is still exercised. The case list is
fixed by the seed (the same cases on every run). A second, smaller set draws full-size grids (M up to 2048, N and K
up to the model's projection sizes), where a tile's split-K or stream-K bookkeeping spans hundreds of workgroups;
its comparison stays on the GPU.
"""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = dict(max_rel=1e-2, mean_abs_rms=1e-3)
N_CASES = int(os.environ.get("OJX_RANDOM_CASES", "160"))
N_LARGE = int(os.environ.get("OJX_RANDOM_LARGE_CASES", "24"))
SEED = int(os.environ.get("OJX_RANDOM_SEED", "20261202"))


def _cases():
    rng = np.random.default_rng(SEED)
    out = []
    for i in range(N_CASES):
        kind = int(rng.integers(0, 3))
        packed = bool(rng.integers(0, 2))
        M = int(rng.choice([1, 3, 7, 16, 31, 64, 100, 128, 200, 288, 301, 539]))
        if packed:
            N = 16 * int(rng.integers(1, 160))
            K = 64 * int(rng.integers(1, 40))
        else:
            N = 8 * int(rng.integers(1, 320))
            K = 8 * int(rng.integers(1, 320))
        if kind == 1 and N % 16:  # gate/up pairs come in blocks of 8 packed rows
            N += 8
        out.append((i, kind, packed, M, N, K, int(rng.integers(0, 1 << 30))))
    return out


def _say(*a):
    print(*a, flush=True)


def _large_cases():
    rng = np.random.default_rng(SEED + 1)
    out = []
    for i in range(N_LARGE):
        kind = int(rng.integers(0, 3))
        packed = bool(rng.integers(0, 2))
        M = int(rng.choice([200, 288, 539, 1024, 1500, 2048]))
        while True:
            if packed:
                N, K = 16 * int(rng.integers(64, 2177)), 64 * int(rng.integers(16, 273))
            else:
                N, K = 8 * int(rng.integers(128, 4353)), 8 * int(rng.integers(128, 2177))
            if kind == 1 and N % 16:
                N += 8
            if N * K <= 100_000_000 and (kind != 2 or N <= 8192):  # the residual row pass holds N/8 <= 1024 lanes
                break
        out.append((i, kind, packed, M, N, K, int(rng.integers(0, 1 << 30))))
    return out


def _check(O, got, want, what, cpu=True):
    if cpu:
        got, want = got.float().cpu(), want.float().cpu()
    ok, a, b = O.tolerance_ok(got, want, **TOL)
    assert ok, f"{what}: max_rel {a:.3e} mean/rms {b:.3e}"


def _run_case(pkg, ext, O, dev, case, cpu=True):
    i, kind, packed, M, N, K, seed = case
    L = pkg._lib
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=dev).bfloat16()
    w = (torch.randn(N, K, generator=g, device=dev) * K ** -0.5).bfloat16()
    cands = L.candidates(M, N, K, kind | (L.KIND_PACKED if packed else 0))
    pick = int(np.random.default_rng(seed).integers(0, len(cands) + 1))
    cfg = cands[pick] if pick < len(cands) else None  # None: the plan
    _say(f"case random {i}: kind={kind} packed={packed} M={M} N={N} K={K} cfg={cfg}")
    if kind == 1:
        gate, up = w[: N // 2].contiguous(), w[N // 2:].contiguous()
        wgu = ext.pack_gate_up(gate, up)
        out = ext.mm_silu_mul(x, ext.pack_weight(wgu) if packed else wgu, cfg=cfg)
        _check(O, out, O.gate_up_silu(x, gate, up), "silu", cpu)
    elif kind == 0:
        y = ext.mm(x, ext.pack_weight(w) if packed else w, cfg=cfg)
        _check(O, y, O.linear_bf16(x, w), "plain", cpu)
    else:
        res = torch.randn(M, N, generator=g, device=dev).bfloat16()
        w1 = (1.0 + 0.1 * torch.randn(N, generator=g, device=dev)).float()
        mask = (torch.rand(M, generator=g, device=dev) > 0.25).int()
        h, hn = ext.mm_residual_rmsnorm(res, x, ext.pack_weight(w) if packed else w, w1, mask, 1e-6, cfg=cfg)
        rh, rhn = O.residual_proj(res, x, w, w1, mask, 1e-6)
        _check(O, h, rh, "residual h", cpu)
        _check(O, hn, rhn, "residual hn", cpu)
        assert int(hn[mask == 0].count_nonzero()) == 0
    torch.cuda.synchronize()


_ID = lambda c: f"c{c[0]}-k{c[1]}-{'pk' if c[2] else 'rm'}-{c[3]}x{c[4]}x{c[5]}"  # noqa: E731


@pytest.mark.parametrize("case", _cases(), ids=_ID)
def test_random_case_vs_oracle(pkg, ext, O, dev, case):
    _run_case(pkg, ext, O, dev, case)


@pytest.mark.parametrize("case", _large_cases(), ids=_ID)
def test_random_large_case_vs_oracle(pkg, ext, O, dev, case):
    _run_case(pkg, ext, O, dev, case, cpu=False)
