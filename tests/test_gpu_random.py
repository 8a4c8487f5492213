"""Seeded random cases through the C-ABI: random shapes (ragged M, N, K), random kinds (plain, SiLU.mul, residual +
RMSNorm with a row mask), row-major or packed weights, and a random configuration drawn from the library's own
candidate list (tile, split-K count or stream-K spread, one-launch variants), or the plan. Every element is checked
against the oracle's arithmetic run on the GPU tensors (torch fp32 GEMM) within the north star's tolerance, so a
tile, split or epilogue combination that the fixed-shape tests do not reach is still exercised. The case list is
fixed by the seed (the same cases on every run).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = dict(max_rel=1e-2, mean_abs_rms=1e-3)
N_CASES = int(__import__("os").environ.get("OJX_RANDOM_CASES", "160"))


def _cases():
    rng = np.random.default_rng(int(__import__("os").environ.get("OJX_RANDOM_SEED", "20261202")))
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


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"c{c[0]}-k{c[1]}-{'pk' if c[2] else 'rm'}-{c[3]}x{c[4]}x{c[5]}")
def test_random_case_vs_oracle(pkg, ext, O, dev, case):
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
        ref = O.gate_up_silu(x, gate, up)
        ok, a, b = O.tolerance_ok(out.float().cpu(), ref.float().cpu(), **TOL)
        assert ok, f"silu: max_rel {a:.3e} mean/rms {b:.3e}"
    elif kind == 0:
        y = ext.mm(x, ext.pack_weight(w) if packed else w, cfg=cfg)
        ok, a, b = O.tolerance_ok(y.float().cpu(), O.linear_bf16(x, w).float().cpu(), **TOL)
        assert ok, f"plain: max_rel {a:.3e} mean/rms {b:.3e}"
    else:
        res = torch.randn(M, N, generator=g, device=dev).bfloat16()
        w1 = (1.0 + 0.1 * torch.randn(N, generator=g, device=dev)).float()
        mask = (torch.rand(M, generator=g, device=dev) > 0.25).int()
        h, hn = ext.mm_residual_rmsnorm(res, x, ext.pack_weight(w) if packed else w, w1, mask, 1e-6, cfg=cfg)
        rh, rhn = O.residual_proj(res, x, w, w1, mask, 1e-6)
        for got, want, what in ((h, rh, "h"), (hn, rhn, "hn")):
            ok, a, b = O.tolerance_ok(got.float().cpu(), want.float().cpu(), **TOL)
            assert ok, f"residual {what}: max_rel {a:.3e} mean/rms {b:.3e}"
        assert int(hn[mask == 0].count_nonzero()) == 0
    torch.cuda.synchronize()
