"""GPU parity of the planned calls on seeded random shapes outside the plan table (ojx_plan's heuristic picks the
configuration), row-major and packed weights, against the CPU oracle, through the C-ABI.

Each case draws M in [1, 700], N a multiple of 16 in [16, 3072] (gate-up: 2 I with I a multiple of 8), K a multiple
of 64 in [64, 2048] (and, row-major only, a multiple of 8 in [8, 2400]) from a fixed seed, so the set is the same on
every run. Tolerance:
max |out - ref| / max |ref| <= 1e-2 and mean |out - ref| <= 1e-3 * RMS(ref).
"""
import random

import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = dict(max_rel=1e-2, mean_abs_rms=1e-3)


def _cases(n=48, seed=2026):
    r = random.Random(seed)
    out = []
    for i in range(n):
        kind = ("plain", "silu", "residual")[i % 3]
        M = r.choice([r.randint(1, 16), r.randint(17, 160), r.randint(161, 700)])
        N = 16 * r.randint(1, 192)
        K = 64 * r.randint(1, 32)
        out.append((kind, M, N, K, bool(i % 2)))
    return out


def _ragged_cases(n=24, seed=7):
    """Row-major weights with K only a multiple of 8: the kernels' partial last K stage."""
    r = random.Random(seed)
    return [(("plain", "silu", "residual")[i % 3], r.randint(1, 700), 16 * r.randint(1, 192), 8 * r.randint(1, 300),
             False) for i in range(n)]


def _tol(O, out, ref, what):
    ok, a, b = O.tolerance_ok(out.float().cpu(), ref.float().cpu(), **TOL)
    assert ok, f"{what}: max_rel {a:.3e} mean/rms {b:.3e}"


@pytest.mark.parametrize("kind,M,N,K,packed", _cases() + _ragged_cases())
def test_planned_call_random_shape(ext, O, dev, kind, M, N, K, packed):
    print(f"case {kind} M={M} N={N} K={K} packed={packed}", flush=True)
    x, w = O.seeded_inputs(M, N, K, seed=M * 7 + N + K)
    xd, wd = x.to(dev), w.to(dev)
    if kind == "plain":
        y = ext.mm(xd, ext.pack_weight(wd) if packed else wd)
        _tol(O, y, O.linear_bf16(x, w), "plain")
    elif kind == "silu":
        I = N // 2
        wg, wu = w[:I], w[I:2 * I]
        gu = ext.pack_gate_up(wd[:I].contiguous(), wd[I:2 * I].contiguous())
        out = ext.mm_silu_mul(xd, ext.pack_weight(gu) if packed else gu)
        _tol(O, out, O.gate_up_silu(x, wg, wu), "gate-up")
    else:
        g = torch.Generator().manual_seed(M + N)
        res = torch.randn(M, N, generator=g).bfloat16()
        w1 = (1.0 + 0.1 * torch.randn(N, generator=g)).float()
        h, hn = ext.mm_residual_rmsnorm(res.to(dev), xd, ext.pack_weight(wd) if packed else wd, w1.to(dev), None,
                                        1e-6)
        rh, rhn = O.residual_proj(res, x, w, w1, None, 1e-6)
        _tol(O, h, rh, "h")
        _tol(O, hn, rhn, "hn")
