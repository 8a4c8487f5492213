"""Tensors past 2 GiB through the C-ABI: row-major weights, activations and outputs each larger than 2^31 bytes.

Every kernel addresses its operands through buffer descriptors based at the tile it works on (32-bit offsets inside
one tile), and its stores through 64-bit pointers; these cases check that no index wraps when the whole tensor is
larger than a 32-bit byte offset reaches. Each runs the plan and three more configurations from the library's
candidate list, and every element is compared with the oracle's arithmetic on the GPU tensors (torch fp32 GEMM)
within the north star's tolerance. (Packed weights are limited to 2 GiB by ojx_pack_weight; that limit is an
error-path check here.)
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = dict(max_rel=1e-2, mean_abs_rms=1e-3)
GIB2 = 1 << 31


def _say(*a):
    print(*a, flush=True)


def _configs(L, M, N, K, kind, seed):
    cands = L.candidates(M, N, K, kind)
    pick = np.random.default_rng(seed).choice(len(cands), size=min(3, len(cands)), replace=False)
    return [None] + [cands[int(i)] for i in pick]


def _check(O, got, want, what):
    ok, a, b = O.tolerance_ok(got, want, **TOL)
    assert ok, f"{what}: max_rel {a:.3e} mean/rms {b:.3e}"


@pytest.mark.parametrize("M,N,K,what", [
    (16, 73728, 16384, "weight"),     # W 2.25 GiB
    (300, 73728, 16384, "weight"),
    (65536, 256, 17408, "x"),         # x 2.125 GiB
    (65536, 16384, 512, "y"),         # y exactly 2^31 bytes
    (65600, 16384, 512, "y"),         # y past 2^31 bytes
])
def test_plain_past_2gib(pkg, ext, O, dev, M, N, K, what):
    L = pkg._lib
    g = torch.Generator(device=dev).manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g, device=dev).bfloat16()
    w = (torch.randn(N, K, generator=g, device=dev) * K ** -0.5).bfloat16()
    big = {"weight": w, "x": x}.get(what)
    assert big is None or big.numel() * 2 > GIB2
    assert what != "y" or M * N * 2 >= GIB2
    ref = O.linear_bf16(x, w)
    for cfg in _configs(L, M, N, K, 0, M):
        _say(f"case limits plain {what} M={M} N={N} K={K} cfg={cfg}")
        y = ext.mm(x, w, cfg=cfg)
        _check(O, y, ref, f"{what} cfg {cfg}")
        del y
    torch.cuda.synchronize()


def test_residual_x_past_2gib(pkg, ext, O, dev):
    """The down projection's shape (N = 5120, K = 17408) at M = 65536: x 2.125 GiB, split-K planes past 2 GiB."""
    L = pkg._lib
    M, N, K = 65536, 5120, 17408
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn(M, K, generator=g, device=dev).bfloat16()
    w = (torch.randn(N, K, generator=g, device=dev) * K ** -0.5).bfloat16()
    res = torch.randn(M, N, generator=g, device=dev).bfloat16()
    w1 = (1.0 + 0.1 * torch.randn(N, generator=g, device=dev)).float()
    mask = (torch.rand(M, generator=g, device=dev) > 0.25).int()
    rh, rhn = O.residual_proj(res, x, w, w1, mask, 1e-6)
    for cfg in _configs(L, M, N, K, L.KIND_RESIDUAL, 3):
        _say(f"case limits residual M={M} N={N} K={K} cfg={cfg}")
        h, hn = ext.mm_residual_rmsnorm(res, x, w, w1, mask, 1e-6, cfg=cfg)
        _check(O, h, rh, f"h cfg {cfg}")
        _check(O, hn, rhn, f"hn cfg {cfg}")
        assert int(hn[mask == 0].count_nonzero()) == 0
        del h, hn
    torch.cuda.synchronize()


def test_packed_weight_limit(pkg, ext, dev):
    """ojx_pack_weight refuses a weight of 2 GiB or more (its layout is addressed with 32-bit offsets)."""
    _say("case limits packed weight refused")
    w = torch.empty(65536, 16384, dtype=torch.bfloat16, device=dev)  # exactly 2 GiB, contents not read
    with pytest.raises(RuntimeError, match="2 GiB"):
        ext.pack_weight(w)
