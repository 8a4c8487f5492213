"""Pins the CPU oracle (oracle/proj_oracle.py) against independent checks: fp64 brute force, closed forms,
a second library's sigmoid (scipy), special values, and the reference's own bit-exactness claims
(tests/test_correct.py:44-45, bench/logs/correct.log:6-7). Each check is chosen so that a plausible mistake in
the oracle (a dropped rounding point, transposed W, a wrong split range, gate/up swapped) fails it."""
import os

import numpy as np
import pytest
import torch
from scipy.special import expit

from oracle import proj_oracle as O


def bits(t):
    return t.view(torch.int16).int()


# ------------------------------------------------------------------------------------------------ GEMM
@pytest.mark.parametrize("M,N,K", [(1, 8, 8), (3, 40, 72), (4, 64, 256), (16, 24, 264)])
def test_linear_vs_f64_bruteforce(M, N, K):
    x, w = O.seeded_inputs(M, N, K, seed=M * N)
    y = O.linear_bf16(x, w).double()
    ref = torch.from_numpy(O.linear_f64(x, w))
    # one bf16 rounding of an fp32-accurate value: |err| <= 2^-9 |ref| (+ fp32 accumulation slack)
    assert bool(((y - ref).abs() <= ref.abs() * 2.0 ** -8 + 1e-5).all())
    # and it is the correctly rounded value almost everywhere
    assert (O._bf16(ref.float()) == O.linear_bf16(x, w)).float().mean().item() > 0.98


def test_golden_vectors_match_oracle():
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "proj_golden.npz"))
    names = sorted({k.split("__")[0] for k in z.files})
    assert len(names) >= 5
    for name in names:
        x = torch.from_numpy(z[f"{name}__x"].view(np.int16)).view(torch.bfloat16)
        w = torch.from_numpy(z[f"{name}__w"].view(np.int16)).view(torch.bfloat16)
        ref = torch.from_numpy(z[f"{name}__y64"])
        y = O.linear_bf16(x, w).double()
        assert bool(((y - ref).abs() <= ref.abs() * 2.0 ** -8 + 1e-5).all()), name


def test_linear_identity_and_permutation_exact():
    x, _ = O.seeded_inputs(5, 8, 64, seed=2)
    eye = torch.eye(64).bfloat16()
    assert torch.equal(O.linear_bf16(x, eye), x)
    perm = torch.randperm(64, generator=torch.Generator().manual_seed(1))
    P = eye[perm]                       # row n of W selects x[:, perm[n]]
    assert torch.equal(O.linear_bf16(x, P), x[:, perm])
    # transposed-operand mistake check: a non-symmetric W gives x @ W^T, not x @ W
    W = torch.zeros(64, 64).bfloat16()
    W[0, 5] = 1.0
    assert torch.equal(O.linear_bf16(x, W)[:, 0], x[:, 5])


def test_linear_rank1_exact():
    # x[m, k] = a_m, W[n, k] = b_n with small integers: y = K a_m b_n exactly representable
    a = torch.tensor([1.0, -2.0, 3.0]).bfloat16()
    b = torch.tensor([0.5, 4.0, -1.0, 2.0, 0.25, 8.0, -0.5, 1.0]).bfloat16()
    K = 32
    x = a[:, None].expand(3, K).contiguous()
    w = b[:, None].expand(8, K).contiguous()
    assert torch.equal(O.linear_bf16(x, w).float(), K * a.float()[:, None] * b.float()[None, :])


def test_splitk_ranges_and_sum():
    assert O.split_ranges(17408, 2) == [(0, 8704), (8704, 17408)]
    assert O.split_ranges(6144, 3) == [(0, 2048), (2048, 4096), (4096, 6144)]
    assert O.split_ranges(64, 3) == [(0, 24), (24, 48), (48, 64)]
    x, w = O.seeded_inputs(6, 16, 2048, seed=4)
    parts = O.splitk_parts(x, w, 4)
    ref = torch.from_numpy(O.linear_f64(x, w))
    assert (parts.double().sum(0) - ref).abs().max().item() < 1e-4
    # each plane is the product over its own K range (the reference's view(M, S, K/S))
    xs = x.float().view(6, 4, 512).transpose(0, 1)
    ws = w.float().view(16, 4, 512).permute(1, 2, 0)
    assert (parts - torch.bmm(xs, ws)).abs().max().item() < 1e-5


# ------------------------------------------------------------------------------------------------ SiLU.mul
def test_silu_mul_vs_scipy():
    g = torch.Generator().manual_seed(3)
    gu = (torch.randn(64, 512, generator=g) * 3).bfloat16()
    out = O.silu_mul(gu)
    gd = gu[:, :256].double().numpy()
    ud = gu[:, 256:].double().numpy()
    s = torch.from_numpy(gd * expit(gd)).float().bfloat16().double().numpy()   # bf16(silu(g)) from fp64
    ref = torch.from_numpy(s * ud).float().bfloat16()
    diff = (bits(out) - bits(ref)).abs()
    assert int(diff.max()) <= 1 and (diff == 0).float().mean().item() > 0.99


def test_silu_mul_special_values():
    g = torch.tensor([0.0, -0.0, 100.0, -100.0, 1.0, float("inf"), float("nan"), -1.0]).bfloat16()
    u = torch.tensor([3.0, 3.0, 2.0, 2.0, 1.0, 1.0, 1.0, 0.0]).bfloat16()
    out = O.silu_mul(torch.cat([g, u])[None, :]).float()[0]
    assert out[0] == 0 and out[1] == 0
    assert out[2] == 200.0                                   # silu(g) = g for large g
    assert out[3] == 0 or abs(out[3].item()) < 1e-30         # silu(-100) * 2 underflows to ~0
    assert out[4].item() == torch.tensor(0.7310585786 * 1.0).bfloat16().float().item() or \
        abs(out[4].item() - 0.731058) < 4e-3
    assert out[5] == float("inf")
    assert torch.isnan(out[6])
    assert out[7] == 0


def test_act_tables_index_by_bits():
    silu_b, sig_f = O.act_tables()
    x = torch.tensor([0.0, 1.0, -2.0, 7.5]).bfloat16()
    idx = x.view(torch.int16).int() & 0xFFFF
    assert torch.equal(silu_b[idx.long()], O._bf16(x.float() / (1 + torch.exp(-x.float()))))
    assert torch.allclose(sig_f[idx.long()], torch.from_numpy(expit(x.double().numpy())).float())
    # table form == computed form for every finite bf16 input (src/kernels.cu:1284-1286 claim)
    allx = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    gu = torch.cat([allx[None, :], torch.ones_like(allx)[None, :]], 1)
    out = O.silu_mul(gu)[0]
    fin = torch.isfinite(silu_b.float())
    assert torch.equal(out[fin].view(torch.int16), silu_b[fin].view(torch.int16))
    assert bool(torch.isnan(out[~fin].float()).all() == torch.isnan(silu_b[~fin].float()).all())


def test_merged_gate_up_bitexact():
    """tests/test_correct.py:44: the merged [gate; up] GEMM equals the two GEMMs bit-exactly."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(16, 128, generator=g).bfloat16()
    wg = (torch.randn(32, 128, generator=g) * 0.02).bfloat16()
    wu = (torch.randn(32, 128, generator=g) * 0.02).bfloat16()
    gu = O.linear_bf16(x, torch.cat([wg, wu]))
    assert torch.equal(gu[:, :32], O.linear_bf16(x, wg)) and torch.equal(gu[:, 32:], O.linear_bf16(x, wu))
    # gate/up order matters: swapping them changes the result
    assert not torch.equal(O.gate_up_silu(x, wg, wu), O.gate_up_silu(x, wu, wg))


def test_pack_gate_up_layout():
    I, K = 8, 16
    gate = torch.arange(I * K).view(I, K).bfloat16()
    up = (1000 + torch.arange(I * K)).view(I, K).bfloat16()
    p = O.pack_gate_up(gate, up)
    assert torch.equal(p[0:4], gate[0:4]) and torch.equal(p[4:8], up[0:4])
    assert torch.equal(p[8:12], gate[4:8]) and torch.equal(p[12:16], up[4:8])


# ------------------------------------------------------------------------------------------------ RMSNorm
def test_add_rmsnorm_vs_f64():
    g = torch.Generator().manual_seed(8)
    M, H = 7, 5120
    x = torch.randn(M, H, generator=g).bfloat16()
    d = (torch.randn(M, H, generator=g) * 0.5).bfloat16()
    w1 = (1 + 0.1 * torch.randn(H, generator=g)).float()
    mask = torch.tensor([1, 0, 1, 1, 0, 1, 1]).int()
    h, hn = O.add_rmsnorm(x, d, w1, mask, 1e-6)
    v = (x.double() + d.double()).float().bfloat16().double()
    assert torch.equal(h, v.float().bfloat16())
    r = 1 / torch.sqrt((v * v).mean(1, keepdim=True) + 1e-6)
    ref = (v * r * w1.double()).float().bfloat16()
    keep = mask != 0
    diff = (bits(hn[keep]) - bits(ref[keep])).abs()
    assert int(diff.max()) <= 1
    assert bool((hn[~keep].float() == 0).all())


def test_add_rmsnorm_closed_forms():
    H = 64
    x = torch.full((2, H), 2.0).bfloat16()
    w1 = torch.ones(H)
    _, hn = O.add_rmsnorm(x, None, w1, None, 0.0)
    assert bool((hn.float() == 1.0).all())              # c / sqrt(c^2) = 1
    x2 = torch.full((1, H), -3.0).bfloat16()
    _, hn2 = O.add_rmsnorm(x2, None, 2 * w1, None, 0.0)
    assert bool((hn2.float() == -2.0).all())
    # delta path: h = bf16(x + delta), and no delta leaves h as x
    d = torch.full((2, H), 0.5).bfloat16()
    h, _ = O.add_rmsnorm(x, d, w1, None, 0.0)
    assert bool((h.float() == 2.5).all())
    h0, _ = O.add_rmsnorm(x, None, w1, None, 0.0)
    assert h0 is x


def test_add_rmsnorm_parts_rounding_point():
    """With partials the delta is rounded to bf16 before the residual add (src/kernels.cu:1475)."""
    H = 16
    x = torch.full((1, H), 256.0).bfloat16()
    parts = torch.zeros(2, 1, H)
    parts[0] += 0.75
    parts[1] += 0.75            # sum 1.5 -> bf16 1.5; 256 + 1.5 = 257.5 -> bf16 258 (ties to even at 2 ulp)
    h, _ = O.add_rmsnorm(x, None, torch.ones(H), None, 1e-6, parts=parts)
    assert bool((h.float() == 258.0).all())
    parts2 = torch.zeros(2, 1, H)
    parts2[0] += 1.0 / 3
    parts2[1] += 1.0 / 3
    h2, _ = O.add_rmsnorm(torch.zeros(1, H).bfloat16(), None, torch.ones(H), None, 1e-6, parts=parts2)
    assert bool((h2.float() == torch.tensor(2.0 / 3).bfloat16().float()).all())


def test_residual_proj_matches_composition():
    g = torch.Generator().manual_seed(12)
    y = torch.randn(5, 256, generator=g).bfloat16()
    w = (torch.randn(64, 256, generator=g) * 0.02).bfloat16()
    res = torch.randn(5, 64, generator=g).bfloat16()
    w1 = torch.ones(64)
    h, hn = O.residual_proj(res, y, w, w1, None, 1e-6, S=2)
    ref = (res.double() + torch.from_numpy(O.linear_f64(y, w)).float().bfloat16().double())
    diff = (h.double() - ref).abs()
    assert bool((diff <= ref.abs() * 2.0 ** -7 + 1e-3).all())


def test_tolerance_function():
    r = torch.randn(100, 100)
    assert O.tolerance_ok(r, r)[0]
    bad = r.clone()
    bad[0, 0] += 10 * r.abs().max()
    assert not O.tolerance_ok(bad, r)[0]
    assert not O.tolerance_ok(r + 0.01 * r.pow(2).mean().sqrt(), r)[0]   # mean error 1e-2 RMS


# ----------------------------------------------------------------------------------------------- scoring head
def test_head_scores_oracle_pinned(O):
    """head_scores against fp64 dot products, one-hot weights (the gathered entry exactly) and a permuted gather."""
    g = torch.Generator().manual_seed(3)
    rows, H, R = 40, 5120, 9
    hn = torch.randn(rows, H, generator=g).bfloat16()
    w = torch.randn(H, generator=g) * 0.02
    b = torch.tensor([0.25])
    idx = torch.randint(0, rows, (R,), generator=g)
    s = O.head_scores(hn, idx, w, b)
    ref = torch.from_numpy(O.head_scores_f64(hn, idx, w, b))
    assert torch.allclose(s.double(), ref, rtol=1e-5, atol=1e-5)
    for j in (0, 17, H - 1):
        e = torch.zeros(H)
        e[j] = 1.0
        assert torch.equal(O.head_scores(hn, idx, e), hn[idx, j].float())
    perm = torch.randperm(R, generator=g)
    assert torch.allclose(O.head_scores(hn, idx[perm], w, b), s[perm], rtol=1e-6, atol=1e-6)


def test_pack_weight_layout_bruteforce():
    """The packed layout against its definition, element by element, on bit patterns that identify every element."""
    N, K = 32, 128
    bits = torch.arange(N * K, dtype=torch.int32).to(torch.int16).view(N, K)
    w = bits.view(torch.bfloat16)
    p = O.pack_weight(w).view(torch.int16)
    assert tuple(p.shape) == (K // 64, N // 16, 16, 64)
    for s in range(K // 64):
        for b in range(N // 16):
            for r in range(16):
                for c in range(64):
                    assert int(p[s, b, r, c]) == int(bits[16 * b + r, 64 * s + c])


def _prep_inputs(N, HQ, HKV, D, RD, seed):
    g = torch.Generator().manual_seed(seed)
    proj = torch.randn(N, (2 * HQ + 2 * HKV) * D, generator=g).bfloat16()
    qw1 = (1.0 + 0.1 * torch.randn(D, generator=g)).float()
    kw1 = (1.0 + 0.1 * torch.randn(D, generator=g)).float()
    ang = torch.rand(N, RD // 2, generator=g) * 6.0
    cos = torch.cat([ang.cos(), ang.cos()], 1).bfloat16()
    sin = torch.cat([ang.sin(), ang.sin()], 1).bfloat16()
    return proj, qw1, kw1, cos, sin


def test_fullattn_prep_vs_f64():
    HQ, HKV, D, RD = 3, 2, 256, 64
    proj, qw1, kw1, cos, sin = _prep_inputs(5, HQ, HKV, D, RD, 1)
    qt, kt, vt, gate = O.fullattn_prep(proj, qw1, kw1, cos, sin, HQ, HKV, D, 1e-6)
    q64, k64 = O.fullattn_prep_f64(proj, qw1, kw1, cos, sin, HQ, HKV, D, 1e-6)
    for got, want in ((qt, q64), (kt, k64)):
        err = np.abs(got.float().numpy() - want)
        # three bf16 roundings along the way, and the RoPE sum of two rounded terms can cancel: within 2^-6 of the
        # row's largest value (a wrong sign or partner index is off by O(1))
        scale = np.abs(want).max(-1, keepdims=True)
        assert (err <= scale * 2.0 ** -6).all(), (err / scale).max()
        assert np.median(err / scale) < 2.0 ** -9


def test_fullattn_prep_rotation_and_copies_exact():
    """cos = 1, sin = 0 leaves the normalised head; cos = 0, sin = 1 gives rotate_half of it: out[d] =
    -xn[d + RD/2] below RD/2 and xn[d - RD/2] up to RD (the sign and the partner index); dims >= RD and the copied
    v / gate heads sit where the reference's indexing puts them (checked element by element)."""
    HQ, HKV, D, RD, N = 2, 1, 256, 64, 3
    proj, qw1, kw1, _, _ = _prep_inputs(N, HQ, HKV, D, RD, 2)
    one, zero = torch.ones(N, RD).bfloat16(), torch.zeros(N, RD).bfloat16()
    q1, k1, v, gate = O.fullattn_prep(proj, qw1, kw1, one, zero, HQ, HKV, D, 1e-6)
    q2, k2, _, _ = O.fullattn_prep(proj, qw1, kw1, zero, one, HQ, HKV, D, 1e-6)
    for a, b in ((q1, q2), (k1, k2)):
        assert torch.equal(b[..., :RD // 2], -a[..., RD // 2:RD])
        assert torch.equal(b[..., RD // 2:RD], a[..., :RD // 2])
        assert torch.equal(b[..., RD:], a[..., RD:])
    P = (2 * HQ + 2 * HKV) * D
    for n in range(N):
        for h in range(HQ):
            assert torch.equal(gate[n, h * D:(h + 1) * D], proj[n, 2 * h * D + D: 2 * h * D + 2 * D])
        for h in range(HKV):
            assert torch.equal(v[h, n], proj[n, 2 * HQ * D + HKV * D + h * D: 2 * HQ * D + HKV * D + (h + 1) * D])
    assert P == proj.shape[1]
    # constant rows: x = 2 everywhere, unit weights, eps 0 -> xn = 1 exactly
    c = torch.full((1, P), 2.0).bfloat16()
    qc, kc, _, _ = O.fullattn_prep(c, torch.ones(D), torch.ones(D), one[:1], zero[:1], HQ, HKV, D, 0.0)
    assert bool((qc == 1.0).all()) and bool((kc == 1.0).all())


# ---------------------------------------------------------------- linear-attention prep (tree layout)

def _lin_case(seed, HK=2, HV=6, HD=128, Lr=5, q_len=(3, 0, 4), groups=(0, 0, 1, 2, 1), l_len=(2, 6, 1, 3, 4)):
    from oracle import linattn_oracle as LO
    lay = LO.tree_layout(Lr, list(q_len), list(groups), list(l_len), NB=16, PB=8)
    KD, VD = HK * HD, HV * HD
    C = 2 * KD + VD
    g = torch.Generator().manual_seed(seed)
    proj = (torch.randn(lay["N"], C + VD + 2 * HV, generator=g) * 1.5).bfloat16()
    convw = (torch.randn(C, 4, generator=g) * 0.5).bfloat16()
    A_log = torch.randn(HV, generator=g).bfloat16()
    dt_bias = (torch.randn(HV, generator=g) * 4).bfloat16()
    return LO, lay, proj, convw, A_log, dt_bias, KD, VD, HV, HK, HD


def test_tree_layout_vs_walk():
    """rep_ptr / rep_pos list, for every packed row, exactly the slots holding it (ascending slot order, padding
    last), and hist[n] is the 4-row window ending at n on any path through n."""
    from oracle import linattn_oracle as LO
    lay = LO.tree_layout(4, [2, 5], [1, 0, 1], [3, 1, 2], NB=16, PB=8)
    N, S, L2, src = lay["N"], lay["S"], lay["L2"], lay["src"]
    assert N % 16 == 0 and L2 % 8 == 0 and src.shape == (S, L2)
    flat = src.reshape(-1)
    for n in range(N + 1):
        got = lay["rep_pos"][lay["rep_ptr"][n]:lay["rep_ptr"][n + 1]].tolist()
        want = [s for s in range(S * L2) if (flat[s] == n if n < N else flat[s] < 0)]
        assert got == want, n
        for s in want if n < N else []:
            c, t = divmod(s, L2)
            assert [src[c, t - 3 + i] if t - 3 + i >= 0 else -1 for i in range(4)] == lay["hist"][n].tolist()
    assert (lay["hist"][N] == -1).all()
    # the root is shared by all paths; a leaf row by exactly one
    assert lay["rep_ptr"][1] - lay["rep_ptr"][0] == S


@pytest.mark.parametrize("rep_qk", [False, True])
def test_linattn_prep_vs_slot_f64(rep_qk):
    LO, lay, proj, convw, A_log, dt_bias, KD, VD, HV, HK, HD = _lin_case(3)
    q, k, v, gg, beta = LO.linattn_prep(proj, lay["hist"], lay["rep_ptr"], lay["rep_pos"], lay["L2"], convw, A_log,
                                        dt_bias, KD, VD, HV, HK, HD, rep_qk)
    qk64, v64, g64, b64 = LO.linattn_slot_f64(proj, lay["src"], convw, A_log, dt_bias, KD, VD, HV, HD)
    rq = HV // HK if rep_qk else 1
    R = lay["S"] * lay["L2"]
    assert q.shape == (R, rq * KD) and v.shape == (R, VD) and gg.dtype == torch.float32
    qf = q.float().numpy().reshape(R, KD // HD, rq, HD)
    kf = k.float().numpy().reshape(R, KD // HD, rq, HD)
    for r in range(1, rq):  # replicated heads are copies
        assert (qf[:, :, r] == qf[:, :, 0]).all() and (kf[:, :, r] == kf[:, :, 0]).all()
    got_qk = np.concatenate([qf[:, :, 0].reshape(R, KD), kf[:, :, 0].reshape(R, KD)], 1)
    # q / k: unit-norm heads, two bf16 roundings (silu output, normalised value): 2^-7 of the value + 2^-9
    assert (np.abs(got_qk - qk64) <= np.abs(qk64) * 2.0 ** -7 + 2.0 ** -9).all()
    # v: one bf16 rounding of silu(conv)
    vf = v.float().numpy()
    assert (np.abs(vf - v64) <= np.abs(v64) * 2.0 ** -8 + 1e-6).all()
    assert np.allclose(gg.numpy(), g64, rtol=1e-5, atol=1e-6)
    assert (np.abs(beta.float().numpy() - b64) <= b64 * 2.0 ** -8).all()
    pad = lay["src"].reshape(-1) < 0
    assert pad.any() and (got_qk[pad] == 0).all() and (vf[pad] == 0).all() and (gg.numpy()[pad] == 0).all()
    # every real slot's q / k head has unit norm (up to bf16 rounding)
    nrm = np.sqrt((got_qk[~pad].reshape(-1, HD) ** 2).sum(1))
    assert np.abs(nrm - 1).max() < 2e-2


def test_linattn_gates_closed_forms():
    """beta against scipy's expit, g against -exp(A_log) * log(1 + e^x) (numpy logaddexp), including the
    softplus branch above 20 and very negative arguments."""
    from scipy.special import expit
    from oracle import linattn_oracle as LO
    b = np.array([-30, -5, -0.5, 0, 0.25, 3, 30], np.float32)
    a = np.array([-40, -3, 0, 1, 19.5, 20.5, 60], np.float32)
    al = np.array([0.5] * 7, np.float32)
    db = np.zeros(7, np.float32)
    beta, g = LO._gates(b, a, al, db)
    want_b = expit(b.astype(np.float64))
    assert (np.abs(beta - want_b) <= want_b * 2.0 ** -8).all()
    want_g = -np.exp(0.5) * np.logaddexp(0.0, a.astype(np.float64))
    assert np.allclose(g, want_g, rtol=2e-6, atol=1e-30)
    assert g[-1] == np.float32(-np.exp(np.float32(0.5)) * np.float32(60))  # x > 20: softplus(x) = x exactly
