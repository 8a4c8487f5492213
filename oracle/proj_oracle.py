"""CPU oracle of the dense bf16 projection path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the
checker or the reported CPU baseline; the product path (libojx.so and the open-jev-fast_amd package) never calls it.

What it restates (reference file:line):
  linear_bf16        y = bf16(x . W^T), fp32 accumulation: lt_matmul's CUBLAS_COMPUTE_32F with bf16 in/out
                     (src/lt.cpp:22-29, 43-55), F.linear in _mm (src/fastmodel.py:168-175); BASELINE names
                     "torch bf16 matmul (fp32 accumulate)" as the oracle, so this is torch.matmul on fp32 copies.
  splitk_parts       parts[s] = x[:, K_s] . W[:, K_s]^T in fp32 (torch.bmm out_dtype=fp32, src/fastmodel.py:166)
  silu_mul           out = bf16(bf16(silu(g)) * u), gu = [g | u] (src/kernels.cu:76-89; LUT form :1288-1331)
  add_rmsnorm        h = bf16(x + bf16(delta)); hn = bf16((h * rsqrt(sum h^2 / H + eps)) * w1), 0 if rowmask == 0
                     (src/kernels.cu:41-73); with fp32 partials delta = bf16(sum_s parts[s]), s ascending
                     (add_rmsnorm_sk2_k, src/kernels.cu:1444-1501)
  residual_proj      _res (src/fastmodel.py:196-203) = splitk_parts + add_rmsnorm with partials
  gate_up_silu       _silu_mul(_mm(hn, cat[gate; up])) (src/fastmodel.py:90, 478, 190-194)
  pack_gate_up       the fused-GEMM weight layout (rows in blocks of 8: 4 gate rows, 4 up rows) — libojx's own
                     layout, restated here so tests can build it on the CPU
  pack_weight        the stage-major packed weight layout of the *_pk projections (libojx's own), likewise
  fullattn_prep      fullattn_prep2_k (src/kernels.cu:302-355) for B = 1, the full-attention consumer of the QKV
                     in-projection (src/fastmodel.py:462): per-head RMSNorm + rotate-half RoPE of q / k, v and gate
                     copied, in the head-major output layout; fullattn_prep_f64 is its fp64 check
  linear_f64         fp64 brute-force dot products (numpy), the independent check the oracle is pinned against
  head_scores        mdl.head(hn[lastidx].float()).squeeze(-1) (src/server.py:37, 57, 129; hn[lastidx] at
                     src/fastmodel.py:314, 482) for a Linear(H, 1) with fp32 weight and bias: torch fp32 on the CPU.
                     The head module belongs to the Open-Jev model package, which the reference does not vendor:
                     Linear(H, 1) in fp32 is read off its call site (input cast .float(), output squeeze(-1)).

Pinning (tests/test_oracle.py): linear_bf16 against linear_f64 and exact closed forms (identity, permutation,
exactly representable rank-1 products); silu_mul against scipy's expit in fp64 and special values; add_rmsnorm
against an fp64 RMSNorm and closed-form constant rows; the gate/up merge bit-exactness of tests/test_correct.py:44;
splitk_parts summing to linear_f64; head_scores against fp64 dot products and one-hot weights (a gathered entry
exactly), with the gather order checked by permuting lastidx. The reference holds no golden vectors for this path (no fixtures in its tree);
tests/golden/ holds fp64 brute-force vectors made by tests/golden/make_golden.py.
"""
import numpy as np
import torch


def _bf16(t):
    return t.to(torch.bfloat16)


def linear_bf16(x, w):
    """bf16(x . w^T) with fp32 accumulation on the CPU (x [M,K], w [N,K] bf16)."""
    return _bf16(torch.matmul(x.float(), w.float().t()))


def linear_f32(x, w):
    return torch.matmul(x.float(), w.float().t())


def linear_f64(x, w):
    """fp64 brute force (numpy), independent of torch's GEMM."""
    xa = x.float().numpy().astype(np.float64)
    wa = w.float().numpy().astype(np.float64)
    return xa @ wa.T


def split_ranges(K, S):
    """K ranges of the S splits: chunk = ceil(K/S) rounded up to a multiple of 8 (equal K/S chunks, as the
    reference's x.view(M, S, K/S), whenever K is a multiple of 8*S)."""
    c = -(-K // S)
    c = -(-c // 8) * 8
    return [(s * c, min(K, (s + 1) * c)) for s in range(S)]


def splitk_parts(x, w, S):
    """[S, M, N] fp32 partial products over the split K ranges."""
    K = x.shape[1]
    return torch.stack([linear_f32(x[:, a:b], w[:, a:b]) for a, b in split_ranges(K, S)])


def silu_mul(gu):
    """gu [M, 2I] bf16 -> bf16(bf16(silu(g)) * u)."""
    I = gu.shape[1] // 2
    g, u = gu[:, :I].float(), gu[:, I:].float()
    s = _bf16(g / (1.0 + torch.exp(-g))).float()
    return _bf16(s * u)


def act_tables():
    """65536-entry tables indexed by the bf16 bit pattern: silu_b bf16, sig_f fp32."""
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    x = bits.view(torch.bfloat16).float()
    return _bf16(x / (1.0 + torch.exp(-x))), 1.0 / (1.0 + torch.exp(-x))


def add_rmsnorm(x, delta, w1, rowmask, eps, parts=None):
    """(h, hn) of add_rmsnorm / add_rmsnorm_sk2. delta bf16 [M,H] or None; parts fp32 [S,M,H] or None."""
    xf = x.float()
    if parts is not None:
        d = _bf16(parts.float().sum(0)).float()  # ascending s, fp32
        v = _bf16(xf + d).float()
    elif delta is not None:
        v = _bf16(xf + delta.float()).float()
    else:
        v = xf
    H = x.shape[1]
    ss = (v * v).sum(1, keepdim=True)
    r = torch.rsqrt(ss / H + eps)
    hn = _bf16((v * r) * w1.float()[None, :])
    if rowmask is not None:
        hn = torch.where(rowmask[:, None] != 0, hn, torch.zeros_like(hn))
    h = _bf16(v) if (parts is not None or delta is not None) else x
    return h, hn


def residual_proj(residual, y, w, w1, rowmask, eps, S=1):
    """_res: (h, hn) after the out / down projection of y with W [N, K]."""
    parts = splitk_parts(y, w, S)
    return add_rmsnorm(residual, None, w1, rowmask, eps, parts=parts)


def gate_up_silu(x, w_gate, w_up):
    """The reference's MLP front: SiLU.mul of the merged gate-up GEMM."""
    gu = linear_bf16(x, torch.cat([w_gate, w_up], 0))
    return silu_mul(gu)


def pack_gate_up(gate, up):
    """[2I, K]: rows in blocks of 8 = gate rows 4b..4b+3 then up rows 4b..4b+3."""
    I, K = gate.shape
    return torch.stack([gate.view(I // 4, 4, K), up.view(I // 4, 4, K)], 1).reshape(2 * I, K)


def pack_weight(w):
    """The packed weight layout of libojx's *_pk projections, restated: W [N, K] -> [K/64, N/16, 16, 64] with
    packed[s, b, r, c] = W[16 b + r, 64 s + c] (libojx's own layout, so that tests can build it on the CPU)."""
    N, K = w.shape
    return w.reshape(N // 16, 16, K // 64, 64).permute(2, 0, 1, 3).contiguous()


def fullattn_prep(proj, qw1, kw1, cos, sin, HQ, HKV, D, eps):
    """fullattn_prep2_k (src/kernels.cu:302-355) for B = 1: proj [N, (2 HQ + 2 HKV) D] bf16 -> (qt [HQ, N, D],
    kt [HKV, N, D], vt [HKV, N, D], gate [N, HQ D]). q/k heads: xn = bf16((x * rsqrt(sum x^2 / D + eps)) * w1),
    then on the first RD = cos.shape[1] dims out = bf16(bf16(xn * cos) + bf16(rh * sin)), rh = -xn[d + RD/2] for
    d < RD/2 and xn[d - RD/2] above; v and gate copied."""
    N = proj.shape[0]
    RD = cos.shape[1]
    p = proj.float().view(N, -1)
    q_g = p[:, :2 * HQ * D].view(N, HQ, 2, D)
    q, gate = q_g[:, :, 0], q_g[:, :, 1]
    k = p[:, 2 * HQ * D:2 * HQ * D + HKV * D].view(N, HKV, D)
    v = p[:, 2 * HQ * D + HKV * D:].view(N, HKV, D)

    def norm_rope(x, w1):
        r = torch.rsqrt((x * x).sum(-1, keepdim=True) / D + eps)
        xn = _bf16((x * r) * w1.float()).float()
        c, s = cos.float()[:, None, :], sin.float()[:, None, :]
        a, b = xn[..., :RD // 2], xn[..., RD // 2:RD]
        rot = torch.cat([-b, a], -1)
        head = _bf16(_bf16(xn[..., :RD] * c).float() + _bf16(rot * s).float()).float()
        return _bf16(torch.cat([head, xn[..., RD:]], -1))

    qt = norm_rope(q, qw1).permute(1, 0, 2).contiguous()
    kt = norm_rope(k, kw1).permute(1, 0, 2).contiguous()
    return qt, kt, _bf16(v).permute(1, 0, 2).contiguous(), _bf16(gate).reshape(N, HQ * D)


def fullattn_prep_f64(proj, qw1, kw1, cos, sin, HQ, HKV, D, eps):
    """fp64 numpy form of fullattn_prep without the intermediate bf16 roundings (the independent check)."""
    N = proj.shape[0]
    RD = cos.shape[1]
    p = proj.float().numpy().astype(np.float64).reshape(N, -1)
    c, s = cos.float().numpy().astype(np.float64), sin.float().numpy().astype(np.float64)
    out = []
    for base, heads, w1, stride in ((0, HQ, qw1, 2 * D), (2 * HQ * D, HKV, kw1, D)):
        w = w1.double().numpy()
        o = np.zeros((heads, N, D))
        for h in range(heads):
            x = p[:, base + h * stride: base + h * stride + D]
            xn = x / np.sqrt((x * x).sum(1, keepdims=True) / D + eps) * w
            y = xn.copy()
            y[:, :RD // 2] = xn[:, :RD // 2] * c[:, :RD // 2] - xn[:, RD // 2:RD] * s[:, :RD // 2]
            y[:, RD // 2:RD] = xn[:, RD // 2:RD] * c[:, RD // 2:] + xn[:, :RD // 2] * s[:, RD // 2:]
            o[h] = y
        out.append(o)
    return out[0], out[1]


def head_scores(hn, lastidx, w, bias=None):
    """scores [R] = hn[lastidx].float() @ w (+ bias), fp32 on the CPU (hn [rows, H] bf16, w [H] fp32)."""
    s = torch.matmul(hn[lastidx].float(), w.reshape(-1).float())
    return s + bias.reshape(()) if bias is not None else s


def head_scores_f64(hn, lastidx, w, bias=None):
    """fp64 brute force of head_scores (numpy)."""
    a = hn[lastidx].float().numpy().astype(np.float64)
    s = a @ w.reshape(-1).double().numpy()
    return s + (float(bias.reshape(())) if bias is not None else 0.0)


# ---------------------------------------------------------------------------------------------- inputs
def seeded_inputs(M, N, K, seed=0, x_std=1.0, w_std=0.02):
    """x ~ N(0, x_std^2) [M,K], W ~ N(0, w_std^2) [N,K], both bf16."""
    g = torch.Generator().manual_seed(seed)
    x = _bf16(torch.randn(M, K, generator=g) * x_std)
    w = _bf16(torch.randn(N, K, generator=g) * w_std)
    return x, w


def tolerance_ok(out, ref, max_rel=1e-2, mean_abs_rms=1e-3):
    """The north-star tolerance: max |d| / max |ref| <= 1e-2 and mean |d| <= 1e-3 * RMS(ref).
    Returns (ok, max_rel, mean_abs / rms)."""
    o, r = out.float(), ref.float()
    d = (o - r).abs()
    mx = r.abs().max().clamp_min(1e-30)
    rms = r.pow(2).mean().sqrt().clamp_min(1e-30)
    a, b = (d.max() / mx).item(), (d.mean() / rms).item()
    ok = bool(torch.isfinite(o).all()) and a <= max_rel and b <= mean_abs_rms
    return ok, a, b
