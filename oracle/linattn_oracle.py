"""CPU oracle of the linear-attention prep on the tree layout — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the
checker; the product path (libojx.so and the open-jev-fast_amd package) never calls it.

What it restates (reference file:line):
  tree_layout      the index fields of FastQwen35.gtree_build (src/fastmodel.py:322-386) that the prep reads:
                   src [S, L2] (packed row of each path slot, -1 = end padding), rep_ptr [N + 2] / rep_pos [S L2]
                   (CSR from packed rows to slots, group N = the padding slots, stable order), hist [N + 1, 4]
                   (rows t-3 .. t of each packed row along its path, -1 = none, row N all -1). The tree is given by
                   its node lengths (root prefix, R group nodes, S leaves); the token ids are irrelevant here.
  linattn_prep     linattn_prep_dedup2_k (src/kernels.cu:1176-1265) in numpy fp32 with the kernel's rounding points
                   and summation orders: conv = ((w0 x[t-3] + w1 x[t-2]) + w2 x[t-1]) + w3 x[t] (bf16 products are
                   exact in fp32), o = bf16(silu(conv)); q / k heads of 128 channels: the sum of squares of 16 groups
                   of 8 (each group in order) added by the xor-8/4/2/1 butterfly, o * (1 / sqrt(ss + 1e-6)) rounded
                   to bf16; beta = bf16(sigmoid(b)); g = -exp(A_log) * softplus(a + dt_bias) with softplus(x) = x
                   above 20; scattered to every slot of the row, zeros to the padding slots; rep_qk writes each q / k
                   head HV / HK times side by side (REPQK 3 of src/kernels.cu:1251-1255).
  linattn_slot_f64 the same quantities computed slot by slot straight from src (the path, not hist / rep_*) in fp64
                   without intermediate roundings: the independent check that pins the oracle's indexing.

Pinning (tests/test_oracle.py): linattn_prep against linattn_slot_f64 on random trees (history, scatter, padding,
head order); the gates against scipy's expit and numpy's logaddexp; q / k head norms equal to 1; tree_layout's CSR
and history against a brute-force walk over src. The reference ships no fixtures for this kernel.
"""
import numpy as np
import torch


def _rbf(a):
    """Round fp32 numpy values to bf16 (nearest even) and back."""
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).bfloat16().float().numpy()


def tree_layout(Lr, q_len, groups, l_len, NB=32, PB=16):
    """Packed rows [root | group nodes | leaves | padding to a multiple of NB]; path c = root, the rows of group
    groups[c], then leaf c, padded with -1 to L2 = (longest path rounded up to PB). Returns dict(N, S, L2, src,
    rep_ptr, rep_pos, hist)."""
    S, R = len(l_len), len(q_len)
    qb = Lr + np.concatenate([[0], np.cumsum(q_len)[:-1]]).astype(np.int64) if R else np.zeros(0, np.int64)
    lb = Lr + sum(q_len) + np.concatenate([[0], np.cumsum(l_len)[:-1]]).astype(np.int64)
    nreal = Lr + sum(q_len) + sum(l_len)
    N = -(-nreal // NB) * NB
    paths = [list(range(Lr)) + list(range(qb[groups[c]], qb[groups[c]] + q_len[groups[c]]))
             + list(range(lb[c], lb[c] + l_len[c])) for c in range(S)]
    L2 = -(-max(len(p) for p in paths) // PB) * PB
    src = np.full((S, L2), -1, np.int32)
    for c, p in enumerate(paths):
        src[c, :len(p)] = p
    flat = src.reshape(-1)
    grp = np.where(flat >= 0, flat, N)
    rep_pos = np.argsort(grp, kind="stable").astype(np.int32)
    rep_ptr = np.concatenate([[0], np.cumsum(np.bincount(grp, minlength=N + 1))]).astype(np.int32)
    hist = np.full((N + 1, 4), -1, np.int32)
    for n in range(N):
        if rep_ptr[n] < rep_ptr[n + 1]:
            c, t = divmod(int(rep_pos[rep_ptr[n]]), L2)
            for i in range(4):
                if t - 3 + i >= 0:
                    hist[n, i] = src[c, t - 3 + i]
    return dict(N=N, S=S, L2=L2, src=src, rep_ptr=rep_ptr, rep_pos=rep_pos, hist=hist)


def _gates(p_b, p_a, A_log, dt_bias):
    """beta (bf16-rounded fp32) and g (fp32) for rows of b / a values [.., HV] (all fp32 numpy)."""
    one = np.float32(1.0)
    beta = _rbf(one / (one + np.exp(-p_b)))
    xs = (p_a + dt_bias).astype(np.float32)
    with np.errstate(over="ignore"):
        sp = np.where(xs > np.float32(20.0), xs, np.log1p(np.exp(xs)).astype(np.float32))
    g = (-np.exp(A_log) * sp).astype(np.float32)
    return beta, g


def linattn_prep(proj, hist, rep_ptr, rep_pos, L2, convw, A_log, dt_bias, KD, VD, HV, HK, HD, rep_qk):
    """numpy restatement of linattn_prep_dedup2 (src/kernels.cu:1176-1290). Tensors in, torch CPU tensors out:
    q, k bf16 [R, RQ KD], v bf16 [R, VD], g fp32 [R, HV], beta bf16 [R, HV]."""
    P = proj.float().numpy()
    hist = np.asarray(hist).reshape(-1, 4)
    rep_ptr, rep_pos = np.asarray(rep_ptr), np.asarray(rep_pos)
    W = convw.float().numpy().astype(np.float32)
    al, db = A_log.float().numpy(), dt_bias.float().numpy()
    N, R = P.shape[0], len(rep_pos)
    C = 2 * KD + VD
    rq = HV // HK if rep_qk else 1
    # per packed row (rows with no slot are computed too, then never scattered)
    acc = np.zeros((N, C), np.float32)
    for i in range(4):
        rows = hist[:N, i]
        x = np.where(rows[:, None] >= 0, P[np.maximum(rows, 0), :C], np.float32(0.0))
        acc = (acc + W[None, :, i] * x).astype(np.float32)
    one = np.float32(1.0)
    o = _rbf(acc / (one + np.exp(-acc)))
    qk = o[:, :2 * KD].reshape(N, 2 * KD // HD, HD // 8, 8)
    ss = np.zeros(qk.shape[:3], np.float32)
    for j in range(8):
        ss = (ss + qk[..., j] * qk[..., j]).astype(np.float32)
    lanes = np.arange(HD // 8)
    for off in (8, 4, 2, 1):
        ss = (ss + ss[..., lanes ^ off]).astype(np.float32)
    rs = (one / np.sqrt(ss + np.float32(1e-6))).astype(np.float32)
    qk = _rbf(qk * rs[..., None]).reshape(N, 2 * KD)
    rows_hv = np.maximum(hist[:N, 3], 0)
    beta_r, g_r = _gates(P[rows_hv, C + VD:C + VD + HV], P[rows_hv, C + VD + HV:C + VD + 2 * HV], al, db)
    q = np.zeros((R, rq * KD), np.float32)
    k = np.zeros((R, rq * KD), np.float32)
    v = np.zeros((R, VD), np.float32)
    g = np.zeros((R, HV), np.float32)
    beta = np.zeros((R, HV), np.float32)
    for n in range(N):
        slots = rep_pos[rep_ptr[n]:rep_ptr[n + 1]]
        if len(slots) == 0:
            continue
        qh = qk[n, :KD].reshape(KD // HD, 1, HD)
        kh = qk[n, KD:].reshape(KD // HD, 1, HD)
        q[slots] = np.broadcast_to(qh, (KD // HD, rq, HD)).reshape(-1)
        k[slots] = np.broadcast_to(kh, (KD // HD, rq, HD)).reshape(-1)
        v[slots] = o[n, 2 * KD:]
        g[slots] = g_r[n]
        beta[slots] = beta_r[n]
    bf = lambda a: torch.from_numpy(a).bfloat16()  # noqa: E731
    return bf(q), bf(k), bf(v), torch.from_numpy(g), bf(beta)


def linattn_slot_f64(proj, src, convw, A_log, dt_bias, KD, VD, HV, HD):
    """fp64, slot by slot from the paths src [S, L2]: (qk [S L2, 2 KD] normalised per head, v [S L2, VD],
    g [S L2, HV], beta [S L2, HV]); padding slots zero. No intermediate roundings."""
    P = proj.float().numpy().astype(np.float64)
    W = convw.float().numpy().astype(np.float64)
    al, db = A_log.float().numpy().astype(np.float64), dt_bias.float().numpy().astype(np.float64)
    S, L2 = src.shape
    C = 2 * KD + VD
    qk = np.zeros((S * L2, 2 * KD))
    v = np.zeros((S * L2, VD))
    g = np.zeros((S * L2, HV))
    beta = np.zeros((S * L2, HV))
    for c in range(S):
        for t in range(L2):
            r = src[c, t]
            if r < 0:
                continue
            conv = np.zeros(C)
            for i in range(4):
                tt = t - 3 + i
                if tt >= 0 and src[c, tt] >= 0:
                    conv += W[:, i] * P[src[c, tt], :C]
            o = conv / (1.0 + np.exp(-conv))
            hq = o[:2 * KD].reshape(-1, HD)
            qk[c * L2 + t] = (hq / np.sqrt((hq * hq).sum(1, keepdims=True) + 1e-6)).reshape(-1)
            v[c * L2 + t] = o[2 * KD:]
            b = P[r, C + VD:C + VD + HV]
            a = P[r, C + VD + HV:C + VD + 2 * HV] + db
            beta[c * L2 + t] = 1.0 / (1.0 + np.exp(-b))
            g[c * L2 + t] = -np.exp(al) * np.logaddexp(0.0, a)
    return qk, v, g, beta
