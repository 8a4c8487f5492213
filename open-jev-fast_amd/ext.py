"""Projection-path functions of the reference's kernel extension `K` (src/ext.py:6-29), on libojx.

Same names, arguments, return values and error behaviour (RuntimeError) as the reference's torch-extension
functions, for the entry points on the projection path:

    add_rmsnorm(x, delta, w1, rowmask, eps) -> [h, hn]        src/kernels.cu:41-73, 755-767
    add_rmsnorm_sk(x, parts, w1, rowmask, eps) -> [h, hn]     src/kernels.cu:475-515, 886-900
    add_rmsnorm_sk2(x, parts, w1, rowmask, eps) -> [h, hn]    src/kernels.cu:1444-1501 (S in 2..4)
    silu_mul(gu) -> out                                       src/kernels.cu:76-89, 769-777
    silu_mul_lut(gu, tab) -> out                              src/kernels.cu:1304-1331
    act_tables(like) -> [silu_b, sig_f]                       src/kernels.cu:1288-1301
    head_scores(hn, lastidx, w, bias) -> scores              src/server.py:37 (mdl.head(hn[lastidx].float()))

plus the fused projections that replace GEMM + epilogue pairs (mm, mm_silu_mul, mm_residual_rmsnorm,
mm_splitk_f32) and pack_gate_up, the weight layout of the fused gate-up.

Tensors must be contiguous GPU tensors (the reference's CHECK, src/kernels.cu:10); outputs come from torch.empty on
the current stream's device and every launch goes on torch's current stream, so all of it can be captured in a
CUDA/HIP graph.
"""
import ctypes
import weakref

import torch

from . import _lib
from ._lib import KIND_PLAIN, KIND_RESIDUAL, KIND_SILU_MUL, check, lib


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _chk(t, name, dtype=None):
    if t is None:
        raise RuntimeError(f"{name} must be a tensor")
    if not (t.is_cuda and t.is_contiguous()):
        raise RuntimeError(f"{name} must be contiguous CUDA")
    if dtype is not None and t.dtype != dtype:
        raise RuntimeError(f"{name} must be {dtype}, got {t.dtype}")


def _cfgp(cfg):
    if cfg is None:
        return None
    if not isinstance(cfg, _lib.OjxCfg):
        cfg = _lib.OjxCfg(*cfg)
    return ctypes.byref(cfg)


_WS = {}        # (device index, stream handle) -> the workspace handed to that stream's eager calls and captures
_WS_KEEP = []   # every workspace a graph capture has used: kept alive for the life of the process


def _workspace(M, N, K, kind, cfg, device):
    """Workspace of one call: split-K fp32 planes or stream-K partial tiles (scratch, contents irrelevant on entry).

    One buffer per stream of each device is kept and grown as needed, so calls on different streams may overlap (the
    library gives each stream its own set of arrival counters for the one-launch plans too). A graph capture records the buffer's address, so a buffer
    that a capture has used is not freed while graphs may replay: when a later call needs a larger one, the old
    buffer moves to _WS_KEEP instead of going back to the caching allocator (where a replay would write into memory
    that other tensors may own by then). The larger buffer becomes the device's buffer for every later call,
    eager or captured, so the kept memory grows only with the largest workspace seen per stream, not with the number
    of captures. release_workspaces() drops the kept buffers once the caller's graphs are gone. A captured graph
    replayed on another stream keeps the capture stream's workspace: replays that overlap with calls on the capture
    stream race on it."""
    n = lib().ojx_workspace_bytes(M, N, K, kind, _cfgp(cfg))
    if n < 0:
        check(1)
    if n == 0:
        return None, 0
    key = (torch.device(device).index, torch.cuda.current_stream(device).cuda_stream)
    ws = _WS.get(key)
    capturing = torch.cuda.is_current_stream_capturing()
    if ws is not None and ws[0].numel() >= n:
        if capturing and not ws[1]:
            _WS[key] = ws = (ws[0], True)
            _WS_KEEP.append(ws[0])
        return ws[0], ws[0].numel()
    buf = torch.empty(max(n, 1 << 20), dtype=torch.uint8, device=device)
    _WS[key] = (buf, capturing)   # the old buffer, if a capture used it, stays alive in _WS_KEEP
    if capturing:
        _WS_KEEP.append(buf)
    return buf, buf.numel()


def release_workspaces():
    """Frees the workspace buffers kept for captured graphs (and the current ones). Call it only after every graph
    captured with this module's calls has been destroyed: a later replay of such a graph would write into freed
    memory."""
    _WS.clear()
    _WS_KEEP.clear()


def _chk_norm(w1, rowmask, M, H):
    """RMSNorm operands: w1 fp32 [H]; rowmask (optional) int32 [M]. The kernels read exactly that many."""
    _chk(w1, "w1", torch.float32)
    if w1.numel() != H:
        raise RuntimeError(f"w1 must have H={H} elements, got {w1.numel()}")
    if rowmask is not None:
        _chk(rowmask, "rowmask", torch.int32)
        if rowmask.numel() != M:
            raise RuntimeError(f"rowmask must have M={M} elements, got {rowmask.numel()}")


# ------------------------------------------------------------------------------------------------ epilogues
def add_rmsnorm(x, delta, w1, rowmask, eps):
    _chk(x, "x", torch.bfloat16)
    M, H = x.shape
    _chk_norm(w1, rowmask, M, H)
    hn = torch.empty_like(x)
    if delta is not None:
        _chk(delta, "delta", torch.bfloat16)
        if tuple(delta.shape) != (M, H):
            raise RuntimeError(f"delta {tuple(delta.shape)} must match x {tuple(x.shape)}")
        h = torch.empty_like(x)
    else:
        h = x
    check(lib().ojx_add_rmsnorm(_ptr(x), _ptr(delta), _ptr(w1), _ptr(rowmask), float(eps),
                                _ptr(h) if delta is not None else None, _ptr(hn), M, H, _stream()))
    return [h, hn]


def add_rmsnorm_sk(x, parts, w1, rowmask, eps):
    _chk(x, "x", torch.bfloat16)
    _chk(parts, "parts", torch.float32)
    M, H = x.shape
    _chk_norm(w1, rowmask, M, H)
    S = parts.shape[0]
    if parts.dim() != 3 or parts.shape[1] != M or parts.shape[2] != H:
        raise RuntimeError("parts must be [S, M, H]")
    h, hn = torch.empty_like(x), torch.empty_like(x)
    check(lib().ojx_add_rmsnorm_sk(_ptr(x), _ptr(parts), S, _ptr(w1), _ptr(rowmask), float(eps), _ptr(h), _ptr(hn),
                                   M, H, _stream()))
    return [h, hn]


def add_rmsnorm_sk2(x, parts, w1, rowmask, eps):
    if not 2 <= parts.shape[0] <= 4:
        raise RuntimeError("S must be 2..4")
    return add_rmsnorm_sk(x, parts, w1, rowmask, eps)


def silu_mul(gu):
    _chk(gu, "gu", torch.bfloat16)
    M, I2 = gu.shape
    out = torch.empty((M, I2 // 2), dtype=gu.dtype, device=gu.device)
    check(lib().ojx_silu_mul(_ptr(gu), _ptr(out), M, I2 // 2, _stream()))
    return out


def silu_mul_lut(gu, tab):
    _chk(gu, "gu", torch.bfloat16)
    _chk(tab, "tab", torch.bfloat16)
    M, I2 = gu.shape
    out = torch.empty((M, I2 // 2), dtype=gu.dtype, device=gu.device)
    check(lib().ojx_silu_mul_lut(_ptr(gu), _ptr(tab), _ptr(out), M, I2 // 2, _stream()))
    return out


def act_tables(like):
    silu_b = torch.empty(65536, dtype=torch.bfloat16, device=like.device)
    sig_f = torch.empty(65536, dtype=torch.float32, device=like.device)
    check(lib().ojx_act_tables(_ptr(silu_b), _ptr(sig_f), _stream()))
    return [silu_b, sig_f]


# ------------------------------------------------------------------------------------------------ projections
def mm(x, w, cfg=None):
    """y = x . w^T, bf16 out (the reference's _mm / lt_matmul / F.linear). w may be a packed weight (pack_weight)."""
    if w.dim() == 4:
        return mm_pk(x, w, cfg)
    _chk(x, "x", torch.bfloat16)
    _chk(w, "w", torch.bfloat16)
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise RuntimeError(f"shape mismatch: x {tuple(x.shape)} w {tuple(w.shape)}")
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    ws, nws = _workspace(M, N, K, KIND_PLAIN, cfg, x.device)
    check(lib().ojx_gemm_bf16(_ptr(x), _ptr(w), _ptr(y), M, N, K, K, K, N, _ptr(ws), nws, _cfgp(cfg), _stream()))
    return y


def mm_splitk_f32(x, w, S, tile=-1):
    """parts [S, M, N] fp32 over S contiguous K ranges (the reference's _skmm torch.bmm with out_dtype=fp32)."""
    _chk(x, "x", torch.bfloat16)
    _chk(w, "w", torch.bfloat16)
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise RuntimeError(f"shape mismatch: x {tuple(x.shape)} w {tuple(w.shape)}")
    parts = torch.empty((S, M, N), dtype=torch.float32, device=x.device)
    check(lib().ojx_gemm_splitk_f32(_ptr(x), _ptr(w), _ptr(parts), M, N, K, K, K, S, tile, _stream()))
    return parts


def mm_silu_mul(x, w_gu_packed, cfg=None):
    """out [M, I] = bf16(bf16(silu(g)) * u), [g | u] = x . W_gu^T, W_gu in pack_gate_up layout [2I, K] (or that
    weight through pack_weight)."""
    if w_gu_packed.dim() == 4:
        return mm_silu_mul_pk(x, w_gu_packed, cfg)
    _chk(x, "x", torch.bfloat16)
    _chk(w_gu_packed, "w_gu", torch.bfloat16)
    M, K = x.shape
    N = w_gu_packed.shape[0]
    if w_gu_packed.shape[1] != K or N % 2:
        raise RuntimeError(f"shape mismatch: x {tuple(x.shape)} w_gu {tuple(w_gu_packed.shape)}")
    out = torch.empty((M, N // 2), dtype=x.dtype, device=x.device)
    ws, nws = _workspace(M, N, K, KIND_SILU_MUL, cfg, x.device)
    check(lib().ojx_gemm_silu_mul(_ptr(x), _ptr(w_gu_packed), _ptr(out), M, N // 2, K, _ptr(ws), nws, _cfgp(cfg),
                                  _stream()))
    return out


def mm_residual_rmsnorm(h, y, w, w1, rowmask, eps, want_hn=True, cfg=None):
    """(h_new, hn): h_new = bf16(h + bf16(y . w^T)); hn = RMSNorm(h_new) * w1 (zero where rowmask == 0). w may be a
    packed weight (pack_weight)."""
    if w.dim() == 4:
        return mm_residual_rmsnorm_pk(h, y, w, w1, rowmask, eps, want_hn, cfg)
    _chk(h, "h", torch.bfloat16)
    _chk(y, "y", torch.bfloat16)
    _chk(w, "w", torch.bfloat16)
    M, K = y.shape
    N = w.shape[0]
    if w.shape[1] != K or tuple(h.shape) != (M, N):
        raise RuntimeError(f"shape mismatch: h {tuple(h.shape)} y {tuple(y.shape)} w {tuple(w.shape)}")
    if want_hn:
        _chk_norm(w1, rowmask, M, N)
    elif rowmask is not None:
        _chk(rowmask, "rowmask", torch.int32)
    h_new = torch.empty_like(h)
    hn = torch.empty_like(h) if want_hn else None
    ws, nws = _workspace(M, N, K, KIND_RESIDUAL, cfg, y.device)
    check(lib().ojx_gemm_residual_rmsnorm(_ptr(y), _ptr(w), _ptr(h), _ptr(w1) if want_hn else None, _ptr(rowmask),
                                          float(eps), _ptr(h_new), _ptr(hn), M, N, K, _ptr(ws), nws, _cfgp(cfg),
                                          _stream()))
    return h_new, hn


def head_scores(hn, lastidx, w, bias=None):
    """scores [R] fp32 = hn[lastidx].float() @ w (+ bias): the scoring head, mdl.head(hn[lastidx].float())
    .squeeze(-1) (src/server.py:37, 57, 129) for a Linear(H, 1) with fp32 weight w [H] (or [1, H]) and bias [1], with
    the row gather fused in. lastidx is int64; an out-of-range index gives NaN for that score."""
    _chk(hn, "hn", torch.bfloat16)
    _chk(lastidx, "lastidx", torch.int64)
    w = w.reshape(-1)
    _chk(w, "w", torch.float32)
    if bias is not None:
        _chk(bias, "bias", torch.float32)
    rows, H = hn.shape
    if w.numel() != H:
        raise RuntimeError(f"w has {w.numel()} elements, hn rows have {H}")
    R = lastidx.numel()
    scores = torch.empty(R, dtype=torch.float32, device=hn.device)
    check(lib().ojx_head_scores(_ptr(hn), rows, H, _ptr(lastidx), R, _ptr(w), _ptr(bias), _ptr(scores), _stream()))
    return scores


def pack_gate_up(gate, up):
    """W_gu for mm_silu_mul: [2I, K], rows in blocks of 8 (4 gate rows, then the same 4 up rows)."""
    _chk(gate, "gate", torch.bfloat16)
    _chk(up, "up", torch.bfloat16)
    if gate.shape != up.shape:
        raise RuntimeError("gate and up must have the same shape")
    I, K = gate.shape
    packed = torch.empty((2 * I, K), dtype=gate.dtype, device=gate.device)
    check(lib().ojx_pack_gate_up(_ptr(gate), _ptr(up), _ptr(packed), I, K, _stream()))
    return packed


# ------------------------------------------------------------------------------------------------ packed weights
def pack_weight(w):
    """The load-time weight layout of the *_pk projections: W [N, K] -> [K/64, N/16, 16, 64] (ojx_pack_weight). For
    the fused gate-up, pack pack_gate_up's output."""
    _chk(w, "w", torch.bfloat16)
    N, K = w.shape
    if N % 16 or K % 64:
        raise RuntimeError(f"pack_weight needs N % 16 == 0 and K % 64 == 0, got {tuple(w.shape)}")
    wp = torch.empty((K // 64, N // 16, 16, 64), dtype=w.dtype, device=w.device)
    check(lib().ojx_pack_weight(_ptr(w), _ptr(wp), N, K, _stream()))
    return wp


_UNSPLIT = {}   # id(split weight) -> (weak reference to it, its version, its address, W [N, K])


def _unsplit_drop(key):
    def drop(ref):  # the split weight died: forget its W, unless the id already names a newer tensor's entry
        if _UNSPLIT.get(key, (None,))[0] is ref:
            del _UNSPLIT[key]
    return drop


def unsplit_weight(wsk):
    """W [N, K] from the reference's split-K copy wsk [S, K/S, N] (src/fastmodel.py:186-188; ojx_unsplit_weight), for
    callers that hold only that copy (lt2_run / _skmm / _res with a weight from the reference's own _split). The
    result is kept while wsk lives and is made again if wsk is modified in place; during a graph capture it is made
    inside the capture and not kept (the graph's memory pool owns it)."""
    _chk(wsk, "wsk", torch.bfloat16)
    if wsk.dim() != 3:
        raise RuntimeError(f"unsplit_weight: wsk must be [S, K/S, N], got {tuple(wsk.shape)}")
    S, KS, N = wsk.shape
    capturing = torch.cuda.is_current_stream_capturing()
    key = id(wsk)
    hit = None if capturing else _UNSPLIT.get(key)
    if hit is not None and hit[0]() is wsk and hit[1] == wsk._version and hit[2] == wsk.data_ptr():
        return hit[3]
    w = torch.empty((N, S * KS), dtype=wsk.dtype, device=wsk.device)
    check(lib().ojx_unsplit_weight(_ptr(wsk), _ptr(w), N, S * KS, S, _stream()))
    if not capturing:
        _UNSPLIT[key] = (weakref.ref(wsk, _unsplit_drop(key)), wsk._version, wsk.data_ptr(), w)
    return w


def _pk_shape(wp):
    _chk(wp, "wp", torch.bfloat16)
    if wp.dim() != 4 or tuple(wp.shape[2:]) != (16, 64):
        raise RuntimeError(f"a packed weight is [K/64, N/16, 16, 64], got {tuple(wp.shape)}")
    return wp.shape[1] * 16, wp.shape[0] * 64


def mm_pk(x, wp, cfg=None):
    """mm with a packed weight (pack_weight)."""
    _chk(x, "x", torch.bfloat16)
    N, K = _pk_shape(wp)
    M = x.shape[0]
    if x.shape[1] != K:
        raise RuntimeError(f"shape mismatch: x {tuple(x.shape)}, packed weight of K={K}")
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    ws, nws = _workspace(M, N, K, KIND_PLAIN | _lib.KIND_PACKED, cfg, x.device)
    check(lib().ojx_gemm_bf16_pk(_ptr(x), _ptr(wp), _ptr(y), M, N, K, K, N, _ptr(ws), nws, _cfgp(cfg), _stream()))
    return y


def mm_silu_mul_pk(x, wgu_pk, cfg=None):
    """mm_silu_mul with the packed gate-up weight (pack_weight(pack_gate_up(gate, up)))."""
    _chk(x, "x", torch.bfloat16)
    N, K = _pk_shape(wgu_pk)
    M = x.shape[0]
    if x.shape[1] != K:
        raise RuntimeError(f"shape mismatch: x {tuple(x.shape)}, packed weight of K={K}")
    out = torch.empty((M, N // 2), dtype=x.dtype, device=x.device)
    ws, nws = _workspace(M, N, K, KIND_SILU_MUL | _lib.KIND_PACKED, cfg, x.device)
    check(lib().ojx_gemm_silu_mul_pk(_ptr(x), _ptr(wgu_pk), _ptr(out), M, N // 2, K, _ptr(ws), nws, _cfgp(cfg),
                                     _stream()))
    return out


def mm_residual_rmsnorm_pk(h, y, wp, w1, rowmask, eps, want_hn=True, cfg=None):
    """mm_residual_rmsnorm with a packed weight."""
    _chk(h, "h", torch.bfloat16)
    _chk(y, "y", torch.bfloat16)
    N, K = _pk_shape(wp)
    M = y.shape[0]
    if y.shape[1] != K or tuple(h.shape) != (M, N):
        raise RuntimeError(f"shape mismatch: h {tuple(h.shape)} y {tuple(y.shape)}, packed weight N={N} K={K}")
    if want_hn:
        _chk_norm(w1, rowmask, M, N)
    elif rowmask is not None:
        _chk(rowmask, "rowmask", torch.int32)
    h_new = torch.empty_like(h)
    hn = torch.empty_like(h) if want_hn else None
    ws, nws = _workspace(M, N, K, KIND_RESIDUAL | _lib.KIND_PACKED, cfg, y.device)
    check(lib().ojx_gemm_residual_rmsnorm_pk(_ptr(y), _ptr(wp), _ptr(h), _ptr(w1) if want_hn else None,
                                             _ptr(rowmask), float(eps), _ptr(h_new), _ptr(hn), M, N, K, _ptr(ws),
                                             nws, _cfgp(cfg), _stream()))
    return h_new, hn


# ------------------------------------------------------------------------------------------------ attention prep
def _prep_outputs(N, HQ, HKV, D, like):
    qt = torch.empty((HQ, N, D), dtype=torch.bfloat16, device=like.device)
    kt = torch.empty((HKV, N, D), dtype=torch.bfloat16, device=like.device)
    vt = torch.empty((HKV, N, D), dtype=torch.bfloat16, device=like.device)
    gate = torch.empty((N, HQ * D), dtype=torch.bfloat16, device=like.device)
    return qt, kt, vt, gate


def _chk_rope(qw1, kw1, cos, sin, N, D):
    """The norm weights are [D] and cos / sin [N, RD] (the kernels read N rows of RD and D weights)."""
    if qw1.numel() != D or kw1.numel() != D:
        raise RuntimeError(f"qw1 and kw1 must have D={D} elements, got {qw1.numel()} and {kw1.numel()}")
    if cos.dim() != 2 or tuple(cos.shape) != tuple(sin.shape) or cos.shape[0] != N:
        raise RuntimeError(f"cos and sin must both be [N={N}, RD], got {tuple(cos.shape)} and {tuple(sin.shape)}")


def fullattn_prep2(proj, qw1, kw1, cos, sin, B, T, HQ, HKV, D, eps):
    """The reference extension's fullattn_prep2 (src/kernels.cu:302-360) for B = 1 (the tree forward's call,
    src/fastmodel.py:462): [qt [1, HQ, T, D], kt [1, HKV, T, D], vt [1, HKV, T, D], gate [T, HQ D]]."""
    _chk(proj, "proj", torch.bfloat16)
    _chk(qw1, "qw1", torch.float32)
    _chk(kw1, "kw1", torch.float32)
    _chk(cos, "cos", torch.bfloat16)
    _chk(sin, "sin", torch.bfloat16)
    if B != 1:
        raise RuntimeError("fullattn_prep2: B must be 1 (the packed-token forward)")
    N = proj.shape[0]
    if N != T or proj.shape[1] != (2 * HQ + 2 * HKV) * D:
        raise RuntimeError(f"proj {tuple(proj.shape)} does not match T={T}, HQ={HQ}, HKV={HKV}, D={D}")
    _chk_rope(qw1, kw1, cos, sin, N, D)
    RD = cos.shape[1]
    qt, kt, vt, gate = _prep_outputs(N, HQ, HKV, D, proj)
    check(lib().ojx_fullattn_prep(_ptr(proj), N, HQ, HKV, D, RD, float(eps), _ptr(qw1), _ptr(kw1), _ptr(cos),
                                  _ptr(sin), _ptr(qt), _ptr(kt), _ptr(vt), _ptr(gate), _stream()))
    return [qt.unsqueeze(0), kt.unsqueeze(0), vt.unsqueeze(0), gate]


def linattn_prep_dedup2(proj, hist, rep_ptr, rep_pos, L2, convw, A_log, dt_bias, KD, VD, HV, HK, HD, rep_qk):
    """The reference extension's linattn_prep_dedup2 (src/kernels.cu:1176-1290), as forward_gtree calls it
    (src/fastmodel.py:420,438): [q [R, RQ KD], k, v [R, VD], g fp32 [R, HV], beta [R, HV]], R = rep_pos.numel(),
    RQ = HV / HK when rep_qk else 1."""
    _chk(proj, "proj", torch.bfloat16)
    for t, nm in ((hist, "hist"), (rep_ptr, "rep_ptr"), (rep_pos, "rep_pos")):
        _chk(t, nm, torch.int32)
    for t, nm in ((convw, "convw"), (A_log, "A_log"), (dt_bias, "dt_bias")):
        _chk(t, nm, torch.bfloat16)
    N, R = proj.shape[0], rep_pos.numel()
    C = 2 * KD + VD
    if proj.dim() != 2 or proj.shape[1] != C + VD + 2 * HV:
        raise RuntimeError(f"proj {tuple(proj.shape)} is not [N, 2 KD + 2 VD + 2 HV] for KD={KD} VD={VD} HV={HV}")
    if convw.numel() != C * 4 or (convw.dim() == 2 and convw.shape[1] != 4):
        raise RuntimeError(f"convw {tuple(convw.shape)} is not [{C}, 4]")
    if hist.numel() != (N + 1) * 4 or rep_ptr.numel() != N + 2 or A_log.numel() != HV or dt_bias.numel() != HV:
        raise RuntimeError("hist must be [N + 1, 4], rep_ptr [N + 2], A_log and dt_bias [HV]")
    rq = HV // HK if rep_qk else 1
    dev = proj.device
    q = torch.empty((R, rq * KD), dtype=torch.bfloat16, device=dev)
    k = torch.empty((R, rq * KD), dtype=torch.bfloat16, device=dev)
    v = torch.empty((R, VD), dtype=torch.bfloat16, device=dev)
    g = torch.empty((R, HV), dtype=torch.float32, device=dev)
    beta = torch.empty((R, HV), dtype=torch.bfloat16, device=dev)
    check(lib().ojx_linattn_prep(_ptr(proj), _ptr(hist), _ptr(rep_ptr), _ptr(rep_pos), N, R, int(L2), _ptr(convw),
                                 _ptr(A_log), _ptr(dt_bias), KD, VD, HV, HK, HD, int(bool(rep_qk)), _ptr(q), _ptr(k),
                                 _ptr(v), _ptr(g), _ptr(beta), _stream()))
    return [q, k, v, g, beta]


def mm_fullattn_prep(x, w_qkv, qw1, kw1, cos, sin, HQ, HKV, D, eps, fused=False):
    """_mm(hn, d.w_in) + fullattn_prep2 (src/fastmodel.py:412,462): the QKV in-projection and the full-attention
    prep. w_qkv row-major [(2 HQ + 2 HKV) D, K] or packed (pack_weight). Returns the prep's outputs
    [qt [1, HQ, M, D], kt, vt, gate [M, HQ D]]. By default the planned GEMM followed by the prep kernel (two
    launches, the faster route at every measured M); fused=True runs ojx_gemm_qkv_fullattn_prep, the prep in the
    GEMM's epilogue (one launch, the [M, (2 HQ + 2 HKV) D] projection never stored)."""
    if not fused:
        rows = _pk_shape(w_qkv)[0] if w_qkv.dim() == 4 else w_qkv.shape[0]
        if rows != (2 * HQ + 2 * HKV) * D:
            raise RuntimeError(f"w_qkv does not match x {tuple(x.shape)}, HQ={HQ}, HKV={HKV}, D={D}")
        return fullattn_prep2(mm(x, w_qkv), qw1, kw1, cos, sin, 1, x.shape[0], HQ, HKV, D, eps)
    _chk(x, "x", torch.bfloat16)
    for t, nm in ((qw1, "qw1"), (kw1, "kw1")):
        _chk(t, nm, torch.float32)
    _chk(cos, "cos", torch.bfloat16)
    _chk(sin, "sin", torch.bfloat16)
    M, K = x.shape
    packed = w_qkv.dim() == 4
    N, Kw = _pk_shape(w_qkv) if packed else tuple(w_qkv.shape)
    if Kw != K or N != (2 * HQ + 2 * HKV) * D:
        raise RuntimeError(f"w_qkv does not match x {tuple(x.shape)}, HQ={HQ}, HKV={HKV}, D={D}")
    _chk_rope(qw1, kw1, cos, sin, M, D)
    qt, kt, vt, gate = _prep_outputs(M, HQ, HKV, D, x)
    check(lib().ojx_gemm_qkv_fullattn_prep(_ptr(x), _ptr(w_qkv), int(packed), _ptr(qw1), _ptr(kw1), _ptr(cos),
                                           _ptr(sin), _ptr(qt), _ptr(kt), _ptr(vt), _ptr(gate), M, K, HQ, HKV, D,
                                           cos.shape[1], float(eps), _stream()))
    return [qt.unsqueeze(0), kt.unsqueeze(0), vt.unsqueeze(0), gate]
