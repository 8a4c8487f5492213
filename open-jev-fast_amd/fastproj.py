"""Projection dispatch of FastQwen35 (src/fastmodel.py:86-112, 114-203) on libojx.

`FastProjections` carries the methods the backbone forwards call (`_mm`, `_res`, `_silu_mul`, `_skmm`, `_split`,
`_tune`, `_tune_sk`) with the reference's signatures, so a FastQwen35-shaped class can inherit it and keep its
forward loops (src/fastmodel.py:205-482) unchanged. One call site may change to use the fused gate-up:

    m = self._silu_mul(self._mm(hn, d.w_gu))      # reference (src/fastmodel.py:478): GEMM, then SiLU.mul pass
    m = self._mm_silu(hn, d.w_gu_packed)          # one kernel, no [M, 2I] round trip through HBM

Tuning never times anything: `_tune` and `_tune_sk` read libojx's plan table, which was measured offline on MI355X,
so they are safe during stream capture (the reference falls back to F.linear while capturing,
src/fastmodel.py:163,173).
"""
import os
from types import SimpleNamespace

import torch

from . import _lib, ext

LUT = os.environ.get("OJ_LUT", "1") == "1"


_SPLIT_ENV = ("OJ_SK_LIN_OUT", "OJ_SK_FULL_OUT", "OJ_SK_DOWN")


def _env_split(name):
    """OJ_SK_* override of the split-K count; unset means the plan table decides."""
    v = os.environ.get(name)
    return int(v) if v else None


def _split_forced():
    """True when the user set one of the reference's split-K variables (src/fastmodel.py:55-57). Only then is the
    S that the forward passes to _res applied; the reference's __init__ always sets S (default 2,
    src/fastmodel.py:92,97,109), and on MI355X the measured plan is better than a fixed split."""
    return any(os.environ.get(n) for n in _SPLIT_ENV)


def _nk(w):
    """(N, K) of a weight, row-major [N, K] or packed [K/64, N/16, 16, 64]."""
    return (w.shape[1] * 16, w.shape[0] * 64) if w.dim() == 4 else (w.shape[0], w.shape[1])


def _wsk_2d(wsk, what):
    """W [N, K] (or packed) for a split-K weight: FastProjections._split returns W itself; the reference's own copy
    [S, K/S, N] (src/fastmodel.py:186-188) is turned back into W once per tensor (ext.unsplit_weight)."""
    if wsk.dim() == 3:
        return ext.unsplit_weight(wsk)
    if wsk.dim() not in (2, 4):
        raise RuntimeError(f"{what}: the split-K weight must be [N, K], packed [K/64, N/16, 16, 64] or the "
                           f"reference's [S, K/S, N]; got shape {tuple(wsk.shape)}")
    return wsk


class FastProjections:
    def __init__(self, eps: float = 1e-6):
        self.eps = eps
        self._lt_best = {}
        self._sk_best = {}

    # ------------------------------------------------------------------------------------- weights (load time)
    @staticmethod
    def _split(W, S):
        """The reference copies W to [S, K/S, N] for torch.bmm (src/fastmodel.py:186-188). libojx's split-K reads
        contiguous K ranges of W [N, K] in place, so the split weight is W itself (no second copy in HBM)."""
        return W

    @staticmethod
    def _layout(W, pack):
        """W itself, or with pack (the default) W in the stage-major packed layout (ext.pack_weight) when its shape
        allows (N % 16 == 0, K % 64 == 0): one copy of every weight, in the layout the kernels stream fastest."""
        W = W.contiguous()
        if pack and W.shape[0] % 16 == 0 and W.shape[1] % 64 == 0:
            return ext.pack_weight(W)
        return W

    @staticmethod
    def merge_mlp(gate_w, up_w, down_w, keep_cat=False, pack=True):
        """d.w_gu / d.w_down of src/fastmodel.py:90-92. d.w_gu_packed is the fused gate-up layout ([2I, K] rows,
        packed by ext.pack_weight when pack); keep_cat also keeps the reference's cat[gate; up] (row-major) for the
        unfused _silu_mul(_mm(hn, d.w_gu)) call."""
        d = SimpleNamespace()
        d.w_gu_packed = FastProjections._layout(ext.pack_gate_up(gate_w.contiguous(), up_w.contiguous()), pack)
        d.w_gu = torch.cat([gate_w, up_w], 0).contiguous() if keep_cat else None
        d.w_down = FastProjections._layout(down_w, pack)
        d.sk_down = _env_split("OJ_SK_DOWN")
        d.w_down_sk = d.w_down
        return d

    @staticmethod
    def merge_linear_attn(d, qkv_w, z_w, b_w, a_w, out_w, pack=True):
        """Linear-attention in/out projections (src/fastmodel.py:93-97): w_in = cat[qkv, z, b, a]."""
        d.w_in = FastProjections._layout(torch.cat([qkv_w, z_w, b_w, a_w], 0), pack)
        d.w_out = FastProjections._layout(out_w, pack)
        d.sk_out = _env_split("OJ_SK_LIN_OUT")
        d.w_out_sk = d.w_out
        return d

    @staticmethod
    def merge_full_attn(d, q_w, k_w, v_w, o_w, pack=True):
        """Full-attention in/out projections (src/fastmodel.py:104-109): w_in = cat[q, k, v]."""
        d.w_in = FastProjections._layout(torch.cat([q_w, k_w, v_w], 0), pack)
        d.w_out = FastProjections._layout(o_w, pack)
        d.sk_out = _env_split("OJ_SK_FULL_OUT")
        d.w_out_sk = d.w_out
        return d

    # ------------------------------------------------------------------------------------- tuning (table)
    def _tune(self, x, w):
        M, K = x.shape
        N, _ = _nk(w)
        c = _lib.plan(M, N, K, _lib.KIND_PLAIN | (_lib.KIND_PACKED if w.dim() == 4 else 0))
        self._lt_best[(M, N, K, w.dim())] = c
        return c

    def _tune_sk(self, y, wsk, S):
        """Tile for the split-K partial GEMM (_skmm): the residual plan's tile when it writes split-K planes, else -1
        (the library then picks a plane-writing tile itself; the persistent family has no K planes)."""
        M, K = y.shape
        W = _wsk_2d(wsk, "_tune_sk")
        if W.dim() == 4:
            raise RuntimeError("_skmm / _tune_sk: the split-K plane GEMM takes a row-major W [N, K]")
        N = W.shape[0]
        c = _lib.plan(M, N, K, _lib.KIND_RESIDUAL)
        tile = c.tile if _lib.tile_info(c.tile)["family"] != 5 else -1
        self._sk_best[(M, N, K, S)] = tile
        return tile

    # ------------------------------------------------------------------------------------- projections
    def _mm(self, x, w):
        key = (x.shape[0], _nk(w)[0], x.shape[1], w.dim())
        c = self._lt_best.get(key)
        if c is None:
            c = self._tune(x, w)
        return ext.mm(x, w, cfg=c)

    def _skmm(self, y, wsk, S):
        """parts [S, M, N] fp32 = the S K-chunks of y times W (the reference's torch.bmm / lt2_run)."""
        M, K = y.shape
        W = _wsk_2d(wsk, "_skmm")
        key = (M, W.shape[0], K, S)
        tile = self._sk_best.get(key)
        if tile is None:
            tile = self._tune_sk(y, W, S)
        return ext.mm_splitk_f32(y, W, S, tile=tile)

    def _silu_mul(self, gu):
        if LUT:
            if not hasattr(self, "_silu_tab"):
                self._silu_tab, self._sig_tab = ext.act_tables(gu)
            return ext.silu_mul_lut(gu, self._silu_tab)
        return ext.silu_mul(gu)

    def _mm_silu(self, x, w_gu_packed):
        return ext.mm_silu_mul(x, w_gu_packed)

    def _res(self, h, y, wsk, S, w1, mask, w=None):
        """(h_new, hn) = residual add + RMSNorm after the out / down projection (src/fastmodel.py:196-203), as one
        call of the fused projection. The configuration (tile, split-K or stream-K spread) comes from the plan
        table. The S the forward passes (the reference's d.sk_out / d.sk_down, 2 by default) is applied only when
        an OJ_SK_* variable is set, as a split-K count with a tile that writes K planes."""
        W = w if w is not None else _wsk_2d(wsk, "_res")
        M, K = y.shape
        N, _ = _nk(W)
        cfg = None
        if S and _split_forced():
            cfg = self._forced_cfg(M, N, K, int(S), W.dim() == 4)
        return ext.mm_residual_rmsnorm(h, y, W, w1, mask, self.eps, want_hn=True, cfg=cfg)

    @staticmethod
    def _forced_cfg(M, N, K, S, packed=False):
        """(tile, S) for an explicit split-K count: the plan's tile if it writes K planes, else the first candidate
        with that split that does. None (the plan) if no candidate takes S for this shape."""
        kind = _lib.KIND_RESIDUAL | (_lib.KIND_PACKED if packed else 0)
        plan = _lib.plan(M, N, K, kind)
        cands = [c for c in _lib.candidates(M, N, K, kind)
                 if c.splitk == S and _lib.tile_info(c.tile)["family"] != 5]
        for c in cands:
            if c.tile == plan.tile:
                return c
        return cands[0] if cands else None
