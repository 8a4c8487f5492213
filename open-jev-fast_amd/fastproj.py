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


def _env_split(name):
    """OJ_SK_* override of the split-K count; unset means the plan table decides."""
    v = os.environ.get(name)
    return int(v) if v else None


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
    def merge_mlp(gate_w, up_w, down_w, keep_cat=False):
        """d.w_gu / d.w_down of src/fastmodel.py:90-92. d.w_gu_packed is the fused gate-up layout ([2I, K]);
        keep_cat also keeps the reference's cat[gate; up] for the unfused _silu_mul(_mm(hn, d.w_gu)) call."""
        d = SimpleNamespace()
        d.w_gu_packed = ext.pack_gate_up(gate_w.contiguous(), up_w.contiguous())
        d.w_gu = torch.cat([gate_w, up_w], 0).contiguous() if keep_cat else None
        d.w_down = down_w.contiguous()
        d.sk_down = _env_split("OJ_SK_DOWN")
        d.w_down_sk = d.w_down
        return d

    @staticmethod
    def merge_linear_attn(d, qkv_w, z_w, b_w, a_w, out_w):
        """Linear-attention in/out projections (src/fastmodel.py:93-97): w_in = cat[qkv, z, b, a]."""
        d.w_in = torch.cat([qkv_w, z_w, b_w, a_w], 0).contiguous()
        d.w_out = out_w.contiguous()
        d.sk_out = _env_split("OJ_SK_LIN_OUT")
        d.w_out_sk = d.w_out
        return d

    @staticmethod
    def merge_full_attn(d, q_w, k_w, v_w, o_w):
        """Full-attention in/out projections (src/fastmodel.py:104-109): w_in = cat[q, k, v]."""
        d.w_in = torch.cat([q_w, k_w, v_w], 0).contiguous()
        d.w_out = o_w.contiguous()
        d.sk_out = _env_split("OJ_SK_FULL_OUT")
        d.w_out_sk = d.w_out
        return d

    # ------------------------------------------------------------------------------------- tuning (table)
    def _tune(self, x, w):
        M, K = x.shape
        N = w.shape[0]
        c = _lib.plan(M, N, K, _lib.KIND_PLAIN)
        self._lt_best[(M, N, K)] = c
        return c

    def _tune_sk(self, y, wsk, S):
        M, K = y.shape
        N = wsk.shape[0]
        c = _lib.plan(M, N, K, _lib.KIND_RESIDUAL)
        self._sk_best[(M, N, K, S)] = c.tile
        return c.tile

    # ------------------------------------------------------------------------------------- projections
    def _mm(self, x, w):
        key = (x.shape[0], w.shape[0], x.shape[1])
        c = self._lt_best.get(key)
        if c is None:
            c = self._tune(x, w)
        return ext.mm(x, w, cfg=c)

    def _skmm(self, y, wsk, S):
        M, K = y.shape
        key = (M, wsk.shape[0], K, S)
        tile = self._sk_best.get(key)
        if tile is None:
            tile = self._tune_sk(y, wsk, S)
        return ext.mm_splitk_f32(y, wsk, S, tile=tile)

    def _silu_mul(self, gu):
        if LUT:
            if not hasattr(self, "_silu_tab"):
                self._silu_tab, self._sig_tab = ext.act_tables(gu)
            return ext.silu_mul_lut(gu, self._silu_tab)
        return ext.silu_mul(gu)

    def _mm_silu(self, x, w_gu_packed):
        return ext.mm_silu_mul(x, w_gu_packed)

    def _res(self, h, y, wsk, S, w1, mask, w=None):
        """(h_new, hn) = residual add + RMSNorm after the out / down projection (src/fastmodel.py:196-203).
        S None / 0 = the plan table's split; an explicit S forces that split with the plan's tile."""
        W = w if w is not None else wsk
        M, K = y.shape
        N = W.shape[0]
        cfg = None
        if S:
            c = _lib.plan(M, N, K, _lib.KIND_RESIDUAL)
            cfg = _lib.cfg(c.tile, int(S))
        return ext.mm_residual_rmsnorm(h, y, W, w1, mask, self.eps, want_hn=True, cfg=cfg)
