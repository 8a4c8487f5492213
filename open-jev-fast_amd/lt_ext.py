"""The reference's cuBLASLt extension surface (src/lt_ext.py, src/lt.cpp) over libojx's tile registry.

    LT = load()
    n = LT.lt_setup(M, N, K, max_algos)   # candidate configurations for the shape  (src/lt.cpp:15-42)
    y = LT.lt_matmul(x, w, idx)           # run candidate idx                        (src/lt.cpp:43-55)
    h = LT.lt2_plan(M, N, K, S, f32, wl)  # split-K plan handle                      (src/lt.cpp:64-87)
    n = LT.lt2_search(h, max, modes)      # candidate tiles for that split           (src/lt.cpp:93-159)
    parts = LT.lt2_run(h, x, w, idx)      # [S, M, N] fp32 partials                  (src/lt.cpp:160-169)
    LT.lt2_info(h, idx); LT.lt2_raw(h, idx); LT.lt2_add_raw(h, raw)                 (src/lt.cpp:170-190)

A "candidate" is a (tile, split-K) pair of libojx rather than a cuBLASLt algorithm; a raw descriptor is that pair.
Differences, on purpose: the kernels read the K chunks of W [N, K] in place, so lt2_run takes W itself; the
reference's split-K copy [S, K/S, N] (wl=1, src/lt.cpp:58-59) is also accepted and turned back into W once per
weight tensor (ext.unsplit_weight, kept while that tensor lives). Only fp32 partials exist (f32=0 raises), which is
what the reference uses.
"""
import torch

from . import _lib, ext


class _LT:
    def __init__(self):
        self._plans = {}   # (M, N, K) -> [OjxCfg]
        self._sk = []      # handle -> dict

    # -------------------------------------------------------------------------------------------- plain GEMM
    def lt_setup(self, M, N, K, max_algos):
        key = (int(M), int(N), int(K))
        if key not in self._plans:
            self._plans[key] = _lib.candidates(*key, _lib.KIND_PLAIN)[: int(max_algos)]
        return len(self._plans[key])

    def lt_matmul(self, x, w, idx):
        if not (x.is_contiguous() and w.is_contiguous() and x.dtype == torch.bfloat16):
            raise RuntimeError("x and w must be contiguous bf16")
        key = (x.shape[0], w.shape[0], x.shape[1])
        plans = self._plans.get(key)
        if plans is None:
            raise RuntimeError("lt_setup not called for this shape")
        if not 0 <= idx < len(plans):
            raise RuntimeError(f"algorithm index {idx} out of range [0, {len(plans)})")
        return ext.mm(x, w, cfg=plans[idx])

    # -------------------------------------------------------------------------------------------- split-K
    def lt2_plan(self, M, N, K, S, f32, wl):
        if not f32:
            raise RuntimeError("only fp32 split-K partials are supported (f32=1)")
        if wl not in (0, 1):
            raise RuntimeError("wl must be 0 or 1")
        if wl == 0 and int(S) != 1:
            raise RuntimeError("wl=0 (w [N, K]) needs S == 1")   # the reference's TORCH_CHECK, src/lt.cpp:67
        # tiles that write split-K planes (the persistent family's splitk is a stream-K spread, with no K planes)
        tiles = sorted({c.tile for c in _lib.candidates(int(M), int(N), int(K), _lib.KIND_RESIDUAL)
                        if c.splitk == int(S) and _lib.tile_info(c.tile)["family"] != 5})
        self._sk.append({"shape": (int(M), int(N), int(K)), "S": int(S), "wl": int(wl), "tiles": tiles,
                         "found": tiles})
        return len(self._sk) - 1

    def _plan(self, h):
        if not 0 <= h < len(self._sk):
            raise RuntimeError(f"bad plan handle {h}")
        return self._sk[h]

    def lt2_search(self, h, max_cands, modes=3):
        p = self._plan(h)
        p["found"] = p["tiles"][: int(max_cands)]
        return len(p["found"])

    def lt2_run(self, h, x, w, idx):
        p = self._plan(h)
        if not 0 <= idx < len(p["found"]):
            raise RuntimeError(f"candidate index {idx} out of range [0, {len(p['found'])})")
        M, N, K = p["shape"]
        if w.dim() == 3:   # the reference's split-K copy [S, K/S, N] (src/lt.cpp:58-59, wl=1)
            if tuple(w.shape) != (p["S"], K // p["S"], N) or K % p["S"]:
                raise RuntimeError(f"w {tuple(w.shape)} does not match the plan's [S, K/S, N] = "
                                   f"[{p['S']}, {K // p['S']}, {N}]")
            w = ext.unsplit_weight(w)
        if tuple(x.shape) != (M, K) or tuple(w.shape) != (N, K):
            raise RuntimeError("x / w do not match the plan's shape (w must be [N, K] or [S, K/S, N])")
        return ext.mm_splitk_f32(x, w, p["S"], tile=p["found"][idx])

    def lt2_info(self, h, idx):
        p = self._plan(h)
        t = p["found"][idx]
        info = _lib.tile_info(t)
        return [t, p["S"], info["bn"], info["bm"], info["bk"], info["threads"]]

    def lt2_raw(self, h, idx):
        p = self._plan(h)
        return [p["found"][idx], p["S"]]

    def lt2_add_raw(self, h, raw):
        p = self._plan(h)
        tile, S = int(raw[0]), int(raw[1])
        if S != p["S"] or not 0 <= tile < _lib.lib().ojx_num_tiles():
            raise RuntimeError("raw descriptor does not fit this plan")
        p["found"] = p["found"] + [tile]
        return len(p["found"]) - 1


def load():
    """Returns the LT object (the reference JIT-builds lt.cpp here; libojx is prebuilt in-tree)."""
    _lib.lib()
    return _LT()
