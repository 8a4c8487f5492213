"""ctypes binding of libojx.so (C-ABI declared in include/ojx.h).

This is the reference-side binding a Python host needs: the reference binds its kernels through
torch.utils.cpp_extension.load_inline (src/ext.py:47-54, src/lt_ext.py:5-9); here the library is a plain C-ABI
shared object, so ctypes is enough and no torch types cross the boundary. Loading fails loudly when the library
has not been built; there is no fallback path.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libojx.so")

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float


class OjxCfg(ctypes.Structure):
    _fields_ = [("tile", ctypes.c_int32), ("splitk", ctypes.c_int32), ("tail_tile", ctypes.c_int32),
                ("tail_splitk", ctypes.c_int32), ("tail_rows", ctypes.c_int32), ("one_launch", ctypes.c_int32)]

    def __repr__(self):
        t = f", tail {self.tail_rows} rows: tile {self.tail_tile} S {self.tail_splitk}" if self.tail_rows else ""
        o = {0: "", 1: ", one launch", 2: ", one launch + RMSNorm"}.get(self.one_launch, f", one_launch {self.one_launch}")
        return f"OjxCfg(tile {self.tile}, S {self.splitk}{t}{o})"


_cfgp = ctypes.POINTER(OjxCfg)

# name -> (restype, argtypes); one entry per function of include/ojx.h
EXPORTS = {
    "ojx_last_error": (ctypes.c_char_p, []),
    "ojx_version": (ctypes.c_char_p, []),
    "ojx_init": (ctypes.c_int, []),
    "ojx_num_tiles": (ctypes.c_int, []),
    "ojx_tile_info": (ctypes.c_int, [_i32, ctypes.POINTER(_i32)]),
    "ojx_plan": (ctypes.c_int, [_i64, _i64, _i64, _i32, _cfgp]),
    "ojx_num_candidates": (ctypes.c_int, [_i64, _i64, _i64, _i32]),
    "ojx_candidate": (ctypes.c_int, [_i64, _i64, _i64, _i32, _i32, _cfgp]),
    "ojx_workspace_bytes": (ctypes.c_int64, [_i64, _i64, _i64, _i32, _cfgp]),
    "ojx_gemm_bf16": (ctypes.c_int, [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64, _cfgp, _p]),
    "ojx_gemm_splitk_f32": (ctypes.c_int, [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _p]),
    "ojx_gemm_silu_mul": (ctypes.c_int, [_p, _p, _p, _i64, _i64, _i64, _p, _i64, _cfgp, _p]),
    "ojx_gemm_residual_rmsnorm": (ctypes.c_int, [_p, _p, _p, _p, _p, _f32, _p, _p, _i64, _i64, _i64, _p, _i64,
                                                 _cfgp, _p]),
    "ojx_gemm_residual_rmsnorm_noalloc": (ctypes.c_int, [_p, _p, _p, _p, _p, _f32, _p, _p, _i64, _i64, _i64, _cfgp,
                                                         _p]),
    "ojx_pack_weight": (ctypes.c_int, [_p, _p, _i64, _i64, _p]),
    "ojx_unsplit_weight": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _p]),
    "ojx_gemm_bf16_pk": (ctypes.c_int, [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _cfgp, _p]),
    "ojx_gemm_silu_mul_pk": (ctypes.c_int, [_p, _p, _p, _i64, _i64, _i64, _p, _i64, _cfgp, _p]),
    "ojx_gemm_residual_rmsnorm_pk": (ctypes.c_int, [_p, _p, _p, _p, _p, _f32, _p, _p, _i64, _i64, _i64, _p, _i64,
                                                    _cfgp, _p]),
    "ojx_fullattn_prep": (ctypes.c_int, [_p, _i64, _i32, _i32, _i32, _i32, _f32, _p, _p, _p, _p, _p, _p, _p, _p, _p]),
    "ojx_gemm_qkv_fullattn_prep": (ctypes.c_int, [_p, _p, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32,
                                                  _i32, _i32, _i32, _f32, _p]),
    "ojx_linattn_prep": (ctypes.c_int, [_p, _p, _p, _p, _i64, _i64, _i64, _p, _p, _p, _i32, _i32, _i32, _i32, _i32,
                                        _i32, _p, _p, _p, _p, _p, _p]),
    "ojx_add_rmsnorm": (ctypes.c_int, [_p, _p, _p, _p, _f32, _p, _p, _i64, _i64, _p]),
    "ojx_add_rmsnorm_sk": (ctypes.c_int, [_p, _p, _i32, _p, _p, _f32, _p, _p, _i64, _i64, _p]),
    "ojx_silu_mul": (ctypes.c_int, [_p, _p, _i64, _i64, _p]),
    "ojx_silu_mul_lut": (ctypes.c_int, [_p, _p, _p, _i64, _i64, _p]),
    "ojx_act_tables": (ctypes.c_int, [_p, _p, _p]),
    "ojx_head_scores": (ctypes.c_int, [_p, _i64, _i64, _p, _i64, _p, _p, _p, _p]),
    "ojx_pack_gate_up": (ctypes.c_int, [_p, _p, _p, _i64, _i64, _p]),
}

KIND_PLAIN, KIND_SILU_MUL, KIND_RESIDUAL, KIND_PACKED = 0, 1, 2, 4

_lib = None


def lib():
    """The loaded library (raises RuntimeError if libojx.so is missing)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() or "
                               "python open-jev-fast_amd/build.py")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in EXPORTS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _check_provenance(L)
        _lib = L
    return _lib


def _check_provenance(L) -> None:
    """The library must have been compiled from the sources beside it: ojx_version() carries a digest of csrc/ and
    include/ojx.h taken at build time. A stale build (sources edited, library not rebuilt) raises, so tests and
    benchmarks never run a binary other than the one the tree describes. OJX_ALLOW_STALE=1 skips the check."""
    from .build import source_digest
    got = L.ojx_version().decode()
    want = source_digest()
    if not got.endswith("src:" + want) and os.environ.get("OJX_ALLOW_STALE") != "1":
        raise RuntimeError(f"{LIB_PATH} ({got}) was not built from these sources (digest {want}): rebuild it with "
                           "__graft_entry__.build() or python open-jev-fast_amd/build.py")


def check(rc: int) -> None:
    """Raises RuntimeError with the library's message for a non-zero status (the reference's TORCH_CHECK path)."""
    if rc != 0:
        raise RuntimeError(f"ojx error {rc}: {lib().ojx_last_error().decode()}")


def cfg(tile: int, splitk: int, tail_tile: int = 0, tail_splitk: int = 1, tail_rows: int = 0,
        one_launch: int = 0) -> OjxCfg:
    return OjxCfg(tile, splitk, tail_tile, tail_splitk, tail_rows, one_launch)


def plan(M: int, N: int, K: int, kind: int = KIND_PLAIN) -> OjxCfg:
    c = OjxCfg()
    check(lib().ojx_plan(M, N, K, kind, ctypes.byref(c)))
    return c


def tile_info(tile: int):
    info = (_i32 * 7)()
    check(lib().ojx_tile_info(tile, info))
    return dict(zip(("bn", "bm", "bk", "wn", "wm", "threads", "family"), list(info)))


def candidates(M: int, N: int, K: int, kind: int = KIND_PLAIN):
    L = lib()
    out = []
    for i in range(L.ojx_num_candidates(M, N, K, kind)):
        c = OjxCfg()
        check(L.ojx_candidate(M, N, K, kind, i, ctypes.byref(c)))
        out.append(c)
    return out


def workspace_bytes(M: int, N: int, K: int, kind: int, c: OjxCfg = None) -> int:
    n = lib().ojx_workspace_bytes(M, N, K, kind, ctypes.byref(c) if c is not None else None)
    if n < 0:
        check(1)
    return n
