"""ojx: MI355X-native dense bf16 projection path of open-jev-fast (gate-up + SiLU.mul, in-projections,
out/down + residual + RMSNorm) as hand-written gfx950 HIP kernels behind a C-ABI (include/ojx.h).

Modules:
    _lib      ctypes binding of libojx.so (C-ABI)
    ext       the reference extension's projection-path functions (add_rmsnorm*, silu_mul*, act_tables) and the
              fused projections (mm, mm_silu_mul, mm_residual_rmsnorm, mm_splitk_f32, pack_gate_up)
    lt_ext    the reference's cuBLASLt extension surface (lt_setup / lt_matmul / lt2_*)
    fastproj  FastQwen35's projection dispatch (_mm, _res, _silu_mul, _skmm, _split, _tune)
    build     in-tree hipcc build of libojx.so
"""
from . import _lib  # noqa: F401

__all__ = ["_lib", "ext", "lt_ext", "fastproj"]


def __getattr__(name):
    if name in ("ext", "lt_ext", "fastproj", "build"):
        import importlib
        return importlib.import_module(f"{__name__}.{name}")
    raise AttributeError(name)
