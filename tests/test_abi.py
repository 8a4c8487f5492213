"""C-ABI checks that need no GPU: the library loads, exports every function include/ojx.h declares, and its host
logic (plan table, candidate list, workspace sizes, argument validation and error messages) behaves."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "ojx.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(ojx_\w+)\s*\(", text, re.M)))


def test_header_symbols_exported(pkg):
    names = header_functions()
    assert len(names) >= 19
    L = ctypes.CDLL(pkg._lib.LIB_PATH)
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(pkg._lib.EXPORTS), "ctypes table out of sync with include/ojx.h"


def test_version_and_tiles(pkg):
    L = pkg._lib.lib()
    assert b"gfx950" in L.ojx_version()
    from importlib import import_module
    build = import_module("open_jev_fast_amd.build")
    # the loaded binary was compiled from this tree's sources (digest of csrc/ and include/ojx.h)
    assert L.ojx_version().decode().endswith("src:" + build.source_digest())
    n = L.ojx_num_tiles()
    assert n >= 8
    live = 0
    for t in range(n):
        info = pkg._lib.tile_info(t)
        if info["family"] < 0:  # a retired id: never planned, fitted or launched
            assert all(c.tile != t for c in pkg._lib.candidates(288, 1024, 2048, 0))
            continue
        live += 1
        assert info["bn"] % 16 == 0 and info["bm"] % 16 == 0 and info["bk"] % 32 == 0
        assert info["threads"] == 64 * info["wn"] * info["wm"]
    assert live >= 8 and pkg._lib.tile_info(52)["family"] == -1
    with pytest.raises(RuntimeError, match="out of range"):
        pkg._lib.tile_info(n)


SHAPES = [(M, N, K) for M in (1, 7, 16, 64, 128, 288, 539, 1024, 2048)
          for N, K in ((14336, 5120), (34816, 5120), (5120, 17408), (5120, 6144), (16384, 5120), (16480, 5120))]


def test_plan_table_names_live_tiles(pkg):
    """Every tile id stored in the plan table (main and tail) is a live tile: a retired id reports family -1."""
    import os
    import re
    src = os.path.join(os.path.dirname(pkg.__file__), "csrc", "plan_table.inc")
    rows = [list(map(int, m.group(1).split(","))) for m in re.finditer(r"^\{([^}]*)\}", open(src).read(), re.M)]
    assert len(rows) > 100
    for r in rows:
        for t in (r[4], r[6]):
            assert pkg._lib.tile_info(t)["family"] >= 0, f"plan row {r} names tile {t}"


@pytest.mark.parametrize("kind", [0, 1, 2, 4, 5, 6])
def test_plan_valid_for_every_contract_shape(pkg, kind):
    L = pkg._lib.lib()
    for M, N, K in SHAPES:
        c = pkg._lib.plan(M, N, K, kind)
        assert 0 <= c.tile < L.ojx_num_tiles() and 1 <= c.splitk <= 16
        live = lambda t: pkg._lib.tile_info(t)["family"] >= 0  # noqa: E731
        assert live(c.tile) and (c.tail_rows == 0 or live(c.tail_tile))
        ws = pkg._lib.workspace_bytes(M, N, K, kind)
        # each launch's data one after the other: split-K planes (rounded up to 256 bytes) or, for the persistent
        # family, partial-tile slots (or nothing)
        parts = [(c.tile, c.splitk, N - c.tail_rows)] + ([(c.tail_tile, c.tail_splitk, c.tail_rows)] if c.tail_rows else [])
        data, sk = 0, False
        for tile, S, n in parts:
            if pkg._lib.tile_info(tile)["family"] == 5:
                sk = True
            elif S > 1:
                data += -(-S * M * n * 4 // 256) * 256
                if c.one_launch:  # the per-tile row sums of squares follow the planes
                    data += -(-(-(-n // pkg._lib.tile_info(tile)["bn"])) * M * 4 // 256) * 256
        if sk:
            assert ws >= data
        else:
            assert ws == data


def test_candidates(pkg):
    cands = pkg._lib.candidates(288, 5120, 5120)
    assert len(cands) > 10
    assert len({(c.tile, c.splitk, c.one_launch) for c in cands}) == len(cands)
    ol = [c for c in cands if c.one_launch]
    assert ol and all(pkg._lib.tile_info(c.tile)["family"] in (0, 6) and c.splitk >= 2 for c in ol)
    assert all(c.one_launch == 1 for c in ol)  # the RMSNorm fold (2) is a residual candidate only
    fold = [c for c in pkg._lib.candidates(7, 5120, 6144, 2) if c.one_launch == 2]
    assert fold and all(pkg._lib.tile_info(c.tile)["family"] == 0 for c in fold)
    # no tile whose x rows are mostly padding at M = 7
    for c in pkg._lib.candidates(7, 5120, 5120):
        assert pkg._lib.tile_info(c.tile)["bm"] == 16
    L = pkg._lib.lib()
    c = pkg._lib.OjxCfg()
    assert L.ojx_candidate(7, 5120, 5120, 0, 10 ** 6, ctypes.byref(c)) == 4
    assert b"out of range" in L.ojx_last_error()


def test_argument_validation_without_gpu(pkg):
    """These return before any HIP call, so they run on a machine without a GPU."""
    L = pkg._lib.lib()
    buf = ctypes.create_string_buffer(1 << 12)
    p = ctypes.cast(ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16, ctypes.c_void_p)
    # N not a multiple of 8
    assert L.ojx_gemm_bf16(p, p, p, 4, 60, 64, 64, 64, 60, None, 0, None, None) == 2
    assert b"multiples of 8" in L.ojx_last_error()
    # null operand
    assert L.ojx_gemm_bf16(None, p, p, 4, 64, 64, 64, 64, 64, None, 0, None, None) == 1
    # misaligned
    mis = ctypes.c_void_p(p.value + 2)
    assert L.ojx_gemm_bf16(mis, p, p, 4, 64, 64, 64, 64, 64, None, 0, None, None) == 1
    # stride smaller than K
    assert L.ojx_gemm_bf16(p, p, p, 4, 64, 64, 32, 64, 64, None, 0, None, None) == 1
    # bad config
    bad = pkg._lib.OjxCfg(999, 1)
    assert L.ojx_gemm_bf16(p, p, p, 4, 64, 64, 64, 64, 64, None, 0, ctypes.byref(bad), None) == 4
    bad = pkg._lib.OjxCfg(0, 17)
    assert L.ojx_gemm_bf16(p, p, p, 4, 64, 64, 64, 64, 64, None, 0, ctypes.byref(bad), None) == 4
    # split-K without workspace
    sk = pkg._lib.OjxCfg(0, 2)
    assert L.ojx_gemm_bf16(p, p, p, 4, 64, 64, 64, 64, 64, None, 0, ctypes.byref(sk), None) == 3
    assert b"workspace" in L.ojx_last_error()
    # RMSNorm row limit (H/8 <= 1024), as the reference's TORCH_CHECK (src/kernels.cu:757)
    assert L.ojx_add_rmsnorm(p, None, p, None, 1e-6, None, p, 4, 8200, None) == 2
    assert L.ojx_add_rmsnorm_sk(p, p, 17, p, None, 1e-6, p, p, 4, 64, None) == 4
    # silu_mul needs I % 8 == 0
    assert L.ojx_silu_mul(p, p, 4, 12, None) == 2
    assert L.ojx_gemm_silu_mul(p, p, p, 4, 6, 64, None, 0, None, None) == 2
    assert L.ojx_pack_gate_up(p, p, p, 6, 64, None) == 2
    # M == 0 is a no-op
    assert L.ojx_gemm_bf16(p, p, p, 0, 64, 64, 64, 64, 64, None, 0, None, None) == 0
    # scoring head: H % 8, null operands, misalignment; R == 0 is a no-op
    assert L.ojx_head_scores(p, 4, 60, p, 3, p, None, p, None) == 2
    assert L.ojx_head_scores(None, 4, 64, p, 3, p, None, p, None) == 1
    assert L.ojx_head_scores(mis, 4, 64, p, 3, p, None, p, None) == 1
    assert L.ojx_head_scores(p, 4, 64, p, 0, p, None, p, None) == 0


def test_prep_argument_validation_without_gpu(pkg):
    """The prep entry points reject what their kernels do not handle before any HIP call (head dims, rotary dims,
    head-count ratios, sizes, alignment); empty inputs are no-ops."""
    L = pkg._lib.lib()
    buf = ctypes.create_string_buffer(1 << 12)
    p = ctypes.cast(ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16, ctypes.c_void_p)
    mis = ctypes.c_void_p(p.value + 2)
    f = ctypes.cast(p, ctypes.POINTER(ctypes.c_float))
    fa = lambda N, HQ, HKV, D, RD, proj=p: L.ojx_fullattn_prep(proj, N, HQ, HKV, D, RD, 1e-6, f, f, p, p, p, p, p,  # noqa: E731
                                                                p, None)
    assert fa(3, 2, 1, 128, 64) == 2 and b"head_dim 256" in L.ojx_last_error()
    assert fa(3, 2, 1, 256, 48) == 2 and b"rotary" in L.ojx_last_error()   # 48 / 16 = 3, not a power of two
    assert fa(3, 2, 1, 256, 8) == 2                                          # below 16
    assert fa(3, 2, 1, 256, 512) == 2                                        # above D
    assert fa(3, 0, 1, 256, 64) == 2
    assert fa(3, 2, 1, 256, 64, proj=mis) == 1
    assert fa(0, 2, 1, 256, 64, proj=None) == 0                              # no tokens: nothing to do
    q = lambda M, K, RD, w=p: L.ojx_gemm_qkv_fullattn_prep(p, w, 0, f, f, p, p, p, p, p, p, M, K, 2, 1, 256, RD,  # noqa: E731
                                                           1e-6, None)
    assert q(4, 256, 32) == 2 and b"RD = 64" in L.ojx_last_error()
    assert q(4, 260, 64) == 2                                                # K not a multiple of 8
    assert q(4, 256, 64, w=None) == 1
    la = lambda N, R, L2, KD, VD, HV, HK, HD, rq, proj=p: L.ojx_linattn_prep(  # noqa: E731
        proj, p, p, p, N, R, L2, p, p, p, KD, VD, HV, HK, HD, rq, p, p, p, f, p, None)
    assert la(5, 32, 16, 256, 768, 6, 2, 64, 0) == 2 and b"head_dim 128" in L.ojx_last_error()
    assert la(5, 32, 16, 384, 768, 6, 2, 128, 0) == 2                       # KD != HK HD
    assert la(5, 30, 16, 256, 768, 6, 2, 128, 0) == 2                       # R not a multiple of L2
    assert la(5, 32, 16, 256, 768, 8, 2, 128, 1) == 2 and b"HV / HK = 3" in L.ojx_last_error()
    assert la(5, 32, 16, 256, 768, 300, 2, 128, 0) == 2                     # HV > 256
    assert la(5, 32, 16, 256, 768, 6, 2, 128, 0, proj=mis) == 1
    assert la(5, 0, 16, 256, 768, 6, 2, 128, 0, proj=None) == 0             # no slots: nothing to do


def test_python_mirror_errors_without_gpu(pkg):
    import torch
    from importlib import import_module
    ext = import_module("open_jev_fast_amd.ext")
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="contiguous CUDA"):
        ext.mm(x, x)
    with pytest.raises(RuntimeError, match="S must be 2..4"):
        ext.add_rmsnorm_sk2(x, torch.zeros(5, 4, 64), torch.ones(64), None, 1e-6)
    lt = import_module("open_jev_fast_amd.lt_ext").load()
    assert lt.lt_setup(288, 5120, 5120, 8) == 8
    with pytest.raises(RuntimeError, match="lt_setup not called"):
        lt.lt_matmul(torch.zeros(3, 64, dtype=torch.bfloat16), torch.zeros(64, 64, dtype=torch.bfloat16), 0)
    with pytest.raises(RuntimeError, match="fp32"):
        lt.lt2_plan(288, 5120, 6144, 2, 0, 1)
    h = lt.lt2_plan(288, 5120, 6144, 2, 1, 1)
    n = lt.lt2_search(h, 400, 3)
    assert n >= 1 and lt.lt2_info(h, 0)[1] == 2
    raw = lt.lt2_raw(h, 0)
    assert lt.lt2_add_raw(h, raw) == n


def test_unsplit_weight_argument_validation(pkg):
    L = pkg._lib.lib()
    buf = ctypes.create_string_buffer(1 << 12)
    p = ctypes.cast(ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16, ctypes.c_void_p)
    assert L.ojx_unsplit_weight(p, p, 64, 96, 5, None) == 2  # K % S != 0
    assert b"multiple of S" in L.ojx_last_error()
    assert L.ojx_unsplit_weight(p, p, 60, 96, 2, None) == 2  # N not a multiple of 8
    assert L.ojx_unsplit_weight(None, p, 64, 96, 2, None) == 1
    assert L.ojx_unsplit_weight(p, ctypes.c_void_p(p.value + 2), 64, 96, 2, None) == 1


C_HOST = r"""
#include <stdio.h>
#include "ojx.h"
int main(void) {
  ojx_cfg c;
  if (ojx_plan(288, 34816, 5120, OJX_KIND_SILU_MUL | OJX_KIND_PACKED, &c) != OJX_OK) return 1;
  long long ws = (long long)ojx_workspace_bytes(288, 34816, 5120, OJX_KIND_SILU_MUL | OJX_KIND_PACKED, &c);
  printf("%s|%d|%d|%d|%lld\n", ojx_version(), ojx_num_tiles(), c.tile, c.splitk, ws);
  return ws < 0;
}
"""


def test_c_host_compiles_links_and_plans(pkg, tmp_path):
    """include/ojx.h is plain C (C99) and C++; a C host links libojx.so and uses its host-side calls (the plan
    lookup and workspace size need no GPU), as the C / C++ integration path does."""
    import shutil
    import subprocess
    inc = os.path.join(ROOT, "include")
    for comp, std, lang in (("gcc", "-std=c99", "c"), ("g++", "-std=c++17", "c++")):
        if shutil.which(comp) is None:
            pytest.skip(f"{comp} not installed")
        r = subprocess.run([comp, std, "-Wall", "-Werror", "-fsyntax-only", "-x", lang, os.path.join(inc, "ojx.h")],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
    src = tmp_path / "host.c"
    src.write_text(C_HOST)
    exe = tmp_path / "host"
    libdir = os.path.dirname(pkg._lib.LIB_PATH)
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", inc, str(src), "-o", str(exe), pkg._lib.LIB_PATH,
                        "-Wl,-rpath," + libdir, "-Wl,--allow-shlib-undefined"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    version, ntiles, tile, splitk, ws = r.stdout.strip().split("|")
    c = pkg._lib.plan(288, 34816, 5120, 1 | 4)
    assert version == pkg._lib.lib().ojx_version().decode()
    assert int(ntiles) == pkg._lib.lib().ojx_num_tiles()
    assert (int(tile), int(splitk)) == (c.tile, c.splitk)
    assert int(ws) == pkg._lib.workspace_bytes(288, 34816, 5120, 1 | 4)
