"""Writes tests/golden/proj_golden.npz: small projection vectors with fp64 brute-force outputs.

The reference commits no golden vectors for this path (its tests print statistics only), so these vectors are
computed here, independently of torch's GEMM: inputs are seeded bf16 (stored as raw uint16 bit patterns) and the
expected output is the exact fp64 dot product (numpy, float64), which both the CPU oracle and the GPU kernels must
match to within one bf16 rounding. Shapes cover M = 1..4 and ragged M, N not a multiple of 64 (the N = 16480
in-projection has a 32-row tail; 1040 = 16 * 65 has the same property), and K not a multiple of 64.

    python tests/golden/make_golden.py
"""
import os

import numpy as np

SHAPES = {
    "m1_n64_k256": (1, 64, 256),
    "m3_n40_k72": (3, 40, 72),
    "m4_n64_k128": (4, 64, 128),
    "m9_n1040_k64": (9, 1040, 64),
    "m17_n24_k264": (17, 24, 264),
}


def bf16_bits(a):
    """float32 -> bf16 bit patterns, round to nearest even."""
    u = a.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bits_to_f64(b):
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def main():
    rng = np.random.default_rng(20260)
    out = {}
    for name, (M, N, K) in SHAPES.items():
        xb = bf16_bits(rng.standard_normal((M, K)))
        wb = bf16_bits(rng.standard_normal((N, K)) * 0.02)
        out[f"{name}__x"] = xb
        out[f"{name}__w"] = wb
        out[f"{name}__y64"] = bits_to_f64(xb) @ bits_to_f64(wb).T
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "proj_golden.npz")
    np.savez_compressed(path, **out)
    print(path, sum(v.nbytes for v in out.values()), "bytes")


if __name__ == "__main__":
    main()
