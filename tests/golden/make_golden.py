"""Write the golden fixtures (tests/golden/*.npz) from the CPU oracle.

The reference ships no golden vectors or known-answer tests for this path, so
these fixtures are this build's own: inputs plus the oracle's outputs at every
rounding point (U, V, M, y) in the reference's GEMM layouts, for shapes that
exercise the edges (C=3, K=48, non-square, pad 0/1/2, H not a multiple of 6,
B>1). tests/test_golden.py checks the oracle still reproduces them bit for
bit; tests/test_gpu_golden.py checks the HIP library against them.

Usage: python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402

CASES = {
    # name: (B, C, K, H, W, pad, seed)
    "c3_k8_13x13_p1_b2": (2, 3, 8, 13, 13, 1, 101),
    "c16_k48_14x9_p0": (1, 16, 48, 14, 9, 0, 102),
    "c24_k16_7x7_p2": (1, 24, 16, 7, 7, 2, 103),
    "c32_k32_8x8_p1": (1, 32, 32, 8, 8, 1, 104),
    "c40_k24_20x17_p1_b2": (2, 40, 24, 20, 17, 1, 105),
}


def make(name, B, C, K, H, W, pad, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, C, H, W)).astype(np.float16)
    w = (rng.standard_normal((K, C, 3, 3)) * np.sqrt(2.0 / (9 * C))).astype(np.float32)
    nh, nw, Ho, Wo = O.tiling(H, W, pad)
    U = O.filter_transform(w)
    V = O.input_transform(x, pad, nh, nw)
    M = O.batched_gemm(U, V)
    y = O.output_transform(M, B, Ho, Wo, nh, nw)
    y_full = O.conv2d(x, w, pad)
    assert np.array_equal(y.view(np.uint16), y_full.view(np.uint16))
    truth = O.direct_conv2d(x, w, pad).astype(np.float32)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), x=x, w=w, U=U, V=V, M=M, y=y,
                        y_direct=truth, shape=np.array([B, C, K, H, W, pad, nh, nw, Ho, Wo]))


if __name__ == "__main__":
    for n, args in CASES.items():
        make(n, *args)
        print("wrote", n)
