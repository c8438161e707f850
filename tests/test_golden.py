"""The CPU oracle reproduces the committed golden fixtures bit for bit, and
the fixtures sit at the reference's error level against the direct
convolution stored beside them."""

import glob
import os

import numpy as np
import pytest

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def test_fixtures_present():
    assert len(GOLDEN) >= 5


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_oracle_reproduces_fixture(oracle, path):
    f = np.load(path)
    B, C, K, H, W, pad, nh, nw, Ho, Wo = (int(v) for v in f["shape"])
    assert oracle.tiling(H, W, pad) == (nh, nw, Ho, Wo)
    U = oracle.filter_transform(f["w"])
    V = oracle.input_transform(f["x"], pad, nh, nw)
    M = oracle.batched_gemm(U, V)
    y = oracle.output_transform(M, B, Ho, Wo, nh, nw)
    for name, got in [("U", U), ("V", V), ("M", M), ("y", y)]:
        assert np.array_equal(got.view(np.uint16), f[name].view(np.uint16)), name
    rel = oracle.rel_l2(f["y"], f["y_direct"])
    assert rel < 0.06, rel
