"""Seeded random shapes through every path, against the CPU oracle.

Forty small layers drawn from one seed (batch 1-6, 1-160 input and output
channels, images 1x1 to 40x40 including non-square ones, pad 0-2) run through
the automatic choice and each forced path (three-pass, fused rows, fused
tile-block, small-problem fused, two-pass, windowed, the input transform in
the products), NCHW and, for C % 8 == 0, channels-last. Every output is
finite and within the reference's tolerance of the oracle; three-pass,
two-pass, windowed and path 7 agree bit for bit (the same arithmetic); a
forced fused path either runs or reports that it fell back to three-pass. The shapes cover edges the hand-picked cases may
miss: one-tile images, channel counts off every 8/16/32 block, K below 16,
tiles past an image edge in every position of a tile block.
"""

import random

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
CL = torch.channels_last


def _shapes(n=40, seed=2024):
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        B = rng.randint(1, 6)
        C = rng.choice([1, 3, 8, 16, 24, 40, 64, 72, 96, 128, 136, 160, rng.randint(1, 160)])
        K = rng.choice([4, 8, 15, 16, 32, 48, 64, 100, 128, 160, rng.randint(1, 160)])
        H = rng.randint(1, 40)
        W = rng.choice([H, rng.randint(1, 40)])
        pad = rng.choice([0, 1, 1, 2])
        if H + 2 * pad < 3 or W + 2 * pad < 3:
            continue
        out.append((B, C, K, H, W, pad))
    return out


SHAPES = _shapes()


def _run(lib, x, w, pad, path, nhwc=False):
    from nova_winograd.ops import check

    B, C, H, W = x.shape
    K = w.shape[0]
    Ho, Wo = H + 2 * pad - 2, W + 2 * pad - 2
    fmt = CL if nhwc else torch.contiguous_format
    y = torch.full((B, K, Ho, Wo), float("nan"), dtype=torch.float16, device=DEV).contiguous(
        memory_format=fmt)
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, path)
        lib.nova_set_layout(h, 1 if nhwc else 0)
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, W, pad)
        took = lib.nova_get_last_path(h)
        torch.cuda.synchronize()
        if path in (2, 3, 5, 7) and took == 1:
            # a forced fused path outside its envelope runs three-pass and says so
            assert lib.nova_get_last_error() != 0
        else:
            check()
    finally:
        lib.nova_destroy(h)
    return y, took


@pytest.mark.parametrize("B,C,K,H,W,pad", SHAPES)
def test_random_shape_all_paths(oracle, B, C, K, H, W, pad):
    from nova_winograd.ops import get_lib

    print(f"[random] B={B} C={C} K={K} H={H} W={W} pad={pad}", flush=True)
    lib = get_lib()
    g = torch.Generator().manual_seed(B * 1000 + C * 37 + K * 11 + H * 3 + W + pad)
    x = torch.randn(B, C, H, W, generator=g).half()
    w = torch.randn(K, C, 3, 3, generator=g) * (2.0 / (9 * C)) ** 0.5
    xd, wd = x.to(DEV), w.to(DEV)
    n = min(B, 2)
    yo = oracle.conv2d(x[:n].numpy(), w.numpy(), pad)
    outs = {}
    for path in (0, 1, 2, 3, 4, 5, 6, 7):
        y, took = _run(lib, xd, wd, pad, path)
        yc = y.cpu()
        a = yc.float().numpy()
        assert np.isfinite(a).all(), (path, took)
        assert oracle.rel_l2(a[:n].astype(np.float16), yo) <= 5e-3, (path, took)
        assert oracle.max_abs(a[:n].astype(np.float16), yo) <= 0.25, (path, took)
        outs[path] = (yc, took)
    y1 = outs[1][0]
    for path in (4, 6, 7):  # same arithmetic as three-pass
        assert torch.equal(outs[path][0], y1), path
    if C % 8 == 0:
        # channels-last: the same kernels' arithmetic, so the same bits per path
        xc = xd.contiguous(memory_format=CL)
        for path in (0, 1, 6, 7):
            y, took = _run(lib, xc, wd, pad, path, nhwc=True)
            ref, took_ref = outs[path]
            if took == took_ref:
                assert torch.equal(y.contiguous().cpu(), ref.contiguous()), (path, took)
            a = y.contiguous().cpu().float().numpy()
            assert oracle.rel_l2(a[:n].astype(np.float16), yo) <= 5e-3, (path, took)
