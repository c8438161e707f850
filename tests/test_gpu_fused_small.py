"""The small-problem fused kernel (path 5: one launch, 2 tiles x 16 output
channels per workgroup, each workgroup recomputing its tiles' input
transform; C, K <= 128) through the C-ABI.

Its transforms are the lane-parallel chains and its products use the fused
tile-block kernel's operand order, so wherever the tile-block kernel runs the
result must equal it bit for bit (C, K <= 64); everywhere it must match the oracle within
the forward parity bar. Covered: batch 1 and small batches, C and K off the
16/32 blocks (C = 3, 20, K = 8, 48), odd and non-square images, pads 0-2,
channels-last, and the bias/residual/ReLU epilogue. A grid of at most one
workgroup per CU runs 1024-thread workgroups, a larger one 512-thread
workgroups; the cases with more than 256 workgroups (conv2_x at batch 2, the
batch-9 case) take the second.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
CL = torch.channels_last


def _run(x, w, pad, path, nhwc=False, bias=None, relu=0, res=None):
    from nova_winograd.ops import check, get_lib

    lib = get_lib()
    B, C, H, W = x.shape
    K = w.shape[0]
    y = torch.empty(B, K, H + 2 * pad - 2, W + 2 * pad - 2, dtype=torch.float16, device=DEV,
                    memory_format=CL if nhwc else torch.contiguous_format)
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, path)
        lib.nova_set_layout(h, 1 if nhwc else 0)
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        lib.nova_set_epilogue(h, bias.data_ptr() if bias is not None else None, relu)
        lib.nova_set_residual(h, res.data_ptr() if res is not None else None)
        lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, W, pad)
        check()
        took = lib.nova_get_last_path(h)
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    return y, took


CASES = [  # (B, C, K, H, W, pad)
    (1, 64, 64, 56, 56, 1),   # ResNet-50 conv2_x, batch 1
    (2, 64, 64, 56, 56, 1),
    (1, 32, 32, 56, 56, 1),
    (1, 3, 64, 30, 30, 1),    # C = 3 (RGB stem-like)
    (3, 20, 48, 13, 17, 0),   # odd, non-square, pad 0
    (1, 64, 8, 9, 9, 2),      # K = 8, pad 2
    (4, 40, 24, 28, 28, 1),
    (1, 64, 64, 7, 7, 1),     # fewer tiles than a group (P = 4)
    (9, 24, 40, 30, 26, 0),   # 270 workgroups: the 512-thread variant, ragged K
    (1, 128, 128, 28, 28, 1), # ResNet-50 conv3_x, batch 1: four 32-channel chunks
    (2, 96, 72, 17, 23, 0),   # C, K between 64 and 128, off the 32-blocks
    (3, 65, 128, 14, 14, 2),  # one channel past a 64-block, pad 2
]


@pytest.mark.parametrize("B,C,K,H,W,pad", CASES)
def test_fused_small_matches_oracle_and_tile_block(oracle, B, C, K, H, W, pad):
    print(f"[fused small] B={B} C={C} K={K} H={H} W={W} pad={pad}", flush=True)
    g = torch.Generator().manual_seed(B * 7 + C + K)
    x = torch.randn(B, C, H, W, generator=g).half()
    w = torch.randn(K, C, 3, 3, generator=g) * (2.0 / (9 * C)) ** 0.5
    xd, wd = x.to(DEV), w.to(DEV)
    y, took = _run(xd, wd, pad, 5)
    assert took == 5
    yb, took_b = _run(xd, wd, pad, 3)
    if took_b == 3:
        assert torch.equal(y, yb), "differs from the fused tile-block kernel"
    yo = oracle.conv2d(x.numpy(), w.numpy(), pad)
    yg = y.cpu().numpy()
    assert np.isfinite(yg.astype(np.float32)).all()
    assert oracle.rel_l2(yg, yo) <= 5e-3
    assert oracle.max_abs(yg, yo) <= 0.25
    # repeatable
    y2, _ = _run(xd, wd, pad, 5)
    assert torch.equal(y, y2)


@pytest.mark.parametrize("B,C,K,H,pad", [(1, 64, 64, 56, 1), (2, 32, 48, 20, 1), (1, 16, 64, 13, 0),
                                         (7, 32, 48, 28, 1), (1, 128, 96, 28, 1)])
def test_fused_small_channels_last_and_epilogue(B, C, K, H, pad):
    """NHWC in and out equals the NCHW result in the other memory format, bit
    for bit; bias/residual/ReLU equal the separate fp16 ops."""
    print(f"[fused small nhwc] B={B} C={C} K={K} H={H} pad={pad}", flush=True)
    torch.manual_seed(41)
    x = torch.randn(B, C, H, H, device=DEV).half()
    w = torch.randn(K, C, 3, 3, device=DEV) * (2.0 / (9 * C)) ** 0.5
    y, _ = _run(x, w, pad, 5)
    yc, took = _run(x.contiguous(memory_format=CL), w, pad, 5, nhwc=True)
    assert took == 5 and yc.is_contiguous(memory_format=CL)
    assert torch.equal(yc, y)
    bias = (torch.randn(K, device=DEV) * 0.5).half()
    res = torch.randn_like(y)
    yb, _ = _run(x, w, pad, 5, bias=bias)
    ye, _ = _run(x, w, pad, 5, bias=bias, relu=1, res=res)
    assert torch.equal(yb, (y.float() + bias.float().view(1, -1, 1, 1)).half())
    assert torch.equal(ye, torch.relu(yb + res))
    yce, _ = _run(x.contiguous(memory_format=CL), w, pad, 5, nhwc=True, bias=bias, relu=1,
                  res=res.contiguous(memory_format=CL))
    assert torch.equal(yce, ye)


@pytest.mark.parametrize("C,K", [(160, 64), (64, 144)])
def test_fused_small_refused_above_128_channels(C, K):
    from nova_winograd.ops import check

    torch.manual_seed(42)
    x = torch.randn(1, C, 14, 14, device=DEV).half()
    w = torch.randn(K, C, 3, 3, device=DEV) * 0.05
    with pytest.raises(RuntimeError, match="fused path unsupported"):
        _run(x, w, 1, 5)
    check()
