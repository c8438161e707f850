"""Two-pass path (nova_set_path(h, 6)): the three-pass input transform, then
the 64 Winograd-domain products and the output transform in one launch
(gemm_out_kernel: 16 tiles x 32 output channels per workgroup, or 16 output
channels and two workgroups per CU where the grid has at most one such
workgroup per CU; M kept in LDS; V written by the input transform in 1 KB
operand blocks of 16 tiles x 32 channels, U copied into the same block
order). The products use the three-pass GEMM's lane layout
and channel order and the output transform its chains, so y must equal
path 1 bit for bit -- for K and C off the 16/32 blocks, tile blocks that cross image
boundaries, pads 0-2, channels-last, the bias/residual/ReLU epilogue and
caller workspaces; and it must match the oracle within the forward bar.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
CL = torch.channels_last


def _run(x, w, pad, path, nhwc=False, bias=None, relu=0, res=None, workspace=False):
    from nova_winograd.ops import check, compute_tiling, get_lib

    lib = get_lib()
    B, C, H, W = x.shape
    K = w.shape[0]
    nh, nw, Ho, Wo = compute_tiling(H, W, pad)
    y = torch.full((B, K, Ho, Wo), float("nan"), dtype=torch.float16, device=DEV)
    if nhwc:
        y = y.contiguous(memory_format=CL)
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, path)
        lib.nova_set_layout(h, 1 if nhwc else 0)
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        lib.nova_set_epilogue(h, bias.data_ptr() if bias is not None else None, relu)
        lib.nova_set_residual(h, res.data_ptr() if res is not None else None)
        check()
        if workspace:
            V = torch.empty(64 * C * B * nh * nw, dtype=torch.float16, device=DEV)
            M = torch.empty(64 * K * B * nh * nw, dtype=torch.float16, device=DEV)
            lib.nova_forward_workspace(h, x.data_ptr(), y.data_ptr(), V.data_ptr(), M.data_ptr(),
                                       B, H, W, pad, nh, nw)
        else:
            lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, W, pad)
        check()
        took = lib.nova_get_last_path(h)
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    return y, took


CASES = [  # (B, C, K, H, W, pad)
    (32, 128, 128, 28, 28, 1),  # ResNet-50 conv3_x, batch 32
    (3, 128, 128, 28, 28, 1),   # 75 tiles: the last tile block is partial and crosses images
    (2, 96, 72, 17, 23, 0),     # K off the 32-blocks, odd non-square image, pad 0
    (5, 40, 8, 13, 13, 2),      # K < 16, pad 2
    (1, 3, 48, 30, 30, 1),      # C = 3 (one 8-channel group)
    (4, 256, 40, 14, 14, 1),    # eight channel steps
    (7, 64, 100, 9, 11, 1),     # tiles of several images per block, K = 100
    (32, 128, 256, 14, 14, 1),  # K = 256 (automatic above 128 output channels from 192 workgroups)
    (6, 64, 200, 28, 28, 1),    # K = 200: a partial last 16-channel output block
    (16, 64, 200, 28, 28, 1),   # 32 channels per workgroup, partial last 32-channel block
]
# every case above but the first, the 128 -> 256 one and the last runs 16
# output channels per workgroup on a 256-CU chip (grid at 16 channels <= CUs)


@pytest.mark.parametrize("B,C,K,H,W,pad", CASES)
def test_two_pass_equals_three_pass(oracle, B, C, K, H, W, pad):
    print(f"[two-pass] B={B} C={C} K={K} H={H} W={W} pad={pad}", flush=True)
    g = torch.Generator().manual_seed(B * 13 + C + K)
    x = torch.randn(B, C, H, W, generator=g).half()
    w = torch.randn(K, C, 3, 3, generator=g) * (2.0 / (9 * C)) ** 0.5
    xd, wd = x.to(DEV), w.to(DEV)
    y6, took6 = _run(xd, wd, pad, 6)
    y1, took1 = _run(xd, wd, pad, 1)
    assert took6 == 6 and took1 == 1
    assert torch.equal(y6, y1), "differs from the three-pass path"
    y6w, _ = _run(xd, wd, pad, 6, workspace=True)
    assert torch.equal(y6w, y1)
    n = min(B, 3)
    yo = oracle.conv2d(x[:n].numpy(), w.numpy(), pad)
    yg = y6[:n].cpu().numpy()
    assert oracle.rel_l2(yg, yo) <= 5e-3
    assert oracle.max_abs(yg, yo) <= 0.25


@pytest.mark.parametrize("B,C,K,H,pad", [(4, 128, 128, 28, 1), (3, 64, 40, 13, 0),
                                         (32, 128, 128, 28, 1)])
def test_two_pass_channels_last_and_epilogue(B, C, K, H, pad):
    print(f"[two-pass nhwc] B={B} C={C} K={K} H={H} pad={pad}", flush=True)
    torch.manual_seed(43)
    x = torch.randn(B, C, H, H, device=DEV).half()
    w = torch.randn(K, C, 3, 3, device=DEV) * (2.0 / (9 * C)) ** 0.5
    bias = (torch.randn(K, device=DEV) * 0.5).half()
    y1, _ = _run(x, w, pad, 1)
    res = torch.randn_like(y1)
    ye1, _ = _run(x, w, pad, 1, bias=bias, relu=1, res=res)
    ye6, took = _run(x, w, pad, 6, bias=bias, relu=1, res=res)
    assert took == 6 and torch.equal(ye6, ye1)
    yb6, _ = _run(x, w, pad, 6, bias=bias, relu=1)
    yb1, _ = _run(x, w, pad, 1, bias=bias, relu=1)
    assert torch.equal(yb6, yb1)
    xc = x.contiguous(memory_format=CL)
    yc6, took = _run(xc, w, pad, 6, nhwc=True)
    assert took == 6 and yc6.is_contiguous(memory_format=CL)
    assert torch.equal(yc6, y1)
    yce6, _ = _run(xc, w, pad, 6, nhwc=True, bias=bias, relu=1,
                   res=res.contiguous(memory_format=CL))
    assert torch.equal(yce6, ye1)


def test_two_pass_workspace_query():
    """nova_workspace_bytes for a forced two-pass forward counts V only, in
    its block layout (16-tile blocks x 32-channel chunks)."""
    from nova_winograd.ops import check, get_lib

    lib = get_lib()
    C, K, B, H = 128, 96, 6, 28
    w = torch.randn(K, C, 3, 3, device=DEV) * 0.05
    h = lib.nova_create()
    try:
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        lib.nova_set_path(h, 1)
        three = lib.nova_workspace_bytes(h, B, H, H, 1)
        lib.nova_set_path(h, 6)
        two = lib.nova_workspace_bytes(h, B, H, H, 1)
        check()
    finally:
        lib.nova_destroy(h)
    P = 25
    assert three == 2 * 64 * (C + K) * B * P
    assert two == 2 * 64 * (-(-B * P // 16) * 16) * (-(-C // 32) * 32)
