"""Input transform fused into the products (path 7, in_gemm_kernel): each
workgroup builds row r of V for its tile group from x in LDS and multiplies
it with the block GEMM's operand lanes and step order, then the three-pass
output transform runs. y must equal path 1 bit for bit -- batch-1 ResNet-50
deep layers, DenseNet-like K off the 16-blocks, C off the 32-steps, pads 0-2,
odd and non-square images, tile groups that cross images, channels-last, the
epilogue, x at odd offsets, caller workspaces -- and match the oracle within
the forward bar. The automatic choice takes it for GEMV-like shapes above 64
channels (the dispatch cases below).
"""

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
    (1, 128, 128, 28, 28, 1),   # ResNet-50 conv3_x, batch 1 (25 tiles)
    (1, 256, 256, 14, 14, 1),   # conv4_x (9 tiles)
    (1, 512, 512, 7, 7, 1),     # conv5_x (4 tiles, 16 channel steps)
    (1, 192, 48, 28, 28, 1),    # DenseNet-161 bottleneck, K = 48
    (1, 192, 48, 7, 7, 1),
    (2, 136, 40, 13, 17, 0),    # C off the 32-steps, K < 16 x 3, pad 0, non-square
    (3, 72, 100, 11, 9, 2),     # pad 2, K = 100, tile groups across images
    (1, 3, 24, 20, 20, 1),      # C = 3
    (4, 320, 96, 8, 8, 1),      # 16 tiles over four images
    (1, 480, 20, 30, 10, 1),    # 15 steps, K = 20, wide tiles
]


@pytest.mark.parametrize("B,C,K,H,W,pad", CASES)
def test_in_gemm_equals_three_pass(oracle, B, C, K, H, W, pad):
    print(f"[in-gemm] B={B} C={C} K={K} H={H} W={W} pad={pad}", flush=True)
    g = torch.Generator().manual_seed(B * 31 + C + 7 * K + H)
    x = torch.randn(B, C, H, W, generator=g).half()
    w = torch.randn(K, C, 3, 3, generator=g) * (2.0 / (9 * C)) ** 0.5
    xd, wd = x.to(DEV), w.to(DEV)
    y7, took7 = _run(xd, wd, pad, 7)
    y1, took1 = _run(xd, wd, pad, 1)
    assert took7 == 7 and took1 == 1
    assert torch.isfinite(y7.float()).all()
    assert torch.equal(y7, y1), "differs from the three-pass path"
    y7w, _ = _run(xd, wd, pad, 7, workspace=True)
    assert torch.equal(y7w, y1)
    yo = oracle.conv2d(x.numpy(), w.numpy(), pad)
    yg = y7.cpu().numpy()
    assert oracle.rel_l2(yg, yo) <= 5e-3
    assert oracle.max_abs(yg, yo) <= 0.25


@pytest.mark.parametrize("B,C,K,H,pad", [(1, 256, 256, 14, 1), (2, 96, 64, 13, 0)])
def test_in_gemm_channels_last_and_epilogue(B, C, K, H, pad):
    print(f"[in-gemm nhwc] B={B} C={C} K={K} H={H} pad={pad}", flush=True)
    torch.manual_seed(47)
    x = torch.randn(B, C, H, H, device=DEV).half()
    w = torch.randn(K, C, 3, 3, device=DEV) * (2.0 / (9 * C)) ** 0.5
    bias = (torch.randn(K, device=DEV) * 0.5).half()
    y1, _ = _run(x, w, pad, 1)
    res = torch.randn_like(y1)
    ye1, _ = _run(x, w, pad, 1, bias=bias, relu=1, res=res)
    ye7, took = _run(x, w, pad, 7, bias=bias, relu=1, res=res)
    assert took == 7 and torch.equal(ye7, ye1)
    xc = x.contiguous(memory_format=CL)
    yc7, took = _run(xc, w, pad, 7, nhwc=True)
    assert took == 7 and yc7.is_contiguous(memory_format=CL)
    assert torch.equal(yc7, y1)
    yce7, _ = _run(xc, w, pad, 7, nhwc=True, bias=bias, relu=1,
                   res=res.contiguous(memory_format=CL))
    assert torch.equal(yce7, ye1)


@pytest.mark.parametrize("shift", [1, 2, 3, 7])
def test_in_gemm_input_offsets(shift):
    """x at 2-byte offsets from a 16-byte boundary, NaN around it: the row
    loads read from the dword at or below each row start and mask the
    columns outside the image, so nothing outside x enters V."""
    print(f"[in-gemm offset] shift={shift}", flush=True)
    torch.manual_seed(5 + shift)
    B, C, K, H, pad = 1, 128, 64, 11, 1
    n = B * C * H * H
    buf = torch.full((n + 64,), float("nan"), dtype=torch.float16, device=DEV)
    x = buf[shift:shift + n].view(B, C, H, H)
    x.copy_(torch.randn(B, C, H, H, device=DEV).half())
    w = torch.randn(K, C, 3, 3, device=DEV) * 0.04
    y7, took = _run(x, w, pad, 7)
    y1, _ = _run(x.clone(), w, pad, 1)
    assert took == 7 and torch.isfinite(y7.float()).all()
    assert torch.equal(y7, y1)


@pytest.mark.parametrize("B,C,K,H,want", [(1, 128, 128, 28, 7), (1, 192, 48, 28, 7),
                                          (1, 192, 48, 14, 7), (1, 192, 48, 7, 7),
                                          (1, 256, 256, 14, 1), (1, 512, 512, 7, 1),
                                          (2, 128, 128, 28, 1)])
def test_in_gemm_automatic_choice(B, C, K, H, want):
    """Batch-1 layers with at most 128 output channels and at most 32 tiles
    (ResNet-50 conv3_x, DenseNet-161 bottlenecks) take path 7 automatically;
    more output channels or tiles keep three-pass. y equals the forced
    three-pass path's either way."""
    torch.manual_seed(11)
    x = torch.randn(B, C, H, H, device=DEV).half()
    w = torch.randn(K, C, 3, 3, device=DEV) * (2.0 / (9 * C)) ** 0.5
    y0, took = _run(x, w, 1, 0)
    y1, _ = _run(x, w, 1, 1)
    assert took == want
    assert torch.equal(y0, y1)
