"""The fused output epilogue (nova_set_epilogue): bias and ReLU applied in
the output transform must equal the reference's separate ops
(`y + bias.half()`, /root/reference/nova_winograd/conv2d.py:240-241, then
ReLU) exactly, on every pipeline, through the C-ABI, the module and the
functional API."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _lib():
    from nova_winograd.ops import get_lib

    return get_lib()


def _check():
    from nova_winograd.ops import check

    check()


def _run(lib, path, x, w, pad, bias=None, relu=0):
    B, C, H, W = x.shape
    K = w.shape[0]
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, path)
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        lib.nova_set_epilogue(h, bias.data_ptr() if bias is not None else None, relu)
        _check()
        y = torch.empty(B, K, H + 2 * pad - 2, W + 2 * pad - 2, dtype=torch.float16, device=DEV)
        lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, W, pad)
        _check()
        took = lib.nova_get_last_path(h)
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    return y, took


CASES = [(1, 64, 64, 56, 1), (8, 64, 64, 56, 1), (2, 48, 40, 13, 1), (1, 256, 200, 14, 1),
         (3, 20, 36, 17, 2)]


@pytest.mark.parametrize("path", [1, 2, 3], ids=["3pass", "fused_rows", "fused_block"])
@pytest.mark.parametrize("B,C,K,H,pad", CASES)
def test_epilogue_matches_separate_ops(B, C, K, H, pad, path):
    print(f"[epilogue] B={B} C={C} K={K} H={H} pad={pad} path={path}", flush=True)
    lib = _lib()
    torch.manual_seed(5)
    x = torch.randn(B, C, H, H, device=DEV).half()
    w = (torch.randn(K, C, 3, 3, device=DEV) * (2.0 / (9 * C)) ** 0.5).float()
    bias = (torch.randn(K, device=DEV) * 0.5).half()
    y0, took0 = _run(lib, path, x, w, pad)
    y1, took1 = _run(lib, path, x, w, pad, bias=bias)
    y2, took2 = _run(lib, path, x, w, pad, bias=bias, relu=1)
    y3, took3 = _run(lib, path, x, w, pad, relu=1)
    assert took0 == took1 == took2 == took3
    ref1 = y0 + bias.view(1, -1, 1, 1)
    assert torch.equal(y1, ref1)
    assert torch.equal(y2, torch.relu(ref1))
    assert torch.equal(y3, torch.relu(y0))


def test_module_bias_fused_and_exact():
    from nova_winograd import NovaWinogradConv2d

    torch.manual_seed(6)
    conv = NovaWinogradConv2d(32, 48, kernel_size=3, padding=1, bias=True).to(DEV)
    with torch.no_grad():
        conv.bias.copy_(torch.randn(48))
    x = torch.randn(2, 32, 20, 20, device=DEV).half()
    with torch.no_grad():
        y = conv(x)
        b = conv.bias.detach().clone()
        conv.bias = None
        y_nobias = conv(x)
        conv.bias = torch.nn.Parameter(b.clone())
        y_again = conv(x)
        # a changed bias is picked up (versioned cache)
        conv.bias.add_(1.0)
        y_changed = conv(x)
    torch.cuda.synchronize()
    ref = y_nobias + b.half().view(1, -1, 1, 1)
    assert torch.equal(y, ref)
    assert torch.equal(y_again, ref)
    assert torch.equal(y_changed, y_nobias + (b + 1.0).half().view(1, -1, 1, 1))


def test_functional_bias_relu():
    from nova_winograd import nova_forward

    torch.manual_seed(7)
    x = torch.randn(1, 16, 12, 12, device=DEV).half()
    w = (torch.randn(24, 16, 3, 3, device=DEV) * 0.1).float()
    b = torch.randn(24, device=DEV)
    y = nova_forward(x, w, 1)
    yb = nova_forward(x, w, 1, bias=b, relu=True)
    torch.cuda.synchronize()
    assert torch.equal(yb, torch.relu(y + b.half().view(1, -1, 1, 1)))
    assert np.isfinite(yb.float().cpu().numpy()).all()
