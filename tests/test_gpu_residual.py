"""Residual in the fused epilogue (nova_set_residual; no counterpart in the
reference): y = relu(fp16(conv) + bias + residual) with every add rounded to
fp16 must equal the separate fp16 ops `y + bias.half()`, `+ residual`,
`relu`, bit for bit, on every pipeline and both output-transform forms, with
the residual aligned like y or only to 2 bytes, through the C-ABI, the module
and the functional API; a following call without a residual must not add it.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _run(path, x, w, pad, bias=None, relu=0, res=None):
    from nova_winograd.ops import check, get_lib

    lib = get_lib()
    B, C, H, W = x.shape
    K = w.shape[0]
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, path)
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        lib.nova_set_epilogue(h, bias.data_ptr() if bias is not None else None, relu)
        lib.nova_set_residual(h, res.data_ptr() if res is not None else None)
        y = torch.empty(B, K, H + 2 * pad - 2, W + 2 * pad - 2, dtype=torch.float16, device=DEV)
        lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, W, pad)
        check()
        took = lib.nova_get_last_path(h)
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    return y, took


# batch 1 / small: lane-parallel output transform; (8,64,64,56) and
# (32,64,64,24): tile-block (the latter with 8-byte row segments);
# (32,128,256,14) and (32,64,512,7): the image-block form (three-pass) with a
# 16-byte aligned residual, the tile-block form with the offset one
CASES = [(1, 64, 64, 56, 1), (8, 64, 64, 56, 1), (32, 64, 64, 24, 1), (2, 48, 40, 13, 1),
         (3, 20, 36, 17, 2), (32, 128, 256, 14, 1), (32, 64, 512, 7, 1)]


@pytest.mark.parametrize("aligned", [True, False], ids=["aligned", "offset2"])
@pytest.mark.parametrize("path", [1, 2, 3], ids=["3pass", "fused_rows", "fused_block"])
@pytest.mark.parametrize("B,C,K,H,pad", CASES)
def test_residual_matches_separate_ops(B, C, K, H, pad, path, aligned):
    print(f"[residual] B={B} C={C} K={K} H={H} pad={pad} path={path} aligned={aligned}",
          flush=True)
    torch.manual_seed(9)
    x = torch.randn(B, C, H, H, device=DEV).half()
    w = (torch.randn(K, C, 3, 3, device=DEV) * (2.0 / (9 * C)) ** 0.5).float()
    bias = (torch.randn(K, device=DEV) * 0.5).half()
    Ho = H + 2 * pad - 2
    n = B * K * Ho * Ho
    store = torch.randn(n + 1, device=DEV).half()
    res = (store[:n] if aligned else store[1:]).view(B, K, Ho, Ho)
    y0, took = _run(path, x, w, pad)
    if path in (2, 3) and took != path:
        pytest.skip("shape outside the forced fused path's envelope")
    yb, _ = _run(path, x, w, pad, bias=bias)
    y1, _ = _run(path, x, w, pad, bias=bias, res=res)
    y2, _ = _run(path, x, w, pad, bias=bias, relu=1, res=res)
    y3, _ = _run(path, x, w, pad, res=res)
    assert torch.equal(y1, yb + res)
    assert torch.equal(y2, torch.relu(yb + res))
    assert torch.equal(y3, y0 + res)


def test_module_and_functional_residual():
    from nova_winograd import NovaWinogradConv2d, nova_forward

    torch.manual_seed(10)
    conv = NovaWinogradConv2d(32, 32, kernel_size=3, padding=1, bias=True).to(DEV)
    with torch.no_grad():
        conv.bias.copy_(torch.randn(32))
    x = torch.randn(2, 32, 20, 20, device=DEV).half()
    r = torch.randn(2, 32, 20, 20, device=DEV).half()
    with torch.no_grad():
        y = conv(x)
        yr = conv(x, residual=r)
        y_again = conv(x)  # the residual is not kept
        y_again2 = conv(x)  # cached path
        yf = nova_forward(x, conv.weight, padding=1, bias=conv.bias, relu=True, residual=r)
    torch.cuda.synchronize()
    assert torch.equal(yr, y + r)
    assert torch.equal(y_again, y)
    assert torch.equal(y_again2, y)
    assert torch.equal(yf, torch.relu(y + r))
    with pytest.raises(ValueError):
        conv(x, residual=r[:1])
