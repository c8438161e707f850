"""fp16 weights at the boundary (no counterpart in the reference): the
library's nova_set_weights_f16 and the Python paths that use it (a module
converted with .half(), nova_forward with an fp16 weight) must give exactly
the result of the fp32 copy of the same weights, bit for bit, on every path.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _run(lib, path, x, w, f16):
    from nova_winograd.ops import check

    B, C, H, W = x.shape
    K = w.shape[0]
    y = torch.empty(B, K, H, W, dtype=torch.float16, device=DEV)
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, path)
        if f16:
            lib.nova_set_weights_f16(h, w.half().contiguous().data_ptr(), K, C)
        else:
            lib.nova_set_weights(h, w.half().float().contiguous().data_ptr(), K, C)
        lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, W, 1)
        check()
        assert lib.nova_get_last_path(h) == path
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    return y


@pytest.mark.parametrize("path", [1, 2, 3], ids=["3pass", "fused_rows", "fused_block"])
@pytest.mark.parametrize("B,C,K,H", [(2, 64, 64, 20), (1, 40, 24, 13)])
def test_f16_weights_equal_fp32_copy(B, C, K, H, path):
    from nova_winograd.ops import get_lib

    print(f"[w16] B={B} C={C} K={K} H={H} path={path}", flush=True)
    torch.manual_seed(5)
    x = torch.randn(B, C, H, H, device=DEV).half()
    w = torch.randn(K, C, 3, 3, device=DEV) * 0.1
    lib = get_lib()
    assert torch.equal(_run(lib, path, x, w, True), _run(lib, path, x, w, False))


def test_half_module_and_functional():
    from nova_winograd import NovaWinogradConv2d, nova_forward

    torch.manual_seed(6)
    conv = NovaWinogradConv2d(32, 48, kernel_size=3, padding=1).to(DEV)
    x = torch.randn(2, 32, 18, 18, device=DEV).half()
    with torch.no_grad():
        w16 = conv.weight.detach().half()
        conv.weight.copy_(w16.float())
        y32 = conv(x)
        conv.half()  # the weight is now fp16: transformed without an fp32 copy
        assert conv.weight.dtype == torch.float16
        y16 = conv(x)
        yf = nova_forward(x, w16, padding=1)
    torch.cuda.synchronize()
    assert torch.equal(y16, y32)
    assert torch.equal(yf, y32)
