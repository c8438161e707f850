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


@pytest.mark.parametrize("K,C", [(64, 64), (48, 40), (200, 96)])
def test_f16_filter_transform_against_oracle(oracle, K, C):
    """nova_set_weights_f16's filter transform against the oracle's on the
    widened weights, bit for bit (U in the library layout [64][K][pad8(C)]),
    and the whole forward with fp16 weights within the forward parity bar."""
    import numpy as np

    from nova_winograd.ops import check, get_lib

    print(f"[w16 oracle] K={K} C={C}", flush=True)
    lib = get_lib()
    torch.manual_seed(7)
    w16 = (torch.randn(K, C, 3, 3) * 0.2).half()
    x = torch.randn(2, C, 19, 19).half()
    wd = w16.to(DEV).contiguous()
    y = torch.empty(2, K, 19, 19, dtype=torch.float16, device=DEV)
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, 1)
        lib.nova_set_weights_f16(h, wd.data_ptr(), K, C)
        check()
        Cp = (C + 7) // 8 * 8
        torch.cuda.synchronize()
        # copy the handle's U out through the HIP runtime torch already loaded
        # (soname libamdhip64.so.7; hipMemcpyDeviceToHost = 2)
        import ctypes

        hip = ctypes.CDLL("libamdhip64.so.7")
        U_host = torch.empty(64 * K * Cp, dtype=torch.float16)
        rc = hip.hipMemcpy(ctypes.c_void_p(U_host.data_ptr()),
                           ctypes.c_void_p(lib.nova_get_U_gemm(h)),
                           ctypes.c_size_t(U_host.numel() * 2), ctypes.c_int(2))
        assert rc == 0
        lib.nova_forward(h, x.to(DEV).data_ptr(), y.data_ptr(), 2, 19, 19, 1)
        check()
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    Uo = oracle.filter_transform(w16.float().numpy())  # [64][C][K]
    Ug = U_host.view(64, K, Cp)[:, :, :C].numpy()
    Uo_lib = np.ascontiguousarray(Uo.transpose(0, 2, 1))  # -> [64][K][C]
    assert np.array_equal(np.ascontiguousarray(Ug).view(np.uint16), Uo_lib.view(np.uint16))
    assert not U_host.view(64, K, Cp)[:, :, C:].any()  # channel padding is zero
    yo = oracle.conv2d(x.numpy(), w16.float().numpy(), 1)
    assert oracle.rel_l2(y.cpu().numpy(), yo) <= 5e-3
