"""Channels-last (NHWC) activations (nova_set_layout; no counterpart in the
reference): for every shape class -- lane-parallel transforms (small
problems), tile-block NHWC transforms (large ones), C not a multiple of 8 and
an x that is not 16-byte aligned (lane-parallel fallback), odd output widths,
pad 0 and 2 -- the NHWC forward must equal the NCHW forward of the same path
bit for bit, in the other memory format: three-pass against three-pass, and
the fused tile-block kernel (forced, and chosen automatically at conv2_x
B=32) against its NCHW form. Likewise with the bias/residual/ReLU epilogue,
through the module (channels_last in, channels_last out) and the functional
API. The NCHW paths are themselves parity-tested against the oracle.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
CL = torch.channels_last


def _run(x, w, pad, nhwc, bias=None, relu=0, res=None, path=0):
    from nova_winograd.ops import check, get_lib

    lib = get_lib()
    B, C, H, W = x.shape
    K = w.shape[0]
    Ho, Wo = H + 2 * pad - 2, W + 2 * pad - 2
    y = torch.empty(B, K, Ho, Wo, dtype=torch.float16, device=DEV,
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


CASES = [
    (1, 64, 64, 56, 1),     # lane-parallel both ways
    (8, 64, 64, 56, 1),     # tile-block NHWC kernels
    (32, 128, 128, 28, 1),
    (4, 256, 200, 14, 1),
    (12, 40, 24, 30, 1),
    (3, 20, 36, 17, 2),     # C % 8 != 0: lane-parallel input
    (16, 24, 16, 13, 0),    # odd output width, pad 0
]


@pytest.mark.parametrize("B,C,K,H,pad", CASES)
def test_nhwc_equals_nchw(B, C, K, H, pad):
    print(f"[nhwc] B={B} C={C} K={K} H={H} pad={pad}", flush=True)
    torch.manual_seed(12)
    x = torch.randn(B, C, H, H, device=DEV).half()
    w = (torch.randn(K, C, 3, 3, device=DEV) * (2.0 / (9 * C)) ** 0.5).float()
    y, took = _run(x.contiguous(memory_format=CL), w, pad, True)
    assert took in (1, 3, 5, 6)  # three-pass, fused tile-block, the small-problem kernel
    #                               for small grids, or two-pass (conv3_x at batch 32)
    y_ref, took_ref = _run(x, w, pad, False, path=took)  # the same path in NCHW
    assert took_ref == took
    assert y.is_contiguous(memory_format=CL)
    assert torch.equal(y, y_ref)
    # epilogue in NHWC: bias, residual (channels-last), ReLU
    bias = (torch.randn(K, device=DEV) * 0.5).half()
    res = torch.randn_like(y_ref).contiguous(memory_format=CL)
    y_e, _ = _run(x.contiguous(memory_format=CL), w, pad, True, bias=bias, relu=1, res=res)
    yb_ref, _ = _run(x, w, pad, False, bias=bias, path=took)
    assert torch.equal(y_e, torch.relu(yb_ref + res))


@pytest.mark.parametrize("B,C,K,H,pad", CASES + [(32, 64, 64, 56, 1), (2, 64, 64, 64, 1)])
def test_nhwc_fused_block_equals_nchw(B, C, K, H, pad):
    """Forced tile-block fused path: NHWC equals NCHW bit for bit (same
    transforms, same 16-channel MFMA steps), with and without the epilogue,
    at any channel count and image width (both layouts run the unstaged
    form up to 64 input channels)."""
    print(f"[nhwc fused] B={B} C={C} K={K} H={H} pad={pad}", flush=True)
    torch.manual_seed(16)
    x = torch.randn(B, C, H, H, device=DEV).half()
    w = (torch.randn(K, C, 3, 3, device=DEV) * (2.0 / (9 * C)) ** 0.5).float()
    xc = x.contiguous(memory_format=CL)
    y, took = _run(xc, w, pad, True, path=3)
    assert took == 3
    assert y.is_contiguous(memory_format=CL)
    y_ref, took_ref = _run(x, w, pad, False, path=3)
    assert took_ref == 3
    assert torch.equal(y, y_ref)
    assert torch.isfinite(y).all()
    bias = (torch.randn(K, device=DEV) * 0.5).half()
    res = torch.randn_like(y).contiguous(memory_format=CL)
    y_e, _ = _run(xc, w, pad, True, bias=bias, relu=1, res=res, path=3)
    yb, _ = _run(xc, w, pad, True, bias=bias, path=3)
    assert torch.equal(y_e, torch.relu(yb + res))
    ya, took_a = _run(xc, w, pad, True)
    if took_a == 3:
        assert torch.equal(ya, y)


@pytest.mark.parametrize("B,C,K,H,W,pad", [(6, 64, 48, 30, 44, 1), (5, 32, 64, 17, 58, 0),
                                             (3, 24, 40, 50, 14, 2)])
def test_nhwc_non_square(B, C, K, H, W, pad):
    """Non-square images, both paths: NHWC equals NCHW bit for bit."""
    print(f"[nhwc] non-square B={B} C={C} K={K} H={H} W={W} pad={pad}", flush=True)
    torch.manual_seed(17)
    x = torch.randn(B, C, H, W, device=DEV).half()
    w = (torch.randn(K, C, 3, 3, device=DEV) * (2.0 / (9 * C)) ** 0.5).float()
    xc = x.contiguous(memory_format=CL)
    for path in (1, 3):
        y_ref, took_ref = _run(x, w, pad, False, path=path)
        y, took = _run(xc, w, pad, True, path=path)
        assert took == took_ref, (path, took, took_ref)
        assert torch.equal(y, y_ref), path


def test_nhwc_unaligned_input():
    torch.manual_seed(13)
    B, C, K, H = 8, 64, 64, 56
    x = torch.randn(B, C, H, H, device=DEV).half()
    w = (torch.randn(K, C, 3, 3, device=DEV) * 0.06).float()
    y_ref, _ = _run(x, w, 1, False, path=1)
    n = x.numel()
    store = torch.empty(n + 8, dtype=torch.float16, device=DEV)
    x_cl = torch.as_strided(store, (B, C, H, H), (H * H * C, 1, H * C, C), storage_offset=1)
    x_cl.copy_(x)
    assert x_cl.is_contiguous(memory_format=CL) and x_cl.data_ptr() % 16 != 0
    y, _ = _run(x_cl, w, 1, True)
    assert torch.equal(y, y_ref)
    # the unstaged fused tile-block form loads x 2 bytes at a time: it takes
    # this x, and gives the NCHW form's bits
    y3, took3 = _run(x_cl, w, 1, True, path=3)
    assert took3 == 3
    y3_ref, _ = _run(x, w, 1, False, path=3)
    assert torch.equal(y3, y3_ref)


def test_module_and_functional_channels_last():
    from nova_winograd import NovaWinogradConv2d, nova_forward

    torch.manual_seed(14)
    conv = NovaWinogradConv2d(64, 48, kernel_size=3, padding=1, bias=True).to(DEV)
    with torch.no_grad():
        conv.bias.copy_(torch.randn(48))
    x = torch.randn(4, 64, 28, 28, device=DEV).half()
    xc = x.contiguous(memory_format=CL)
    with torch.no_grad():
        y = conv(x)
        yc = conv(xc)
        y2 = conv(x)  # back to NCHW: the layout is reset
        y3 = conv(x)  # cached path
        yf = nova_forward(xc, conv.weight, padding=1, bias=conv.bias)
    torch.cuda.synchronize()
    assert yc.is_contiguous(memory_format=CL) and not yc.is_contiguous()
    assert torch.equal(yc, y)
    assert torch.equal(y2, y) and torch.equal(y3, y)
    assert yf.is_contiguous(memory_format=CL) and torch.equal(yf, y)


def _tiles(n):
    return (n + 5) // 6


@pytest.mark.parametrize("B,C,K,H,W,pad", [
    (1, 64, 64, 56, 56, 1),    # lane-parallel NHWC transforms
    (8, 64, 64, 56, 56, 1),    # tile-block NHWC transforms
    (4, 256, 200, 14, 14, 1),
    (3, 24, 40, 50, 14, 2),    # non-square, pad 2
    (16, 24, 16, 13, 13, 0),   # odd output width, pad 0
    (3, 20, 36, 17, 17, 2),    # C % 8 != 0: lane-parallel NHWC input
])
def test_nhwc_transforms_against_oracle(oracle, B, C, K, H, W, pad):
    """The channels-last transform kernels against the oracle directly (not
    only against the NCHW kernels): V from the NHWC input transform equals
    the oracle's input transform bit for bit; y from the NHWC output
    transform equals the oracle's output transform of the GPU's own M bit
    for bit; the whole forward is within the forward parity bar."""
    import numpy as np

    from nova_winograd.ops import check, get_lib

    print(f"[nhwc oracle] B={B} C={C} K={K} H={H} W={W} pad={pad}", flush=True)
    lib = get_lib()
    torch.manual_seed(18)
    x = torch.randn(B, C, H, W).half()
    w = torch.randn(K, C, 3, 3) * (2.0 / (9 * C)) ** 0.5
    Ho, Wo = H + 2 * pad - 2, W + 2 * pad - 2
    nh, nw = _tiles(Ho), _tiles(Wo)
    BP, Cp = B * nh * nw, (C + 7) // 8 * 8
    nh_ref, nw_ref, _, _ = oracle.tiling(H, W, pad)
    nh_user = nh_ref
    while C * nh_user * nw_ref < Cp * nh * nw:  # caller V large enough for the internal pitch
        nh_user += 1
    V = torch.zeros(64 * C * B * nh_user * nw_ref, dtype=torch.float16, device=DEV)
    M = torch.zeros(64 * K * B * nh_user * nw_ref, dtype=torch.float16, device=DEV)
    xc = x.to(DEV).contiguous(memory_format=CL)
    y = torch.empty(B, K, Ho, Wo, dtype=torch.float16, device=DEV, memory_format=CL)
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, 1)
        lib.nova_set_layout(h, 1)
        lib.nova_set_weights(h, w.to(DEV).data_ptr(), K, C)
        lib.nova_forward_workspace(h, xc.data_ptr(), y.data_ptr(), V.data_ptr(), M.data_ptr(),
                                   B, H, W, pad, nh_user, nw_ref)
        check()
        assert lib.nova_get_last_path(h) == 1
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    Vg = V[:64 * BP * Cp].view(64, BP, Cp)[:, :, :C].cpu().numpy()
    Vo = oracle.input_transform(x.numpy(), pad, nh, nw)
    assert np.array_equal(Vg.view(np.uint16), Vo.view(np.uint16))
    Mg = M[:64 * BP * K].view(64, BP, K).cpu().numpy()
    yo = oracle.output_transform(Mg, B, Ho, Wo, nh, nw)
    yg = y.cpu().contiguous().numpy()
    assert np.array_equal(yg.view(np.uint16), yo.view(np.uint16))
    yr = oracle.conv2d(x.numpy(), w.numpy(), pad)
    assert oracle.rel_l2(yg, yr) <= 5e-3


@pytest.mark.parametrize("B,C,K,H", [(32, 64, 64, 56), (4, 48, 64, 30), (2, 64, 64, 64)])
def test_nhwc_fused_block_against_oracle(oracle, B, C, K, H):
    """The channels-last fused tile-block kernel against the oracle: the
    whole forward (first two images) within the forward parity bar, plus its
    bias/residual/ReLU epilogue against the oracle's output and the same
    separate fp16 ops."""
    import numpy as np

    print(f"[nhwc fused oracle] B={B} C={C} K={K} H={H}", flush=True)
    torch.manual_seed(19)
    x = torch.randn(B, C, H, H).half()
    w = torch.randn(K, C, 3, 3) * (2.0 / (9 * C)) ** 0.5
    xc = x.to(DEV).contiguous(memory_format=CL)
    wd = w.to(DEV)
    y, took = _run(xc, wd, 1, True, path=3)
    assert took == 3
    n = min(B, 2)
    yo = oracle.conv2d(x[:n].numpy(), w.numpy(), 1)
    yg = y[:n].cpu().contiguous().numpy()
    assert oracle.rel_l2(yg, yo) <= 5e-3
    assert oracle.max_abs(yg, yo) <= 0.25
    bias = (torch.randn(K) * 0.5).half()
    res = torch.randn(B, K, H, H).half()
    y_e, _ = _run(xc, wd, 1, True, bias=bias.to(DEV), relu=1,
                  res=res.to(DEV).contiguous(memory_format=CL), path=3)
    ref = torch.relu((torch.from_numpy(yo).float() + bias.float().view(1, -1, 1, 1)).half()
                     .float() + res[:n].float()).half()
    assert oracle.rel_l2(y_e[:n].cpu().contiguous().numpy(), ref.numpy()) <= 5e-3
