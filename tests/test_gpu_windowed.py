"""Windowed three-pass path (nova_set_path(h, 4); the reference's BP-windowed
pipeline, /root/reference/tests/test_bp_tiled.hip:482-571, run in windows of
whole images): the batch runs as consecutive windows whose V + M fit the
window budget (nova_set_window_bytes), each window's input transform, GEMM
and output transform back to back. Every image's arithmetic is the
three-pass path's, so the result must equal path 1 bit for bit -- for
windows of one image, a few images and the whole batch, with the
bias/residual/ReLU epilogue, in NHWC and with caller workspaces. The number
of windows is checked through the per-kernel profiler (one GEMM launch per
window)."""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
CL = torch.channels_last


def _run(x, w, pad, path, window=0, nhwc=False, bias=None, relu=0, res=None,
         workspace=False, count_gemms=False):
    from nova_winograd.ops import check, compute_tiling, get_lib

    lib = get_lib()
    B, C, H, W = x.shape
    K = w.shape[0]
    nh, nw, Ho, Wo = compute_tiling(H, W, pad)
    y = torch.empty(B, K, Ho, Wo, dtype=torch.float16, device=DEV,
                    memory_format=CL if nhwc else torch.contiguous_format)
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, path)
        lib.nova_set_window_bytes(h, window)
        lib.nova_set_layout(h, 1 if nhwc else 0)
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        lib.nova_set_epilogue(h, bias.data_ptr() if bias is not None else None, relu)
        lib.nova_set_residual(h, res.data_ptr() if res is not None else None)
        check()
        if count_gemms:
            lib.nova_profile_enable(h, 1)
        if workspace:
            V = torch.empty(64 * C * B * nh * nw, dtype=torch.float16, device=DEV)
            M = torch.empty(64 * K * B * nh * nw, dtype=torch.float16, device=DEV)
            lib.nova_forward_workspace(h, x.data_ptr(), y.data_ptr(), V.data_ptr(), M.data_ptr(),
                                       B, H, W, pad, nh, nw)
        else:
            lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, W, pad)
        check()
        took = lib.nova_get_last_path(h)
        gemms = None
        if count_gemms:
            tot = (ctypes.c_double * 4)()
            cnt = (ctypes.c_longlong * 4)()
            lib.nova_profile_read(h, tot, cnt)
            gemms = cnt[1]
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    return y, took, gemms


def _per_image_bytes(C, K, H, pad):
    Cp = (C + 7) // 8 * 8
    P = (-(-(H + 2 * pad - 2) // 6)) ** 2
    return 2 * 64 * (Cp + K) * P


# (B, C, K, H, pad)
CASES = [(32, 128, 128, 28, 1), (12, 64, 64, 56, 1), (7, 256, 200, 14, 1),
         (9, 40, 24, 30, 0), (5, 20, 36, 17, 2)]


@pytest.mark.parametrize("B,C,K,H,pad", CASES)
def test_windowed_equals_three_pass(B, C, K, H, pad):
    print(f"[windowed] B={B} C={C} K={K} H={H} pad={pad}", flush=True)
    torch.manual_seed(31)
    x = torch.randn(B, C, H, H, device=DEV).half()
    w = (torch.randn(K, C, 3, 3, device=DEV) * (2.0 / (9 * C)) ** 0.5).float()
    y1, took1, _ = _run(x, w, pad, 1)
    assert took1 == 1
    per = _per_image_bytes(C, K, H, pad)
    for imgs in (1, 3, B):
        y4, took4, gemms = _run(x, w, pad, 4, window=imgs * per, count_gemms=True)
        assert took4 == 4
        assert gemms == -(-B // imgs), (imgs, gemms)
        assert torch.equal(y4, y1), imgs
    # the default budget (4 MiB, at least one image per window)
    y4, _, gemms = _run(x, w, pad, 4, count_gemms=True)
    assert gemms == -(-B // max(1, (4 << 20) // per))
    assert torch.equal(y4, y1)
    # caller workspaces sized for the whole batch
    y4, _, _ = _run(x, w, pad, 4, window=2 * per, workspace=True)
    assert torch.equal(y4, y1)


def test_windowed_epilogue_and_nhwc():
    torch.manual_seed(32)
    B, C, K, H = 6, 64, 48, 28
    x = torch.randn(B, C, H, H, device=DEV).half()
    w = (torch.randn(K, C, 3, 3, device=DEV) * 0.06).float()
    bias = (torch.randn(K, device=DEV) * 0.5).half()
    per = _per_image_bytes(C, K, H, 1)
    res = torch.randn(B, K, H, H, device=DEV).half()
    y1, _, _ = _run(x, w, 1, 1, bias=bias, relu=1, res=res)
    y4, took, _ = _run(x, w, 1, 4, window=2 * per, bias=bias, relu=1, res=res)
    assert took == 4 and torch.equal(y4, y1)
    xc = x.contiguous(memory_format=CL)
    rc = res.contiguous(memory_format=CL)
    y4n, took, _ = _run(xc, w, 1, 4, window=per, nhwc=True, bias=bias, relu=1, res=rc)
    assert took == 4 and torch.equal(y4n, y1)


def test_window_bytes_validation():
    from nova_winograd.ops import get_lib

    lib = get_lib()
    h = lib.nova_create()
    try:
        lib.nova_set_window_bytes(h, -1)
        assert lib.nova_get_last_error() != 0
        lib.nova_set_path(h, 8)  # paths are 0..7
        assert lib.nova_get_last_error() != 0
        lib.nova_set_path(h, 4)
        assert lib.nova_get_last_error() == 0
    finally:
        lib.nova_destroy(h)
