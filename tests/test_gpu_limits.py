"""Limits of the forward (no counterpart in the reference, which mallocs one
workspace for the whole batch):

* an empty batch is a no-op that reports no error (module and C-ABI);
* a batch whose buffers pass the 32-bit byte-offset budget runs in
  sub-batches. Checked at C = K = 64, 512 x 512 images, batch 20: the
  workspace query covers one sub-batch, not the batch; every image of the
  batch equals a single-image forward bit for bit (both three-pass), across
  the sub-batch boundary; the same holds in NHWC and with a residual, whose
  pointers advance with the sub-batch;
* one image too large for the budget is refused with an error before any
  GPU work.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
CL = torch.channels_last


def test_empty_batch():
    from nova_winograd import NovaWinogradConv2d, nova_forward
    from nova_winograd.ops import check, get_lib

    conv = NovaWinogradConv2d(16, 24, padding=1).to(DEV)
    x = torch.empty(0, 16, 12, 12, device=DEV, dtype=torch.float16)
    with torch.no_grad():
        y = conv(x)
    assert y.shape == (0, 24, 12, 12)
    assert nova_forward(x, conv.weight, padding=1).shape == (0, 24, 12, 12)
    lib = get_lib()
    h = lib.nova_create()
    try:
        lib.nova_set_weights(h, conv.weight.data_ptr(), 24, 16)
        lib.nova_forward(h, 1, 2, 0, 12, 12, 1)  # nothing to read or write
        check()
    finally:
        lib.nova_destroy(h)
    torch.cuda.synchronize()


def _forward(lib, x, w, nhwc=False, res=None):
    from nova_winograd.ops import check

    B, C, H, W = x.shape
    K = w.shape[0]
    y = torch.empty(B, K, H, W, dtype=torch.float16, device=DEV,
                    memory_format=CL if nhwc else torch.contiguous_format)
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, 1)
        lib.nova_set_layout(h, 1 if nhwc else 0)
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        lib.nova_set_residual(h, res.data_ptr() if res is not None else None)
        ws = lib.nova_workspace_bytes(h, B, H, W, 1)
        lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, W, 1)
        check()
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    return y, ws


def test_sub_batches_match_single_images():
    from nova_winograd.ops import get_lib

    lib = get_lib()
    B, C, K, H = 20, 64, 64, 512
    print(f"[limits] sub-batches B={B} C={C} K={K} H={H}", flush=True)
    torch.manual_seed(41)
    x = torch.randn(B, C, H, H, device=DEV, dtype=torch.float16)
    w = (torch.randn(K, C, 3, 3, device=DEV) * 0.06).float()
    res = torch.randn(B, K, H, H, device=DEV, dtype=torch.float16)
    y, ws = _forward(lib, x, w, res=res)
    # per-image V + M at the minimal tiling; the workspace covers a sub-batch
    per_img = 2 * 64 * (C + K) * (-(-H // 6)) ** 2
    assert per_img < ws < B * per_img, (ws, per_img)
    chunk = ws // per_img
    for i in sorted({0, chunk - 1, chunk, B - 1}):
        yi, _ = _forward(lib, x[i:i + 1].contiguous(), w, res=res[i:i + 1].contiguous())
        assert torch.equal(yi[0], y[i]), i
    # channels-last: same values, other layout, across the same boundary
    yc, _ = _forward(lib, x.contiguous(memory_format=CL), w, nhwc=True,
                     res=res.contiguous(memory_format=CL))
    assert torch.equal(yc, y)
    del x, y, yc, res
    torch.cuda.empty_cache()


def test_image_over_budget_is_refused():
    from nova_winograd.ops import get_lib

    lib = get_lib()
    C = K = 512
    w = torch.zeros(K, C, 3, 3, device=DEV)
    h = lib.nova_create()
    try:
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        assert lib.nova_get_last_error() == 0
        # V of one 1024 x 1024 image: 2 * 64 * 512 * 171^2 bytes = 1.9 GB
        lib.nova_forward(h, 1, 2, 1, 1024, 1024, 1)
        assert lib.nova_get_last_error() == 1
        assert b"exceeds" in lib.nova_get_last_error_message()
    finally:
        lib.nova_destroy(h)
    torch.cuda.synchronize()


def test_fused_operands_built_only_when_a_fused_path_can_run():
    """The fragment-ordered copy of U that the fused kernels read is built
    only for handles that can run them: a 1280 x 1280 layer on the automatic
    path holds U alone (210 MB); forcing a fused path after the weights builds
    the copy (another 210 MB). A small layer forced onto the fused kernel
    after its weights matches the three-pass result."""
    from nova_winograd.ops import check, get_lib

    lib = get_lib()
    K = C = 1280
    u_bytes = 64 * K * C * 2
    w = torch.zeros(K, C, 3, 3, device=DEV)
    torch.cuda.synchronize()
    h = lib.nova_create()
    try:
        free0 = torch.cuda.mem_get_info()[0]
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        check()
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
        assert u_bytes <= free0 - free1 < 1.5 * u_bytes, (free0 - free1)
        lib.nova_set_path(h, 3)
        check()
        torch.cuda.synchronize()
        free2 = torch.cuda.mem_get_info()[0]
        assert 0.9 * u_bytes <= free1 - free2 < 1.5 * u_bytes, (free1 - free2)
    finally:
        lib.nova_destroy(h)
    del w
    torch.cuda.synchronize()

    B, C, K, H = 4, 96, 80, 12
    print(f"[limits] fused forced after weights B={B} C={C} K={K} H={H}", flush=True)
    torch.manual_seed(5)
    x = torch.randn(B, C, H, H, device=DEV, dtype=torch.float16)
    w = torch.randn(K, C, 3, 3, device=DEV) * 0.05
    ys = {}
    for path in (1, 3):
        h = lib.nova_create()
        try:
            lib.nova_set_weights(h, w.data_ptr(), K, C)
            lib.nova_set_path(h, path)
            y = torch.empty(B, K, H, H, device=DEV, dtype=torch.float16)
            lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, H, 1)
            check()
            assert lib.nova_get_last_path(h) == path
            torch.cuda.synchronize()
            ys[path] = y.float()
        finally:
            lib.nova_destroy(h)
    rel = ((ys[3] - ys[1]).norm() / ys[1].norm()).item()
    assert rel <= 2e-3, rel
