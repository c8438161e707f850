"""The three-pass GEMM on operand blocks at GEMV-like shapes (at most 32 tiles
per launch: batch-1 and small-batch deep layers), through the C-ABI.

nova_forward takes it there (U from the handle's block copy, V in the
two-pass layout); nova_forward_noalloc keeps the product-layout GEMM. Both
multiply in the same lane layout and channel-step order, so the two outputs
must agree bit for bit, and both stay within the reference's tolerance of the
oracle. Cases cover K off the 4- and 16-row blocks, channel counts off the
32-channel steps, exactly 16 and 32 tiles (one and two tile blocks per wave),
a partial second block, pad 0 and pad 2.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _lib():
    from nova_winograd.ops import get_lib

    return get_lib()


# (B, C, K, H, pad): tiles = B * ceil(Ho / 6)^2 <= 32, or <= 48 above K = 1024
CASES = [
    (1, 512, 512, 7, 1),    # ResNet-50 conv5_x, 4 tiles
    (1, 256, 256, 14, 1),   # conv4_x, 9 tiles
    (4, 512, 512, 7, 1),    # exactly 16 tiles
    (1, 200, 50, 13, 1),    # Cp = 200 (partial 32-channel step), K % 4 != 0
    (2, 96, 40, 9, 0),      # pad 0, 8 tiles
    (1, 64, 8, 11, 2),      # K < 16, pad 2
    (3, 1280, 1280, 8, 1),  # SD-1.5 1280@8^2 shape at batch 3: 12 tiles
    (1, 128, 128, 28, 1),   # conv3_x: 25 tiles, a partial second block
    (8, 512, 512, 7, 1),    # exactly 32 tiles
    (3, 72, 36, 14, 1),     # 27 tiles, K % 16 != 0, Cp = 72
    (1, 64, 1040, 32, 1),   # 36 tiles above K = 1024: three tile blocks per wave
]


@pytest.mark.parametrize("B,C,K,H,pad", CASES)
def test_block_gemm_equals_product_gemm(oracle, B, C, K, H, pad):
    from nova_winograd.ops import check

    print(f"[gemv blocks] B={B} C={C} K={K} H={H} pad={pad}", flush=True)
    lib = _lib()
    g = torch.Generator().manual_seed(B * 7 + C + K)
    x = torch.randn(B, C, H, H, generator=g).half()
    w = torch.randn(K, C, 3, 3, generator=g) * (2.0 / (9 * C)) ** 0.5
    xd, wd = x.to(DEV), w.to(DEV)
    Ho = H + 2 * pad - 2
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, 1)
        lib.nova_set_weights(h, wd.data_ptr(), K, C)
        y_blocks = torch.empty(B, K, Ho, Ho, dtype=torch.float16, device=DEV)
        y_plain = torch.full_like(y_blocks, float("nan"))
        lib.nova_forward(h, xd.data_ptr(), y_blocks.data_ptr(), B, H, H, pad)
        check("forward")
        assert lib.nova_get_last_path(h) == 1
        lib.nova_forward_noalloc(h, xd.data_ptr(), y_plain.data_ptr(), B, H, H, pad)
        check("forward_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(y_blocks.view(torch.int16), y_plain.view(torch.int16))
        # the workspace query covers V in blocks plus M
        nh = -(-Ho // 6)
        bp = B * nh * nh
        cp = -(-C // 8) * 8
        v_blocks = 64 * -(-bp // 16) * -(-cp // 32) * 512
        assert lib.nova_workspace_bytes(h, B, H, H, pad) == 2 * (v_blocks + 64 * K * bp)
    finally:
        lib.nova_destroy(h)
    n = min(B, 2)
    yo = oracle.conv2d(x[:n].numpy(), w.numpy(), pad)
    yg = y_blocks[:n].cpu().numpy()
    assert np.isfinite(yg).all()
    assert oracle.rel_l2(yg, yo) <= 5e-3
    assert oracle.max_abs(yg, yo) <= 0.25


def test_block_gemm_follows_new_weights():
    """Setting new weights rebuilds the block copy: the forward after the
    second set_weights matches a fresh handle with those weights."""
    from nova_winograd.ops import check

    print("[gemv blocks] weights replaced", flush=True)
    lib = _lib()
    B, C, K, H = 1, 256, 256, 14
    torch.manual_seed(5)
    x = torch.randn(B, C, H, H, device=DEV).half()
    w1 = torch.randn(K, C, 3, 3, device=DEV) * 0.03
    w2 = torch.randn(K, C, 3, 3, device=DEV) * 0.03
    y = torch.empty(B, K, H, H, dtype=torch.float16, device=DEV)
    y_fresh = torch.empty_like(y)
    h = lib.nova_create()
    h2 = lib.nova_create()
    try:
        lib.nova_set_weights(h, w1.data_ptr(), K, C)
        lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, H, 1)
        lib.nova_set_weights(h, w2.data_ptr(), K, C)
        lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, H, 1)
        lib.nova_set_weights(h2, w2.data_ptr(), K, C)
        lib.nova_forward(h2, x.data_ptr(), y_fresh.data_ptr(), B, H, H, 1)
        check("forward")
        torch.cuda.synchronize()
        assert torch.equal(y, y_fresh)
    finally:
        lib.nova_destroy(h)
        lib.nova_destroy(h2)
