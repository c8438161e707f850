"""The unstaged form of the fused tile-block kernel (path 3 at up to 64 input
channels, NCHW and channels-last), through the C-ABI.

Each thread loads its patch rows straight from global memory as a 16-byte
and a 4-byte load from the dword at or below the row start, so the cases
cover the address arithmetic the staged form never had: x at 2-, 6- and
14-byte offsets from a 16-byte boundary, left padding of 1 and 2 columns on
the first row of the tensor (the rows that start before the buffer), images
wider than the staged form allowed (nw > 10), one and two 32-channel steps,
channel counts off the 8/16/32 blocks and more than one 64-channel output
block. Every output is checked against the oracle; the same input at another
alignment gives the same bits, and so does the channels-last form from the
same alignment (one 2-byte load per pixel; same transforms, same MFMA
order).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")

# (B, C, K, H, W, pad, offset in halves of x from a 16-byte boundary)
CASES = [
    (2, 64, 64, 112, 112, 1, 0),   # nw = 19: wider than the staged form allowed
    (3, 64, 64, 20, 20, 2, 0),     # pad 2: first rows start 4 bytes before x
    (2, 40, 24, 17, 23, 2, 1),     # x at +2 bytes, pad 2: 2 bytes before the boundary
    (2, 24, 64, 9, 9, 1, 3),       # x at +6 bytes, one step
    (1, 64, 64, 70, 130, 1, 0),    # non-square, nw = 22
    (4, 8, 16, 30, 30, 0, 0),      # pad 0, C = 8
    (2, 33, 65, 14, 14, 1, 7),     # two output blocks, Cp = 40, x at +14 bytes
    (5, 64, 48, 28, 28, 1, 0),     # K = 48: three of the output block's four row tiles
    (2, 3, 5, 11, 7, 1, 1),        # tiny channel counts
]


def _forward(lib, x, w, pad, path, nhwc=False):
    from nova_winograd.ops import check

    B, C, H, W = x.shape
    K = w.shape[0]
    Ho, Wo = H + 2 * pad - 2, W + 2 * pad - 2
    fmt = torch.channels_last if nhwc else torch.contiguous_format
    y = torch.full((B, K, Ho, Wo), float("nan"), dtype=torch.float16,
                   device=DEV).contiguous(memory_format=fmt)
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, path)
        lib.nova_set_layout(h, 1 if nhwc else 0)
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, W, pad)
        took = lib.nova_get_last_path(h)
        if path == 3 and took != 3:
            # a forced fused path outside its envelope runs three-pass and says so
            assert lib.nova_get_last_error() != 0
        else:
            check("forward")
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    return y, took


def _at_offset(x, off):
    """x's values in a fresh buffer starting `off` halves past a 256-byte
    aligned allocation."""
    n = x.numel()
    buf = torch.empty(n + 64, dtype=torch.float16, device=DEV)
    assert buf.data_ptr() % 256 == 0
    xv = buf[off:off + n].view(x.shape)
    xv.copy_(x)
    return xv


@pytest.mark.parametrize("B,C,K,H,W,pad,off", CASES)
def test_fused_direct_matches_oracle(oracle, B, C, K, H, W, pad, off):
    from nova_winograd.ops import get_lib

    print(f"[fused direct] B={B} C={C} K={K} H={H} W={W} pad={pad} off={off}", flush=True)
    lib = get_lib()
    g = torch.Generator().manual_seed(B * 131 + C * 7 + K + H + W + pad + off)
    x = torch.randn(B, C, H, W, generator=g).half()
    w = torch.randn(K, C, 3, 3, generator=g) * (2.0 / (9 * C)) ** 0.5
    wd = w.to(DEV)
    xo = _at_offset(x.to(DEV), off)
    assert (xo.data_ptr() - off * 2) % 256 == 0
    y, took = _forward(lib, xo, wd, pad, 3)
    assert took == 3
    yc = y.cpu()
    assert torch.isfinite(yc.float()).all()
    n = min(B, 2)
    yo = oracle.conv2d(x[:n].numpy(), w.numpy(), pad)
    yg = yc[:n].numpy()
    assert oracle.rel_l2(yg, yo) <= 5e-3
    assert oracle.max_abs(yg, yo) <= 0.25
    # another alignment of the same input: the same bits
    y0, _ = _forward(lib, _at_offset(x.to(DEV), 0 if off else 5), wd, pad, 3)
    assert torch.equal(y0.cpu().view(torch.int16), yc.view(torch.int16))
    # channels-last, from the same alignment: the same bits
    n_el = x.numel()
    store = torch.empty(n_el + 64, dtype=torch.float16, device=DEV)
    xc = torch.as_strided(store, (B, C, H, W), (H * W * C, 1, W * C, C), storage_offset=off)
    xc.copy_(x.to(DEV))
    assert xc.is_contiguous(memory_format=torch.channels_last)
    yn, took_n = _forward(lib, xc, wd, pad, 3, nhwc=True)
    assert took_n == 3
    assert torch.equal(yn.contiguous().cpu().view(torch.int16), yc.view(torch.int16))
