"""Input alignment and size do not change the output.

The kernels that read x with 4- and 16-byte loads (the tile-block and run
input transforms of the three- and two-pass paths, the fused position-row
kernel, both forms of the fused tile-block kernel) address it from a 16-byte
boundary through a buffer resource whose size must cover the dword that
holds x's last element: a load returns zero for a dword that extends past
the size. Each case runs the same input from several offsets (x_bytes 0, 2
and 4 mod 8 past a 256-byte boundary) on every path, and all outputs of a
path must agree bit for bit; the shapes put an odd element count (the last
element alone in its dword) and the tile-block input kernel's grid (256
workgroups or more) in play.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")

# (B, C, K, H, W, pad)
CASES = [
    (2, 64, 64, 112, 112, 1),  # tile-block input transform, fused tile-block (wide)
    (25, 33, 40, 27, 27, 1),   # odd element count, tile-block input transform
    (1, 3, 5, 13, 13, 1),      # odd element count, small
    (3, 24, 16, 30, 30, 2),    # pad 2
    (33, 65, 48, 27, 27, 1),   # two-pass: the run-form input transform (260 workgroups),
                               # odd element count
    (48, 64, 48, 28, 28, 2),   # the run form with pad 2
]
OFFSETS = [0, 1, 2, 5, 7]  # halves past a 256-byte boundary


def _forward(lib, x, w, pad, path):
    from nova_winograd.ops import check

    B, C, H, W = x.shape
    K = w.shape[0]
    y = torch.full((B, K, H + 2 * pad - 2, W + 2 * pad - 2), float("nan"), dtype=torch.float16,
                   device=DEV)
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, path)
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, W, pad)
        took = lib.nova_get_last_path(h)
        if path in (2, 3, 5) and took == 1:
            assert lib.nova_get_last_error() != 0  # forced fused path outside its envelope
        else:
            check("forward")
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    return y, took


@pytest.mark.parametrize("B,C,K,H,W,pad", CASES)
@pytest.mark.parametrize("path", [1, 2, 3, 6])
def test_output_independent_of_input_offset(B, C, K, H, W, pad, path):
    from nova_winograd.ops import get_lib

    print(f"[alignment] path={path} B={B} C={C} K={K} H={H} W={W} pad={pad}", flush=True)
    lib = get_lib()
    g = torch.Generator().manual_seed(B + C + K + H + W + pad)
    x = torch.randn(B, C, H, W, generator=g).half().to(DEV)
    w = (torch.randn(K, C, 3, 3, generator=g) * (2.0 / (9 * C)) ** 0.5).to(DEV)
    n = x.numel()
    buf = torch.empty(n + 64, dtype=torch.float16, device=DEV)
    assert buf.data_ptr() % 256 == 0
    ref, took_ref = None, None
    for off in OFFSETS:
        buf.fill_(float("nan"))  # bytes around x must not reach the output
        xv = buf[off:off + n].view(x.shape)
        xv.copy_(x)
        y, took = _forward(lib, xv, w, pad, path)
        assert torch.isfinite(y.float()).all(), off
        if ref is None:
            ref, took_ref = y, took
        else:
            assert took == took_ref, off
            assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), off
