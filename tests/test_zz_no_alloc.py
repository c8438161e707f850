"""nova_forward_noalloc: the allocation-free forward (no counterpart in the
reference), through the C-ABI.

It must give nova_forward's result on the same handle, bit for bit, over two
calls in a row -- the second with a smaller input, so a stale tail of the
shared scratch from the first call would show -- on the three-pass path
(workspace in the library's scratch array), on the fused tile-block path (no
workspace), in channels-last layout with the epilogue, and on a batch large
enough to be split into several scratch-sized launches. A shape whose single
image needs more workspace than the scratch holds is refused and its output
left untouched.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
SCRATCH_BYTES = 64 << 20  # NOVA_NOALLOC_SCRATCH_BYTES in include/nova_winograd.h


def _lib():
    from nova_winograd.ops import get_lib

    return get_lib()


def _weights(K, C, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.empty(K, C, 3, 3)
    torch.nn.init.kaiming_normal_(w, mode="fan_in", nonlinearity="relu", generator=g)
    return w.to(DEV)


def _pair(lib, h, x, K, pad=1, nhwc=False):
    """(nova_forward output, nova_forward_noalloc output) on handle h."""
    from nova_winograd.ops import check

    B, C, H, W = x.shape
    fmt = torch.channels_last if nhwc else torch.contiguous_format
    shape = (B, K, H + 2 * pad - 2, W + 2 * pad - 2)
    y_ref = torch.empty(shape, dtype=torch.float16, device=DEV, memory_format=fmt)
    y = torch.full(shape, float("nan"), dtype=torch.float16, device=DEV).contiguous(
        memory_format=fmt)
    lib.nova_forward(h, x.data_ptr(), y_ref.data_ptr(), B, H, W, pad)
    check("forward")
    path_ref = lib.nova_get_last_path(h)
    lib.nova_forward_noalloc(h, x.data_ptr(), y.data_ptr(), B, H, W, pad)
    check("forward_noalloc")
    path = lib.nova_get_last_path(h)
    torch.cuda.synchronize()
    return y_ref, y, path_ref, path


# (C, K, H, pad, first batch, second batch, expected path): second call
# smaller; a path per batch where they differ, and a (nova_forward,
# nova_forward_noalloc) pair where the allocation-free form runs three-pass
# in place of the two-pass path (bit-identical to it)
CASES = [
    (128, 128, 28, 1, 8, 3, 1),     # three-pass, conv3_x
    (64, 64, 56, 1, 4, 2, ((6, 1), 5)),  # two-pass / three-pass, then the small-problem kernel
    (64, 64, 56, 1, 32, 24, 3),     # fused tile-block, conv2_x (no workspace)
    (512, 512, 7, 1, 32, 1, 1),     # three-pass, conv5_x, then batch 1
    (100, 24, 17, 0, 6, 2, (1, 7)),  # C % 8 != 0 (padded channel pitch), pad 0; batch 2
                                     # takes the input transform in the products (M only)
    (40, 24, 17, 0, 6, 2, 5),       # the small-problem fused kernel (no workspace)
]


@pytest.mark.parametrize("C,K,H,pad,B1,B2,path", CASES)
def test_noalloc_equals_forward_twice(C, K, H, pad, B1, B2, path):
    print(f"[noalloc] C={C} K={K} H={H} pad={pad} B={B1} then {B2}", flush=True)
    lib = _lib()
    torch.manual_seed(31)
    w = _weights(K, C, 32)
    h = lib.nova_create()
    try:
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        for B, want in zip((B1, B2), path if isinstance(path, tuple) else (path, path)):
            want_ref, want_na = want if isinstance(want, tuple) else (want, want)
            x = torch.randn(B, C, H, H, device=DEV).half()
            y_ref, y, p_ref, p = _pair(lib, h, x, K, pad)
            assert (p_ref, p) == (want_ref, want_na)
            assert torch.equal(y, y_ref), f"B={B}"
    finally:
        lib.nova_destroy(h)


def test_noalloc_channels_last_with_epilogue():
    from nova_winograd.ops import check

    print("[noalloc] NHWC + bias/residual/ReLU", flush=True)
    lib = _lib()
    torch.manual_seed(33)
    C, K, H = 128, 96, 20
    w = _weights(K, C, 34)
    bias = (torch.randn(K, device=DEV) * 0.5).half()
    h = lib.nova_create()
    try:
        lib.nova_set_layout(h, 1)
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        lib.nova_set_epilogue(h, bias.data_ptr(), 1)
        for B in (6, 2):
            x = torch.randn(B, C, H, H, device=DEV).half().contiguous(
                memory_format=torch.channels_last)
            res = torch.randn(B, K, H, H, device=DEV).half().contiguous(
                memory_format=torch.channels_last)
            lib.nova_set_residual(h, res.data_ptr())
            y_ref, y, p_ref, p = _pair(lib, h, x, K, 1, nhwc=True)
            lib.nova_set_residual(h, None)
            check()
            # batch 2 (32 tiles, 96 output channels): the input transform in
            # the products, M in the scratch
            assert p == p_ref == (1 if B == 6 else 7), (p, p_ref)
            assert torch.equal(y, y_ref), f"B={B}"
    finally:
        lib.nova_destroy(h)


def test_noalloc_splits_large_batches():
    """conv3_x at B=128 needs 105 MB of V + M: the allocation-free forward
    runs it as two scratch-sized launches. Each image's arithmetic is the same
    kernels', so the result is nova_forward's within the fp32 accumulation
    bound (the GEMM's tile shape follows the launch's batch) -- and bit for
    bit against nova_forward on the same sub-batches."""
    from nova_winograd.ops import check

    print("[noalloc] batch split", flush=True)
    lib = _lib()
    torch.manual_seed(35)
    B, C, K, H = 128, 128, 128, 28
    per_img = 2 * 64 * (C + K) * 25
    chunk = (SCRATCH_BYTES - 256) // per_img
    assert chunk < B
    w = _weights(K, C, 36)
    x = torch.randn(B, C, H, H, device=DEV).half()
    h = lib.nova_create()
    try:
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        y = torch.empty(B, K, H, H, dtype=torch.float16, device=DEV)
        lib.nova_forward_noalloc(h, x.data_ptr(), y.data_ptr(), B, H, H, 1)
        check()
        y_ref = torch.empty_like(y)
        lib.nova_forward(h, x.data_ptr(), y_ref.data_ptr(), B, H, H, 1)
        check()
        y_sub = torch.empty_like(y)
        for b0 in range(0, B, chunk):
            n = min(chunk, B - b0)
            lib.nova_forward(h, x[b0:].data_ptr(), y_sub[b0:].data_ptr(), n, H, H, 1)
            check()
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    assert torch.equal(y, y_sub)
    a, b = y.float(), y_ref.float()
    assert ((a - b).norm() / b.norm()).item() <= 2e-3


def test_noalloc_refuses_oversized_images():
    """One SDXL-sized image (1280 channels at 128 x 128) needs 79 MB of V + M,
    more than the scratch: refused with the workspace error, output untouched;
    the handle stays usable."""
    from nova_winograd.ops import check

    print("[noalloc] oversized image", flush=True)
    lib = _lib()
    C = K = 1280
    H = 128
    w = torch.randn(K, C, 3, 3, device=DEV) * 0.01
    x = torch.randn(1, C, H, H, device=DEV).half()
    y = torch.zeros(1, K, H, H, dtype=torch.float16, device=DEV)
    h = lib.nova_create()
    try:
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        check()
        lib.nova_forward_noalloc(h, x.data_ptr(), y.data_ptr(), 1, H, H, 1)
        assert lib.nova_get_last_error() == 4
        assert b"allocation-free" in lib.nova_get_last_error_message()
        torch.cuda.synchronize()
        assert not y.any()
        xs = x[:, :, :32, :32].contiguous()  # a small image still runs
        ys = torch.empty(1, K, 32, 32, dtype=torch.float16, device=DEV)
        lib.nova_forward_noalloc(h, xs.data_ptr(), ys.data_ptr(), 1, 32, 32, 1)
        check()
        torch.cuda.synchronize()
        assert torch.isfinite(ys).all()
    finally:
        lib.nova_destroy(h)


def test_noalloc_declared_in_header():
    import os
    import re

    hdr = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                            "include", "nova_winograd.h")).read()
    assert re.search(r"NOVA_API void nova_forward_noalloc\(", hdr)
    m = re.search(r"#define NOVA_NOALLOC_SCRATCH_BYTES \((\d+)ll << (\d+)\)", hdr)
    assert m and int(m.group(1)) << int(m.group(2)) == SCRATCH_BYTES
    assert ctypes.cast(_lib().nova_forward_noalloc, ctypes.c_void_p).value
