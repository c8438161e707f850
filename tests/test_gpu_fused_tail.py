"""The tile-block fused kernel with the short last run of every image left to
the small-problem kernel (path 3 at batches where the full 16-tile runs need
one round of workgroups less than all runs), through the C-ABI.

At ResNet-50 conv2_x (100 tiles per image: six full runs and one of 4
tiles) the split happens at batches 37-42 on 256 CUs with 2 tiles per
small-problem workgroup, and at 74-85 and 110-128 with 4 (2 would put more
than 2 workgroups on a CU). A tile gives the same bits in either kernel,
and every image is independent, so the batch is checked bit for bit
against the same images run in batches of eight (where no split happens),
NCHW and channels-last, with and without a bias/ReLU epilogue, and its
first two images against the oracle.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
CL = torch.channels_last


def _forward(lib, x, w, pad, nhwc=False, bias=None, relu=0, names=None):
    from nova_winograd.ops import check

    B, C, H, W = x.shape
    K = w.shape[0]
    Ho, Wo = H + 2 * pad - 2, W + 2 * pad - 2
    fmt = CL if nhwc else torch.contiguous_format
    y = torch.full((B, K, Ho, Wo), float("nan"), dtype=torch.float16,
                   device=DEV).contiguous(memory_format=fmt)
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, 3)
        lib.nova_set_layout(h, 1 if nhwc else 0)
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        if bias is not None or relu:
            lib.nova_set_epilogue(h, bias.data_ptr() if bias is not None else None, relu)
        if names is not None:
            lib.nova_profile_enable(h, 1)
        lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, W, pad)
        check("forward")
        assert lib.nova_get_last_path(h) == 3
        torch.cuda.synchronize()
        if names is not None:
            # the fused kind's span names the tail launch when it ran
            names.append(lib.nova_profile_kernel_name(h, 3).decode())
            lib.nova_profile_enable(h, 0)
    finally:
        lib.nova_destroy(h)
    return y


# (B, C, K, H, pad); on 256 CUs every case splits (asserted through the
# profiler's name for the fused span), and no batch of eight does
CASES = [
    (40, 64, 64, 56, 1),    # conv2_x: 280 workgroups, 240 full runs
    (37, 48, 64, 56, 1),    # 259 workgroups, 222 full runs, 48 input channels
    (128, 64, 64, 56, 1),   # conv2_x: 896 workgroups, 768 full runs, 4-tile tail groups
    (40, 40, 24, 56, 1),    # channel counts off the 32/16 blocks
    (40, 32, 32, 56, 1),    # one 32-channel chunk
    (43, 64, 64, 52, 2),    # 81 tiles per image: a 1-tile last run
]


@pytest.mark.parametrize("B,C,K,H,pad", CASES)
@pytest.mark.parametrize("nhwc", [False, True])
def test_fused_tail_matches_chunks(oracle, B, C, K, H, pad, nhwc):
    from nova_winograd.ops import get_lib

    print(f"[fused tail] B={B} C={C} K={K} H={H} pad={pad} nhwc={nhwc}", flush=True)
    lib = get_lib()
    g = torch.Generator().manual_seed(B * 7 + C + K + H + pad)
    x = torch.randn(B, C, H, H, generator=g).half()
    w = torch.randn(K, C, 3, 3, generator=g) * (2.0 / (9 * C)) ** 0.5
    bias = (torch.randn(K, generator=g) * 0.1).half().to(DEV)
    xd, wd = x.to(DEV), w.to(DEV)
    if nhwc:
        xd = xd.contiguous(memory_format=CL)
    cus = torch.cuda.get_device_properties(DEV).multi_processor_count
    for epi in (False, True):
        b_, r_ = (bias, 1) if epi else (None, 0)
        names, part_names = [], []
        y = _forward(lib, xd, wd, pad, nhwc, b_, r_, names).contiguous().cpu()
        assert torch.isfinite(y.float()).all()
        parts = [_forward(lib, xd[i:i + 8], wd, pad, nhwc, b_, r_, part_names).contiguous().cpu()
                 for i in range(0, B, 8)]
        print(f"[fused tail] {cus} CUs: batch ran {names[0]}, chunks {set(part_names)}",
              flush=True)
        assert all(n == "fused_block_kernel" for n in part_names)
        if cus == 256:  # the CU count these batches were chosen for
            assert names[0] == "fused_block_kernel+fused_small_kernel"
        assert torch.equal(y.view(torch.int16), torch.cat(parts).view(torch.int16))
        if not epi:
            # the parity bar for unit-scale outputs: rel-L2 5e-3, max-abs 0.5
            # (fp16 rounding of V, M and y in different summation orders; the
            # 43-image case reads 0.27 at one element of its first two)
            yo = oracle.conv2d(x[:2].numpy(), w.numpy(), pad)
            assert oracle.rel_l2(y[:2].numpy(), yo) <= 5e-3
            assert oracle.max_abs(y[:2].numpy(), yo) <= 0.5
