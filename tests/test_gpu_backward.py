"""Backward of the trainable module and the custom op's filter cache.

grad input runs on the NOVA forward path with the flipped, channel-swapped
filter at padding 2 - p: it must equal the oracle's NOVA convolution of
grad_output with that filter (same parity bar as the forward), for every
padding that has such a form; padding 3 falls back to fp32 PyTorch.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.mark.parametrize("B,C,K,H,pad", [(2, 16, 24, 14, 1), (1, 32, 8, 11, 0), (2, 8, 16, 9, 2),
                                         (1, 64, 64, 28, 1)])
def test_grad_input_matches_oracle(oracle, B, C, K, H, pad):
    from nova_winograd import NovaWinogradConv2dTrainable

    print(f"[backward] B={B} C={C} K={K} H={H} pad={pad}", flush=True)
    torch.manual_seed(11)
    conv = NovaWinogradConv2dTrainable(C, K, kernel_size=3, padding=pad).to(DEV)
    x = torch.randn(B, C, H, H, device=DEV).half().requires_grad_(True)
    y = conv(x)
    go = torch.randn_like(y)
    y.backward(go)
    torch.cuda.synchronize()
    gi = x.grad.float().cpu().numpy()
    wflip = conv.weight.detach().flip(2, 3).transpose(0, 1).contiguous().float().cpu().numpy()
    want = oracle.conv2d(go.cpu().numpy(), wflip, 2 - pad)
    assert gi.shape == want.shape
    assert np.isfinite(gi).all()
    assert oracle.rel_l2(gi.astype(np.float16), want) <= 5e-3
    # and close to the exact gradient (fp32 autograd), like the forward
    xr = x.detach().float().requires_grad_(True)
    torch.nn.functional.conv2d(xr, conv.weight.detach().float(), padding=pad).backward(go.float())
    exact = xr.grad.cpu().numpy()
    assert np.linalg.norm(gi - exact) / np.linalg.norm(exact) < 0.10


def test_grad_input_padding_fallback():
    from nova_winograd import NovaWinogradConv2dTrainable

    torch.manual_seed(12)
    conv = NovaWinogradConv2dTrainable(8, 8, kernel_size=3, padding=3).to(DEV)
    x = torch.randn(1, 8, 10, 10, device=DEV).half().requires_grad_(True)
    y = conv(x)
    y.float().sum().backward()
    xr = x.detach().float().requires_grad_(True)
    torch.nn.functional.conv2d(xr, conv.weight.detach().float(), padding=3).sum().backward()
    torch.cuda.synchronize()
    rel = (torch.linalg.vector_norm(x.grad.float() - xr.grad)
           / torch.linalg.vector_norm(xr.grad)).item()
    assert rel < 1e-2


def test_custom_op_caches_filter_transform(monkeypatch):
    from nova_winograd import conv2d as mod

    mod._register_custom_op()
    calls = []
    orig = mod._Handle.set_weights

    def counting(self, w):
        calls.append(1)
        return orig(self, w)

    monkeypatch.setattr(mod._Handle, "set_weights", counting)
    torch.manual_seed(13)
    w = torch.randn(16, 8, 3, 3, device=DEV) * 0.1
    x = torch.randn(1, 8, 12, 12, device=DEV).half()
    y1 = torch.ops.nova.winograd_conv2d(x, w, 1)
    y2 = torch.ops.nova.winograd_conv2d(x, w, 1)
    n_same = len(calls)
    with torch.no_grad():
        w.mul_(2.0)  # version bump -> re-transformed
    y3 = torch.ops.nova.winograd_conv2d(x, w, 1)
    w2 = w.clone()  # a different tensor object -> re-transformed
    y4 = torch.ops.nova.winograd_conv2d(x, w2, 1)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert n_same <= 1  # the first call may transform, the repeat must not
    assert len(calls) == n_same + 2
    assert torch.equal(y3, y4)
    assert not torch.equal(y1, y3)


def test_grad_input_follows_weight_updates():
    """The backward's flipped-filter transform is cached per weight tensor:
    an in-place update (optimizer step), a rebound weight and a ``.data``
    write followed by invalidate_weight_cache() are all picked up; each grad
    input equals a fresh module's with the same weights, bit for bit."""
    from nova_winograd import NovaWinogradConv2dTrainable

    torch.manual_seed(13)
    conv = NovaWinogradConv2dTrainable(16, 24, kernel_size=3, padding=1).to(DEV)
    x = torch.randn(2, 16, 12, 12, device=DEV).half()

    def grad_input(module):
        xi = x.clone().requires_grad_(True)
        y = module(xi)
        y.backward(torch.ones_like(y))
        torch.cuda.synchronize()
        return xi.grad.clone()

    def fresh():
        m = NovaWinogradConv2dTrainable(16, 24, kernel_size=3, padding=1).to(DEV)
        with torch.no_grad():
            m.weight.copy_(conv.weight)
        return m

    g0 = grad_input(conv)
    assert torch.equal(g0, grad_input(fresh()))
    with torch.no_grad():
        conv.weight.mul_(-0.5)  # in place: version bump
    g1 = grad_input(conv)
    assert torch.equal(g1, grad_input(fresh())) and not torch.equal(g1, g0)
    conv.weight = torch.nn.Parameter(torch.randn(24, 16, 3, 3, device=DEV) * 0.1)  # rebound
    g2 = grad_input(conv)
    assert torch.equal(g2, grad_input(fresh()))
    conv.weight.data.mul_(3.0)  # through .data: no version bump
    conv.invalidate_weight_cache()
    g3 = grad_input(conv)
    assert torch.equal(g3, grad_input(fresh())) and not torch.equal(g3, g2)


# (B, C, K, H, W, pad): edge tiles, K and C off the 64-blocks, pads 0-2,
# non-square, the ResNet-50 layers at B=1 and B=32, a stem-like 3 -> 64 layer
# at 224^2, and one batch the library splits into sub-batches: at 3 -> 64 on
# 224^2 (1 444 tiles per image) a sub-batch holds at most 43 images (Vt and Mt
# together within 1 GiB), so batch 44 runs as 43 + 1 images and the second
# sub-batch adds into the first one's filter gradient (the accumulate pass of
# wg_gemm_proj_kernel, with the tile range split over the CUs)
WGRAD_CASES = [
    (2, 16, 24, 14, 14, 1), (1, 32, 8, 11, 11, 0), (2, 8, 16, 9, 9, 2), (3, 40, 72, 13, 17, 1),
    (1, 64, 64, 56, 56, 1), (1, 512, 512, 7, 7, 1), (32, 64, 64, 56, 56, 1),
    (32, 256, 256, 14, 14, 1), (2, 3, 64, 224, 224, 1), (44, 3, 64, 224, 224, 1),
]


def wgrad_chunk_images(B, C, K, H, W, pad):
    """Images per sub-batch of nova_weight_grad (the library's rule: Vt and Mt
    in fp32, 256 bytes per channel and tile, each below 2^31 bytes and
    together within 1 GiB)."""
    P = -(-(H + 2 * pad - 2) // 6) * -(-(W + 2 * pad - 2) // 6)
    per_img = 256 * P
    by_off = ((1 << 31) - 256 * 16 - 1) // (per_img * max(C, K))
    by_total = (1 << 30) // (per_img * (C + K))
    return max(1, min(max(B, 1), by_off, by_total))


def test_wgrad_cases_include_a_split_batch():
    assert wgrad_chunk_images(44, 3, 64, 224, 224, 1) == 43
    assert any(wgrad_chunk_images(*c) < c[0] for c in WGRAD_CASES)


@pytest.mark.parametrize("B,C,K,H,W,pad", WGRAD_CASES)
@pytest.mark.parametrize("gdt", ["f16", "f32"])
def test_weight_grad_matches_fp64(oracle, B, C, K, H, W, pad, gdt):
    """nova_weight_grad (fp32 Winograd-domain products reduced over the tiles)
    against the fp64 direct gradient of the same fp16 input: rel-L2 <= 1e-4
    and max-abs <= 1e-4 of the largest entry (the reference's bar for grad
    weight is 0.15, tests/test_correctness.py:164). The output gradient comes
    in fp16 or fp32; the result is deterministic."""
    from nova_winograd.ops import check, get_lib

    print(f"[wgrad] B={B} C={C} K={K} H={H} W={W} pad={pad} dy={gdt}", flush=True)
    lib = get_lib()
    g = torch.Generator().manual_seed(B + C + K + H)
    x = torch.randn(B, C, H, W, generator=g).half()
    Ho, Wo = H + 2 * pad - 2, W + 2 * pad - 2
    dy = torch.randn(B, K, Ho, Wo, generator=g) * 1e-3
    if gdt == "f16":
        dy = dy.half()
    xd, gd = x.to(DEV), dy.to(DEV)
    outs = []
    h = lib.nova_create()
    try:
        for _ in range(2):
            gw = torch.full((K, C, 3, 3), float("nan"), device=DEV)
            lib.nova_weight_grad(h, xd.data_ptr(), gd.data_ptr(), gw.data_ptr(), B, C, K, H, W,
                                 pad, 1 if gdt == "f32" else 0)
            check()
            outs.append(gw)
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    assert torch.equal(outs[0], outs[1]), "not deterministic"
    n = min(B, 4)  # the fp64 truth on the first images of a large batch ...
    if n < B:  # ... against the GPU on those images alone
        h = lib.nova_create()
        try:
            gw_n = torch.empty(K, C, 3, 3, device=DEV)
            lib.nova_weight_grad(h, xd.data_ptr(), gd.data_ptr(), gw_n.data_ptr(), n, C, K, H, W,
                                 pad, 1 if gdt == "f32" else 0)
            check()
            torch.cuda.synchronize()
        finally:
            lib.nova_destroy(h)
    else:
        gw_n = outs[0]
    got = gw_n.cpu().numpy().astype(np.float64)
    want = oracle.weight_grad(x[:n].numpy(), dy[:n].float().numpy(), pad)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    worst = np.abs(got - want).max() / np.abs(want).max()
    print(f"[wgrad] rel-L2 {rel:.2e}, max-abs/max {worst:.2e}", flush=True)
    assert np.isfinite(got).all()
    assert rel <= 1e-4
    assert worst <= 1e-4
    if n < B:  # the whole batch: linear in the images, so it is the sum over sub-batches
        rest = torch.empty(K, C, 3, 3, device=DEV)
        h = lib.nova_create()
        try:
            lib.nova_weight_grad(h, xd[n:].contiguous().data_ptr(), gd[n:].contiguous().data_ptr(),
                                 rest.data_ptr(), B - n, C, K, H, W, pad,
                                 1 if gdt == "f32" else 0)
            check()
            torch.cuda.synchronize()
        finally:
            lib.nova_destroy(h)
        # each side is within ~3e-5 of the exact gradient (fp32 sums over
        # different partitions of the tiles)
        total = (gw_n + rest).double()
        full = outs[0].double()
        assert ((full - total).norm() / full.norm()).item() <= 1e-4


def test_weight_grad_empty_batch_is_zero():
    from nova_winograd.ops import check, get_lib

    lib = get_lib()
    gw = torch.full((8, 4, 3, 3), 7.0, device=DEV)
    h = lib.nova_create()
    try:
        lib.nova_weight_grad(h, None, None, gw.data_ptr(), 0, 4, 8, 9, 9, 1, 0)
        check()
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    assert not gw.any()


def test_trainable_weight_grad_on_hip_path(oracle):
    """The module's backward takes grad weight from nova_weight_grad: it
    matches the fp64 gradient of the fp16 input the forward convolved, with
    an fp16 output gradient as autograd delivers it, and the bias gradient is
    the channel sum."""
    from nova_winograd import NovaWinogradConv2dTrainable

    torch.manual_seed(14)
    conv = NovaWinogradConv2dTrainable(24, 40, kernel_size=3, padding=1, bias=True).to(DEV)
    x = torch.randn(3, 24, 20, 20, device=DEV)
    y = conv(x)
    go = (torch.randn_like(y.float()) * 0.01).half()
    y.backward(go)
    torch.cuda.synchronize()
    want = oracle.weight_grad(x.half().cpu().numpy(), go.float().cpu().numpy(), 1)
    got = conv.weight.grad.double().cpu().numpy()
    assert np.linalg.norm(got - want) / np.linalg.norm(want) <= 1e-4
    gb = go.float().sum(dim=(0, 2, 3))
    assert torch.allclose(conv.bias.grad, gb, rtol=1e-5, atol=1e-6)
