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
