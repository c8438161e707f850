"""The module's cached forward: after a first call, repeated calls with the
same input shape, weight and bias (same objects, same versions, same storage)
on the same stream only allocate the output and launch. Every change that
the cache keys on must send the next call back through the full path: an
in-place weight update, a weight re-bound through ``.data``, a new weight
Parameter, a new bias, a
new input shape and a different current stream. Each result is compared
bitwise with a freshly built module holding the same parameters.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _fresh(conv):
    from nova_winograd import NovaWinogradConv2d

    ref = NovaWinogradConv2d(conv.in_channels, conv.out_channels, padding=conv.padding,
                             bias=conv.bias is not None).to(DEV)
    with torch.no_grad():
        ref.weight.copy_(conv.weight)
        if conv.bias is not None:
            ref.bias.copy_(conv.bias)
    return ref


def test_cached_forward_invalidation():
    from nova_winograd import NovaWinogradConv2d

    print("[module cache]", flush=True)
    torch.manual_seed(11)
    conv = NovaWinogradConv2d(16, 24, kernel_size=3, padding=1, bias=True).to(DEV)
    with torch.no_grad():
        conv.bias.copy_(torch.randn(24))
    x = torch.randn(2, 16, 12, 12, device=DEV).half()
    with torch.no_grad():
        y0 = conv(x)
        assert conv._state is not None  # the next call takes the cached path
        y1 = conv(x)
        assert torch.equal(y0, y1)
        assert torch.equal(y1, _fresh(conv)(x))

        conv.weight.mul_(0.5)  # in place: version bump
        y2 = conv(x)
        assert torch.equal(y2, _fresh(conv)(x))
        assert not torch.equal(y2, y1)

        conv.weight.data = torch.randn(24, 16, 3, 3, device=DEV)  # new storage, no bump
        y3 = conv(x)
        assert torch.equal(y3, _fresh(conv)(x))

        conv.weight = torch.nn.Parameter(torch.randn(24, 16, 3, 3, device=DEV))  # new object
        y3b = conv(x)
        assert torch.equal(y3b, _fresh(conv)(x))

        conv.bias = torch.nn.Parameter(torch.randn(24, device=DEV))  # new bias object
        y4 = conv(x)
        assert torch.equal(y4, _fresh(conv)(x))

        x2 = torch.randn(1, 16, 20, 18, device=DEV).half()  # new shape
        y5 = conv(x2)
        assert y5.shape == (1, 24, 20, 18)
        assert torch.equal(y5, _fresh(conv)(x2))

        s = torch.cuda.Stream()  # new current stream
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            y6 = conv(x)
            y6b = conv(x)  # cached path on the side stream
        s.synchronize()
        torch.cuda.current_stream().wait_stream(s)
        assert torch.equal(y6, y4)
        assert torch.equal(y6b, y4)
        y7 = conv(x)  # back on the default stream
        assert torch.equal(y7, y4)
    torch.cuda.synchronize()


def test_cached_forward_bias_changes_and_fresh_outputs():
    """The cached path reads the parameters from the module's parameter
    table: an in-place bias update, a bias set to None and a removed bias
    entry are all seen; and the output it allocates (like the input when the
    shapes agree) is a new tensor at every call."""
    from nova_winograd import NovaWinogradConv2d

    print("[module cache: bias, outputs]", flush=True)
    torch.manual_seed(12)
    conv = NovaWinogradConv2d(32, 32, kernel_size=3, padding=1, bias=True).to(DEV)
    with torch.no_grad():
        conv.bias.copy_(torch.randn(32))
    x = torch.randn(2, 32, 14, 14, device=DEV).half()
    with torch.no_grad():
        ya = conv(x)
        yb = conv(x)  # cached path, output allocated like x
        assert conv._state is not None
        assert yb.shape == x.shape and yb.dtype == torch.float16 and yb.is_contiguous()
        assert ya.data_ptr() != yb.data_ptr() and yb.data_ptr() != x.data_ptr()
        assert torch.equal(ya, yb)

        conv.bias.add_(0.25)  # in place: the bias version changes
        yc = conv(x)
        assert torch.equal(yc, _fresh(conv)(x))
        assert not torch.equal(yc, yb)

        conv.bias = None  # the entry stays, holding None
        yd = conv(x)
        assert torch.equal(yd, _fresh(conv)(x))
        ye = conv(x)  # cached path without a bias
        assert torch.equal(ye, yd)

        del conv.bias  # no entry at all: the full path, as nn.Conv2d would fail
        with pytest.raises(AttributeError):
            conv(x)
    torch.cuda.synchronize()


def test_functional_cached_handle(monkeypatch):
    """nova_forward runs on the persistent per-device handle: the filter is
    transformed once for repeated calls with the same weight, again after an
    in-place update, and a bias or residual of one call never leaks into the
    next (temporaries included)."""
    from nova_winograd import conv2d as cv
    from nova_winograd import nova_forward

    torch.manual_seed(15)
    x = torch.randn(2, 16, 14, 14, device=DEV).half()
    w = torch.randn(24, 16, 3, 3, device=DEV) * 0.1
    calls = []
    orig = cv._Handle.set_weights
    monkeypatch.setattr(cv._Handle, "set_weights",
                        lambda self, weight: (calls.append(1), orig(self, weight))[1])
    y0 = nova_forward(x, w)
    y1 = nova_forward(x, w)
    assert torch.equal(y0, y1) and len(calls) == 1
    yb = nova_forward(x, w, bias=torch.full((24,), 0.5, device=DEV))
    yb2 = nova_forward(x, w, bias=torch.full((24,), -0.25, device=DEV))  # a new temporary
    yr = nova_forward(x, w, residual=torch.ones_like(y0))
    y2 = nova_forward(x, w)
    torch.cuda.synchronize()
    assert torch.equal(yb, y0 + torch.tensor(0.5, dtype=torch.float16, device=DEV))
    assert torch.equal(yb2, y0 + torch.tensor(-0.25, dtype=torch.float16, device=DEV))
    assert torch.equal(yr, y0 + 1)
    assert torch.equal(y2, y0)  # neither bias nor residual left on the handle
    with torch.no_grad():
        w.mul_(2.0)
    y3 = nova_forward(x, w)
    assert len(calls) == 2
    assert not torch.equal(y3, y0)


def test_cached_forward_ctypes_fallback_raises_library_errors(monkeypatch):
    """Without the CPython fast-call binding the cached path launches through
    ctypes; a library error recorded by that launch must still raise (it is
    read once, by the check that raises). The error is provoked from the
    host: a fused path forced on a channels-last handle runs three-pass and
    reports it."""
    from nova_winograd import NovaWinogradConv2d, conv2d

    print("[module cache ctypes fallback]", flush=True)
    monkeypatch.setattr(conv2d, "_FASTCALL", [None])
    conv = NovaWinogradConv2d(16, 16, kernel_size=3, padding=1).to(DEV)
    x = torch.randn(1, 16, 12, 12, device=DEV).half()
    with torch.no_grad():
        y0 = conv(x)  # full path; records the cached launch (ctypes)
        assert conv._state is not None
        assert torch.equal(conv(x), y0)  # cached path, no error
        lib, h = conv._handle.lib, conv._handle.h
        lib.nova_set_layout(h, 1)
        lib.nova_set_path(h, 2)
        try:
            with pytest.raises(RuntimeError, match="fused path unsupported"):
                conv(x)
        finally:
            lib.nova_set_path(h, 0)
            lib.nova_set_layout(h, 0)
        assert lib.nova_get_last_error() == 0
        torch.cuda.synchronize()
