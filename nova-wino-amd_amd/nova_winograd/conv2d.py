"""NOVA Winograd Conv2d modules -- drop-in replacements for ``torch.nn.Conv2d``
(3x3, stride 1), mirroring /root/reference/nova_winograd/conv2d.py.

Classes:
    NovaWinogradConv2d           inference module: cached filter transform,
                                 weight versioning, workspace caching
    NovaWinogradConv2dTrainable  HIP forward and backward (grad input through the
                                 forward kernels, grad weight on the Winograd domain)
    NovaWinogradConv2dCompilable ``torch.compile`` through the custom op
                                 ``torch.ops.nova.winograd_conv2d`` (bias fused)

The forward runs on the gfx950 library through the C-ABI; there is no CPU
fallback (a CPU input raises).
"""

import atexit
import ctypes
import math
import threading
import weakref
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from nova_winograd.ops import (
    _raw_stream,
    check,
    compute_tiling,
    current_stream_ptr,
    get_lib,
    ptr,
    require_gpu_tensor,
)

_MISSING = object()  # a parameter entry that is not there


def _weight_key(weight):
    """State of the weight contents the cached filter transform was built
    from, checked together with the weight object's identity (held by weak
    reference). ``_version`` catches in-place updates (optimizer steps,
    ``load_state_dict``); identity, pointer, dtype and shape catch
    re-binding, ``.to()`` and ``.half()``. (The reference keys on ``_version``
    alone, /root/reference/nova_winograd/conv2d.py:195-203.)"""
    return (weight._version, weight.data_ptr(), weight.dtype, tuple(weight.shape),
            weight.device)


_FASTCALL = []  # [forward_ws or None], resolved once


def _fastcall(lib):
    """The CPython fast-call binding of nova_forward_workspace (one foreign
    call that also raises on a library error), or None when it is not built;
    the cached forward path then uses ctypes."""
    if not _FASTCALL:
        fn = None
        try:
            from nova_winograd import _nova_call

            addr = lambda f: ctypes.cast(f, ctypes.c_void_p).value  # noqa: E731
            _nova_call.bind(addr(lib.nova_forward_workspace), addr(lib.nova_get_last_error),
                            addr(lib.nova_get_last_error_message))
            fn = _nova_call.forward_ws
        except ImportError:
            pass
        _FASTCALL.append(fn)
    return _FASTCALL[0]


def _is_nhwc(x):
    """True for a channels-last 4-d tensor that is not also NCHW-contiguous
    (those run the NHWC kernels)."""
    return (x.dim() == 4 and not x.is_contiguous()
            and x.is_contiguous(memory_format=torch.channels_last))


_exiting = False


def _mark_exiting():
    global _exiting
    _exiting = True


atexit.register(_mark_exiting)


class _Handle:
    """Owns one library handle; destroyed with the Python object (at
    interpreter exit the process releases device memory itself)."""

    __slots__ = ("h", "lib", "stream", "key", "bias_key", "bias16", "b_ref", "w_ref", "res_ptr",
                 "nhwc")

    def __init__(self):
        self.lib = get_lib()
        self.h = self.lib.nova_create()
        check("create")
        self.stream = 0
        self.key = None
        self.bias_key = (None, 0)  # the library's default epilogue: none
        self.bias16 = None
        self.b_ref = None
        self.w_ref = None
        self.res_ptr = None
        self.nhwc = 0

    def set_weights_cached(self, weight):
        """Transform the filter unless this exact tensor object, unchanged
        (same storage, same version), was the last one transformed. The
        tensor is held by weak reference, so a freed temporary whose memory
        is reused can never match."""
        key = (weight.data_ptr(), weight._version, tuple(weight.shape), weight.dtype)
        ref = self.w_ref
        if ref is not None and ref[0]() is weight and ref[1] == key:
            return
        self.set_weights(weight)
        self.w_ref = (weakref.ref(weight), key)

    def set_bias(self, bias, relu=0):
        """Fuse the bias add (and optionally a ReLU) into the output
        transform: the library adds an fp16 copy of ``bias`` with the rounding
        of the reference's separate ``output + bias.half()``. The copy is kept
        here while kernels may read it and rebuilt when the tensor (held by
        weak reference), its version or its storage changes."""
        if bias is None:
            if self.bias_key != (None, relu):
                self.lib.nova_set_epilogue(self.h, None, relu)
                check("set_epilogue")
                self.bias_key = (None, relu)
                self.bias16 = None
                self.b_ref = None
            return
        key = (bias._version, bias.data_ptr(), bias.dtype, relu)
        ref = self.b_ref
        if ref is not None and ref() is bias and self.bias_key == key:
            return
        self.bias16 = bias.detach().to(torch.float16).contiguous()
        self.lib.nova_set_epilogue(self.h, ptr(self.bias16), relu)
        check("set_epilogue")
        self.bias_key = key
        self.b_ref = weakref.ref(bias)

    def set_layout(self, nhwc):
        """Activation layout of the next launches: 0 NCHW, 1 NHWC."""
        if nhwc != self.nhwc:
            self.lib.nova_set_layout(self.h, nhwc)
            check("set_layout")
            self.nhwc = nhwc

    def set_residual(self, residual):
        """Residual operand of the next launch (None: none)."""
        p = residual.data_ptr() if residual is not None else None
        if p != self.res_ptr:
            self.lib.nova_set_residual(self.h, p)
            self.res_ptr = p

    def set_stream(self, device):
        s = current_stream_ptr(device)
        if s != self.stream:
            self.lib.nova_set_stream(self.h, s)
            self.stream = s

    def set_weights(self, weight):
        # fp16 weights (a .half()'d module) go to the library as they are,
        # anything else as an fp32 contiguous copy; both give the same
        # transform. A temporary stays valid for the asynchronous transform
        # because both run on the current stream (the caching allocator is
        # stream-ordered).
        w = weight.detach()
        if w.dtype == torch.float16:
            w = w.contiguous()
            self.lib.nova_set_weights_f16(self.h, ptr(w), w.shape[0], w.shape[1])
        else:
            w = w.to(torch.float32).contiguous()
            self.lib.nova_set_weights(self.h, ptr(w), w.shape[0], w.shape[1])
        check("set_weights")

    def __del__(self):
        try:
            if self.h and not _exiting:
                self.lib.nova_destroy(self.h)
                self.h = None
        except Exception:
            pass


def _init_conv_parameters(mod, in_channels, out_channels, kernel_size, padding, bias):
    """Geometry and parameters shared by the NOVA modules: a float32
    ``weight`` [out, in, 3, 3] with ``nn.Conv2d``'s default initialisation and
    an optional zero ``bias`` (the constructor contract of
    /root/reference/nova_winograd/conv2d.py:168-181)."""
    assert kernel_size == 3, "Only 3x3 kernels supported"
    mod.in_channels, mod.out_channels, mod.padding = in_channels, out_channels, padding
    mod.weight = nn.Parameter(torch.empty(out_channels, in_channels, 3, 3))
    nn.init.kaiming_uniform_(mod.weight, a=math.sqrt(5))
    mod.register_parameter("bias", nn.Parameter(torch.zeros(out_channels)) if bias else None)


def _module_like(cls, conv):
    """A ``cls`` module with the geometry of ``nn.Conv2d`` ``conv`` and float32
    copies of its parameters, on conv's device (the ``from_conv2d`` contract,
    /root/reference/nova_winograd/conv2d.py:253-267). Only square 3x3,
    stride-1, numeric symmetric padding is representable."""
    assert conv.kernel_size == (3, 3), "Only 3x3 kernels supported"
    assert conv.stride == (1, 1), "Only stride=1 supported"
    assert not isinstance(conv.padding, str), "padding must be numeric"
    assert conv.padding[0] == conv.padding[1], "Only symmetric padding supported"
    mod = cls(conv.in_channels, conv.out_channels, kernel_size=3, padding=conv.padding[0],
              bias=conv.bias is not None).to(conv.weight.device)
    with torch.no_grad():
        for name in ("weight", "bias"):
            src = getattr(conv, name)
            if src is not None:
                getattr(mod, name).copy_(src.detach().float())
    return mod


def _conv_repr(mod):
    """``extra_repr`` text of the NOVA modules (the reference's wording)."""
    return (f"in_channels={mod.in_channels}, out_channels={mod.out_channels}, "
            f"kernel_size=3, padding={mod.padding}, tile=F(6,3), points=NOVA")


# ─────────────────────────────────────────────────────────────────────────
# torch.compile custom op (/root/reference/nova_winograd/conv2d.py:25-85)
# ─────────────────────────────────────────────────────────────────────────

_custom_op_registered = False
_op_lock = threading.Lock()
_OP_HANDLES = {}  # device index -> _Handle


def _op_handle(device):
    """One persistent handle per device for the custom op (the reference's op
    creates and destroys a handle, transforms the filter and synchronises
    twice per call). The filter transform is cached for the exact weight
    tensor and version last seen (held by weak reference)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    hd = _OP_HANDLES.get(idx)
    if hd is None:
        hd = _Handle()
        _OP_HANDLES[idx] = hd
    return hd


def _grad_input(go, weight, padding, dtype):
    return F.conv_transpose2d(go.float(), weight.float(), padding=padding).to(dtype)


def _grad_input_nova(holder, go, weight, padding, dtype):
    """dL/dx of a stride-1 3x3 convolution is itself a 3x3 convolution of
    dL/dy with the filter flipped in both spatial axes and its channel axes
    swapped, at padding 2 - padding -- so it runs on the NOVA forward path
    (fp16, the same tolerance class as the forward). Padding above 2 has no
    such form and falls back to PyTorch's fp32 transposed convolution."""
    pb = 2 - padding
    if pb < 0:
        return _grad_input(go, weight, padding, dtype)
    hd = _bwd_handle(holder)
    hd.set_stream(go.device)
    # the flipped filter is cached for this exact weight tensor (weak
    # reference: a freed tensor whose memory is reused can never match) at
    # this version and storage
    key = (weight.data_ptr(), weight._version, tuple(weight.shape), weight.dtype)
    ref = hd.key
    if not (ref is not None and ref[0]() is weight and ref[1] == key):
        hd.set_weights(weight.detach().flip(2, 3).transpose(0, 1))
        hd.key = (weakref.ref(weight), key)
    g16 = go.to(torch.float16).contiguous()
    B, K, Ho, Wo = g16.shape
    C = weight.shape[1]
    gi = torch.empty(B, C, Ho + 2 * pb - 2, Wo + 2 * pb - 2, dtype=torch.float16,
                     device=go.device)
    hd.lib.nova_forward(hd.h, ptr(g16), ptr(gi), B, Ho, Wo, pb)
    check("backward (grad input)")
    return gi.to(dtype)


def _bwd_handle(holder):
    """The handle a module (or the custom op's per-device holder) uses for
    its backward kernels: the flipped filter of grad input, and the
    workspace and stream of grad weight."""
    hd = getattr(holder, "_bwd_handle", None)
    if hd is None:
        hd = _Handle()
        holder._bwd_handle = hd
    return hd


def _grad_weight(holder, inp, go, weight, padding):
    """dL/dw on the HIP path (nova_weight_grad): the Winograd-domain
    products of the transformed input and the transformed output gradient,
    reduced over the tiles and mapped back through G, all in fp32 -- in place
    of the reference's per-sample fp32 unfold loop
    (/root/reference/nova_winograd/conv2d.py:121-147). The input is the fp16
    tensor the forward convolved, so this is the gradient of the forward as
    computed."""
    hd = _bwd_handle(holder)
    hd.set_stream(go.device)
    x16 = inp.detach().to(torch.float16).contiguous()
    g = go.detach()
    if g.dtype not in (torch.float16, torch.float32):
        g = g.float()
    g = g.contiguous()
    B, C, H, W = x16.shape
    K = weight.shape[0]
    gw = torch.empty(K, C, 3, 3, dtype=torch.float32, device=go.device)
    hd.lib.nova_weight_grad(hd.h, ptr(x16), ptr(g), ptr(gw), B, C, K, H, W, padding,
                            1 if g.dtype == torch.float32 else 0)
    check("backward (grad weight)")
    return gw.to(weight.dtype)


class _BackwardHandles:
    """Holder of a grad-input handle (``_bwd_handle``) for the custom op."""


_OP_BWD = {}  # device index -> _BackwardHandles


def _op_bwd_holder(device):
    idx = device.index if device.index is not None else torch.cuda.current_device()
    holder = _OP_BWD.get(idx)
    if holder is None:
        holder = _OP_BWD[idx] = _BackwardHandles()
    return holder


def _register_custom_op():
    """Register ``nova::winograd_conv2d(input, weight, padding, bias=None)``
    (the reference's op, /root/reference/nova_winograd/conv2d.py:25-85, with
    an optional bias added in the output epilogue) as a torch.library custom
    op, once per process."""
    global _custom_op_registered
    with _op_lock:
        if _custom_op_registered:
            return
        _custom_op_registered = True

    @torch.library.custom_op("nova::winograd_conv2d", mutates_args=())
    def nova_winograd_conv2d(input: torch.Tensor, weight: torch.Tensor, padding: int,
                             bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        require_gpu_tensor(input, "input")
        x = input.contiguous().to(torch.float16)
        B, _, H, W = x.shape
        _, _, H_out, W_out = compute_tiling(H, W, padding)
        out = torch.empty(B, weight.shape[0], H_out, W_out, dtype=torch.float16,
                          device=x.device)
        with _op_lock:  # the per-device handle is shared with nova_forward
            hd = _op_handle(x.device)
            hd.set_stream(x.device)
            hd.set_weights_cached(weight)
            hd.set_bias(bias)
            hd.set_residual(None)
            hd.set_layout(0)
            hd.lib.nova_forward(hd.h, ptr(x), ptr(out), B, H, W, padding)
            check("forward")
        return out

    @nova_winograd_conv2d.register_fake
    def _(input, weight, padding, bias=None):
        B, _, H, W = input.shape
        return input.new_empty(B, weight.shape[0], H + 2 * padding - 2, W + 2 * padding - 2,
                               dtype=torch.float16)

    # The backward is a custom op of its own: under torch.compile the
    # autograd formula is traced with fake tensors, which have no device
    # pointers, so the HIP calls must sit behind an op with a fake kernel.
    @torch.library.custom_op("nova::winograd_conv2d_backward", mutates_args=())
    def nova_winograd_conv2d_backward(grad_output: torch.Tensor, input: torch.Tensor,
                                      weight: torch.Tensor,
                                      padding: int) -> Tuple[torch.Tensor, torch.Tensor]:
        go = grad_output.contiguous()
        holder = _op_bwd_holder(go.device)
        with _op_lock:
            gi = _grad_input_nova(holder, go, weight, padding, input.dtype)
            gw = _grad_weight(holder, input, go, weight, padding)
        return gi, gw

    @nova_winograd_conv2d_backward.register_fake
    def _(grad_output, input, weight, padding):
        return torch.empty_like(input), torch.empty_like(weight)

    def _keep(ctx, inputs, output):
        input, weight, padding, bias = inputs
        ctx.save_for_backward(input, weight)
        ctx.padding = padding
        ctx.bias_dtype = None if bias is None else bias.dtype

    def _grads(ctx, grad_output):
        input, weight = ctx.saved_tensors
        gi, gw = torch.ops.nova.winograd_conv2d_backward(grad_output, input, weight, ctx.padding)
        gb = (None if ctx.bias_dtype is None
              else grad_output.float().sum(dim=(0, 2, 3)).to(ctx.bias_dtype))
        return gi, gw, None, gb

    nova_winograd_conv2d.register_autograd(_grads, setup_context=_keep)


# ─────────────────────────────────────────────────────────────────────────
# Autograd Function (/root/reference/nova_winograd/conv2d.py:92-147)
# ─────────────────────────────────────────────────────────────────────────

class NovaWinogradFunction(torch.autograd.Function):
    """HIP forward; backward: grad input through the HIP forward (flipped
    filter), grad weight through nova_weight_grad (fp32, Winograd domain),
    grad bias a channel sum."""

    @staticmethod
    def forward(ctx, input, weight, bias, padding, handle_holder):
        ctx.save_for_backward(input, weight, bias)
        ctx.padding = padding
        ctx.holder = handle_holder
        x = input.half().contiguous() if input.dtype != torch.float16 else input.contiguous()
        return handle_holder._run(x, bias)

    @staticmethod
    def backward(ctx, grad_output):
        input, weight, bias = ctx.saved_tensors
        padding = ctx.padding
        grad_input = grad_weight = grad_bias = None
        go = grad_output.contiguous()
        if ctx.needs_input_grad[0]:
            grad_input = _grad_input_nova(ctx.holder, go, weight, padding, input.dtype)
        if ctx.needs_input_grad[1]:
            grad_weight = _grad_weight(ctx.holder, input, go, weight, padding)
        if bias is not None and ctx.needs_input_grad[2]:
            grad_bias = go.float().sum(dim=(0, 2, 3)).to(bias.dtype)
        return grad_input, grad_weight, grad_bias, None, None


# ─────────────────────────────────────────────────────────────────────────
# NovaWinogradConv2d -- inference module
# ─────────────────────────────────────────────────────────────────────────

class NovaWinogradConv2d(nn.Module):
    """Drop-in replacement for nn.Conv2d using NOVA Winograd F(6,3)
    (/root/reference/nova_winograd/conv2d.py:154-273).

    Supports kernel_size=3, stride=1 only. Input must be float16. Weights are
    stored in float32 and transformed on first use and whenever they change.

    Args:
        in_channels:  Number of input channels.
        out_channels: Number of output channels.
        kernel_size:  Must be 3.
        padding:      Convolution padding (default 1).
        bias:         Whether to include bias (default False).
    """

    def __init__(self, in_channels, out_channels, kernel_size=3, padding=1, bias=False):
        super().__init__()
        _init_conv_parameters(self, in_channels, out_channels, kernel_size, padding, bias)
        self._handle = None
        self._weight_version = -1
        self._V_gemm = None
        self._M_gemm = None
        self._last_config = None
        self._tiling = None
        self._state = None

    # -- caches -------------------------------------------------------------
    def invalidate_weight_cache(self):
        """Force the filter transform to be rebuilt on the next forward (use
        after writing the weights through ``.data``, which PyTorch does not
        version)."""
        self._weight_version = -1
        self._state = None
        if self._handle is not None:
            self._handle.key = None
        bwd = getattr(self, "_bwd_handle", None)  # the flipped filter of the backward
        if bwd is not None:
            bwd.key = None

    def _apply(self, fn, *args, **kwargs):
        out = super()._apply(fn, *args, **kwargs)
        self.invalidate_weight_cache()
        self._V_gemm = self._M_gemm = None
        self._last_config = None
        self._state = None
        return out

    def _load_from_state_dict(self, *args, **kwargs):
        super()._load_from_state_dict(*args, **kwargs)
        self.invalidate_weight_cache()

    def _ensure_handle(self):
        """Create the handle and re-transform the filter if the weight changed."""
        if self._handle is None:
            self._handle = _Handle()
        hd = self._handle
        hd.set_stream(self.weight.device)
        key = _weight_key(self.weight)
        ref = hd.key
        if not (ref is not None and ref[0]() is self.weight and ref[1] == key):
            hd.set_weights(self.weight)
            hd.key = (weakref.ref(self.weight), key)
            self._weight_version = self.weight._version
            self._V_gemm = None
            self._M_gemm = None
            self._last_config = None

    def _ensure_workspace(self, batch, H, W):
        """Allocate the reference-sized workspace when the configuration
        changes (/root/reference/nova_winograd/conv2d.py:205-220). Layers
        served by the fused kernel need none."""
        config = (batch, H, W, self.padding)
        if self._last_config != config:
            nh, nw, H_out, W_out = compute_tiling(H, W, self.padding)
            BP = batch * nh * nw
            lib = self._handle.lib
            need = lib.nova_workspace_bytes(self._handle.h, batch, H, W, self.padding)
            check("workspace_bytes")
            device = self.weight.device
            if need > 0:
                self._V_gemm = torch.empty(64, self.in_channels, BP, dtype=torch.float16,
                                           device=device)
                self._M_gemm = torch.empty(64, self.out_channels, BP, dtype=torch.float16,
                                           device=device)
            else:
                self._V_gemm = self._M_gemm = None
            self._tiling = (nh, nw, H_out, W_out)
            self._last_config = config
        return self._tiling

    # -- forward ------------------------------------------------------------
    def _run(self, x, bias, residual=None):
        """Launch the HIP path on a contiguous (NCHW) or channels-last (NHWC)
        fp16 input; returns fp16 in the same memory format."""
        require_gpu_tensor(x, "input")
        B, C, H, W = x.shape
        nhwc = _is_nhwc(x)
        if C != self.in_channels:
            raise ValueError(f"expected {self.in_channels} input channels, got {C}")
        self._ensure_handle()
        nh, nw, H_out, W_out = self._ensure_workspace(B, H, W)
        hd = self._handle
        hd.set_bias(bias)
        fmt = torch.channels_last if nhwc else torch.contiguous_format
        if residual is not None:
            require_gpu_tensor(residual, "residual")
            if (residual.dtype != torch.float16 or not residual.is_contiguous(memory_format=fmt)
                    or tuple(residual.shape) != (B, self.out_channels, H_out, W_out)):
                raise ValueError("residual must be a float16 tensor of the output's shape "
                                 f"{(B, self.out_channels, H_out, W_out)} in the input's "
                                 "memory format")
        hd.set_layout(1 if nhwc else 0)
        hd.set_residual(residual)
        output = torch.empty(B, self.out_channels, H_out, W_out, dtype=torch.float16,
                             device=x.device, memory_format=fmt)
        V, M = self._V_gemm, self._M_gemm
        hd.lib.nova_forward_workspace(
            hd.h, x.data_ptr(), output.data_ptr(),
            V.data_ptr() if V is not None else None,
            M.data_ptr() if M is not None else None,
            B, H, W, self.padding, nh, nw,
        )
        check("forward")
        return output

    def forward(self, x, residual=None):
        """y = conv(x) (+ bias). ``residual`` (an extension): a float16
        tensor of the output's shape added after the bias, with the rounding
        of a separate ``y + residual``."""
        # Fast path: the same input shape, weight and bias objects at the same
        # versions, and the same current stream as the previous call -- only
        # the output allocation and the launch remain.
        # The parameters are read from ``_parameters`` (nn.Module attribute
        # lookup of a parameter costs several times a dict read); a bias
        # entry that was removed reads as _MISSING and takes the full path.
        st = self._state
        if st is not None and residual is None:
            p = self._parameters
            w, b = p.get("weight"), p.get("bias", _MISSING)
            if (x.shape == st[0] and w is st[1] and w._version == st[2]
                    and w.data_ptr() == st[13] and b is st[3]
                    and (b is None or (b._version, b.data_ptr()) == st[4])
                    and x.dtype is torch.float16
                    and x.is_contiguous() and x.get_device() == st[6]
                    and _raw_stream(st[6]) == st[7]):
                # an output of the input's shape (C == K, pad 1) is allocated
                # like x: the cheapest allocation call; else new_empty
                out = torch.empty_like(x) if st[14] else x.new_empty(st[8])
                st[9](st[10], x.data_ptr(), out.data_ptr(), *st[11])
                if st[12] is not None:  # ctypes launch: read (and clear) the error code
                    st[12]("forward")
                return out
        assert x.dtype == torch.float16, f"Input must be float16, got {x.dtype}"
        assert x.is_contiguous() or _is_nhwc(x), \
            "Input must be contiguous (NCHW) or channels_last"
        assert x.dim() == 4 and x.shape[1] == self.in_channels
        out = self._run(x, self.bias, residual)
        if residual is None and x.is_contiguous():
            self._remember(x)
        else:
            # the next call resets the residual / layout on the full path
            self._state = None
        return out

    def _remember(self, x):
        """Record what the fast path of ``forward`` checks and replays. The
        weight and bias objects are held, so their identities cannot be
        reused by other tensors while the record exists."""
        hd = self._handle
        B, C, H, W = x.shape
        nh, nw, H_out, W_out = self._tiling
        V, M = self._V_gemm, self._M_gemm
        w, b = self.weight, self.bias
        idx = x.device.index if x.device.index is not None else torch.cuda.current_device()
        fast = _fastcall(hd.lib)
        self._state = (
            x.shape, w, w._version, b, None if b is None else (b._version, b.data_ptr()),
            x.device, idx,
            hd.stream, (B, self.out_channels, H_out, W_out),
            fast if fast is not None else hd.lib.nova_forward_workspace,
            hd.h,
            (V.data_ptr() if V is not None else None, M.data_ptr() if M is not None else None,
             B, H, W, self.padding, nh, nw),
            None if fast is not None else check,
            w.data_ptr(),
            (B, self.out_channels, H_out, W_out) == tuple(x.shape),
        )

    @classmethod
    def from_conv2d(cls, conv):
        """Create from an existing nn.Conv2d
        (/root/reference/nova_winograd/conv2d.py:253-267)."""
        mod = _module_like(cls, conv)
        mod.invalidate_weight_cache()
        return mod

    def extra_repr(self):
        return _conv_repr(self)


# ─────────────────────────────────────────────────────────────────────────
# NovaWinogradConv2dTrainable (/root/reference/nova_winograd/conv2d.py:280-293)
# ─────────────────────────────────────────────────────────────────────────

class NovaWinogradConv2dTrainable(NovaWinogradConv2d):
    """NOVA conv with backward support: HIP forward, grad input and grad
    weight."""

    def forward(self, x):
        if not x.is_contiguous():
            x = x.contiguous()
        if x.dtype != torch.float16:
            x = x.half()
        assert x.shape[1] == self.in_channels
        return NovaWinogradFunction.apply(x, self.weight, self.bias, self.padding, self)


# ─────────────────────────────────────────────────────────────────────────
# NovaWinogradConv2dCompilable (interface of
# /root/reference/nova_winograd/conv2d.py:300-344)
# ─────────────────────────────────────────────────────────────────────────

class NovaWinogradConv2dCompilable(nn.Module):
    """The convolution as one traceable graph node: ``forward`` is a single
    call of the custom op ``torch.ops.nova.winograd_conv2d`` with the bias
    passed in, so ``torch.compile(fullgraph=True)`` sees no Python control
    flow, shapes come from the op's fake kernel, gradients from its autograd
    formula, and the bias is added in the kernels' output epilogue (rounded
    like the reference's separate ``out + bias.half()``)."""

    def __init__(self, in_channels, out_channels, kernel_size=3, padding=1, bias=False):
        super().__init__()
        _register_custom_op()
        _init_conv_parameters(self, in_channels, out_channels, kernel_size, padding, bias)

    def forward(self, x):
        return torch.ops.nova.winograd_conv2d(x, self.weight, self.padding, self.bias)

    @classmethod
    def from_conv2d(cls, conv):
        return _module_like(cls, conv)

    def extra_repr(self):
        return _conv_repr(self) + ", compilable=True"
