"""ctypes bridge to libnova_winograd.so (the gfx950 HIP library).

Mirrors the reference's bridge (/root/reference/nova_winograd/ops.py:1-176):
same library name and search order, same functions (``get_lib``, ``ptr``,
``compute_tiling``, ``nova_forward``) and the same C signatures. Differences:

* loading the library does not initialise the GPU, so host-only entry points
  (``compute_tiling``) work on a machine without one; every entry point that
  touches device memory checks for a ROCm device and raises otherwise -- there
  is no CPU fallback;
* the library reports errors through ``nova_get_last_error`` instead of
  exiting the process; :func:`check` turns them into ``RuntimeError``;
* launches follow PyTorch's current stream (``nova_set_stream``).
"""

import ctypes
import os
import threading

import torch

_lib = None
_lib_lock = threading.Lock()
_LIB_NAME = "libnova_winograd.so"

_vp = ctypes.c_void_p
_i = ctypes.c_int
_ip = ctypes.POINTER(ctypes.c_int)

# name -> (restype, argtypes). The first twelve are the reference's
# (/root/reference/nova_winograd/ops.py:66-114); the rest are this library's.
_SIGNATURES = {
    "nova_create": (_vp, []),
    "nova_destroy": (None, [_vp]),
    "nova_set_weights": (None, [_vp, _vp, _i, _i]),
    "nova_forward": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "nova_forward_workspace": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i]),
    "nova_compute_tiling": (None, [_i, _i, _i, _ip, _ip, _ip, _ip]),
    "nova_filter_transform": (None, [_vp, _vp, _i, _i]),
    "nova_input_transform": (None, [_vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i]),
    "nova_output_transform": (None, [_vp, _vp, _i, _i, _i, _i, _i, _i, _i]),
    "nova_get_K": (_i, [_vp]),
    "nova_get_C": (_i, [_vp]),
    "nova_get_U_gemm": (_vp, [_vp]),
    # reference fused C-API (/root/reference/csrc/nova_winograd_fused.hip:619-652)
    "nova_fused_create": (_vp, []),
    "nova_fused_destroy": (None, [_vp]),
    "nova_fused_set_weights": (None, [_vp, _vp, _i, _i]),
    "nova_fused_forward": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "nova_fused_compute_tiling": (None, [_i, _i, _i, _ip, _ip, _ip, _ip]),
    # extensions
    "nova_get_last_error": (_i, []),
    "nova_get_last_error_message": (ctypes.c_char_p, []),
    "nova_set_stream": (None, [_vp, _vp]),
    "nova_set_path": (None, [_vp, _i]),
    "nova_set_window_bytes": (None, [_vp, ctypes.c_longlong]),
    "nova_set_epilogue": (None, [_vp, _vp, _i]),
    "nova_set_weights_f16": (None, [_vp, _vp, _i, _i]),
    "nova_set_residual": (None, [_vp, _vp]),
    "nova_set_layout": (None, [_vp, _i]),
    "nova_get_last_path": (_i, [_vp]),
    "nova_workspace_bytes": (ctypes.c_longlong, [_vp, _i, _i, _i, _i]),
    "nova_forward_noalloc": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "nova_weight_grad": (None, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i]),
    "nova_profile_enable": (None, [_vp, _i]),
    "nova_profile_read": (_i, [_vp, ctypes.POINTER(ctypes.c_double),
                               ctypes.POINTER(ctypes.c_longlong)]),
    "nova_profile_replay": (ctypes.c_double, [_vp, _i, _i]),
    "nova_profile_kernel_name": (ctypes.c_char_p, [_vp, _i]),
    "nova_version": (ctypes.c_char_p, []),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def _find_lib():
    """Locate the shared library: package ``lib/`` first, then the cwd
    (same order as /root/reference/nova_winograd/ops.py:16-28)."""
    candidates = [
        os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", _LIB_NAME),
        os.path.join(os.getcwd(), _LIB_NAME),
    ]
    for path in candidates:
        if os.path.exists(path):
            return path
    raise FileNotFoundError(
        f"Cannot find {_LIB_NAME}. Build it with: make -C nova-wino-amd_amd "
        f"(or python -c 'import __graft_entry__ as g; g.build()')\nSearched: {candidates}"
    )


def _ensure_lib():
    """Load the library once per process and declare every signature."""
    global _lib
    if _lib is not None:
        return
    with _lib_lock:
        if _lib is not None:
            return
        lib = ctypes.CDLL(_find_lib(), mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib


def get_lib():
    """Get the loaded ctypes library handle."""
    _ensure_lib()
    return _lib


def lib_path():
    """Filesystem path of the loaded library."""
    return _find_lib()


def ptr(tensor):
    """Raw device pointer of a tensor (as the reference's ``ptr``)."""
    return ctypes.c_void_p(tensor.data_ptr())


def check(where=""):
    """Raise RuntimeError if the library recorded an error on this thread."""
    lib = get_lib()
    code = lib.nova_get_last_error()
    if code:
        msg = lib.nova_get_last_error_message().decode(errors="replace")
        raise RuntimeError(f"nova_winograd{(' ' + where) if where else ''}: {msg} (code {code})")


def require_gpu_tensor(t, name="input"):
    """The product path runs only on a ROCm GPU; fail loudly otherwise."""
    if not t.is_cuda:
        raise RuntimeError(
            f"nova_winograd: {name} is on {t.device}; NOVA Winograd runs only on a ROCm GPU "
            "(no CPU fallback)"
        )


_raw_stream = torch._C._cuda_getCurrentRawStream  # device index -> hipStream_t (int)


def current_stream_ptr(device):
    """Raw hipStream_t of torch's current stream on ``device`` (an int)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return _raw_stream(idx)


def compute_tiling(H, W, pad):
    """Tiling parameters (nh, nw, H_out, W_out) by the reference's law
    (/root/reference/csrc/nova_winograd.hip:617-631): nh = ceil((Ho-1)/6)+1."""
    _ensure_lib()
    nh, nw, H_out, W_out = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _lib.nova_compute_tiling(
        H, W, pad,
        ctypes.byref(nh), ctypes.byref(nw), ctypes.byref(H_out), ctypes.byref(W_out),
    )
    return nh.value, nw.value, H_out.value, W_out.value


def nova_forward(input_fp16, weight_fp32, padding=1, bias=None, relu=False, residual=None):
    """Functional API: NOVA Winograd F(6,3) forward pass
    (/root/reference/nova_winograd/ops.py:147-176).

    Args:
        input_fp16:  [B, C, H, W] float16 tensor on GPU.
        weight_fp32: [K, C, 3, 3] float32 tensor on GPU (float16 is accepted
                     too, as an extension, and gives the same result as its
                     float32 copy).
        padding:     Convolution padding (default 1).
        bias:        optional [K] tensor on GPU, added in the output transform
                     with the rounding of ``output + bias.half()`` (an
                     extension: the reference has no bias here).
        relu:        clamp negative outputs to zero in the same pass
                     (extension).
        residual:    optional float16 tensor of the output's shape, added
                     after the bias and before the ReLU with the rounding of a
                     separate ``output + residual`` (extension).

    Returns:
        output: [B, K, H_out, W_out] float16 tensor on GPU.

    Unlike the reference (a handle created, the filter transformed and the
    device synchronised twice per call), it runs on one persistent handle per
    device and transforms the filter only for a new weight tensor or a new
    version of it; all work is ordered on PyTorch's current stream, so no
    device-wide synchronisation is needed around it.
    """
    _ensure_lib()
    require_gpu_tensor(input_fp16, "input")
    require_gpu_tensor(weight_fp32, "weight")
    assert input_fp16.dtype == torch.float16
    assert weight_fp32.dtype in (torch.float32, torch.float16)
    nhwc = (input_fp16.dim() == 4 and not input_fp16.is_contiguous()
            and input_fp16.is_contiguous(memory_format=torch.channels_last))
    assert (input_fp16.is_contiguous() or nhwc) and weight_fp32.is_contiguous()
    assert input_fp16.dim() == 4 and weight_fp32.dim() == 4
    assert tuple(weight_fp32.shape[1:]) == (input_fp16.shape[1], 3, 3)

    B, C, H, W = input_fp16.shape
    K = weight_fp32.shape[0]
    nh, nw, H_out, W_out = compute_tiling(H, W, padding)
    fmt = torch.channels_last if nhwc else torch.contiguous_format
    output = torch.empty(B, K, H_out, W_out, dtype=torch.float16, device=input_fp16.device,
                         memory_format=fmt)

    if residual is not None:
        require_gpu_tensor(residual, "residual")
        assert residual.dtype == torch.float16 and residual.is_contiguous(memory_format=fmt)
        assert tuple(residual.shape) == (B, K, H_out, W_out)
    if bias is not None:
        require_gpu_tensor(bias, "bias")
        assert bias.numel() == K
    # One persistent handle per device, shared with the torch.compile op; the
    # filter transform is cached for the exact weight tensor and version last
    # used (the reference creates a handle, transforms the filter and
    # synchronises twice per call, ops.py:166-174).
    from nova_winograd.conv2d import _op_handle, _op_lock

    with _op_lock:
        hd = _op_handle(input_fp16.device)
        hd.set_stream(input_fp16.device)
        hd.set_weights_cached(weight_fp32)
        hd.set_bias(bias, 1 if relu else 0)  # keeps an fp16 copy of bias
        hd.set_residual(residual)
        hd.set_layout(1 if nhwc else 0)
        try:
            _lib.nova_forward(hd.h, ptr(input_fp16), ptr(output), B, H, W, padding)
            check("forward")
        finally:
            hd.set_residual(None)
    return output
