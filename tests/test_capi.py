"""The C-ABI library on the CPU: it loads, exports every symbol the public
header declares (with the reference's 12 among them), and its host-side logic
(tiling, handle lifecycle, argument validation, error reporting) works without
a GPU. No kernel is launched here."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nova_winograd.h")

REFERENCE_SYMBOLS = [  # /root/reference/nova_winograd/ops.py:66-114
    "nova_create", "nova_destroy", "nova_set_weights", "nova_forward", "nova_forward_workspace",
    "nova_compute_tiling", "nova_filter_transform", "nova_input_transform",
    "nova_output_transform", "nova_get_K", "nova_get_C", "nova_get_U_gemm",
]


@pytest.fixture(scope="module")
def lib():
    from nova_winograd.ops import get_lib

    return get_lib()


def header_symbols():
    text = open(HEADER).read()
    return re.findall(r"NOVA_API\s+[\w\s\*]+?\b(nova_\w+)\s*\(", text)


def test_header_declares_reference_symbols():
    syms = header_symbols()
    for s in REFERENCE_SYMBOLS:
        assert s in syms
    assert len(syms) == len(set(syms))


def test_library_exports_every_header_symbol(lib):
    from nova_winograd.ops import EXPORTED_SYMBOLS, lib_path

    raw = ctypes.CDLL(lib_path())
    for s in header_symbols():
        assert hasattr(raw, s), s
    assert set(header_symbols()) == set(EXPORTED_SYMBOLS)


def test_compute_tiling_matches_reference_law(lib):
    from nova_winograd import compute_tiling

    for pad in (0, 1, 2):
        for H in range(3, 130):
            nh, nw, Ho, Wo = compute_tiling(H, H + 3, pad)
            assert Ho == H + 2 * pad - 2 and Wo == H + 3 + 2 * pad - 2
            assert nh == -(-(Ho - 1) // 6) + 1
            assert nw == -(-(Wo - 1) // 6) + 1
    assert compute_tiling(56, 56, 1) == (11, 11, 56, 56)
    assert compute_tiling(7, 7, 1) == (2, 2, 7, 7)


def test_handle_lifecycle_and_errors(lib):
    assert lib.nova_get_last_error() == 0
    h = lib.nova_create()
    assert h
    assert lib.nova_get_K(h) == 0 and lib.nova_get_C(h) == 0 and not lib.nova_get_U_gemm(h)
    lib.nova_set_weights(h, None, 64, 64)
    assert lib.nova_get_last_error() == 1
    assert b"bad arguments" in lib.nova_get_last_error_message()
    assert lib.nova_get_last_error() == 0  # cleared
    lib.nova_forward(h, 1, 2, 1, 8, 8, 1)  # weights never set: refused before any GPU work
    assert lib.nova_get_last_error() == 2
    lib.nova_set_path(h, 8)
    assert lib.nova_get_last_error() == 1
    lib.nova_set_path(h, 1)
    assert lib.nova_get_last_error() == 0
    lib.nova_forward(h, 1, 2, 1, 1, 1, 0)  # empty output (Ho = -1)
    assert lib.nova_get_last_error() == 1
    lib.nova_destroy(h)
    lib.nova_destroy(None)
    assert lib.nova_get_last_error() == 0
    assert lib.nova_get_K(None) == 0  # NULL handle is reported, not dereferenced
    assert lib.nova_get_last_error() == 1
    assert lib.nova_version().startswith(b"nova-winograd")


def test_entry_points_reject_bad_shapes_without_gpu(lib):
    lib.nova_input_transform(1, 2, 1, 4, 8, 8, 1, 2, 2, 3)  # BP < B*nh*nw
    assert lib.nova_get_last_error() == 1
    lib.nova_output_transform(1, 2, 1, 4, 8, 8, 2, 2, 3)
    assert lib.nova_get_last_error() == 1
    lib.nova_filter_transform(None, None, 4, 4)
    assert lib.nova_get_last_error() == 1


def test_fastcall_binding_raises_library_errors(lib):
    """The CPython fast-call binding of nova_forward_workspace (the module's
    cached path) reports library errors as RuntimeError; exercised on a handle
    without weights, which the library refuses before any GPU work."""
    import ctypes

    from nova_winograd import _nova_call
    from nova_winograd.conv2d import _fastcall

    fwd = _fastcall(lib)
    assert fwd is _nova_call.forward_ws
    h = lib.nova_create()
    try:
        with pytest.raises(RuntimeError, match="weights"):
            fwd(h, 1, 2, None, None, 1, 8, 8, 1, 2, 2)
        assert lib.nova_get_last_error() == 0  # the binding consumed the error
        with pytest.raises(TypeError):
            fwd(h, 1, 2)
    finally:
        lib.nova_destroy(h)
    with pytest.raises(ValueError):
        _nova_call.bind(0, 0, 0)
    assert ctypes.cast(lib.nova_forward_workspace, ctypes.c_void_p).value


def test_oversized_filter_rejected_before_device_work(lib):
    """The GEMM kernels address the transformed filter U (64*K*pad8(C) fp16
    values) with 32-bit byte offsets: a layer whose U reaches 2^31 bytes is
    refused by nova_set_weights before any allocation or launch (the pointer
    below is never dereferenced)."""
    h = lib.nova_create()
    try:
        for K, C in ((4096, 4096), (4200, 4200), (1 << 20, 64)):
            lib.nova_set_weights(h, 16, K, C)
            assert lib.nova_get_last_error() == 1, (K, C)
            assert b"2^31" in lib.nova_get_last_error_message()
            assert lib.nova_get_K(h) == 0 and not lib.nova_get_U_gemm(h)
        lib.nova_forward(h, 1, 2, 1, 8, 8, 1)  # still not initialized
        assert lib.nova_get_last_error() == 2
    finally:
        lib.nova_destroy(h)
