"""CPU oracle for the NOVA F(6,3) path -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg may
import this module; the product package never does. It wraps the C
restatement in ``nova_oracle.c`` (see that file's header for the canonical
arithmetic and the reference lines each function follows) with numpy arrays:

* fp16 tensors are numpy ``float16`` arrays (passed as their uint16 bits);
* layouts are the reference's GEMM layouts (``U[64][C][K]``, ``V[64][BP][C]``,
  ``M[64][BP][K]``), so results compare directly with the reference-layout
  entry points of the C-ABI (``nova_filter_transform``,
  ``nova_input_transform``, ``nova_output_transform``).

Pinning (tests/test_oracle.py): exact-table derivation, exact-arithmetic
Winograd identity, fp16 conversion vs numpy, tiling brute force, special
inputs (zero, delta, constant, linearity), error level vs fp64 direct conv,
golden fixtures under tests/golden/.
"""

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libnova_oracle.so")
REF_LIB_PATH = os.path.join(_HERE, "_ref", "libnova_winograd_ref.so")
_lib = None

_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_ip = ctypes.POINTER(ctypes.c_int)
_c_int = ctypes.c_int
_c_long = ctypes.c_long


def build():
    """Compile the oracle library (gcc, seconds)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    L = ctypes.CDLL(_LIB_PATH)
    L.nvo_set_threads.argtypes = [_c_int]
    L.nvo_get_threads.restype = _c_int
    L.nvo_tables.argtypes = [_f32p] * 5
    L.nvo_f32_to_f16.argtypes = [_f32p, _u16p, _c_long]
    L.nvo_f64_to_f16.argtypes = [_f64p, _u16p, _c_long]
    L.nvo_f16_to_f32.argtypes = [_u16p, _f32p, _c_long]
    L.nvo_tiling.argtypes = [_c_int, _c_int, _c_int, _ip, _ip, _ip, _ip]
    L.nvo_filter.argtypes = [_f32p, _c_int, _c_int, _u16p]
    L.nvo_input.argtypes = [_u16p] + [_c_int] * 7 + [_u16p]
    L.nvo_gemm.argtypes = [_u16p, _u16p, _c_int, _c_int, _c_long, _u16p,
                           ctypes.c_void_p]
    L.nvo_output.argtypes = [_u16p] + [_c_int] * 6 + [_u16p]
    L.nvo_conv.argtypes = [_u16p, _f32p] + [_c_int] * 6 + [_u16p]
    L.nvo_conv.restype = _c_int
    L.nvo_direct.argtypes = [_u16p, _f32p] + [_c_int] * 6 + [_f64p]
    L.nvo_weight_grad.argtypes = [_u16p, _f32p] + [_c_int] * 6 + [_f64p]
    _lib = L
    return L


def set_threads(n):
    lib().nvo_set_threads(int(n))


def get_threads():
    return lib().nvo_get_threads()


def _h(a):
    a = np.ascontiguousarray(a, dtype=np.float16)
    return a.view(np.uint16)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def tables():
    """(A 6x8, B 8x8, G 8x3) fp32 and (Ah, Bh) fp16-rounded, as fp32 arrays."""
    A = np.zeros((6, 8), np.float32)
    B = np.zeros((8, 8), np.float32)
    G = np.zeros((8, 3), np.float32)
    Ah = np.zeros((6, 8), np.float32)
    Bh = np.zeros((8, 8), np.float32)
    lib().nvo_tables(A, B, G, Ah, Bh)
    return A, B, G, Ah, Bh


def f32_to_f16(a):
    a = _f32(a)
    out = np.empty(a.shape, np.uint16)
    lib().nvo_f32_to_f16(a.reshape(-1), out.reshape(-1), a.size)
    return out.view(np.float16)


def f64_to_f16(a):
    a = np.ascontiguousarray(a, dtype=np.float64)
    out = np.empty(a.shape, np.uint16)
    lib().nvo_f64_to_f16(a.reshape(-1), out.reshape(-1), a.size)
    return out.view(np.float16)


def tiling(H, W, pad):
    """(nh, nw, Ho, Wo) by the reference's tiling law."""
    v = [ctypes.c_int() for _ in range(4)]
    lib().nvo_tiling(H, W, pad, *[ctypes.byref(x) for x in v])
    return tuple(x.value for x in v)


def filter_transform(w):
    """w fp32 [K,C,3,3] -> U fp16 [64, C, K]."""
    w = _f32(w)
    K, C = w.shape[:2]
    U = np.empty((64, C, K), np.uint16)
    lib().nvo_filter(w.reshape(-1), K, C, U.reshape(-1))
    return U.view(np.float16)


def input_transform(x, pad, nh, nw):
    """x fp16 [B,C,H,W] -> V fp16 [64, B*nh*nw, C]."""
    xb = _h(x)
    B, C, H, W = x.shape
    BP = B * nh * nw
    V = np.empty((64, BP, C), np.uint16)
    lib().nvo_input(xb.reshape(-1), B, C, H, W, pad, nh, nw, V.reshape(-1))
    return V.view(np.float16)


def batched_gemm(U, V, with_abs=False):
    """U fp16 [64,C,K], V fp16 [64,BP,C] -> M fp16 [64,BP,K] (correctly
    rounded), and optionally sum|U||V| fp32 [64,BP,K] for error bounds."""
    Ub, Vb = _h(U), _h(V)
    _, C, K = U.shape
    BP = V.shape[1]
    M = np.empty((64, BP, K), np.uint16)
    Mabs = np.empty((64, BP, K), np.float32) if with_abs else None
    lib().nvo_gemm(Ub.reshape(-1), Vb.reshape(-1), K, C, BP, M.reshape(-1),
                   Mabs.ctypes.data if with_abs else None)
    M = M.view(np.float16)
    return (M, Mabs) if with_abs else M


def output_transform(M, B, Ho, Wo, nh, nw):
    """M fp16 [64, BP, K] -> y fp16 [B, K, Ho, Wo]."""
    Mb = _h(M)
    K = M.shape[2]
    y = np.zeros((B, K, Ho, Wo), np.uint16)
    lib().nvo_output(Mb.reshape(-1), B, K, Ho, Wo, nh, nw, y.reshape(-1))
    return y.view(np.float16)


def conv2d(x, w, pad=1):
    """Whole NOVA path, reference tiling: x fp16 [B,C,H,W], w fp32 [K,C,3,3]."""
    xb = _h(x)
    w = _f32(w)
    B, C, H, W = x.shape
    K = w.shape[0]
    nh, nw, Ho, Wo = tiling(H, W, pad)
    y = np.empty((B, K, Ho, Wo), np.uint16)
    rc = lib().nvo_conv(xb.reshape(-1), w.reshape(-1), B, C, K, H, W, pad, y.reshape(-1))
    if rc != 0:
        raise ValueError(f"oracle conv2d failed ({rc})")
    return y.view(np.float16)


def direct_conv2d(x, w, pad=1):
    """Truth: fp64 direct correlation of fp16 x with fp32 w."""
    xb = _h(x)
    w = _f32(w)
    B, C, H, W = x.shape
    K = w.shape[0]
    Ho, Wo = H + 2 * pad - 2, W + 2 * pad - 2
    y = np.empty((B, K, Ho, Wo), np.float64)
    lib().nvo_direct(xb.reshape(-1), w.reshape(-1), B, C, K, H, W, pad, y.reshape(-1))
    return y


def weight_grad(x, dy, pad=1):
    """Truth for the weight gradient: fp64 accumulation of
    dy[n,k,oh,ow] * x[n,c,oh-pad+a,ow-pad+b] for fp16 x [B,C,H,W] and fp32 dy
    [B,K,Ho,Wo]; returns fp64 [K,C,3,3]."""
    xb = _h(x)
    dy = _f32(dy)
    B, C, H, W = x.shape
    K = dy.shape[1]
    gw = np.empty((K, C, 3, 3), np.float64)
    lib().nvo_weight_grad(xb.reshape(-1), dy.reshape(-1), B, C, K, H, W, pad, gw.reshape(-1))
    return gw


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def max_abs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))
