"""Parity of the gfx950 HIP path with the CPU oracle, stage by stage and end
to end, through the C-ABI.

Bars:
* filter, input and output transforms: bit-exact (same fp32 FMA chains and
  fp16 rounding points as the oracle);
* Winograd-domain GEMM: |M_gpu - M_oracle| <= 2*C*2^-24*sum|U||V| + 1 ulp16,
  the fp32 summation bound for any accumulation order (the oracle's M is the
  correctly rounded one);
* whole path: rel-L2(gpu, oracle) <= 5e-3, max-abs <= 0.25 at unit-scale
  outputs; against the fp64 direct convolution the GPU error is no worse than
  1.05x the oracle's rel-L2 and 1.25x its max-abs; zero NaN/Inf.
"""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _lib():
    from nova_winograd.ops import get_lib

    return get_lib()


def _check():
    from nova_winograd.ops import check

    check()


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def assert_same_bits(got, want, what=""):
    """Bit-exact comparison of two fp16 arrays with a compact report."""
    g = np.ascontiguousarray(got).view(np.uint16)
    w = np.ascontiguousarray(want).view(np.uint16)
    assert g.shape == w.shape, (g.shape, w.shape)
    bad = np.flatnonzero(g != w)
    if bad.size:
        first = bad[:6]
        idx = [tuple(int(v) for v in t) for t in zip(*np.unravel_index(first, g.shape))]
        gv = g.flat[first].view(np.float16).astype(np.float32)
        wv = w.flat[first].view(np.float16).astype(np.float32)
        raise AssertionError(
            f"{what}: {bad.size}/{g.size} elements differ; first at {idx}: "
            f"got {gv.tolist()} want {wv.tolist()} (bits {g.flat[first].tolist()} vs "
            f"{w.flat[first].tolist()})")


def _ulp16(x):
    a = np.abs(x.astype(np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 2.0 ** (e - 10)


def _kaiming(K, C, gen=None):
    w = torch.empty(K, C, 3, 3)
    torch.nn.init.kaiming_normal_(w, mode="fan_in", nonlinearity="relu", generator=gen)
    return w


FILTER_CASES = [(64, 64), (48, 192), (8, 3), (128, 256), (40, 24), (1, 1)]


@pytest.mark.parametrize("K,C", FILTER_CASES)
def test_filter_transform_bitexact(oracle, K, C):
    print(f"[filter] K={K} C={C}", flush=True)
    w = torch.randn(K, C, 3, 3) * 0.7
    U = torch.empty(64, C, K, dtype=torch.float16, device=DEV)
    _lib().nova_filter_transform(w.to(DEV).data_ptr(), U.data_ptr(), K, C)
    _check()
    ref = oracle.filter_transform(w.numpy())
    assert_same_bits(_u16(U), ref, f"U K={K} C={C}")


# Small problems run the lane-parallel kernel, large ones (the last two: a
# tile-block grid of 256 workgroups or more) the tile-block kernel.
INPUT_CASES = [
    (1, 64, 56, 56, 1), (2, 3, 13, 13, 1), (1, 128, 28, 28, 1), (1, 16, 7, 7, 1),
    (1, 24, 14, 9, 0), (1, 8, 11, 11, 2), (3, 72, 20, 17, 1), (1, 130, 5, 5, 1),
    (8, 64, 56, 56, 1), (12, 130, 27, 29, 1),
]


@pytest.mark.parametrize("B,C,H,W,pad", INPUT_CASES)
def test_input_transform_bitexact(oracle, B, C, H, W, pad):
    print(f"[input] B={B} C={C} H={H} W={W} pad={pad}", flush=True)
    x = torch.randn(B, C, H, W).half()
    nh, nw, Ho, Wo = oracle.tiling(H, W, pad)
    BP = B * nh * nw
    V = torch.full((64, BP, C), float("nan"), dtype=torch.float16, device=DEV)
    _lib().nova_input_transform(x.to(DEV).data_ptr(), V.data_ptr(), B, C, H, W, pad, nh, nw, BP)
    _check()
    ref = oracle.input_transform(x.numpy(), pad, nh, nw)
    assert_same_bits(_u16(V), ref, "V")


# Output: the lane-parallel kernel below 256 tile-block workgroups, and for
# an odd row pitch on images at most two tiles wide below 640 ((16, 512, 7,
# 7)); the tile-block kernel for (8, 64, 56, 56) and, odd rows, (12, 130, 27,
# 29) and (32, 130, 27, 29); the image-block kernel (whole images per
# workgroup, 16-byte span stores) for (32, 256, 14, 14) (32 channels per
# workgroup, 16 reference tiles per image, dead ones included), (32, 512, 7,
# 7) (64, odd rows) and (32, 200, 14, 14) (16 channels, a partial last
# channel block).
OUTPUT_CASES = [(1, 64, 56, 56), (2, 48, 14, 14), (1, 130, 7, 9), (3, 8, 13, 11), (1, 16, 1, 1),
                (8, 64, 56, 56), (12, 130, 27, 29), (16, 512, 7, 7), (32, 130, 27, 29),
                (32, 256, 14, 14), (32, 512, 7, 7), (32, 200, 14, 14)]


@pytest.mark.parametrize("B,K,Ho,Wo", OUTPUT_CASES)
def test_output_transform_bitexact(oracle, B, K, Ho, Wo):
    print(f"[output] B={B} K={K} Ho={Ho} Wo={Wo}", flush=True)
    # reference tiling for pad=1 (H = Ho)
    nh, nw, _, _ = oracle.tiling(Ho, Wo, 1)
    BP = B * nh * nw
    M = (torch.randn(64, BP, K) * 3).half()
    y = torch.full((B, K, Ho, Wo), float("nan"), dtype=torch.float16, device=DEV)
    _lib().nova_output_transform(M.to(DEV).data_ptr(), y.data_ptr(), B, K, Ho, Wo, nh, nw, BP)
    _check()
    ref = oracle.output_transform(M.numpy(), B, Ho, Wo, nh, nw)
    assert_same_bits(_u16(y), ref, "y")


# GEMM shapes by tile kernel: at most 32 tiles first (the operand-block
# kernel: its V is in blocks, so only M is read back; the product-layout
# register-direct kernel it replaces is compared with it bit for bit in
# test_gpu_gemv_blocks.py), small grids (64 x 64), larger BP with K, Cp <= 128 (several
# bp tiles per position, two stages in flight), partial 32-channel steps, K not
# a multiple of 4; K >= 512 from 128 tiles (64 x 128, with a partial k tile
# and a partial bp tile), K > 256 below 128 tiles (the four-wave 64 x 64
# kernel); then 64 x 128 at K <= 128 from 1600 tiles (16 x 64@56^2), K >= 256
# from 200 and K >= 640 from 64, 128 x 128 at K >= 512 from 256 tiles, and
# 128 x 64 at K >= 1024 below 128 tiles, each with partial tiles; last the
# 64 x 96 tile (288 tiles at K = 256, 72 at K = 640) and 64 x 64 at K <= 128
# below 1600 tiles (225 tiles, K = 120).
GEMM_CASES = [(1, 64, 64, 56), (1, 512, 512, 7), (2, 192, 48, 14), (4, 128, 256, 28),
              (1, 256, 256, 14), (1, 16, 40, 9), (8, 128, 128, 28), (2, 136, 200, 30),
              (4, 72, 132, 40),
              (16, 64, 64, 56), (12, 128, 128, 28), (12, 40, 24, 30), (12, 104, 100, 28),
              (12, 96, 98, 28),
              (32, 40, 520, 7), (33, 24, 516, 7),
              (2, 64, 320, 14), (3, 48, 264, 20),
              (8, 40, 264, 28), (2, 32, 648, 32), (66, 24, 516, 7), (1, 16, 1032, 28),
              (32, 64, 256, 14), (2, 40, 640, 32), (9, 56, 120, 28)]


@pytest.mark.parametrize("B,C,K,H", GEMM_CASES)
def test_gemm_within_fp32_bound(oracle, B, C, K, H):
    """White-box: force the 3-pass path with caller workspaces; for C % 8 == 0
    the workspace then holds V[64][BP][C] (above 32 tiles; at most 32 the GEMM
    reads V in operand blocks, checked through M) and M[64][BP][K] at the
    minimal tiling ceil(Ho/6) x ceil(Wo/6)."""
    print(f"[gemm] B={B} C={C} K={K} H={H}", flush=True)
    assert C % 8 == 0
    lib = _lib()
    x = torch.randn(B, C, H, H).half()
    w = _kaiming(K, C)
    nh, nw, Ho, Wo = oracle.tiling(H, H, 1)
    nhm, nwm = -(-Ho // 6), -(-Wo // 6)
    BP, BPm = B * nh * nw, B * nhm * nwm
    V = torch.empty(64 * C * BP, dtype=torch.float16, device=DEV)
    M = torch.empty(64 * K * BP, dtype=torch.float16, device=DEV)
    y = torch.empty(B, K, Ho, Wo, dtype=torch.float16, device=DEV)
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, 1)
        wd = w.to(DEV)
        lib.nova_set_weights(h, wd.data_ptr(), K, C)
        xd = x.to(DEV)
        lib.nova_forward_workspace(h, xd.data_ptr(), y.data_ptr(), V.data_ptr(), M.data_ptr(),
                                   B, H, H, 1, nh, nw)
        _check()
        assert lib.nova_get_last_path(h) == 1
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    Vg = V[: 64 * C * BPm].view(64, BPm, C)
    Mg = M[: 64 * K * BPm].view(64, BPm, K)
    Vo = oracle.input_transform(x.numpy(), 1, nhm, nwm)
    if BPm > 32:
        assert_same_bits(_u16(Vg), Vo, "V (workspace)")
    Uo = oracle.filter_transform(w.numpy())
    Mo, Mabs = oracle.batched_gemm(Uo, Vo, with_abs=True)
    mg = Mg.float().cpu().numpy().astype(np.float64)
    mo = Mo.astype(np.float64)
    bound = 2.0 * C * 2.0 ** -24 * Mabs.astype(np.float64) + _ulp16(mo) * 1.0001
    err = np.abs(mg - mo)
    assert np.isfinite(mg).all()
    worst = np.argmax(err - bound)
    assert (err <= bound).all(), f"M mismatch at {np.unravel_index(worst, err.shape)}: err {err.flat[worst]} bound {bound.flat[worst]}"
    # the output transform of the GPU's own M is bit-exact
    yo = oracle.output_transform(Mg.cpu().numpy(), B, Ho, Wo, nhm, nwm)
    assert_same_bits(_u16(y), yo, "y from GPU M")


FORWARD_CASES = [
    # (B, C, K, H, W, pad) -- BASELINE configs 1-2 and edge shapes
    (1, 64, 64, 56, 56, 1),
    (4, 64, 64, 56, 56, 1),
    (3, 32, 96, 20, 20, 1),
    (1, 128, 128, 28, 28, 1),
    (1, 256, 256, 14, 14, 1),
    (1, 512, 512, 7, 7, 1),
    (1, 192, 48, 56, 56, 1),
    (1, 192, 48, 7, 7, 1),
    (2, 3, 64, 32, 32, 1),
    (2, 20, 36, 13, 17, 0),
    (1, 40, 24, 10, 10, 2),
]


def _forward_case(oracle, B, C, K, H, W, pad, path):
    torch.manual_seed(0)
    x = torch.randn(B, C, H, W).half()
    w = _kaiming(K, C)
    lib = _lib()
    h = lib.nova_create()
    Ho, Wo = H + 2 * pad - 2, W + 2 * pad - 2
    y = torch.empty(B, K, Ho, Wo, dtype=torch.float16, device=DEV)
    try:
        lib.nova_set_path(h, path)
        wd, xd = w.to(DEV), x.to(DEV)
        lib.nova_set_weights(h, wd.data_ptr(), K, C)
        lib.nova_forward(h, xd.data_ptr(), y.data_ptr(), B, H, W, pad)
        _check()
        took = lib.nova_get_last_path(h)
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    yg = y.cpu().numpy()
    yo = oracle.conv2d(x.numpy(), w.numpy(), pad)
    truth = oracle.direct_conv2d(x.numpy(), w.numpy(), pad)
    return yg, yo, truth, took


@pytest.mark.parametrize("path", [1, 2, 3, 6, 7], ids=["3pass", "fused_rows", "fused_block",
                                                        "two_pass", "in_gemm"])
@pytest.mark.parametrize("B,C,K,H,W,pad", FORWARD_CASES)
def test_forward_matches_oracle(oracle, B, C, K, H, W, pad, path):
    print(f"[forward] B={B} C={C} K={K} H={H} W={W} pad={pad} path={path}", flush=True)
    if path == 7 and B * -(-(H + 2 * pad - 2) // 6) * -(-(W + 2 * pad - 2) // 6) > 64:
        pytest.skip("path 7 serves at most 64 tiles")
    yg, yo, truth, took = _forward_case(oracle, B, C, K, H, W, pad, path)
    assert took == path
    assert np.isfinite(yg.astype(np.float32)).all()
    rel = oracle.rel_l2(yg, yo)
    assert rel <= 5e-3, rel
    assert oracle.max_abs(yg, yo) <= 0.25
    rel_g, rel_o = oracle.rel_l2(yg, truth), oracle.rel_l2(yo, truth)
    mx_g, mx_o = oracle.max_abs(yg, truth), oracle.max_abs(yo, truth)
    assert rel_g <= 1.05 * rel_o, (rel_g, rel_o)
    assert mx_g <= 1.25 * mx_o, (mx_g, mx_o)


def test_forward_deterministic():
    lib = _lib()
    x = torch.randn(2, 64, 28, 28, device=DEV).half()
    w = _kaiming(64, 64).to(DEV)
    h = lib.nova_create()
    try:
        lib.nova_set_weights(h, w.data_ptr(), 64, 64)
        outs = []
        for _ in range(3):
            y = torch.empty(2, 64, 28, 28, dtype=torch.float16, device=DEV)
            lib.nova_forward(h, x.data_ptr(), y.data_ptr(), 2, 28, 28, 1)
            _check()
            outs.append(y.clone())
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


def test_forward_follows_stream(oracle):
    """Work goes to the stream set on the handle, ordered after the producer
    of its input on that stream."""
    lib = _lib()
    s = torch.cuda.Stream()
    w = _kaiming(32, 32).to(DEV)
    h = lib.nova_create()
    try:
        lib.nova_set_stream(h, ctypes.c_void_p(s.cuda_stream))
        with torch.cuda.stream(s):
            x = torch.randn(1, 32, 20, 20, device=DEV).half()
            lib.nova_set_weights(h, w.data_ptr(), 32, 32)
            y = torch.empty(1, 32, 20, 20, dtype=torch.float16, device=DEV)
            lib.nova_forward(h, x.data_ptr(), y.data_ptr(), 1, 20, 20, 1)
            _check()
        s.synchronize()
        yo = oracle.conv2d(x.cpu().numpy(), w.cpu().numpy(), 1)
    finally:
        lib.nova_destroy(h)
    assert oracle.rel_l2(y.cpu().numpy(), yo) < 5e-3


def test_concurrent_handles_on_two_streams():
    """Two handles on two streams (default priority) run different layers and
    paths concurrently, each forward repeated; every result equals the same
    forward run alone on the default stream, bit for bit."""
    lib = _lib()
    cases = [(32, 64, 64, 56, 0), (8, 128, 96, 28, 1)]  # fused tile-block, three-pass
    data, ref = [], []
    torch.manual_seed(61)
    for B, C, K, H, path in cases:
        x = torch.randn(B, C, H, H, device=DEV).half()
        w = (torch.randn(K, C, 3, 3, device=DEV) * 0.05).float()
        data.append((x, w))
        y = torch.empty(B, K, H, H, dtype=torch.float16, device=DEV)
        h = lib.nova_create()
        try:
            lib.nova_set_path(h, path)
            lib.nova_set_weights(h, w.data_ptr(), K, C)
            lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, H, 1)
            _check()
            torch.cuda.synchronize()
        finally:
            lib.nova_destroy(h)
        ref.append(y)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    handles = [lib.nova_create(), lib.nova_create()]
    outs = [[], []]
    try:
        for i, ((B, C, K, H, path), (x, w)) in enumerate(zip(cases, data)):
            lib.nova_set_stream(handles[i], ctypes.c_void_p(streams[i].cuda_stream))
            lib.nova_set_path(handles[i], path)
            streams[i].wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(streams[i]):
                lib.nova_set_weights(handles[i], w.data_ptr(), K, C)
        for rep in range(4):
            for i, ((B, C, K, H, path), (x, w)) in enumerate(zip(cases, data)):
                with torch.cuda.stream(streams[i]):
                    y = torch.empty(B, K, H, H, dtype=torch.float16, device=DEV)
                    lib.nova_forward(handles[i], x.data_ptr(), y.data_ptr(), B, H, H, 1)
                    _check()
                    outs[i].append(y)
        for s in streams:
            s.synchronize()
    finally:
        for h in handles:
            lib.nova_destroy(h)
    for i in range(2):
        for y in outs[i]:
            assert torch.equal(y, ref[i]), i
