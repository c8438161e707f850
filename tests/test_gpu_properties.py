"""Size-independent properties at BASELINE's full sizes (the oracle is too
slow for every image there), on the automatically chosen path:

* negation: the transforms (fp32 FMA chains from +0, round-to-nearest-even)
  are odd-symmetric, so V(-x) == -V(x) exactly; the MFMA accumulation is not
  (measured on gfx950: M(-x) and -M(x) differ by one fp16 ulp in about 3 of
  100 000 elements -- its internal rounding is not sign-symmetric), so M is
  held to one ulp and y(-x) to a tight tolerance around -y(x);
* translation: shifting the input right by 6 pixels shifts the tile grid by
  one tile, so every output tile whose input patch stays inside the image is
  shifted unchanged, bit for bit;
* batch independence: an image's output does not depend on the rest of the
  batch -- bit for bit where the batch and single-image runs use the same
  arithmetic (the transforms always; the products when both run three-pass),
  within the fp32 accumulation-order bound where the batch runs the fused
  tile-block kernel (16- instead of 32-channel MFMA steps);
* output-channel rotation: rolling the filters by 16 output channels rolls
  the output channels by 16, bit for bit (each output channel's products and
  transforms do not depend on its neighbours; 16 keeps every channel in the
  same lane of its MFMA tile) -- the translation check's stand-in where the
  image is narrower than two tiles plus the shift (7 x 7);
* the first two images of every batch against the oracle;
* finiteness and bitwise repeatability.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")

# (B, C, K, H): BASELINE config 3 -- the four ResNet-50 layers at B=32 (the
# bench's batch) and at B=128
SHAPES = [(32, 64, 64, 56), (32, 128, 128, 28), (32, 256, 256, 14), (32, 512, 512, 7),
          (128, 64, 64, 56), (128, 128, 128, 28), (128, 256, 256, 14), (128, 512, 512, 7)]


def _forward(lib, x, w, pad=1):
    from nova_winograd.ops import check

    B, C, H, W = x.shape
    K = w.shape[0]
    y = torch.empty(B, K, H + 2 * pad - 2, W + 2 * pad - 2, dtype=torch.float16, device=DEV)
    h = lib.nova_create()
    try:
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, W, pad)
        check()
        took = lib.nova_get_last_path(h)
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    return y, took


def _data(B, C, K, H, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, C, H, H, generator=g).half().to(DEV)
    w = torch.empty(K, C, 3, 3)
    torch.nn.init.kaiming_normal_(w, mode="fan_in", nonlinearity="relu", generator=g)
    return x, w.to(DEV)


@pytest.mark.parametrize("B,C,K,H", SHAPES)
def test_negation_and_repeatability(B, C, K, H):
    from nova_winograd.ops import get_lib

    print(f"[props] negation B={B} C={C} K={K} H={H}", flush=True)
    lib = get_lib()
    x, w = _data(B, C, K, H, 21)
    y, _ = _forward(lib, x, w)
    y_neg, _ = _forward(lib, -x, w)
    y_again, _ = _forward(lib, x, w)
    assert torch.isfinite(y).all()
    assert torch.equal(y_again.view(torch.int16), y.view(torch.int16))
    a, b = y_neg.float(), -y.float()
    assert ((a - b).norm() / b.norm()).item() <= 5e-4
    # one ulp of a large Winograd-domain M value moves y by up to ~0.06; the
    # forward parity bar against the oracle is 0.25
    assert (a - b).abs().max().item() <= 0.25
    assert (a != b).float().mean().item() <= 2e-3


def _ulp16(v):
    """Spacing of fp16 values at |v| (normal range; subnormal spacing below)."""
    e = torch.floor(torch.log2(v.abs().clamp(min=2.0 ** -14)))
    return torch.pow(2.0, e - 10)


def test_negation_white_box_v_exact_m_within_gemm_bound(oracle):
    """Three-pass workspaces at conv3_x B=32: V(-x) == -V(x) bit for bit; the
    MFMA's sums of x and -x differ by at most their two fp32 summation error
    bounds (2·C·2^-24·Σ|U||V| each, the bound the GEMM parity test uses)
    plus one fp16 ulp each."""
    import numpy as np

    from nova_winograd.ops import check, get_lib

    lib = get_lib()
    B, C, K, H = 32, 128, 128, 28
    x, w = _data(B, C, K, H, 24)
    BPm = B * 5 * 5  # minimal tiling of 28 x 28
    res = []
    for sign in (1, -1):
        V = torch.empty(64 * C * B * 36, dtype=torch.float16, device=DEV)  # reference tiling
        M = torch.empty(64 * K * B * 36, dtype=torch.float16, device=DEV)
        y = torch.empty(B, K, H, H, dtype=torch.float16, device=DEV)
        h = lib.nova_create()
        try:
            lib.nova_set_path(h, 1)
            lib.nova_set_weights(h, w.data_ptr(), K, C)
            xs = (x if sign == 1 else -x).contiguous()
            lib.nova_forward_workspace(h, xs.data_ptr(), y.data_ptr(), V.data_ptr(),
                                       M.data_ptr(), B, H, H, 1, 6, 6)
            check()
            torch.cuda.synchronize()
        finally:
            lib.nova_destroy(h)
        res.append((V[:64 * C * BPm].clone(), M[:64 * K * BPm].float()))
    (v1, m1), (v2, m2) = res
    assert torch.equal(v2, -v1)
    Uo = oracle.filter_transform(w.cpu().numpy())
    Vo = v1.view(64, BPm, C).cpu().numpy()
    _, Mabs = oracle.batched_gemm(Uo, Vo, with_abs=True)
    bound = (2 * 2.0 * C * 2.0 ** -24 * torch.from_numpy(Mabs.astype(np.float32)).to(DEV).view(-1)
             + 2 * _ulp16(m1) * 1.0001)
    err = (m2 + m1).abs()
    print(f"[props] M(-x) vs -M(x): {(m2 != -m1).float().mean().item():.2e} of elements "
          f"differ, worst at {(err / bound).max().item():.3f} of the bound", flush=True)
    assert (err <= bound).all()


@pytest.mark.parametrize("B,C,K,H", SHAPES)
def test_translation_by_one_tile(B, C, K, H):
    from nova_winograd.ops import get_lib

    print(f"[props] translation B={B} C={C} K={K} H={H}", flush=True)
    lib = get_lib()
    x, w = _data(B, C, K, H, 22)
    xs = torch.zeros_like(x)
    xs[..., 6:] = x[..., :-6]  # content moved right by exactly one tile
    y, _ = _forward(lib, x, w)
    ys, _ = _forward(lib, xs, w)
    # Output tile tw of the original and tile tw + 1 of the shifted run read
    # the same 8x8 patch (columns 6tw-1 .. 6tw+6 of x; column -1 is padding in
    # one and a zero column in the other) as long as that patch does not reach
    # the 6 columns the shift pushed out of the image: 6tw + 6 <= W - 7.
    T = (H - 13) // 6 + 1 if H >= 13 else 0
    if T == 0:
        pytest.skip("image narrower than two tiles plus the shift")
    assert torch.equal(ys[..., 6:6 + 6 * T], y[..., 0:6 * T])


@pytest.mark.parametrize("B,C,K,H", SHAPES)
def test_batch_independence(B, C, K, H):
    from nova_winograd.ops import get_lib

    print(f"[props] batch independence B={B} C={C} K={K} H={H}", flush=True)
    lib = get_lib()
    x, w = _data(B, C, K, H, 23)
    y, took = _forward(lib, x, w)
    for i in (0, B // 2, B - 1):
        yi, took_i = _forward(lib, x[i:i + 1].contiguous(), w)
        if took == took_i:
            assert torch.equal(yi[0], y[i]), f"image {i}"
        else:  # fused batch vs three-pass single image: accumulation order only
            a, b = yi[0].float(), y[i].float()
            rel = ((a - b).norm() / b.norm()).item()
            assert rel <= 2e-3, (i, rel)
            assert (a - b).abs().max().item() <= 0.1


@pytest.mark.parametrize("B,C,K,H", SHAPES)
def test_output_channel_rotation(B, C, K, H):
    from nova_winograd.ops import get_lib

    print(f"[props] channel rotation B={B} C={C} K={K} H={H}", flush=True)
    lib = get_lib()
    x, w = _data(B, C, K, H, 25)
    y, took = _forward(lib, x, w)
    yr, took_r = _forward(lib, x, torch.roll(w, 16, dims=0).contiguous())
    assert took == took_r
    assert torch.equal(yr, torch.roll(y, 16, dims=1))


@pytest.mark.parametrize("B,C,K,H", SHAPES)
def test_first_images_against_oracle(oracle, B, C, K, H):
    print(f"[props] oracle B={B} C={C} K={K} H={H}", flush=True)
    from nova_winograd.ops import get_lib

    lib = get_lib()
    x, w = _data(B, C, K, H, 26)
    y, _ = _forward(lib, x, w)
    yo = oracle.conv2d(x[:2].cpu().numpy(), w.cpu().numpy(), 1)
    yg = y[:2].cpu().numpy()
    assert oracle.rel_l2(yg, yo) <= 5e-3
    assert oracle.max_abs(yg, yo) <= 0.25
