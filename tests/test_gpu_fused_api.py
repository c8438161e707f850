"""The reference's fused C-API (/root/reference/csrc/nova_winograd_fused.hip:
619-652; declared there, never bound by its Python package): the five
nova_fused_* symbols drive the same handle as the main API. Checked: a
forward through nova_fused_create / set_weights / forward equals
nova_forward on the same data bit for bit (including the shapes where the
reference would pick its fused kernel, C, K <= 64), and
nova_fused_compute_tiling follows the same tiling law as
nova_compute_tiling."""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.mark.parametrize("B,C,K,H,pad", [(1, 64, 64, 56, 1), (32, 64, 64, 56, 1),
                                         (2, 128, 96, 28, 1), (3, 40, 24, 17, 0)])
def test_fused_api_equals_main_api(B, C, K, H, pad):
    from nova_winograd.ops import check, get_lib

    print(f"[fused api] B={B} C={C} K={K} H={H} pad={pad}", flush=True)
    lib = get_lib()
    torch.manual_seed(51)
    x = torch.randn(B, C, H, H, device=DEV).half()
    w = (torch.randn(K, C, 3, 3, device=DEV) * 0.05).float()
    Ho = H + 2 * pad - 2
    ys = []
    for create, setw, fwd, destroy in (
            (lib.nova_create, lib.nova_set_weights, lib.nova_forward, lib.nova_destroy),
            (lib.nova_fused_create, lib.nova_fused_set_weights, lib.nova_fused_forward,
             lib.nova_fused_destroy)):
        y = torch.empty(B, K, Ho, Ho, dtype=torch.float16, device=DEV)
        h = create()
        try:
            setw(h, w.data_ptr(), K, C)
            fwd(h, x.data_ptr(), y.data_ptr(), B, H, H, pad)
            check()
            torch.cuda.synchronize()
        finally:
            destroy(h)
        ys.append(y)
    assert torch.equal(ys[0], ys[1])
    assert torch.isfinite(ys[0]).all()


def test_fused_compute_tiling():
    from nova_winograd.ops import get_lib

    lib = get_lib()
    for H, W, pad in [(56, 56, 1), (28, 17, 0), (7, 7, 1), (64, 33, 2), (3, 3, 0)]:
        a = [ctypes.c_int() for _ in range(4)]
        b = [ctypes.c_int() for _ in range(4)]
        lib.nova_compute_tiling(H, W, pad, *[ctypes.byref(v) for v in a])
        lib.nova_fused_compute_tiling(H, W, pad, *[ctypes.byref(v) for v in b])
        assert [v.value for v in a] == [v.value for v in b], (H, W, pad)
