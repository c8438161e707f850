"""BASELINE configs 4 and 5 at their real shapes: SD-1.5-style UNet convs at
B=2 (320@64, 640@32, 1280@16, 1280@8 and the 320->640, 640->1280,
1280->640, 640->320 transitions), SDXL-style B=1 (320@128, 640@64,
1280@32) and DenseNet-161 bottleneck 192->48 at 56/28/14/7 (K not a tile
multiple, H and W not multiples of 6). Each runs on the automatically chosen
path and is compared with the CPU oracle on the full problem (the oracle
finishes these in seconds): rel-L2 <= 5e-3, max-abs <= 0.25 at unit scale,
zero NaN/Inf.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")

CONFIGS = [
    # (name, B, C, K, H)
    ("sd15_320@64", 2, 320, 320, 64),
    ("sd15_640@32", 2, 640, 640, 32),
    ("sd15_1280@16", 2, 1280, 1280, 16),
    ("sd15_1280@8", 2, 1280, 1280, 8),
    ("sd15_320to640@32", 2, 320, 640, 32),
    ("sd15_640to1280@16", 2, 640, 1280, 16),
    ("sd15_1280to640@32", 2, 1280, 640, 32),
    ("sd15_640to320@64", 2, 640, 320, 64),
    ("sdxl_320@128", 1, 320, 320, 128),
    ("sdxl_640@64", 1, 640, 640, 64),
    ("sdxl_1280@32", 1, 1280, 1280, 32),
    ("dn161_192to48@56", 1, 192, 48, 56),
    ("dn161_192to48@28", 1, 192, 48, 28),
    ("dn161_192to48@14", 1, 192, 48, 14),
    ("dn161_192to48@7", 1, 192, 48, 7),
]


@pytest.mark.parametrize("name,B,C,K,H", CONFIGS, ids=[c[0] for c in CONFIGS])
def test_config_shape_matches_oracle(oracle, name, B, C, K, H):
    from nova_winograd.ops import check, get_lib

    print(f"[config] {name} B={B} C={C} K={K} H={H}", flush=True)
    lib = get_lib()
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, C, H, H, generator=g).half()
    w = torch.empty(K, C, 3, 3)
    torch.nn.init.kaiming_normal_(w, mode="fan_in", nonlinearity="relu", generator=g)
    xd, wd = x.to(DEV), w.to(DEV)
    y = torch.empty(B, K, H, H, dtype=torch.float16, device=DEV)
    h = lib.nova_create()
    try:
        lib.nova_set_weights(h, wd.data_ptr(), K, C)
        lib.nova_forward(h, xd.data_ptr(), y.data_ptr(), B, H, H, 1)
        check("forward")
        torch.cuda.synchronize()
    finally:
        lib.nova_destroy(h)
    yg = y.cpu().numpy()
    assert np.isfinite(yg.astype(np.float32)).all()
    yo = oracle.conv2d(x.numpy(), w.numpy(), 1)
    assert oracle.rel_l2(yg, yo) <= 5e-3
    assert oracle.max_abs(yg, yo) <= 0.25
