"""The HIP library against the committed golden fixtures (no oracle call):
transforms bit-exact through the reference-layout entry points, the whole
forward (both paths) within the parity tolerance of the fixture's y."""

import glob
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_library_matches_fixture(path):
    from nova_winograd.ops import check, get_lib

    lib = get_lib()
    f = np.load(path)
    B, C, K, H, W, pad, nh, nw, Ho, Wo = (int(v) for v in f["shape"])
    print(f"[golden] {os.path.basename(path)}", flush=True)
    BP = B * nh * nw
    x = torch.from_numpy(f["x"]).to(DEV)
    w = torch.from_numpy(f["w"]).to(DEV)
    U = torch.empty(64, C, K, dtype=torch.float16, device=DEV)
    lib.nova_filter_transform(w.data_ptr(), U.data_ptr(), K, C)
    check()
    V = torch.empty(64, BP, C, dtype=torch.float16, device=DEV)
    lib.nova_input_transform(x.data_ptr(), V.data_ptr(), B, C, H, W, pad, nh, nw, BP)
    check()
    M = torch.from_numpy(f["M"]).to(DEV)
    y = torch.zeros(B, K, Ho, Wo, dtype=torch.float16, device=DEV)
    lib.nova_output_transform(M.data_ptr(), y.data_ptr(), B, K, Ho, Wo, nh, nw, BP)
    check()
    torch.cuda.synchronize()
    assert np.array_equal(_u16(U), f["U"].view(np.uint16))
    assert np.array_equal(_u16(V), f["V"].view(np.uint16))
    assert np.array_equal(_u16(y), f["y"].view(np.uint16))
    for path_id in (1, 2):
        h = lib.nova_create()
        try:
            lib.nova_set_path(h, path_id)
            lib.nova_set_weights(h, w.data_ptr(), K, C)
            yf = torch.empty(B, K, Ho, Wo, dtype=torch.float16, device=DEV)
            lib.nova_forward(h, x.data_ptr(), yf.data_ptr(), B, H, W, pad)
            check()
            torch.cuda.synchronize()
        finally:
            lib.nova_destroy(h)
        a = yf.float().cpu().numpy().astype(np.float64)
        b = f["y"].astype(np.float64)
        assert np.linalg.norm(a - b) <= 5e-3 * np.linalg.norm(b), path_id
        assert np.abs(a - b).max() <= 0.25
