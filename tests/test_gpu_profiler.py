"""Per-kernel timing (nova_profile_enable / nova_profile_read; no
counterpart in the reference): every kernel of a timed forward records its
own start and end into a pair of hipEvents. Checked: one interval per kernel
launched (three per three-pass forward, one per fused forward), positive
intervals whose sum stays below the wall-clock time of the forwards, outputs
bit-identical to unprofiled forwards, and reads that reset the record."""

import ctypes
import time

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.mark.parametrize("path,B,C,K,H", [(1, 2, 64, 64, 28), (3, 32, 64, 64, 56),
                                          (1, 4, 128, 96, 14), (6, 4, 128, 96, 14)])
def test_profile_counts_and_intervals(path, B, C, K, H):
    from nova_winograd.ops import check, get_lib

    print(f"[profiler] path={path} B={B} C={C} K={K} H={H}", flush=True)
    lib = get_lib()
    torch.manual_seed(3)
    x = torch.randn(B, C, H, H, device=DEV).half()
    w = (torch.randn(K, C, 3, 3, device=DEV) * 0.05).float()
    y0 = torch.empty(B, K, H, H, dtype=torch.float16, device=DEV)
    y1 = torch.empty_like(y0)
    tot = (ctypes.c_double * 4)()
    cnt = (ctypes.c_longlong * 4)()
    n = 5
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, path)
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        lib.nova_forward(h, x.data_ptr(), y0.data_ptr(), B, H, H, 1)
        check()
        assert lib.nova_get_last_path(h) == path
        lib.nova_profile_enable(h, 1)
        check()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            lib.nova_forward(h, x.data_ptr(), y1.data_ptr(), B, H, H, 1)
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3
        check()
        timed = lib.nova_profile_read(h, tot, cnt)
        check()
        assert torch.equal(y0, y1)
        kinds = {1: [0, 1, 2], 6: [0, 3]}.get(path, [3])
        assert timed == n * len(kinds)
        for k in range(4):
            if k in kinds:
                assert cnt[k] == n
                assert 0.0 < tot[k] / n < wall_ms / n, (k, tot[k], wall_ms)
                name = lib.nova_profile_kernel_name(h, k).decode()
                assert name, k
            else:
                assert cnt[k] == 0 and tot[k] == 0.0
        assert sum(tot) < wall_ms
        # a read resets the record; disabled profiling records nothing
        assert lib.nova_profile_read(h, tot, cnt) == 0
        lib.nova_profile_enable(h, 0)
        lib.nova_forward(h, x.data_ptr(), y1.data_ptr(), B, H, H, 1)
        torch.cuda.synchronize()
        assert lib.nova_profile_read(h, tot, cnt) == 0
        check()
    finally:
        lib.nova_destroy(h)


@pytest.mark.parametrize("path,B,C,K,H", [(1, 2, 64, 64, 28), (3, 32, 64, 64, 56),
                                          (6, 3, 96, 128, 28)])
def test_profile_replay(path, B, C, K, H):
    """nova_profile_replay re-launches the last forward's kernels (they are
    idempotent: the output is unchanged), returns a positive mean time for
    every kind the forward launched and an error for the others."""
    from nova_winograd.ops import check, get_lib

    print(f"[profiler] replay path={path} B={B}", flush=True)
    lib = get_lib()
    torch.manual_seed(4)
    x = torch.randn(B, C, H, H, device=DEV).half()
    w = (torch.randn(K, C, 3, 3, device=DEV) * 0.05).float()
    y = torch.empty(B, K, H, H, dtype=torch.float16, device=DEV)
    h = lib.nova_create()
    try:
        lib.nova_set_path(h, path)
        lib.nova_set_weights(h, w.data_ptr(), K, C)
        lib.nova_forward(h, x.data_ptr(), y.data_ptr(), B, H, H, 1)
        check()
        torch.cuda.synchronize()
        y0 = y.clone()
        kinds = {1: [0, 1, 2], 6: [0, 3]}.get(path, [3])
        for k in range(4):
            ms = lib.nova_profile_replay(h, k, 5)
            if k in kinds:
                assert ms > 0.0, k
                assert lib.nova_get_last_error() == 0
            else:
                assert ms < 0.0
                assert lib.nova_get_last_error() != 0
        torch.cuda.synchronize()
        assert torch.equal(y, y0)
        assert lib.nova_get_U_gemm(h)
    finally:
        lib.nova_destroy(h)
