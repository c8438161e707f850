"""Stream ordering of a shared handle.

``nova_forward`` (like the custom op) runs on one persistent handle per
device, whose transformed filter and workspace every call reuses. When a call
arrives on a different stream than the last one, the library makes the new
stream wait for the work already queued on the old one (nova_set_stream), so
a filter transform for new weights on stream 2 cannot overwrite the filter a
GEMM still reads on stream 1. Here two streams alternate weights with no
synchronisation between them; every output must equal its single-stream
result bit for bit.
"""

import pytest
import torch

import nova_winograd as nw

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.mark.parametrize("B,C,H", [(8, 128, 28), (2, 64, 56), (1, 512, 7)])
def test_two_streams_alternating_weights(B, C, H):
    print(f"[streams] B={B} C={C} H={H}", flush=True)
    torch.manual_seed(5)
    x = torch.randn(B, C, H, H, device=DEV).half()
    w1 = torch.randn(C, C, 3, 3, device=DEV) * 0.05
    w2 = torch.randn(C, C, 3, 3, device=DEV) * 0.05
    ref1 = nw.nova_forward(x, w1)
    ref2 = nw.nova_forward(x, w2)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for _ in range(6):
        with torch.cuda.stream(s1):
            y1 = nw.nova_forward(x, w1)
        with torch.cuda.stream(s2):
            y2 = nw.nova_forward(x, w2)
        outs.append((y1, y2))
    torch.cuda.synchronize()
    for y1, y2 in outs:
        assert torch.equal(y1, ref1)
        assert torch.equal(y2, ref2)
