"""The drop-in Python surface on the CPU: names and behaviour that do not
need a GPU (construction, from_conv2d, surgery, cache keys), and the loud
failure of every compute entry point on CPU tensors (no CPU fallback)."""

import subprocess
import sys

import pytest
import torch
import torch.nn as nn

import nova_winograd as nw
from nova_winograd import (
    NovaWinogradConv2d,
    NovaWinogradConv2dCompilable,
    NovaWinogradConv2dTrainable,
    nova_forward,
    replace_conv2d_with_nova,
)


def test_exports():
    assert nw.__version__ == "1.0.0"
    assert set(nw.__all__) == {
        "NovaWinogradConv2d", "NovaWinogradConv2dTrainable", "NovaWinogradConv2dCompilable",
        "nova_forward", "compute_tiling", "replace_conv2d_with_nova"}


def test_module_construction_and_repr():
    m = NovaWinogradConv2d(16, 32, kernel_size=3, padding=1, bias=True)
    assert m.weight.shape == (32, 16, 3, 3) and m.weight.dtype == torch.float32
    assert m.bias.shape == (32,) and torch.count_nonzero(m.bias) == 0
    assert "tile=F(6,3), points=NOVA" in repr(m)
    assert "compilable=True" in repr(NovaWinogradConv2dCompilable(4, 4))
    with pytest.raises(AssertionError):
        NovaWinogradConv2d(4, 4, kernel_size=5)


def test_from_conv2d_copies_parameters():
    conv = nn.Conv2d(8, 12, 3, padding=2, bias=True)
    m = NovaWinogradConv2d.from_conv2d(conv)
    assert m.padding == 2
    assert torch.equal(m.weight, conv.weight) and torch.equal(m.bias, conv.bias)
    t = NovaWinogradConv2dTrainable.from_conv2d(conv)
    assert isinstance(t, NovaWinogradConv2dTrainable)
    with pytest.raises(AssertionError):
        NovaWinogradConv2d.from_conv2d(nn.Conv2d(8, 8, 3, stride=2))


def test_surgery_replaces_eligible_layers():
    model = nn.Sequential(
        nn.Conv2d(3, 64, 3, padding=1, bias=False),      # eligible
        nn.ReLU(),
        nn.Conv2d(64, 128, 3, stride=2, padding=1),      # stride 2
        nn.ReLU(),
        nn.Conv2d(128, 128, 3, padding=1, bias=True),    # eligible
        nn.ReLU(),
        nn.Conv2d(128, 256, 1),                          # 1x1
        nn.Conv2d(256, 256, 3, padding=1, groups=2),     # grouped
        nn.Conv2d(256, 256, 3, padding=1, dilation=2),   # dilated
        nn.Conv2d(256, 256, 3, padding="same"),          # string padding
        nn.Conv2d(256, 256, 3, padding=(1, 2)),          # asymmetric
        nn.Conv2d(256, 256, 3, padding=1, padding_mode="reflect"),
    )
    n = replace_conv2d_with_nova(model, verbose=False)
    assert n == 2
    assert isinstance(model[0], NovaWinogradConv2d) and isinstance(model[4], NovaWinogradConv2d)
    assert isinstance(model[2], nn.Conv2d)
    assert torch.count_nonzero(model[4].bias) == torch.count_nonzero(model[4].bias)
    nested = nn.Sequential(nn.Sequential(nn.Conv2d(4, 4, 3, padding=1)))
    assert replace_conv2d_with_nova(nested, trainable=True, verbose=False) == 1
    assert isinstance(nested[0][0], NovaWinogradConv2dTrainable)


def test_cpu_tensors_fail_loudly():
    m = NovaWinogradConv2d(4, 4)
    x = torch.randn(1, 4, 8, 8).half()
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        m(x)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        nova_forward(x, torch.randn(4, 4, 3, 3))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        NovaWinogradConv2dTrainable(4, 4)(x.float())


def test_weight_cache_key_tracks_in_place_updates():
    from nova_winograd.conv2d import _weight_key

    m = NovaWinogradConv2d(4, 4)
    k0 = _weight_key(m.weight)
    with torch.no_grad():
        m.weight.add_(1.0)
    assert _weight_key(m.weight) != k0
    k1 = _weight_key(m.weight)
    m.half()
    assert _weight_key(m.weight) != k1


def test_bench_refuses_multi_gpu():
    import os

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_bench_kernel_stats_summary(tmp_path):
    """bench.py's kernel-trace summary writer: per-family agreement of the
    bench line's event times with a rocprofv3 trace (synthetic CSVs here)."""
    import importlib.util
    import json
    import os

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(root, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    trace = tmp_path / "trace"
    trace.mkdir()
    (trace / "run_kernel_stats.csv").write_text(
        '"Name","Calls","TotalDurationNs","AverageNs","Percentage","MinNs","MaxNs","StdDev"\n'
        '"_ZN4nova16wgemm_lds_kernelILi64E",4,40000,10000.0,60.0,9000,11000,1.0\n'
        '"_ZN4nova22input_transform_kernelILi2E",4,20000,5000.0,40.0,4000,6000,1.0\n')
    rows = ["Kernel_Name,Grid_Size_X,Grid_Size_Y,Grid_Size_Z,Start_Timestamp,End_Timestamp"]
    for i in range(4):
        rows.append(f"_ZN4nova16wgemm_lds_kernelILi64E,1024,1,1,{1000 * i},{1000 * i + 10000}")
        rows.append(f"_ZN4nova15input_lp_kernelILb0E,256,1,1,{1000 * i},{1000 * i + 5000}")
    (trace / "run_kernel_trace.csv").write_text("\n".join(rows) + "\n")
    line = {"value": 1.0, "ms_per_step": 0.1,
            "roofline": {"kernel": "wgemm", "avg_launch_us": 11.0, "achieved": 1.0, "frac": 0.1,
                         "peak": 8000.0},
            "kernel_families": {"wgemm": {"avg_launch_us": 11.0, "achieved_gbs": 4000.0,
                                          "frac_hbm": 0.5, "frac_hbm_cold": 0.25},
                                "input_transform_kernel": {"avg_launch_us": 5.5,
                                                           "achieved_gbs": 800.0,
                                                           "frac_hbm": 0.1,
                                                           "frac_hbm_cold": 0.05}}}
    bl = tmp_path / "line.json"
    bl.write_text("log line\n" + json.dumps(line) + "\n")
    out = tmp_path / "summary.md"
    bench.kernel_stats_from(str(trace), str(bl), str(out))
    text = out.read_text()
    # 4000 GB/s x 11 us = 44 MB per launch; over the trace's 10 us: 4.4 TB/s = 0.55
    assert "| wgemm | 11.000 | 10.000 | 4 | 1.100 | 44.00 | 0.5000 | 0.5500 | 0.2500 |" in text
    # 800 GB/s x 5.5 us = 4.4 MB; over 5 us: 0.88 TB/s = 0.11
    assert ("| input_transform_kernel | 5.500 | 5.000 | 4 | 1.100 | 4.40 | 0.1000 | 0.1100 | "
            "0.0500 |") in text


def test_bench_mfma_summary(tmp_path):
    """bench.py's MFMA counter summary: executed FLOPs from
    SQ_INSTS_VALU_MFMA_MOPS_F16 (x 512), busy cycles per 512 FLOPs, and the
    peak and busy shares over the bench line's event-timed launch (synthetic
    database with the columns rocprofv3's counter table has)."""
    import importlib.util
    import json
    import os
    import sqlite3

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(root, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    d = tmp_path / "pmc"
    d.mkdir()
    con = sqlite3.connect(d / "pmc_results.db")
    con.execute("create table counters (kernel_name text, grid_size int, counter_name text, "
                "value real)")
    g = "_ZN4nova16wgemm_lds_kernelILi64E"
    rows = []
    for grid, mops in ((1024, 1000.0), (2048, 3000.0)):
        for _ in range(2):
            rows += [(g, grid, "SQ_INSTS_VALU_MFMA_MOPS_F16", mops),
                     (g, grid, "SQ_VALU_MFMA_BUSY_CYCLES", 0.5 * mops)]
    rows.append(("_ZN4nova22input_transform_kernelILi2E", 256, "SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0))
    con.executemany("insert into counters values (?,?,?,?)", rows)
    con.commit()
    con.close()
    line = {"kernel_families": {"wgemm": {"avg_launch_us": 2.048,
                                          "alg_gflop_per_launch": 0.001}}}
    bl = tmp_path / "line.json"
    bl.write_text(json.dumps(line) + "\n")
    out = tmp_path / "mfma.json"
    bench.mfma_from(str(d), str(bl), str(out), cus=4)
    data = json.loads(out.read_text())
    (rec,) = data["kernels"]
    assert rec["kernel"] == "wgemm"
    assert rec["executed_flops_per_launch"] == 2000 * 512
    assert rec["busy_per_512_flops"] == 0.5
    assert rec["busy_cycles_per_launch"] == 1000
    assert rec["mfma_busy_frac"] == pytest.approx(1000 / (2.048e-6 * 2.4e9 * 16), abs=1e-4)
    assert rec["executed_tflops"] == pytest.approx(2000 * 512 / 2.048e-6 / 1e12, abs=0.1)
    assert rec["alg_flops_per_launch"] == 1000000
    assert "| wgemm |" in (tmp_path / "mfma_resnet50_3x3s1_b1_b32.md").read_text()
