#!/usr/bin/env python3
"""Benchmark: NOVA F(6,3) Winograd 3x3 stride-1 convolution on one MI355X.

Workload (BASELINE.json metric: per-layer ms + effective TFLOP/s on the
ResNet-50 3x3 s1 convolutions at B=1 and B=32): the four layers
conv2_x (64ch, 56^2), conv3_x (128, 28^2), conv4_x (256, 14^2),
conv5_x (512, 7^2), pad 1, C=K, at B=1 and at B=32 -- eight layer runs.
A "step" is one forward of all eight through the drop-in module
(NovaWinogradConv2d), inputs resident in HBM, weights transformed once.

Reported on one JSON line (stdout):
  value        effective TFLOP/s of the step = sum of direct-conv FLOPs
               (2*B*K*C*Ho*Wo*9, /root/reference/benchmarks/bench_layers.py:58)
               / step time
  layers       per layer: NOVA ms and MIOpen (nn.Conv2d fp16) ms, eager and
               HIP-graph replayed (ten forwards per graph: GPU time),
               effective TFLOP/s, path, roofline fraction
               T_roof/T (T_roof = max(2*64*K*C*B*P_min / 2.5 PF,
               (2BCHW + 2BKHoWo + 2*64*K*C) / 8 TB/s)), warm and cold
  roofline     the dominant kernel family of the step (largest summed time),
               timed live: every kernel records its own start and end events
               (its dispatch packet, on its launch stream) over a timed region
               of K steps; algorithmic bytes per launch / average launch time
               vs 8 TB/s in cold forwards (frac: a 512 MiB write before each
               forward, so x and U come from HBM), with the warm steady-state
               loop's figures beside them (frac_warm)
  cpu_baseline the CPU oracle (the reference's NOVA arithmetic, C, OpenMP) on
               a bounded sample of the same layers, on this host's cores

Synthetic inputs: torch.manual_seed(0) per layer, x ~ N(0,1) fp16,
w Kaiming-normal (fan_in, relu) fp32, no bias.
"""

import argparse
import ctypes
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "nova-wino-amd_amd")
for _p in (PKG_DIR, ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "per-layer ms + effective TFLOP/s, ResNet-50 3x3 s1 convs at B=1 and B=32"
LAYERS = [("conv2_x", 64, 56), ("conv3_x", 128, 28), ("conv4_x", 256, 14), ("conv5_x", 512, 7)]
BATCHES = [1, 32]
PEAK_HBM_GBS = 8000.0
PEAK_FP16_TFLOPS = 2500.0
KIND_NAMES = ["input", "gemm", "output", "fused"]
GRAPH_CALLS = 10  # forwards captured per layer graph (per-layer GPU time)
PATH_NAMES = {1: "3-pass", 2: "fused_rows", 3: "fused_block", 4: "windowed", 5: "fused_small",
              6: "two_pass", 7: "in_gemm"}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def direct_flops(B, C, K, Ho, Wo):
    return 2.0 * B * K * C * Ho * Wo * 9


def layer_roofline_us(B, C, K, H):
    Ho = Wo = H
    pmin = -(-Ho // 6) * -(-Wo // 6)
    f_alg = 2.0 * 64 * K * C * B * pmin
    b_alg = 2.0 * B * C * H * H + 2.0 * B * K * Ho * Wo + 2.0 * 64 * K * C
    return max(f_alg / (PEAK_FP16_TFLOPS * 1e12), b_alg / (PEAK_HBM_GBS * 1e9)) * 1e6


def kernel_alg_bytes(kind, B, C, K, H, name=""):
    """Algorithmic HBM bytes of one launch of a kernel kind (fp16 = 2 B):
    input transform reads x, writes V; GEMM reads U and V, writes M; output
    transform reads M, writes y; fused reads x and U, writes y -- except the
    two-pass path's second kernel (gemm_out_kernel), which reads V and U and
    writes y, and the input transform fused into the products (in_gemm_kernel,
    the GEMM kind of path 7), which reads x and U and writes M. Minimal tiling
    P = ceil(Ho/6)^2, channel pitch C rounded up to 8."""
    Cp = (C + 7) // 8 * 8
    Ho = H
    BP = B * (-(-Ho // 6)) ** 2
    x, y = 2 * B * C * H * H, 2 * B * K * Ho * Ho
    V, M, U = 2 * 64 * Cp * BP, 2 * 64 * K * BP, 2 * 64 * K * Cp
    if kind == "fused" and name.startswith("gemm_out"):
        return V + U + y
    if kind == "gemm" and name.startswith("in_gemm"):
        return x + U + M
    return {"input": x + V, "gemm": U + V + M, "output": M + y, "fused": x + U + y}[kind]


def kernel_alg_flops(kind, B, C, K, H):
    """Algorithmic MFMA FLOPs of one launch: the 64 Winograd-domain products,
    2*64*K*C*BP at minimal tiling (GEMM and fused kinds; the transforms are
    VALU work and count 0)."""
    BP = B * (-(-H // 6)) ** 2
    return 2.0 * 64 * K * C * BP if kind in ("gemm", "fused") else 0.0


def time_region(fn, reps, torch):
    """Mean ms per call over `reps` calls, CUDA events on the current stream."""
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


def time_steady(fn, reps, torch, tries=3, warm=10):
    """Steady-state ms per call: `warm` untimed calls, then the best of
    `tries` time_region runs. A host-bound call (batch-1 layers: ~2.7 us of
    HIP host time per kernel launch plus the module's Python) needs the
    warm-up: the first tens of calls after a synchronisation run slower."""
    for _ in range(warm):
        fn()
    return min(time_region(fn, reps, torch) for _ in range(tries))


def graph_of(fn, torch, n=1):
    """Capture n calls of fn into one HIP graph (after an eager warm-up);
    None if capture is not possible."""
    try:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                fn()
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(n):
                fn()
        torch.cuda.synchronize()
        return g
    except Exception as exc:  # report, do not hide: the field becomes null
        log(f"graph capture failed: {exc!r}")
        torch.cuda.synchronize()
        return None


def load_traffic(kernel_name):
    """HBM bytes per launch (mean over the step's layers) measured offline with
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes (profiles/traffic.json), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        data = json.load(f)
    for rec in data.get("kernels", []):
        if rec.get("kernel") == kernel_name:
            return rec.get("hbm_bytes_per_launch")
    return None


def load_mfma(kernel_name):
    """Executed MFMA FLOPs per launch (mean over the step's layers) of a kernel
    family, measured offline with rocprofv3 SQ_INSTS_VALU_MFMA_MOPS_F16
    (profiles/mfma.json), or None."""
    path = os.path.join(ROOT, "profiles", "mfma.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        data = json.load(f)
    for rec in data.get("kernels", []):
        if rec.get("kernel") == kernel_name:
            return {k: rec[k] for k in ("executed_flops_per_launch", "alg_flops_per_launch",
                                        "busy_per_512_flops") if k in rec}
    return None


COPY_MIB = 256


def pmc_workload(runs, reps, torch):
    """Short run for rocprofv3 --pmc passes: one plain device copy of a known
    size (the FETCH_SIZE/WRITE_SIZE calibration) and a few forwards per layer."""
    n = COPY_MIB * (1 << 20) // 2
    src = torch.ones(n, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)  # one elementwise kernel: reads and writes COPY_MIB each
    torch.cuda.synchronize()
    for r in runs:
        for _ in range(reps):
            r["mod"](r["x"])
    torch.cuda.synchronize()


# Kernel families, one per pipeline stage: the tile-block, lane-parallel and
# channels-last forms of a transform, and every tile configuration of the
# GEMM, belong to their stage's family. The roofline's dominant kernel is the
# family with the largest summed time per step.
KERNEL_FAMILY = {"input_transform_kernel": ("input_transform_kernel", "input_lp_kernel",
                                            "input_nhwc_kernel", "input_run_kernel"),
                 "wgemm": ("wgemm_kernel", "wgemm_lds_kernel", "wgemm_block_kernel"),
                 "output_transform_kernel": ("output_transform_kernel", "output_lp_kernel",
                                             "output_nhwc_kernel", "output_image_kernel"),
                 "in_gemm_kernel": ("in_gemm_kernel",)}
FAMILY_OF_KIND = {0: "input_transform_kernel", 1: "wgemm", 2: "output_transform_kernel"}


def family_of(kind, kname):
    """Kernel family of a profiled launch: its stage's family, except the
    input transform fused into the products (path 7), a family of its own."""
    if kname.startswith("in_gemm"):
        return "in_gemm_kernel"
    return FAMILY_OF_KIND.get(kind, kname)

NOVA_KERNELS = ["input_transform_kernel", "wgemm", "output_transform_kernel",
                "fused_block_kernel", "fused_small_kernel", "gemm_out_kernel", "in_gemm_kernel",
                "fused_kernel<1>",
                "fused_kernel<2>", "fused_kernel<4>"]


def _name_keys(name):
    """Prefixes of the kernel's name as it appears demangled and
    Itanium-mangled (int template arguments only), for matching rocprofv3
    records; trailing template arguments the library's short name leaves
    out (tuning depths) still match."""
    if name in KERNEL_FAMILY:
        return list(KERNEL_FAMILY[name])
    if "<" not in name:
        return [name]
    base, args = name.split("<", 1)
    args = [a.strip() for a in args.rstrip(">").split(",")]
    return [name.rstrip(">"), base + "I" + "".join(f"Li{a}E" for a in args)]


def pmc_rows(d, counter):
    """Per-dispatch means of one counter from the rocprofv3 --pmc database
    under d: [(kernel name, grid size, mean value, dispatches)], grouped by
    kernel name and grid size."""
    import glob
    import sqlite3

    dbs = sorted(glob.glob(os.path.join(d, "**", "*.db"), recursive=True))
    if not dbs:
        raise SystemExit(f"no rocprofv3 database under {d}")
    con = sqlite3.connect(dbs[-1])
    tabs = [r[0] for r in con.execute("select name from sqlite_master where type in "
                                      "('table','view')")]
    for t in tabs:
        cols = [c[1] for c in con.execute(f"pragma table_info('{t}')")]
        if {"kernel_name", "counter_name", "value"} <= set(cols):
            gcol = "grid_size" if "grid_size" in cols else "grid_size_x"
            rows = con.execute(f"select kernel_name, {gcol}, avg(value), count(*) from '{t}' "
                               f"where counter_name = ? group by kernel_name, {gcol}",
                               (counter,)).fetchall()
            return rows, dbs[-1]
    raise SystemExit(f"no counter table in {dbs[-1]}: {tabs}")


MFMA_COUNTERS = ("SQ_INSTS_VALU_MFMA_MOPS_F16", "SQ_VALU_MFMA_BUSY_CYCLES")
CLOCK_GHZ = 2.4  # MI355X peak engine clock (2.5 PFLOP/s = 256 CUs x 4 SIMDs x 1024 x 2.4 GHz)


def mfma_from(pmc_dir, bench_json, out_path, cus=256):
    """MFMA work of the library's product kernels from one rocprofv3 --pmc run
    of `bench.py --pmc-mode` with MFMA_COUNTERS: executed fp16 MFMA FLOPs per
    dispatch (SQ_INSTS_VALU_MFMA_MOPS_F16 counts multiply and add operations
    in units of 512) and the matrix units' busy cycles summed over SIMDs
    (SQ_VALU_MFMA_BUSY_CYCLES). Over each family's event-timed launch
    duration in the unprofiled bench line (bench_json) they give the share of
    the 2.5 PFLOP/s dense fp16 peak reached and the share of SIMD cycles the
    matrix units were busy; busy cycles per 512 FLOPs tell the instruction's
    rate (0.5 = the full dense rate of v_mfma_f32_16x16x32_f16)."""
    with open(bench_json) as f:
        line = json.loads([ln for ln in f if ln.startswith("{")][-1])
    fams = line.get("kernel_families", {})
    per = {c: pmc_rows(pmc_dir, c)[0] for c in MFMA_COUNTERS}
    data = {"method": "rocprofv3 --pmc " + " ".join(MFMA_COUNTERS) + " of bench.py --pmc-mode; "
                      "executed FLOPs = 512 x SQ_INSTS_VALU_MFMA_MOPS_F16; busy share = "
                      "SQ_VALU_MFMA_BUSY_CYCLES / (bench avg_launch_us x "
                      f"{CLOCK_GHZ} GHz x {cus} CUs x 4 SIMDs)",
            "peak_tflops": PEAK_FP16_TFLOPS, "clock_ghz": CLOCK_GHZ, "kernels": []}
    for name in ("wgemm", "fused_block_kernel", "fused_small_kernel", "gemm_out_kernel",
                 "in_gemm_kernel", "fused_kernel<1>", "fused_kernel<2>", "fused_kernel<4>"):
        sel = {c: [r for r in per[c] if any(k in r[0] for k in _name_keys(name))]
               for c in MFMA_COUNTERS}
        mops = sel["SQ_INSTS_VALU_MFMA_MOPS_F16"]
        if not mops:
            continue
        n = sum(r[3] for r in mops)
        flops = sum(r[2] * r[3] for r in mops) / n * 512.0
        busy_rows = sel["SQ_VALU_MFMA_BUSY_CYCLES"]
        busy = (sum(r[2] * r[3] for r in busy_rows) / sum(r[3] for r in busy_rows)
                if busy_rows else None)
        bmap = {(r[0], r[1]): r[2] for r in busy_rows}
        grids = [{"kernel": r[0], "grid": r[1], "dispatches": r[3],
                  "executed_gflop": round(r[2] * 512.0 / 1e9, 4),
                  "busy_cycles": round(bmap.get((r[0], r[1]), 0.0)),
                  "busy_per_512_flops": (round(bmap[(r[0], r[1])] / r[2], 3)
                                         if r[2] and (r[0], r[1]) in bmap else None)}
                 for r in mops]
        rec = {"kernel": name, "executed_flops_per_launch": round(flops), "by_grid": grids}
        if busy is not None:
            rec["busy_cycles_per_launch"] = round(busy)
            rec["busy_per_512_flops"] = round(busy / (flops / 512.0), 3) if flops else None
        fam = fams.get(name)
        if fam and "alg_gflop_per_launch" in fam:
            rec["alg_flops_per_launch"] = round(fam["alg_gflop_per_launch"] * 1e9)
            rec["avg_launch_us"] = fam["avg_launch_us"]
            tf = flops / (fam["avg_launch_us"] * 1e-6) / 1e12
            rec["executed_tflops"] = round(tf, 1)
            rec["frac_of_peak"] = round(tf / PEAK_FP16_TFLOPS, 4)
            if busy is not None:
                simd_cycles = fam["avg_launch_us"] * 1e-6 * CLOCK_GHZ * 1e9 * cus * 4
                rec["mfma_busy_frac"] = round(busy / simd_cycles, 4)
        data["kernels"].append(rec)
    with open(out_path, "w") as f:
        json.dump(data, f, indent=1)
    write_mfma_summary(data, os.path.join(os.path.dirname(out_path),
                                          "mfma_resnet50_3x3s1_b1_b32.md"))
    print(json.dumps(data))


def write_mfma_summary(data, path):
    """Markdown summary of mfma.json."""
    short = lambda n, k=60: (n[:k] + "…") if len(n) > k else n  # noqa: E731
    lines = [
        "# MFMA work per launch, product kernels, ResNet-50 3x3 s1 layers at B=1 and B=32",
        "",
        "Commands (from the repository root, on one MI355X):",
        "",
        "```",
        "python3 -u bench.py --details out/bench_details.json > out/bench_line.json",
        "cd /tmp && export TMPDIR=/tmp && cd -",
        "timeout -s KILL 120 rocprofv3 --pmc " + " ".join(MFMA_COUNTERS)
        + " -d out/pmc_mfma -o pmc -- python3 -u bench.py --pmc-mode",
        "python3 bench.py --mfma-from out/pmc_mfma out/bench_line.json"
        "   # -> profiles/mfma.json + this file",
        "```",
        "",
        data["method"] + ".",
        "",
        "| kernel | grid (threads) | dispatches | executed GFLOP | MFMA busy cycles | "
        "busy cycles per 512 FLOPs |",
        "|---|---:|---:|---:|---:|---:|",
    ]
    for k in data["kernels"]:
        for g in k["by_grid"]:
            lines.append(f"| `{short(g['kernel'])}` | {g['grid']} | {g['dispatches']} | "
                         f"{g['executed_gflop']} | {g['busy_cycles']} | "
                         f"{g['busy_per_512_flops']} |")
    lines += ["", "| family | executed GFLOP / launch | algorithmic GFLOP / launch | "
                  "bench avg_launch_us | executed TFLOP/s | of 2.5 PFLOP/s | MFMA busy share |",
              "|---|---:|---:|---:|---:|---:|---:|"]
    for k in data["kernels"]:
        alg = k.get("alg_flops_per_launch")
        lines.append(f"| {k['kernel']} | {k['executed_flops_per_launch'] / 1e9:.4f} | "
                     f"{(alg / 1e9) if alg else float('nan'):.4f} | {k.get('avg_launch_us')} | "
                     f"{k.get('executed_tflops')} | {k.get('frac_of_peak')} | "
                     f"{k.get('mfma_busy_frac')} |")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def traffic_from(fetch_dir, write_dir, out_path):
    """HBM bytes per launch of each library kernel from two rocprofv3 --pmc runs
    of `bench.py --pmc-mode` (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch),
    each scaled by the same counter's reading for the known-size copy kernel.
    The figure kept per kernel is the mean over the layers it ran on, the same
    averaging as the bench line's avg_launch_us."""
    def read(d, counter):
        rows, db = pmc_rows(d, counter)
        copy = [r for r in rows if "copy" in r[0].lower() or "elementwise" in r[0].lower()]
        copy = [r for r in copy if r[2] > COPY_MIB * 1024 * 0.5]
        if not copy:
            raise SystemExit(f"{counter}: calibration copy not found in {db}")
        copy_kib = min(copy, key=lambda r: abs(r[2] - COPY_MIB * 1024))[2]
        factor = COPY_MIB * 1024.0 / copy_kib
        per = {}
        for name in NOVA_KERNELS:
            kern = [r for r in rows if any(k in r[0] for k in _name_keys(name))]
            if kern:
                # mean over dispatches (a row can hold several layers that
                # share a kernel and a grid size)
                per[name] = (sum(r[2] * r[3] for r in kern) / sum(r[3] for r in kern)
                             * 1024.0 * factor,
                             [(r[1], round(r[2], 1)) for r in kern])
        return per, factor, copy_kib

    fetch, ff, fcopy = read(fetch_dir, "FETCH_SIZE")
    write, wf, wcopy = read(write_dir, "WRITE_SIZE")
    data = {"method": "rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (separate runs) of "
                      "bench.py --pmc-mode; each scaled by copy_bytes / counter reading of a "
                      f"{COPY_MIB} MiB device copy in the same run",
            "copy_bytes": COPY_MIB * (1 << 20), "fetch_copy_kib": round(fcopy, 1),
            "write_copy_kib": round(wcopy, 1), "fetch_scale": round(ff, 4),
            "write_scale": round(wf, 4), "kernels": []}
    for name in NOVA_KERNELS:
        if name in fetch and name in write:
            data["kernels"].append({
                "kernel": name,
                "hbm_bytes_per_launch": round(fetch[name][0] + write[name][0]),
                "fetch_bytes_per_launch": round(fetch[name][0]),
                "write_bytes_per_launch": round(write[name][0]),
                "fetch_kib_by_grid": fetch[name][1], "write_kib_by_grid": write[name][1]})
    with open(out_path, "w") as f:
        json.dump(data, f, indent=1)
    write_traffic_summary(data, os.path.join(os.path.dirname(out_path),
                                             "traffic_resnet50_3x3s1_b1_b32.md"))
    print(json.dumps(data))


def kernel_stats_from(trace_dir, bench_json, out_path):
    """Markdown summary of a `rocprofv3 --kernel-trace --stats --output-format
    csv` run of bench.py: the --stats table, the library's kernels per launch
    grid, and the agreement of each kernel family's mean duration in the trace
    with the unprofiled bench line (bench_json: a file holding that line)."""
    import csv
    import glob

    def one(pattern):
        files = sorted(glob.glob(os.path.join(trace_dir, "**", pattern), recursive=True))
        if not files:
            raise SystemExit(f"no {pattern} under {trace_dir}")
        with open(files[-1]) as f:
            return list(csv.DictReader(f))

    stats, trace = one("*kernel_stats.csv"), one("*kernel_trace.csv")
    with open(bench_json) as f:
        line = json.loads([ln for ln in f if ln.startswith("{")][-1])
    short = lambda n, k=72: (n[:k] + "…") if len(n) > k else n  # noqa: E731
    lines = [
        "# Library kernels, ResNet-50 3x3 s1 layers at B=1 and B=32 (bench.py default workload)",
        "",
        "Commands (from the repository root, on one MI355X):",
        "",
        "```",
        "python3 -u bench.py --details out/bench_details.json > out/bench_line.json",
        "cd /tmp && export TMPDIR=/tmp && cd - && rocprofv3 --kernel-trace --stats "
        "--output-format csv -d out/prof_bench -o bench -- python3 -u bench.py "
        "--no-extra --no-cpu",
        "python3 bench.py --kernel-stats-from out/prof_bench out/bench_line.json"
        "   # -> this file",
        "```",
        "",
        "## rocprofv3 --stats (kernel_stats.csv), all kernels of the run",
        "",
        "| kernel | calls | avg us | min us | max us | % time |",
        "|---|---:|---:|---:|---:|---:|",
    ]
    for r in stats[:20]:
        lines.append(f"| `{short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.3f} | "
                     f"{float(r['MinNs']) / 1e3:.3f} | {float(r['MaxNs']) / 1e3:.3f} | "
                     f"{float(r['Percentage']):.2f} |")
    lines += ["", "## Library kernels per launch grid (kernel_trace.csv, End - Start)", "",
              "| kernel | grid (threads) | calls | mean us | median us |",
              "|---|---:|---:|---:|---:|"]
    groups = {}
    for r in trace:
        if "nova" not in r["Kernel_Name"]:
            continue
        key = (r["Kernel_Name"], int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"]))
        groups.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    for (name, grid), v in sorted(groups.items()):
        lines.append(f"| `{short(name, 60)}` | {grid} | {len(v)} | {statistics.mean(v):.3f} | "
                     f"{statistics.median(v):.3f} |")
    lines += ["", "## Agreement with the bench line", "",
              "The bench line's per-family times are hipEvents recorded by each kernel's own "
              "dispatch packet over a timed region of the unprofiled run (first command); the "
              "trace's are End - Start of every launch of the family in the profiled run "
              "(call-weighted over the step's layers, as the bench averages them). The event "
              "pair also holds each dispatch's wait behind the kernel before it (the barrier "
              "and cache flush between dependent launches), which the trace leaves out: about "
              "0.1-1.3 us per launch, so the ratio runs from 1.0 to 1.3 with the box.", "",
              "Fractions of 8 TB/s use the family's algorithmic bytes per launch (the bench "
              "line's achieved GB/s x its event-timed launch) over each duration: the bench's "
              "warm and cold event times, and the trace's warm End - Start.", "",
              "| family | bench avg_launch_us | rocprofv3 mean us | calls | ratio | "
              "alg MB/launch | frac (events, warm) | frac (trace, warm) | frac (events, cold) |",
              "|---|---:|---:|---:|---:|---:|---:|---:|---:|"]
    fams = line.get("kernel_families", {})
    for fam, rec in fams.items():
        keys = KERNEL_FAMILY.get(fam, (fam,))
        d = [v for (name, _), vs in groups.items() for v in vs if any(k in name for k in keys)]
        if not d:
            continue
        m = statistics.mean(d)
        alg = rec["achieved_gbs"] * rec["avg_launch_us"] * 1e3  # bytes per launch
        lines.append(f"| {fam} | {rec['avg_launch_us']:.3f} | {m:.3f} | {len(d)} | "
                     f"{rec['avg_launch_us'] / m:.3f} | {alg / 1e6:.2f} | "
                     f"{rec['frac_hbm']:.4f} | {alg / (m * 1e-6) / 1e9 / PEAK_HBM_GBS:.4f} | "
                     f"{rec.get('frac_hbm_cold', float('nan')):.4f} |")
    rl = line["roofline"]
    warm = (f"; warm loop {rl['avg_launch_us_warm']} us, {rl['frac_warm']}"
            if "frac_warm" in rl else "")
    lines += ["", f"Dominant family in the bench line: `{rl['kernel']}`, avg_launch_us = "
                  f"{rl['avg_launch_us']} ({rl.get('cache', 'warm')}), achieved "
                  f"{rl['achieved']} GB/s = {rl['frac']} of {rl['peak']} GB/s{warm} "
                  f"(bench value {line['value']} TFLOP/s, {line['ms_per_step']} ms per step)."]
    with open(out_path, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(f"wrote {out_path}")


def write_traffic_summary(data, path):
    """Markdown summary of traffic.json (the figures the bench line uses)."""
    lines = [
        "# HBM traffic per launch, library kernels, ResNet-50 3x3 s1 layers at B=1 and B=32",
        "",
        "Commands (from the repository root, on one MI355X; two passes, one counter each):",
        "",
        "```",
        "cd /tmp && export TMPDIR=/tmp && cd -",
        "timeout -s KILL 120 rocprofv3 --pmc FETCH_SIZE -d out/pmc_fetch -o pmc -- "
        "python3 -u bench.py --pmc-mode",
        "timeout -s KILL 120 rocprofv3 --pmc WRITE_SIZE -d out/pmc_write -o pmc -- "
        "python3 -u bench.py --pmc-mode",
        "python3 bench.py --traffic-from out/pmc_fetch out/pmc_write   "
        "# -> profiles/traffic.json + this file",
        "```",
        "",
        f"Calibration: the same run launches one elementwise kernel that reads and writes "
        f"{COPY_MIB} MiB. FETCH_SIZE read {data['fetch_copy_kib']} KiB for its "
        f"{COPY_MIB * 1024} KiB of reads (scale {data['fetch_scale']}), WRITE_SIZE "
        f"{data['write_copy_kib']} KiB for its writes (scale {data['write_scale']}). Every "
        "kernel's counters are multiplied by these factors.",
        "",
        "| kernel | grid (threads) | FETCH KiB (raw) | WRITE KiB | HBM MB (scaled) |",
        "|---|---:|---:|---:|---:|",
    ]
    for k in data["kernels"]:
        writes = dict(k["write_kib_by_grid"])
        for grid, fkib in k["fetch_kib_by_grid"]:
            wkib = writes.get(grid, 0.0)
            mb = (fkib * data["fetch_scale"] + wkib * data["write_scale"]) * 1024 / 1e6
            lines.append(f"| `{k['kernel']}` | {grid} | {fkib} | {wkib} | {mb:.3f} |")
        lines.append(f"| **{k['kernel']} mean per launch** | | | | "
                     f"**{k['hbm_bytes_per_launch'] / 1e6:.3f}** |")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def cpu_model():
    """The host CPU's model name (the `lscpu` "Model name" field), read from
    /proc/cpuinfo; falls back to platform.processor()."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(layers_spec, budget_s, threads):
    """Time the CPU oracle (C restatement of the reference arithmetic, OpenMP)
    on a bounded sample: every B=1 layer, and each B=32 layer on `sample_b`
    images (work and FLOPs scale linearly in B)."""
    import numpy as np
    import torch

    from oracle import oracle as O

    O.set_threads(threads)
    torch.set_num_threads(threads)
    sample_b = 2
    jobs = []
    for (name, C, H), B in layers_spec:
        b = B if B == 1 else sample_b
        torch.manual_seed(0)
        x = torch.randn(b, C, H, H).half().numpy()
        w = torch.empty(C, C, 3, 3)
        torch.nn.init.kaiming_normal_(w, mode="fan_in", nonlinearity="relu")
        jobs.append((name, B, b, x, w.numpy()))
    flops = 0.0
    secs = 0.0
    conv_secs = 0.0
    conv_flops = 0.0
    rounds = 0
    t_start = time.perf_counter()
    while rounds == 0 or (time.perf_counter() - t_start) < budget_s:
        for name, B, b, x, w in jobs:
            t0 = time.perf_counter()
            O.conv2d(x, w, 1)
            secs += time.perf_counter() - t0
            flops += direct_flops(b, x.shape[1], w.shape[0], x.shape[2], x.shape[3])
        rounds += 1
        if rounds >= 50:
            break
    # F.conv2d fp32 on the same sample, once per job (reference CPU path (b))
    import torch.nn.functional as F

    with torch.no_grad():
        for name, B, b, x, w in jobs:
            xt, wt = torch.from_numpy(x.astype(np.float32)), torch.from_numpy(w)
            F.conv2d(xt, wt, padding=1)
            t0 = time.perf_counter()
            F.conv2d(xt, wt, padding=1)
            conv_secs += time.perf_counter() - t0
            conv_flops += direct_flops(b, x.shape[1], w.shape[0], x.shape[2], x.shape[3])
    return {
        "value": flops / secs / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle NOVA F(6,3) path (C, OpenMP {threads} threads) over the 4 ResNet-50 "
                   f"layers at B=1 and on {sample_b} of the 32 images per B=32 layer, "
                   f"{rounds} round(s), {secs:.1f} s; effective TFLOP/s with the direct-conv "
                   "FLOP count"),
        "ms_per_step_equiv": 1e3 * secs / rounds * (
            sum(direct_flops(B, C, C, H, H) for (n, C, H), B in layers_spec)
            / (flops / rounds)),
        "fconv2d_fp32_tflops": conv_flops / conv_secs / 1e12,
        "host": cpu_model(),
        "arch": platform.machine(),
        "os_cpu_count": os.cpu_count(),
    }


FLUSH_MIB = 512  # > the 256 MB memory-side cache + 8 x 4 MB of L2


def cold_measurements(runs, lib, torch, reps):
    """Cold-cache numbers. Before every forward a 512 MiB device write evicts
    the memory-side cache and the L2s, so the forward's inputs (x, U) come
    from HBM. Per layer: the median forward time between a hipEvent pair
    (r["cold_ms"]). Per kernel: each kernel's own duration from the events
    its dispatch packet records (nova_profile_enable), averaged over the same
    kind of cold forwards (r["event_cold"], ms per kind). Inside a cold
    three-pass forward V and M are still written and read back on chip: that
    is the pipeline's own behaviour, not a warm start."""
    flush = torch.empty(FLUSH_MIB << 20, dtype=torch.uint8, device="cuda")
    for r in runs:
        ts = []
        for _ in range(reps):
            flush.fill_(1)
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            r["mod"](r["x"])
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        r["cold_ms"] = statistics.median(ts)
    tot = (ctypes.c_double * 4)()
    cnt = (ctypes.c_longlong * 4)()
    for r in runs:
        h = r["mod"]._handle.h
        lib.nova_profile_enable(h, 1)
        for _ in range(reps):
            flush.fill_(1)
            r["mod"](r["x"])
        torch.cuda.synchronize()
        if lib.nova_profile_read(h, tot, cnt) < 0:
            raise RuntimeError(lib.nova_get_last_error_message().decode())
        lib.nova_profile_enable(h, 0)
        r["event_cold"] = {k: tot[k] / cnt[k] for k in range(4) if cnt[k] > 0}
    del flush
    torch.cuda.synchronize()


EXTRA_LAYERS = [
    # (name, B, C, K, H): BASELINE config 3 (B=128), 4 (SD-1.5, B=2), 5 (SDXL B=1,
    # DenseNet-161 bottleneck 192->48 B=1)
    ("r50_conv2_x", 128, 64, 64, 56), ("r50_conv3_x", 128, 128, 128, 28),
    ("r50_conv4_x", 128, 256, 256, 14), ("r50_conv5_x", 128, 512, 512, 7),
    ("sd15_320@64", 2, 320, 320, 64), ("sd15_640@32", 2, 640, 640, 32),
    ("sd15_1280@16", 2, 1280, 1280, 16), ("sd15_1280@8", 2, 1280, 1280, 8),
    ("sd15_320to640@32", 2, 320, 640, 32), ("sd15_640to1280@16", 2, 640, 1280, 16),
    ("sd15_1280to640@32", 2, 1280, 640, 32), ("sd15_640to320@64", 2, 640, 320, 64),
    ("sdxl_320@128", 1, 320, 320, 128), ("sdxl_640@64", 1, 640, 640, 64),
    ("sdxl_1280@32", 1, 1280, 1280, 32),
    ("dn161_192to48@56", 1, 192, 48, 56), ("dn161_192to48@28", 1, 192, 48, 28),
    ("dn161_192to48@14", 1, 192, 48, 14), ("dn161_192to48@7", 1, 192, 48, 7),
]


def extra_measurements(runs, lib, torch, nn, nw, reps):
    """Per-layer NOVA vs MIOpen on the other BASELINE configs and the full
    random-init ResNet-50 forward with and without surgery."""
    dev = torch.device("cuda:0")
    path_names = PATH_NAMES
    out = {"layers": []}
    for name, B, C, K, H in EXTRA_LAYERS:
        torch.manual_seed(0)
        x = torch.randn(B, C, H, H, device=dev).half()
        w = torch.empty(K, C, 3, 3)
        nn.init.kaiming_normal_(w, mode="fan_in", nonlinearity="relu")
        mod = nw.NovaWinogradConv2d(C, K, kernel_size=3, padding=1).to(dev)
        mio = nn.Conv2d(C, K, 3, padding=1, bias=False).to(dev).half()
        with torch.no_grad():
            mod.weight.copy_(w.to(dev))
            mio.weight.copy_(w.half().to(dev))
            tn = time_steady(lambda: mod(x), reps, torch)
            tm = time_steady(lambda: mio(x), reps, torch)
        f = direct_flops(B, C, K, H, H)
        rec = {"layer": name, "B": B, "C": C, "K": K, "H": H,
               "path": path_names.get(lib.nova_get_last_path(mod._handle.h), "?"),
               "nova_ms": round(tn, 5), "miopen_ms": round(tm, 5),
               "nova_tflops": round(f / (tn * 1e-3) / 1e12, 2),
               "speedup_vs_miopen": round(tm / tn, 3),
               "roofline_frac": round(layer_roofline_us(B, C, K, H) / (tn * 1e3), 4)}
        out["layers"].append(rec)
        log(f"{name:18s} B={B:<3d} {rec['path']:11s} nova {tn*1e3:9.2f} us  miopen "
            f"{tm*1e3:9.2f} us")
        del x, mod, mio
    # channels-last activations (an extension): the headline layers at B=32
    # with NHWC input and output, NOVA (NHWC kernels) vs MIOpen on the same
    # channels-last tensor
    out["nhwc"] = []
    for r in runs:
        if r["B"] == 1:
            continue
        xc = r["x"].contiguous(memory_format=torch.channels_last)
        mio = r["mio"].to(memory_format=torch.channels_last)
        with torch.no_grad():
            tn = time_steady(lambda: r["mod"](xc), reps, torch)
            tm = time_steady(lambda: mio(xc), reps, torch)
        rec = {"layer": r["name"], "B": r["B"],
               "path": path_names.get(lib.nova_get_last_path(r["mod"]._handle.h), "?"),
               "nova_ms": round(tn, 5), "miopen_ms": round(tm, 5),
               "speedup_vs_miopen": round(tm / tn, 3)}
        out["nhwc"].append(rec)
        log(f"{r['name']:8s} B={r['B']:<3d} NHWC {rec['path']:11s} nova {tn*1e3:8.2f} us  "
            f"miopen {tm*1e3:8.2f} us")
        r["mio"].to(memory_format=torch.contiguous_format)
        del xc
    # full ResNet-50, eager, MIOpen fp16 vs after surgery
    import copy
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from resnet50 import ResNet50

    out["resnet50"] = []
    for B in (1, 32):
        torch.manual_seed(0)
        m16 = ResNet50().eval().to(dev).half()
        nova = copy.deepcopy(m16)
        nw.replace_conv2d_with_nova(nova, verbose=False)
        x = torch.randn(B, 3, 224, 224, device=dev).half()
        with torch.no_grad():
            m16(x)
            nova(x)
            t16 = time_region(lambda: m16(x), 20, torch)
            tn = time_region(lambda: nova(x), 20, torch)
            # the eager forward is bound by Python launch overhead (~160 modules);
            # HIP-graph replay shows the GPU time of each model
            g16, gn = graph_of(lambda: m16(x), torch), graph_of(lambda: nova(x), torch)
            tg16 = time_region(g16.replay, 20, torch) if g16 is not None else None
            tgn = time_region(gn.replay, 20, torch) if gn is not None else None
        rec = {"B": B, "miopen_ms": round(t16, 4), "nova_ms": round(tn, 4),
               "speedup": round(t16 / tn, 3)}
        if tg16 is not None and tgn is not None:
            rec.update({"miopen_graph_ms": round(tg16, 4), "nova_graph_ms": round(tgn, 4),
                        "graph_speedup": round(tg16 / tgn, 3)})
        out["resnet50"].append(rec)
        log(f"resnet50 B={B:<3d} model forward: miopen {t16:8.3f} ms  nova {tn:8.3f} ms"
            + (f"  | graph: miopen {tg16:7.3f} ms  nova {tgn:7.3f} ms"
               if tg16 is not None and tgn is not None else ""))
        del m16, nova, x
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layer-reps", type=int, default=200)
    ap.add_argument("--kernel-reps", type=int, default=100)
    ap.add_argument("--cold-reps", type=int, default=20,
                    help="cold-cache forwards per layer (a 512 MiB write before each)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-miopen", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--details", default="", help="write the full per-layer report here")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the extra measurements (BASELINE configs 3-5 layers, full "
                         "ResNet-50)")
    ap.add_argument("--pmc-mode", action="store_true",
                    help="short run for rocprofv3 --pmc passes (copy calibration + forwards)")
    ap.add_argument("--kernel-stats-from", nargs=2, metavar=("TRACE_DIR", "BENCH_JSON"),
                    help="write profiles/kernels_resnet50_3x3s1_b1_b32.md from a rocprofv3 "
                         "kernel-trace run and the unprofiled bench line")
    ap.add_argument("--mfma-from", nargs=2, metavar=("PMC_DIR", "BENCH_JSON"),
                    help="write profiles/mfma.json + its summary from a rocprofv3 --pmc run "
                         "with the MFMA counters and a bench line")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn two --pmc-mode profiles into profiles/traffic.json and exit")
    args = ap.parse_args()

    if args.kernel_stats_from:
        kernel_stats_from(args.kernel_stats_from[0], args.kernel_stats_from[1],
                          os.path.join(ROOT, "profiles", "kernels_resnet50_3x3s1_b1_b32.md"))
        return
    if args.traffic_from:
        traffic_from(args.traffic_from[0], args.traffic_from[1],
                     os.path.join(ROOT, "profiles", "traffic.json"))
        return
    if args.mfma_from:
        mfma_from(args.mfma_from[0], args.mfma_from[1], os.path.join(ROOT, "profiles", "mfma.json"))
        return

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the NOVA conv would shard by batch or by output channel, with no "
              "exchange during a layer). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import torch.nn as nn

    import nova_winograd as nw
    from nova_winograd.ops import get_lib

    lib = get_lib()
    dev = torch.device("cuda:0")
    prop = torch.cuda.get_device_properties(dev)
    log(f"device: {prop.name} ({getattr(prop, 'gcnArchName', '?')}), "
        f"{prop.multi_processor_count} CUs, lib {lib.nova_version().decode()}")

    spec = [(layer, B) for B in BATCHES for layer in LAYERS]
    runs = []
    for (name, C, H), B in spec:
        torch.manual_seed(0)
        x = torch.randn(B, C, H, H).half().to(dev)
        w = torch.empty(C, C, 3, 3)
        nn.init.kaiming_normal_(w, mode="fan_in", nonlinearity="relu")
        mod = nw.NovaWinogradConv2d(C, C, kernel_size=3, padding=1).to(dev)
        with torch.no_grad():
            mod.weight.copy_(w.to(dev))
        mio = nn.Conv2d(C, C, 3, padding=1, bias=False).to(dev).half()
        with torch.no_grad():
            mio.weight.copy_(w.half().to(dev))
        runs.append({"name": name, "B": B, "C": C, "K": C, "H": H, "x": x, "mod": mod,
                     "mio": mio})

    total_flops = sum(direct_flops(r["B"], r["C"], r["K"], r["H"], r["H"]) for r in runs)

    def step():
        for r in runs:
            r["mod"](r["x"])

    if args.pmc_mode:
        with torch.no_grad():
            step()
            pmc_workload(runs, 3, torch)
        return

    with torch.no_grad():
        # MIOpen's first forward of each layer (its solution search) first,
        # then the W warm-up steps (filter transforms, workspaces) right before
        # the timed region: run between the warm-up and the timed steps, the
        # search left the first 20 timed steps 7 % slower (0.145 vs 0.135 ms)
        for r in runs:
            r["mio"](r["x"])
        torch.cuda.synchronize()
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()

        # ---- timed region: exactly K steps -----------------------------------
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        ms_per_step = (t1 - t0) * 1e3 / args.steps
        value = total_flops / (ms_per_step * 1e-3) / 1e12

        # ---- per-kernel durations over a timed region: the same K steps
        # again, every kernel of every forward timed by a pair of hipEvents
        # that its own dispatch packet records on the library's stream
        # (nova_profile_enable: hipExtLaunchKernelGGL start/stop events), i.e.
        # the kernel's execution without the dispatch gap in front of it.
        for r in runs:
            lib.nova_profile_enable(r["mod"]._handle.h, 1)
        torch.cuda.synchronize()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        tot = (ctypes.c_double * 4)()
        cnt = (ctypes.c_longlong * 4)()
        for r in runs:
            h = r["mod"]._handle.h
            if lib.nova_profile_read(h, tot, cnt) < 0:
                raise RuntimeError(lib.nova_get_last_error_message().decode())
            lib.nova_profile_enable(h, 0)
            r["event"] = {k: tot[k] / cnt[k] for k in range(4) if cnt[k] > 0}

        # ---- cold caches: per layer and per kernel (a 512 MiB write before
        # every forward)
        cold_measurements(runs, lib, torch, args.cold_reps)

        # ---- cross-check: each kernel of each layer's forward re-launched
        # back to back by the library (nova_profile_replay), one hipEvent pair
        # on its stream around the loop -> mean launch time without the
        # dependent-launch gap.
        kernels = {}
        for r in runs:
            y_keep = r["mod"](r["x"])  # the forward whose launches are replayed
            h = r["mod"]._handle.h
            r["kernels"] = {}
            for k in range(4):
                kname = lib.nova_profile_kernel_name(h, k).decode()
                if not kname or k not in r["event"]:
                    continue
                per = lib.nova_profile_replay(h, k, args.kernel_reps)
                if per < 0:
                    lib.nova_get_last_error()  # kind not launched by this path
                    continue
                ev = r["event"][k]
                ab = kernel_alg_bytes(KIND_NAMES[k], r["B"], r["C"], r["K"], r["H"], kname)
                r["kernels"][KIND_NAMES[k]] = {"kernel": kname, "avg_us": ev * 1e3,
                                              "replay_us": per * 1e3, "alg_bytes": ab,
                                              "gbs": ab / (ev * 1e-3) / 1e9}
                fam = family_of(k, kname)
                agg = kernels.setdefault(fam, {"ms": 0.0, "replay_ms": 0.0, "launches": 0,
                                               "bytes": 0.0, "flops": 0.0, "by_layer": [],
                                               "members": {}, "ms_cold": 0.0})
                agg["ms_cold"] += r["event_cold"].get(k, ev)
                r["kernels"][KIND_NAMES[k]]["avg_us_cold"] = r["event_cold"].get(k, ev) * 1e3
                agg["flops"] += kernel_alg_flops(KIND_NAMES[k], r["B"], r["C"], r["K"], r["H"])
                agg["members"][kname] = agg["members"].get(kname, 0) + 1
                agg["ms"] += ev
                agg["replay_ms"] += per
                agg["launches"] += 1
                agg["bytes"] += ab
                agg["by_layer"].append(f"{r['name']}_b{r['B']}")
            torch.cuda.synchronize()
            del y_keep

        # ---- per-layer timings: NOVA vs MIOpen, eager and graph -----------------
        for r in runs:
            mod, mio, x = r["mod"], r["mio"], r["x"]
            r["nova_ms"] = time_region(lambda: mod(x), args.layer_reps, torch)
            r["path"] = PATH_NAMES.get(lib.nova_get_last_path(mod._handle.h), "?")
            if not args.no_miopen:
                r["miopen_ms"] = time_region(lambda: mio(x), args.layer_reps, torch)
            if not args.no_graph:
                # ten forwards per graph: one replay's host cost (~16-20 us)
                # is spread over ten layers' GPU time, so this reads the GPU
                g = graph_of(lambda: mod(x), torch, GRAPH_CALLS)
                reps = max(10, args.layer_reps // GRAPH_CALLS)
                r["nova_graph_ms"] = (time_region(g.replay, reps, torch) / GRAPH_CALLS
                                      if g is not None else None)
                if not args.no_miopen:
                    gm = graph_of(lambda: mio(x), torch, GRAPH_CALLS)
                    r["miopen_graph_ms"] = (time_region(gm.replay, reps, torch) / GRAPH_CALLS
                                            if gm is not None else None)

    # ---- dominant kernel roofline -----------------------------------------------
    dom_name, dom = max(kernels.items(), key=lambda kv: kv[1]["ms"])
    avg_s = dom["ms"] / dom["launches"] * 1e-3
    bytes_per_launch = dom["bytes"] / dom["launches"]  # launches: one per layer per step
    achieved = bytes_per_launch / avg_s / 1e9
    dom_desc = ",".join(sorted(set(dom["by_layer"])))
    # Headline fraction = cold launches (a 512 MiB write before each forward,
    # so x and U come from HBM; see cold_measurements): at these sizes a warm
    # loop keeps U in the 256 MB memory-side cache and can read above the HBM
    # roofline. The warm steady-state figures (the ones a kernel trace of the
    # same loop reproduces) stay beside them.
    avg_cold_s = dom["ms_cold"] / dom["launches"] * 1e-3
    achieved_cold = bytes_per_launch / avg_cold_s / 1e9
    roofline = {
        "bound": "hbm",
        "achieved": round(achieved_cold, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(achieved_cold / PEAK_HBM_GBS, 4),
        "traffic": load_traffic(dom_name),
        "kernel": dom_name,
        "avg_launch_us": round(avg_cold_s * 1e6, 3),
        "timing": "hipEvents recorded by each kernel's dispatch packet over a timed region of K steps",
        "cache": "cold (512 MiB write before each forward)",
        "avg_launch_us_warm": round(avg_s * 1e6, 3),
        "achieved_warm": round(achieved, 1),
        "frac_warm": round(achieved / PEAK_HBM_GBS, 4),
        "replay_avg_launch_us": round(dom["replay_ms"] / dom["launches"] * 1e3, 3),
        "members": dom["members"],
        "alg_bytes_per_launch": round(bytes_per_launch),
        "launches_per_step": dom["launches"],
        "share_of_kernel_time": round(dom["ms"] / sum(v["ms"] for v in kernels.values()), 3),
        "layers": dom_desc,
    }
    if dom["flops"] > 0:
        # the same launches against the dense fp16 MFMA peak (algorithmic
        # FLOPs; profiles/mfma.json holds the executed ones from the counters)
        tf = dom["flops"] / (dom["ms"] * 1e-3) / 1e12
        roofline["mfma"] = {"achieved": round(tf, 1), "peak": PEAK_FP16_TFLOPS,
                            "unit": "TFLOP/s", "frac": round(tf / PEAK_FP16_TFLOPS, 4),
                            "alg_flops_per_launch": round(dom["flops"] / dom["launches"]),
                            "counters": load_mfma(dom_name)}

    families = {
        fam: {"avg_launch_us": round(v["ms"] / v["launches"] * 1e3, 3),
              "launches_per_step": v["launches"],
              "ms_per_step": round(v["ms"], 4),
              "achieved_gbs": round(v["bytes"] / (v["ms"] * 1e-3) / 1e9, 1),
              "frac_hbm": round(v["bytes"] / (v["ms"] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
              "avg_launch_us_cold": round(v["ms_cold"] / v["launches"] * 1e3, 3),
              "frac_hbm_cold": round(v["bytes"] / (v["ms_cold"] * 1e-3) / 1e9 / PEAK_HBM_GBS,
                                     4)}
        for fam, v in sorted(kernels.items(), key=lambda kv: -kv[1]["ms"])}
    for fam, v in kernels.items():
        if v["flops"] > 0:
            tf = v["flops"] / (v["ms"] * 1e-3) / 1e12
            families[fam].update({"alg_gflop_per_launch": round(v["flops"] / v["launches"] / 1e9, 4),
                                  "achieved_tflops": round(tf, 1),
                                  "frac_mfma": round(tf / PEAK_FP16_TFLOPS, 4)})

    layers_out = []
    for r in runs:
        f = direct_flops(r["B"], r["C"], r["K"], r["H"], r["H"])
        troof = layer_roofline_us(r["B"], r["C"], r["K"], r["H"])
        rec = {
            "layer": r["name"], "B": r["B"], "C": r["C"], "K": r["K"], "H": r["H"],
            "path": r["path"],
            "nova_ms": round(r["nova_ms"], 5),
            "nova_tflops": round(f / (r["nova_ms"] * 1e-3) / 1e12, 2),
            "roofline_us": round(troof, 3),
            "roofline_frac": round(troof / (r["nova_ms"] * 1e3), 4),
            "nova_cold_ms": round(r["cold_ms"], 5),
            "roofline_frac_cold": round(troof / (r["cold_ms"] * 1e3), 4),
            "kernels": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv)
                            for kk, vv in v.items()} for k, v in r["kernels"].items()},
        }
        if "miopen_ms" in r:
            rec["miopen_ms"] = round(r["miopen_ms"], 5)
            rec["speedup_vs_miopen"] = round(r["miopen_ms"] / r["nova_ms"], 3)
        if r.get("nova_graph_ms") is not None:
            rec["nova_graph_ms"] = round(r["nova_graph_ms"], 5)
        if r.get("miopen_graph_ms") is not None:
            rec["miopen_graph_ms"] = round(r["miopen_graph_ms"], 5)
        layers_out.append(rec)
        log(f"{r['name']:8s} B={r['B']:<3d} {r['path']:6s} nova {r['nova_ms']*1e3:8.2f} us"
            + (f"  miopen {r['miopen_ms']*1e3:8.2f} us" if "miopen_ms" in r else "")
            + (f"  graph nova {r['nova_graph_ms']*1e3:7.2f} us" if r.get("nova_graph_ms") else "")
            + (f" miopen {r['miopen_graph_ms']*1e3:7.2f} us" if r.get("miopen_graph_ms") else "")
            + f"  roofline {troof:6.2f} us")

    extra = None
    if not args.no_extra:
        extra = extra_measurements(runs, lib, torch, nn, nw, 50)

    cpu = None
    if not args.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        cpu = cpu_baseline([(( r["name"], r["C"], r["H"]), r["B"]) for r in runs],
                           args.cpu_seconds, threads)
        cpu = {k: (round(v, 6) if isinstance(v, float) else v) for k, v in cpu.items()}

    out = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": "resnet50_3x3s1_layers_b1_b32",
            "layers": [f"{n}:C=K={C},H=W={H}" for n, C, H in LAYERS],
            "batches": BATCHES,
            "pad": 1,
            "direct_gflop_per_step": round(total_flops / 1e9, 3),
            "interface": "NovaWinogradConv2d module (ctypes C-ABI), eager",
        },
        "roofline": roofline,
        "kernel_families": families,
        "cpu_baseline": cpu,
        "layers": layers_out,
    }
    if extra is not None:
        out["resnet50_model"] = extra["resnet50"]
    if args.details:
        with open(args.details, "w") as f:
            json.dump({"bench": out, "kernels": kernels, "extra": extra}, f, indent=2)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
