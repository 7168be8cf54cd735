"""Benchmark of one submanifold 3x3x3 sparse conv layer on one MI355X.

A step is one conv over the whole voxel set (inputs resident in HBM): the fused gather-GEMM
kernel of libtrellis_sparse.so. The neighbour table is built once beforehand (it is shared by
every conv of a decoder stage) and its build time is reported separately.

Prints one JSON line. `value` is active voxels per second; `roofline` prices the conv kernel's
average launch time (HIP events over the timed region, on the stream the kernel runs on)
against MI355X's dense bf16 MFMA peak; `cpu_baseline` is the CPU oracle (a C restatement of
the reference's tap-sequential fp32 algorithm) timed on this host's cores over a bounded row
sample of the same workload.

    python bench.py [--steps 50] [--warmup 5] [--workload shells256-c128-bf16]
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))

PEAK_TFLOPS = {"bf16": 2500.0, "f16": 2500.0, "f32": 157.3}   # MI355X dense, datasheet
PEAK_HBM_GBS = 8000.0


def _load(name, path, pkg_dir=None):
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(
        name, path, submodule_search_locations=[pkg_dir] if pkg_dir else None)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def load_package():
    pkg_dir = os.path.join(ROOT, "trellis.cpp_amd")
    return _load("trellis_cpp_amd", os.path.join(pkg_dir, "__init__.py"), pkg_dir)


def cpu_baseline(w, nbr, budget_s: float):
    """The CPU oracle (a C restatement of the reference's algorithm: all 27 taps against the
    zero row, fp32, tap-sequential accumulation, bias last, OpenMP over output rows) timed on
    this host: one warm-up, then the median of >= 3 timed runs over a contiguous output-row
    range sized so the timed runs take about budget_s (the whole conv when it is fast enough);
    a 1-thread run over a smaller range; and the neighbour-table build (hash restatement,
    single-threaded like the reference's build_neighbor_table)."""
    import statistics
    orc = _load("trellis_oracle", os.path.join(ROOT, "oracle", "oracle.py"))
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    n = w.n

    def timed(r0, r1, th):
        t = time.perf_counter()
        orc.subm_conv_f32_rows(w.feats, nbr, w.weight, w.bias, r0, r1, th)
        return time.perf_counter() - t

    probe = min(n, 4000)
    per_row = timed(0, probe, threads) / probe                     # also the warm-up
    rows = int(min(n, max(probe, budget_s / 3 / max(per_row, 1e-12))))
    r0 = (n - rows) // 2
    reps = int(min(20, max(3, budget_s / max(rows * per_row, 1e-12))))
    runs = [timed(r0, r0 + rows, threads) for _ in range(reps)]
    dt = statistics.median(runs)
    rows1 = max(1, min(rows, int(max(budget_s / 4, 1.0) / max(per_row * threads, 1e-12))))
    dt1 = timed(r0, r0 + rows1, 1)
    t = time.perf_counter()
    orc.neighbor_table(w.coords)
    rb_s = time.perf_counter() - t
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": rows / dt, "unit": "voxels/s", "cores": threads, "kind": "port",
        "sample": f"output rows [{r0}, {r0 + rows}) of {n}: median of {reps} runs "
                  f"({', '.join(f'{x:.2f}' for x in runs)} s) after a warm-up; fp32, all 27 "
                  f"taps against the zero row, tap-sequential accumulation "
                  f"(CPU restatement of sparse.cpp; ggml unavailable)",
        "value_1core": rows1 / dt1, "sample_1core": f"{rows1} rows in {dt1:.2f} s on 1 thread",
        "rulebook_s_1thread": rb_s,
        "cpu_model": cpu_model,
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="shells256-c128-bf16")
    ap.add_argument("--algo", default="auto", choices=["auto", "mfma", "narrow", "mfma_gather"])
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a device-to-device copy of MIB MiB (the known-size kernel "
                         "that scales the FETCH_SIZE / WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    if args.copy_calibration:
        nbytes = args.copy_calibration << 20
        src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": nbytes}))
        return

    pkg = load_package()
    import trellis_cpp_amd.shells as shells
    pkg.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    w = shells.workload(args.workload)
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[w.dtype]
    coords = torch.from_numpy(w.coords).to(dev)
    feats = torch.from_numpy(w.feats).to(tdt).to(dev)
    weight = torch.from_numpy(w.weight).to(tdt).to(dev)
    bias = torch.from_numpy(w.bias).to(dev)
    out = torch.empty((w.n, w.co), dtype=tdt, device=dev)
    stream = torch.cuda.current_stream()

    # neighbour table: built once, timed on its own
    nbr = pkg.rulebook_build(coords)
    torch.cuda.synchronize()
    rb_ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    rb_ev[0].record(stream)
    for _ in range(5):
        nbr = pkg.rulebook_build(coords, check=False)
    rb_ev[1].record(stream)
    torch.cuda.synchronize()
    rulebook_ms = rb_ev[0].elapsed_time(rb_ev[1]) / 5
    pairs = pkg.count_pairs(nbr, w.n)

    # The MFMA path runs with a conv plan of the table and packed weights, both built once
    # (like the table, a plan serves every conv of a stage; weights are packed at model load).
    planned = (args.algo in ("auto", "mfma") and w.dtype in ("bf16", "f16")
               and w.ci % 16 == 0 and w.co % 64 == 0)
    plan_ms = None
    if planned:
        plan = pkg.conv_plan_build(nbr, w.n)
        packed = pkg.conv_weight_pack(weight)
        torch.cuda.synchronize()
        rb_ev[0].record(stream)
        for _ in range(5):
            plan = pkg.conv_plan_build(nbr, w.n)
        rb_ev[1].record(stream)
        torch.cuda.synchronize()
        plan_ms = rb_ev[0].elapsed_time(rb_ev[1]) / 5

        def step():
            pkg.subm_conv3x3_planned(feats, nbr, plan, packed, bias, w.co, out=out)
    else:
        def step():
            pkg.subm_conv3x3(feats, nbr, weight, bias, out=out, algo=args.algo)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    t0 = time.perf_counter()
    ev[0].record(stream)
    for _ in range(args.steps):
        step()
    ev[1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = ev[0].elapsed_time(ev[1]) / args.steps

    flops = 2.0 * w.ci * w.co * pairs
    flops_dense = 2.0 * w.ci * w.co * 27 * w.n
    es = 2 if w.dtype != "f32" else 4
    compulsory = w.n * w.ci * es + w.n * w.co * es + 27 * w.ci * w.co * es + 4 * w.co + 108 * w.n
    tflops = flops / (ms * 1e-3) / 1e12
    peak = PEAK_TFLOPS[w.dtype]
    bound = "mfma" if flops / compulsory > peak * 1e12 / (PEAK_HBM_GBS * 1e9) else "hbm"
    if bound == "mfma":
        roof = {"bound": "mfma", "achieved": tflops, "peak": peak, "unit": "TFLOP/s",
                "frac": tflops / peak}
    else:
        gbs = compulsory / (ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": gbs / PEAK_HBM_GBS}
    # HBM bytes per launch of the conv kernel, measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
    # passes scaled by a copy kernel of known size (profiles/traffic_<workload>.md)
    roof["traffic"] = None
    tj = os.path.join(ROOT, "profiles", "traffic.json")
    if planned and os.path.exists(tj):
        rec = json.load(open(tj)).get(w.name)
        if rec:
            roof["traffic"] = rec["bytes_per_launch"]
            roof["traffic_source"] = rec["source"]
    roof["algorithmic_flops_per_launch"] = flops
    roof["compulsory_bytes_per_launch"] = compulsory

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(w, nbr.cpu().numpy(), args.cpu_seconds)

    res = {
        "metric": "active voxels/s & TFLOP/s per sparse conv layer; % MFMA/HBM roofline",
        "value": w.n / (ms * 1e-3),
        "unit": "voxels/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": "synthetic",
        "config": {
            "workload": w.name, "grid": w.grid, "n_voxels": w.n, "active_pairs": pairs,
            "pairs_per_voxel": pairs / max(w.n, 1), "c_in": w.ci, "c_out": w.co,
            "accumulate": "f32", "out_dtype": w.dtype,
            "algo": "mfma-planned" if planned else args.algo,
            "parallelism": "single-gpu",
        },
        "tflops": tflops,
        "tflops_dense27_equivalent": flops_dense / (ms * 1e-3) / 1e12,
        "rulebook_ms": rulebook_ms,
        "plan_ms": plan_ms,
        "wall_s_timed_region": wall,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(res))


if __name__ == "__main__":
    main()
