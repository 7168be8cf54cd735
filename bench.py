"""Benchmark of one submanifold 3x3x3 sparse conv layer on one MI355X.

A step is one conv over the whole voxel set (inputs resident in HBM): the fused gather-GEMM
kernel of libtrellis_sparse.so. The neighbour table is built once beforehand (it is shared by
every conv of a decoder stage) and its build time is reported separately.

Prints one JSON line. `value` is active voxels per second; `roofline` prices the conv kernel's
average launch time (HIP events over the timed region, on the stream the kernel runs on)
against MI355X's dense bf16 MFMA peak; `cpu_baseline` is the CPU oracle (a C restatement of
the reference's tap-sequential fp32 algorithm) timed on this host's cores over a bounded row
sample of the same workload. The table, plan and extra-configuration timings each follow
SETTLE_MS of untimed calls of the same kind (the shader clock ramps up over the first tens of
milliseconds of activity; the headline conv follows those builds and its own warm-up steps).

    python bench.py [--steps 50] [--warmup 5] [--workload shells256-c128-bf16]

`--workload decoder-shells64-c1024` times the whole texture decoder stack instead (one decode
per step, through the C++ host library): see trellis_cpp_amd.shells.decoder_workload. The default
line's `extra` holds the other conv configurations and 3 decodes of that stack.
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
# fp32 FMA on the VALU without packed-fp32 instructions (which this build does not emit):
# 256 CUs x 4 SIMDs x 16 lanes x 2 FLOP x 2.4 GHz
PEAK_VALU_TFLOPS = 78.6


def _load(name, path, pkg_dir=None):
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(
        name, path, submodule_search_locations=[pkg_dir] if pkg_dir else None)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def progress(msg: str) -> None:
    """A line on stderr as each part of the run ends (stdout holds only the JSON line)."""
    print(f"bench: {msg}", file=sys.stderr, flush=True)


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
    cpu = host_cpu()
    return {
        "value": rows / dt, "unit": "voxels/s", "cores": threads, "kind": "port",
        "sample": f"output rows [{r0}, {r0 + rows}) of {n}: median of {reps} runs "
                  f"({', '.join(f'{x:.2f}' for x in runs)} s) after a warm-up; fp32, all 27 "
                  f"taps against the zero row, tap-sequential accumulation "
                  f"(CPU restatement of sparse.cpp; ggml unavailable)",
        "value_1core": rows1 / dt1, "sample_1core": f"{rows1} rows in {dt1:.2f} s on 1 thread",
        "rulebook_s_1thread": rb_s,
        "cpu_model": cpu["model"],
        "host_cpu": cpu,
    }


def host_cpu() -> dict:
    """The host CPU as lscpu reports it (model, sockets, cores, threads, flags of note), the
    logical CPUs this process may use, and /proc/cpuinfo's model string."""
    import subprocess
    info = {"model": "", "logical_cpus_usable": len(os.sched_getaffinity(0))}
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                info["cpuinfo_model"] = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        keys = {"Model name": "model", "Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket",
                "Thread(s) per core": "threads_per_core", "CPU(s)": "logical_cpus", "CPU max MHz": "max_mhz",
                "Vendor ID": "vendor", "CPU family": "family", "Model": "model_number",
                "Hypervisor vendor": "hypervisor"}
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in keys:
                info[keys[k.strip()]] = v.strip()
        flags = next((l.split(":", 1)[1].split() for l in out.splitlines() if l.startswith("Flags")), [])
        info["simd"] = [f for f in ("avx2", "fma", "avx512f", "avx512_bf16") if f in flags]
    except (OSError, subprocess.SubprocessError):
        pass
    if not info["model"]:
        info["model"] = info.get("cpuinfo_model", "")
    return info


def decoder_bench(args) -> dict:
    """The texture decoder stack (trellis::tex_decode through the C++ host library) on a
    synthetic decoder workload: random-init bf16 weights written to a GGUF under the reference's
    key names, latent and subdivision masks as .npy files; host/bin/decoder_bench times
    whole decodes (host inputs in, host output back, as the reference's API has it)."""
    import subprocess
    import tempfile

    import numpy as np
    import torch

    pkg = load_package()
    import trellis_cpp_amd.shells as shells
    from trellis_cpp_amd.gguf_writer import write as write_gguf

    w = shells.decoder_workload(args.workload)
    exe = os.path.join(ROOT, "trellis.cpp_amd", "host", "bin", "decoder_bench")
    if not os.path.exists(exe):
        raise SystemExit(f"{exe} is not built (make -C trellis.cpp_amd/host)")
    def prepare(d):
        p = shells.decoder_params(w.channels, w.blocks, w.latent.shape[1], w.out_ch, w.std, w.seed)
        write_gguf(os.path.join(d, "model.gguf"), p,
                   dtypes={k: ("bf16" if v.ndim >= 2 else "f32") for k, v in p.items()},
                   arch="trellis2-tex-dec")
        np.save(os.path.join(d, "latent.npy"), w.latent)
        np.save(os.path.join(d, "coords.npy"), np.ascontiguousarray(w.coords, np.int32))
        for s, m in enumerate(w.masks):
            np.save(os.path.join(d, f"subs_{s}.npy"), np.ascontiguousarray(m, np.uint8))

    if args.prepare_only:
        os.makedirs(args.prepare_only, exist_ok=True)
        prepare(args.prepare_only)
        return {"prepared": args.prepare_only, "voxels_per_level": w.counts,
                "run": f"{exe} {args.prepare_only}/model.gguf {args.prepare_only} 0 <warmup> <steps>"}
    with tempfile.TemporaryDirectory(prefix="decoder_bench_", dir="/tmp") as d:
        prepare(d)
        r = subprocess.run([exe, os.path.join(d, "model.gguf"), d, "0", str(args.warmup), str(args.steps)],
                           capture_output=True, text=True, timeout=900)
    if r.returncode != 0:
        raise SystemExit(f"decoder_bench failed ({r.returncode}): {r.stderr[-2000:]}")
    run = json.loads(r.stdout.strip().splitlines()[-1])

    # algorithmic FLOPs: active pairs of every level from the device neighbour table
    pairs = []
    for c in w.level_coords:
        nbr = pkg.rulebook_build(torch.from_numpy(np.ascontiguousarray(c, np.int32)).cuda())
        pairs.append(pkg.count_pairs(nbr, len(c)))
        del nbr
    ch, nb, cl = w.channels, w.blocks, w.latent.shape[1]

    def total(pp):
        f = 2.0 * cl * ch[0] * w.counts[0]                          # from_latent
        for s in range(len(ch) - 1):
            ci, co, n = ch[s], ch[s + 1], w.counts[s]
            f += nb * (2.0 * ci * ci * pp[s] + 16.0 * ci * ci * n)  # ConvNeXt: conv + MLP
            f += 2.0 * ci * 8 * co * pp[s] + 2.0 * co * co * pp[s + 1]   # C2S conv1, conv2
        return f + 2.0 * ch[-1] * w.out_ch * w.counts[-1]           # output_layer
    flops = total(pairs)
    flops_dense = total([27 * n for n in w.counts])
    ms = run["decode_ms"]
    tflops = flops / (ms * 1e-3) / 1e12

    cpu = None
    if not args.no_cpu:
        cpu = decoder_cpu_baseline(w, flops_dense, args.cpu_seconds)
    return {
        "metric": "decoder voxels/s & TFLOP/s (texture decoder stack, one decode per step)",
        "value": run["voxels_out"] / (ms * 1e-3),
        "unit": "voxels/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": w.name, "voxels_per_level": w.counts, "active_pairs_per_level": pairs,
                   "channels": list(ch), "convnext_blocks_per_stage": nb, "latent_ch": cl,
                   "out_ch": w.out_ch, "weights": f"bf16 ~ N(0, {w.std})", "accumulate": "f32",
                   "model_bytes": run["model_bytes"], "parallelism": "single-gpu"},
        "tflops": tflops,
        "tflops_dense27_equivalent": flops_dense / (ms * 1e-3) / 1e12,
        "min_ms": run["min_ms"], "model_load_ms": run["load_ms"],
        "device_gb_in_use": run.get("device_bytes_in_use", 0) / 1e9,
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": PEAK_TFLOPS["bf16"], "unit": "TFLOP/s",
                     "frac": tflops / PEAK_TFLOPS["bf16"], "traffic": None,
                     "note": "whole decode, host transfers included; the conv kernels dominate"},
        "cpu_baseline": cpu,
    }


DECODER_WORKLOAD = "decoder-shells64-c1024"


def decoder_extra(args) -> dict:
    """decoder_bench on the decoder workload with a short step count and no CPU leg, for the
    default line's `extra`; a failure is reported in the entry, not raised."""
    import torch
    torch.cuda.empty_cache()
    dargs = argparse.Namespace(**vars(args))
    dargs.workload, dargs.steps, dargs.warmup = DECODER_WORKLOAD, 3, 1
    dargs.no_cpu, dargs.prepare_only = True, ""
    t0 = time.perf_counter()
    try:
        d = decoder_bench(dargs)
    except (SystemExit, Exception) as e:    # decoder_bench raises SystemExit on a failed child
        return {"error": str(e)[-2000:]}
    return {"ms_per_step": d["ms_per_step"], "min_ms": d["min_ms"], "steps": dargs.steps,
            "warmup_steps": dargs.warmup, "voxels_per_s": d["value"], "tflops": d["tflops"],
            "frac": d["roofline"]["frac"], "device_gb_in_use": d["device_gb_in_use"],
            "voxels_per_level": d["config"]["voxels_per_level"], "channels": d["config"]["channels"],
            "wall_s": time.perf_counter() - t0,
            "note": "one decode per step: host latent, coordinates and masks in, host features out "
                    "(trellis::tex_decode, random-init bf16 weights)"}


def decoder_cpu_baseline(w, flops_dense: float, budget_s: float) -> dict:
    """The CPU oracle's conv (the reference's dense-over-27-taps fp32 algorithm) timed on a row
    sample of the decoder's widest conv (stage 0: ch[0] -> ch[0] on the latent voxels), its
    dense-27 FLOP rate then pricing the decoder's dense-27 FLOPs: an extrapolation, since a full
    CPU decode takes far longer than the time budget."""
    import statistics

    import numpy as np
    orc = _load("trellis_oracle", os.path.join(ROOT, "oracle", "oracle.py"))
    import trellis_cpp_amd.shells as shells
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    c, n = w.channels[0], len(w.coords)
    rng = np.random.default_rng(w.seed)
    x = shells.round_to(shells.standard_normal_rows(rng, n, c), "bf16")
    wt = shells.round_to(rng.standard_normal((c, 27, c), dtype=np.float32) * np.float32(w.std), "bf16")
    b = np.zeros(c, np.float32)
    nbr = orc.neighbor_table(w.coords)

    def timed(r0, r1):
        t = time.perf_counter()
        orc.subm_conv_f32_rows(x, nbr, wt, b, r0, r1, threads)
        return time.perf_counter() - t

    probe = min(n, 256)
    per_row = timed(0, probe) / probe
    rows = int(min(n, max(probe, budget_s / 3 / max(per_row, 1e-12))))
    r0 = (n - rows) // 2
    runs = [timed(r0, r0 + rows) for _ in range(3)]
    dt = statistics.median(runs)
    rate = 2.0 * 27 * c * c * rows / dt
    est = flops_dense / rate
    return {"value": w.counts[-1] / est, "unit": "voxels/s", "cores": threads, "kind": "port",
            "sample": f"extrapolated: the oracle's conv ({c} -> {c} channels, rows [{r0}, {r0 + rows}) of "
                      f"{n}, median of 3: {dt:.2f} s) runs {rate / 1e9:.1f} dense-27 GFLOP/s; the "
                      f"decoder's {flops_dense / 1e12:.1f} dense-27 TFLOP at that rate take {est:.0f} s "
                      f"(LayerNorm, SiLU and gathers not counted)",
            "host_cpu": host_cpu()}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="shells256-c128-bf16")
    ap.add_argument("--algo", default="auto", choices=["auto", "mfma", "narrow", "mfma_gather", "thin", "thin_mfma", "f32_mfma"])
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the other conv configurations")
    ap.add_argument("--plan-order", default="morton", choices=["morton", "rows"],
                    help="conv plan tiles: Morton order of 8^3 cells, or consecutive rows")
    ap.add_argument("--prepare-only", default="", metavar="DIR",
                    help="decoder workloads: only write the model and inputs into DIR (for running "
                         "trellis.cpp_amd/host/bin/decoder_bench on them, e.g. under a profiler)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a device-to-device copy of MIB MiB (the known-size kernel "
                         "that scales the FETCH_SIZE / WRITE_SIZE counters) and exit")
    ap.add_argument("--mlp-rows", type=int, default=0, metavar="N",
                    help="only time the fused ConvNeXt MLP (tsp_convnext_mlp, C = 128, bf16) on N rows "
                         "of random data and print its line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)

    if args.workload.startswith("decoder-"):
        print(json.dumps(decoder_bench(args)))
        return

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
    if args.mlp_rows:
        print(json.dumps(mlp_bench(pkg, torch, args.mlp_rows, args.steps, args.warmup)))
        return
    import trellis_cpp_amd.shells as shells
    pkg.lib()
    torch.cuda.set_device(torch.device("cuda:0"))

    w = shells.workload(args.workload)
    r = time_conv(pkg, w, args, args.steps, args.warmup)
    progress(f"{w.name}: {r['ms']:.4f} ms per step")
    ms, pairs, planned = r["ms"], r["pairs"], r["planned"]
    flops = 2.0 * w.ci * w.co * pairs
    flops_dense = 2.0 * w.ci * w.co * 27 * w.n
    compulsory = compulsory_bytes(w)
    path = conv_path(w, args.algo, planned)
    roof = roofline(w, flops, compulsory, ms, valu=path in ("thin", "narrow"))
    add_traffic(roof, w, path)
    roof["algorithmic_flops_per_launch"] = flops
    roof["compulsory_bytes_per_launch"] = compulsory
    # the peaks this box reaches with library code, as a second denominator beside the datasheet's
    mp = measured_peaks(torch, w.dtype)
    roof["measured_peaks"] = mp
    if roof["bound"] == "mfma" and mp.get("gemm_tflops"):
        roof["frac_of_measured_gemm"] = roof["achieved"] / mp["gemm_tflops"]
    elif roof["bound"] == "hbm" and mp.get("copy_gb_s"):
        roof["frac_of_measured_copy"] = roof["achieved"] / mp["copy_gb_s"]

    # the same conv with f32 output (what the decoders and the parity tests read), and for the
    # 256^3 C=128 configuration the same shells at ~640K voxels (the size the target names)
    extra = {}
    if w.dtype != "f32" and planned:
        rf = time_conv(pkg, w, args, max(5, args.steps // 2), 2, out_dtype=torch.float32, reuse=r,
                       settle_ms=SETTLE_MS)
        extra["f32_out"] = {"ms_per_step": rf["ms"], "tflops": flops / (rf["ms"] * 1e-3) / 1e12,
                            "frac": flops / (rf["ms"] * 1e-3) / 1e12 / PEAK_TFLOPS[w.dtype]}
    if w.name == "shells256-c128-bf16" and not args.no_extra:
        # every other conv configuration, timed the same way: the same shells at ~640K voxels
        # (the size the target names), 128^3 ellipsoids at C = 256, the 512^3 band at C = 64, the
        # fp32 64^3 shell (the CPU-reference configuration) and a thin C = 8 layer
        for name in EXTRA_WORKLOADS:
            we = shells.workload(name)
            re_ = time_conv(pkg, we, args, max(5, args.steps // 2), 2, settle_ms=SETTLE_MS)
            fe = 2.0 * we.ci * we.co * re_["pairs"]
            path_e = conv_path(we, args.algo, re_["planned"])
            roof_e = roofline(we, fe, compulsory_bytes(we), re_["ms"], valu=path_e in ("thin", "narrow"))
            add_traffic(roof_e, we, path_e)
            extra[name] = {
                "n_voxels": we.n, "active_pairs": re_["pairs"], "c_in": we.ci, "c_out": we.co,
                "dtype": we.dtype, "algo": path_e,
                "ms_per_step": re_["ms"], "steps": max(5, args.steps // 2), "warmup_steps": re_["warmup_steps"],
                "voxels_per_s": we.n / (re_["ms"] * 1e-3),
                "tflops": fe / (re_["ms"] * 1e-3) / 1e12, "frac": roof_e["frac"], "roofline": roof_e,
                "rulebook_ms": re_["rulebook_ms"], "plan_ms": re_["plan_ms"],
                "table_plan_ms": re_["table_plan_ms"]}
            progress(f"{name}: {re_['ms']:.4f} ms per step")
            del re_
        # the whole texture decoder stack (a few decodes through the C++ host library, in a
        # child process), so that its time is in the same line
        extra[DECODER_WORKLOAD] = decoder_extra(args)
        progress(f"{DECODER_WORKLOAD}: {extra[DECODER_WORKLOAD].get('ms_per_step')} ms per decode")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(w, r["nbr"].cpu().numpy(), args.cpu_seconds)
        progress("cpu baseline done")

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
            "algo": path,
            "plan_order": args.plan_order if planned else None,
            "parallelism": "single-gpu",
        },
        "tflops": flops / (ms * 1e-3) / 1e12,
        "tflops_dense27_equivalent": flops_dense / (ms * 1e-3) / 1e12,
        "rulebook_ms": r["rulebook_ms"],
        "plan_ms": r["plan_ms"],
        "table_plan_ms": r["table_plan_ms"],
        "wall_s_timed_region": r["wall"],
        "gpu": torch.cuda.get_device_name(0),
        "roofline": roof,
        "extra": extra,
        "cpu_baseline": cpu,
    }
    print(json.dumps(res))


def mlp_bench(pkg, torch, n: int, steps: int, warmup: int) -> dict:
    """The ConvNeXt MLP kernel alone: y = x + b2 + W2 . silu(W0 . xn + b0) at C = 128 on n rows
    (xn bf16, x and y f32, weights bf16 ~ N(0, 1/sqrt(fan-in)), biases ~ N(0, 0.1))."""
    c = 128
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(5)
    xn = torch.randn(n, c, device=dev, generator=g).to(torch.bfloat16)
    w0 = (torch.randn(4 * c, c, device=dev, generator=g) / c ** 0.5).to(torch.bfloat16)
    w2 = (torch.randn(c, 4 * c, device=dev, generator=g) / (4 * c) ** 0.5).to(torch.bfloat16)
    b0 = torch.randn(4 * c, device=dev, generator=g) * 0.1
    b2 = torch.randn(c, device=dev, generator=g) * 0.1
    x = torch.randn(n, c, device=dev, generator=g)
    y = torch.empty_like(x)
    packed = pkg.convnext_mlp_pack(w0, w2)
    step = lambda: pkg.convnext_mlp(xn, packed, b0, b2, x, out=y)
    for _ in range(warmup):
        step()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(s)
    for _ in range(steps):
        step()
    e1.record(s)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flops = 16.0 * n * c * c
    nbytes = n * c * (2 + 4 + 4)
    return {"kernel": "k_mlp_ws", "rows": n, "c": c, "dtype": "bf16", "ms": ms,
            "tflops": flops / (ms * 1e-3) / 1e12, "frac_bf16_peak": flops / (ms * 1e-3) / 1e12 / PEAK_TFLOPS["bf16"],
            "compulsory_gb_s": nbytes / (ms * 1e-3) / 1e9}


def measured_peaks(torch, dtype: str) -> dict:
    """Achievable peaks on this box: a dense 8192^3 GEMM in the conv's 16-bit type (torch.mm,
    which runs hipBLASLt) and a 1 GiB device-to-device copy (read + write bytes counted), each the
    median of 20 timed calls after 5 warm-up calls."""
    def med(fn, it=20):
        ts = []
        for _ in range(5):
            fn()
        for _ in range(it):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            e1.synchronize()
            ts.append(e0.elapsed_time(e1))
        return sorted(ts)[len(ts) // 2]
    out = {}
    if dtype in ("bf16", "f16"):
        tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
        m = 8192
        a = torch.randn(m, m, device="cuda").to(tdt)
        b = torch.randn(m, m, device="cuda").to(tdt)
        c = torch.empty(m, m, device="cuda", dtype=tdt)
        t = med(lambda: torch.mm(a, b, out=c))
        out["gemm_tflops"] = 2.0 * m ** 3 / (t * 1e-3) / 1e12
        out["gemm"] = f"{m}x{m}x{m} {dtype} torch.mm"
        del a, b, c
    src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    t = med(lambda: dst.copy_(src))
    out["copy_gb_s"] = 2.0 * src.numel() * 4 / (t * 1e-3) / 1e9
    out["copy"] = "1 GiB device-to-device, read + write"
    del src, dst
    torch.cuda.empty_cache()
    return out


def add_traffic(roof: dict, w, path: str) -> None:
    """roof["traffic"]: HBM bytes per launch of the conv kernel, measured with rocprofv3
    FETCH_SIZE / WRITE_SIZE passes scaled by a copy kernel of known size (profiles/traffic.json
    and the summary it names); used only while the kernel's sources are the ones that profile
    measured, else null."""
    roof["traffic"] = None
    tj = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tj):
        rec = json.load(open(tj)).get(w.name)
        if rec and rec.get("path") == path and rec.get("sources_sha256") == kernel_sources_sha(rec["sources"]):
            roof["traffic"] = rec["bytes_per_launch"]
            roof["traffic_source"] = rec["source"]
        elif rec:
            roof["traffic_note"] = "profile predates the current kernel sources; re-measure"


def kernel_sources_sha(files) -> str:
    """sha256 over a conv kernel's sources (file names under trellis.cpp_amd/csrc): a traffic
    profile is valid for these only."""
    import hashlib
    h = hashlib.sha256()
    for f in files:
        with open(os.path.join(ROOT, "trellis.cpp_amd", "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()


def conv_path(w, algo: str, planned: bool) -> str:
    """The kernel the library runs for workload w under `algo` (tsp_subm_conv3x3's AUTO order:
    matrix-core for 16-bit Ci % 32 / Co % 64 shapes -- here with a plan --, then the thin
    matrix-core kernel, the thin VALU kernel, the fp32 matrix-core kernel, the tiled VALU
    kernel)."""
    if planned:
        return "mfma-planned"
    if algo != "auto":
        return algo
    thin = w.co in (4, 8, 16, 32) and w.ci * w.co <= 512
    if thin and w.dtype in ("bf16", "f16") and w.ci in (8, 16, 32):
        return "thin_mfma"
    if thin and w.ci % 4 == 0:
        return "thin"
    if w.dtype == "f32" and w.ci % 16 == 0 and w.co % 32 == 0:
        return "f32_mfma"
    return "narrow"


EXTRA_WORKLOADS = ("shells600k-c128-bf16", "ellipsoids128-c256-bf16", "band512-c64-bf16", "shell64-c64-f32",
                   "shells256-c8-bf16")


def compulsory_bytes(w) -> float:
    es = 2 if w.dtype != "f32" else 4
    return w.n * w.ci * es + w.n * w.co * es + 27 * w.ci * w.co * es + 4 * w.co + 108 * w.n


def roofline(w, flops: float, compulsory: float, ms: float, valu: bool = False) -> dict:
    """The bound of the conv kernel: the matrix cores (or, for the VALU kernels, fp32 FMA issue)
    when its FLOPs over the compulsory bytes exceed the ridge of that peak over HBM's, else HBM."""
    tflops = flops / (ms * 1e-3) / 1e12
    if valu:
        peak = PEAK_VALU_TFLOPS
        if flops / compulsory > peak * 1e12 / (PEAK_HBM_GBS * 1e9):
            return {"bound": "valu", "achieved": tflops, "peak": peak, "unit": "TFLOP/s", "frac": tflops / peak}
        gbs = compulsory / (ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS}
    peak = PEAK_TFLOPS[w.dtype]
    if flops / compulsory > peak * 1e12 / (PEAK_HBM_GBS * 1e9):
        return {"bound": "mfma", "achieved": tflops, "peak": peak, "unit": "TFLOP/s", "frac": tflops / peak}
    gbs = compulsory / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS}


SETTLE_MS = 100.0   # untimed calls before a timed loop of short calls: the clock ramps over tens of ms


def settle(fn, ms: float = SETTLE_MS) -> int:
    """Calls fn until `ms` of wall time have passed (at least once), synchronising every few
    calls so that the time is the device's; returns the number of calls."""
    import torch
    t0, k = time.perf_counter(), 0
    while True:
        fn()
        k += 1
        if k % 4 == 0 or k == 1:
            torch.cuda.synchronize()
            if (time.perf_counter() - t0) * 1e3 >= ms:
                return k


def time_conv(pkg, w, args, steps: int, warmup: int, out_dtype=None, reuse=None, settle_ms: float = 0.0) -> dict:
    """Times one conv of workload w: the neighbour table and (16-bit, matrix-core shapes) the
    conv plan are built and timed first, each on its own after SETTLE_MS of untimed calls
    (reuse: the table and plan of an earlier call on the same workload); then `warmup` untimed
    convs (and, with settle_ms, more until that much time has passed), then `steps` convs
    between two HIP events on the stream the kernel runs on."""
    import numpy as np
    import torch
    dev = torch.device("cuda:0")
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[w.dtype]
    stream = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    if reuse is None:
        coords = torch.from_numpy(np.ascontiguousarray(w.coords, np.int32)).to(dev)
        feats = torch.from_numpy(w.feats).to(tdt).to(dev)
        weight = torch.from_numpy(w.weight).to(tdt).to(dev)
        bias = torch.from_numpy(w.bias).to(dev)
        # neighbour table: built once (range-checked), then timed on its own with its buffers
        # allocated once, as a decoder level reuses them
        nbr = pkg.rulebook_build(coords)
        ws = torch.empty(pkg.lib().tsp_rulebook_workspace_bytes(w.n), dtype=torch.uint8, device=dev)
        settle(lambda: pkg.rulebook_build(coords, check=False, nbr=nbr, workspace=ws))
        torch.cuda.synchronize()
        ev[0].record(stream)
        for _ in range(5):
            pkg.rulebook_build(coords, check=False, nbr=nbr, workspace=ws)
        ev[1].record(stream)
        torch.cuda.synchronize()
        rulebook_ms = ev[0].elapsed_time(ev[1]) / 5
        pairs = pkg.count_pairs(nbr, w.n)
    else:
        coords, feats, weight, bias, nbr = (reuse[k] for k in ("coords", "feats", "weight", "bias", "nbr"))
        rulebook_ms, pairs = reuse["rulebook_ms"], reuse["pairs"]
    out = torch.empty((w.n, w.co), dtype=out_dtype or tdt, device=dev)

    # The MFMA path runs with a conv plan of the table and packed weights, both built once
    # (like the table, a plan serves every conv of a stage; weights are packed at model load).
    planned = (args.algo in ("auto", "mfma") and w.dtype in ("bf16", "f16")
               and w.ci % 16 == 0 and w.co % 64 == 0)
    plan = packed = plan_ms = table_plan_ms = None
    if planned and reuse is not None:
        plan, packed, plan_ms = reuse["plan"], reuse["packed"], reuse["plan_ms"]
        table_plan_ms = reuse["table_plan_ms"]
    elif planned:
        # tiles in the Morton order of the voxels' 8^3 cells (or, with --plan-order rows, runs of
        # consecutive rows)
        pcoords = coords if args.plan_order == "morton" else None
        plan = pkg.conv_plan_build(nbr, w.n, coords=pcoords)
        packed = pkg.conv_weight_pack(weight)
        settle(lambda: pkg.conv_plan_build(nbr, w.n, coords=pcoords, plan=plan))
        torch.cuda.synchronize()
        ev[0].record(stream)
        for _ in range(5):
            pkg.conv_plan_build(nbr, w.n, coords=pcoords, plan=plan)
        ev[1].record(stream)
        torch.cuda.synchronize()
        plan_ms = ev[0].elapsed_time(ev[1]) / 5
        if pcoords is not None:
            # the table and the Morton plan in one call, on one cell grid (what a decoder level
            # runs); the same table and plan as the two calls above
            settle(lambda: pkg.rulebook_build_planned(coords, check=False, nbr=nbr, workspace=ws, plan=plan))
            torch.cuda.synchronize()
            ev[0].record(stream)
            for _ in range(5):
                pkg.rulebook_build_planned(coords, check=False, nbr=nbr, workspace=ws, plan=plan)
            ev[1].record(stream)
            torch.cuda.synchronize()
            table_plan_ms = ev[0].elapsed_time(ev[1]) / 5
    if planned:
        def step():
            pkg.subm_conv3x3_planned(feats, nbr, plan, packed, bias, w.co, out=out, out_dtype=out.dtype)
    else:
        def step():
            pkg.subm_conv3x3(feats, nbr, weight, bias, out=out, out_dtype=out.dtype, algo=args.algo)

    for _ in range(warmup):
        step()
    extra_warmup = settle(step, settle_ms) if settle_ms > 0 else 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev[0].record(stream)
    for _ in range(steps):
        step()
    ev[1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return {"ms": ev[0].elapsed_time(ev[1]) / steps, "wall": wall, "pairs": pairs, "planned": planned,
            "warmup_steps": warmup + extra_warmup,
            "rulebook_ms": rulebook_ms, "plan_ms": plan_ms, "table_plan_ms": table_plan_ms,
            "coords": coords, "feats": feats,
            "weight": weight, "bias": bias, "nbr": nbr, "plan": plan, "packed": packed}


if __name__ == "__main__":
    main()
