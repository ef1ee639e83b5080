"""Benchmark of the MI355X DCNv2 hot path (BASELINE metric: DCNv2 forward us/call and
TFLOP/s as a fraction of the HBM / MFMA rooflines at 1x128x64x64 -> 64, 16 groups).

A step is one DCNv2 forward call at the workload shape on device-resident synthetic
inputs: the NCHW -> padded channel-block repack plus the fused sampler + MFMA kernel,
exactly what dcn_forward_f16_prepacked_dev launches. K steps are captured into one
hipGraph (torch.cuda.CUDAGraph) and replayed once inside the timed region, so host
launch cost is not what is measured.

The dominant kernel (the fused sampler + MFMA GEMM) is also timed alone, from a graph of
fused-only launches, with HIP events on the stream it runs on; roofline.achieved is the
algorithmic bytes per launch over that duration.

cpu_baseline: the CPU oracle (a C restatement of the reference's DeformConvCPU.run),
single thread, on the FP32 version of the same shape.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "DCNv2 fwd µs/call + TFLOP/s (% HBM/MFMA roofline) at 1×128×64×64→64, 16 dg"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0

WORKLOADS = {
    2: "C2: DCNv2 1x128x64x64 -> 64, 3x3, 16 deformable groups, FP16 storage, FP32 accumulate, prepacked weights",
    3: "C3: DCNv2 16x128x64x64 -> 64, 3x3, 16 deformable groups, FP16, prepacked weights (batched 8K-eye tiles)",
    5: "C5: DCNv2 1x128x180x320 -> 64, 3x3, 16 deformable groups, FP16, prepacked weights (large map)",
}


KERNEL_NAMES = {1: "fused_kernel", 2: "staged_kernel", 3: "window_kernel", 4: "window_kernel",
                5: "narrow_kernel"}


def algorithmic_bytes(shape, elem=2) -> int:
    c = shape.counts()
    return elem * (c["input"] + c["offset"] + c["mask"] + c["output"] + c["weight"] + c["bias"])


def read_traffic(name: str):
    """HBM bytes per launch (FETCH_SIZE + WRITE_SIZE, copy-calibrated) from the committed
    rocprofv3 --pmc summary of this kernel and workload, if one exists."""
    path = ROOT / "profiles" / f"{name}.md"
    if not path.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", path.read_text())
    return float(m.group(1)) if m else None


def cpu_baseline(budget_s: float = 25.0) -> dict:
    import numpy as np

    import oracle
    from jasnamacos_amd import deform_conv as dc

    d = dc.generate_config_inputs(1, 1)
    s = d["shape"]
    args = [d[k] for k in ("input", "offset", "mask", "weight", "bias")]
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        oracle.forward_f32(s, *args)
        times.append(time.perf_counter() - t0)
        if len(times) >= 3 or time.perf_counter() - t_start + times[-1] > budget_s:
            break
    med = statistics.median(times)
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": med * 1e6,
        "unit": "us/call",
        "cores": 1,
        "kind": "port",
        "sample": (f"full FP32 call at 1x128x64x64->64, 16 dg (config 1), {len(times)} run(s), median; "
                   f"C restatement of DeformConvCPU.run, gcc -O2 -ffp-contract=off; host {cpu}, "
                   f"nproc {os.cpu_count()}"),
        "tflops": s.flops / med / 1e12,
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=2, choices=sorted(WORKLOADS))
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=5, help="repetitions of the fused-only timing")
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="after timing, run three device copies of this many MiB (the known-size "
                         "reference kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (tiles shard with no "
              "exchange; see DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        return 2
    if args.steps < 1:
        print("--steps must be >= 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from jasnamacos_amd import deform_conv as dc

    torch.cuda.set_device(0)
    d = dc.generate_config_inputs(args.config, args.seed)
    s = d["shape"]
    h = {k: np.asarray(d[k], np.float32).astype(np.float16) for k in ("input", "offset", "mask", "weight", "bias")}
    dev = {k: torch.from_numpy(h[k].view(np.int16)).cuda() for k in ("input", "offset", "mask", "weight", "bias")}
    ctx = dc.HipDeformConv(0)
    packed = ctx.prepack_dev(s, dev["weight"], dev["bias"])
    ctx.reserve(s)
    fused_cfg = ctx.get_fused_config(s)
    out = torch.empty(s.output_count, dtype=torch.int16, device="cuda")
    cb8 = torch.empty(ctx.cb8_count(s), dtype=torch.int16, device="cuda")
    stream = torch.cuda.Stream()

    def step(cur):
        ctx.forward_f16_prepacked_dev(s, dev["input"], dev["offset"], dev["mask"], packed, out, stream=cur)

    def fused_only(cur):
        ctx.forward_f16_prepacked_cb8_dev(s, cb8, dev["offset"], dev["mask"], packed, out, stream=cur)

    with torch.cuda.stream(stream):
        for _ in range(max(args.warmup, 1)):
            step(stream)
        ctx.pack_input_cb8_dev(s, dev["input"], cb8, stream=stream)
    torch.cuda.synchronize()

    g_step = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_step, stream=stream):
        cur = torch.cuda.current_stream()
        for _ in range(args.steps):
            step(cur)
    g_kernel = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_kernel, stream=stream):
        cur = torch.cuda.current_stream()
        for _ in range(args.steps):
            fused_only(cur)
    # untimed replays (graph upload, caches)
    with torch.cuda.stream(stream):
        g_step.replay()
        g_kernel.replay()
    torch.cuda.synchronize()

    # ---- timed region: exactly K steps -------------------------------------------
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        start.record(stream)
        g_step.replay()
        end.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    step_ms = start.elapsed_time(end) / args.steps
    us_per_call = step_ms * 1e3

    # ---- dominant kernel alone (events on its stream) ------------------------------
    kernel_us = []
    for _ in range(args.kernel_reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            a.record(stream)
            g_kernel.replay()
            b.record(stream)
        torch.cuda.synchronize()
        kernel_us.append(a.elapsed_time(b) * 1e3 / args.steps)
    k_us = statistics.median(kernel_us)

    if args.calibration_copy_mib > 0:
        src = torch.ones(args.calibration_copy_mib << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # correctness of what was timed: finite output with the expected checksum scale
    res = out.cpu().numpy().view(np.float16)
    finite = bool(np.all(np.isfinite(res.astype(np.float32))))

    nbytes = algorithmic_bytes(s)
    flops = s.flops
    achieved = nbytes / (k_us * 1e-6) / 1e9
    workload_name = {2: "dcn_c2_fp16", 3: "dcn_c3_fp16", 5: "dcn_c5_fp16"}[args.config]
    kernel_name = KERNEL_NAMES.get(fused_cfg["variant"], "fused_kernel")
    traffic = read_traffic(f"{kernel_name}_{workload_name}")
    line = {
        "metric": METRIC,
        "value": round(us_per_call, 4),
        "unit": "us/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_ms,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded SplitMix64/Box-Muller inputs of the BASELINE distributions; random weights)",
        "config": {
            "workload": WORKLOADS[args.config],
            "batch": s.batch, "in_channels": s.input_channels, "height": s.input_height, "width": s.input_width,
            "out_channels": s.output_channels, "kernel": [s.kernel_height, s.kernel_width],
            "deformable_groups": s.offset_groups, "fused_config": fused_cfg,
            "timing": f"{args.steps} calls captured in one hipGraph, one replay timed with HIP events",
        },
        "tflops": flops / (us_per_call * 1e-6) / 1e12,
        "step_hbm_frac": nbytes / (us_per_call * 1e-6) / 1e9 / HBM_PEAK_GBS,
        "step_mfma_frac": flops / (us_per_call * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS,
        "kernel_us": k_us,
        "kernel_tflops": flops / (k_us * 1e-6) / 1e12,
        "wall_ms_timed_region": wall_ms,
        "output_finite": finite,
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "kernel": kernel_name + " (sampler + MFMA GEMM)",
            "traffic_source": f"profiles/{kernel_name}_{workload_name}.md" if traffic else None,
            "algorithmic_bytes_per_launch": nbytes,
            "mfma_frac": flops / (k_us * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS,
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
    packed.free()
    ctx.close()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
