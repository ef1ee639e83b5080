"""Benchmark of the MI355X DCNv2 hot path (headline metric: DCNv2 forward us/call and
TFLOP/s as a fraction of the HBM / MFMA rooflines at 1x128x64x64 -> 64, 16 groups).

A step is one DCNv2 forward call at the workload shape on device-resident synthetic
inputs: the NCHW -> padded channel-block repack plus the fused sampler + MFMA kernel,
exactly what dcn_forward_f16_prepacked_dev launches. K steps are captured into one
hipGraph (torch.cuda.CUDAGraph) and replayed once inside the timed region, so host
launch cost is not what is measured.

The dominant kernel (the fused sampler + MFMA GEMM) is also timed alone, from a graph of
fused-only launches, with HIP events on the stream it runs on; roofline.achieved is the
algorithmic bytes per launch over that duration.

Config 1 is the FP32 entry point (runFloat32): one direct kernel per call, in the CPU
oracle's summation order, priced against the FP32 matrix peak.

--dtype bf16 (configs 2, 3, 5) measures the BF16 storage path instead (dcn_forward_bf16_
prepacked_dev: the same repack, then the narrow kernel (C2) or the window kernel (C3,
C5) with the BF16 sampler and BF16 MFMA); its timed output is checked against the FP32
oracle on the widened BF16 inputs with bars 8x the FP16 ones.

config.sampler names the sampler arithmetic of the timed kernel: "fast" (the mask folded
into the four bilinear weights, rounded to FP16, packed-FP16 blend) or "exact" (the
reference's half(FP32 bilinear x mask), MetalShader.swift:371-379). For FP16 storage the
exact sampler is also timed beside it (exact_sampler, exact_kernel_us) on the kernel the
library picks for it.

cpu_baseline: the CPU oracle (a C restatement of the reference's DeformConvCPU.run),
single thread, on a bounded sample of the benchmarked workload with the same inputs. In
the same leg the oracle's output of the whole call (C3/C5: the same restatement on the
host's threads) checks the GPU's timed output (timed_output_check) and the exact
sampler's output (exact_sampler.output_check).

Diagnostics (one JSON line each, instead of the bench line): --launch-floor (empty
kernels of the fused kernels' launch shapes in a hipGraph), --gather (the reference's
gather phase alone, im2col to HBM, at C2) and --tile-clock (configs 3, 5: the tile
kernel's per-workgroup start/end stamps, so the spread of workgroup times behind the
kernel's duration). --seed-sweep N runs the bench at input seeds 0 .. N-1 and reports
the per-seed times and their spread (the C3/C5 kernel times depend on the offset field).
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
FP32_PEAK_TFLOPS = 157.3

WORKLOADS = {
    1: "C1: DCNv2 1x128x64x64 -> 64, 3x3, 16 deformable groups, FP32 (runFloat32, oracle summation order, bit-exact)",
    2: "C2: DCNv2 1x128x64x64 -> 64, 3x3, 16 deformable groups, FP16 storage, FP32 accumulate, prepacked weights",
    3: "C3: DCNv2 16x128x64x64 -> 64, 3x3, 16 deformable groups, FP16, prepacked weights (batched 8K-eye tiles)",
    5: "C5: DCNv2 1x128x180x320 -> 64, 3x3, 16 deformable groups, FP16, prepacked weights (large map)",
    4: "C4: BasicVSR++ propagation body per frame (hipGraph)",
}


KERNEL_NAMES = {0: "direct_shared_f32_kernel", 1: "fused_kernel", 2: "staged_kernel", 3: "window_kernel", 4: "window_kernel",
                5: "narrow_kernel", 6: "window_async_kernel", 7: "tile_kernel"}


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


# The FP16 paths' parity bar against the FP32 oracle (the tests' tolerance).
MAX_ABS_F16, MEAN_ABS_F16 = 2e-2, 1e-3
# Output channels of the C5 sample: both ends of both 32-channel MFMA column blocks.
C5_SAMPLE_OCS = (0, 1, 2, 3, 28, 29, 30, 31, 60, 61, 62, 63)


def _cpu_name() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(config: int, s, inputs: dict, gpu_out, budget_s: float = 25.0,
                 bars: tuple[float, float] = (MAX_ABS_F16, MEAN_ABS_F16)) -> tuple[dict, dict]:
    """The CPU oracle (C restatement of DeformConvCPU.run, DeformConv.swift:76-138) timed on
    a bounded sample of the benchmarked workload, single thread, on the same (FP16-rounded
    for C2/C3/C5) inputs the GPU ran; value is scaled to one whole call. The oracle's output
    of the whole call then checks the GPU's outputs: `gpu_out` is one output or a dict of
    named outputs; returns (baseline, check) or (baseline, {name: check})."""
    import dataclasses

    import numpy as np

    import oracle

    args = [np.asarray(inputs[k], np.float32) for k in ("input", "offset", "mask", "weight", "bias")]
    c = s.counts()
    if config in (1, 2):
        sample, scale = "the full call", 1.0

        def run():
            return [(slice(0, c["output"]), oracle.forward_f32(s, *args))]
    elif config == 3:
        tile = dataclasses.replace(s, batch=1)
        tc = tile.counts()
        images = (0, s.batch - 1)
        sample, scale = f"images {images[0]} and {images[1]} of {s.batch} (x{s.batch // len(images)})", s.batch / 2

        def run():
            res = []
            for b in images:
                part = [args[0][b * tc["input"]:(b + 1) * tc["input"]], args[1][b * tc["offset"]:(b + 1) * tc["offset"]],
                        args[2][b * tc["mask"]:(b + 1) * tc["mask"]], args[3], args[4]]
                res.append((slice(b * tc["output"], (b + 1) * tc["output"]), oracle.forward_f32(tile, *part)))
            return res
    else:  # C5: a slice of output channels, every pixel and sample
        plane = s.output_height * s.output_width
        ocs = C5_SAMPLE_OCS
        sample = f"output channels {list(ocs)} of {s.output_channels} (x{s.output_channels / len(ocs):.2f})"
        scale = s.output_channels / len(ocs)

        def run():
            res = []
            for oc in ocs:
                ref = oracle.forward_f32_oc_range(s, *args, oc, oc + 1)
                res.append((slice(oc * plane, (oc + 1) * plane), ref[oc * plane:(oc + 1) * plane]))
            return res

    times, t_start = [], time.perf_counter()
    while True:
        t0 = time.perf_counter()
        ref = run()
        times.append(time.perf_counter() - t0)
        if len(times) >= 3 or time.perf_counter() - t_start + times[-1] > budget_s:
            break
    med = statistics.median(times) * scale
    baseline = {
        "value": med * 1e6,
        "unit": "us/call",
        "cores": 1,
        "kind": "port",
        "sample": (f"{sample} at {s.batch}x{s.input_channels}x{s.input_height}x{s.input_width}->"
                   f"{s.output_channels}, {s.offset_groups} dg, {len(times)} run(s), median scaled to one call; "
                   f"C restatement of DeformConvCPU.run, gcc -O2 -ffp-contract=off; host {_cpu_name()}, "
                   f"nproc {os.cpu_count()}"),
        "tflops": s.flops / med / 1e12,
    }
    # The same restatement spread over the host's cores (at most 16, the box's CPU share),
    # bit-identical results, for the shapes where one call fits the budget.
    if config in (1, 2):
        threads = min(16, os.cpu_count() or 1)
        mt = []
        for _ in range(3):
            t0 = time.perf_counter()
            oracle.forward_f32_threads(s, *args, threads=threads)
            mt.append(time.perf_counter() - t0)
        baseline["all_cores"] = {"value": statistics.median(mt) * 1e6, "unit": "us/call", "cores": threads,
                                 "sample": "same call, output channels split over threads, median of 3"}

    # The checker of the timed outputs: the whole call. For C1/C2 the timed sample is the
    # whole call; for C3/C5 the same restatement runs once more over output channels on the
    # host's threads (bit-identical to the single-threaded one).
    if config in (1, 2):
        want = np.concatenate([r for _, r in ref])
        check_sample = sample
    else:
        want = oracle.forward_f32_threads(s, *args, threads=min(16, os.cpu_count() or 1))
        check_sample = "the full call (every output channel and pixel)"
    outputs = gpu_out if isinstance(gpu_out, dict) else {"timed": gpu_out}
    checks = {}
    for name, o in outputs.items():
        got = np.asarray(o, np.float32).reshape(-1)
        err = np.abs(got.astype(np.float64) - want.astype(np.float64))
        check = {"oracle": "FP32 DeformConvCPU.run restatement on the inputs the GPU ran", "sample": check_sample,
                 "values": int(want.size), "max_abs_err": float(err.max()), "mean_abs_err": float(err.mean())}
        if config == 1:
            check["bound"] = "bit-exact"
            check["within"] = bool(np.array_equal(got.view(np.uint32), want.view(np.uint32)))
        else:
            check["bound"] = {"max": bars[0], "mean": bars[1]}
            check["within"] = bool(check["max_abs_err"] <= bars[0] and check["mean_abs_err"] <= bars[1])
        checks[name] = check
    return baseline, (checks if isinstance(gpu_out, dict) else checks["timed"])


def calibration_copies(mib: int) -> None:
    """Three device copies of `mib` MiB: the known-size kernel that scales rocprofv3's
    FETCH_SIZE / WRITE_SIZE readings to bytes."""
    import torch

    src = torch.ones(mib << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def bench_body(args) -> int:
    """Config C4: one BasicVSR++ propagation body per frame, each frame one hipGraph launch.

    30 frames of a synthetic clip are captured once (one graph per frame: frame t reads
    the features of steps t-1 and t-2); a step is one frame's graph launch. The timed
    region replays K frames, cycling through the clip."""
    import numpy as np
    import torch

    from jasnamacos_amd import deform_conv as dc

    clip = dc.generate_body_inputs(seed=args.seed)
    H, W, frames, blocks = clip["height"], clip["width"], clip["frames"], clip["blocks"]
    plane = H * W
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()  # noqa: E731
    ctx = dc.HipDeformConv(0)
    wd = {k: dev(v) for k, v in clip["weights"].items()}
    body = ctx.body(H, W, wd, branch=0, blocks=blocks)
    feats, flows = dev(clip["feats"]), dev(clip["flows"])
    props = torch.zeros(frames, 64 * plane, dtype=torch.int16, device="cuda")
    flow2s = torch.zeros(frames, 2 * plane, dtype=torch.int16, device="cuda")
    zero_f = torch.zeros(64 * plane, dtype=torch.int16, device="cuda")
    zero_flow = torch.zeros(2 * plane, dtype=torch.int16, device="cuda")
    # The clip's form of a step: the warped features come from CB8 copies that each step
    # writes beside its NCHW output (dcn_body_capture_cb8).
    props_cb8 = torch.zeros(frames, dc.cb8_tensor_count(64, H, W), dtype=torch.int16, device="cuda")
    graphs = []
    for t in range(frames):
        # Frame 0 and 1 read the previous clip's last features, so that every replay
        # of the cycle is a full second-order step.
        graphs.append(body.capture_cb8(feats[t], flows[t], flows[t - 1], props_cb8[t - 1], props_cb8[t - 2],
                                       flow2s[t], props[t], props_cb8[t], has_second_order=True))
    stream = torch.cuda.Stream()
    for i in range(max(args.warmup, frames)):
        graphs[i % frames].launch(stream)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        start.record(stream)
        for i in range(args.steps):
            graphs[i % frames].launch(stream)
        end.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    step_ms = start.elapsed_time(end) / args.steps
    out = props.cpu().numpy().view(np.float16)
    flops = dc.body_flops(H, W, 0, blocks)
    tflops = flops / (step_ms * 1e-3) / 1e12
    for g in graphs:
        g.free()
    body.free()
    clip_line = tiles_line = None
    if not args.frames_only:
        clip_line = bench_clip(args, ctx, dc, clip, dev)
        tiles_line = bench_body_tiles(args, ctx, dc, clip, dev)
    if args.calibration_copy_mib > 0:
        calibration_copies(args.calibration_copy_mib)
    cpu = None if args.no_cpu_baseline else cpu_baseline_body(clip)
    line = {
        "metric": "BasicVSR++ propagation body us/frame (C4: offset convs + DCNv2 + 5-block backbone, hipGraph per frame)",
        "value": round(step_ms * 1e3, 3),
        "unit": "us/frame",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_ms,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (numpy PCG64 clip: N(0,1) features, smooth +-4 px flows, N(0,0.02) weights)",
        "config": {"workload": "C4: one propagation body per frame, 1x64x64x64 features, branch 0, "
                               f"{blocks} residual blocks, {frames}-frame clip, one hipGraph per frame",
                   "height": H, "width": W, "frames": frames, "blocks": blocks},
        "tflops": tflops,
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": tflops / MFMA_F16_PEAK_TFLOPS, "traffic": None,
                     "kernel": "whole body graph (temporal + conv_offset 1, 6 conv pairs, offsets conv + DCN, input conv)",
                     "flops_per_step": flops},
        "wall_ms_timed_region": wall_ms,
        "output_finite": bool(np.all(np.isfinite(out.astype(np.float32)))),
        "clip": clip_line,
        "tiles": tiles_line,
        "cpu_baseline": cpu,
    }
    ctx.close()
    print(json.dumps(line), flush=True)
    return 0


def bench_body_tiles(args, ctx, dc, clip, dev, tiles: int = 16) -> dict:
    """The same body step over 16 tiles at once (dcn_body_create_tiles: every kernel runs
    once over the batch), one captured graph replayed; the production pipeline runs many
    tiles of a frame (README.md:589-591). Reported beside the one-tile frame time."""
    import numpy as np
    import torch

    H, W, blocks = clip["height"], clip["width"], clip["blocks"]
    plane = H * W
    wd = {k: dev(v) for k, v in clip["weights"].items()}
    body = ctx.body(H, W, wd, branch=0, blocks=blocks, tiles=tiles)
    rng = np.random.default_rng(args.seed + 7)
    f16 = lambda a: np.asarray(a, np.float32).astype(np.float16)  # noqa: E731
    feats = [dev(f16(rng.standard_normal(tiles * 64 * plane))) for _ in range(3)]
    flows = [dev(f16(rng.uniform(-4, 4, tiles * 2 * plane))) for _ in range(2)]
    flow2 = torch.zeros(tiles * 2 * plane, dtype=torch.int16, device="cuda")
    out = torch.zeros(tiles * 64 * plane, dtype=torch.int16, device="cuda")
    graph = body.capture(feats[0], flows[0], flows[1], feats[1], feats[2], flow2, out, has_second_order=True)
    stream = torch.cuda.Stream()
    for _ in range(10):
        graph.launch(stream)
    torch.cuda.synchronize()
    reps = 50
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(reps):
            graph.launch(stream)
        end.record(stream)
    torch.cuda.synchronize()
    step_ms = start.elapsed_time(end) / reps
    result = out.cpu().numpy().view(np.float16).astype(np.float32)
    flops = tiles * dc.body_flops(H, W, 0, blocks)
    graph.free()
    body.free()
    return {"workload": f"one body step (branch 0, {blocks} blocks) over {tiles} 64x64 tiles, one hipGraph",
            "tiles": tiles, "us_per_step": step_ms * 1e3, "us_per_tile": step_ms * 1e3 / tiles,
            "tflops": flops / (step_ms * 1e-3) / 1e12, "replays_timed": reps,
            "output_finite": bool(np.all(np.isfinite(result)))}


def bench_spynet(args) -> int:
    """SPyNet flow of a frame pair, both directions, from two 256 x 256 RGB LQ tiles: the
    quarter bicubic downsample of each tile, then the six-level network on the 64 x 64
    copies, all in one hipGraph; a step is one replay (one bidirectional pair)."""
    import numpy as np
    import torch

    from jasnamacos_amd import deform_conv as dc

    d = dc.generate_spynet_inputs(seed=args.seed)
    tile = d["tile"]
    H = W = tile // 4
    dev = lambda a: torch.from_numpy(np.array(a, np.float16).view(np.int16)).cuda()  # noqa: E731
    ctx = dc.HipDeformConv(0)
    spy = ctx.spynet(H, W, {k: dev(v) for k, v in d["weights"].items()})
    lq = [dev(d["reference"]), dev(d["support"])]
    small = [torch.zeros(3 * H * W, dtype=torch.int16, device="cuda") for _ in range(2)]
    flow = torch.zeros(2 * 2 * H * W, dtype=torch.int16, device="cuda")
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        cur = torch.cuda.current_stream()
        for i in range(2):
            ctx.bicubic_quarter_f16_dev(3, tile, tile, lq[i], small[i], stream=cur)
        spy.flow_dev(small[0], small[1], flow, both_directions=True, stream=cur)
    for _ in range(max(args.warmup, 1)):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(args.steps):
            graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    step_ms = start.elapsed_time(end) / args.steps
    out = flow.cpu().numpy().view(np.float16).astype(np.float32)
    flops = 2 * dc.spynet_flops(H, W)
    tflops = flops / (step_ms * 1e-3) / 1e12
    del graph
    spy.free()
    clip_line = bench_spynet_clip(args, ctx, dc, d, dev)
    cpu = None if args.no_cpu_baseline else cpu_baseline_spynet(d)
    line = {
        "metric": "SPyNet bidirectional flow pair us (two 256x256 RGB tiles -> bicubic 1/4 -> six-level net at 64x64)",
        "value": round(step_ms * 1e3, 3),
        "unit": "us/pair",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_ms,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (numpy PCG64: sinusoid RGB tiles, He-normal random SPyNet weights)",
        "config": {"workload": "SPyNet pair: 2 x bicubic quarter downsample + spynet(ref, sup) and "
                               "spynet(sup, ref), 6 levels 2..64, one hipGraph", "height": H, "width": W},
        "tflops": tflops,
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": tflops / MFMA_F16_PEAK_TFLOPS, "traffic": None,
                     "kernel": "whole pair graph (2 bicubic, pyramid, 6 x (prepare + 5 convk))",
                     "flops_per_step": flops},
        "wall_ms_timed_region": wall_ms,
        "flow_abs_max": float(np.abs(out).max()),
        "output_finite": bool(np.all(np.isfinite(out))),
        "clip": clip_line,
        "cpu_baseline": cpu,
    }
    ctx.close()
    print(json.dumps(line), flush=True)
    return 0


def bench_spynet_clip(args, ctx, dc, d, dev, frames: int = 30) -> dict:
    """All flows of a 30-frame clip (both directions of the 29 adjacent pairs) from 256 x 256
    tiles: one bicubic launch over every frame, then dcn_spynet_clip_flows_dev, which runs
    each level once over the batch of 58 images; one hipGraph, a step is one clip."""
    import numpy as np
    import torch

    tile = d["tile"]
    H = W = tile // 4
    rng = np.random.default_rng(args.seed + 1)
    shifts = np.cumsum(rng.uniform(-2, 2, (frames, 2)), axis=0)
    lq = [dc.generate_spynet_inputs(tile, seed=args.seed)["reference"]]
    base = np.asarray(lq[0], np.float16).reshape(3, tile, tile)
    for t in range(1, frames):  # the first tile moved by a random walk of whole pixels
        lq.append(np.roll(base, (int(round(shifts[t, 0])), int(round(shifts[t, 1]))), axis=(1, 2)).ravel())
    spy = ctx.spynet(H, W, {k: dev(v) for k, v in d["weights"].items()}, max_frames=frames)
    lq_t = dev(np.concatenate(lq))
    small = torch.zeros(frames * 3 * H * W, dtype=torch.int16, device="cuda")
    flows = torch.zeros(2 * (frames - 1) * 2 * H * W, dtype=torch.int16, device="cuda")
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        cur = torch.cuda.current_stream()
        ctx.bicubic_quarter_f16_dev(3 * frames, tile, tile, lq_t, small, stream=cur)
        spy.clip_flows_dev(small, frames, flows, stream=cur)
    graph.replay()
    torch.cuda.synchronize()
    reps = 10
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(reps):
            graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    clip_ms = start.elapsed_time(end) / reps
    out = flows.cpu().numpy().view(np.float16).astype(np.float32)
    flops = 2 * (frames - 1) * dc.spynet_flops(H, W)
    del graph
    spy.free()
    return {"workload": f"{frames} frames: bicubic 1/4 of every tile + both directions of the {frames - 1} pairs",
            "ms_per_clip": clip_ms, "pairs": frames - 1, "us_per_pair": clip_ms * 1e3 / (frames - 1),
            "tflops": flops / (clip_ms * 1e-3) / 1e12, "replays_timed": reps,
            "output_finite": bool(np.all(np.isfinite(out)))}


def cpu_baseline_spynet(d) -> dict:
    """The same pair through the C oracle on the host: two bicubic downsamples, both
    pyramids, both directions' six levels (7x7 convs on all host cores, OpenMP)."""
    import os

    import numpy as np

    import oracle

    oracle.load()
    tile = d["tile"]
    H = W = tile // 4
    w = d["weights"]
    t0 = time.perf_counter()
    small = [oracle.bicubic_quarter_f16(3, tile, tile, d[k]) for k in ("reference", "support")]
    pyr = [oracle.spynet_pyramid_f16(H, W, 6, s) for s in small]
    for a, b in ((0, 1), (1, 0)):
        flow, fh, fw = None, 1, 1
        for level in range(6):
            h, ww = H >> (5 - level), W >> (5 - level)
            x, base = oracle.spynet_prepare_f16(ww, h, level == 0, pyr[a][level], pyr[b][level], flow, fw, fh)
            for i, (ci, co) in enumerate([(8, 32), (32, 64), (64, 32), (32, 16), (16, 2)]):
                x = oracle.convk_f16(7, ci, co, h, ww, x, w[f"w{level}_{i}"], w[f"b{level}_{i}"], 2 if i < 4 else 0)
            flow, fh, fw = oracle.add_f16(base, x), h, ww
    seconds = time.perf_counter() - t0
    return {"value": seconds * 1e6, "unit": "us/pair", "cores": os.cpu_count() or 1, "kind": "port",
            "sample": "one bidirectional pair (64x64, six levels) through the C oracle, "
                      f"flow finite: {bool(np.all(np.isfinite(flow.astype(np.float32))))}"}


def bench_clip(args, ctx, dc, clip, dev) -> dict:
    """All four branches over the 30-frame clip captured as ONE hipGraph (the whole-clip
    command buffer of the reference): 4 x 30 body steps, backbone inputs 128..320
    channels. Reported beside the per-frame line; one replay is one clip."""
    import numpy as np
    import torch

    H, W, frames, blocks = clip["height"], clip["width"], clip["frames"], clip["blocks"]
    plane = H * W
    weights = [clip["weights"]] + [dc.generate_body_inputs(H, W, 1, branch=b, blocks=blocks,
                                                           seed=args.seed + b)["weights"] for b in (1, 2, 3)]
    wd = [{k: dev(v) for k, v in w.items()} for w in weights]
    pc = ctx.clip(H, W, frames, wd, blocks=blocks)
    spatial = dev(clip["feats"])
    flows = dev(clip["flows"]).view(frames, 2 * plane)
    backward, forward = flows[: frames - 1].contiguous(), flows[1:].contiguous()
    prop = torch.zeros(4 * frames * 64 * plane, dtype=torch.int16, device="cuda")
    graph = pc.capture(spatial, backward, forward, prop)
    stream = torch.cuda.Stream()
    graph.launch(stream)
    torch.cuda.synchronize()
    reps = 3
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(reps):
            graph.launch(stream)
        end.record(stream)
    torch.cuda.synchronize()
    clip_ms = start.elapsed_time(end) / reps
    out = prop.cpu().numpy().view(np.float16)
    flops = dc.clip_flops(H, W, frames, blocks)
    graph.free()
    # The same clip fed by learned flows: the 256 x 256 LQ tiles downsampled, SPyNet over
    # every adjacent pair (dcn_spynet_clip_flows_dev) and the four branches, one stream.
    sd = dc.generate_spynet_inputs(4 * H, seed=args.seed)
    spy = ctx.spynet(H, W, {k: dev(v) for k, v in sd["weights"].items()}, max_frames=frames)
    base_tile = np.asarray(sd["reference"], np.float16).reshape(3, 4 * H, 4 * W)
    lq = dev(np.concatenate([np.roll(base_tile, (t, -t), axis=(1, 2)).ravel() for t in range(frames)]))
    small = torch.zeros(frames * 3 * plane, dtype=torch.int16, device="cuda")
    learned = torch.zeros(2 * (frames - 1) * 2 * plane, dtype=torch.int16, device="cuda")
    half = (frames - 1) * 2 * plane

    def learned_clip(cur):
        ctx.bicubic_quarter_f16_dev(3 * frames, 4 * H, 4 * W, lq, small, stream=cur)
        spy.clip_flows_dev(small, frames, learned, stream=cur)
        pc.run_dev(spatial, learned[:half], learned[half:], prop, 0, stream=cur)

    lgraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(lgraph, stream=stream):
        learned_clip(torch.cuda.current_stream())
    lgraph.replay()
    torch.cuda.synchronize()
    start2, end2 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start2.record(stream)
        for _ in range(reps):
            lgraph.replay()
        end2.record(stream)
    torch.cuda.synchronize()
    learned_ms = start2.elapsed_time(end2) / reps
    learned_out = prop.cpu().numpy().view(np.float16)
    del lgraph
    spy.free()
    pc.free()
    # The same clip over 16 tiles at once (dcn_clip_create_tiles): every kernel of a body
    # step runs once over the tiles, whose inputs are the clip's shifted per tile.
    tiles = 16
    pt = ctx.clip(H, W, frames, wd, blocks=blocks, tiles=tiles)
    feats = np.asarray(clip["feats"]).reshape(frames, 1, -1)
    fl = np.asarray(clip["flows"]).reshape(frames, 1, -1)
    t_spatial = dev(np.concatenate([np.roll(feats, t, axis=2) for t in range(tiles)], axis=1))
    t_flows = dev(np.concatenate([np.roll(fl, t, axis=2) for t in range(tiles)], axis=1)).view(frames, -1)
    t_prop = torch.zeros(4 * frames * tiles * 64 * plane, dtype=torch.int16, device="cuda")
    tgraph = pt.capture(t_spatial, t_flows[: frames - 1].contiguous(), t_flows[1:].contiguous(), t_prop)
    tgraph.launch(stream)
    torch.cuda.synchronize()
    start3, end3 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start3.record(stream)
        for _ in range(reps):
            tgraph.launch(stream)
        end3.record(stream)
    torch.cuda.synchronize()
    tiles_ms = start3.elapsed_time(end3) / reps
    tiles_finite = bool(np.all(np.isfinite(t_prop.cpu().numpy().view(np.float16).astype(np.float32))))
    tgraph.free()
    pt.free()
    return {"workload": f"4 branches x {frames} frames (backward_1, forward_1, backward_2, forward_2), one hipGraph",
            "ms_per_clip": clip_ms, "body_steps": 4 * frames, "us_per_body_step": clip_ms * 1e3 / (4 * frames),
            "tflops": flops / (clip_ms * 1e-3) / 1e12, "flops_per_clip": flops, "replays_timed": reps,
            "output_finite": bool(np.all(np.isfinite(out.astype(np.float32)))),
            "with_spynet_flows": {"ms_per_clip": learned_ms,
                                  "workload": "bicubic 1/4 of 30 LQ tiles + SPyNet clip flows + the four branches, "
                                              "one hipGraph",
                                  "output_finite": bool(np.all(np.isfinite(learned_out.astype(np.float32))))},
            "tiles": {"tiles": tiles, "ms_per_clip": tiles_ms, "ms_per_tile_clip": tiles_ms / tiles,
                      "tflops": tiles * flops / (tiles_ms * 1e-3) / 1e12, "output_finite": tiles_finite,
                      "workload": f"the clip over {tiles} 64x64 tiles at once (dcn_clip_create_tiles), one hipGraph"}}


def cpu_baseline_body(clip) -> dict:
    """One C4 body step (branch 0) on the host through the C oracle: temporal preparation,
    the four offset convs, the offset transform, the FP32 DCN and the backbone, FP16 between
    layers; the convs run on all host cores (OpenMP), the DCN on the same threads."""
    import os

    import numpy as np

    import oracle

    oracle.load()
    H, W, blocks = clip["height"], clip["width"], clip["blocks"]
    w = clip["weights"]
    feats, flows = clip["feats"], clip["flows"].reshape(clip["frames"], -1)
    threads = os.cpu_count() or 1
    f16 = lambda a: np.asarray(a, np.float32).astype(np.float16)  # noqa: E731
    t0 = time.perf_counter()
    flow2, cond, dinp = oracle.temporal_prepare_f16(W, H, True, feats[1], feats[2], feats[0], flows[2], flows[1])
    h = cond
    for i, (ci, co) in enumerate([(196, 64), (64, 64), (64, 64)]):
        h = oracle.conv3x3_f16(ci, co, H, W, h, w[f"offset_w{i}"], w[f"offset_b{i}"], 1, 0.1)
    raw = oracle.conv3x3_f16(64, 432, H, W, h, w["offset_w3"], w["offset_b3"], 0, 0.1)
    off, msk = oracle.offset_transform_f16(H * W, raw, flows[2], flow2)
    shape = oracle.OracleShape(1, 128, H, W, 64, H, W, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
    aligned = f16(oracle.forward_f32_threads(shape, dinp.astype(np.float32), off.astype(np.float32),
                                             msk.astype(np.float32), w["dcn_w"].astype(np.float32),
                                             w["dcn_b"].astype(np.float32), threads))
    bb = np.concatenate([feats[2], aligned])
    feat = oracle.conv3x3_f16(128, 64, H, W, bb, w["backbone_w0"], w["backbone_b0"], 1, 0.1)
    for i in range(blocks):
        t = oracle.conv3x3_f16(64, 64, H, W, feat, w[f"backbone_w{1 + 2 * i}"], w[f"backbone_b{1 + 2 * i}"], 2, 0.1)
        feat = oracle.conv3x3_f16(64, 64, H, W, t, w[f"backbone_w{2 + 2 * i}"], w[f"backbone_b{2 + 2 * i}"], 0,
                                  0.1, feat)
    out = f16(aligned.astype(np.float32) + feat.astype(np.float32))
    seconds = time.perf_counter() - t0
    return {"value": seconds * 1e6, "unit": "us/frame", "cores": threads, "kind": "port",
            "sample": "one full body step (branch 0, 64x64, 5 blocks) through the C oracle, "
                      f"output finite: {bool(np.all(np.isfinite(out.astype(np.float32))))}"}


def bench_share(args, ctx, dc, d, dev, share: int = 2) -> dict:
    """C3 at one GPU's share of an 8-GPU split: the first `share` tiles of the same inputs
    (tiles shard with no exchange, so a rank runs exactly this), timed like the main line:
    `steps` calls (repack + fused) in one hipGraph, HIP events around one replay."""
    import dataclasses

    import torch

    s = dataclasses.replace(d["shape"], batch=share)
    per = {k: d["shape"].counts()[k] // d["shape"].batch for k in ("input", "offset", "mask")}
    x, off, msk = (dev[k][: per[k] * share] for k in ("input", "offset", "mask"))
    packed = ctx.prepack_dev(s, dev["weight"], dev["bias"])
    ctx.reserve(s)
    cfg = ctx.get_fused_config(s)
    out = torch.empty(s.output_count, dtype=torch.int16, device="cuda")
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for _ in range(max(args.warmup, 1)):
            ctx.forward_f16_prepacked_dev(s, x, off, msk, packed, out, stream=stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        cur = torch.cuda.current_stream()
        for _ in range(args.steps):
            ctx.forward_f16_prepacked_dev(s, x, off, msk, packed, out, stream=cur)
    with torch.cuda.stream(stream):
        graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        a.record(stream)
        graph.replay()
        b.record(stream)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / args.steps
    packed.free()
    nbytes = algorithmic_bytes(s)
    return {"workload": f"C3 per-GPU share on 8 GPUs: the first {share} of the 16 tiles", "batch": share,
            "us_per_call": us, "tflops": s.flops / (us * 1e-6) / 1e12,
            "hbm_frac": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, "fused_config": cfg}


def _graph_us(torch, stream, fn, steps: int, reps: int = 5) -> float:
    """`fn(stream)` captured `steps` times in one hipGraph; median over `reps` replays of the
    replay time (HIP events on the capture stream) per launch, in us."""
    with torch.cuda.stream(stream):
        fn(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        cur = torch.cuda.current_stream()
        for _ in range(steps):
            fn(cur)
    with torch.cuda.stream(stream):
        graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            a.record(stream)
            graph.replay()
            b.record(stream)
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b) * 1e3 / steps)
    return statistics.median(times)


# Launch shapes of the kernels a DCN call runs: (name, workgroups, threads, LDS bytes).
FLOOR_SHAPES = [
    ("narrow_kernel C2 (256 x 12 waves, 48 KB LDS)", 256, 768, 49152),
    ("pack_cb8_kernel C2 (19 x 16 blocks of 256)", 304, 256, 0),
    ("tile_kernel C3 (512 x 4 waves, 77.6 KB LDS)", 512, 256, 79456),
    ("tile_kernel C5 (464 x 4 waves, 77.6 KB LDS)", 464, 256, 79456),
    ("one wave", 1, 64, 0),
]


def bench_launch_floor(args) -> int:
    """Empty kernels (dcn_launch_floor_dev) of the launch shapes of the C2/C3/C5 kernels,
    each captured `steps` times in a hipGraph: the per-launch floor inside a graph, the
    part of a kernel's in-graph time that no change to its body removes."""
    import torch

    from jasnamacos_amd import deform_conv as dc

    ctx = dc.HipDeformConv(0)
    stream = torch.cuda.Stream()
    rows = []
    for name, wg, threads, lds in FLOOR_SHAPES:
        us = _graph_us(torch, stream, lambda st, wg=wg, t=threads, l=lds: ctx.launch_floor_dev(wg, t, l, stream=st),
                       args.steps, args.kernel_reps)
        rows.append({"shape": name, "workgroups": wg, "threads": threads, "lds_bytes": lds, "us_per_launch": us})
    ctx.close()
    print(json.dumps({"metric": "launch floor: empty kernel per launch in a hipGraph", "unit": "us", "n_gpus": 1,
                      "steps": args.steps, "data": "no data (empty kernels)", "shapes": rows}), flush=True)
    return 0


def bench_tile_clock(args) -> int:
    """Per-workgroup clock stamps of the tile kernel (variant 7) at config 3 or 5
    (dcn_set_tile_clock_dev): each workgroup's start and end on the 100 MHz constant clock,
    its tile and its CU (HW_ID, XCC_ID), from the last of 10 back-to-back fused launches on
    the CB8 input, repeated --clock-runs times. Prints one JSON line: the spread of the
    workgroup durations, how many CUs ran one and two workgroups and the durations of
    each kind, the slowest workgroups; the output with the stamps on is compared bit for
    bit with the output with them off."""
    import numpy as np
    import torch

    from jasnamacos_amd import deform_conv as dc

    d = dc.generate_config_inputs(args.config, args.seed)
    s = d["shape"]
    dev = {k: torch.from_numpy(np.asarray(d[k], np.float32).astype(np.float16).view(np.int16)).cuda()
           for k in ("input", "offset", "mask", "weight", "bias")}
    ctx = dc.HipDeformConv(0)
    stream = torch.cuda.Stream()
    packed = ctx.prepack_dev(s, dev["weight"], dev["bias"])
    ctx.reserve(s)
    if args.variant or args.mt or args.ks:
        ctx.set_fused_config(args.mt, args.ks, -1, args.variant)
    cfg = ctx.get_fused_config(s)
    if cfg["variant"] != 7:
        print(f"--tile-clock: config {args.config} runs fused variant {cfg['variant']}, not the tile kernel",
              file=sys.stderr)
        return 2
    tw = 32 if cfg["mt"] == 32 else 16
    th = 128 // tw
    tiles = s.batch * -(-s.output_height // th) * -(-s.output_width // tw)
    grid = (tiles + 7) // 8 * 8
    out = torch.empty(s.output_count, dtype=torch.int16, device="cuda")
    cb8 = torch.empty(ctx.cb8_count(s), dtype=torch.int16, device="cuda")
    clock = torch.zeros(4 * grid, dtype=torch.int64, device="cuda")
    launches = 10

    def fused(n):
        with torch.cuda.stream(stream):
            for _ in range(n):
                ctx.forward_f16_prepacked_cb8_dev(s, cb8, dev["offset"], dev["mask"], packed, out, stream=stream)

    with torch.cuda.stream(stream):
        ctx.pack_input_cb8_dev(s, dev["input"], cb8, stream=stream)
    fused(20)
    torch.cuda.synchronize()
    ref = out.clone()
    ctx.set_tile_clock_dev(clock)
    runs, identical, launch_us = [], True, []
    try:
        for _ in range(args.clock_runs):
            clock.zero_()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            fused(launches)
            b.record(stream)
            torch.cuda.synchronize()
            launch_us.append(a.elapsed_time(b) * 1e3 / launches)
            runs.append(clock.cpu().numpy().view(np.uint64).reshape(grid, 4).copy())
            identical = identical and bool(torch.equal(out, ref))
    finally:
        ctx.set_tile_clock_dev(None)

    def analyse(rec):
        valid = rec[:, 0] != 0
        blocks = np.nonzero(valid)[0]
        start = rec[valid, 0].astype(np.int64)
        end = np.maximum(rec[valid, 1], rec[valid, 2]).astype(np.int64)
        meta = rec[valid, 3]
        tile = (meta & np.uint64(0x0FFFFFFF)).astype(np.int64)
        xcc = ((meta >> np.uint64(28)) & np.uint64(15)).astype(np.int64)
        cu = xcc * 256 + ((meta >> np.uint64(40)) & np.uint64(0xFF)).astype(np.int64)  # HW_ID bits 15:8
        dur = (end - start) * 0.01  # 100 MHz ticks -> us
        _, inverse, counts = np.unique(cu, return_inverse=True, return_counts=True)
        per_wg = counts[inverse]
        # On a CU that runs two workgroups, the one with the lower blockIdx was dispatched first.
        first = np.array([blocks[i] == blocks[inverse == inverse[i]].min() for i in range(len(blocks))])
        mod8 = blocks % 8
        xcd_map = {int(m): sorted(set(xcc[mod8 == m].tolist())) for m in range(8)}
        return {
            "span_us": round(float((end.max() - start.min()) * 0.01), 2),
            "start_skew_us": round(float((start.max() - start.min()) * 0.01), 2),
            "dur": dur, "per_wg": per_wg, "tile": tile, "counts": counts, "first": first,
            "tiles_once": bool(np.array_equal(np.sort(tile), np.arange(tiles))),
            "xcd_is_block_mod_8": all(len(v) == 1 for v in xcd_map.values()) and
                                  len({v[0] for v in xcd_map.values()}) == 8,
        }

    if args.clock_dump:
        np.save(args.clock_dump, np.stack(runs))  # [runs][workgroups][4] uint64, as written
    res = [analyse(r) for r in runs]
    med = sorted(res, key=lambda r: r["span_us"])[len(res) // 2]  # the run of median span
    q = lambda x, p: round(float(np.percentile(x, p)), 2) if len(x) else None  # noqa: E731
    dur, per_wg = med["dur"], med["per_wg"]
    stats = lambda x: {"n": int(len(x)), "min": q(x, 0), "median": q(x, 50), "p90": q(x, 90),  # noqa: E731
                       "max": q(x, 100)}
    order = np.argsort(-dur)[:8]
    print(json.dumps({
        "metric": "tile kernel per-workgroup clock (us, 100 MHz constant clock)",
        "config": {"workload": WORKLOADS[args.config], "tile": f"{th}x{tw}", "tiles": tiles, "workgroups": grid,
                   "fused_config": cfg},
        "runs": args.clock_runs, "launches_per_run": launches,
        "us_per_launch_back_to_back": round(statistics.median(launch_us), 2),
        "span_us": {"median_run": med["span_us"], "all_runs": [r["span_us"] for r in res]},
        "start_skew_us": med["start_skew_us"],
        "workgroup_us": stats(dur),
        "workgroup_us_alone_on_cu": stats(dur[per_wg == 1]),
        "workgroup_us_sharing_cu": stats(dur[per_wg >= 2]),
        "workgroup_us_sharing_cu_dispatched_first": stats(dur[(per_wg == 2) & med["first"]]),
        "workgroup_us_sharing_cu_dispatched_second": stats(dur[(per_wg == 2) & ~med["first"]]),
        "cus": {"one_workgroup": int(np.sum(med["counts"] == 1)), "two": int(np.sum(med["counts"] == 2)),
                "more": int(np.sum(med["counts"] > 2))},
        "slowest": [{"tile": int(med["tile"][i]), "us": round(float(dur[i]), 2), "sharing_cu": bool(per_wg[i] >= 2)}
                    for i in order],
        "tiles_once": all(r["tiles_once"] for r in res),
        "xcd_is_block_mod_8": all(r["xcd_is_block_mod_8"] for r in res),
        "bit_identical_with_clock_off": identical,
    }))
    return 0 if identical and all(r["tiles_once"] for r in res) else 1


def bench_gather(args) -> int:
    """The reference's gather phase alone at C2 (dcn_im2col_f16_dev: the modulated FP16
    im2col matrix [4096][1152] written to HBM, MetalShader.swift:299-381), the counterpart
    of the reference's gather-only timing (MetalRunner.swift:311-326). Algorithmic bytes:
    NCHW input, offsets and mask read once, the columns written once."""
    import numpy as np
    import torch

    from jasnamacos_amd import deform_conv as dc

    d = dc.generate_config_inputs(2, args.seed)
    s = d["shape"]
    dev = {k: torch.from_numpy(np.asarray(d[k], np.float32).astype(np.float16).view(np.int16)).cuda()
           for k in ("input", "offset", "mask")}
    ctx = dc.HipDeformConv(0)
    stream = torch.cuda.Stream()
    cols = torch.empty(s.batch * s.output_height * s.output_width * s.input_channels * s.kernel_area,
                       dtype=torch.int16, device="cuda")
    us = _graph_us(torch, stream, lambda st: ctx.im2col_f16_dev(s, dev["input"], dev["offset"], dev["mask"], cols,
                                                                 stream=st), args.steps, args.kernel_reps)
    c = s.counts()
    nbytes = 2 * (c["input"] + c["offset"] + c["mask"] + cols.numel())
    ctx.close()
    print(json.dumps({"metric": "DCNv2 gather phase (reference im2col) at C2", "value": us, "unit": "us/call",
                      "n_gpus": 1, "steps": args.steps, "higher_is_better": False, "dtype": "f16",
                      "data": "synthetic (the C2 benchmark distributions)",
                      "config": {"workload": "C2 gather: im2col_kernel 1x128x64x64, 16 dg -> [4096][1152] FP16"},
                      "algorithmic_bytes": nbytes, "achieved_gbs": nbytes / (us * 1e-6) / 1e9,
                      "hbm_frac": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}), flush=True)
    return 0


def seed_sweep(args) -> int:
    """--seed-sweep N: the bench of config 2, 3 or 5 at input seeds 0 .. N-1, each in a child
    process (this process never touches the GPU), without the CPU baseline or the cold
    calls. The seed changes the offset field and with it the tile kernel's windows, so the
    C3/C5 kernel times depend on it. Prints one JSON line: each seed's call and kernel
    times (and the exact sampler's kernel time for FP16) and their mean, min and max."""
    import subprocess

    if args.config not in (2, 3, 5) or args.spynet or args.seed_sweep < 1:
        print("--seed-sweep N (N >= 1) sweeps configs 2, 3 and 5", file=sys.stderr)
        return 2
    passthrough = ["--config", str(args.config), "--steps", str(args.steps), "--warmup", str(args.warmup),
                   "--kernel-reps", str(args.kernel_reps), "--dtype", args.dtype, "--no-cpu-baseline",
                   "--cold-calls", "0"]
    for flag in ("variant", "mt", "ks"):
        if getattr(args, flag):
            passthrough += [f"--{flag}", str(getattr(args, flag))]
    rows = []
    for seed in range(args.seed_sweep):
        r = subprocess.run([sys.executable, str(Path(__file__).resolve()), "--seed", str(seed), *passthrough],
                           capture_output=True, text=True)
        lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
        if r.returncode != 0 or not lines:
            print(f"seed {seed}: bench.py exited {r.returncode}\n{r.stderr[-2000:]}", file=sys.stderr)
            return r.returncode or 1
        d = json.loads(lines[-1])
        row = {"seed": seed, "us_per_call": round(d["ms_per_step"] * 1e3, 3), "kernel_us": round(d["kernel_us"], 3)}
        if d.get("exact_kernel_us"):
            row["exact_kernel_us"] = round(d["exact_kernel_us"], 3)
        rows.append(row)
        print(f"seed {seed}: {row}", file=sys.stderr, flush=True)

    def summary(key):
        v = [r[key] for r in rows if key in r]
        return {"mean": round(statistics.mean(v), 3), "min": min(v), "max": max(v)} if v else None

    print(json.dumps({"metric": "DCNv2 fwd us/call and fused kernel us over input seeds", "unit": "us",
                      "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": False,
                      "data": "synthetic (dcn_generate_config_inputs at each seed)",
                      "config": {"workload": WORKLOADS[args.config], "dtype": args.dtype,
                                 "seeds": list(range(args.seed_sweep))},
                      "per_seed": rows, "us_per_call": summary("us_per_call"), "kernel_us": summary("kernel_us"),
                      "exact_kernel_us": summary("exact_kernel_us")}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=2, choices=sorted(WORKLOADS))
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--spynet", action="store_true",
                    help="measure the SPyNet flow pair (the producer of the body's flows) instead of a config")
    ap.add_argument("--kernel-reps", type=int, default=5, help="repetitions of the fused-only timing")
    ap.add_argument("--cold-calls", type=int, default=20,
                    help="single calls timed after flushing the caches with a 512 MB write (0: skip)")
    ap.add_argument("--variant", type=int, default=0,
                    help="pin the fused variant (0 = the library's automatic choice)")
    ap.add_argument("--mt", type=int, default=0, help="pin the fused config's mt (0 = automatic)")
    ap.add_argument("--ks", type=int, default=0, help="pin the fused config's ks (0 = automatic)")
    ap.add_argument("--frames-only", action="store_true",
                    help="config 4: time the per-frame graphs only (no clip, no 16-tile step)")
    ap.add_argument("--dtype", choices=("f16", "bf16"), default="f16",
                    help="configs 2, 3, 5: FP16 storage (the reference's) or BF16 storage (the BF16 "
                         "fused path)")
    ap.add_argument("--launch-floor", action="store_true",
                    help="time empty kernels of the C2/C3/C5 kernels' launch shapes in a hipGraph")
    ap.add_argument("--gather", action="store_true",
                    help="time the reference's gather phase alone at C2 (im2col columns to HBM)")
    ap.add_argument("--tile-clock", action="store_true",
                    help="configs 3, 5: per-workgroup clock stamps of the tile kernel (the spread of "
                         "workgroup times, CU sharing, the slowest tiles)")
    ap.add_argument("--clock-runs", type=int, default=5, help="--tile-clock: runs of 10 launches")
    ap.add_argument("--clock-dump", default="",
                    help="--tile-clock: also save every run's raw records to this .npy file")
    ap.add_argument("--seed-sweep", type=int, default=0,
                    help="configs 2, 3, 5: run the bench at input seeds 0 .. N-1 (one child process "
                         "each) and print the per-seed and mean/min/max kernel and call times")
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="after timing, run three device copies of this many MiB (the known-size "
                         "reference kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (independent tiles "
              "would shard with no exchange). Run with --gpus 1.", file=sys.stderr)
        return 2
    if args.steps < 1:
        print("--steps must be >= 1", file=sys.stderr)
        return 2
    if args.seed_sweep:
        return seed_sweep(args)
    bf16 = args.dtype == "bf16"
    if bf16 and (args.spynet or args.config in (1, 4) or args.variant or args.mt or args.ks):
        print("--dtype bf16 measures the BF16 fused forward of configs 2, 3 and 5 (its automatic "
              "kernel choice)", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from jasnamacos_amd import deform_conv as dc

    torch.cuda.set_device(0)
    if args.launch_floor:
        return bench_launch_floor(args)
    if args.tile_clock:
        return bench_tile_clock(args)
    if args.gather:
        rc = bench_gather(args)
        if args.calibration_copy_mib > 0:
            calibration_copies(args.calibration_copy_mib)
        return rc
    if args.spynet:
        return bench_spynet(args)
    if args.config == 4:
        return bench_body(args)
    d = dc.generate_config_inputs(args.config, args.seed)
    s = d["shape"]
    f32 = args.config == 1
    keys = ("input", "offset", "mask", "weight", "bias")
    if f32:
        h = {k: np.asarray(d[k], np.float32) for k in keys}
        dev = {k: torch.from_numpy(h[k]).cuda() for k in keys}
    elif bf16:
        h = {k: dc.f32_to_bf16_bits(d[k]) for k in keys}
        dev = {k: torch.from_numpy(h[k].view(np.int16)).cuda() for k in keys}
    else:
        h = {k: np.asarray(d[k], np.float32).astype(np.float16) for k in keys}
        dev = {k: torch.from_numpy(h[k].view(np.int16)).cuda() for k in keys}
    ctx = dc.HipDeformConv(0)
    stream = torch.cuda.Stream()
    packed = None
    if f32:
        fused_cfg = None
        out = torch.empty(s.output_count, dtype=torch.float32, device="cuda")

        def step(cur):
            ctx.forward_f32_dev(s, dev["input"], dev["offset"], dev["mask"], dev["weight"], dev["bias"], out,
                                stream=cur)

        fused_only = step  # one kernel per call
    elif bf16:
        packed = ctx.prepack_bf16_dev(s, dev["weight"], dev["bias"])
        ctx.reserve(s)
        # The BF16 forward's fixed choice: 16-pixel tiles on 12 waves (the narrow kernel) up
        # to 1024 tiles of 32 pixels; above, LDS windows over 4 x 32 tiles on 4 waves for the
        # shapes the window kernel takes (all of C3 and C5), else the register variant.
        many = (s.batch * s.output_height * s.output_width + 31) // 32 > 1024
        window_ok = (s.groups == 1 and s.kernel_height == 3 and s.kernel_width == 3 and
                     s.input_channels == 8 * s.offset_groups and s.output_channels % 32 == 0 and
                     s.output_channels <= 128)
        fused_cfg = ({"variant": 5, "mt": 1, "ks": 12, "sampler": "bf16"} if not many
                     else {"variant": 3, "mt": 4, "ks": 4, "sampler": "bf16"} if window_ok
                     else {"variant": 1, "mt": 2, "ks": 4, "sampler": "bf16"})
        out = torch.empty(s.output_count, dtype=torch.int16, device="cuda")
        cb8 = torch.empty(ctx.cb8_count(s), dtype=torch.int16, device="cuda")

        def step(cur):
            ctx.forward_bf16_prepacked_dev(s, dev["input"], dev["offset"], dev["mask"], packed, out, stream=cur)

        def fused_only(cur):
            ctx.forward_bf16_prepacked_cb8_dev(s, cb8, dev["offset"], dev["mask"], packed, out, stream=cur)
    else:
        packed = ctx.prepack_dev(s, dev["weight"], dev["bias"])
        ctx.reserve(s)
        if args.variant or args.mt or args.ks:
            ctx.set_fused_config(args.mt, args.ks, -1, args.variant)
        fused_cfg = ctx.get_fused_config(s)
        out = torch.empty(s.output_count, dtype=torch.int16, device="cuda")
        cb8 = torch.empty(ctx.cb8_count(s), dtype=torch.int16, device="cuda")

        def step(cur):
            ctx.forward_f16_prepacked_dev(s, dev["input"], dev["offset"], dev["mask"], packed, out, stream=cur)

        def fused_only(cur):
            ctx.forward_f16_prepacked_cb8_dev(s, cb8, dev["offset"], dev["mask"], packed, out, stream=cur)

    with torch.cuda.stream(stream):
        for _ in range(max(args.warmup, 1)):
            step(stream)
        if not f32:
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

    def time_graph(graph) -> float:
        """Median over kernel_reps replays of `graph` (args.steps launches), us per launch."""
        reps = []
        for _ in range(args.kernel_reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(stream):
                a.record(stream)
                graph.replay()
                b.record(stream)
            torch.cuda.synchronize()
            reps.append(a.elapsed_time(b) * 1e3 / args.steps)
        return statistics.median(reps)

    # What was timed: the output of the last timed call (checked against the oracle in the
    # cpu_baseline leg below).
    if f32:
        res = out.cpu().numpy()
    elif bf16:
        res = dc.bf16_bits_to_f32(out.cpu().numpy().view(np.uint16))
    else:
        res = out.cpu().numpy().view(np.float16).astype(np.float32)

    # ---- the reference's sampler arithmetic (FP16 storage): half(FP32 bilinear x mask),
    # MetalShader.swift:371-379, on the kernel the library picks for it, timed like the
    # default; its output is checked in the cpu_baseline leg too ------------------------
    exact = None
    if not f32 and not bf16:
        ctx.set_fused_config(args.mt, args.ks, dc.SAMPLER_EXACT, args.variant)
        exact_cfg = ctx.get_fused_config(s)
        with torch.cuda.stream(stream):
            fused_only(stream)
        torch.cuda.synchronize()
        g_exact = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_exact, stream=stream):
            cur = torch.cuda.current_stream()
            for _ in range(args.steps):
                fused_only(cur)
        g_exact_step = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_exact_step, stream=stream):
            cur = torch.cuda.current_stream()
            for _ in range(args.steps):
                step(cur)
        with torch.cuda.stream(stream):
            g_exact.replay()
            g_exact_step.replay()
        torch.cuda.synchronize()
        exact = {"sampler": "exact", "fused_config": exact_cfg,
                 "kernel": KERNEL_NAMES.get(exact_cfg["variant"], "fused_kernel"),
                 "kernel_us": time_graph(g_exact), "us_per_call": time_graph(g_exact_step)}
        exact["hbm_frac"] = algorithmic_bytes(s) / (exact["kernel_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS
        exact_res = out.cpu().numpy().view(np.float16).astype(np.float32)
        del g_exact, g_exact_step
        ctx.set_fused_config(args.mt, args.ks, -1, args.variant)

    # ---- cold cache: a 512 MB scratch write (twice the 256 MB MALL) before each call --
    cold_us = warm_single_us = cold_kernel_us = warm_kernel_us = None
    if args.cold_calls > 0:
        scratch = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")

        def single_calls(fn, flush: bool) -> float:
            samples = []
            with torch.cuda.stream(stream):
                for i in range(args.cold_calls):
                    if flush:
                        scratch.fill_(i & 0xFF)
                    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    a.record(stream)
                    fn(stream)
                    b.record(stream)
                    b.synchronize()
                    samples.append(a.elapsed_time(b) * 1e3)
            torch.cuda.synchronize()
            return statistics.median(samples)

        cold_us = single_calls(step, True)
        warm_single_us = single_calls(step, False)
        if not f32:
            # The fused kernel alone on the CB8 input, one eager launch each.
            cold_kernel_us = single_calls(fused_only, True)
            warm_kernel_us = single_calls(fused_only, False)
        del scratch

    if args.calibration_copy_mib > 0:
        calibration_copies(args.calibration_copy_mib)

    finite = bool(np.all(np.isfinite(res)))

    nbytes = algorithmic_bytes(s, elem=4 if f32 else 2)
    flops = s.flops
    workload_name = {1: "dcn_c1_fp32", 2: "dcn_c2_fp16", 3: "dcn_c3_fp16", 5: "dcn_c5_fp16"}[args.config]
    if bf16:
        workload_name = workload_name.replace("fp16", "bf16")
    kernel_name = KERNEL_NAMES[0] if f32 else KERNEL_NAMES.get(fused_cfg["variant"], "fused_kernel")
    traffic = read_traffic(f"{kernel_name}_{workload_name}")
    if f32:
        # FP32 arithmetic: priced against the FP32 matrix peak (the HBM bytes take
        # 10.5 MB / 8 TB/s = 1.3 us, below the 3.8 us of the FLOPs).
        achieved = flops / (k_us * 1e-6) / 1e12
        roofline = {"bound": "mfma", "achieved": achieved, "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": achieved / FP32_PEAK_TFLOPS, "traffic": traffic,
                    "kernel": kernel_name + " (FP32, samples shared by 64 output channels, oracle summation order)",
                    "traffic_source": f"profiles/{kernel_name}_{workload_name}.md" if traffic else None,
                    "algorithmic_bytes_per_launch": nbytes,
                    "hbm_frac": nbytes / (k_us * 1e-6) / 1e9 / HBM_PEAK_GBS}
    else:
        achieved = nbytes / (k_us * 1e-6) / 1e9
        roofline = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                    "kernel": kernel_name + " (sampler + MFMA GEMM)",
                    "traffic_source": f"profiles/{kernel_name}_{workload_name}.md" if traffic else None,
                    "algorithmic_bytes_per_launch": nbytes,
                    "mfma_frac": flops / (k_us * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS}
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
        "dtype": "f32" if f32 else args.dtype,
        "data": "synthetic (seeded SplitMix64/Box-Muller inputs of the benchmark distributions; random weights)",
        "config": {
            "workload": WORKLOADS[args.config].replace("FP16", "BF16") if bf16 else WORKLOADS[args.config],
            "batch": s.batch, "in_channels": s.input_channels, "height": s.input_height, "width": s.input_width,
            "out_channels": s.output_channels, "kernel": [s.kernel_height, s.kernel_width],
            "deformable_groups": s.offset_groups, "fused_config": fused_cfg,
            "sampler": "bf16" if bf16 else None if f32 else ("exact" if fused_cfg["sampler"] == dc.SAMPLER_EXACT
                                                              else "fast"),
            "timing": f"{args.steps} calls captured in one hipGraph, one replay timed with HIP events",
            # samples whose four corners all lie outside the input (they contribute zero)
            "sample_oob_fraction": round(dc.out_of_bounds_fraction(
                s, dc.bf16_bits_to_f32(h["offset"]) if bf16 else np.asarray(h["offset"], np.float32)), 4),
        },
        "tflops": flops / (us_per_call * 1e-6) / 1e12,
        "step_hbm_frac": nbytes / (us_per_call * 1e-6) / 1e9 / HBM_PEAK_GBS,
        "step_mfma_frac": flops / (us_per_call * 1e-6) / 1e12 / (FP32_PEAK_TFLOPS if f32 else MFMA_F16_PEAK_TFLOPS),
        "kernel_us": k_us,
        "cold_us_per_call": cold_us,
        "warm_single_us_per_call": warm_single_us,
        "cold_kernel_us": cold_kernel_us,
        "warm_single_kernel_us": warm_kernel_us,
        "cold_note": ("medians of single eager calls (whole call; *_kernel_us: the fused kernel alone on "
                      "the CB8 input) timed with HIP events on the call's stream (launch latency "
                      "included), cold = each after a 512 MB scratch write (twice the MALL), warm = "
                      "back to back") if cold_us is not None else None,
        "kernel_tflops": flops / (k_us * 1e-6) / 1e12,
        "wall_ms_timed_region": wall_ms,
        "output_finite": finite,
        "roofline": roofline,
        "cpu_baseline": None,
    }
    if args.config == 3 and not bf16:
        line["per_gpu_share"] = bench_share(args, ctx, dc, d, dev)
    line["exact_sampler"] = exact
    line["exact_kernel_us"] = exact["kernel_us"] if exact else None
    line["timed_output_check"] = None
    if not args.no_cpu_baseline:
        # BF16 keeps 3 fewer significant bits than FP16: bars 8x the FP16 ones.
        widened = {k: dc.bf16_bits_to_f32(h[k]) if bf16 else h[k].astype(np.float32) for k in keys}
        outputs = {"timed": res, "exact": exact_res} if exact else res
        line["cpu_baseline"], checks = cpu_baseline(
            args.config, s, widened, outputs,
            bars=(8 * MAX_ABS_F16, 8 * MEAN_ABS_F16) if bf16 else (MAX_ABS_F16, MEAN_ABS_F16))
        if exact:
            line["timed_output_check"] = checks["timed"]
            exact["output_check"] = checks["exact"]
        else:
            line["timed_output_check"] = checks
    if packed is not None:
        packed.free()
    ctx.close()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
