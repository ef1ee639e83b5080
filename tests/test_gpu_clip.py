"""GPU tests of the four-branch propagation clip (dcn_clip).

Bars:
  * orchestration: the clip equals the same steps driven one at a time from the
    TemporalSchedule through single bodies, bit for bit (same kernels, same inputs);
  * semantics, teacher-forced: every step's output (first steps without alignment
    included) against the oracle chain run on that step's GPU inputs, within the one-step
    FP16 tolerance (max 2e-2, mean 1e-3), so errors do not compound over the recurrence;
  * one captured graph for the whole clip replays bit-identically to the eager run;
  * chunked recurrences equal independent clips over the chunk ranges;
  * the recovery ladder (dcn_clip_run_with_fallback_dev): a finite clip runs whole; NaN
    motion falls through to the zero-motion triplets, whose kept middle frames equal
    3-frame clips run alone; overflowing weights end in finite-input passthrough;
    non-finite features end in commandFailed.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import body_reference as br

pytestmark = pytest.mark.gpu


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(np.asarray(a, np.float16)).view(np.int16)).cuda()


def host(t):
    return t.cpu().numpy().view(np.float16)


@pytest.fixture(scope="module")
def torch():
    import torch as t

    return t


def _clip_case(torch, frames, h, w, blocks, seed, flow_px=3.0):
    rng = np.random.default_rng(seed)
    weights = [br.body_weights(rng, b, blocks) for b in range(4)]
    plane = h * w
    x = {
        "spatial": br.f16(rng.standard_normal(frames * 64 * plane)),
        "bflows": br.f16(rng.uniform(-flow_px, flow_px, max(frames - 1, 1) * 2 * plane)),
        "fflows": br.f16(rng.uniform(-flow_px, flow_px, max(frames - 1, 1) * 2 * plane)),
    }
    wd = [{k: dev(torch, v) for k, v in wb.items()} for wb in weights]
    xd = {k: dev(torch, v) for k, v in x.items()}
    return weights, wd, x, xd


def _run_clip(torch, ctx, wd, xd, frames, h, w, blocks, chunk=0):
    clip = ctx.clip(h, w, frames, wd, blocks=blocks)
    prop = torch.zeros(4 * frames * 64 * h * w, dtype=torch.int16, device="cuda")
    clip.run_dev(xd["spatial"], xd["bflows"], xd["fflows"], prop, chunk)
    torch.cuda.synchronize()
    out = host(prop).copy().reshape(4, frames, 64 * h * w)
    clip.free()
    return out


def test_clip_matches_schedule_driven_bodies(gpu_ctx, dcn, torch):
    frames, h, w, blocks = 4, 16, 24, 2
    weights, wd, x, xd = _clip_case(torch, frames, h, w, blocks, 3)
    log("case: clip vs schedule-driven bodies", frames, h, w)
    got = _run_clip(torch, gpu_ctx, wd, xd, frames, h, w, blocks)
    plane = h * w
    bodies = [gpu_ctx.body(h, w, wd[b], branch=b, blocks=blocks) for b in range(4)]
    prop = torch.zeros(4, frames, 64 * plane, dtype=torch.int16, device="cuda")
    spatial = xd["spatial"].view(frames, 64 * plane)
    flows = {"backward": xd["bflows"].view(-1, 2 * plane), "forward": xd["fflows"].view(-1, 2 * plane)}
    zero = torch.zeros(64 * plane, dtype=torch.int16, device="cuda")
    flow2 = torch.zeros(2 * plane, dtype=torch.int16, device="cuda")
    schedule = dcn.TemporalSchedule(frames)
    for s in schedule.steps:
        b = s.branch.branch_index
        prefix = [prop[i, s.frame_index] for i in range(b)] or None
        if s.position == 0:
            bodies[b].initial_step_dev(spatial[s.frame_index], prop[b, s.frame_index], prefix=prefix)
            continue
        steps = [t for t in schedule.steps if t.branch == s.branch]
        prev = steps[s.position - 1]
        f = flows[s.branch.direction]
        prev_flow = f[prev.flow_index] if s.position >= 2 else f[s.flow_index]
        feat_n2 = prop[b, s.second_order_frame_index] if s.second_order_frame_index is not None else zero
        bodies[b].step_dev(spatial[s.frame_index], f[s.flow_index], prev_flow, prop[b, prev.frame_index], feat_n2,
                           flow2, prop[b, s.frame_index], has_second_order=s.position >= 2, prefix=prefix)
    torch.cuda.synchronize()
    ref = host(prop).copy()
    for body in bodies:
        body.free()
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    assert np.all(np.isfinite(got.astype(np.float32)))


def test_clip_steps_match_oracle_teacher_forced(gpu_ctx, dcn, torch):
    frames, h, w, blocks = 4, 12, 20, 1
    weights, wd, x, xd = _clip_case(torch, frames, h, w, blocks, 5)
    log("case: clip teacher-forced oracle", frames, h, w)
    got = _run_clip(torch, gpu_ctx, wd, xd, frames, h, w, blocks)
    plane = h * w
    spatial = x["spatial"].reshape(frames, 64 * plane)
    flows = {"backward": x["bflows"].reshape(-1, 2 * plane), "forward": x["fflows"].reshape(-1, 2 * plane)}
    schedule = dcn.TemporalSchedule(frames)
    worst = 0.0
    for s in schedule.steps:
        b = s.branch.branch_index
        prefix = [got[i, s.frame_index] for i in range(b)]
        out = got[b, s.frame_index].astype(np.float64)
        if s.position == 0:
            ref = br.body_initial_step(weights[b], spatial[s.frame_index], prefix, h, w, blocks).astype(np.float64)
            e = np.abs(out - ref)
            assert e.max() <= 2e-2 and e.mean() <= 1e-3, (s, e.max(), e.mean())
            continue
        steps = [t for t in schedule.steps if t.branch == s.branch]
        prev = steps[s.position - 1]
        f = flows[s.branch.direction]
        step_in = {
            "feat_current": spatial[s.frame_index],
            "flow1": f[s.flow_index],
            "prev_flow": f[prev.flow_index] if s.position >= 2 else f[s.flow_index],
            "feat_prop": got[b, prev.frame_index],
            "feat_n2": got[b, s.second_order_frame_index] if s.second_order_frame_index is not None
            else np.zeros(64 * plane, np.float16),
            "prefix": prefix,
        }
        _, ref, _ = br.body_step(weights[b], step_in, h, w, blocks, s.position >= 2)
        e = np.abs(out - ref.astype(np.float64))
        worst = max(worst, e.max())
        assert e.max() <= 2e-2 and e.mean() <= 1e-3, (s, e.max(), e.mean())
    log(f"  worst step max err {worst:.3e}")


def test_clip_graph_replays_match_eager(gpu_ctx, torch):
    frames, h, w, blocks = 5, 16, 16, 1
    weights, wd, x, xd = _clip_case(torch, frames, h, w, blocks, 7)
    log("case: clip graph replay", frames, h, w)
    eager = _run_clip(torch, gpu_ctx, wd, xd, frames, h, w, blocks)
    clip = gpu_ctx.clip(h, w, frames, wd, blocks=blocks)
    prop = torch.zeros(4 * frames * 64 * h * w, dtype=torch.int16, device="cuda")
    graph = clip.capture(xd["spatial"], xd["bflows"], xd["fflows"], prop)
    scratch = torch.zeros_like(prop)
    for i in range(3):
        prop.zero_()
        torch.cuda.synchronize()
        graph.launch()
        torch.cuda.synchronize()
        assert np.array_equal(host(prop).view(np.uint16), eager.reshape(-1).view(np.uint16)), i
        clip.run_dev(xd["spatial"], xd["bflows"], xd["fflows"], scratch)  # eager work between replays
        torch.cuda.synchronize()
    graph.free()
    clip.free()


def test_clip_chunks_equal_independent_clips(gpu_ctx, dcn, torch):
    frames, h, w, blocks = 7, 12, 16, 1
    weights, wd, x, xd = _clip_case(torch, frames, h, w, blocks, 9)
    log("case: chunked clip", frames, h, w)
    got = _run_clip(torch, gpu_ctx, wd, xd, frames, h, w, blocks, chunk=3)
    plane = h * w
    ranges = dcn.temporal_chunk_ranges(frames, 3)
    assert ranges == [range(0, 4), range(4, 7)]
    for r in ranges:
        n = len(r)
        sub = {
            "spatial": dev(torch, x["spatial"].reshape(frames, -1)[r.start:r.stop]),
            "bflows": dev(torch, x["bflows"].reshape(frames - 1, -1)[r.start:r.stop - 1]),
            "fflows": dev(torch, x["fflows"].reshape(frames - 1, -1)[r.start:r.stop - 1]),
        }
        ref = _run_clip(torch, gpu_ctx, wd, sub, n, h, w, blocks)
        assert np.array_equal(got[:, r.start:r.stop].view(np.uint16), ref.view(np.uint16)), r
    assert got.shape == (4, frames, 64 * plane)


def test_clip_tiles_equal_single_tile_clips(gpu_ctx, torch):
    """A clip over 2 tiles ([T][tiles][...] tensors) == one clip per tile, bit for bit."""
    frames, h, w, blocks, tiles = 4, 16, 24, 2, 2
    cases = [_clip_case(torch, frames, h, w, blocks, 90 + t) for t in range(tiles)]
    wd = cases[0][1]
    plane = h * w
    log("case: clip tiles", frames, h, w, tiles)

    def interleave(key, per_frame):
        arrs = [c[2][key].reshape(-1, per_frame) for c in cases]
        return dev(torch, np.stack(arrs, axis=1).ravel())

    spatial = interleave("spatial", 64 * plane)
    bflows = interleave("bflows", 2 * plane)
    fflows = interleave("fflows", 2 * plane)
    clip = gpu_ctx.clip(h, w, frames, wd, blocks=blocks, tiles=tiles)
    prop = torch.zeros(4 * frames * tiles * 64 * plane, dtype=torch.int16, device="cuda")
    clip.run_dev(spatial, bflows, fflows, prop)
    torch.cuda.synchronize()
    got = host(prop).reshape(4, frames, tiles, 64 * plane)
    clip.free()
    for t, c in enumerate(cases):
        want = _run_clip(torch, gpu_ctx, wd, c[3], frames, h, w, blocks)
        assert np.array_equal(got[:, :, t].view(np.uint16), want.view(np.uint16)), t


def _ladder(torch, gpu_ctx, wd, xd, frames, h, w, blocks):
    clip = gpu_ctx.clip(h, w, frames, wd, blocks=blocks)
    prop = torch.zeros(4 * frames * 64 * h * w, dtype=torch.int16, device="cuda")
    msgs = []
    try:
        rung = clip.run_with_fallback_dev(xd["spatial"], xd["bflows"], xd["fflows"], prop, report=msgs.append)
        torch.cuda.synchronize()
        return rung, host(prop).copy().reshape(4, frames, 64 * h * w), msgs
    finally:
        clip.free()


def test_clip_ladder_full_window_when_finite(gpu_ctx, dcn, torch):
    frames, h, w, blocks = 6, 8, 8, 1
    weights, wd, x, xd = _clip_case(torch, frames, h, w, blocks, 12)
    log("case: ladder, finite clip")
    rung, got, msgs = _ladder(torch, gpu_ctx, wd, xd, frames, h, w, blocks)
    assert rung == 0 and msgs == []
    want = _run_clip(torch, gpu_ctx, wd, xd, frames, h, w, blocks)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_clip_ladder_recovers_with_zero_motion_triplets(gpu_ctx, dcn, torch):
    """NaN motion into frame 1 (backward flow 1) poisons the whole clip and every chunking
    (frame 1 never starts a chunk of 6 frames); each frame alone as [t, t, t] with zero
    flows does not. Every branch keeps the triplet's middle feat_prop, bit for bit."""
    frames, h, w, blocks = 6, 8, 8, 1
    weights, wd, x, xd = _clip_case(torch, frames, h, w, blocks, 13)
    plane = h * w
    bflows = x["bflows"].copy()
    bflows[1 * 2 * plane:2 * 2 * plane] = np.float16(np.nan)
    xd["bflows"] = dev(torch, bflows)
    log("case: ladder, NaN motion -> zero-motion triplets")
    rung, got, msgs = _ladder(torch, gpu_ctx, wd, xd, frames, h, w, blocks)
    assert rung == dcn.RECOVERED_TRIPLETS, msgs
    assert [m.split(" (")[0] for m in msgs] == [
        "clip failed its full temporal window", "clip also failed with 5-frame chunks",
        "clip also failed with 3-frame chunks", "clip recovered with independent zero-motion frame triplets"]
    zero = np.zeros(2 * 2 * plane, np.float16)
    for t in range(frames):
        f = x["spatial"][t * 64 * plane:(t + 1) * 64 * plane]
        trip = {"spatial": dev(torch, np.tile(f, 3)), "bflows": dev(torch, zero), "fflows": dev(torch, zero)}
        want = _run_clip(torch, gpu_ctx, wd, trip, 3, h, w, blocks)
        assert np.array_equal(got[:, t].view(np.uint16), want[:, 1].view(np.uint16)), t


def test_clip_ladder_passes_finite_input_through(gpu_ctx, dcn, torch):
    """Weights ~N(0, 20) overflow FP16 within two convs at every rung; the features are
    finite, so every branch's output is the spatial input, unchanged."""
    frames, h, w, blocks = 4, 8, 8, 1
    rng = np.random.default_rng(14)
    weights = [br.body_weights(rng, b, blocks, std=20.0) for b in range(4)]
    wd = [{k: dev(torch, v) for k, v in wb.items()} for wb in weights]
    plane = h * w
    x = {"spatial": br.f16(rng.standard_normal(frames * 64 * plane)),
         "bflows": br.f16(rng.uniform(-2, 2, (frames - 1) * 2 * plane)),
         "fflows": br.f16(rng.uniform(-2, 2, (frames - 1) * 2 * plane))}
    xd = {k: dev(torch, v) for k, v in x.items()}
    log("case: ladder, overflowing weights -> passthrough")
    rung, got, msgs = _ladder(torch, gpu_ctx, wd, xd, frames, h, w, blocks)
    assert rung == dcn.RECOVERED_PASSTHROUGH, msgs
    assert msgs[-1].startswith("WARNING: clip is using finite input passthrough")
    for b in range(4):
        assert np.array_equal(got[b].ravel().view(np.uint16), x["spatial"].view(np.uint16)), b


def test_clip_nonfinite_input_ends_the_ladder_in_command_failed(gpu_ctx, dcn, torch):
    frames, h, w, blocks = 6, 8, 8, 1
    weights, wd, x, xd = _clip_case(torch, frames, h, w, blocks, 11)
    spatial = x["spatial"].copy()
    spatial[5] = np.float16(np.inf)
    xd["spatial"] = dev(torch, spatial)
    log("case: ladder, non-finite input -> commandFailed")
    with pytest.raises(dcn.DeformConvError) as e:
        _ladder(torch, gpu_ctx, wd, xd, frames, h, w, blocks)
    assert e.value.status == dcn.COMMAND_FAILED
    assert "non-finite input features" in str(e.value)


def test_clip_free_running_c4_size_matches_oracle_chain(gpu_ctx, dcn, torch):
    """The four-branch clip at config C4's size (64 x 64, 5 blocks) over 8 frames, free
    running: the GPU clip runs once on its own outputs, and the oracle chain runs the whole
    TemporalSchedule the same way on the CPU (each step's feat_prop, feat_n2 and prefix are
    the oracle's own earlier outputs), so any compounding through the recurrence or across
    branches (branches 1-3 read the earlier branches' outputs, 192-320 backbone input
    channels) shows. Smooth synthetic flows of up to +-4 px (generate_body_inputs).
    Per-step max / mean absolute error is logged; each step must stay within the one-step
    FP16 bars (max 2e-2, mean 1e-3)."""
    frames, h, w, blocks = 8, 64, 64, 5
    plane = h * w
    gens = [dcn.generate_body_inputs(h, w, frames, b, blocks, seed=40 + b) for b in range(4)]
    weights = [g["weights"] for g in gens]
    spatial = gens[0]["feats"].reshape(frames, 64 * plane)
    bflows = gens[1]["flows"].reshape(frames, 2 * plane)[:frames - 1]
    fflows = gens[2]["flows"].reshape(frames, 2 * plane)[:frames - 1]
    wd = [{k: dev(torch, v) for k, v in wb.items()} for wb in weights]
    xd = {"spatial": dev(torch, spatial.ravel()), "bflows": dev(torch, bflows.ravel()),
          "fflows": dev(torch, fflows.ravel())}
    log("case: free-running four-branch clip", frames, h, w, "blocks", blocks)
    got = _run_clip(torch, gpu_ctx, wd, xd, frames, h, w, blocks).astype(np.float64)
    assert np.all(np.isfinite(got))

    flows = {"backward": bflows, "forward": fflows}
    zero = np.zeros(64 * plane, np.float16)
    ref = np.zeros((4, frames, 64 * plane), np.float16)
    schedule = dcn.TemporalSchedule(frames)
    worst = (0.0, 0.0)
    for n, s in enumerate(schedule.steps):
        b = s.branch.branch_index
        prefix = [ref[i, s.frame_index] for i in range(b)]
        if s.position == 0:
            ref[b, s.frame_index] = br.body_initial_step(weights[b], spatial[s.frame_index], prefix, h, w, blocks)
        else:
            steps = [t for t in schedule.steps if t.branch == s.branch]
            prev = steps[s.position - 1]
            f = flows[s.branch.direction]
            x = {"feat_current": spatial[s.frame_index], "flow1": f[s.flow_index],
                 "prev_flow": f[prev.flow_index] if s.position >= 2 else f[s.flow_index],
                 "feat_prop": ref[b, prev.frame_index],
                 "feat_n2": ref[b, s.second_order_frame_index] if s.second_order_frame_index is not None else zero,
                 "prefix": prefix}
            _, ref[b, s.frame_index], _ = br.body_step(weights[b], x, h, w, blocks, s.position >= 2)
        e = np.abs(got[b, s.frame_index] - ref[b, s.frame_index].astype(np.float64))
        log(f"  step {n:2d} branch {b} frame {s.frame_index}: max {e.max():.3e} mean {e.mean():.3e}")
        worst = (max(worst[0], e.max()), max(worst[1], e.mean()))
        assert e.max() <= 2e-2 and e.mean() <= 1e-3, (n, b, s.frame_index, e.max(), e.mean())
    log(f"  worst over {len(schedule.steps)} steps: max {worst[0]:.3e} mean {worst[1]:.3e}")
