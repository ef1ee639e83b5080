"""GPU parity of SPyNet flow estimation against the CPU oracle chain.

Bars:
  * bicubic quarter downsample and the pyramid: bit-identical to the oracle (same FP32
    expression order);
  * the six-level flow: within 2e-2 * max(1, |flow|max) max and 1e-3 * max(1, |flow|max)
    mean of the oracle's FP16 chain (the conv sums are ordered differently and each of the
    30 layers rounds to FP16);
  * the reverse direction of a pair equals a single call with the frames swapped, and the
    forward image of a pair equals the single-direction call, bit for bit;
  * a captured graph replays bit-identically to the eager call.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import spynet_reference as sr

pytestmark = pytest.mark.gpu


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as t

    return t


def dev(torch, a):
    return torch.from_numpy(np.array(a, np.float16).view(np.int16)).cuda()


def host(t):
    return t.cpu().numpy().view(np.float16)


@pytest.mark.parametrize("c,h,w", [(3, 256, 256), (3, 36, 20), (5, 4, 8)])
def test_bicubic_quarter_bit_exact(gpu_ctx, oracle, torch, c, h, w):
    rng = np.random.default_rng(h + w)
    x = sr.f16(rng.random(c * h * w) * 2 - 0.5)
    log("case: bicubic", c, h, w)
    out = torch.zeros(c * (h // 4) * (w // 4), dtype=torch.int16, device="cuda")
    gpu_ctx.bicubic_quarter_f16_dev(c, h, w, dev(torch, x), out)
    torch.cuda.synchronize()
    assert np.array_equal(host(out).view(np.uint16), oracle.bicubic_quarter_f16(c, h, w, x).view(np.uint16))


def test_bicubic_rejects_bad_sizes(gpu_ctx, dcn, torch):
    buf = torch.zeros(64, dtype=torch.int16, device="cuda")
    with pytest.raises(dcn.DeformConvError) as e:
        gpu_ctx.bicubic_quarter_f16_dev(1, 6, 8, buf, buf)
    assert e.value.status == dcn.INVALID_SHAPE


@pytest.mark.parametrize("h,w,offset", [(64, 64, 0), (32, 96, 0), (64, 64, 3)])
def test_pyramid_bit_exact(gpu_ctx, oracle, torch, h, w, offset):
    """Both load paths (16-byte rows; scalar for a frame that is not 16-byte aligned)."""
    frame = sr.smooth_frame(np.random.default_rng(h + offset), h, w)
    log("case: pyramid", h, w, offset)
    buf = dev(torch, np.concatenate([np.zeros(offset, np.float16), frame]))
    want = np.concatenate(oracle.spynet_pyramid_f16(h, w, 6, frame))
    out = torch.zeros(want.size, dtype=torch.int16, device="cuda")
    gpu_ctx.spynet_pyramid_f16_dev(h, w, buf[offset:], out)
    torch.cuda.synchronize()
    assert np.array_equal(host(out).view(np.uint16), want.view(np.uint16))


def _spynet(torch, gpu_ctx, h, w, seed):
    rng = np.random.default_rng(seed)
    weights = sr.spynet_weights(rng)
    spy = gpu_ctx.spynet(h, w, {k: dev(torch, v) for k, v in weights.items()})
    ref = sr.smooth_frame(rng, h, w)
    sup = sr.smooth_frame(rng, h, w, shift=(1.5, -2.0))
    return weights, spy, ref, sup


@pytest.mark.parametrize("h,w", [(64, 64), (32, 96)])
def test_spynet_pair_matches_oracle_chain(gpu_ctx, torch, h, w):
    weights, spy, ref, sup = _spynet(torch, gpu_ctx, h, w, 20 + w)
    log("case: spynet pair", h, w)
    flow = torch.zeros(2 * 2 * h * w, dtype=torch.int16, device="cuda")
    spy.flow_dev(dev(torch, ref), dev(torch, sup), flow, both_directions=True)
    torch.cuda.synchronize()
    got = host(flow).astype(np.float64).reshape(2, -1)
    for i, (a, b) in enumerate(((ref, sup), (sup, ref))):
        want = sr.spynet_flow(weights, a, b, h, w).astype(np.float64)
        scale = max(1.0, np.abs(want).max())
        err = np.abs(got[i] - want)
        log(f"direction {i}: |flow| max {np.abs(want).max():.3f}, err max {err.max():.3e} mean {err.mean():.3e}")
        assert err.max() <= 2e-2 * scale and err.mean() <= 1e-3 * scale
    spy.free()


def test_spynet_directions_bit_consistent(gpu_ctx, torch):
    h = w = 64
    _, spy, ref, sup = _spynet(torch, gpu_ctx, h, w, 31)
    r, s = dev(torch, ref), dev(torch, sup)
    log("case: spynet direction consistency")
    pair = torch.zeros(4 * h * w, dtype=torch.int16, device="cuda")
    one = torch.zeros(2 * h * w, dtype=torch.int16, device="cuda")
    rev = torch.zeros(2 * h * w, dtype=torch.int16, device="cuda")
    spy.flow_dev(r, s, pair, both_directions=True)
    spy.flow_dev(r, s, one, both_directions=False)
    spy.flow_dev(s, r, rev, both_directions=False)
    torch.cuda.synchronize()
    assert torch.equal(pair[: 2 * h * w], one)
    assert torch.equal(pair[2 * h * w:], rev)
    spy.free()


def test_clip_flows_equal_pair_calls(gpu_ctx, torch):
    """All pairs of a 5-frame clip in one pass == one pair call per adjacent pair, bit for
    bit (each image of the batch is computed independently of the others)."""
    h = w = 64
    frames = 5
    rng = np.random.default_rng(51)
    weights = sr.spynet_weights(rng)
    spy = gpu_ctx.spynet(h, w, {k: dev(torch, v) for k, v in weights.items()}, max_frames=frames)
    clip = [sr.smooth_frame(rng, h, w, shift=(0.7 * t, -1.1 * t)) for t in range(frames)]
    fr = dev(torch, np.concatenate(clip))
    log("case: spynet clip flows", frames)
    flows = torch.zeros(2 * (frames - 1) * 2 * h * w, dtype=torch.int16, device="cuda")
    spy.clip_flows_dev(fr, frames, flows)
    pair = torch.zeros(4 * h * w, dtype=torch.int16, device="cuda")
    plane = 3 * h * w
    f2 = 2 * h * w
    for t in range(frames - 1):
        spy.flow_dev(fr[t * plane:(t + 1) * plane], fr[(t + 1) * plane:(t + 2) * plane], pair)
        torch.cuda.synchronize()
        assert torch.equal(flows[t * f2:(t + 1) * f2], pair[:f2]), t
        assert torch.equal(flows[(frames - 1 + t) * f2:(frames + t) * f2], pair[f2:]), t
    with pytest.raises(Exception):
        spy.clip_flows_dev(fr, frames + 1, flows)
    spy.free()


def test_spynet_graph_replays_match_eager(gpu_ctx, torch):
    h = w = 64
    _, spy, ref, sup = _spynet(torch, gpu_ctx, h, w, 41)
    r, s = dev(torch, ref), dev(torch, sup)
    log("case: spynet graph")
    eager = torch.zeros(4 * h * w, dtype=torch.int16, device="cuda")
    spy.flow_dev(r, s, eager)
    torch.cuda.synchronize()
    out = torch.zeros_like(eager)
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        spy.flow_dev(r, s, out, stream=torch.cuda.current_stream())
    scratch = torch.zeros_like(eager)
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        spy.flow_dev(s, r, scratch)  # eager work between replays
        torch.cuda.synchronize()
    spy.free()


def test_spynet_rejects_bad_plane(gpu_ctx, dcn, torch):
    weights = sr.spynet_weights(np.random.default_rng(0))
    wd = {k: dev(torch, v) for k, v in weights.items()}
    with pytest.raises(dcn.DeformConvError) as e:
        gpu_ctx.spynet(48, 64, wd)
    assert e.value.status == dcn.INVALID_SHAPE
