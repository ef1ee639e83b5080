"""The allocation-free fused entry point (dcn_forward_f16_prepacked_noalloc_dev), through
the C ABI: bit-identical to dcn_forward_f16_prepacked_dev on the same inputs for two
calls in a row, the second with a smaller input (the shared scratch array still holds
the first call's larger copy), inside a captured hipGraph too, ordered across two streams,
and shapes whose padded input exceeds the scratch array are rejected before anything runs."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(dcn, torch, shape, seed):
    rng = np.random.default_rng(seed)
    c = shape.counts()
    h = {"input": rng.standard_normal(c["input"]).astype(np.float16),
         "offset": (10 * np.tanh(rng.standard_normal(c["offset"]))).astype(np.float16),
         "mask": (1 / (1 + np.exp(-rng.standard_normal(c["mask"])))).astype(np.float16),
         "weight": rng.uniform(-0.072, 0.072, c["weight"]).astype(np.float16),
         "bias": rng.uniform(-0.1, 0.1, c["bias"]).astype(np.float16)}
    return {k: torch.from_numpy(v.view(np.int16)).cuda() for k, v in h.items()}


def _run(ctx, shape, d, packed, noalloc, torch):
    out = torch.empty(shape.output_count, dtype=torch.int16, device="cuda")
    call = ctx.forward_f16_prepacked_noalloc_dev if noalloc else ctx.forward_f16_prepacked_dev
    call(shape, d["input"], d["offset"], d["mask"], packed, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_noalloc_matches_workspace_path_twice(dcn):
    import torch

    ctx = dcn.HipDeformConv(0)
    try:
        big = dcn.DeformConvShape(2, 128, 64, 64, 64, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
        small = dcn.DeformConvShape(1, 128, 24, 40, 64, 24, 40, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
        assert ctx.cb8_count(small) < ctx.cb8_count(big)
        d_big = _case(dcn, torch, big, 1)
        d_small = _case(dcn, torch, small, 2)
        packed = ctx.prepack_dev(big, d_big["weight"], d_big["bias"])  # same layer for both sizes
        for shape, d in ((big, d_big), (small, d_small)):  # larger, then smaller
            print("case: noalloc", shape.batch, shape.input_height, shape.input_width, flush=True)
            want = _run(ctx, shape, d, packed, False, torch)
            got = _run(ctx, shape, d, packed, True, torch)
            assert np.array_equal(got, want)
            assert np.all(np.isfinite(got.view(np.float16).astype(np.float32)))
        packed.free()
    finally:
        ctx.close()


def test_noalloc_in_captured_graph(dcn):
    """Replays of a captured graph holding the allocation-free call equal eager calls,
    with eager work on the device between the replays."""
    import torch

    ctx = dcn.HipDeformConv(0)
    try:
        s = dcn.DeformConvShape(1, 128, 64, 64, 64, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
        d = _case(dcn, torch, s, 3)
        packed = ctx.prepack_dev(s, d["weight"], d["bias"])
        want = _run(ctx, s, d, packed, False, torch)
        out = torch.empty(s.output_count, dtype=torch.int16, device="cuda")
        stream = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            ctx.forward_f16_prepacked_noalloc_dev(s, d["input"], d["offset"], d["mask"], packed, out,
                                                  stream=torch.cuda.current_stream())
        for i in range(3):
            out.zero_()
            _run(ctx, s, d, packed, True, torch)  # eager use of the same scratch between replays
            with torch.cuda.stream(stream):
                g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy(), want), i
        packed.free()
    finally:
        ctx.close()


def test_noalloc_calls_on_two_streams_are_ordered(dcn):
    """Calls on two streams, issued back to back without a host synchronisation, share the
    device's scratch array: the library makes each stream wait for the other's previous
    call, so every output equals the workspace path's."""
    import torch

    ctx = dcn.HipDeformConv(0)
    try:
        s = dcn.DeformConvShape(2, 128, 64, 64, 64, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
        cases = [_case(dcn, torch, s, 10 + i) for i in range(4)]
        packed = ctx.prepack_dev(s, cases[0]["weight"], cases[0]["bias"])
        want = [_run(ctx, s, d, packed, False, torch) for d in cases]
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        for rep in range(3):
            print("case: noalloc two streams, round", rep, flush=True)
            outs = [torch.zeros(s.output_count, dtype=torch.int16, device="cuda") for _ in cases]
            torch.cuda.synchronize()
            for i, d in enumerate(cases):  # streams 0, 1, 0, 1
                ctx.forward_f16_prepacked_noalloc_dev(s, d["input"], d["offset"], d["mask"], packed, outs[i],
                                                      stream=streams[i % 2])
            torch.cuda.synchronize()
            for i in range(len(cases)):
                assert np.array_equal(outs[i].cpu().numpy(), want[i]), (rep, i)
        packed.free()
    finally:
        ctx.close()


def test_noalloc_rejects_inputs_over_the_scratch_size(dcn):
    import torch

    ctx = dcn.HipDeformConv(0)
    try:
        s = dcn.DeformConvShape(16, 128, 256, 256, 64, 256, 256, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
        limit = 24 << 20  # DCN_NOALLOC_SCRATCH_BYTES
        assert ctx.cb8_count(s) * 2 > limit
        small = dcn.DeformConvShape(1, 128, 8, 8, 64, 8, 8, 3, 3, 1, 1, 1, 1, 1, 1, 1, 16)
        d = _case(dcn, torch, small, 4)
        packed = ctx.prepack_dev(small, d["weight"], d["bias"])
        with pytest.raises(dcn.DeformConvError) as e:  # fails validation before any launch
            ctx.forward_f16_prepacked_noalloc_dev(s, d["input"], d["offset"], d["mask"], packed, d["input"])
        assert e.value.status == dcn.INVALID_SHAPE
        assert "allocation-free" in e.value.message and str(limit) in e.value.message
        packed.free()
    finally:
        ctx.close()
