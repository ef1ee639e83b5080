"""This build against the reference's own test vectors for the DCN path and its host logic,
kept as data in tests/golden/reference_tests.json (each entry cites the reference test it
comes from): the CPU oracle and the host functions on the CPU, the library's FP32 entry
point and its non-finite flag on the GPU."""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_tests.json").read_text())


def _values(xs):
    return [float(x) for x in xs]  # "inf" / "nan" strings included


def _kat(dcn):
    k = GOLDEN["deform_conv_cpu_known_answer"]
    s = dcn.DeformConvShape(**k["shape"])
    c = s.counts()
    args = [np.asarray(k["input"], np.float32), np.full(c["offset"], k["offset_fill"], np.float32),
            np.full(c["mask"], k["mask_fill"], np.float32), np.asarray(k["weight"], np.float32),
            np.asarray(k["bias"], np.float32)]
    return s, args, np.asarray(k["expected"], np.float32)


def test_oracle_known_answer(dcn, oracle):
    s, args, want = _kat(dcn)
    got = oracle.forward_f32(s, *args)
    assert np.array_equal(got, want)


@pytest.mark.gpu
def test_fp32_entry_point_known_answer(gpu_ctx, dcn):
    s, args, want = _kat(dcn)
    got = gpu_ctx.run_float32(s, *args)
    assert np.array_equal(got, want)


def test_recoverable_errors(dcn):
    r = GOLDEN["recoverable_errors"]
    status = {"nonFiniteOutput": dcn.NONFINITE_OUTPUT, "invalidShape": dcn.INVALID_SHAPE,
              "metalUnavailable": dcn.DEVICE_UNAVAILABLE, "shaderResourceMissing": dcn.KERNEL_MISSING,
              "commandFailed": dcn.COMMAND_FAILED}
    for name in r["recoverable"]:
        assert dcn.DeformConvError(status[name]).is_recoverable_numerical_failure, name
    for name in r["not_recoverable"]:
        assert not dcn.DeformConvError(status[name]).is_recoverable_numerical_failure, name


def test_benchmark_statistics(dcn):
    b = GOLDEN["benchmark_statistics"]
    st = dcn.BenchmarkStatistics.of(b["samples"])
    tol = b["tolerance"]
    assert list(st.samples) == b["sorted"]
    assert st.minimum == b["minimum"] and st.maximum == b["maximum"]
    assert st.median == b["median"] and st.mean == b["mean"]
    assert abs(st.standard_deviation - math.sqrt(b["standard_deviation_squared"])) < tol
    assert abs(st.percentile10 - b["percentile10"]) < tol and abs(st.percentile90 - b["percentile90"]) < tol
    for case in b["rejected"]["cases"]:
        assert dcn.BenchmarkStatistics.of(_values(case)) is None, case


@pytest.mark.gpu
@pytest.mark.parametrize("case", GOLDEN["nonfinite_flag"]["cases"], ids=lambda c: str(c["values"]))
def test_nonfinite_flag(gpu_ctx, case):
    import torch

    v = torch.from_numpy(np.asarray(_values(case["values"]), np.float16).view(np.int16)).cuda()
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    gpu_ctx.flag_nonfinite_f16_dev(v, v.numel(), flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == case["flag"]


def _branch(schedule, name):
    return [s for s in schedule.steps if s.branch.name == name]


def test_temporal_schedule(dcn):
    t = GOLDEN["temporal_schedule"]
    four = dcn.TemporalSchedule(t["four_frames"]["frames"])
    for name in ("backward_1", "forward_1"):
        steps = _branch(four, name)
        assert [s.frame_index for s in steps] == t["four_frames"][name]["frame"]
        assert [s.flow_index for s in steps] == t["four_frames"][name]["flow"]
        assert steps[2].second_order_frame_index == t["four_frames"][name]["second_order_at_2"]
    three = dcn.TemporalSchedule(t["three_frames"]["frames"])
    assert [b.backbone_input_channels for b in three.branches] == t["three_frames"]["backbone_input_channels"]
    assert len(three.steps) == t["three_frames"]["steps"]
    assert three.flow_count_per_direction == t["three_frames"]["flows_per_direction"]
    five = dcn.TemporalSchedule(t["five_frames"]["frames"])
    for name in ("backward_1", "forward_1"):
        steps = _branch(five, name)
        assert [s.frame_index for s in steps] == t["five_frames"][name]["frame"]
        assert [s.flow_index for s in steps] == t["five_frames"][name]["flow"]
        assert [s.second_order_frame_index for s in steps] == t["five_frames"][name]["second_order"]
    thirty = dcn.TemporalSchedule(t["thirty_frames"]["frames"])
    assert thirty.flow_count_per_direction == t["thirty_frames"]["flows_per_direction"]
    assert len(thirty.steps) == t["thirty_frames"]["steps"]
    assert thirty.persistent_tensor_bytes == t["thirty_frames"]["persistent_tensor_bytes"]


@pytest.mark.parametrize("case", GOLDEN["temporal_chunk_ranges"]["cases"],
                         ids=lambda c: f"{c['frames']}-{c['max_per_chunk']}")
def test_temporal_chunk_ranges(dcn, case):
    got = dcn.temporal_chunk_ranges(case["frames"], case["max_per_chunk"])
    assert [(r.start, r.stop) for r in got] == [tuple(r) for r in case["ranges"]]
