"""TemporalSchedule, temporalChunkRanges and the recoverable-error ladder (CPU).

The first five tests restate the reference's own tests with their expected values:
TemporalScheduleTests.swift:4-40 and RestorationResumeTests.swift:51-72."""
from __future__ import annotations

import pytest


def test_temporal_schedule_matches_basicvsr_traversal(dcn):
    schedule = dcn.TemporalSchedule(4)
    backward = [s for s in schedule.steps if s.branch.name == "backward_1"]
    forward = [s for s in schedule.steps if s.branch.name == "forward_1"]
    assert [s.frame_index for s in backward] == [3, 2, 1, 0]
    assert [s.flow_index for s in backward] == [None, 2, 1, 0]
    assert [s.frame_index for s in forward] == [0, 1, 2, 3]
    assert [s.flow_index for s in forward] == [None, 0, 1, 2]
    assert backward[2].second_order_frame_index == 3
    assert forward[2].second_order_frame_index == 0


def test_temporal_schedule_uses_expected_backbone_widths(dcn):
    schedule = dcn.TemporalSchedule(3)
    assert [b.backbone_input_channels for b in schedule.branches] == [128, 192, 256, 320]
    assert len(schedule.steps) == 12
    assert schedule.flow_count_per_direction == 2


def test_five_frame_schedule_carries_rolling_second_order_history(dcn):
    schedule = dcn.TemporalSchedule(5)
    backward = [s for s in schedule.steps if s.branch.name == "backward_1"]
    forward = [s for s in schedule.steps if s.branch.name == "forward_1"]
    assert [s.frame_index for s in backward] == [4, 3, 2, 1, 0]
    assert [s.flow_index for s in backward] == [None, 3, 2, 1, 0]
    assert [s.second_order_frame_index for s in backward] == [None, None, 4, 3, 2]
    assert [s.frame_index for s in forward] == [0, 1, 2, 3, 4]
    assert [s.flow_index for s in forward] == [None, 0, 1, 2, 3]
    assert [s.second_order_frame_index for s in forward] == [None, None, 0, 1, 2]


def test_thirty_frame_schedule_has_production_length_resources(dcn):
    schedule = dcn.TemporalSchedule(30)
    assert schedule.flow_count_per_direction == 29
    assert len(schedule.steps) == 120
    assert schedule.persistent_tensor_bytes == 91_389_952


def test_temporal_chunk_ranges_match_the_reference(dcn):
    r = dcn.temporal_chunk_ranges
    assert r(30, 10) == [range(0, 10), range(10, 20), range(20, 30)]
    assert r(29, 10) == [range(0, 10), range(10, 20), range(20, 29)]
    assert r(11, 5) == [range(0, 4), range(4, 8), range(8, 11)]
    assert r(5, 3) == [range(0, 5)]


@pytest.mark.parametrize("frames,chunk", [(2, 10), (30, 2), (0, 3)])
def test_temporal_chunk_ranges_reject_short_inputs(dcn, frames, chunk):
    with pytest.raises(dcn.DeformConvError) as e:
        dcn.temporal_chunk_ranges(frames, chunk)
    assert e.value.status == dcn.INVALID_SHAPE


def test_schedule_rejects_empty_clip(dcn):
    with pytest.raises(dcn.DeformConvError) as e:
        dcn.TemporalSchedule(0)
    assert e.value.status == dcn.INVALID_SHAPE


@pytest.mark.parametrize("frames", [1, 2, 7, 30])
def test_schedule_invariants(dcn, frames):
    """Each branch visits every frame once in its direction; the flow index is the pair
    between the frame and the previous one in traversal order; second order is two back."""
    schedule = dcn.TemporalSchedule(frames)
    for b in schedule.branches:
        steps = [s for s in schedule.steps if s.branch == b]
        order = list(range(frames))[::-1] if b.direction == "backward" else list(range(frames))
        assert [s.frame_index for s in steps] == order
        for p, s in enumerate(steps):
            assert s.position == p
            if p == 0:
                assert s.flow_index is None
            else:
                assert {s.flow_index, s.flow_index + 1} == {order[p], order[p - 1]}
            assert s.second_order_frame_index == (order[p - 2] if p >= 2 else None)


def _fake_runner(dcn, fails_above: int | None, other_error: bool = False):
    calls = []

    def run(chunk):
        calls.append(chunk)
        if other_error:
            raise dcn.DeformConvError(dcn.COMMAND_FAILED, "device lost")
        size = 30 if chunk == 0 else chunk
        if fails_above is not None and size > fails_above:
            raise dcn.DeformConvError(dcn.NONFINITE_OUTPUT, "overflow")

    return run, calls


def test_fallback_ladder_recovers_with_shorter_chunks(dcn):
    run, calls = _fake_runner(dcn, fails_above=5)
    assert dcn.propagate_with_fallback(run, 30) == 5
    assert calls == [0, 10, 5]


def test_fallback_ladder_full_window_first(dcn):
    run, calls = _fake_runner(dcn, fails_above=None)
    assert dcn.propagate_with_fallback(run, 30) == 0
    assert calls == [0]


def test_fallback_ladder_skips_chunks_not_shorter_than_the_clip(dcn):
    run, calls = _fake_runner(dcn, fails_above=2)
    with pytest.raises(dcn.DeformConvError) as e:
        dcn.propagate_with_fallback(run, 6)
    assert calls == [0, 5, 3]
    assert e.value.status == dcn.COMMAND_FAILED


def test_fallback_ladder_does_not_retry_unrecoverable_errors(dcn):
    run, calls = _fake_runner(dcn, fails_above=None, other_error=True)
    with pytest.raises(dcn.DeformConvError) as e:
        dcn.propagate_with_fallback(run, 30)
    assert calls == [0]
    assert e.value.status == dcn.COMMAND_FAILED
