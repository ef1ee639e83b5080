"""TemporalSchedule, temporalChunkRanges and the recoverable-error ladder (CPU).

The first five tests restate the reference's own tests with their expected values:
TemporalScheduleTests.swift:4-40 and RestorationResumeTests.swift:51-72."""
from __future__ import annotations

import numpy as np
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


class _StandInClip:
    """Stand-in runner for the recovery ladder: a recurrence in FP16,
    out[t] = out[t-1] / 2 + frame[t] + flow[t] (flow[t] = the motion into frame t, none at
    a chunk's first frame). NaN motion poisons every chunk that crosses it but not the
    zero-motion triplets; frames near the FP16 maximum overflow every rung."""

    def __init__(self, dcn, frames, flows, other_error_at=None):
        self.dcn = dcn
        self.frames = np.asarray(frames, np.float16)
        self.flows = np.asarray(flows, np.float16)  # flows[t - 1]: motion into frame t
        self.out = np.zeros_like(self.frames)
        self.calls = []
        self.other_error_at = other_error_at

    def _recur(self, frames, flows):
        prev, out = np.float16(0), []
        with np.errstate(over="ignore", invalid="ignore"):
            for i, f in enumerate(frames):
                prev = np.float16(prev / np.float16(2) + f + (flows[i - 1] if i else np.float16(0)))
                out.append(prev)
        return out

    def _step(self, name):
        self.calls.append(name)
        if name == self.other_error_at:
            raise self.dcn.DeformConvError(self.dcn.COMMAND_FAILED, "device lost")

    def _check(self):
        if not np.isfinite(self.out).all():
            raise self.dcn.DeformConvError(self.dcn.NONFINITE_OUTPUT, "overflow")

    def run(self, chunk):
        self._step(chunk)
        T = len(self.frames)
        ranges = [range(T)] if chunk == 0 else self.dcn.temporal_chunk_ranges(T, chunk)
        for r in ranges:
            self.out[r.start:r.stop] = self._recur(self.frames[r.start:r.stop], self.flows[r.start:r.stop - 1])
        self._check()

    def run_triplets(self):
        self._step("triplets")
        for t, f in enumerate(self.frames):
            trip = self._recur([f, f, f], np.zeros(2, np.float16))
            if not np.isfinite(trip).all():
                raise self.dcn.DeformConvError(self.dcn.NONFINITE_OUTPUT, "overflow")
            self.out[t] = trip[1]

    def input_is_finite(self):
        self._step("finite?")
        return bool(np.isfinite(self.frames).all())

    def pass_through(self):
        self._step("passthrough")
        self.out[:] = self.frames

    def ladder(self, report=None):
        return self.dcn.propagate_with_fallback(self.run, len(self.frames), report, run_triplets=self.run_triplets,
                                                input_is_finite=self.input_is_finite, pass_through=self.pass_through)


def _clip(dcn, T=30, scale=1.0, gain_frames=(), nan_flow_into=None, **kw):
    frames = np.full(T, scale, np.float32)
    for t, v in gain_frames:
        frames[t] = v
    flows = np.full(T - 1, 0.25, np.float32)
    if nan_flow_into is not None:
        flows[nan_flow_into - 1] = np.nan
    return _StandInClip(dcn, frames, flows, **kw)


def test_fallback_ladder_full_window_first(dcn):
    c = _clip(dcn)
    assert c.ladder() == 0
    assert c.calls == [0]
    assert np.isfinite(c.out).all()


def test_fallback_ladder_recovers_with_shorter_chunks(dcn):
    # 60000 then 40000 at frames 4 and 5: 30000 + 40000 overflows where frame 5 follows
    # frame 4 in one chunk (the whole clip, chunks of 10); chunks of 5 start at frame 5.
    c = _clip(dcn, gain_frames=[(4, 60000.0), (5, 40000.0)])
    assert c.ladder() == 5
    assert c.calls == [0, 10, 5]
    want = np.concatenate([c._recur(c.frames[r.start:r.stop], c.flows[r.start:r.stop - 1])
                           for r in dcn.temporal_chunk_ranges(30, 5)])
    assert np.array_equal(c.out, want)


def test_fallback_ladder_zero_motion_triplets_keep_the_middle_frame(dcn):
    # NaN motion into frame 4 lies inside a chunk at every chunk size.
    c = _clip(dcn, nan_flow_into=4)
    c.frames[:] = np.arange(30, dtype=np.float16)
    msgs = []
    assert c.ladder(msgs.append) == dcn.RECOVERED_TRIPLETS
    assert c.calls == [0, 10, 5, 3, "triplets"]
    f = c.frames
    assert np.array_equal(c.out, (f / np.float16(2) + f).astype(np.float16))  # [f, f, f] -> f, 1.5 f, 1.75 f
    assert msgs[-1] == "recovered with independent zero-motion frame triplets"


def test_fallback_ladder_passes_finite_input_through(dcn):
    c = _clip(dcn, scale=60000.0)  # the second step of every rung overflows
    msgs = []
    assert c.ladder(msgs.append) == dcn.RECOVERED_PASSTHROUGH
    assert c.calls == [0, 10, 5, 3, "triplets", "finite?", "passthrough"]
    assert np.array_equal(c.out, c.frames)
    assert msgs[-1].startswith("WARNING: using finite input passthrough")


def test_fallback_ladder_fails_on_non_finite_input(dcn):
    c = _clip(dcn, T=6, gain_frames=[(2, np.inf)])
    with pytest.raises(dcn.DeformConvError) as e:
        c.ladder()
    assert e.value.status == dcn.COMMAND_FAILED
    assert "non-finite input" in str(e.value)
    # Chunks not shorter than the clip are skipped; nothing is passed through.
    assert c.calls == [0, 5, 3, "triplets", "finite?"]


@pytest.mark.parametrize("where", [0, 10, "triplets"])
def test_fallback_ladder_does_not_retry_unrecoverable_errors(dcn, where):
    c = _clip(dcn, scale=60000.0, other_error_at=where)
    with pytest.raises(dcn.DeformConvError) as e:
        c.ladder()
    assert e.value.status == dcn.COMMAND_FAILED
    assert c.calls[-1] == where
