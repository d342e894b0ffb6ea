"""Plan types and the JSONL trace format, on the CPU (the reference's
tests/test_types.py:10-24 and tests/test_trace.py:6-28 cases, restated, plus
the validation messages and wire format a drop-in must keep)."""

import json
import os
import threading

import pytest

from cacheblend_vllm.trace import PipelineTracer
from cacheblend_vllm.types import BlendPlan, BlendSegment, SegmentId


def segment(source: int, target: int, length: int = 4) -> BlendSegment:
    return BlendSegment(SegmentId("model", source + 7, source, length), target)


def test_plan_round_trip_and_gaps():
    # reference tests/test_types.py:10-15
    plan = BlendPlan.from_segments(4, [segment(0, 4), segment(8, 12)])
    assert (plan.allocation_end, plan.hit_tokens, plan.gap_tokens) == (16, 8, 4)
    assert plan.allocation_tokens == 12
    assert BlendPlan.from_dict(plan.to_dict()) == plan
    assert plan.gap_runs() == [(8, 12)]
    # duplicates dropped, order restored; an empty plan spans nothing
    assert BlendPlan.from_segments(4, [segment(8, 12), segment(0, 4), segment(0, 4)]) == plan
    empty = BlendPlan.from_segments(3, [])
    assert (empty.allocation_end, empty.hit_tokens, empty.segments) == (3, 0, ())


def test_plan_wire_format():
    plan = BlendPlan(1, 9, 4, (segment(0, 2),))
    assert plan.to_dict() == {
        "apc_prefix_tokens": 1, "allocation_end": 9, "hit_tokens": 4,
        "segments": [{"segment_id": {"model_scope": "model", "content_hash": 7, "source_start": 0,
                                     "token_count": 4}, "target_start": 2}],
    }
    assert BlendPlan.from_dict({"apc_prefix_tokens": "2", "allocation_end": 2, "hit_tokens": 0}) == \
        BlendPlan(2, 2, 0, ())


@pytest.mark.parametrize("args, message", [
    ((0, 8, 8, (segment(0, 0), segment(4, 2))), "segments cannot overlap"),   # test_types.py:22-24
    ((-1, 8, 0, ()), "invalid CacheBlend allocation span"),
    ((5, 4, 0, ()), "invalid CacheBlend allocation span"),
    ((4, 20, 4, (segment(0, 2),)), "segments must start after the APC prefix"),
    ((0, 5, 4, (segment(0, 2),)), "segment exceeds allocation span"),
    ((0, 20, 5, (segment(0, 2),)), "hit_tokens=5 does not match segments=4"),
    ((0, 20, 8, (segment(8, 10), segment(0, 2))), "segments must be sorted"),
])
def test_plan_validation_messages(args, message):
    with pytest.raises(ValueError, match=message):
        BlendPlan(*args)


def test_segment_validation_messages():
    with pytest.raises(ValueError, match="model_scope cannot be empty"):
        SegmentId("", 1, 0, 4)
    for start, count in ((-1, 4), (0, 0)):
        with pytest.raises(ValueError, match="invalid source segment"):
            SegmentId("m", 1, start, count)
    with pytest.raises(ValueError, match="target_start cannot be negative"):
        BlendSegment(SegmentId("m", 1, 0, 4), -1)
    seg = segment(3, 10, 5)
    assert (seg.source_start, seg.length, seg.target_end) == (3, 5, 15)
    assert SegmentId.from_dict(seg.segment_id.to_dict()) == seg.segment_id


def test_trace_is_disabled_by_default(monkeypatch, tmp_path):
    # reference tests/test_trace.py:6-11
    monkeypatch.delenv("CACHEBLEND_TRACE_DIR", raising=False)
    tracer = PipelineTracer("worker")
    assert not tracer.enabled
    tracer.emit("ignored", request_id="r")
    tracer.close()
    assert not list(tmp_path.iterdir())


def test_trace_writes_structured_events(monkeypatch, tmp_path):
    # reference tests/test_trace.py:14-28
    monkeypatch.setenv("CACHEBLEND_TRACE_DIR", str(tmp_path / "sub"))
    tracer = PipelineTracer("scheduler")
    assert tracer.enabled
    tracer.emit("lookup_done", request_id="r", duration_us=12.5, hit_tokens=256)
    tracer.emit("no_request")
    tracer.close()
    tracer.emit("after_close")  # ignored once closed
    (path,) = (tmp_path / "sub").iterdir()
    assert path.name == f"scheduler-pid-{os.getpid()}.jsonl"
    lines = path.read_text().splitlines()
    rows = [json.loads(line) for line in lines]
    assert [r["event"] for r in rows] == ["trace_started", "lookup_done", "no_request"]
    assert rows[1]["component"] == "scheduler" and rows[1]["request_id"] == "r"
    assert rows[1]["duration_us"] == 12.5 and rows[1]["hit_tokens"] == 256
    assert "request_id" not in rows[2]
    assert rows[1]["pid"] == os.getpid() and rows[1]["thread_id"] == threading.get_ident()
    assert rows[1]["monotonic_ns"] >= rows[0]["monotonic_ns"]
    # compact, key-sorted lines
    assert lines[1] == json.dumps(rows[1], sort_keys=True, separators=(",", ":"))


def test_trace_appends_across_tracers(monkeypatch, tmp_path):
    monkeypatch.setenv("CACHEBLEND_TRACE_DIR", str(tmp_path))
    for _ in range(2):
        t = PipelineTracer("worker")
        t.emit("x")
        t.close()
    (path,) = tmp_path.iterdir()
    assert [json.loads(s)["event"] for s in path.read_text().splitlines()] == \
        ["trace_started", "x", "trace_started", "x"]


def test_roctx_ranges_are_opt_in(monkeypatch):
    """Without CACHEBLEND_ROCTX the phase decorators and roctx_range touch no
    profiler API; with it, each call sits inside one push/pop pair."""
    import torch

    from cacheblend_vllm import trace

    calls = []
    monkeypatch.setattr(torch.cuda.nvtx, "range_push", lambda name: calls.append(("push", name)))
    monkeypatch.setattr(torch.cuda.nvtx, "range_pop", lambda: calls.append(("pop",)))

    @trace.roctx_phase("phase")
    def work(x, *, y=1):
        calls.append(("work", x, y))
        return x + y

    monkeypatch.setattr(trace, "_roctx_on", False)
    assert work(2, y=3) == 5
    with trace.roctx_range("r"):
        pass
    assert calls == [("work", 2, 3)]
    calls.clear()
    monkeypatch.setattr(trace, "_roctx_on", True)
    assert work(1) == 2
    with trace.roctx_range("r"):
        calls.append(("inside",))
    assert calls == [("push", "phase"), ("work", 1, 1), ("pop",), ("push", "r"), ("inside",), ("pop",)]
