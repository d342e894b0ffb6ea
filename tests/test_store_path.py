"""Save-pipeline ordering and failure handling, checked with fake streams on
the CPU (the reference's tests/test_connector_writeback.py and
tests/test_connector_scheduler.py cases, restated for this package)."""

import threading
from contextlib import nullcontext

import torch

from cacheblend_vllm import store_path as SP
from cacheblend_vllm.host_store import content_hash
from cacheblend_vllm.store_path import RequestMetadata, StoreStreamWriter, _slot_mapping
from cacheblend_vllm.trace import PipelineTracer
from cacheblend_vllm.types import SegmentId


class RecordingStream:
    def __init__(self):
        self.streams = []
        self.synchronize_calls = 0

    def wait_stream(self, stream):
        self.streams.append(stream)

    def synchronize(self):
        self.synchronize_calls += 1


class RecordingEvent:
    def __init__(self):
        self.recorded_on = None
        self.synchronize_calls = 0

    def record(self, stream):
        self.recorded_on = stream

    def synchronize(self):
        self.synchronize_calls += 1


class RecordingStore:
    def __init__(self):
        self.layers = []
        self.aborted = []

    def put_layer_host(self, segment_id, layer_id, tensor):
        self.layers.append((segment_id, layer_id, tensor))
        return True

    def abort_put(self, segment_id):
        self.aborted.append(segment_id)


class RecordingTracer:
    enabled = True

    def __init__(self):
        self.events = []

    def emit(self, event, request_id=None, **fields):
        self.events.append((event, request_id, fields))


class FakeStreams:
    def __init__(self, serving):
        self.serving = serving
        self.events = []

    def current_stream(self):
        return self.serving

    def stream(self, s):
        return nullcontext(s)

    def Event(self):  # noqa: N802
        event = RecordingEvent()
        self.events.append(event)
        return event

    def Stream(self):  # noqa: N802
        return RecordingStream()


def _writer(store, tracer=None, streams=None, store_stream=None):
    streams = streams or FakeStreams(RecordingStream())
    return StoreStreamWriter(store, block_size=2, chunk_size=4, num_layers=2, model_scope="m",
                             store_workers=1, max_inflight_store_batches=2,
                             tracer=tracer or PipelineTracer("test"), streams=streams,
                             store_stream=store_stream or RecordingStream())


def test_wait_for_save_synchronizes_single_store_stream():
    # reference tests/test_connector_writeback.py:72-86
    w = _writer(RecordingStore())
    w.wait_for_save()
    assert w._store_stream.synchronize_calls == 1
    assert not w._inflight
    w.close()


def test_enqueue_store_reuses_staging_and_offloads_on_one_stream(monkeypatch):
    # reference tests/test_connector_writeback.py:89-162
    serving = RecordingStream()
    streams = FakeStreams(serving)
    tracer = RecordingTracer()
    store = RecordingStore()
    w = _writer(store, tracer=tracer, streams=streams)
    gathered = [torch.arange(8).reshape(2, 4), torch.arange(8, 16).reshape(2, 4)]
    outputs = []
    original_empty = torch.empty

    def gather(_kv, _slots, _bs, out=None):
        source = gathered[len(outputs)]
        outputs.append(out)
        if out is None:
            return source.clone()
        out.copy_(source)
        return out

    def unpinned_empty(*args, **kwargs):
        kwargs.pop("pin_memory", None)
        return original_empty(*args, **kwargs)

    monkeypatch.setattr(SP, "gather_paged_kv", gather)
    monkeypatch.setattr(torch, "empty", unpinned_empty)
    # the fake layer has no device planes: keep the host slot list (a GPU
    # host would otherwise upload it next to the fake cache)
    monkeypatch.setattr(w, "_upload_slots", lambda _rid, slots, _kv: slots)
    w._enqueue_store_batch([("segment", 0, 4)], object(), torch.arange(4), request_id="request")
    first_staging = w._staging.live["request"]
    w._enqueue_store_batch([("segment", 1, 4)], object(), torch.arange(4), request_id="request")
    w.wait_for_save()
    w.close()

    assert w._store_stream.streams == [serving, serving]
    assert w._store_stream.synchronize_calls == 1
    assert streams.events[0].recorded_on is w._store_stream
    assert streams.events[0].synchronize_calls == 1
    assert outputs[0] is None and outputs[1] is first_staging
    assert w._staging.live == {} and w._staging.retired == []
    assert torch.equal(store.layers[0][2], gathered[0])
    assert torch.equal(store.layers[1][2], gathered[1])
    assert any(e == "save_store_wait_finished" and r == "request" and f["stores"] == 2
               for e, r, f in tracer.events)


def test_async_publish_aborts_the_whole_segment_on_failure(monkeypatch):
    # reference tests/test_connector_writeback.py:165-181
    store = RecordingStore()
    w = _writer(store)

    def fail(_batch, _kept):
        raise RuntimeError("publication failed")

    monkeypatch.setattr(w, "_put_chunks", fail)
    batch = SP._StoreBatch("r", [("segment-a", 3, 2), ("segment-b", 3, 2)],
                           torch.arange(8).reshape(2, 4), RecordingEvent())
    assert not w._publish(batch)
    assert batch.ready.synchronize_calls == 1
    assert store.aborted == ["segment-a", "segment-b"]
    w.close()


def test_publication_uses_views_of_the_pinned_batch():
    store = RecordingStore()
    w = _writer(store)
    host = torch.arange(2 * 8 * 3).reshape(2, 8, 3)
    kept = [None, None]
    assert w._put_chunks(SP._StoreBatch("r", [("a", 0, 4), ("b", 0, 4)], host), kept)
    assert kept == [False, False]  # the recording store cannot say it holds them
    (_, _, first), (_, _, second) = store.layers
    assert first.data_ptr() == host.data_ptr()
    assert torch.equal(second, host[:, 4:8])
    w.close()


class CountingStore:
    def __init__(self):
        self.calls = []

    def begin_put(self, model_scope, source_start, tokens, num_layers):
        tokens = tuple(tokens)
        self.calls.append((model_scope, source_start, tokens, num_layers))
        return SegmentId(model_scope, content_hash(tokens), source_start, len(tokens))


def test_save_segment_hashes_are_built_once_per_request():
    # reference tests/test_connector_scheduler.py:115-137
    store = CountingStore()
    w = _writer(store)
    request = RequestMetadata("r", list(range(12)), torch.arange(12), None, True, 12)
    first = w._request_save_segments(request, 8)
    assert [start for start, _ in first] == [0, 4] and len(store.calls) == 2
    grown = w._request_save_segments(request, 12)
    assert [start for start, _ in grown] == [0, 4, 8] and len(store.calls) == 3
    assert w._request_save_segments(request, 12) == grown and len(store.calls) == 3
    w.close()


def test_slot_mapping_known_answers(golden):
    for case in golden["slot_mapping"]["cases"]:
        got = _slot_mapping(case["block_ids"], case["block_size"], case["token_count"])
        assert got.tolist() == case["expected"]


def test_save_layer_fuses_pending_chunks_and_aborts_on_error(monkeypatch):
    class Store(CountingStore):
        def __init__(self):
            super().__init__()
            self.reserved, self.aborted = [], []

        def reserve_layer(self, sid, layer):
            self.reserved.append((sid.source_start, layer))
            return sid.source_start != 4  # chunk at 4 already stored

        def abort_put(self, sid):
            self.aborted.append(sid.source_start)

    store = Store()
    w = _writer(store)
    seen = {}

    def enqueue(pending, kv, slots, request_id, store_enqueued_ns=None):
        seen["slots"] = slots.tolist()
        seen["pending"] = [p[0].source_start for p in pending]
        raise RuntimeError("device failure")

    monkeypatch.setattr(w, "_enqueue_store_batch", enqueue)
    request = RequestMetadata("r", list(range(14)), torch.arange(100, 114), None, True, 13)
    try:
        w.save_layer(1, object(), [request])
    except RuntimeError:
        pass
    # usable = 13 // 4 * 4 = 12 -> chunks 0, 4, 8; chunk 4 skipped
    assert seen["pending"] == [0, 8]
    assert seen["slots"] == list(range(100, 104)) + list(range(108, 112))
    assert store.aborted == [0, 8]
    w.close()


def test_inflight_saves_bound_and_release():
    # the limit bounds batches in flight; a slot frees when its future completes
    from concurrent.futures import Future

    inflight = SP._InflightSaves(2)
    futures = [Future(), Future()]
    for f in futures:
        inflight.admit()
        inflight.track("r", f)
    blocked = threading.Thread(target=inflight.admit)
    blocked.start()
    blocked.join(0.05)
    assert blocked.is_alive()          # third admission waits ...
    futures[0].set_result(True)
    blocked.join(2)
    assert not blocked.is_alive()      # ... until a publication finishes
    assert inflight and list(inflight.take()) == ["r"] and not inflight
