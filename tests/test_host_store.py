"""CPU: the pinned chunk store's segment lifecycle, LRU eviction, byte cap
and token-range lookup (reference storage.py:33-294 semantics)."""

import pytest
import torch

import oracle as O
from cacheblend_vllm.host_store import PinnedChunkStore
from cacheblend_vllm.types import BlendSegment, SegmentId

CH = 4
CHUNK_BYTES = 2 * CH * 8 * 4  # [2, 4, 8] float32


def _chunk(v):
    return torch.full((2, CH, 8), float(v))


def _put(store, start, layers=1, value=0.0):
    sid = store.begin_put("m", start, list(range(start, start + CH)), layers)
    results = [store.put_layer_host(sid, l, _chunk(value)) for l in range(layers)]
    return sid, results


def test_commit_after_all_layers_and_known_hash():
    store = PinnedChunkStore(CH, 1 << 20)
    sid, results = _put(store, 0, layers=3)
    assert results == [False, False, True] and store.is_committed(sid)
    assert sid.content_hash == O.content_hash(range(CH)) and store.committed_entries == 1
    assert store.put_layer_host(sid, 1, _chunk(9)) is False  # committed entries are immutable
    with pytest.raises(RuntimeError, match="collision"):
        store._entries[sid].tokens = (7,) * CH
        store.begin_put("m", 0, list(range(CH)), 3)


def test_lru_eviction_skips_pinned_and_uncommitted_then_fails_closed():
    released = []
    store = PinnedChunkStore(CH, 3 * CHUNK_BYTES, on_release=lambda t, events: released.append(t))
    a, _ = _put(store, 0)
    b, _ = _put(store, 100)
    c, _ = _put(store, 200)
    store.pin("r", [BlendSegment(a, 0)])          # a pinned and most recent
    store.validate([BlendSegment(c, 0)])          # c touched: LRU order b, a, c
    d, res = _put(store, 300)                     # evicts b (oldest unpinned committed)
    assert res == [True] and not store.is_committed(b) and store.is_committed(a)
    assert len(released) == 1 and store.current_bytes == 3 * CHUNK_BYTES
    e, res = _put(store, 400)                     # evicts c next, a stays pinned
    assert res == [True] and not store.is_committed(c) and store.is_committed(a)
    store.pin("s", [BlendSegment(d, 0), BlendSegment(e, 0)])
    f, res = _put(store, 500)                     # everything pinned: fail closed
    assert res == [None] and f not in store._entries
    store.release("s")                            # unpinned now, still within the cap
    assert store.current_bytes == 3 * CHUNK_BYTES
    g, res = _put(store, 600)
    assert res == [True] and not store.is_committed(d)


def test_cancel_abort_and_failed_segments_drop_as_a_unit():
    released = []
    store = PinnedChunkStore(CH, 1 << 20, on_release=lambda t, events: released.append(t))
    sid = store.begin_put("m", 0, list(range(CH)), 2)
    assert store.reserve_layer(sid, 0) and store.reserve_layer(sid, 1)
    assert not store.reserve_layer(sid, 1)         # already in flight
    assert store.put_layer_host(sid, 0, _chunk(1)) is False
    store.cancel_layer(sid, 1)                     # uncommitted: the segment fails
    assert sid not in store._entries and len(released) == 1 and store.current_bytes == 0
    sid2 = store.begin_put("m", 8, list(range(8, 8 + CH)), 2)
    store.put_layer_host(sid2, 0, _chunk(2))
    store.abort_put(sid2)
    assert sid2 not in store._entries and store.current_bytes == 0


def test_put_layer_copies_and_get_layer_requires_pin():
    store = PinnedChunkStore(CH, 1 << 20)
    sid = store.begin_put("m", 0, list(range(CH)), 1)
    src = _chunk(3)
    assert store.put_layer(sid, 0, src) is True
    seg = BlendSegment(sid, 0)
    with pytest.raises(RuntimeError, match="not pinned"):
        store.get_layer("r", seg, 0)
    assert store.pin("r", [seg]) == (seg,)
    got = store.get_layer("r", seg, 0)
    assert torch.equal(got, src) and got.data_ptr() != src.data_ptr()
    with pytest.raises(KeyError):
        store.put_layer(SegmentId("m", 1, 0, CH), 0, src)  # never begun


def _put_ref(store, scope, source, token_base, value):
    """Reference tests/test_storage.py:6-12: a two-layer segment is not found
    by ``match`` until its last layer commits."""
    tokens = list(range(token_base, token_base + 4))
    sid = store.begin_put(scope, source, tokens, num_layers=2)
    assert not store.put_layer(sid, 0, torch.full((2, 4, 2), value))
    assert store.match(scope, tokens, 0) == ()
    assert store.put_layer(sid, 1, torch.full((2, 4, 2), value + 1))
    return sid, tokens


def test_match_sees_only_committed_segments_and_they_pin():
    """Reference tests/test_storage.py:15-22."""
    store = PinnedChunkStore(4, 4096)
    sid, tokens = _put_ref(store, "m", 0, 10, 1)
    (segment,) = store.match("m", tokens, 0)
    assert segment.segment_id == sid and segment.target_start == 0
    assert store.pin("r", [segment]) == (segment,)
    assert torch.equal(store.get_layer("r", segment, 1), torch.full((2, 4, 2), 2))
    store.release("r")
    # found again at any offset of a longer prompt, and not in another scope
    (again,) = store.match("m", [0, 0, 0] + tokens + [5], 1)
    assert again.target_start == 3 and store.match("x", tokens, 0) == ()


def test_match_forgets_evicted_and_rejected_segments():
    """Reference tests/test_storage.py:25-43: the pinned entry survives, the
    rejected one is never matched, the evicted one is no longer matched."""
    per_entry = 2 * 2 * 4 * 2 * 4
    store = PinnedChunkStore(4, per_entry)
    _, tokens1 = _put_ref(store, "m", 0, 10, 1.0)
    (segment1,) = store.match("m", tokens1, 0)
    store.pin("r", [segment1])
    tokens2 = list(range(20, 24))
    sid2 = store.begin_put("m", 4, tokens2, num_layers=2)
    assert store.put_layer(sid2, 0, torch.full((2, 4, 2), 2.0)) is None
    assert store.match("m", tokens1, 0) == (segment1,)
    assert store.match("m", tokens2, 0) == ()
    assert store.current_bytes == per_entry
    store.release("r")
    _, tokens3 = _put_ref(store, "m", 8, 30, 3.0)
    assert store.current_bytes <= store.max_bytes
    assert store.match("m", tokens1, 0) == ()
    assert store.match("m", tokens3, 0)
    assert store.committed_entries == 1


def test_cancelled_and_cleared_segments_are_not_matched():
    """Reference tests/test_storage.py:60-73, and ``clear``."""
    store = PinnedChunkStore(4, 4096)
    tokens = [1, 2, 3, 4]
    sid = store.begin_put("m", 0, tokens, num_layers=2)
    assert store.reserve_layer(sid, 0)
    assert not store.put_layer_host(sid, 0, torch.ones(2, 4, 2))
    assert store.reserve_layer(sid, 1)
    store.cancel_layer(sid, 1)
    assert store.current_bytes == 0 and store.match("m", tokens, 0) == ()
    sid = store.begin_put("m", 0, tokens, num_layers=1)
    assert store.put_layer_host(sid, 0, torch.ones(2, 4, 2))
    assert len(store.match("m", tokens + tokens, 0)) == 2
    store.clear()
    assert store.match("m", tokens, 0) == () and store.committed_entries == 0


def test_begin_put_chunks_equals_per_chunk_begin_put():
    tokens = list(range(1000, 1000 + 4 * CH)) + [7]
    a, b = PinnedChunkStore(CH, 1 << 20), PinnedChunkStore(CH, 1 << 20)
    ids = a.begin_put_chunks("m", tokens, CH, 4 * CH, 2)
    assert ids == [b.begin_put("m", s, tokens[s:s + CH], 2) for s in range(CH, 4 * CH, CH)]
    assert [sid.content_hash for sid in ids] == [O.content_hash(tokens[s:s + CH]) for s in range(CH, 4 * CH, CH)]
    assert a.begin_put_chunks("m", tokens, 0, 0, 2) == []
    with pytest.raises(ValueError, match="whole number"):
        a.begin_put_chunks("m", tokens, 0, CH + 1, 2)
    with pytest.raises(ValueError, match="num_layers changed"):
        a.begin_put_chunks("m", tokens, CH, 2 * CH, 3)
    assert a.reserve_layers(ids + [SegmentId("m", 1, 0, CH)], 1) == [True, True, True, False]
    assert a.reserve_layers(ids, 1) == [False, False, False]
    with pytest.raises(ValueError, match="outside"):
        a.reserve_layers(ids, 2)


class _Event:
    """A GPU event stand-in whose completion the test controls."""

    def __init__(self, done=False):
        self.done = done

    def query(self):
        return self.done


def test_release_event_travels_with_evicted_chunks():
    """A load's last host-read event, given at release, is handed to the
    release hook with every chunk the store drops afterwards; completed
    events are pruned when new ones arrive."""
    released = []
    store = PinnedChunkStore(CH, 2 * CHUNK_BYTES, on_release=lambda t, ev: released.append((t, ev)))
    a, _ = _put(store, 0)
    b, _ = _put(store, 100)
    store.pin("r", [BlendSegment(a, 0), BlendSegment(b, 0)])
    old, live = _Event(done=True), _Event()
    store.release("r", old)
    store.pin("s", [BlendSegment(a, 0)])
    store.release("s", live)                       # a: the completed event is pruned
    assert store._entries[a].read_events == [live]
    assert store._entries[b].read_events == [old]
    _put(store, 200)                               # evicts b (pinning "s" touched a)
    _put(store, 300)                               # evicts a
    assert [ev for _, ev in released] == [(old,), (live,)]
    assert store.current_bytes == 2 * CHUNK_BYTES
    store.clear()                                  # entries never read: no events
    assert [ev for _, ev in released[2:]] == [(), ()]
