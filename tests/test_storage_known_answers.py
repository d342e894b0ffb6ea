"""``cacheblend_vllm.storage.LocalPinnedCPUStore`` on the reference's own store
scenarios (tests/test_storage.py:15-82 of the reference), restated: 4-token
chunks, two-layer segments of float32 ``[2, 4, 2]`` planes, pinning off (CPU).

* a segment is invisible to ``match`` until its last layer lands; once
  committed it can be pinned and read back;
* the LRU never evicts a pinned segment: a put that would need it is
  rejected (None) without passing the byte cap, and after the release the
  old segment is the one evicted;
* a layer reservation is granted once, and the host tensor handed to
  ``put_layer_host`` is stored as is (the same object comes back);
* cancelling a reserved layer drops the whole incomplete segment and its
  bytes, and the segment takes no further reservations;
* a segment larger than the store is rejected with nothing stored.
"""

import torch

from cacheblend_vllm.storage import LocalPinnedCPUStore

PLANE = (2, 4, 2)
ENTRY_BYTES = 2 * 2 * 4 * 2 * 4  # two layers of float32 [2, 4, 2]


def _store(max_bytes):
    return LocalPinnedCPUStore(4, max_bytes=max_bytes, pin_memory=False)


def _commit_two_layers(store, scope, source_start, first_token, value):
    """Puts a 4-token segment layer by layer; returns (segment id, tokens)."""
    tokens = [first_token + i for i in range(4)]
    sid = store.begin_put(scope, source_start, tokens, num_layers=2)
    assert not store.put_layer(sid, 0, torch.full(PLANE, value))
    assert store.match(scope, tokens, 0) == ()  # half a segment is not visible
    assert store.put_layer(sid, 1, torch.full(PLANE, value + 1))  # the last layer commits
    return sid, tokens


def test_committed_segment_matches_pins_and_reads_back():
    store = _store(4096)
    sid, tokens = _commit_two_layers(store, "m", 0, 10, 1)
    (segment,) = store.match("m", tokens, 0)
    assert segment.segment_id == sid
    assert store.pin("req", [segment]) == (segment,)
    assert torch.equal(store.get_layer("req", segment, 1), torch.full(PLANE, 2))
    store.release("req")


def test_pinned_segment_survives_and_blocks_a_put_until_released():
    store = _store(ENTRY_BYTES)
    _, first = _commit_two_layers(store, "m", 0, 10, 1.0)
    (held,) = store.match("m", first, 0)
    store.pin("req", [held])
    second = [20, 21, 22, 23]
    sid2 = store.begin_put("m", 4, second, num_layers=2)
    assert store.put_layer(sid2, 0, torch.full(PLANE, 2.0)) is None  # no room without the pinned one
    assert store.match("m", first, 0) == (held,)
    assert store.match("m", second, 0) == ()
    assert store.current_bytes == ENTRY_BYTES
    store.release("req")
    _, third = _commit_two_layers(store, "m", 8, 30, 3.0)
    assert store.current_bytes <= store.max_bytes
    assert store.match("m", first, 0) == ()  # the released segment was evicted
    assert store.match("m", third, 0)


def test_layer_reservation_is_granted_once_and_the_host_tensor_is_kept():
    store = _store(4096)
    sid = store.begin_put("m", 0, [1, 2, 3, 4], num_layers=1)
    assert store.reserve_layer(sid, 0)
    assert not store.reserve_layer(sid, 0)
    host = torch.ones(2, 8, 2)[:, 2:6]  # a non-contiguous view, as a batch slice is
    assert not host.is_contiguous()
    assert store.put_layer_host(sid, 0, host)
    (segment,) = store.match("m", [1, 2, 3, 4], 0)
    store.pin("req", [segment])
    assert store.get_layer("req", segment, 0) is host


def test_cancelled_layer_drops_the_incomplete_segment():
    store = _store(4096)
    tokens = [1, 2, 3, 4]
    sid = store.begin_put("m", 0, tokens, num_layers=2)
    assert store.reserve_layer(sid, 0)
    assert not store.put_layer_host(sid, 0, torch.ones(PLANE))
    assert store.current_bytes > 0
    assert store.reserve_layer(sid, 1)
    store.cancel_layer(sid, 1)
    assert store.current_bytes == 0
    assert store.match("m", tokens, 0) == ()
    assert not store.reserve_layer(sid, 1)


def test_segment_larger_than_the_store_is_rejected():
    store = _store(32)
    sid = store.begin_put("m", 0, [1, 2, 3, 4], num_layers=1)
    assert store.put_layer_host(sid, 0, torch.ones(PLANE)) is None
    assert store.current_bytes == 0
    assert store.committed_entries == 0
