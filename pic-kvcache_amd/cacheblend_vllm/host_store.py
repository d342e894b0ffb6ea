"""Pinned host chunk store: the part of the reference store the KV path uses.

The store/load kernels exchange KV with host memory in the reference's
chunk format: per segment (one ``chunk_size``-token chunk) and layer, a host
tensor ``[2, chunk, *row]`` whose K and V planes are each contiguous -- a
slot of the pinned chunk slab, or a view ``host[:, off:off + chunk]`` of one
pinned per-layer batch (reference connector.py:449-466). This class keeps
that contract and the method names/semantics of ``LocalPinnedCPUStore``
(reference storage.py:33-294) that the save and load paths call:
``begin_put`` (with the content-hash collision check), ``reserve_layer``,
``cancel_layer``, ``put_layer``, ``put_layer_host``, ``abort_put``,
``match``, ``validate``, ``pin``, ``release``, ``get_layer``, ``clear``. A
segment commits when every layer is present and is then registered with the
token-range matcher; a failed or aborted segment is dropped as a unit; the
byte cap is fail-closed after evicting least recently used, committed,
unpinned segments. The lookup RPC around ``match`` is the scheduler's
control plane and is not part of this package.
"""

from __future__ import annotations

import ctypes
import math
import threading
from collections import OrderedDict
from collections.abc import Callable, Iterable, Sequence
from dataclasses import dataclass, field

import torch

from . import _native
from .hashing import as_token_array, content_hash, rolling_hash_values
from .matcher import FingerprintRecord, TokenRangeMatcher
from .types import BlendSegment, SegmentId

@dataclass
class _Entry:
    num_layers: int
    tokens: tuple[int, ...] = ()
    layers: dict[int, torch.Tensor] = field(default_factory=dict)
    reserved: set[int] = field(default_factory=set)
    size_bytes: int = 0
    pins: int = 0
    committed: bool = False
    failed: bool = False
    # layer -> in-place address of the stored chunk (see chunk_address)
    addresses: dict[int, tuple | None] = field(default_factory=dict)
    # GPU events of loads that read this entry's host memory: the memory is
    # handed back (on_release) only together with them
    read_events: list = field(default_factory=list)


def chunk_address(t: torch.Tensor) -> tuple | None:
    """``(k_ptr, v_ptr, (chunk_tokens, row_shape, dtype))`` when kernels can
    read/write the ``[2, chunk, *row]`` host tensor ``t`` in place: each plane
    contiguous and 16-byte aligned, all of it in page-locked host memory
    mapped at its host address; else None."""
    if t.device.type != "cpu" or t.dim() < 3 or t.shape[0] != 2 or t.numel() == 0:
        return None
    shape, stride = t.shape, t.stride()
    expect = 1
    for d in range(t.dim() - 1, 0, -1):
        if shape[d] != 1 and stride[d] != expect:
            return None
        expect *= shape[d]
    es = t.element_size()
    plane = expect * es
    k = t.data_ptr()
    v = k + stride[0] * es
    if k % 16 or v % 16:
        return None
    lo, hi = min(k, v), max(k, v) + plane  # one storage, hence one allocation
    ok = ctypes.c_int32()
    _native.check(_native.load().cbk_host_accessible(lo, hi - lo, ctypes.byref(ok)), "host_accessible")
    if not ok.value:
        return None
    return k, v, (int(shape[1]), tuple(int(x) for x in shape[2:]), t.dtype)


class PinnedChunkSlab:
    """Chunk-sized pinned host slots from the native slab (``cbk_slab_*``).

    Each slot is a CPU tensor ``[2, chunk, *row]`` over pinned, coherent
    host memory that GPU kernels read and write directly. ``free`` with an
    event defers reuse until the event (the last GPU access) completes.
    The slab must outlive every tensor it handed out.
    """

    def __init__(self, chunk_shape: Sequence[int], dtype: torch.dtype, chunks_per_arena: int = 128,
                 max_bytes: int = 0):
        self.chunk_shape = tuple(int(d) for d in chunk_shape)
        self.dtype = dtype
        elem = torch.empty((), dtype=dtype).element_size()
        self.nbytes = math.prod(self.chunk_shape) * elem
        self.chunk_bytes = (self.nbytes + 255) // 256 * 256
        handle = ctypes.c_void_p()
        _native.check(_native.load().cbk_slab_create(self.chunk_bytes, chunks_per_arena, max_bytes,
                                                     ctypes.byref(handle)), "slab create")
        self._handle = handle
        self._lock = threading.Lock()
        self._pending: list[tuple[int, object]] = []
        self._tensors: dict[int, torch.Tensor] = {}  # slot address -> its tensor

    def _reclaim(self) -> None:
        keep = []
        lib = _native.load()
        for ptr, events in self._pending:
            if all(e.query() for e in events):
                _native.check(lib.cbk_slab_free(self._handle, ptr), "slab free")
            else:
                keep.append((ptr, events))
        self._pending = keep

    def alloc(self) -> torch.Tensor:
        """One free slot as a ``chunk_shape`` tensor. A slot keeps one tensor
        object for the slab's life, so recycling a slot costs no tensor
        construction."""
        with self._lock:
            if self._pending:
                self._reclaim()
            ptr = ctypes.c_void_p()
            _native.check(_native.load().cbk_slab_alloc(self._handle, ctypes.byref(ptr)), "slab alloc")
            tensor = self._tensors.get(ptr.value)
            if tensor is None:
                raw = (ctypes.c_uint8 * self.nbytes).from_address(ptr.value)
                tensor = torch.frombuffer(raw, dtype=torch.uint8).view(self.dtype).view(self.chunk_shape)
                self._tensors[ptr.value] = tensor
            return tensor

    def alloc_run(self, n: int) -> list[torch.Tensor]:
        """``n`` slots, consecutive in host memory whenever the slab can
        (``cbk_slab_alloc_run``), so one DMA copy can fill them in order."""
        with self._lock:
            if self._pending:
                self._reclaim()
            ptrs = (ctypes.c_void_p * n)()
            _native.check(_native.load().cbk_slab_alloc_run(self._handle, n, ptrs), "slab alloc_run")
            out = []
            for p in ptrs:
                tensor = self._tensors.get(p)
                if tensor is None:
                    raw = (ctypes.c_uint8 * self.nbytes).from_address(p)
                    tensor = torch.frombuffer(raw, dtype=torch.uint8).view(self.dtype).view(self.chunk_shape)
                    self._tensors[p] = tensor
                out.append(tensor)
            return out

    def free(self, tensor: torch.Tensor, event=None) -> None:
        """Give a slot back. ``event`` (a GPU event, or a sequence of them)
        marks the last GPU access: the slot is reused only once every one
        of them has completed."""
        events = tuple(e for e in (event if isinstance(event, (list, tuple)) else (event,))
                       if e is not None)
        with self._lock:
            self._pending.append((tensor.data_ptr(), events))
            self._reclaim()

    def stats(self) -> dict[str, int]:
        arenas, free, live = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
        _native.check(_native.load().cbk_slab_stats(self._handle, ctypes.byref(arenas), ctypes.byref(free),
                                                    ctypes.byref(live)), "slab stats")
        return {"arenas": arenas.value, "free": free.value, "live": live.value,
                "pending": len(self._pending)}

    def close(self) -> None:
        self._tensors.clear()
        if self._handle is not None:
            _native.check(_native.load().cbk_slab_destroy(self._handle), "slab destroy")
            self._handle = None


class PinnedChunkStore:
    def __init__(self, chunk_size: int, max_bytes: int,
                 on_release: Callable[[torch.Tensor, tuple], None] | None = None):
        if max_bytes <= 0:
            raise ValueError("max_bytes must be positive")
        self.chunk_size = int(chunk_size)
        self.max_bytes = int(max_bytes)
        # put_layer's host copies are page-locked (when a GPU runtime is there)
        self.pin_memory = True
        # called with every layer tensor the store drops (e.g. slab slots)
        # and the GPU events of loads that may still read it (see release)
        self._on_release = on_release
        # least recently used first (reference storage.py:42, 273-275)
        self._entries: OrderedDict[SegmentId, _Entry] = OrderedDict()
        self._pins: dict[str, tuple[SegmentId, ...]] = {}
        self._pin_sets: dict[str, frozenset[SegmentId]] = {}
        # request -> (segment tuple, [(id, entry)]) for layer_chunk_addresses
        self._pin_entries: dict[str, tuple] = {}
        self._bytes = 0
        self._lock = threading.RLock()
        # committed segments, found at any prompt offset by ``match``
        self.matcher = TokenRangeMatcher(self.chunk_size)

    @property
    def current_bytes(self) -> int:
        with self._lock:
            return self._bytes

    @property
    def committed_entries(self) -> int:
        return len(self.matcher)

    def begin_put(self, model_scope: str, source_start: int, tokens: Sequence[int],
                  num_layers: int) -> SegmentId:
        if num_layers <= 0:
            raise ValueError("num_layers must be positive")
        if len(tokens) != self.chunk_size:
            raise ValueError(f"fingerprint requires exactly {self.chunk_size} tokens, got {len(tokens)}")
        key = tuple(int(t) for t in tokens)
        sid = SegmentId(model_scope, content_hash(key), source_start, len(key))
        with self._lock:
            self._begin_locked(sid, key, num_layers)
        return sid

    def begin_put_chunks(self, model_scope: str, tokens: Sequence[int], start: int, end: int,
                         num_layers: int) -> list[SegmentId]:
        """``begin_put`` for every ``chunk_size`` chunk of ``tokens[start:end]``
        (source_start = the chunk's offset), hashing all of them in one
        native call."""
        if num_layers <= 0:
            raise ValueError("num_layers must be positive")
        c = self.chunk_size
        if start < 0 or end > len(tokens) or (end - start) % c:
            raise ValueError(f"[{start}, {end}) is not a whole number of {c}-token chunks of the prompt")
        if end <= start:
            return []
        values = as_token_array(tokens[start:end])
        hashes = rolling_hash_values(values, c)[::c].tolist()
        span = values.tolist()  # Python ints, for the collision check
        ids = []
        with self._lock:
            for i, value in enumerate(hashes):
                key = tuple(span[i * c:(i + 1) * c])
                sid = SegmentId(model_scope, int(value), start + i * c, c)
                self._begin_locked(sid, key, num_layers)
                ids.append(sid)
        return ids

    def _begin_locked(self, sid: SegmentId, key: tuple[int, ...], num_layers: int) -> None:
        entry = self._entries.get(sid)
        if entry is None:
            self._entries[sid] = _Entry(num_layers, key)
        else:
            if entry.tokens != key:
                raise RuntimeError("content-hash collision for an existing segment id")
            if entry.num_layers != num_layers:
                raise ValueError("num_layers changed for an existing segment")
            self._entries.move_to_end(sid)

    def cancel_layer(self, segment_id: SegmentId, layer_id: int) -> None:
        """Give up a reserved layer: an uncommitted segment fails as a unit
        (reference storage.py:120-129)."""
        with self._lock:
            entry = self._entries.get(segment_id)
            if entry is None:
                return
            entry.reserved.discard(layer_id)
            if not entry.committed:
                entry.failed = True
            if entry.failed:
                self._drop_if_idle(segment_id, entry)

    def put_layer(self, segment_id: SegmentId, layer_id: int, kv: torch.Tensor) -> bool | None:
        """Copy one layer ``[2, chunk, *row]`` (any device) into fresh host
        memory, page-locked unless ``pin_memory`` is off, and publish it
        (reference storage.py:78-102)."""
        with self._lock:
            entry = self._entries.get(segment_id)
            if entry is None:
                raise KeyError(segment_id)
            if not 0 <= layer_id < entry.num_layers:
                raise ValueError(f"layer {layer_id} is outside [0, {entry.num_layers})")
        host = torch.empty(kv.shape, dtype=kv.dtype, pin_memory=self.pin_memory and torch.cuda.is_available())
        host.copy_(kv.detach())
        return self.put_layer_host(segment_id, layer_id, host)

    def reserve_layer(self, segment_id: SegmentId, layer_id: int) -> bool:
        with self._lock:
            return self._reserve_locked(segment_id, layer_id)

    def reserve_layers(self, segment_ids: Sequence[SegmentId], layer_id: int) -> list[bool]:
        """``reserve_layer`` for each segment under one lock acquisition."""
        with self._lock:
            return [self._reserve_locked(sid, layer_id) for sid in segment_ids]

    def _reserve_locked(self, segment_id: SegmentId, layer_id: int) -> bool:
        entry = self._entries.get(segment_id)
        if entry is None:
            return False
        if not 0 <= layer_id < entry.num_layers:
            raise ValueError(f"layer {layer_id} is outside [0, {entry.num_layers})")
        if entry.failed or layer_id in entry.layers or layer_id in entry.reserved:
            return False
        entry.reserved.add(layer_id)
        return True

    def put_layer_host(self, segment_id: SegmentId, layer_id: int,
                       cpu_tensor: torch.Tensor) -> bool | None:
        """Publish a host tensor (or view) for one layer; True when the
        segment became committed, None when it was rejected."""
        if cpu_tensor.device.type != "cpu":
            raise ValueError("put_layer_host requires a CPU tensor")
        with self._lock:
            entry = self._entries.get(segment_id)
            if entry is None:
                return None
            if not 0 <= layer_id < entry.num_layers:
                raise ValueError(f"layer {layer_id} is outside [0, {entry.num_layers})")
            if entry.failed:
                entry.reserved.discard(layer_id)
                self._drop_if_idle(segment_id, entry)
                return None
            if entry.committed:
                entry.reserved.discard(layer_id)
                return False
            added = cpu_tensor.numel() * cpu_tensor.element_size()
            previous = entry.layers.get(layer_id)
            growth = added - (previous.numel() * previous.element_size() if previous is not None else 0)
            if growth > 0:
                self._evict(growth, exclude=segment_id)
            if self._bytes + growth > self.max_bytes:
                entry.reserved.discard(layer_id)
                entry.failed = True
                self._drop_if_idle(segment_id, entry)
                return None
            entry.reserved.discard(layer_id)
            if previous is not None and self._on_release is not None:
                self._on_release(previous, tuple(entry.read_events))
            entry.layers[layer_id] = cpu_tensor
            entry.addresses.pop(layer_id, None)
            entry.size_bytes += growth
            self._bytes += growth
            self._entries.move_to_end(segment_id)
            if len(entry.layers) == entry.num_layers:
                entry.committed = True
                self.matcher.register(FingerprintRecord(segment_id, entry.tokens))
                return True
            return False

    def abort_put(self, segment_id: SegmentId) -> None:
        with self._lock:
            entry = self._entries.get(segment_id)
            if entry is None or entry.committed:
                return
            entry.failed = True
            self._drop_if_idle(segment_id, entry)

    def holds(self, segment_id: SegmentId, layer_id: int, tensor: torch.Tensor) -> bool:
        """Whether the store kept ``tensor`` as that segment layer."""
        with self._lock:
            entry = self._entries.get(segment_id)
            return entry is not None and entry.layers.get(layer_id) is tensor

    def is_committed(self, segment_id: SegmentId) -> bool:
        with self._lock:
            entry = self._entries.get(segment_id)
            return entry is not None and entry.committed

    def match(self, model_scope: str, tokens: Sequence[int],
              start_offset: int) -> tuple[BlendSegment, ...]:
        """Committed segments found in ``tokens[start_offset:]``, leftmost
        first and non-overlapping (reference storage.py:201-208)."""
        return self.validate(self.matcher.match(model_scope, tokens, start_offset))

    def validate(self, segments: Iterable[BlendSegment]) -> tuple[BlendSegment, ...]:
        """The committed subset of ``segments`` (reference storage.py:210-219)."""
        valid = []
        with self._lock:
            for seg in segments:
                entry = self._entries.get(seg.segment_id)
                if entry is None or not entry.committed:
                    continue
                self._entries.move_to_end(seg.segment_id)
                valid.append(seg)
        return tuple(valid)

    def pin(self, request_id: str, segments: Iterable[BlendSegment]) -> tuple[BlendSegment, ...]:
        requested = tuple(segments)
        with self._lock:
            self.release(request_id)
            valid = []
            for seg in requested:
                entry = self._entries.get(seg.segment_id)
                if entry is None or not entry.committed:
                    continue
                entry.pins += 1
                self._entries.move_to_end(seg.segment_id)
                valid.append(seg)
            if valid:
                self._pins[request_id] = tuple(s.segment_id for s in valid)
                self._pin_sets[request_id] = frozenset(self._pins[request_id])
            return tuple(valid)

    def release(self, request_id: str, event=None) -> None:
        """Drop ``request_id``'s pins. ``event``: a GPU event recorded after
        the request's last read of the pinned chunks (a load still in
        flight); chunks dropped later keep it, so their host memory is not
        reused before the read completes."""
        with self._lock:
            self._pin_sets.pop(request_id, None)
            self._pin_entries.pop(request_id, None)
            for sid in self._pins.pop(request_id, ()):
                entry = self._entries.get(sid)
                if entry is not None:
                    entry.pins = max(0, entry.pins - 1)
                    if event is not None:
                        entry.read_events = [e for e in entry.read_events if not e.query()]
                        entry.read_events.append(event)
            self._evict(0)

    def get_layer(self, request_id: str, segment: BlendSegment, layer_id: int) -> torch.Tensor:
        with self._lock:
            if segment.segment_id not in self._pin_sets.get(request_id, ()):
                raise RuntimeError(f"segment {segment.segment_id} is not pinned by {request_id}")
            entry = self._entries.get(segment.segment_id)
            if entry is None or not entry.committed:
                raise KeyError(segment.segment_id)
            try:
                tensor = entry.layers[layer_id]
            except KeyError as error:
                raise KeyError(f"layer {layer_id} is not stored for {segment.segment_id}") from error
            self._entries.move_to_end(segment.segment_id)
            return tensor

    def layer_chunk_addresses(self, request_id: str, segments: Sequence[BlendSegment],
                              layer_id: int) -> tuple[tuple, list[int]] | None:
        """``(geometry, [k0, v0, k1, v1, ...])``: in-place host addresses of
        one layer of pinned segments, for kernels that read the chunks over
        the host link, with their common ``(chunk_tokens, row_shape, dtype)``;
        None when any chunk is not kernel-addressable (``chunk_address``) or
        the geometries differ. Each stored chunk is validated once; the
        segments' entries are looked up (and touched for the LRU order) once
        per request and segment tuple: a loader asks for every layer of the
        same plan, and pinned entries stay put until ``release``."""
        with self._lock:
            cached = self._pin_entries.get(request_id)
            if cached is not None and cached[0] is segments:
                entries = cached[1]
            else:
                pinned = self._pin_sets.get(request_id, ())
                entries = []
                for seg in segments:
                    if seg.segment_id not in pinned:
                        raise RuntimeError(f"segment {seg.segment_id} is not pinned by {request_id}")
                    entry = self._entries.get(seg.segment_id)
                    if entry is None or not entry.committed:
                        raise KeyError(seg.segment_id)
                    self._entries.move_to_end(seg.segment_id)
                    entries.append((seg.segment_id, entry))
                if request_id in self._pin_sets and isinstance(segments, tuple):
                    self._pin_entries[request_id] = (segments, entries)
            flat: list[int] = []
            geometry = None
            for sid, entry in entries:
                info = entry.addresses.get(layer_id, False)
                if info is False:
                    tensor = entry.layers.get(layer_id)
                    if tensor is None:
                        raise KeyError(f"layer {layer_id} is not stored for {sid}")
                    info = entry.addresses[layer_id] = chunk_address(tensor)
                if info is None or (geometry is not None and info[2] != geometry):
                    return None
                geometry = info[2]
                flat.append(info[0])
                flat.append(info[1])
            return (geometry, flat) if geometry is not None else None

    def clear(self) -> None:
        with self._lock:
            for sid, entry in self._entries.items():
                self.matcher.unregister(sid)
                self._release_layers(entry)
            self._entries.clear()
            self._pins.clear()
            self._pin_sets.clear()
            self._pin_entries.clear()
            self._bytes = 0

    def _release_layers(self, entry: _Entry) -> None:
        if self._on_release is not None:
            events = tuple(entry.read_events)
            for tensor in entry.layers.values():
                self._on_release(tensor, events)
        entry.layers.clear()
        entry.addresses.clear()
        entry.read_events.clear()

    def _evict(self, required_bytes: int, exclude: SegmentId | None = None) -> None:
        """Drop least recently used committed, unpinned segments until
        ``required_bytes`` more fit (reference storage.py:282-294)."""
        if self._bytes + required_bytes <= self.max_bytes:
            return
        for sid, entry in list(self._entries.items()):
            if self._bytes + required_bytes <= self.max_bytes:
                break
            if sid == exclude or entry.pins or not entry.committed:
                continue
            self._entries.pop(sid, None)
            self.matcher.unregister(sid)
            self._bytes -= entry.size_bytes
            self._release_layers(entry)

    def _drop_if_idle(self, segment_id: SegmentId, entry: _Entry) -> None:
        if not entry.reserved and not entry.pins:
            self._entries.pop(segment_id, None)
            self.matcher.unregister(segment_id)
            self._bytes -= entry.size_bytes
            self._release_layers(entry)
