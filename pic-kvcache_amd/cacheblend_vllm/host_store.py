"""Pinned host chunk store: the part of the reference store the KV path uses.

The store/load kernels exchange KV with host memory in the reference's
chunk format: per segment (one ``chunk_size``-token chunk) and layer, a host
tensor ``[2, chunk, *row]`` whose K and V planes are each contiguous -- in
practice a view ``host[:, off:off + chunk]`` of one pinned per-layer batch
(reference connector.py:449-466). This class keeps that contract and the
method names/semantics the save and load paths call on
``LocalPinnedCPUStore`` (reference storage.py:56-263): ``begin_put``,
``reserve_layer``, ``put_layer_host``, ``abort_put``, ``pin``, ``release``,
``get_layer``. Commit happens when every layer is present; a failed or
aborted segment is dropped as a unit; the byte cap is fail-closed.
The content-addressed matcher, LRU eviction and lookup RPC are the
scheduler's control plane and are not part of this package.
"""

from __future__ import annotations

import threading
from collections.abc import Iterable, Sequence
from dataclasses import dataclass, field

import torch

from .types import BlendSegment, SegmentId

MASK64 = (1 << 64) - 1
POLY_BASE = 1_000_003


def content_hash(tokens: Sequence[int]) -> int:
    """Polynomial token hash mod 2^64 (reference hashing.py:10-22)."""
    value = 0
    for token in tokens:
        value = (value * POLY_BASE + ((int(token) + 1) & MASK64)) & MASK64
    return value


@dataclass
class _Entry:
    num_layers: int
    layers: dict[int, torch.Tensor] = field(default_factory=dict)
    reserved: set[int] = field(default_factory=set)
    size_bytes: int = 0
    pins: int = 0
    committed: bool = False
    failed: bool = False


class PinnedChunkStore:
    def __init__(self, chunk_size: int, max_bytes: int):
        if max_bytes <= 0:
            raise ValueError("max_bytes must be positive")
        self.chunk_size = int(chunk_size)
        self.max_bytes = int(max_bytes)
        self._entries: dict[SegmentId, _Entry] = {}
        self._pins: dict[str, tuple[SegmentId, ...]] = {}
        self._bytes = 0
        self._lock = threading.RLock()

    @property
    def current_bytes(self) -> int:
        return self._bytes

    def begin_put(self, model_scope: str, source_start: int, tokens: Sequence[int],
                  num_layers: int) -> SegmentId:
        if num_layers <= 0:
            raise ValueError("num_layers must be positive")
        if len(tokens) != self.chunk_size:
            raise ValueError(f"fingerprint requires exactly {self.chunk_size} tokens, got {len(tokens)}")
        sid = SegmentId(model_scope, content_hash(tokens), source_start, len(tokens))
        with self._lock:
            entry = self._entries.get(sid)
            if entry is None:
                self._entries[sid] = _Entry(num_layers)
            elif entry.num_layers != num_layers:
                raise ValueError("num_layers changed for an existing segment")
        return sid

    def reserve_layer(self, segment_id: SegmentId, layer_id: int) -> bool:
        with self._lock:
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
            if self._bytes + growth > self.max_bytes:
                entry.reserved.discard(layer_id)
                entry.failed = True
                self._drop_if_idle(segment_id, entry)
                return None
            entry.reserved.discard(layer_id)
            entry.layers[layer_id] = cpu_tensor
            entry.size_bytes += growth
            self._bytes += growth
            if len(entry.layers) == entry.num_layers:
                entry.committed = True
                return True
            return False

    def abort_put(self, segment_id: SegmentId) -> None:
        with self._lock:
            entry = self._entries.get(segment_id)
            if entry is None or entry.committed:
                return
            entry.failed = True
            self._drop_if_idle(segment_id, entry)

    def is_committed(self, segment_id: SegmentId) -> bool:
        entry = self._entries.get(segment_id)
        return entry is not None and entry.committed

    def pin(self, request_id: str, segments: Iterable[BlendSegment]) -> tuple[BlendSegment, ...]:
        with self._lock:
            self.release(request_id)
            valid = []
            for seg in segments:
                entry = self._entries.get(seg.segment_id)
                if entry is None or not entry.committed:
                    continue
                entry.pins += 1
                valid.append(seg)
            if valid:
                self._pins[request_id] = tuple(s.segment_id for s in valid)
            return tuple(valid)

    def release(self, request_id: str) -> None:
        with self._lock:
            for sid in self._pins.pop(request_id, ()):
                entry = self._entries.get(sid)
                if entry is not None:
                    entry.pins = max(0, entry.pins - 1)

    def get_layer(self, request_id: str, segment: BlendSegment, layer_id: int) -> torch.Tensor:
        with self._lock:
            if segment.segment_id not in self._pins.get(request_id, ()):
                raise RuntimeError(f"segment {segment.segment_id} is not pinned by {request_id}")
            entry = self._entries.get(segment.segment_id)
            if entry is None or not entry.committed:
                raise KeyError(segment.segment_id)
            try:
                return entry.layers[layer_id]
            except KeyError as error:
                raise KeyError(f"layer {layer_id} is not stored for {segment.segment_id}") from error

    def clear(self) -> None:
        with self._lock:
            self._entries.clear()
            self._pins.clear()
            self._bytes = 0

    def _drop_if_idle(self, segment_id: SegmentId, entry: _Entry) -> None:
        if not entry.reserved and not entry.pins:
            self._entries.pop(segment_id, None)
            self._bytes -= entry.size_bytes
