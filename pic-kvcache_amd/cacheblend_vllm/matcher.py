"""Content-addressed token-range matcher (reference cacheblend_vllm/matcher.py).

``TokenRangeMatcher`` finds registered ``chunk_size``-token chunks at every
offset of a prompt: leftmost-greedy, non-overlapping, each candidate window
verified token for token, so a hash collision never yields a match
(reference matcher.py:80-125). Same class, method names, argument meaning
and errors as the reference. The records live in the native library
(``cbk_matcher_*``): window hashes come from the O(n) rolling update and
candidates are compared with one memcmp each, instead of a per-candidate
Python tuple. This object keeps the segment-id <-> record-key mapping.
"""

from __future__ import annotations

import ctypes
import threading
from collections.abc import Iterable, Sequence
from dataclasses import dataclass

import numpy as np

from . import _native
from .hashing import as_token_array, content_hash
from .types import BlendSegment, SegmentId


@dataclass(frozen=True, slots=True)
class FingerprintRecord:
    segment_id: SegmentId
    tokens: tuple[int, ...]


class TokenRangeMatcher:
    """Match fixed-size stored chunks at every query-token offset."""

    def __init__(self, chunk_size: int):
        if chunk_size <= 0:
            raise ValueError("chunk_size must be positive")
        self.chunk_size = int(chunk_size)
        self._lib = _native.load()
        handle = ctypes.c_void_p()
        _native.check(self._lib.cbk_matcher_create(self.chunk_size, ctypes.byref(handle)),
                      "TokenRangeMatcher")
        self._handle = handle.value
        self._by_id: dict[SegmentId, tuple[int, FingerprintRecord]] = {}
        self._by_key: dict[int, FingerprintRecord] = {}
        self._scopes: dict[str, int] = {}
        self._next_key = 1
        self._lock = threading.RLock()

    def __del__(self):
        handle = getattr(self, "_handle", None)
        if handle:
            self._handle = None
            self._lib.cbk_matcher_destroy(handle)

    def _scope_id(self, model_scope: str) -> int:
        scope = self._scopes.get(model_scope)
        if scope is None:
            scope = self._scopes[model_scope] = len(self._scopes) + 1
        return scope

    def make_record(self, model_scope: str, source_start: int,
                    tokens: Sequence[int]) -> FingerprintRecord:
        """A chunk's record, keyed as the store keys it (reference
        matcher.py:34-51): the id is (scope, content hash of the tokens as
        Python ints, start, length), and only whole ``chunk_size`` chunks
        have one."""
        chunk = tuple(map(int, tokens))
        if len(chunk) != self.chunk_size:
            raise ValueError(
                f"fingerprint requires exactly {self.chunk_size} tokens, got {len(chunk)}"
            )
        sid = SegmentId(model_scope, content_hash(chunk), source_start, self.chunk_size)
        return FingerprintRecord(sid, chunk)

    def register(self, record: FingerprintRecord) -> None:
        """Reference matcher.py:53-63: re-registering an identical record is a
        no-op; a changed record for the same id replaces the old one. A
        record whose length is not ``chunk_size`` is kept but can never match
        (as in the reference, whose windows are ``chunk_size`` long)."""
        sid = record.segment_id
        with self._lock:
            previous = self._by_id.get(sid)
            if previous is not None and previous[1] == record:
                return
            if previous is not None:
                self.unregister(sid)
            key = self._next_key
            self._next_key += 1
            if len(record.tokens) == self.chunk_size:
                tokens = as_token_array(record.tokens)
                _native.check(
                    self._lib.cbk_matcher_register(self._handle, self._scope_id(sid.model_scope), key,
                                                   sid.content_hash & ((1 << 64) - 1),
                                                   tokens.ctypes.data),
                    "TokenRangeMatcher.register",
                )
            self._by_id[sid] = (key, record)
            self._by_key[key] = record

    def unregister(self, segment_id: SegmentId) -> None:
        """Reference matcher.py:65-78."""
        with self._lock:
            entry = self._by_id.pop(segment_id, None)
            if entry is None:
                return
            key, _ = entry
            del self._by_key[key]
            _native.check(self._lib.cbk_matcher_unregister(self._handle, key),
                          "TokenRangeMatcher.unregister")

    def match(self, model_scope: str, tokens: Sequence[int],
              start_offset: int = 0) -> tuple[BlendSegment, ...]:
        """Return leftmost-greedy, non-overlapping exact token matches
        (reference matcher.py:80-125)."""
        if start_offset < 0 or start_offset > len(tokens):
            raise ValueError("start_offset is outside the token sequence")
        with self._lock:
            scope = self._scopes.get(model_scope)
            if scope is None or not self._by_key:
                return ()
            values = as_token_array(tokens)
            n = values.shape[0]
            capacity = max(1, (n - start_offset) // self.chunk_size + 1)
            starts = np.empty(capacity, dtype=np.int64)
            keys = np.empty(capacity, dtype=np.uint64)
            count = ctypes.c_int64()
            _native.check(
                self._lib.cbk_matcher_match(self._handle, scope, values.ctypes.data, n, start_offset,
                                            starts.ctypes.data, keys.ctypes.data, capacity,
                                            ctypes.byref(count)),
                "TokenRangeMatcher.match",
            )
            return tuple(
                BlendSegment(segment_id=self._by_key[int(keys[i])].segment_id,
                             target_start=int(starts[i]))
                for i in range(count.value)
            )

    def validate(self, segments: Iterable[BlendSegment]) -> tuple[BlendSegment, ...]:
        """Reference matcher.py:127-129."""
        with self._lock:
            return tuple(segment for segment in segments if segment.segment_id in self._by_id)

    def __len__(self) -> int:
        with self._lock:
            return len(self._by_id)
