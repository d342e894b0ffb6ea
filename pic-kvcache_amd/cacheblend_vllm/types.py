"""Blend plan types: the input format of the load and selection path.

Field names, invariants and error messages follow the reference
(cacheblend_vllm/types.py:10-163) so plans built by the reference scheduler
are accepted unchanged. A plan describes one request's blend span:
``[apc_prefix_tokens, allocation_end)``, holding sorted, non-overlapping hit
segments; every other token of the span is a gap.
"""

from __future__ import annotations

from collections.abc import Iterable
from dataclasses import dataclass, field
from typing import Any


@dataclass(frozen=True, order=True, slots=True)
class SegmentId:
    model_scope: str
    content_hash: int
    source_start: int
    token_count: int

    def __post_init__(self) -> None:
        if not self.model_scope:
            raise ValueError("model_scope cannot be empty")
        if self.source_start < 0 or self.token_count <= 0:
            raise ValueError("invalid source segment")

    def to_dict(self) -> dict[str, Any]:
        return {
            "model_scope": self.model_scope,
            "content_hash": self.content_hash,
            "source_start": self.source_start,
            "token_count": self.token_count,
        }

    @classmethod
    def from_dict(cls, value: dict[str, Any]) -> "SegmentId":
        return cls(
            str(value["model_scope"]),
            int(value["content_hash"]),
            int(value["source_start"]),
            int(value["token_count"]),
        )


@dataclass(frozen=True, order=True, slots=True)
class BlendSegment:
    segment_id: SegmentId
    target_start: int

    def __post_init__(self) -> None:
        if self.target_start < 0:
            raise ValueError("target_start cannot be negative")

    @property
    def source_start(self) -> int:
        return self.segment_id.source_start

    @property
    def length(self) -> int:
        return self.segment_id.token_count

    @property
    def target_end(self) -> int:
        return self.target_start + self.length

    def to_dict(self) -> dict[str, Any]:
        return {"segment_id": self.segment_id.to_dict(), "target_start": self.target_start}

    @classmethod
    def from_dict(cls, value: dict[str, Any]) -> "BlendSegment":
        return cls(SegmentId.from_dict(value["segment_id"]), int(value["target_start"]))


@dataclass(frozen=True, slots=True)
class BlendPlan:
    apc_prefix_tokens: int
    allocation_end: int
    hit_tokens: int
    segments: tuple[BlendSegment, ...] = field(default_factory=tuple)

    def __post_init__(self) -> None:
        if self.apc_prefix_tokens < 0 or self.allocation_end < self.apc_prefix_tokens:
            raise ValueError("invalid CacheBlend allocation span")
        ordered = tuple(sorted(self.segments, key=lambda s: s.target_start))
        cursor = self.apc_prefix_tokens
        total = 0
        for seg in ordered:
            if seg.target_start < self.apc_prefix_tokens:
                raise ValueError("segments must start after the APC prefix")
            if seg.target_start < cursor:
                raise ValueError("segments cannot overlap")
            if seg.target_end > self.allocation_end:
                raise ValueError("segment exceeds allocation span")
            total += seg.length
            cursor = seg.target_end
        if total != self.hit_tokens:
            raise ValueError(f"hit_tokens={self.hit_tokens} does not match segments={total}")
        if ordered != self.segments:
            raise ValueError("segments must be sorted")

    @classmethod
    def from_segments(cls, apc_prefix_tokens: int, segments: Iterable[BlendSegment]) -> "BlendPlan":
        ordered = tuple(sorted(set(segments), key=lambda s: s.target_start))
        if not ordered:
            return cls(apc_prefix_tokens, apc_prefix_tokens, 0, ())
        return cls(
            apc_prefix_tokens,
            max(s.target_end for s in ordered),
            sum(s.length for s in ordered),
            ordered,
        )

    @property
    def allocation_tokens(self) -> int:
        return self.allocation_end - self.apc_prefix_tokens

    @property
    def gap_tokens(self) -> int:
        return self.allocation_tokens - self.hit_tokens

    def passes_gate(
        self,
        min_retrieve_tokens: int,
        min_hit_ratio: float,
        min_saved_tokens: int,
        max_apc_prefix_to_hit_ratio: float = 0.0,
    ) -> bool:
        if self.hit_tokens < min_retrieve_tokens or self.hit_tokens < min_saved_tokens:
            return False
        if self.hit_tokens / max(self.allocation_tokens, 1) < min_hit_ratio:
            return False
        return not (
            max_apc_prefix_to_hit_ratio > 0
            and self.apc_prefix_tokens / max(self.hit_tokens, 1) > max_apc_prefix_to_hit_ratio
        )

    def gap_runs(self) -> list[tuple[int, int]]:
        """Half-open gap ranges of the span (what the loader zeroes)."""
        runs = []
        cursor = self.apc_prefix_tokens
        for seg in self.segments:
            if seg.target_start > cursor:
                runs.append((cursor, seg.target_start))
            cursor = max(cursor, seg.target_end)
        if cursor < self.allocation_end:
            runs.append((cursor, self.allocation_end))
        return runs

    def to_dict(self) -> dict[str, Any]:
        return {
            "apc_prefix_tokens": self.apc_prefix_tokens,
            "allocation_end": self.allocation_end,
            "hit_tokens": self.hit_tokens,
            "segments": [s.to_dict() for s in self.segments],
        }

    @classmethod
    def from_dict(cls, value: dict[str, Any]) -> "BlendPlan":
        return cls(
            int(value["apc_prefix_tokens"]),
            int(value["allocation_end"]),
            int(value["hit_tokens"]),
            tuple(BlendSegment.from_dict(s) for s in value.get("segments", [])),
        )
