"""Blend plan types: the input format of the load and selection path.

A plan describes one request's blend span ``[apc_prefix_tokens,
allocation_end)``: the hit segments (cached chunks placed at target
positions, sorted and non-overlapping) and, implicitly, the gaps between
them. The field names, the dict wire format and the validation messages are
the interface of the reference's plan types (cacheblend_vllm/types.py:10-141),
so plans and segment ids produced by the reference scheduler load unchanged.
The scheduler's admission gate is control plane and is not part of this
package.
"""

from __future__ import annotations

from collections.abc import Iterable
from dataclasses import astuple, dataclass, field
from operator import attrgetter
from typing import Any

_by_target = attrgetter("target_start")


@dataclass(frozen=True, order=True, slots=True)
class SegmentId:
    """Identity of one stored chunk: model scope, content hash of its
    tokens, where it started in the prompt that stored it, its length."""

    model_scope: str
    content_hash: int
    source_start: int
    token_count: int

    def __post_init__(self) -> None:
        if not self.model_scope:
            raise ValueError("model_scope cannot be empty")
        if min(self.source_start, self.token_count - 1) < 0:
            raise ValueError("invalid source segment")

    def to_dict(self) -> dict[str, Any]:
        names = ("model_scope", "content_hash", "source_start", "token_count")
        return dict(zip(names, astuple(self)))

    @classmethod
    def from_dict(cls, value: dict[str, Any]) -> SegmentId:
        scope, digest, start, count = (value[k] for k in
                                       ("model_scope", "content_hash", "source_start", "token_count"))
        return cls(str(scope), int(digest), int(start), int(count))


@dataclass(frozen=True, order=True, slots=True)
class BlendSegment:
    """A stored chunk placed at ``target_start`` of the current prompt."""

    segment_id: SegmentId
    target_start: int

    def __post_init__(self) -> None:
        if self.target_start < 0:
            raise ValueError("target_start cannot be negative")

    source_start = property(lambda self: self.segment_id.source_start)
    length = property(lambda self: self.segment_id.token_count)
    target_end = property(lambda self: self.target_start + self.segment_id.token_count)

    def to_dict(self) -> dict[str, Any]:
        return {"segment_id": self.segment_id.to_dict(), "target_start": self.target_start}

    @classmethod
    def from_dict(cls, value: dict[str, Any]) -> BlendSegment:
        return cls(SegmentId.from_dict(value["segment_id"]), int(value["target_start"]))


def _plan_error(apc: int, end: int, hit_tokens: int, segments: tuple[BlendSegment, ...]) -> str | None:
    """The first rule a plan breaks, or None. Segments are checked in target
    order, each against the APC prefix, the end of the one before it and the
    span end; then the hit count, then that they were given sorted."""
    if apc < 0 or end < apc:
        return "invalid CacheBlend allocation span"
    ordered = sorted(segments, key=_by_target)
    previous_ends = [apc] + [seg.target_end for seg in ordered]
    for seg, previous_end in zip(ordered, previous_ends):
        if seg.target_start < apc:
            return "segments must start after the APC prefix"
        if seg.target_start < previous_end:
            return "segments cannot overlap"
        if seg.target_end > end:
            return "segment exceeds allocation span"
    covered = sum(seg.length for seg in ordered)
    if covered != hit_tokens:
        return f"hit_tokens={hit_tokens} does not match segments={covered}"
    if tuple(ordered) != segments:
        return "segments must be sorted"
    return None


@dataclass(frozen=True, slots=True)
class BlendPlan:
    """One request's blend span and the hit segments inside it."""

    apc_prefix_tokens: int
    allocation_end: int
    hit_tokens: int
    segments: tuple[BlendSegment, ...] = field(default_factory=tuple)

    def __post_init__(self) -> None:
        error = _plan_error(self.apc_prefix_tokens, self.allocation_end, self.hit_tokens,
                            tuple(self.segments))
        if error is not None:
            raise ValueError(error)

    @classmethod
    def from_segments(cls, apc_prefix_tokens: int, segments: Iterable[BlendSegment]) -> BlendPlan:
        """The tightest plan holding ``segments`` (duplicates dropped): its
        span ends where the last segment ends."""
        unique = tuple(sorted(set(segments), key=_by_target))
        end = max((seg.target_end for seg in unique), default=apc_prefix_tokens)
        return cls(apc_prefix_tokens, end, sum(seg.length for seg in unique), unique)

    @property
    def allocation_tokens(self) -> int:
        return self.allocation_end - self.apc_prefix_tokens

    @property
    def gap_tokens(self) -> int:
        return self.allocation_tokens - self.hit_tokens

    def gap_runs(self) -> list[tuple[int, int]]:
        """Half-open ``[start, end)`` ranges of the span no segment covers
        (the rows the loader zeroes)."""
        bounds = [self.apc_prefix_tokens]
        for seg in self.segments:
            bounds += [seg.target_start, seg.target_end]
        bounds.append(self.allocation_end)
        return [(a, b) for a, b in zip(bounds[0::2], bounds[1::2]) if b > a]

    def to_dict(self) -> dict[str, Any]:
        return {
            "apc_prefix_tokens": self.apc_prefix_tokens,
            "allocation_end": self.allocation_end,
            "hit_tokens": self.hit_tokens,
            "segments": [seg.to_dict() for seg in self.segments],
        }

    @classmethod
    def from_dict(cls, value: dict[str, Any]) -> BlendPlan:
        segments = tuple(map(BlendSegment.from_dict, value.get("segments", ())))
        return cls(int(value["apc_prefix_tokens"]), int(value["allocation_end"]),
                   int(value["hit_tokens"]), segments)
