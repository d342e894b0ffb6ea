"""CacheBlend connector configuration (the hot path's knobs).

Same field names, defaults and validation errors as the reference
``CacheBlendConfig`` (cacheblend_vllm/config.py:10-96), so an existing
``kv_connector_extra_config`` JSON loads unchanged; unknown fields are an
error there and here, so a config written for one loads in the other. The
MI355X loader's one extra knob, the depth of its device ring of hit
stagings, is read from the environment (``load_staging_layers``) instead of
being a field.
"""

from __future__ import annotations

from dataclasses import dataclass, fields
import os
from typing import Any

# Layers of hit staging one request's DMA ring holds on the device (at least
# 2, default 4). Not a config field: the reference's unknown-field rule
# would reject a config that names it.
LOAD_STAGING_LAYERS_ENV = "CACHEBLEND_LOAD_STAGING_LAYERS"


def load_staging_layers() -> int:
    """``CACHEBLEND_LOAD_STAGING_LAYERS`` (default 4, at least 2)."""
    raw = os.environ.get(LOAD_STAGING_LAYERS_ENV, "").strip()
    if not raw:
        return 4
    try:
        value = int(raw)
    except ValueError:
        raise ValueError(f"{LOAD_STAGING_LAYERS_ENV} must be an integer, got {raw!r}") from None
    if value < 2:
        raise ValueError(f"{LOAD_STAGING_LAYERS_ENV} must be at least 2, got {value}")
    return value


@dataclass(frozen=True, slots=True)
class CacheBlendConfig:
    chunk_size: int = 256
    local_cpu_gb: float = 16.0
    min_retrieve_tokens: int = 256
    min_hit_ratio: float = 0.10
    min_saved_tokens: int = 0
    max_apc_prefix_to_hit_ratio: float = 0.0
    check_layers: tuple[int, ...] = (1,)
    recompute_ratios: tuple[float, ...] = (0.15,)
    selection_strategy: str = "kv_deviation"
    query_score_chunk_size: int = 8
    overflow_blocks: int = 1
    tail_query_tokens: int = 64
    save_decode_cache: bool = False
    tp_global_selection: bool = True
    event_pipeline: bool = True
    fused_segment_copy: bool = True
    cache_attention_mask: bool = True
    lookup_timeout_ms: int = 10_000
    store_workers: int = 1
    max_inflight_store_batches: int = 8
    strict_version_check: bool = True
    ipc_root: str = "/tmp/cacheblend-v1"
    model_scope: str | None = None

    @classmethod
    def from_extra_config(cls, values: dict[str, Any] | None) -> "CacheBlendConfig":
        raw = dict(values or {})
        names = {f.name for f in fields(cls)}
        unknown = sorted(set(raw) - names)
        if unknown:
            raise ValueError(f"Unknown CacheBlend config fields: {unknown}")
        for name in ("check_layers", "recompute_ratios"):
            if name in raw:
                value = raw[name]
                raw[name] = tuple([value] if isinstance(value, (int, float)) else value)
        config = cls(**raw)
        config.validate()
        return config

    def validate(self) -> None:
        checks = (
            (self.chunk_size > 0, "chunk_size must be positive"),
            (self.local_cpu_gb > 0, "local_cpu_gb must be positive"),
            (self.min_retrieve_tokens >= 0 and self.min_saved_tokens >= 0,
             "token thresholds cannot be negative"),
            (0.0 <= self.min_hit_ratio <= 1.0, "min_hit_ratio must be between 0 and 1"),
            (self.max_apc_prefix_to_hit_ratio >= 0,
             "max_apc_prefix_to_hit_ratio cannot be negative"),
            (self.lookup_timeout_ms > 0, "lookup_timeout_ms must be positive"),
            (self.store_workers > 0, "store_workers must be positive"),
            (self.max_inflight_store_batches > 0, "max_inflight_store_batches must be positive"),
            (bool(self.check_layers), "at least one check layer is required"),
            (len(self.recompute_ratios) in (1, len(self.check_layers)),
             "recompute_ratios must contain one value or one per check layer"),
            (all(layer >= 0 for layer in self.check_layers),
             "check layer indices cannot be negative"),
            (all(0.0 <= r <= 1.0 for r in self.recompute_ratios),
             "recompute ratios must be between 0 and 1"),
            (self.selection_strategy in {"kv_deviation", "sparse_q", "compare"},
             "selection_strategy must be kv_deviation, sparse_q, or compare"),
            (self.selection_strategy == "kv_deviation" or len(self.check_layers) == 1,
             "Sparse-Q selection requires exactly one check layer"),
            (self.query_score_chunk_size > 0, "query_score_chunk_size must be positive"),
            (self.overflow_blocks >= 0, "overflow_blocks cannot be negative"),
            (self.tail_query_tokens >= 0, "tail_query_tokens cannot be negative"),
            (self.selection_strategy == "kv_deviation" or self.tail_query_tokens > 0,
             "Sparse-Q selection requires tail_query_tokens > 0"),
        )
        for ok, message in checks:
            if not ok:
                raise ValueError(message)

    @property
    def max_local_cpu_bytes(self) -> int:
        return int(self.local_cpu_gb * 1024**3)

    def ratio_for(self, layer_id: int | None) -> float:
        """Recompute ratio of a check layer (reference ascend.py:776-780)."""
        index = self.check_layers.index(layer_id) if layer_id in self.check_layers else 0
        return self.recompute_ratios[min(len(self.recompute_ratios) - 1, index)]
