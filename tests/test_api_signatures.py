"""The drop-in boundary's call signatures: every public function and method
the reference's callers use keeps the reference's parameter names in the
reference's order (extra parameters come after them, with defaults), and
what the reference exposes as a property stays a property. The expected
lists restate the reference's signatures (cacheblend_vllm/kv_layout.py,
ascend.py, connector.py, config.py, types.py, hashing.py, matcher.py,
storage.py, registry.py, trace.py)."""

import inspect

import pytest
import torch

from cacheblend_vllm import attention, config, connector, hashing, kv_layout, loader, matcher, rope
from cacheblend_vllm import registry, selection, storage, trace, types

FUNCTIONS = [
    # kv_layout.py:90, 125
    (kv_layout.gather_paged_kv, ["kv_layer", "slot_mapping", "block_size", "out"]),
    (kv_layout.scatter_paged_kv, ["contiguous", "kv_layer", "slot_mapping", "block_size"]),
    # ascend.py:52, 106 (module functions)
    (rope.relocate_key, ["rotary_emb", "old_positions", "new_positions", "key"]),
    (rope.validate_rope_support, ["model", "rotary_emb"]),
    # ascend.py:798 Qwen3BlendExecutor._attention (self dropped)
    (attention.blend_attention, ["query", "key", "value", "q_positions", "scale", "state"]),
    # hashing.py
    (hashing.content_hash, ["tokens"]),
    (hashing.rolling_hashes, ["tokens", "window"]),
    (hashing.rolling_hash_values, ["tokens", "window"]),
    # registry.py:13-41
    (registry.register_model, ["engine_id", "model"]),
    (registry.get_model, ["engine_id"]),
    (registry.unregister_model, ["engine_id"]),
    (registry.clear_for_test, []),
]

METHODS = [
    # ascend.py:170-407
    (loader.PagedBlendLoader, "__init__", ["kv_caches", "store", "request_id", "plan", "slot_mapping",
                                           "block_size", "config", "tracer", "load_stream"]),
    (loader.PagedBlendLoader, "prefetch", ["layer_id", "rotary_emb"]),
    (loader.PagedBlendLoader, "get", ["layer_id"]),
    (loader.PagedBlendLoader, "commit", ["layer_id", "contiguous"]),
    # ascend.py:638, 757 (Qwen3BlendExecutor's selection methods)
    (selection.BlendSelector, "_sparse_q_scores", ["query", "key", "absolute_indices", "gap_mask", "scale"]),
    (selection.BlendSelector, "_select", ["scores", "gap_mask", "layer_id", "forced_mask"]),
    # connector.py (worker and scheduler entry points vLLM calls)
    (connector.CacheBlendConnectorV1, "__init__", ["vllm_config", "role", "kv_cache_config"]),
    (connector.CacheBlendConnectorV1, "register_kv_caches", ["kv_caches"]),
    (connector.CacheBlendConnectorV1, "start_load_kv", ["forward_context"]),
    (connector.CacheBlendConnectorV1, "wait_for_layer_load", ["layer_name"]),
    (connector.CacheBlendConnectorV1, "save_kv_layer", ["layer_name", "kv_layer", "attn_metadata"]),
    (connector.CacheBlendConnectorV1, "wait_for_save", []),
    (connector.CacheBlendConnectorV1, "get_finished", ["finished_req_ids"]),
    (connector.CacheBlendConnectorV1, "get_block_ids_with_load_errors", []),
    (connector.CacheBlendConnectorV1, "get_num_new_matched_tokens", ["request", "num_computed_tokens"]),
    (connector.CacheBlendConnectorV1, "update_state_after_alloc", ["request", "blocks", "num_external_tokens"]),
    (connector.CacheBlendConnectorV1, "build_connector_meta", ["scheduler_output"]),
    (connector.CacheBlendConnectorV1, "request_finished", ["request", "block_ids"]),
    (connector.CacheBlendConnectorV1, "request_finished_all_groups", ["request", "block_ids"]),
    (connector.CacheBlendConnectorV1, "close", []),
    # config.py, types.py
    (config.CacheBlendConfig, "validate", []),
    (types.SegmentId, "to_dict", []),
    (types.BlendSegment, "to_dict", []),
    (types.BlendPlan, "to_dict", []),
    # matcher.py:54-133
    (matcher.TokenRangeMatcher, "__init__", ["chunk_size"]),
    (matcher.TokenRangeMatcher, "make_record", ["model_scope", "source_start", "tokens"]),
    (matcher.TokenRangeMatcher, "register", ["record"]),
    (matcher.TokenRangeMatcher, "unregister", ["segment_id"]),
    (matcher.TokenRangeMatcher, "match", ["model_scope", "tokens", "start_offset"]),
    (matcher.TokenRangeMatcher, "validate", ["segments"]),
    # storage.py:35-279
    (storage.LocalPinnedCPUStore, "__init__", ["chunk_size", "max_bytes", "pin_memory"]),
    (storage.LocalPinnedCPUStore, "begin_put", ["model_scope", "source_start", "tokens", "num_layers"]),
    (storage.LocalPinnedCPUStore, "put_layer", ["segment_id", "layer_id", "kv"]),
    (storage.LocalPinnedCPUStore, "reserve_layer", ["segment_id", "layer_id"]),
    (storage.LocalPinnedCPUStore, "cancel_layer", ["segment_id", "layer_id"]),
    (storage.LocalPinnedCPUStore, "put_layer_host", ["segment_id", "layer_id", "cpu_tensor"]),
    (storage.LocalPinnedCPUStore, "abort_put", ["segment_id"]),
    (storage.LocalPinnedCPUStore, "match", ["model_scope", "tokens", "start_offset"]),
    (storage.LocalPinnedCPUStore, "validate", ["segments"]),
    (storage.LocalPinnedCPUStore, "pin", ["request_id", "segments"]),
    (storage.LocalPinnedCPUStore, "release", ["request_id"]),
    (storage.LocalPinnedCPUStore, "get_layer", ["request_id", "segment", "layer_id"]),
    (storage.LocalPinnedCPUStore, "clear", []),
    # trace.py
    (trace.PipelineTracer, "__init__", ["component"]),
    (trace.PipelineTracer, "emit", ["event", "request_id"]),
    (trace.PipelineTracer, "close", []),
]

CLASS_METHODS = [
    (connector.CacheBlendConnectorV1, "requires_piecewise_for_cudagraph", ["extra_config"]),
    (config.CacheBlendConfig, "from_extra_config", ["values"]),
    (types.SegmentId, "from_dict", ["value"]),
    (types.BlendSegment, "from_dict", ["value"]),
    (types.BlendPlan, "from_dict", ["value"]),
    (types.BlendPlan, "from_segments", ["apc_prefix_tokens", "segments"]),
]

PROPERTIES = [
    (config.CacheBlendConfig, "max_local_cpu_bytes"),
    (types.BlendSegment, "source_start"),
    (types.BlendSegment, "length"),
    (types.BlendSegment, "target_end"),
    (types.BlendPlan, "allocation_tokens"),
    (types.BlendPlan, "gap_tokens"),
    (storage.LocalPinnedCPUStore, "current_bytes"),
    (storage.LocalPinnedCPUStore, "committed_entries"),
    (trace.PipelineTracer, "enabled"),
]


def _check(params, want, label):
    names = [p.name for p in params]
    assert names[: len(want)] == want, f"{label}: {names} does not start with {want}"
    for p in params[len(want):]:
        ok = p.default is not inspect.Parameter.empty or p.kind in (p.VAR_POSITIONAL, p.VAR_KEYWORD)
        assert ok, f"{label}: extra parameter {p.name} has no default"


@pytest.mark.parametrize("fn,want", FUNCTIONS, ids=[f.__qualname__ for f, _ in FUNCTIONS])
def test_function_signatures(fn, want):
    _check(list(inspect.signature(fn).parameters.values()), want, fn.__qualname__)


@pytest.mark.parametrize("cls,name,want", METHODS, ids=[f"{c.__name__}.{n}" for c, n, _ in METHODS])
def test_method_signatures(cls, name, want):
    params = list(inspect.signature(getattr(cls, name)).parameters.values())
    assert params[0].name == "self"
    _check(params[1:], want, f"{cls.__name__}.{name}")


@pytest.mark.parametrize("cls,name,want", CLASS_METHODS, ids=[f"{c.__name__}.{n}" for c, n, _ in CLASS_METHODS])
def test_classmethod_signatures(cls, name, want):
    assert isinstance(inspect.getattr_static(cls, name), classmethod)
    _check(list(inspect.signature(getattr(cls, name)).parameters.values()), want, f"{cls.__name__}.{name}")


@pytest.mark.parametrize("cls,name", PROPERTIES, ids=[f"{c.__name__}.{n}" for c, n in PROPERTIES])
def test_properties(cls, name):
    assert isinstance(inspect.getattr_static(cls, name), property)


def test_local_pinned_cpu_store_round_trip_without_pinning():
    """The reference constructor, pin_memory off: a two-layer segment goes in
    through put_layer and comes back through match, pin and get_layer."""
    store = storage.LocalPinnedCPUStore(4, 1 << 20, pin_memory=False)
    assert store.pin_memory is False
    tokens = [5, 6, 7, 8]
    sid = store.begin_put("scope", 0, tokens, 2)
    layers = [torch.arange(16, dtype=torch.float32).reshape(2, 4, 2) + 100 * i for i in range(2)]
    assert store.put_layer(sid, 0, layers[0]) is False
    assert store.put_layer(sid, 1, layers[1]) is True
    assert store.committed_entries == 1 and store.current_bytes > 0
    segments = store.match("scope", [9] + tokens, 1)
    assert len(segments) == 1 and segments[0].target_start == 1
    store.pin("req", segments)
    for i in range(2):
        got = store.get_layer("req", segments[0], i)
        assert not got.is_pinned()
        assert torch.equal(got, layers[i])
    store.release("req")
    with pytest.raises(ValueError, match="max_bytes must be positive"):
        storage.LocalPinnedCPUStore(4, 0)
