"""Connector boundary and model registry on the CPU: the class-level and
scheduler-side methods vLLM calls, and the registry the worker finds its
layerwise executor in (reference connector.py:75-83, 868-882;
registry.py:13-41)."""

import gc
import json
from types import SimpleNamespace

import pytest
import torch

from cacheblend_vllm import registry
from cacheblend_vllm.connector import CacheBlendConnectorV1, KVConnectorRole


def _config(engine="e"):
    return SimpleNamespace(
        kv_transfer_config=SimpleNamespace(kv_connector_extra_config={}, engine_id=engine,
                                           kv_load_failure_policy=None),
        cache_config=SimpleNamespace(block_size=16),
        parallel_config=SimpleNamespace(pipeline_parallel_size=1, tensor_parallel_size=1),
        model_config=SimpleNamespace(model="m"),
    )


def test_requires_piecewise_for_cudagraph_follows_decode_cache_saving():
    assert CacheBlendConnectorV1.requires_piecewise_for_cudagraph({}) is False
    assert CacheBlendConnectorV1.requires_piecewise_for_cudagraph({"save_decode_cache": True}) is True
    assert CacheBlendConnectorV1.requires_piecewise_for_cudagraph({"save_decode_cache": 0}) is False


def test_scheduler_methods_are_control_plane():
    conn = CacheBlendConnectorV1(_config(), KVConnectorRole.SCHEDULER)
    for call in (lambda: conn.request_finished(None, []),
                 lambda: conn.request_finished_all_groups(None, ([],)),
                 lambda: conn.get_num_new_matched_tokens(None, 0),
                 lambda: conn.build_connector_meta(None)):
        with pytest.raises(NotImplementedError, match="control plane"):
            call()
    # the scheduler role registers nothing
    conn.register_kv_caches({"model.layers.0.attn": torch.zeros(2, 1, 16, 1, 8)})
    conn.close()


def test_model_scope_default_and_initialized_event(tmp_path, monkeypatch):
    """Reference connector.py:130-144, 158-166: the default store scope is
    ``<model>@<revision>|<dtype>|tp=<tp>`` and every connector announces
    itself with a ``connector_initialized`` trace event."""
    monkeypatch.setenv("CACHEBLEND_TRACE_DIR", str(tmp_path))
    cfg = _config("eng")
    cfg.model_config = SimpleNamespace(model="Qwen/Qwen3-8B", revision="main", dtype=torch.bfloat16)
    cfg.parallel_config.tensor_parallel_size = 2
    conn = CacheBlendConnectorV1(cfg, KVConnectorRole.WORKER)
    assert conn.model_scope == "Qwen/Qwen3-8B@main|torch.bfloat16|tp=2"
    assert conn.tp_size == 2
    conn.close()
    # a configured scope wins; missing model fields fall back as the reference's do
    cfg2 = _config()
    cfg2.kv_transfer_config.kv_connector_extra_config = {"model_scope": "fixed"}
    assert CacheBlendConnectorV1(cfg2, KVConnectorRole.SCHEDULER).model_scope == "fixed"
    cfg3 = _config()
    cfg3.model_config = SimpleNamespace()
    assert CacheBlendConnectorV1(cfg3, KVConnectorRole.SCHEDULER).model_scope == "unknown-model@|unknown|tp=1"
    records = [json.loads(line) for f in sorted(tmp_path.iterdir()) for line in f.read_text().splitlines()]
    init = [r for r in records if r["event"] == "connector_initialized"]
    assert len(init) == 3
    first = next(r for r in init if r["component"] == "worker")
    assert first["engine_id"] == "eng" and first["tp_size"] == 2
    assert first["model_scope"] == "Qwen/Qwen3-8B@main|torch.bfloat16|tp=2"
    assert first["role"] == str(KVConnectorRole.WORKER)
    assert {r["role"] for r in init} == {str(KVConnectorRole.WORKER), str(KVConnectorRole.SCHEDULER)}


def test_pipeline_parallel_is_rejected():
    cfg = _config()
    cfg.parallel_config.pipeline_parallel_size = 2
    with pytest.raises(ValueError, match="pipeline_parallel_size=1"):
        CacheBlendConnectorV1(cfg, KVConnectorRole.WORKER)


def test_worker_without_registered_model_fails_at_registration():
    registry.clear_for_test()
    conn = CacheBlendConnectorV1(_config("nobody"), KVConnectorRole.WORKER)
    with pytest.raises(RuntimeError, match="was not registered before connector initialization"):
        conn.register_kv_caches({"model.layers.0.attn": torch.zeros(2, 1, 16, 1, 8)})
    with pytest.raises(RuntimeError, match="received no KV caches"):
        conn.register_kv_caches({})
    conn.close()


class _Model:
    pass


class _Executor:
    def run(self, request_id, tokens, plan, loader):
        return None


def test_registry_register_get_unregister():
    registry.clear_for_test()
    model = _Model()
    with pytest.raises(ValueError, match="engine_id cannot be empty"):
        registry.register_model("", model)
    registry.register_model("a", model)
    registry.register_model("a", model)            # the same model again is fine
    assert registry.get_model("a") is model
    with pytest.raises(RuntimeError, match="a different model is already registered for engine a"):
        registry.register_model("a", _Model())
    registry.unregister_model("a")
    registry.unregister_model("a")                 # unknown ids are ignored
    with pytest.raises(RuntimeError, match="cacheblend_models vLLM general plugin"):
        registry.get_model("a")


def test_registry_holds_models_weakly():
    registry.clear_for_test()
    registry.register_model("w", _Model())         # no other reference: collected
    gc.collect()
    with pytest.raises(RuntimeError):
        registry.get_model("w")
    registry.register_model("w", _Model())         # a dead entry does not block a new model
    plain = {"not": "weakly referenceable"}
    registry.register_model("d", plain)
    assert registry.get_model("d") is plain
    registry.clear_for_test()


def test_build_executor_factory_model_run_or_error():
    registry.clear_for_test()
    model, executor = _Model(), _Executor()
    with pytest.raises(RuntimeError, match="no CacheBlend layerwise executor for _Model"):
        registry.build_executor(model, None, 16)
    assert registry.build_executor(executor, None, 16) is executor
    seen = []
    registry.set_executor_factory(lambda m, cfg, bs: seen.append((m, cfg, bs)) or executor)
    assert registry.build_executor(model, "cfg", 16) is executor and seen == [(model, "cfg", 16)]
    registry.set_executor_factory(None)
    with pytest.raises(RuntimeError):
        registry.build_executor(model, None, 16)
    registry.clear_for_test()
