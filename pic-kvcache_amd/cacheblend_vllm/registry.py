"""Process-local registry joining vLLM's model construction to the connector.

vLLM builds the model and the KV connector separately. A model plugin
publishes each engine's model with ``register_model(engine_id, model)``;
the worker connector's ``register_kv_caches`` looks it up with
``get_model(engine_id)`` and turns it into the layerwise executor that
drives the blend loader. These four functions keep the names, arguments
and errors of the reference's registry (cacheblend_vllm/registry.py:13-41),
so the reference's model plugin registers into this package unchanged.
Models are held weakly where they allow it: a model that is gone is not
registered.

The executor that runs the model's layers over a blend span (norms,
projections, MLP) is model code, outside this package. ``build_executor``
finds it: the factory installed with ``set_executor_factory``, else the
registered object itself when it already is an executor (it has
``run(request_id, tokens, plan, loader)``).
"""

from __future__ import annotations

import threading
import weakref
from collections.abc import Callable
from typing import Any

_guard = threading.RLock()
_models: dict[str, Callable[[], Any]] = {}
_executor_factory: Callable[[Any, Any, int], Any] | None = None


def _holder(model: Any) -> Callable[[], Any]:
    try:
        return weakref.ref(model)
    except TypeError:  # objects without weak reference support are held strongly
        return lambda: model


def register_model(engine_id: str, model: Any) -> None:
    if not engine_id:
        raise ValueError("engine_id cannot be empty")
    with _guard:
        holder = _models.get(engine_id)
        current = holder() if holder is not None else None
        if current is not None and current is not model:
            raise RuntimeError(f"a different model is already registered for engine {engine_id}")
        _models[engine_id] = _holder(model)


def get_model(engine_id: str) -> Any:
    with _guard:
        holder = _models.get(engine_id)
        model = holder() if holder is not None else None
        if holder is not None and model is None:
            del _models[engine_id]
    if model is None:
        raise RuntimeError(
            "CacheBlend model was not registered before connector initialization. "
            "Ensure the cacheblend_models vLLM general plugin is loaded."
        )
    return model


def unregister_model(engine_id: str) -> None:
    with _guard:
        _models.pop(engine_id, None)


def clear_for_test() -> None:
    global _executor_factory
    with _guard:
        _models.clear()
        _executor_factory = None


def set_executor_factory(factory: Callable[[Any, Any, int], Any] | None) -> None:
    """Install ``factory(model, config, block_size) -> executor`` (None
    removes it). The executor's ``run(request_id, tokens, plan, loader)``
    drives ``loader.prefetch/get/commit`` over the model's layers."""
    global _executor_factory
    with _guard:
        _executor_factory = factory


def build_executor(model: Any, config: Any, block_size: int) -> Any:
    with _guard:
        factory = _executor_factory
    if factory is not None:
        return factory(model, config, block_size)
    if callable(getattr(model, "run", None)):
        return model
    raise RuntimeError(
        f"no CacheBlend layerwise executor for {type(model).__name__}: install one with "
        "cacheblend_vllm.registry.set_executor_factory, or register an object with "
        "run(request_id, tokens, plan, loader)"
    )
