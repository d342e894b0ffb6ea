"""CacheBlendConnectorV1, worker data path, on MI355X.

Keeps the reference connector's class name, constructor and worker-side
methods (cacheblend_vllm/connector.py:75-568) for the KV data path:

  register_kv_caches   layer order, pinned chunk store, Store/Load streams,
                       the layerwise executor of the engine's registered
                       model (``registry.get_model`` / ``build_executor``)
  save_kv_layer        Store-stream gather + pinned D2H + async publication
  wait_for_save        the Store-completion / publication boundary
  start_load_kv        PagedBlendLoader + the executor, failure policy
                       ``kv_load_failure_policy=recompute``
  get_finished, get_block_ids_with_load_errors, close

The scheduler half (lookup RPC, matcher, plan gating, metadata building)
is the reference's control plane and is not part of this package: those
methods raise NotImplementedError; ``_slot_mapping`` (the slot format the
kernels consume) is provided in ``store_path``.
"""

from __future__ import annotations

import re
import time
from typing import Any

import torch

from . import registry
from .config import CacheBlendConfig
from .host_store import PinnedChunkSlab, PinnedChunkStore
from .kv_layout import kv_planes
from .loader import PagedBlendLoader
from .store_path import (  # noqa: F401 - re-exported reference names
    CacheBlendConnectorMetadata,
    RequestMetadata,
    StoreStreamWriter,
    _slot_mapping,
)
from .streams import LOAD, side_stream
from .trace import PipelineTracer

try:  # vLLM's connector base when vLLM is installed
    from vllm.distributed.kv_transfer.kv_connector.v1.base import (  # type: ignore
        KVConnectorBase_V1 as _Base,
        KVConnectorRole,
    )

    try:  # hybrid-memory-allocator support marker (reference connector.py:13-18, 75)
        from vllm.distributed.kv_transfer.kv_connector.v1.base import SupportsHMA as _HMA  # type: ignore
    except ImportError:
        _HMA = object
except ImportError:  # vLLM absent: a minimal stand-in with the same role enum
    _HMA = object

    import enum

    class KVConnectorRole(enum.Enum):  # type: ignore[no-redef]
        SCHEDULER = 0
        WORKER = 1

    class _Base:  # type: ignore[no-redef]
        def __init__(self, vllm_config, role, kv_cache_config=None):
            self._vllm_config = vllm_config
            self._role = role
            self._connector_metadata = None

        @property
        def role(self):
            return self._role

        def bind_connector_metadata(self, metadata) -> None:
            self._connector_metadata = metadata

        def clear_connector_metadata(self) -> None:
            self._connector_metadata = None

        def _get_connector_metadata(self):
            return self._connector_metadata


def _layer_sort_key(name: str) -> tuple[int, str]:
    """Trailing layer index of a vLLM layer name (reference connector.py:48-50)."""
    matches = re.findall(r"(?:layers?\.)?(\d+)", name)
    return (int(matches[-1]) if matches else 1 << 30, name)


class CacheBlendConnectorV1(_Base, *(() if _HMA is object else (_HMA,))):
    """CacheBlend KV connector (worker data path on MI355X)."""

    @classmethod
    def requires_piecewise_for_cudagraph(cls, extra_config: dict[str, Any]) -> bool:
        """Reference connector.py:78-83: only storing the decode cache needs
        Python between graph pieces (its save runs per layer during decode);
        prompt-only stores run outside decode graph replay."""
        return bool(extra_config.get("save_decode_cache", False))

    def __init__(self, vllm_config, role, kv_cache_config=None):
        super().__init__(vllm_config, role, kv_cache_config)
        transfer = vllm_config.kv_transfer_config
        self.config = CacheBlendConfig.from_extra_config(transfer.kv_connector_extra_config)
        self._recompute_on_failure = getattr(transfer, "kv_load_failure_policy", None) == "recompute"
        self.engine_id = str(transfer.engine_id)
        self.block_size = int(vllm_config.cache_config.block_size)
        self.tp_size = int(vllm_config.parallel_config.tensor_parallel_size)
        if int(vllm_config.parallel_config.pipeline_parallel_size) != 1:
            raise ValueError("CacheBlendConnectorV1 currently requires pipeline_parallel_size=1")
        self.model_scope = self.config.model_scope or self._make_model_scope(vllm_config)
        self._trace = PipelineTracer("scheduler" if role is KVConnectorRole.SCHEDULER else "worker")
        self._trace.emit("connector_initialized", engine_id=self.engine_id,
                         model_scope=self.model_scope, role=str(role), tp_size=self.tp_size)
        self._store: PinnedChunkStore | None = None
        self._writer: StoreStreamWriter | None = None
        self._slab: PinnedChunkSlab | None = None
        self._kv_caches: list = []
        self._layer_ids: dict[str, int] = {}
        self._executor = None
        self._load_stream = None
        self._load_errors: set[int] = set()

    @staticmethod
    def _make_model_scope(vllm_config) -> str:
        """The store's namespace when ``model_scope`` is not configured
        (reference connector.py:158-166): model name, revision, dtype and
        tensor-parallel size, so chunks of another revision, dtype or TP
        split never match. Written ``<model>@<revision>|<dtype>|tp=<tp>``."""
        model_config = vllm_config.model_config
        name = getattr(model_config, "model", "unknown-model")
        revision = getattr(model_config, "revision", "")
        dtype = getattr(model_config, "dtype", "unknown")
        tp = int(vllm_config.parallel_config.tensor_parallel_size)
        return f"{name}@{revision}|{dtype}|tp={tp}"

    # ---------------------------------------------------------- worker

    def register_kv_caches(self, kv_caches: dict[str, Any]) -> None:
        """Reference connector.py:168-213. The layerwise executor comes from
        the model registered for this engine (``registry.get_model``, as the
        reference does at :205-206) through ``registry.build_executor``; its
        ``run(request_id, tokens, plan, loader)`` drives the loader."""
        if self.role is not KVConnectorRole.WORKER:
            return
        ordered = sorted(kv_caches.items(), key=lambda item: _layer_sort_key(item[0]))
        self._layer_ids = {name: i for i, (name, _) in enumerate(ordered)}
        self._kv_caches = [value for _, value in ordered]
        if not self._kv_caches:
            raise RuntimeError("CacheBlendConnectorV1 received no KV caches")
        key, _ = kv_planes(self._kv_caches[0])
        executor = registry.build_executor(registry.get_model(self.engine_id), self.config,
                                           self.block_size)
        # chunks live in pinned slab slots (one pinned arena per 128 chunks,
        # bounded by the store's byte cap) instead of a fresh pinned batch per
        # layer; slots go back to the slab when the store drops a segment
        self._slab = PinnedChunkSlab((2, self.config.chunk_size, *key.shape[2:]), key.dtype,
                                     chunks_per_arena=128, max_bytes=0)
        self._store = PinnedChunkStore(self.config.chunk_size, self.config.max_local_cpu_bytes,
                                       on_release=self._slab.free)
        self._load_stream = side_stream(LOAD, key.device)
        self._writer = StoreStreamWriter(
            self._store, self.block_size, self.config.chunk_size, len(self._kv_caches),
            self.model_scope, self.config.store_workers, self.config.max_inflight_store_batches,
            tracer=self._trace, slab=self._slab,
        )
        self._executor = executor
        self._trace.emit("worker_registered", rank=0, layers=len(self._kv_caches),
                         cpu_cache_bytes=self.config.max_local_cpu_bytes)

    def _layer_id(self, layer_name: str) -> int | None:
        layer_id = self._layer_ids.get(layer_name)
        if layer_id is None:
            key = _layer_sort_key(layer_name)[0]
            layer_id = next(
                (i for name, i in self._layer_ids.items() if _layer_sort_key(name)[0] == key), None
            )
        return layer_id

    def save_kv_layer(self, layer_name: str, kv_layer: Any, attn_metadata: Any, **kwargs: Any) -> None:
        """Reference connector.py:281-361."""
        if self._writer is None:
            return
        metadata = self._get_connector_metadata()
        if not isinstance(metadata, CacheBlendConnectorMetadata):
            return
        layer_id = self._layer_id(layer_name)
        if layer_id is None:
            return
        self._writer.save_layer(layer_id, kv_layer, metadata.requests)

    def wait_for_save(self) -> None:
        if self._writer is not None:
            self._writer.wait_for_save()

    def wait_for_layer_load(self, layer_name: str) -> None:
        return

    def start_load_kv(self, forward_context: Any, **kwargs: Any) -> None:
        """Reference connector.py:215-276."""
        metadata = self._get_connector_metadata()
        if not isinstance(metadata, CacheBlendConnectorMetadata):
            raise TypeError("unexpected CacheBlend connector metadata")
        if self._store is None or self._executor is None:
            if any(request.plan is not None for request in metadata.requests):
                raise RuntimeError("CacheBlend worker was not initialized")
            return
        for request in metadata.requests:
            if request.plan is None:
                continue
            self._blend_one(forward_context, request)

    def _blend_one(self, forward_context: Any, request: RequestMetadata) -> None:
        """Load and blend one planned request. The executor may move the
        forward context's per-layer cursors (``layer_idx``,
        ``moe_layer_index``); they are put back afterwards. The request's
        pins are released with the loader's last host-read event, so chunks
        the store drops meanwhile are not reused under an in-flight copy."""
        plan = request.plan
        trace = self._trace.enabled
        started = time.monotonic_ns() if trace else 0
        if trace:
            self._trace.emit("blend_started", request_id=request.request_id,
                             apc_prefix_tokens=plan.apc_prefix_tokens,
                             allocation_tokens=plan.allocation_tokens, hit_tokens=plan.hit_tokens,
                             gap_tokens=plan.gap_tokens, segments=len(plan.segments))
        saved = {name: getattr(forward_context, name) for name in ("moe_layer_index", "layer_idx")
                 if hasattr(forward_context, name)}
        loader = None
        failure = None
        try:
            loader = PagedBlendLoader(
                self._kv_caches, self._store, request.request_id, plan,
                request.slot_mapping, self.block_size, self.config, tracer=self._trace,
                load_stream=self._load_stream,
            )
            self._executor.run(request.request_id, request.token_ids, plan, loader)
        except Exception as error:
            failure = type(error).__name__
            self._record_load_error(request)
            if not self._recompute_on_failure:
                raise
        finally:
            for name, value in saved.items():
                setattr(forward_context, name, value)
            self._store.release(request.request_id,
                                loader.host_reads_done() if loader is not None else None)
            if trace:
                self._trace.emit("blend_finished", request_id=request.request_id,
                                 duration_us=(time.monotonic_ns() - started) / 1000, error=failure)

    def get_finished(self, finished_req_ids: set[str]):
        if self._writer is not None:
            self._writer.finished(finished_req_ids)
        return None, None

    def get_block_ids_with_load_errors(self) -> set[int]:
        result, self._load_errors = self._load_errors, set()
        return result

    def _record_load_error(self, request: RequestMetadata) -> None:
        """Block ids of the externally allocated span (reference connector.py:564-568)."""
        if request.plan is None:
            return
        slots = request.slot_mapping[request.plan.apc_prefix_tokens : request.plan.allocation_end]
        self._load_errors.update(int(v) for v in torch.unique(slots // self.block_size))

    def close(self) -> None:
        if self._writer is not None:
            self._writer.close()
            self._writer = None
        if self._store is not None:
            self._store.clear()
        if self._slab is not None:
            self._slab.close()
            self._slab = None
        self._trace.close()

    # ------------------------------------------------------- scheduler

    def _control_plane(self, name: str):
        raise NotImplementedError(
            f"CacheBlendConnectorV1.{name} is the scheduler-side control plane (lookup RPC, "
            "matcher, plan gating); this package implements the worker KV data path only"
        )

    def get_num_new_matched_tokens(self, request, num_computed_tokens):
        return self._control_plane("get_num_new_matched_tokens")

    def update_state_after_alloc(self, request, blocks, num_external_tokens):
        return self._control_plane("update_state_after_alloc")

    def build_connector_meta(self, scheduler_output):
        return self._control_plane("build_connector_meta")

    def request_finished(self, request, block_ids):
        return self._control_plane("request_finished")

    def request_finished_all_groups(self, request, block_ids):
        return self._control_plane("request_finished_all_groups")
