"""Worker-side save pipeline of CacheBlendConnectorV1 on MI355X.

Same protocol and method names as the reference connector's save half
(cacheblend_vllm/connector.py:281-549), with the gather running in the
gfx950 paged-gather kernel and the copies on a HIP side stream:

  save_kv_layer(layer)      per request: complete chunk_size chunks up to
                            save_end, one reservation per (chunk, layer),
                            one fused slot list over every pending chunk
  _enqueue_store_batch      Store stream: wait for the serving stream, then
                            with a pinned chunk slab: slots allocated as
                            consecutive runs, filled either by gather into a
                            chunk-major device staging + one D2H per run
                            ("dma") or by the gather kernel writing the
                            slots over the host link ("host_write");
                            without one: gather into the request's reused
                            staging + D2H into a freshly pinned batch, as
                            the reference does. Then an event, and the batch
                            goes to a publisher thread (backpressure
                            semaphore)
  _publish                  publisher thread: wait for the batch's event,
                            then put the per-chunk slots (or views of the
                            batch) into the store; any failure aborts every
                            chunk of the batch
  wait_for_save             Store-stream sync + join publishers; staging freed

A batch in flight is a ``_StoreBatch``; ``_InflightSaves`` bounds and tracks
the publications per request, ``_StagingCache`` owns the pinned-batch
scheme's device stagings until the Store stream drains.

Everything enqueued goes to one default-priority Store stream, so the D2H of
layer l and the gather of layer l + 1 are ordered on it while the serving
stream keeps computing.
"""

from __future__ import annotations

import ctypes
import queue
import threading
import time
from concurrent.futures import Future, ThreadPoolExecutor
from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch

from . import _native
from .kv_layout import gather_paged_kv, kv_desc, kv_planes
from .streams import STORE, STORE_COPY, side_stream
from .trace import PipelineTracer, roctx_phase
from .types import BlendPlan, SegmentId


def _slot_mapping(block_ids: list[int], block_size: int, token_count: int) -> torch.Tensor:
    """``block * bs + offset`` over ``block_ids``, first ``token_count`` slots
    (reference connector.py:42-45)."""
    blocks = torch.tensor(block_ids, dtype=torch.long)
    offsets = torch.arange(block_size, dtype=torch.long)
    return (blocks[:, None] * block_size + offsets[None, :]).flatten()[:token_count]


@dataclass(slots=True)
class RequestMetadata:
    """Per-request worker metadata (reference connector.py:53-60)."""

    request_id: str
    token_ids: list[int]
    slot_mapping: torch.Tensor
    plan: BlendPlan | None
    save: bool
    save_end: int


try:  # vLLM's metadata base, which bind_connector_metadata expects, when vLLM is installed
    from vllm.distributed.kv_transfer.kv_connector.v1.base import (  # type: ignore
        KVConnectorMetadata as _MetadataBase,
    )
except ImportError:
    _MetadataBase = object


@dataclass(slots=True)
class CacheBlendConnectorMetadata(_MetadataBase):
    """What the scheduler hands the worker each step (reference connector.py:70-72)."""

    requests: list[RequestMetadata] = field(default_factory=list)


class CudaStreams:
    """torch.cuda stream/event factory (replaceable by fakes in tests)."""

    @staticmethod
    def current_stream():
        return torch.cuda.current_stream()

    @staticmethod
    def stream(s):
        return torch.cuda.stream(s)

    @staticmethod
    def Event():  # noqa: N802 - mirrors torch.cuda.Event
        return torch.cuda.Event()

    @staticmethod
    def Stream():  # noqa: N802
        return side_stream(STORE)

    @staticmethod
    def CopyStream():  # noqa: N802
        return side_stream(STORE_COPY)


def _chain(inner: Future, outer: Future) -> None:
    """Complete ``outer`` with ``inner``'s outcome."""
    error = inner.exception()
    if error is not None:
        outer.set_exception(error)
    else:
        outer.set_result(inner.result())


@dataclass(slots=True)
class _StoreBatch:
    """One request's chunks of one layer on their way into the store.

    ``pending`` lists ``(segment id, layer, tokens)`` per chunk, in the order
    of ``host``: one pinned slab slot per chunk, or one pinned
    ``[2, tokens, *row]`` batch whose consecutive token ranges are the chunks.
    ``ready`` is the GPU event after which ``host`` holds the bytes.
    """

    request_id: str
    pending: list[tuple[Any, int, int]]
    host: Any
    ready: Any = None
    enqueued_ns: int | None = None

    def chunks(self):
        """``(index, segment id, layer, host tensor)`` per chunk; chunks of a
        pinned batch are views of it, so the store keeps the batch alive."""
        offset = 0
        for index, (segment_id, layer_id, tokens) in enumerate(self.pending):
            if isinstance(self.host, list):
                yield index, segment_id, layer_id, self.host[index]
            else:
                yield index, segment_id, layer_id, self.host[:, offset:offset + tokens]
            offset += tokens

    @property
    def tokens(self) -> int:
        return sum(tokens for _, _, tokens in self.pending)


class _InflightSaves:
    """Publication futures per request, at most ``limit`` batches at once:
    ``admit`` blocks the saving thread while the limit is reached and a
    batch's slot frees when its future completes."""

    def __init__(self, limit: int):
        self._slots = threading.Semaphore(limit)
        self._lock = threading.Lock()
        self._futures: dict[str, list[Future]] = {}

    def admit(self) -> None:
        self._slots.acquire()

    def cancel_admission(self) -> None:
        self._slots.release()

    def track(self, request_id: str, future: Future) -> None:
        with self._lock:
            self._futures.setdefault(request_id, []).append(future)
        future.add_done_callback(lambda _f: self._slots.release())

    def take(self) -> dict[str, list[Future]]:
        """Every tracked future, grouped by request; tracking starts over."""
        with self._lock:
            taken, self._futures = self._futures, {}
        return taken

    def __bool__(self) -> bool:
        with self._lock:
            return any(self._futures.values())


class _StagingCache:
    """Device stagings of the per-layer pinned-batch scheme: one per request,
    refilled in place while a layer has as many pending tokens as the last.
    A staging of another size is retired, not freed, because the D2H of an
    earlier layer may still read it; everything goes at the Store-stream
    boundary (``clear``)."""

    def __init__(self):
        self.live: dict[str, torch.Tensor] = {}
        self.retired: list[torch.Tensor] = []

    def gather(self, request_id: str, kv_layer: Any, slots: torch.Tensor, block_size: int) -> torch.Tensor:
        staging = self.live.get(request_id)
        if staging is not None and staging.shape[1] == slots.numel():
            gather_paged_kv(kv_layer, slots, block_size, out=staging)
            return staging
        if staging is not None:
            self.retired.append(staging)
        staging = self.live[request_id] = gather_paged_kv(kv_layer, slots, block_size).contiguous()
        return staging

    def clear(self) -> None:
        self.live.clear()
        self.retired.clear()


class StoreStreamWriter:
    """The save half of CacheBlendConnectorV1 (worker role)."""

    def __init__(
        self,
        store,
        block_size: int,
        chunk_size: int,
        num_layers: int,
        model_scope: str,
        store_workers: int = 1,
        max_inflight_store_batches: int = 8,
        tracer: PipelineTracer | None = None,
        streams=CudaStreams,
        store_stream=None,
        slab=None,
        max_workgroups: int = 256,
        slab_transfer: str = "dma",
    ):
        """``slab`` (a PinnedChunkSlab): every chunk gets its own pinned slot,
        allocated as consecutive runs, so no pinned memory is allocated per
        layer. ``slab_transfer`` picks how the bytes get there:
        "dma"        -- (default) gather into a chunk-major device staging
                        on the Store stream; a copier thread waits for each
                        layer's gather on the host and issues one
                        hipMemcpyAsync per run of consecutive slots on the
                        store's copy stream, so the layers' copies run
                        back to back with no stream waits between them
                        (the runtime runs a contiguous device-to-pinned
                        copy as a short blit kernel; 91-94% of the
                        transfer hides behind compute that fills every
                        CU);
        "host_write" -- the gather kernel writes the slots directly over
                        the host link: no staging, one launch per layer,
                        holding up to ``max_workgroups`` workgroups for the
                        transfer (zero-copy write rate grows with the CUs
                        issuing: 256 reach about 55 GB/s);
        None: gather into device staging + one pinned D2H per layer into a
        freshly pinned batch, as the reference does."""
        if slab_transfer not in ("dma", "host_write"):
            raise ValueError("slab_transfer must be 'dma' or 'host_write'")
        self._store = store
        self._slab = slab
        self._slab_transfer = slab_transfer
        self._max_workgroups = max_workgroups
        self.block_size = block_size
        self.chunk_size = chunk_size
        self.num_layers = num_layers
        self.model_scope = model_scope
        self._trace = tracer or PipelineTracer("worker")
        self._streams = streams
        self._store_stream = store_stream if store_stream is not None else streams.Stream()
        self._publishers = ThreadPoolExecutor(max_workers=store_workers,
                                              thread_name_prefix="cacheblend-save")
        self._inflight = _InflightSaves(max_inflight_store_batches)
        self._staging = _StagingCache()
        # chunk identities per request, hashed once: [(prompt offset, id)]
        self._chunk_ids: dict[str, list[tuple[int, SegmentId]]] = {}
        # per request: (host slot list, device copy); the fused slot list is
        # normally identical for every layer, so it is uploaded once
        self._device_slots: dict[str, tuple[torch.Tensor, torch.Tensor]] = {}
        # slab_transfer="dma": the copier thread and its stream (made on first use)
        self._copy_jobs: queue.Queue | None = None
        self._copier: threading.Thread | None = None
        self._copy_stream = None

    # ------------------------------------------------------------- save

    @roctx_phase("cacheblend.save_layer")
    def save_layer(self, layer_id: int, kv_layer: Any, requests: list[RequestMetadata]) -> None:
        """The per-request body of save_kv_layer (reference connector.py:308-361)."""
        for request in requests:
            if not request.save:
                continue
            usable = min(request.save_end, len(request.token_ids), request.slot_mapping.numel())
            usable = usable // self.chunk_size * self.chunk_size
            segments = self._request_save_segments(request, usable)
            reserve_many = getattr(self._store, "reserve_layers", None)
            if reserve_many is not None:
                reserved = reserve_many([sid for _, sid in segments], layer_id)
            else:
                reserved = [self._store.reserve_layer(sid, layer_id) for _, sid in segments]
            pending: list[tuple[SegmentId, int, int]] = [
                (sid, layer_id, self.chunk_size) for (_, sid), ok in zip(segments, reserved) if ok
            ]
            if not pending:
                continue
            if len(pending) == len(segments):  # chunks 0..n-1: one slice of the slot mapping
                slots = request.slot_mapping[: len(segments) * self.chunk_size]
            else:
                slots = torch.cat([request.slot_mapping[start : start + self.chunk_size]
                                   for (start, _), ok in zip(segments, reserved) if ok])
            trace = self._trace.enabled
            started = time.monotonic_ns() if trace else 0
            try:
                self._enqueue_store_batch(
                    pending, kv_layer, slots, request_id=request.request_id,
                    store_enqueued_ns=time.monotonic_ns() if trace else None,
                )
                if trace:
                    self._trace.emit(
                        "save_store_enqueued",
                        request_id=request.request_id,
                        layer_id=layer_id,
                        chunks=len(pending),
                        tokens=sum(n for _, _, n in pending),
                        duration_us=(time.monotonic_ns() - started) / 1000,
                    )
            except Exception:
                for segment_id, _, _ in pending:
                    self._store.abort_put(segment_id)
                raise

    def _request_save_segments(self, request: RequestMetadata, usable: int) -> list[tuple[int, SegmentId]]:
        """Chunk identities hashed once per request (reference connector.py:363-382)."""
        segments = self._chunk_ids.setdefault(request.request_id, [])
        start = len(segments) * self.chunk_size
        begin_chunks = getattr(self._store, "begin_put_chunks", None)
        if begin_chunks is not None and start < usable:
            ids = begin_chunks(self.model_scope, request.token_ids, start, usable, self.num_layers)
            segments.extend(zip(range(start, usable, self.chunk_size), ids))
            start = usable
        while start < usable:
            end = start + self.chunk_size
            segment_id = self._store.begin_put(
                self.model_scope, start, request.token_ids[start:end], self.num_layers
            )
            segments.append((start, segment_id))
            start = end
        return segments[: usable // self.chunk_size]

    def _enqueue_store_batch(
        self,
        pending: list[tuple[Any, int, int]],
        kv_layer: Any,
        slots: torch.Tensor,
        request_id: str,
        store_enqueued_ns: int | None = None,
    ) -> None:
        """Gather + D2H on the Store stream, then publication off the saving
        thread (reference connector.py:384-447)."""
        batch = _StoreBatch(request_id, pending, None, enqueued_ns=store_enqueued_ns)
        self._inflight.admit()
        try:
            if self._store_stream is None:
                raise RuntimeError("CacheBlend Store stream was not initialized")
            serving = self._streams.current_stream()
            with self._streams.stream(self._store_stream):
                self._store_stream.wait_stream(serving)
                slots = self._upload_slots(request_id, slots, kv_layer)
                if self._slab is not None:
                    batch.host = self._slab.alloc_run(len(pending))
                    if self._slab_transfer == "host_write":
                        self._gather_to_chunks(kv_layer, slots, [h.data_ptr() for h in batch.host])
                    else:
                        staging, runs = self._gather_for_dma(kv_layer, slots, batch.host)
                else:
                    staging = self._staging.gather(request_id, kv_layer, slots, self.block_size)
                    batch.host = torch.empty(staging.shape, dtype=staging.dtype, device="cpu",
                                             pin_memory=True)
                    batch.host.copy_(staging, non_blocking=True)
                event = self._streams.Event()
                event.record(self._store_stream)
            if self._slab is not None and self._slab_transfer == "dma":
                # the copier issues the D2H once the gather is done and sets
                # batch.ready to the copy's event
                future = Future()
                self._copier_queue().put((event, staging, runs, batch, future))
                del staging
            else:
                batch.ready = event
                future = self._publishers.submit(self._publish, batch)
        except Exception:
            self._inflight.cancel_admission()
            if self._slab is not None and isinstance(batch.host, list):
                for chunk in batch.host:
                    self._slab.free(chunk)
            raise
        self._inflight.track(request_id, future)

    def _upload_slots(self, request_id: str, slots: torch.Tensor, kv_layer: Any) -> torch.Tensor:
        """Device copy of a host slot list, reused while it does not change.
        The upload is a pinned, non-blocking copy on the Store stream, so the
        host never waits for earlier Store work here."""
        if slots.device.type != "cpu" or not torch.cuda.is_available():
            return slots
        cached = self._device_slots.get(request_id)
        if cached is not None and cached[0].shape == slots.shape and torch.equal(cached[0], slots):
            return cached[1]
        key, _ = kv_planes(kv_layer)
        num_slots = key.shape[0] * self.block_size
        if slots.numel() and (int(slots.min()) < 0 or int(slots.max()) >= num_slots):
            raise IndexError(f"slot_mapping holds slots outside [0, {num_slots})")
        host = slots.to(torch.long).contiguous().pin_memory()
        device = host.to("cuda", non_blocking=True)
        self._device_slots[request_id] = (host, device)
        return device

    def _gather_to_chunks(self, kv_layer: Any, slots: torch.Tensor, chunk_ptrs: list[int]) -> None:
        """cbk_paged_gather_chunks: the layer's pending tokens into chunks
        ``[2, chunk, *row]`` at ``chunk_ptrs`` (pinned host slots or device
        staging), on the current (Store) stream."""
        desc, key = kv_desc(kv_layer, self.block_size)
        n = len(chunk_ptrs)
        plane = self.chunk_size * desc.row_bytes
        k_ptrs = (ctypes.c_void_p * n)(*chunk_ptrs)
        v_ptrs = (ctypes.c_void_p * n)(*[k + plane for k in chunk_ptrs])
        rc = _native.load().cbk_paged_gather_chunks(
            desc, slots.data_ptr(), slots.numel(), self.chunk_size, k_ptrs, v_ptrs, desc.row_bytes,
            self._max_workgroups, None, _native.stream_handle(key.device),
        )
        _native.check(rc, "gather to chunks")

    def _gather_for_dma(self, kv_layer: Any, slots: torch.Tensor,
                        host: list[torch.Tensor]) -> tuple[torch.Tensor, tuple]:
        """Gather the layer's chunks into a fresh chunk-major device staging
        laid out like the slots (``chunk_bytes`` apart) on the current
        (Store) stream; returns it with the D2H run table (host dst, device
        src, bytes: one run per chunk, which ``cbk_memcpy_runs`` folds into
        one copy for consecutive slots) that the copier issues once the
        gather is done."""
        stride = self._slab.chunk_bytes
        n = len(host)
        key, _ = kv_planes(kv_layer)
        staging = torch.empty(n * stride, dtype=torch.uint8, device=key.device)
        base = staging.data_ptr()
        self._gather_to_chunks(kv_layer, slots, [base + i * stride for i in range(n)])
        dst = np.array([h.data_ptr() for h in host], dtype=np.uint64)
        src = np.uint64(base) + np.arange(n, dtype=np.uint64) * np.uint64(stride)
        return staging, (dst, src, np.full(n, stride, dtype=np.uint64))

    def _copier_queue(self) -> queue.Queue:
        if self._copier is None:
            self._copy_stream = self._streams.CopyStream()
            self._copy_jobs = queue.Queue()
            self._copier = threading.Thread(target=self._copier_loop, name="cacheblend-copier", daemon=True)
            self._copier.start()
        return self._copy_jobs

    def _copier_loop(self) -> None:
        """Copier thread: per layer, in order, wait (host side) for the
        gather, issue the runs' D2H copies on the Copy stream, hand the
        publication to the publisher pool. A wait between two copies on one
        stream left the DMA engine idle ~50-100 us whenever the submitting
        thread was busy between them; here the copies follow each other."""
        while True:
            job = self._copy_jobs.get()
            if job is None:
                return
            gathered, staging, (dst, src, nbytes), batch, future = job
            try:
                gathered.synchronize()
                _native.memcpy_runs(dst, src, nbytes, self._copy_stream.cuda_stream, "chunk runs D2H")
                staging.record_stream(self._copy_stream)
                batch.ready = self._streams.Event()
                batch.ready.record(self._copy_stream)
            except BaseException as error:  # the batch fails as a unit
                for segment_id, _, _ in batch.pending:
                    self._store.abort_put(segment_id)
                for chunk in batch.host:
                    self._slab.free(chunk)
                future.set_exception(error)
                continue
            finally:
                del staging
            inner = self._publishers.submit(self._publish, batch)
            inner.add_done_callback(lambda f, out=future: _chain(f, out))

    def _put_chunks(self, batch: _StoreBatch, kept: list[bool]) -> bool:
        """Each chunk into the store (reference connector.py:449-466);
        ``kept[i]`` says whether the store holds chunk i afterwards. True
        when some segment became committed."""
        holds = getattr(self._store, "holds", None)
        committed = False
        for index, segment_id, layer_id, chunk in batch.chunks():
            committed |= bool(self._store.put_layer_host(segment_id, layer_id, chunk))
            kept[index] = holds is not None and holds(segment_id, layer_id, chunk)
        return committed

    def _publish(self, batch: _StoreBatch) -> bool:
        """Publisher thread (reference connector.py:468-499): wait for the
        batch's bytes, publish every chunk, trace. Any failure drops the
        batch's segments as a unit. Slab slots the store did not keep go
        back to the slab at once; kept ones return through the store's
        release hook when it drops them."""
        kept = [False] * len(batch.pending)
        try:
            batch.ready.synchronize()
            committed = self._put_chunks(batch, kept)
        except Exception:
            for segment_id, _, _ in batch.pending:
                self._store.abort_put(segment_id)
            committed = None
        finally:
            if self._slab is not None and isinstance(batch.host, list):
                for chunk, held in zip(batch.host, kept):
                    if not held:
                        self._slab.free(chunk)
        if committed is None:
            return False
        if self._trace.enabled:
            self._trace.emit(
                "save_store_finished",
                request_id=batch.request_id,
                layer_id=batch.pending[0][1] if batch.pending else None,
                chunks=len(batch.pending),
                tokens=batch.tokens,
                duration_us=((time.monotonic_ns() - batch.enqueued_ns) / 1000
                             if batch.enqueued_ns is not None else None),
                committed_segment=committed,
            )
        return committed

    @roctx_phase("cacheblend.wait_for_save")
    def wait_for_save(self) -> None:
        """The save boundary (reference connector.py:504-534): drain the Store
        stream, then every publication enqueued so far; stagings are freed
        afterwards whatever happened."""
        started = time.monotonic_ns() if self._trace.enabled else 0
        taken: dict[str, list[Future]] = {}
        try:
            if self._store_stream is not None:
                self._store_stream.synchronize()
            taken = self._inflight.take()
            for futures in taken.values():
                for future in futures:
                    future.result()
        finally:
            self._staging.clear()
            self._device_slots.clear()
        if self._trace.enabled:
            duration = (time.monotonic_ns() - started) / 1000
            for request_id, futures in taken.items():
                self._trace.emit("save_store_wait_finished", request_id=request_id,
                                 stores=len(futures), duration_us=duration)

    def finished(self, request_ids) -> None:
        """get_finished's store cleanup (reference connector.py:551-557)."""
        for request_id in request_ids:
            self._store.release(request_id)
            for _, segment_id in self._chunk_ids.pop(request_id, ()):
                self._store.abort_put(segment_id)

    def close(self) -> None:
        """Wait for every publication (including ones enqueued meanwhile),
        then stop the copier and the publisher pool."""
        try:
            while self._inflight:
                for futures in self._inflight.take().values():
                    for future in futures:
                        future.result()
        finally:
            if self._copier is not None:
                self._copy_jobs.put(None)
                self._copier.join()
                self._copier = None
            self._staging.clear()
            self._publishers.shutdown(wait=True, cancel_futures=False)
