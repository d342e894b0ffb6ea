"""Layerwise blend loader on MI355X: H2D of cached hits + one fused kernel.

``PagedBlendLoader`` keeps the reference's constructor and its
``prefetch`` / ``get`` / ``commit`` protocol (cacheblend_vllm/ascend.py:
170-407), so a layerwise executor drives it unchanged:

    loader.prefetch(0, rope)
    for l in layers:
        buf = loader.get(l)            # [2, allocation_end, H, D]
        loader.prefetch(l + 1, rope)   # overlaps with layer l's compute
        ... compute, writing recomputed K/V into buf ...
        loader.commit(l, buf)          # scatter [apc:] into the vLLM pages

Per layer, on the Load stream (a default-priority side stream):
  1. the hit chunks cross the host link: either DMA (``cbk_memcpy_runs``:
     chunks adjacent in pinned host memory folded into one copy per run and
     plane, chunks at a constant slot pitch into one 2D copy per plane, into
     a ring of device hit stagings ``[2, hit_tokens, H, D]``) or, for chunks
     scattered over the slab, in place -- the assembly kernel reads them
     from pinned host memory through a per-layer address table;
  2. ``cbk_blend_assemble`` (``_chunks`` for in-place reads) writes the
     layer buffer in one pass: APC prefix from the pages, zeros for gaps,
     hit rows with their K RoPE-relocated from source to target positions;
  3. an event, waited on by ``get``.
Two buffers alternate by layer parity; ``commit`` records a reuse event so
buffer ``l % 2`` is not overwritten before layer ``l``'s scatter has run.
All per-request tables (source map, old positions, slots) are built on the
host once and uploaded once.
"""

from __future__ import annotations

import time

import numpy as np
import torch

from . import _native
from .config import CacheBlendConfig, load_staging_layers
from .kv_layout import kv_desc, kv_planes
from .rope import cos_sin_table, rope_style
from .streams import COPY, LOAD, side_stream
from .trace import PipelineTracer, roctx_phase
from .types import BlendPlan

SRC_ZERO = -1
SRC_PAGE = -2


def build_source_map(plan: BlendPlan) -> tuple[np.ndarray, np.ndarray, bool]:
    """(src_map[allocation_end] int32, old_pos[hit_tokens] int32, relocate).

    src_map: ``-2`` APC prefix (page), ``-1`` gap (zero), ``r >= 0`` hit row r
    of the staging (segments concatenated in plan order, as the reference's
    fused copy stacks them, ascend.py:333-342). ``relocate`` is False exactly
    when every hit keeps its position (reference ``torch.equal`` shortcut,
    ascend.py:64-65).
    """
    src = np.full(plan.allocation_end, SRC_ZERO, dtype=np.int32)
    src[: plan.apc_prefix_tokens] = SRC_PAGE
    old = np.empty(plan.hit_tokens, dtype=np.int32)
    relocate = False
    off = 0
    for seg in plan.segments:
        n = seg.length
        src[seg.target_start : seg.target_end] = np.arange(off, off + n, dtype=np.int32)
        old[off : off + n] = np.arange(seg.source_start, seg.source_start + n, dtype=np.int32)
        relocate |= seg.source_start != seg.target_start
        off += n
    return src, old, relocate


def coalesce_host_runs(hosts: list[torch.Tensor]) -> list[tuple[int, int, torch.Tensor, torch.Tensor]]:
    """Group consecutive host chunks whose K planes (and V planes) are adjacent
    in one pinned allocation into ``(dst_offset, tokens, k_run, v_run)``."""
    runs: list[list] = []
    off = 0
    for host in hosts:
        k, v = host[0], host[1]
        n = k.shape[0]
        if not (k.is_contiguous() and v.is_contiguous()):
            k, v = k.contiguous(), v.contiguous()
        if runs:
            run = runs[-1]
            rk, rv = run[2], run[3]
            nbytes = rk.element_size() * rk[0].numel()
            if (
                k.untyped_storage().data_ptr() == rk.untyped_storage().data_ptr()
                and v.untyped_storage().data_ptr() == rv.untyped_storage().data_ptr()
                and k.data_ptr() == rk.data_ptr() + run[1] * nbytes
                and v.data_ptr() == rv.data_ptr() + run[1] * nbytes
                and k.dtype == rk.dtype
            ):
                run[1] += n
                off += n
                continue
        runs.append([off, n, k, v])
        off += n
    out = []
    for start, n, k, v in runs:
        if k.shape[0] != n:
            k = k.as_strided((n, *k.shape[1:]), k.stride(), k.storage_offset())
            v = v.as_strided((n, *v.shape[1:]), v.stride(), v.storage_offset())
        out.append((start, n, k, v))
    return out


class PagedBlendLoader:
    """Double-buffered layerwise H2D load, fused assembly and paged scatter."""

    def __init__(
        self,
        kv_caches: list,
        store,
        request_id: str,
        plan: BlendPlan,
        slot_mapping: torch.Tensor,
        block_size: int,
        config: CacheBlendConfig,
        tracer: PipelineTracer | None = None,
        load_stream: torch.cuda.Stream | None = None,
        copy_stream: torch.cuda.Stream | None = None,
        zero_copy: bool | str = "auto",
        max_workgroups: int = 256,
        dma_min_run_bytes: int = 1 << 20,
        dma_staging_layers: int | None = None,
    ):
        """How hit rows cross the host link, per layer:
        DMA -- the chunks, coalesced into runs where adjacent in host
               memory, are copied into a device hit staging by the DMA
               engines (no CUs taken from the layer's compute);
        host read -- when every hit chunk is a kernel-addressable
               ``[2, chunk, *row]`` host tensor (page-locked, contiguous
               16-byte aligned planes), the assembly kernel can read the hit
               rows in place (``max_workgroups`` bounds the CUs it holds).
        ``zero_copy``: True forces host reads where possible, False forces
        DMA, "auto" reads in place only when the DMA commands would average
        fewer than ``dma_min_run_bytes`` each, where per-command DMA cost
        (about 9 us, the time of 0.5 MB) dominates.
        ``dma_staging_layers`` (default: ``CACHEBLEND_LOAD_STAGING_LAYERS``
        from the environment, else 4):
        layers of hits the device ring the DMA fills holds (at least 2, at
        most the layer count). The host refills a slot only after the
        assembly that read it, so the copies run at most that many layers
        ahead of the assemblies; the ring costs that many layers' hit bytes
        of device memory per request (C3-shaped: 57 MB a layer)."""
        if zero_copy not in (True, False, "auto"):
            raise ValueError("zero_copy must be True, False or 'auto'")
        self.kv_caches = kv_caches
        self.store = store
        self.request_id = request_id
        self.plan = plan
        self.slot_mapping = slot_mapping[: plan.allocation_end]
        self.block_size = block_size
        self.config = config
        self.tracer = tracer
        key, _ = kv_planes(kv_caches[0])
        _native.require_device(key, "paged KV cache")
        self.device = key.device
        self.dtype = key.dtype
        self.row_shape = tuple(key.shape[2:])
        self._row_bytes = int(np.prod(self.row_shape)) * key.element_size()
        # hit bytes of each segment's plane, for the run search over host addresses
        lengths = np.array([seg.length for seg in plan.segments], dtype=np.int64)
        self._seg_plane_bytes = lengths * self._row_bytes
        self._seg_row_off = np.concatenate(([0], np.cumsum(lengths)))
        if self.slot_mapping.numel() < plan.allocation_end:
            raise ValueError(
                f"slot_mapping has {self.slot_mapping.numel()} slots for an allocation of "
                f"{plan.allocation_end} tokens"
            )
        src, old, relocate = build_source_map(plan)
        self._relocate = relocate
        self._src_map = torch.from_numpy(src).to(self.device)
        self._old_pos = torch.from_numpy(old).to(self.device) if old.size else None
        num_slots = key.shape[0] * block_size
        if self.slot_mapping.device.type == "cpu" and self.slot_mapping.numel():
            lo, hi = int(self.slot_mapping.min()), int(self.slot_mapping.max())
            if lo < 0 or hi >= num_slots:
                raise IndexError(f"slot_mapping holds slots in [{lo}, {hi}], outside [0, {num_slots})")
        self._slots = self.slot_mapping.to(device=self.device, dtype=torch.long).contiguous()
        self._buffers: dict[int, torch.Tensor] = {}
        self._events: dict[int, torch.cuda.Event] = {}
        self._reuse_events: dict[int, torch.cuda.Event] = {}
        self._staging: list[torch.Tensor] = []
        # ring of hit stagings, dma_staging_layers slots: the copy stream
        # carries no cross-stream waits (a wait between two DMA copies on
        # one stream left the engine idle ~50-100 us per layer); the host
        # fences a slot's reuse (_hit_free) when the ring wraps
        self._hit_ring: torch.Tensor | None = None
        self._hit_free: dict[int, torch.cuda.Event] = {}
        layers = load_staging_layers() if dma_staging_layers is None else int(dma_staging_layers)
        if layers < 2:
            raise ValueError("dma_staging_layers must be at least 2")
        self._ring_layers = layers
        # the last GPU event after which this loader reads no host memory
        self._host_reads: torch.cuda.Event | None = None
        self._copy_stream: torch.cuda.Stream | None = None
        self._descs: dict[int, _native.KVDesc] = {}
        self._zero_copy = zero_copy
        self._max_workgroups = max_workgroups
        self._dma_min_run_bytes = int(dma_min_run_bytes)
        self._ptr_host: torch.Tensor | None = None  # [layers, chunks, 2] pinned
        self._ptr_dev: torch.Tensor | None = None
        self._zc_layers: set[int] = set()
        self._load_stream = None
        if config.event_pipeline:
            self._load_stream = load_stream or side_stream(LOAD, self.device)
            self._copy_stream = copy_stream or side_stream(COPY, self.device)
            # tables made on the current stream are read on the Load stream
            for table in (self._src_map, self._old_pos, self._slots):
                if table is not None:
                    table.record_stream(self._load_stream)
        if tracer is not None and tracer.enabled:
            tracer.emit(
                "loader_initialized",
                request_id=request_id,
                apc_prefix_tokens=plan.apc_prefix_tokens,
                allocation_tokens=plan.allocation_tokens,
                hit_tokens=plan.hit_tokens,
                gap_tokens=plan.gap_tokens,
                segments=len(plan.segments),
            )

    # ------------------------------------------------------------ helpers

    def _desc(self, layer_id: int) -> _native.KVDesc:
        desc = self._descs.get(layer_id)
        if desc is None:
            desc, _ = kv_desc(self.kv_caches[layer_id], self.block_size)
            self._descs[layer_id] = desc
        return desc

    def _chunk_addresses(self, layer_id: int) -> tuple[int, list[int]] | None:
        """(chunk_tokens, flat [k0, v0, k1, v1, ...] host addresses) of the
        layer's hit chunks when every chunk is kernel-addressable and full
        (row h of the hits is row h % chunk of chunk h // chunk), else None."""
        lookup = getattr(self.store, "layer_chunk_addresses", None)
        if lookup is None:
            return None
        found = lookup(self.request_id, self.plan.segments, layer_id)
        if found is None:
            return None
        (chunk, row_shape, dtype), flat = found
        if row_shape != self.row_shape or dtype != self.dtype:
            return None
        if any(seg.length != chunk for seg in self.plan.segments[:-1]) or self.plan.segments[-1].length > chunk:
            return None
        return chunk, flat

    def _hit_copies(self, flat: list[int]) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """DMA run table of the layer's hits as uint64 arrays ``(dst offset in
        the hit staging, host src, bytes)``: every segment's K plane, then
        every V plane. ``cbk_memcpy_runs`` folds runs adjacent on both sides,
        and equal runs at constant pitches (consecutive slab slots), into
        single DMA commands."""
        kv = np.array(flat, dtype=np.uint64).reshape(-1, 2)
        off = self._seg_row_off[:-1].astype(np.uint64) * np.uint64(self._row_bytes)
        v_plane = np.uint64(self.plan.hit_tokens * self._row_bytes)
        plane = self._seg_plane_bytes.astype(np.uint64)
        return (np.concatenate((off, off + v_plane)), np.ascontiguousarray(kv.T).reshape(-1),
                np.concatenate((plane, plane)))

    def _hit_slot(self, layer_id: int) -> int:
        return layer_id % self._hit_ring.shape[0]

    def _ensure_hit_staging(self, layer_id: int) -> torch.Tensor:
        """The layer's slot of the hit ring, allocated on first use on the
        stream that fills it (the copy stream when there is one) and kept
        alive for the Load stream that reads it."""
        if self._hit_ring is None:
            slots = max(2, min(len(self.kv_caches), self._ring_layers))
            shape = (slots, 2, self.plan.hit_tokens, *self.row_shape)
            if self._copy_stream is not None:
                with torch.cuda.stream(self._copy_stream):
                    self._hit_ring = torch.empty(shape, dtype=self.dtype, device=self.device)
                self._hit_ring.record_stream(self._load_stream)
            else:
                self._hit_ring = torch.empty(shape, dtype=self.dtype, device=self.device)
        return self._hit_ring[self._hit_slot(layer_id)]

    def _load_hits(self, layer_id: int) -> None:
        found = self._chunk_addresses(layer_id)
        if found is not None:
            chunk, flat = found
            dst_off, src, nbytes = self._hit_copies(flat)
            host_read = self._zero_copy is True
            if self._zero_copy == "auto":
                commands = _native.memcpy_commands(dst_off, src, nbytes)
                host_read = int(nbytes.sum()) / max(1, commands) < self._dma_min_run_bytes
            if host_read:
                # publish the layer's chunk addresses; the assembly kernel
                # reads the hit rows over the host link
                if self._ptr_host is None:
                    layers = len(self.kv_caches)
                    self._ptr_host = torch.empty((layers, len(flat)), dtype=torch.int64, pin_memory=True)
                    self._ptr_dev = torch.empty((layers, len(flat)), dtype=torch.int64, device=self.device)
                table = self._ptr_host[layer_id]
                table.copy_(torch.tensor(flat, dtype=torch.int64))
                self._ptr_dev[layer_id].copy_(table, non_blocking=True)
                self._zc_layers.add(layer_id)
                self._zc_chunk = chunk
                return
            self._zc_layers.discard(layer_id)
            hit = self._ensure_hit_staging(layer_id)
            dst = dst_off + np.uint64(hit.data_ptr())
            if self._load_stream is None:
                _native.memcpy_runs(dst, src, nbytes, _native.stream_handle(self.device), "hit runs H2D")
                return
            # DMA on the copy stream, back to back with the previous layer's;
            # a ring slot is refilled only after the assembly that read it
            # (host-side fence: the host is then a full ring ahead of the copies)
            free = self._hit_free.pop(self._hit_slot(layer_id), None)
            if free is not None and not free.query():
                free.synchronize()
            _native.memcpy_runs(dst, src, nbytes, self._copy_stream.cuda_stream, "hit runs H2D")
            copied = torch.cuda.Event()
            copied.record(self._copy_stream)
            self._load_stream.wait_event(copied)
            return
        self._zc_layers.discard(layer_id)
        hosts = [self.store.get_layer(self.request_id, seg, layer_id) for seg in self.plan.segments]
        hit = self._ensure_hit_staging(layer_id)
        for off, n, k, v in coalesce_host_runs(hosts):
            hit[0, off : off + n].copy_(k, non_blocking=True)
            hit[1, off : off + n].copy_(v, non_blocking=True)

    def _assemble(self, layer_id: int, buffer: torch.Tensor, rotary_emb) -> None:
        es = buffer.element_size()
        hit = self._hit_ring[self._hit_slot(layer_id)] if self._hit_ring is not None else None
        heads = int(np.prod(self.row_shape[:-1])) if len(self.row_shape) > 1 else 1
        head_dim = self.row_shape[-1]
        table = None
        neox = 0
        if self._relocate:
            head_size, neox_style = rope_style(rotary_emb)
            if head_size != head_dim or int(getattr(rotary_emb, "rotary_dim", head_size)) != head_size:
                raise ValueError("CacheBlend relocation requires rotary_dim == head_size == head_dim")
            table = cos_sin_table(rotary_emb, self.dtype, self.device)
            neox = int(neox_style)
            limit = max(self.plan.allocation_end, max(
                (s.source_start + s.length for s in self.plan.segments), default=0))
            if limit > table.shape[0]:
                raise IndexError(f"positions up to {limit} exceed the RoPE cache of {table.shape[0]}")
        apc = self.plan.apc_prefix_tokens
        if layer_id in self._zc_layers:
            row_bytes = int(np.prod(self.row_shape)) * es
            rc = _native.load().cbk_blend_assemble_chunks(
                self._desc(layer_id) if apc else None,
                self._slots.data_ptr() if apc else None,
                self._src_map.data_ptr(),
                self.plan.allocation_end,
                self._ptr_dev[layer_id].data_ptr(),
                self._zc_chunk,
                row_bytes,
                self.plan.hit_tokens,
                _native.ptr(self._old_pos),
                _native.ptr(table),
                table.stride(0) if table is not None else 0,
                table.shape[0] if table is not None else 0,
                heads,
                head_dim,
                int(self._relocate),
                neox,
                _native.DTYPE_CODES[self.dtype],
                buffer[0].data_ptr(),
                buffer[1].data_ptr(),
                buffer.stride(1) * es,
                None,
                self._max_workgroups,
                _native.stream_handle(self.device),
            )
            _native.check(rc, "blend assemble (host chunks)")
            return
        rc = _native.load().cbk_blend_assemble(
            self._desc(layer_id) if apc else None,
            self._slots.data_ptr() if apc else None,
            self._src_map.data_ptr(),
            self.plan.allocation_end,
            hit[0].data_ptr() if hit is not None else None,
            hit[1].data_ptr() if hit is not None else None,
            hit.stride(1) * es if hit is not None else 0,
            self.plan.hit_tokens,
            _native.ptr(self._old_pos),
            None,
            _native.ptr(table),
            table.stride(0) if table is not None else 0,
            table.shape[0] if table is not None else 0,
            heads,
            head_dim,
            int(self._relocate),
            neox,
            _native.DTYPE_CODES[self.dtype],
            buffer[0].data_ptr(),
            buffer[1].data_ptr(),
            buffer.stride(1) * es,
            None,
            _native.stream_handle(self.device),
        )
        _native.check(rc, "blend assemble")

    # ----------------------------------------------------------- protocol

    @roctx_phase("cacheblend.prefetch")
    def prefetch(self, layer_id: int, rotary_emb) -> None:
        """Enqueue layer ``layer_id``'s load (reference ascend.py:224-278)."""
        if layer_id in self._buffers or layer_id >= len(self.kv_caches):
            return
        trace = self.tracer is not None and self.tracer.enabled
        started = time.monotonic_ns() if trace else 0

        def load() -> None:
            if not self._staging:
                shape = (2, self.plan.allocation_end, *self.row_shape)
                self._staging = [
                    torch.empty(shape, dtype=self.dtype, device=self.device) for _ in range(2)
                ]
            index = layer_id % 2
            reuse = self._reuse_events.pop(index, None)
            if reuse is not None:
                torch.cuda.current_stream(self.device).wait_event(reuse)
            buffer = self._staging[index]
            if self.plan.segments:
                self._load_hits(layer_id)
            self._assemble(layer_id, buffer, rotary_emb)
            if self._copy_stream is not None and self._hit_ring is not None and layer_id not in self._zc_layers:
                done = torch.cuda.Event()
                done.record(self._load_stream)
                self._hit_free[self._hit_slot(layer_id)] = done
            self._buffers[layer_id] = buffer

        if self._load_stream is None:
            load()
            if self.plan.segments:
                self._host_reads = torch.cuda.Event()
                self._host_reads.record(torch.cuda.current_stream(self.device))
        else:
            with torch.cuda.stream(self._load_stream):
                load()
                event = torch.cuda.Event()
                event.record(self._load_stream)
                self._events[layer_id] = event
            if self.plan.segments:
                # the Load stream ran this layer's assembly after its copies
                self._host_reads = event
        if trace:
            self.tracer.emit(
                "layer_prefetch_enqueued",
                request_id=self.request_id,
                layer_id=layer_id,
                duration_us=(time.monotonic_ns() - started) / 1000,
            )

    def host_reads_done(self) -> torch.cuda.Event | None:
        """GPU event after which no load enqueued so far reads the store's
        host memory (hit copies and in-place reads both complete before the
        Load stream passes it); None when nothing was read. The connector
        hands it to ``store.release`` so chunks evicted afterwards are not
        reused while a copy may still read them."""
        return self._host_reads

    def get(self, layer_id: int) -> torch.Tensor:
        """The layer's buffer, ordered after its load (ascend.py:372-383)."""
        event = self._events.pop(layer_id, None)
        current = torch.cuda.current_stream(self.device)
        if event is not None:
            current.wait_event(event)
            # the buffer was allocated on the Load stream; keep its memory
            # until the consuming stream is done with it
            self._buffers[layer_id].record_stream(current)
        if self.tracer is not None and self.tracer.enabled:
            self.tracer.emit(
                "layer_prefetch_wait_enqueued",
                request_id=self.request_id,
                layer_id=layer_id,
                had_event=event is not None,
            )
        return self._buffers.pop(layer_id)

    @roctx_phase("cacheblend.commit")
    def commit(self, layer_id: int, contiguous: torch.Tensor) -> None:
        """Scatter ``contiguous[:, apc:]`` into the layer's vLLM pages through
        ``slot_mapping[apc:]`` (ascend.py:385-407); APC pages are untouched."""
        start = self.plan.apc_prefix_tokens
        end = self.plan.allocation_end
        if start >= end:
            return
        if tuple(contiguous.shape) != (2, end, *self.row_shape) or contiguous.dtype != self.dtype:
            raise ValueError(
                f"commit expects [2, {end}, {', '.join(map(str, self.row_shape))}] {self.dtype}"
            )
        src = contiguous if contiguous[0].is_contiguous() and contiguous[1].is_contiguous() else contiguous.contiguous()
        es = src.element_size()
        rc = _native.load().cbk_paged_scatter(
            src[0, start].data_ptr(),
            src[1, start].data_ptr(),
            src.stride(1) * es,
            self._desc(layer_id),
            self._slots[start:].data_ptr(),
            end - start,
            None,
            _native.stream_handle(self.device),
        )
        _native.check(rc, "blend commit")
        if self._load_stream is not None:
            event = torch.cuda.Event()
            event.record(torch.cuda.current_stream(self.device))
            self._reuse_events[layer_id % 2] = event
        if self.tracer is not None and self.tracer.enabled:
            self.tracer.emit(
                "layer_committed",
                request_id=self.request_id,
                layer_id=layer_id,
                suffix_tokens=end - start,
            )
