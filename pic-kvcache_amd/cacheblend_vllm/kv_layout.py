"""Paged KV gather/scatter for vLLM KV layouts on MI355X.

Drop-in for the reference module of the same name
(cacheblend_vllm/kv_layout.py): same functions, arguments, return values and
exceptions, executed by the gfx950 bandwidth kernels of libcacheblend_hip.so
(cbk_paged_gather / cbk_paged_scatter and their multi-layer forms).

Layouts (reference kv_layout.py:12-20, 110-118):
  separate      (K, V), each [num_blocks, block_size, *row]
  merged_first  [2, num_blocks, block_size, *row]   (tested first)
  merged_block  [num_blocks, 2, block_size, *row]
The ``*row`` dims of one token (normally [kv_heads, head_dim]) must be
contiguous. Slots index ``block * block_size + offset``.

Differences from the reference torch path, on purpose:
  * slots outside ``[0, num_blocks * block_size)`` raise ``IndexError`` when
    the slot tensor is on the host (torch would wrap negative slots). Device
    slot tensors are not read back (no sync); an out-of-range device slot
    gathers a zero row / skips the write instead of faulting.
  * results are always contiguous ``[2, T, *row]`` (the reference returns a
    transposed view for merged_block).
"""

from __future__ import annotations

import ctypes
from collections.abc import Sequence

import torch

from . import _native

KVLayer = torch.Tensor | Sequence[torch.Tensor]


def _separate(kv_layer: KVLayer) -> tuple[torch.Tensor, torch.Tensor] | None:
    """Follows reference kv_layout.py:12-20."""
    if isinstance(kv_layer, torch.Tensor):
        return None
    if len(kv_layer) != 2:
        raise ValueError(f"separate KV layout requires two tensors, got {len(kv_layer)}")
    key, value = kv_layer
    if not isinstance(key, torch.Tensor) or not isinstance(value, torch.Tensor):
        raise TypeError("separate KV layout must contain tensors")
    return key, value


def kv_planes(kv_layer: KVLayer) -> tuple[torch.Tensor, torch.Tensor]:
    """``(K, V)`` views shaped ``[num_blocks, block_size, *row]``."""
    separate = _separate(kv_layer)
    if separate is not None:
        return separate
    assert isinstance(kv_layer, torch.Tensor)
    if kv_layer.shape[0] == 2:
        return kv_layer[0], kv_layer[1]
    if kv_layer.ndim >= 4 and kv_layer.shape[1] == 2:
        return kv_layer[:, 0], kv_layer[:, 1]
    raise ValueError(f"unsupported vLLM KV layout {tuple(kv_layer.shape)}")


def _rows_contiguous(t: torch.Tensor, first_row_dim: int) -> bool:
    expected = 1
    for dim in range(t.ndim - 1, first_row_dim - 1, -1):
        if t.shape[dim] != 1 and t.stride(dim) != expected:
            return False
        expected *= t.shape[dim]
    return True


def kv_desc(kv_layer: KVLayer, block_size: int) -> tuple[_native.KVDesc, torch.Tensor]:
    """Describe one paged layer for the C ABI; returns (desc, K plane)."""
    key, value = kv_planes(kv_layer)
    if key.shape != value.shape or key.dtype != value.dtype or key.device != value.device:
        raise ValueError("K and V planes must share shape, dtype and device")
    if key.ndim < 3:
        raise ValueError(f"unsupported vLLM KV layout {tuple(key.shape)}")
    if block_size <= 0 or block_size > key.shape[1]:
        raise ValueError(f"block_size {block_size} does not fit KV blocks of {key.shape[1]} tokens")
    if key.stride() != value.stride():
        raise ValueError("K and V planes must share strides")
    if not _rows_contiguous(key, 2):
        raise ValueError("each token's KV row must be contiguous in the paged cache")
    _native.require_device(key, "paged KV cache")
    es = key.element_size()
    row_elems = 1
    for d in key.shape[2:]:
        row_elems *= d
    desc = _native.KVDesc(
        key.data_ptr(),
        value.data_ptr(),
        key.shape[0],
        block_size,
        key.stride(0) * es,
        key.stride(1) * es,
        row_elems * es,
    )
    return desc, key


def _device_slots(slot_mapping: torch.Tensor, device: torch.device, num_slots: int) -> torch.Tensor:
    """Reference kv_layout.py:23-24, plus a host-side range check."""
    if slot_mapping.device.type == "cpu" and slot_mapping.numel():
        lo = int(slot_mapping.min())
        hi = int(slot_mapping.max())
        if lo < 0 or hi >= num_slots:
            raise IndexError(
                f"slot_mapping holds slots in [{lo}, {hi}], outside [0, {num_slots})"
            )
    return slot_mapping.to(device=device, dtype=torch.long, non_blocking=True).contiguous()


def _plane_rows_ok(plane: torch.Tensor) -> bool:
    return _rows_contiguous(plane, 1)


def gather_paged_kv(
    kv_layer: KVLayer,
    slot_mapping: torch.Tensor,
    block_size: int,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Gather paged KV as contiguous ``[2, tokens, *row]``.

    Drop-in for reference kv_layout.py:90-122; runs cbk_paged_gather.
    """
    desc, key = kv_desc(kv_layer, block_size)
    tokens = int(slot_mapping.numel())
    shape = (2, tokens, *key.shape[2:])
    if out is not None:
        if tuple(out.shape) != shape:
            raise ValueError(f"gather output has shape {tuple(out.shape)}, expected {shape}")
        if out.dtype != key.dtype or out.device != key.device:
            raise ValueError("gather output must match the KV cache dtype and device")
        target = out
    else:
        target = torch.empty(shape, dtype=key.dtype, device=key.device)
    if tokens == 0:
        return target
    direct = (
        _plane_rows_ok(target[0])
        and _plane_rows_ok(target[1])
        and target.stride(1) == target[0].stride(0)
    )
    dst = target if direct else torch.empty(shape, dtype=key.dtype, device=key.device)
    slots = _device_slots(slot_mapping, key.device, desc.num_blocks * block_size)
    es = key.element_size()
    lib = _native.load()
    rc = lib.cbk_paged_gather(
        desc,
        slots.data_ptr(),
        tokens,
        dst[0].data_ptr(),
        dst[1].data_ptr(),
        dst.stride(1) * es,
        None,
        _native.stream_handle(key.device),
    )
    _native.check(rc, "gather_paged_kv")
    if dst is not target:
        target.copy_(dst)
    return target


def scatter_paged_kv(
    contiguous: torch.Tensor,
    kv_layer: KVLayer,
    slot_mapping: torch.Tensor,
    block_size: int,
) -> None:
    """Scatter ``[2, tokens, *row]`` into a vLLM paged KV layer in place.

    Drop-in for reference kv_layout.py:125-161; runs cbk_paged_scatter.
    """
    if contiguous.shape[0] != 2:
        raise ValueError("contiguous KV must have K/V as its first dimension")
    desc, key = kv_desc(kv_layer, block_size)
    tokens = int(slot_mapping.numel())
    shape = (2, tokens, *key.shape[2:])
    if tuple(contiguous.shape) != shape:
        raise ValueError(f"contiguous KV has shape {tuple(contiguous.shape)}, expected {shape}")
    if contiguous.dtype != key.dtype:
        raise RuntimeError(
            "Index put requires the source and destination dtypes match, "
            f"got {key.dtype} for the destination and {contiguous.dtype} for the source."
        )
    if tokens == 0:
        return
    src = contiguous.to(device=key.device)
    if not (_plane_rows_ok(src[0]) and _plane_rows_ok(src[1]) and src.stride(1) == src[0].stride(0)):
        src = src.contiguous()
    slots = _device_slots(slot_mapping, key.device, desc.num_blocks * block_size)
    es = key.element_size()
    lib = _native.load()
    rc = lib.cbk_paged_scatter(
        src[0].data_ptr(),
        src[1].data_ptr(),
        src.stride(1) * es,
        desc,
        slots.data_ptr(),
        tokens,
        None,
        _native.stream_handle(key.device),
    )
    _native.check(rc, "scatter_paged_kv")


def _layer_descs(kv_layers: Sequence[KVLayer], block_size: int):
    if len(kv_layers) == 0:
        raise ValueError("at least one KV layer is required")
    descs = (_native.KVDesc * len(kv_layers))()
    first = None
    for i, layer in enumerate(kv_layers):
        desc, key = kv_desc(layer, block_size)
        if first is None:
            first = key
        elif key.shape != first.shape or key.dtype != first.dtype or key.stride() != first.stride():
            raise ValueError("every KV layer must share shape, dtype and strides")
        descs[i] = desc
    return descs, first


def gather_paged_kv_layers(
    kv_layers: Sequence[KVLayer],
    slot_mapping: torch.Tensor,
    block_size: int,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Gather the same slots of every layer into ``[L, 2, tokens, *row]``.

    One kernel launch per 64 layers (cbk_paged_gather_layers); equals
    ``stack([gather_paged_kv(l, slot_mapping, block_size) for l in kv_layers])``.
    """
    descs, key = _layer_descs(kv_layers, block_size)
    tokens = int(slot_mapping.numel())
    shape = (len(kv_layers), 2, tokens, *key.shape[2:])
    if out is None:
        out = torch.empty(shape, dtype=key.dtype, device=key.device)
    elif tuple(out.shape) != shape or out.dtype != key.dtype or out.device != key.device:
        raise ValueError(f"gather output has shape {tuple(out.shape)}, expected {shape}")
    if tokens == 0:
        return out
    if not out[0, 0].is_contiguous() or not out[0, 1].is_contiguous():
        raise ValueError("multi-layer gather output needs contiguous [tokens, *row] planes")
    slots = _device_slots(slot_mapping, key.device, descs[0].num_blocks * block_size)
    es = key.element_size()
    rc = _native.load().cbk_paged_gather_layers(
        descs,
        len(kv_layers),
        slots.data_ptr(),
        tokens,
        out.data_ptr(),
        out.stride(0) * es,
        out.stride(1) * es,
        out.stride(2) * es,
        None,
        _native.stream_handle(key.device),
    )
    _native.check(rc, "gather_paged_kv_layers")
    return out


def scatter_paged_kv_layers(
    contiguous: torch.Tensor,
    kv_layers: Sequence[KVLayer],
    slot_mapping: torch.Tensor,
    block_size: int,
) -> None:
    """Inverse of :func:`gather_paged_kv_layers` (cbk_paged_scatter_layers)."""
    descs, key = _layer_descs(kv_layers, block_size)
    tokens = int(slot_mapping.numel())
    shape = (len(kv_layers), 2, tokens, *key.shape[2:])
    if tuple(contiguous.shape) != shape:
        raise ValueError(f"contiguous KV has shape {tuple(contiguous.shape)}, expected {shape}")
    if contiguous.dtype != key.dtype:
        raise RuntimeError("source and destination dtypes must match")
    if tokens == 0:
        return
    src = contiguous.to(device=key.device)
    if not src[0, 0].is_contiguous() or not src[0, 1].is_contiguous():
        src = src.contiguous()
    slots = _device_slots(slot_mapping, key.device, descs[0].num_blocks * block_size)
    es = key.element_size()
    rc = _native.load().cbk_paged_scatter_layers(
        src.data_ptr(),
        src.stride(0) * es,
        src.stride(1) * es,
        src.stride(2) * es,
        descs,
        len(kv_layers),
        slots.data_ptr(),
        tokens,
        None,
        _native.stream_handle(key.device),
    )
    _native.check(rc, "scatter_paged_kv_layers")


def _row_table(t: torch.Tensor, what: str) -> tuple[int, int]:
    """(row stride, row bytes) of a tensor whose dim 0 indexes rows and whose
    remaining dims are contiguous."""
    if t.dim() < 1 or not _rows_contiguous(t, 1):
        raise ValueError(f"{what} rows must be contiguous after dim 0")
    es = t.element_size()
    return t.stride(0) * es, (t.numel() // max(1, t.shape[0])) * es


def write_rows(dst: torch.Tensor, indices: torch.Tensor, src: torch.Tensor) -> None:
    """``dst[indices] = src`` for a row table ``dst [R, ...]`` and ``src [T, ...]``
    (same row shape and dtype, unique indices): the reference's
    ``score_keys[absolute_indices] = k`` (cacheblend_vllm/ascend.py:552), one
    ``cbk_paged_scatter`` launch over a block-size-1, K-only descriptor."""
    _native.require_device(dst, "dst")
    _native.require_device(src, "src")
    if src.dtype != dst.dtype:
        raise ValueError(f"src dtype {src.dtype} does not match dst dtype {dst.dtype}")
    if indices.numel() != src.shape[0]:
        raise ValueError(f"{indices.numel()} indices for {src.shape[0]} rows")
    d_stride, row_bytes = _row_table(dst, "dst")
    s_stride, s_row = _row_table(src, "src")
    if s_row != row_bytes:
        raise ValueError("src and dst rows differ in size")
    if src.shape[0] == 0:
        return
    desc = _native.KVDesc(dst.data_ptr(), None, dst.shape[0], 1, d_stride, d_stride, row_bytes)
    slots = _device_slots(indices, dst.device, dst.shape[0])
    rc = _native.load().cbk_paged_scatter(src.data_ptr(), None, s_stride, ctypes.byref(desc),
                                          slots.data_ptr(), src.shape[0], None,
                                          _native.stream_handle(dst.device))
    _native.check(rc, "write_rows")


def write_back_kv(old_kv: torch.Tensor, indices: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """``old_kv[0][indices] = k`` and ``old_kv[1][indices] = v`` for the layer
    buffer ``[2, A, H, D]`` and recomputed ``k``/``v`` ``[T, H*D]`` -- the
    check layer's write-back (reference ascend.py:592-595) -- in one launch."""
    _native.require_device(old_kv, "old_kv")
    if old_kv.dim() < 3 or old_kv.shape[0] != 2:
        raise ValueError("old_kv must be [2, tokens, ...]")
    if k.shape != v.shape or k.dtype != old_kv.dtype or v.dtype != old_kv.dtype:
        raise ValueError("k and v must have the same shape and the buffer's dtype")
    if indices.numel() != k.shape[0]:
        raise ValueError(f"{indices.numel()} indices for {k.shape[0]} rows")
    planes_ok = _rows_contiguous(old_kv[0], 1) and _rows_contiguous(old_kv[1], 1)
    if not planes_ok or old_kv[0].stride(0) != old_kv[1].stride(0):
        raise ValueError("old_kv planes must hold contiguous rows with one row stride")
    es = old_kv.element_size()
    row_bytes = (old_kv[0].numel() // old_kv.shape[1]) * es
    if k.numel() // max(1, k.shape[0]) * es != row_bytes:
        raise ValueError("k/v rows do not match the buffer's rows")
    if k.shape[0] == 0:
        return
    if not (_rows_contiguous(k, 1) and _rows_contiguous(v, 1)) or k.stride(0) != v.stride(0):
        k, v = k.contiguous(), v.contiguous()
    stride = old_kv.stride(1) * es
    desc = _native.KVDesc(old_kv[0].data_ptr(), old_kv[1].data_ptr(), old_kv.shape[1], 1, stride, stride,
                          row_bytes)
    slots = _device_slots(indices, old_kv.device, old_kv.shape[1])
    rc = _native.load().cbk_paged_scatter(k.data_ptr(), v.data_ptr(), k.stride(0) * es, ctypes.byref(desc),
                                          slots.data_ptr(), k.shape[0], None,
                                          _native.stream_handle(old_kv.device))
    _native.check(rc, "write_back_kv")


def scatter_chunks(chunks: Sequence[torch.Tensor], kv_layer: KVLayer, slot_mapping: torch.Tensor,
                   block_size: int, max_workgroups: int = 256) -> None:
    """Scatter chunk-format rows into a paged layer in place: token ``t`` of
    ``slot_mapping`` is row ``t % chunk`` of ``chunks[t // chunk]``, each a
    ``[2, chunk, *row]`` tensor with contiguous K and V planes -- the store's
    host chunks (page-locked memory, read over the host link) or device
    tensors. The reload of stored chunks (the reference's H2D copy then
    ``scatter_paged_kv``, ascend.py:224-278 and kv_layout.py:125-161) in one
    launch and without a device staging: cbk_paged_scatter_chunks.
    ``max_workgroups`` bounds the CUs the copy holds (over the host link the
    rate grows with them)."""
    desc, key = kv_desc(kv_layer, block_size)
    tokens = int(slot_mapping.numel())
    if tokens == 0:
        return
    if not chunks:
        raise ValueError("no chunks to scatter")
    first = chunks[0]
    chunk = int(first.shape[1]) if first.dim() >= 2 else 0
    shape = (2, chunk, *key.shape[2:])
    needed = (tokens + chunk - 1) // chunk if chunk else 0
    if chunk <= 0 or len(chunks) < needed:
        raise ValueError(f"{tokens} tokens need {needed} chunks of {chunk}, got {len(chunks)}")
    k_ptrs = (ctypes.c_void_p * needed)()
    v_ptrs = (ctypes.c_void_p * needed)()
    for i, c in enumerate(chunks[:needed]):
        if tuple(c.shape) != shape or c.dtype != key.dtype:
            raise ValueError(f"chunk {i} is {tuple(c.shape)} {c.dtype}, expected {shape} {key.dtype}")
        if not (c[0].is_contiguous() and c[1].is_contiguous()):
            raise ValueError(f"chunk {i}: K and V planes must each be contiguous")
        if c.device.type == "cpu":
            if not _native.host_accessible(c):
                raise ValueError(f"chunk {i} is not page-locked host memory the GPU can read")
        elif c.device != key.device:
            raise ValueError(f"chunk {i} is on {c.device}, the cache on {key.device}")
        k_ptrs[i] = c[0].data_ptr()
        v_ptrs[i] = c[1].data_ptr()
    slots = _device_slots(slot_mapping, key.device, desc.num_blocks * block_size)
    rc = _native.load().cbk_paged_scatter_chunks(
        k_ptrs, v_ptrs, chunk, desc.row_bytes, desc, slots.data_ptr(), tokens, int(max_workgroups), None,
        _native.stream_handle(key.device),
    )
    _native.check(rc, "scatter_chunks")


class PagedKVCache:
    """A model's registered paged KV layers (one descriptor per layer, built
    once, as the connector's ``register_kv_caches`` receives them, reference
    connector.py:168-175), with batched gather/scatter over any subset.

    Calls cost one C-ABI launch per 64 layers and no per-layer Python work.
    """

    def __init__(self, kv_layers: Sequence[KVLayer], block_size: int):
        self.kv_layers = list(kv_layers)
        self.block_size = int(block_size)
        self._descs, self._key = _layer_descs(self.kv_layers, self.block_size)
        self.num_layers = len(self.kv_layers)
        self.row_shape = tuple(self._key.shape[2:])
        self.dtype = self._key.dtype
        self.device = self._key.device
        self.num_slots = self._descs[0].num_blocks * self.block_size
        self._es = self._key.element_size()

    def _slots(self, slot_mapping: torch.Tensor) -> torch.Tensor:
        if slot_mapping.device == self.device and slot_mapping.dtype == torch.long:
            return slot_mapping if slot_mapping.is_contiguous() else slot_mapping.contiguous()
        return _device_slots(slot_mapping, self.device, self.num_slots)

    def layer_desc(self, layer: int) -> _native.KVDesc:
        return self._descs[layer]

    def gather(self, slot_mapping: torch.Tensor, out: torch.Tensor | None = None,
               layers: tuple[int, int] | None = None) -> torch.Tensor:
        """``out[l, c, t] = layer l plane c at slot t`` for layers ``[l0, l1)``."""
        l0, l1 = layers or (0, self.num_layers)
        tokens = int(slot_mapping.numel())
        shape = (l1 - l0, 2, tokens, *self.row_shape)
        if out is None:
            out = torch.empty(shape, dtype=self.dtype, device=self.device)
        elif tuple(out.shape) != shape or out.dtype != self.dtype:
            raise ValueError(f"gather output has shape {tuple(out.shape)}, expected {shape}")
        if tokens == 0:
            return out
        slots = self._slots(slot_mapping)
        es = self._es
        rc = _native.load().cbk_paged_gather_layers(
            ctypes_addressof(self._descs, l0), l1 - l0, slots.data_ptr(), tokens, out.data_ptr(),
            out.stride(0) * es, out.stride(1) * es, out.stride(2) * es, None,
            _native.stream_handle(self.device),
        )
        _native.check(rc, "PagedKVCache.gather")
        return out

    def scatter(self, contiguous: torch.Tensor, slot_mapping: torch.Tensor,
                layers: tuple[int, int] | None = None) -> None:
        """Inverse of :meth:`gather`."""
        l0, l1 = layers or (0, self.num_layers)
        tokens = int(slot_mapping.numel())
        shape = (l1 - l0, 2, tokens, *self.row_shape)
        if tuple(contiguous.shape) != shape or contiguous.dtype != self.dtype:
            raise ValueError(f"contiguous KV has shape {tuple(contiguous.shape)}, expected {shape}")
        if tokens == 0:
            return
        if not contiguous[0, 0].is_contiguous() or not contiguous[0, 1].is_contiguous():
            contiguous = contiguous.contiguous()
        slots = self._slots(slot_mapping)
        es = self._es
        rc = _native.load().cbk_paged_scatter_layers(
            contiguous.data_ptr(), contiguous.stride(0) * es, contiguous.stride(1) * es,
            contiguous.stride(2) * es, ctypes_addressof(self._descs, l0), l1 - l0,
            slots.data_ptr(), tokens, None, _native.stream_handle(self.device),
        )
        _native.check(rc, "PagedKVCache.scatter")


def ctypes_addressof(descs, index: int):
    """Pointer to ``descs[index]`` inside a ctypes array of KVDesc."""
    import ctypes

    return ctypes.cast(
        ctypes.byref(descs, index * ctypes.sizeof(_native.KVDesc)), ctypes.POINTER(_native.KVDesc)
    )
