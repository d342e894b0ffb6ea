"""Recompute-token selection on MI355X: K-deviation, budgeted top-k, Sparse-Q.

Mirrors the selection half of the reference ``Qwen3BlendExecutor``
(cacheblend_vllm/ascend.py:534-566, 638-711, 757-796): the K-deviation score,
``_select`` and ``_sparse_q_scores`` keep their names, arguments and
results. The work runs in libcacheblend_hip.so:

* ``cbk_kdev_scores``  per-token sum of squared K differences (HBM-bound)
* ``cbk_select``       gap/forced/dilation masks + radix top-k + ordered
                       compaction, entirely on the GPU (the reference's
                       ``torch.topk`` + ``torch.where`` + host budget syncs)
* ``cbk_dilate``       overflow-block dilation of the gap mask

Ties at the k-th score go to the lower index (deterministic on every run and
every rank). The only host synchronisation is reading the selected count to
size the returned tensor, as the reference's ``torch.where`` does;
``select_async`` avoids even that.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native
from .trace import roctx_phase
from .config import CacheBlendConfig
from .kv_layout import write_rows


def _mask_u8(mask: torch.Tensor, n: int, what: str) -> torch.Tensor:
    if mask.shape != (n,):
        raise ValueError(f"{what} must have shape ({n},), got {tuple(mask.shape)}")
    if mask.dtype == torch.bool:
        mask = mask.contiguous().view(torch.uint8)
    else:
        mask = (mask != 0).contiguous().view(torch.uint8)
    return mask


def _row_view(t: torch.Tensor, what: str) -> torch.Tensor:
    if t.ndim != 2:
        t = t.reshape(t.shape[0], -1)
    if t.stride(1) != 1:
        t = t.contiguous()
    if t.dtype not in _native.DTYPE_CODES:
        raise ValueError(f"{what} dtype {t.dtype} is not supported")
    return t


def kdev_scores(
    fresh: torch.Tensor,
    cached: torch.Tensor,
    absolute_indices: torch.Tensor | None = None,
    row0: int = 0,
) -> torch.Tensor:
    """``sum((fresh.float() - cached[idx].float())**2, dim=-1)`` as float32.

    Reference ascend.py:534-538 (``cached`` is ``flat_old_k``, ``idx`` is
    ``absolute_indices``, or ``row0 + arange(N)`` when it is None).
    """
    fresh = _row_view(fresh, "fresh K")
    cached = _row_view(cached, "cached K")
    _native.require_device(fresh, "fresh K")
    if fresh.dtype != cached.dtype or fresh.device != cached.device:
        raise ValueError("fresh and cached K must share dtype and device")
    if fresh.shape[1] != cached.shape[1]:
        raise ValueError(f"row widths differ: {fresh.shape[1]} vs {cached.shape[1]}")
    n = fresh.shape[0]
    scores = torch.empty(n, dtype=torch.float32, device=fresh.device)
    idx = None
    if absolute_indices is not None:
        idx = absolute_indices.to(device=fresh.device, dtype=torch.long).contiguous()
        if idx.shape != (n,):
            raise ValueError("absolute_indices must have one entry per fresh row")
    rc = _native.load().cbk_kdev_scores(
        fresh.data_ptr(), fresh.stride(0), cached.data_ptr(), cached.stride(0), cached.shape[0],
        _native.ptr(idx), row0, n, fresh.shape[1], _native.DTYPE_CODES[fresh.dtype],
        scores.data_ptr(), _native.stream_handle(fresh.device),
    )
    _native.check(rc, "kdev_scores")
    return scores


def select_async(
    scores: torch.Tensor,
    gap_mask: torch.Tensor,
    ratio: float,
    forced_mask: torch.Tensor | None = None,
    radius: int = 0,
    flags: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Selection without a host sync: ``(indices[N] int64, count[1] int64)``;
    the first ``count`` entries of ``indices`` are the sorted selection.

    The count is -1 when the one-launch select could not hold the device (its
    workgroups must all be resident at once; kernels on other streams can
    keep CUs busy past its bounded wait) and wrote no index. ``select`` reads
    the count and then runs the multi-launch select; a caller of this
    function that cannot read it in between -- under graph capture, say --
    passes ``flags=_native.SELECT_MULTI_LAUNCH``, which never returns -1."""
    n = int(scores.shape[0])
    _native.require_device(scores, "scores")
    if scores.ndim != 1:
        raise ValueError("scores must be one-dimensional")
    if forced_mask is not None and forced_mask.shape != gap_mask.shape:
        raise ValueError("forced selection mask must match the active token shape")
    if scores.dtype != torch.float32:
        scores = scores.float()
    scores = scores.contiguous()
    gap = _mask_u8(gap_mask.to(scores.device), n, "gap_mask")
    forced = None if forced_mask is None else _mask_u8(forced_mask.to(scores.device), n, "forced_mask")
    out = torch.empty(max(n, 1), dtype=torch.long, device=scores.device)
    count = torch.empty(1, dtype=torch.long, device=scores.device)
    _launch_select(scores, gap, forced, n, radius, ratio, out, count, flags)
    return out, count


def _launch_select(scores, gap, forced, n, radius, ratio, out, count, flags):
    lib = _native.load()
    ws = _native.workspace(scores.device, lib.cbk_select_workspace_bytes(n))
    rc = lib.cbk_select_ex(
        scores.data_ptr(), gap.data_ptr(), _native.ptr(forced), n, int(radius), float(ratio),
        out.data_ptr(), count.data_ptr(), ws.data_ptr(), ws.numel(), int(flags),
        _native.stream_handle(scores.device),
    )
    _native.check(rc, "select")


def select(
    scores: torch.Tensor,
    gap_mask: torch.Tensor,
    ratio: float,
    forced_mask: torch.Tensor | None = None,
    radius: int = 0,
    flags: int = 0,
) -> torch.Tensor:
    """Sorted int64 indices of ``gap | forced | dilate(gap, radius) | top-k``.

    Reference ``_select`` (ascend.py:757-796) at TP1, with the budget
    ``int((N - #gap) * ratio)`` clamped to ``[1, available]``. A one-launch
    select that gave up (count -1) is run again as the multi-launch select.
    """
    out, count = select_async(scores, gap_mask, ratio, forced_mask, radius, flags)
    value = int(count.item())
    if value < 0:
        n = int(scores.shape[0])
        dev = scores.device
        forced = None if forced_mask is None else _mask_u8(forced_mask.to(dev), n, "forced_mask")
        _launch_select(scores.float().contiguous(), _mask_u8(gap_mask.to(dev), n, "gap_mask"), forced,
                       n, radius, ratio, out, count, _native.SELECT_MULTI_LAUNCH)
        value = _checked_count(count)
    return out[:value]


def _checked_count(count: torch.Tensor) -> int:
    value = int(count.item())
    if value < 0:  # the multi-launch select never writes -1
        raise RuntimeError(f"selection wrote a count of {value}")
    return value


def kdev_select(
    fresh: torch.Tensor,
    cached: torch.Tensor,
    absolute_indices: torch.Tensor | None,
    gap_mask: torch.Tensor,
    ratio: float,
    radius: int = 0,
    row0: int = 0,
    flags: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """K-deviation scores and their selection in one call (``cbk_kdev_select``).

    Returns ``(selected, scores)``; ``radius`` > 0 also forces every token
    within ``radius`` of a gap (overflow blocks). A one-launch select that
    gave up (count -1) is run again on the scores as the multi-launch select.
    """
    fresh = _row_view(fresh, "fresh K")
    cached = _row_view(cached, "cached K")
    _native.require_device(fresh, "fresh K")
    if fresh.dtype != cached.dtype or fresh.device != cached.device:
        raise ValueError("fresh and cached K must share dtype and device")
    n = fresh.shape[0]
    idx = None
    if absolute_indices is not None:
        idx = absolute_indices.to(device=fresh.device, dtype=torch.long).contiguous()
        if idx.shape != (n,):
            raise ValueError("absolute_indices must have one entry per fresh row")
    gap = _mask_u8(gap_mask.to(fresh.device), n, "gap_mask")
    scores = torch.empty(n, dtype=torch.float32, device=fresh.device)
    out = torch.empty(max(n, 1), dtype=torch.long, device=fresh.device)
    count = torch.empty(1, dtype=torch.long, device=fresh.device)
    lib = _native.load()
    nbytes = lib.cbk_select_workspace_bytes(n)
    ws = _native.workspace(fresh.device, nbytes)
    rc = lib.cbk_kdev_select_ex(
        fresh.data_ptr(), fresh.stride(0), cached.data_ptr(), cached.stride(0), cached.shape[0],
        _native.ptr(idx), row0, n, fresh.shape[1], _native.DTYPE_CODES[fresh.dtype],
        gap.data_ptr(), None, int(radius), float(ratio), scores.data_ptr(), out.data_ptr(),
        count.data_ptr(), ws.data_ptr(), ws.numel(), int(flags), _native.stream_handle(fresh.device),
    )
    _native.check(rc, "kdev_select")
    value = int(count.item())
    if value < 0:
        _launch_select(scores, gap, None, n, radius, ratio, out, count, _native.SELECT_MULTI_LAUNCH)
        value = _checked_count(count)
    return out[:value], scores


def dilate(gap_mask: torch.Tensor, radius: int) -> torch.Tensor:
    """``forced[i] = any(gap[i - radius : i + radius + 1])`` (ascend.py:662-671)."""
    n = int(gap_mask.shape[0])
    _native.require_device(gap_mask, "gap_mask")
    gap = _mask_u8(gap_mask, n, "gap_mask")
    out = torch.empty(n, dtype=torch.bool, device=gap_mask.device)
    rc = _native.load().cbk_dilate(
        gap.data_ptr(), n, int(radius), out.view(torch.uint8).data_ptr(),
        _native.stream_handle(gap_mask.device),
    )
    _native.check(rc, "dilate")
    return out


_ROUND_MODES = {torch.bfloat16: 1, torch.float16: 2, torch.float32: 0}


def sparse_q_full_scores(
    query: torch.Tensor,
    key: torch.Tensor,
    query_rows: torch.Tensor | None,
    positions: torch.Tensor,
    scale: float,
    out_index: torch.Tensor | None = None,
    want_full: bool = False,
) -> tuple[torch.Tensor | None, torch.Tensor | None]:
    """Per-key causal attention mass (``cbk_sparse_q_scores``).

    ``query`` is ``[N, Hq, D]``, ``key`` ``[K, Hkv, D]``; the sparse queries
    are ``query[query_rows]`` (all rows when None) at ``positions[row]``.
    Returns ``(full[out_index], full)`` (each None when not requested).
    Reference ascend.py:683-701.
    """
    _native.require_device(query, "query")
    if query.ndim != 3 or key.ndim != 3:
        raise ValueError("query must be [N, Hq, D] and key [K, Hkv, D]")
    n, hq, d = query.shape
    nk, hkv, dk = key.shape
    if hq % hkv:
        raise ValueError(
            "Sparse-Q requires query heads to be divisible by KV heads; "
            f"got {hq} and {hkv}"
        )
    if d != dk or query.dtype != key.dtype or query.device != key.device:
        raise ValueError("query and key must share head_dim, dtype and device")
    if query.dtype not in _ROUND_MODES:
        raise ValueError(f"Sparse-Q dtype {query.dtype} is not supported")
    if query.stride(2) != 1 or query.stride(1) != d:
        query = query.contiguous()
    if key.stride(2) != 1 or key.stride(1) != d:
        key = key.contiguous()
    dev = query.device
    rows = None
    nq = n
    if query_rows is not None:
        rows = query_rows.to(device=dev, dtype=torch.long).contiguous()
        nq = rows.numel()
    pos = positions.to(device=dev, dtype=torch.long).contiguous()
    out = full = None
    idx = None
    n_out = 0
    if out_index is not None:
        idx = out_index.to(device=dev, dtype=torch.long).contiguous()
        n_out = idx.numel()
        out = torch.empty(n_out, dtype=torch.float32, device=dev)
    if want_full:
        full = torch.empty(nk, dtype=torch.float32, device=dev)
    lib = _native.load()
    ws = _native.workspace(dev, lib.cbk_sparse_q_workspace_bytes(nq, nk, hq, hkv))
    rc = lib.cbk_sparse_q_scores(
        query.data_ptr(), query.stride(0), _native.ptr(rows), nq, pos.data_ptr(),
        key.data_ptr(), key.stride(0), nk, hq, hkv, d, float(scale),
        _native.DTYPE_CODES[query.dtype], _ROUND_MODES[query.dtype],
        _native.ptr(idx), n_out, _native.ptr(out), _native.ptr(full),
        ws.data_ptr(), ws.numel(), _native.stream_handle(dev),
    )
    _native.check(rc, "sparse_q_scores")
    return out, full


def sparse_q_masks(gap_mask: torch.Tensor, tail_query_tokens: int, radius: int, gap_count: int | None = None):
    """``(query_mask, forced_mask, has_gap)`` (reference ascend.py:652-671).

    Without gaps the last ``min(tail, N)`` tokens are queries and forced;
    with gaps and ``radius`` > 0 the forced set is dilated (``cbk_dilate``).
    ``gap_count``, when the caller has read it already, spares a host read.
    """
    query_mask = gap_mask.clone()
    forced = gap_mask.clone()
    has_gap = (gap_count > 0) if gap_count is not None else bool(gap_mask.any().item())
    if not has_gap:
        tail = min(tail_query_tokens, gap_mask.shape[0])
        query_mask[-tail:] = True
        forced[-tail:] = True
    if radius and has_gap:
        forced |= dilate(gap_mask, radius)
    return query_mask, forced, has_gap


def sparse_q_query_rows(query_mask: torch.Tensor, has_gap: bool, gap_count: int, tail_query_tokens: int):
    """The rows of ``query_mask`` in index order (``torch.nonzero``), with
    their count known from ``sparse_q_masks``' rule -- the gaps, else the
    tail, all N for a tail of 0 as Python's ``x[-0:]`` is ``x`` -- so the
    compaction needs no host read of its own."""
    n = int(query_mask.shape[0])
    if has_gap:
        n_rows = gap_count
    else:
        n_rows = min(tail_query_tokens, n) if tail_query_tokens else n
    return torch.nonzero_static(query_mask, size=n_rows).flatten()


@dataclass
class CheckLayerSelection:
    """What the check layer's selection block produces (ascend.py:529-531)."""

    deviation_selected: torch.Tensor | None
    sparse_q_selected: torch.Tensor | None
    sparse_q_stats: dict


class BlendSelector:
    """The selection methods of the reference ``Qwen3BlendExecutor``.

    ``_select`` and the K-deviation block keep the reference's signatures so
    an executor can delegate to them unchanged. With a TP group of more than
    one rank the scores are all-reduced first (reference ascend.py:768-769);
    every rank then runs the same deterministic selection, which replaces the
    reference's rank-0 top-k plus broadcast (ascend.py:787-796).
    """

    def __init__(self, config: CacheBlendConfig, block_size: int, tp_group=None):
        if block_size <= 0:
            raise ValueError("vLLM KV cache block_size must be positive")
        self.config = config
        self.block_size = block_size
        self.tp_group = tp_group

    def _reduce(self, scores: torch.Tensor) -> torch.Tensor:
        tp = self.tp_group
        if self.config.tp_global_selection and tp is not None and tp.world_size > 1:
            return tp.all_reduce(scores)
        return scores

    def _select(
        self,
        scores: torch.Tensor,
        gap_mask: torch.Tensor,
        layer_id: int | None = None,
        forced_mask: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Reference ascend.py:757-796."""
        if forced_mask is not None and forced_mask.shape != gap_mask.shape:
            raise ValueError("forced selection mask must match the active token shape")
        scores = self._reduce(scores)
        return select(scores, gap_mask, self.config.ratio_for(layer_id), forced_mask)

    def _sparse_q_scores(
        self,
        query: torch.Tensor,
        key: torch.Tensor,
        absolute_indices: torch.Tensor,
        gap_mask: torch.Tensor,
        scale: float,
    ) -> tuple[torch.Tensor, torch.Tensor, dict]:
        """Reference ascend.py:638-711: ``(scores[N], forced[N], stats)``.

        ``query`` ``[N, Hq, D]`` (active tokens), ``key`` ``[K, Hkv, D]`` (the
        whole context), ``absolute_indices[N]`` their positions. The score
        loop is one MFMA kernel pair instead of ``N / query_score_chunk_size``
        matmul + softmax launches; ``query_score_chunk_size`` bounds nothing
        here (the kernel streams K through registers and LDS).
        """
        radius = self.config.overflow_blocks * self.block_size
        if gap_mask.dtype != torch.bool:
            gap_mask = gap_mask != 0
        # the one host read before the scores; count_nonzero, as the masks
        # treat any nonzero entry as set (a sum would overcount 2s and size
        # the query compaction past the set rows)
        gap_count = int(gap_mask.count_nonzero().item())
        tail = self.config.tail_query_tokens
        query_mask, forced, has_gap = sparse_q_masks(gap_mask, tail, radius, gap_count=gap_count)
        sparse = sparse_q_query_rows(query_mask, has_gap, gap_count, tail)
        scores, _ = sparse_q_full_scores(query, key, sparse, absolute_indices, scale,
                                         out_index=absolute_indices)
        stats = {
            "active_tokens": int(query.shape[0]),
            "gap_tokens": gap_count,
            "cached_tokens": int(query.shape[0]) - gap_count,
            "sparse_query_tokens": int(sparse.numel()),
            "tail_fallback": not has_gap,
            "overflow_blocks": self.config.overflow_blocks,
        }
        return scores, forced, stats

    def sparse_q_select(
        self,
        query: torch.Tensor,
        score_keys: torch.Tensor,
        absolute_indices: torch.Tensor,
        gap_mask: torch.Tensor,
        scale: float,
        layer_id: int | None = None,
    ) -> tuple[torch.Tensor, dict]:
        """The check-layer Sparse-Q block (ascend.py:545-566): scores, then
        ``_select`` with the forced (gap + overflow / tail) mask."""
        scores, forced, stats = self._sparse_q_scores(query, score_keys, absolute_indices, gap_mask, scale)
        return self._select(scores, gap_mask, layer_id, forced_mask=forced), stats

    @roctx_phase("cacheblend.check_layer")
    def check_layer(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        flat_old_k: torch.Tensor,
        absolute_indices: torch.Tensor,
        active_gap_mask: torch.Tensor,
        layer_id: int,
        scale: float,
        num_heads: int,
        num_kv_heads: int,
        head_size: int,
        strategy: str | None = None,
        tracer=None,
        request_id: str | None = None,
    ) -> CheckLayerSelection:
        """The selection part of the reference's check layer
        (``Qwen3BlendExecutor._compute_layer``, ascend.py:533-580), for the
        configured (or given) ``selection_strategy``:

        kv_deviation -- K-deviation scores of the fresh ``k`` against
                        ``flat_old_k[absolute_indices]``, then ``_select``;
        sparse_q     -- ``flat_old_k[absolute_indices] = k`` in place (the
                        reference aliases ``score_keys`` to ``flat_old_k``),
                        Sparse-Q scores against it, then ``_select`` with the
                        forced mask;
        compare      -- both, Sparse-Q on a copy of ``flat_old_k``, and a
                        ``selection_compared`` trace event.
        The caller applies the result as the reference does: K-deviation
        (and compare) prune before the check-layer attention, Sparse-Q after.
        """
        strategy = strategy or self.config.selection_strategy
        if strategy not in ("kv_deviation", "sparse_q", "compare"):
            raise ValueError(f"unknown selection strategy {strategy!r}")
        result = CheckLayerSelection(None, None, {})
        if strategy in ("kv_deviation", "compare"):
            result.deviation_selected = self.kv_deviation_select(
                k, flat_old_k, absolute_indices, active_gap_mask, layer_id)
        if strategy in ("sparse_q", "compare"):
            score_keys = flat_old_k if strategy == "sparse_q" else flat_old_k.clone()
            write_rows(score_keys, absolute_indices, k.reshape(k.shape[0], -1))
            result.sparse_q_selected, result.sparse_q_stats = self.sparse_q_select(
                q.reshape(-1, num_heads, head_size), score_keys.view(-1, num_kv_heads, head_size),
                absolute_indices, active_gap_mask, scale, layer_id)
        if strategy == "sparse_q" and tracer is not None and tracer.enabled:
            # reference ascend.py:627-635 emits this once the Sparse-Q set is
            # applied to the check layer's output; the set is final here
            tracer.emit("selection_finished", request_id=request_id, layer_id=layer_id,
                        strategy="sparse_q", selected_tokens=result.sparse_q_selected.numel(),
                        **result.sparse_q_stats)
        if strategy == "compare" and tracer is not None and tracer.enabled:
            dev, sq = result.deviation_selected, result.sparse_q_selected
            size = max(int(dev.max()) if dev.numel() else -1, int(sq.max()) if sq.numel() else -1) + 1
            a = torch.zeros(size, dtype=torch.bool, device=dev.device)
            b = torch.zeros_like(a)
            a[dev] = True
            b[sq] = True
            overlap, union = int((a & b).sum()), int((a | b).sum())
            tracer.emit("selection_compared", request_id=request_id, layer_id=layer_id,
                        deviation_tokens=dev.numel(), sparse_q_tokens=sq.numel(), overlap_tokens=overlap,
                        jaccard=overlap / max(union, 1), **result.sparse_q_stats)
        return result

    def kv_deviation_select(
        self,
        k: torch.Tensor,
        flat_old_k: torch.Tensor,
        absolute_indices: torch.Tensor,
        gap_mask: torch.Tensor,
        layer_id: int | None = None,
        overflow_blocks: int = 0,
    ) -> torch.Tensor:
        """The check-layer K-deviation block (ascend.py:534-543).

        ``overflow_blocks`` > 0 additionally forces tokens within that many
        vLLM blocks of a gap (the dilation the reference applies to Sparse-Q
        only); 0 is the reference's K-deviation path exactly.
        """
        radius = overflow_blocks * self.block_size
        ratio = self.config.ratio_for(layer_id)
        if self.tp_group is not None and self.tp_group.world_size > 1:
            scores = self._reduce(kdev_scores(k, flat_old_k, absolute_indices))
            return select(scores, gap_mask, ratio, None, radius)
        selected, _ = kdev_select(k, flat_old_k, absolute_indices, gap_mask, ratio, radius)
        return selected
