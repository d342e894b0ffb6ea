"""The reference's torch path restated with the same torch ops, on the CPU.

TEST / BASELINE INFRASTRUCTURE ONLY: ``bench.py`` times these functions as
the ``cpu_baseline`` (kind "port") and ``tests/`` pins them against the numpy
oracle. They use exactly the torch operations the reference uses, so their
host-core time is the reference's CPU cost for the same work:

* gather: advanced indexing ``kv[:, blocks, offsets]`` (cacheblend_vllm/kv_layout.py:110-121)
* scatter: ``kv[:, blocks, offsets] = contiguous`` (kv_layout.py:152-155)
* K-deviation: ``torch.sum((k.float() - old.float()) ** 2, dim=-1)`` (ascend.py:535-538)
* select: ``masked_fill`` + ``torch.topk`` + ``torch.where`` (ascend.py:770-793)
"""

from __future__ import annotations

import torch


def gather(kv_layer: torch.Tensor, slots: torch.Tensor, block_size: int) -> torch.Tensor:
    blocks, offsets = slots // block_size, slots % block_size
    return kv_layer[:, blocks, offsets]


def scatter(contiguous: torch.Tensor, kv_layer: torch.Tensor, slots: torch.Tensor, block_size: int) -> None:
    blocks, offsets = slots // block_size, slots % block_size
    kv_layer[:, blocks, offsets] = contiguous


def kdev_scores(k: torch.Tensor, old_k: torch.Tensor) -> torch.Tensor:
    return torch.sum((k.float() - old_k.float()) ** 2, dim=-1)


def select(scores: torch.Tensor, gap_mask: torch.Tensor, ratio: float,
           forced_mask: torch.Tensor | None = None) -> torch.Tensor:
    base = gap_mask.clone()
    if forced_mask is not None:
        base |= forced_mask
    cached = scores.numel() - torch.where(gap_mask)[0].numel()
    topk = int(cached * ratio)
    available = scores.numel() - torch.where(base)[0].numel()
    topk = min(max(topk, 1), available) if cached and available else 0
    selected = base
    if topk:
        masked = scores.masked_fill(base, float("-inf"))
        selected[torch.topk(masked, k=topk).indices] = True
    return torch.where(selected)[0]


def dilate(gap_mask: torch.Tensor, radius: int) -> torch.Tensor:
    values = gap_mask.to(torch.int32)
    prefix = torch.cat((values.new_zeros(1), values.cumsum(0)))
    positions = torch.arange(values.numel())
    left = (positions - radius).clamp_min(0)
    right = (positions + radius + 1).clamp_max(values.numel())
    return prefix[right] > prefix[left]
