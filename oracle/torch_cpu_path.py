"""The reference's torch path restated with the same torch ops, on the CPU.

TEST / BASELINE INFRASTRUCTURE ONLY: ``bench.py`` times these functions as
the ``cpu_baseline`` (kind "port") and ``tests/test_torch_cpu_path.py`` pins
them against the numpy oracle. They use exactly the torch operations the
reference uses, so their host-core time is the reference's CPU cost for the
same work:

* gather: advanced indexing ``kv[:, blocks, offsets]`` (cacheblend_vllm/kv_layout.py:110-121)
* scatter: ``kv[:, blocks, offsets] = contiguous`` (kv_layout.py:152-155)
* K-deviation: ``torch.sum((k.float() - old.float()) ** 2, dim=-1)`` (ascend.py:535-538)
* select: ``masked_fill`` + ``torch.topk`` + ``torch.where`` (ascend.py:770-793)
* relocate_key: delta cos/sin and the rotation in the key dtype (ascend.py:76-103)
* blend_load_layer: one layer of the loader -- APC gather, gap zeroing, per
  segment plane copies into the hit staging, K relocation, index scatter
  into the buffer, commit scatter (ascend.py:224-253, 280-287, 313-370, 385-396)
* sparse_q_full_scores: the chunked bf16 matmul / softmax loop (ascend.py:683-698)
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


def relocate_key(cos_sin_cache: torch.Tensor, old_positions: torch.Tensor, new_positions: torch.Tensor,
                 key: torch.Tensor, head_size: int, neox: bool) -> torch.Tensor:
    """``R(new) R(old)^-1`` on RoPE-encoded ``key [T, H * head_size]`` with
    rotary_dim == head_size (ascend.py:76-103)."""
    if torch.equal(old_positions, new_positions):
        return key
    cache = cos_sin_cache.to(dtype=key.dtype)
    old_cos, old_sin = cache.index_select(0, old_positions).chunk(2, dim=-1)
    new_cos, new_sin = cache.index_select(0, new_positions).chunk(2, dim=-1)
    delta_cos = (new_cos * old_cos + new_sin * old_sin).unsqueeze(1)
    delta_sin = (new_sin * old_cos - new_cos * old_sin).unsqueeze(1)
    shaped = key.reshape(key.shape[0], -1, head_size)
    if neox:
        first, second = torch.chunk(shaped, 2, dim=-1)
        out = torch.cat((first * delta_cos - second * delta_sin,
                         second * delta_cos + first * delta_sin), dim=-1)
    else:
        first, second = shaped[..., ::2], shaped[..., 1::2]
        out = torch.stack((first * delta_cos - second * delta_sin,
                           second * delta_cos + first * delta_sin), dim=-1).flatten(-2)
    return out.reshape(key.shape)


def blend_load_layer(pages: torch.Tensor, slot_mapping: torch.Tensor, block_size: int, apc: int,
                     allocation_end: int, segments: list[tuple[int, int, torch.Tensor]],
                     cos_sin_cache: torch.Tensor | None, head_size: int, neox: bool,
                     buffer: torch.Tensor | None = None) -> torch.Tensor:
    """One layer of the reference loader on a merged ``[2, NB, bs, H, D]``
    page tensor: the buffer ``[2, allocation_end, H, D]`` gets the APC
    prefix gathered through ``slot_mapping[:apc or 1]``, zeros on gaps, the
    hit segments ``(source_start, target_start, host [2, L, H, D])`` copied
    plane by plane into one hit staging whose K is relocated (when
    ``cos_sin_cache`` is given) and index-put at the targets; then
    ``buffer[:, apc:]`` is scattered into the pages through
    ``slot_mapping[apc:]``. Returns the buffer."""
    slots = slot_mapping[:allocation_end]
    sample = gather(pages, slots[: apc or 1], block_size)
    if buffer is None:
        buffer = torch.empty((2, allocation_end, *sample.shape[2:]), dtype=sample.dtype)
    if apc:
        buffer[:, :apc].copy_(sample)
    cursor = apc
    for source_start, target_start, host in segments:
        if target_start > cursor:
            buffer[:, cursor:target_start].zero_()
        cursor = max(cursor, target_start + host.shape[1])
    if cursor < allocation_end:
        buffer[:, cursor:allocation_end].zero_()
    if segments:
        hit_tokens = sum(host.shape[1] for _, _, host in segments)
        hit = torch.empty((2, hit_tokens, *segments[0][2].shape[2:]), dtype=buffer.dtype)
        offset = 0
        for _, _, host in segments:
            end = offset + host.shape[1]
            hit[0, offset:end].copy_(host[0])
            hit[1, offset:end].copy_(host[1])
            offset = end
        old = torch.cat([torch.arange(s, s + h.shape[1]) for s, _, h in segments])
        new = torch.cat([torch.arange(t, t + h.shape[1]) for _, t, h in segments])
        if cos_sin_cache is not None:
            k = hit[0].reshape(hit_tokens, -1)
            hit[0] = relocate_key(cos_sin_cache, old, new, k, head_size, neox).reshape(hit[0].shape)
        buffer[:, new] = hit
    if apc < allocation_end:
        scatter(buffer[:, apc:], pages, slots[apc:], block_size)
    return buffer


def sparse_q_full_scores(sparse_query: torch.Tensor, key: torch.Tensor, sparse_positions: torch.Tensor,
                         scale: float, chunk: int = 8) -> torch.Tensor:
    """Per-key causal attention mass of the sparse queries ``[Q, Hq, D]``
    over ``key [K, Hkv, D]`` summed over heads and queries: for each chunk of
    ``chunk`` queries a matmul in the input dtype, ``.float() * scale``, the
    causal mask at float32's minimum, a float32 softmax over all K keys,
    summed into ``full[K]`` (ascend.py:683-698)."""
    num_heads, num_kv_heads = sparse_query.shape[1], key.shape[1]
    groups = num_heads // num_kv_heads
    key_transposed = key.permute(1, 2, 0).contiguous()
    key_positions = torch.arange(key.shape[0])
    full = torch.zeros(key.shape[0], dtype=torch.float32)
    for start in range(0, sparse_query.shape[0], chunk):
        end = min(start + chunk, sparse_query.shape[0])
        q = sparse_query[start:end].view(end - start, num_kv_heads, groups, -1).permute(1, 2, 0, 3).contiguous()
        logits = torch.matmul(q, key_transposed[:, None]).float()
        logits.mul_(scale)
        mask = sparse_positions[start:end, None] < key_positions[None, :]
        logits.masked_fill_(mask[None, None], torch.finfo(logits.dtype).min)
        full.add_(torch.softmax(logits, dim=-1).sum(dim=(0, 1, 2)))
    return full
