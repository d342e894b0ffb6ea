"""Seeded synthetic inputs for the paged-KV and selection workloads.

Used by the benchmark and the parity tests; nothing here is on the serving
path. Shapes follow vLLM's merged_first paged cache ``[2, NB, bs, H, D]``.
"""

from __future__ import annotations

import numpy as np
import torch


def gap_layout(n: int, seed: int, hit_chunk: int = 256, max_hit_chunks: int = 7,
               max_gap: int = 511) -> np.ndarray:
    """Boolean gap mask of ``n`` tokens: hit runs of ``hit_chunk * U{1..max_hit_chunks}``
    tokens alternating with gap runs of ``U{1..max_gap}`` tokens (about 20%
    gaps with the defaults)."""
    rng = np.random.default_rng(seed)
    gaps = np.zeros(n, dtype=bool)
    pos = 0
    while pos < n:
        pos += hit_chunk * int(rng.integers(1, max_hit_chunks + 1))
        g = int(rng.integers(1, max_gap + 1))
        gaps[pos: pos + g] = True
        pos += g
    return gaps


def kdev_inputs(n: int, heads: int, head_dim: int, dtype: torch.dtype, device, seed: int = 0,
                gap_mask: np.ndarray | None = None):
    """(fresh_k [n, H*D], cached_k [n, H*D], gap_mask[n] bool) on ``device``.

    cached ~ N(0, 1) (zero on gap tokens, as the loader zeroes gaps); fresh =
    cached + sigma_t * N(0, 1) on hit tokens with sigma_t = 0.02 * exp(N(0, 1)),
    and a fresh N(0, 1) row on gap tokens.
    """
    g = torch.Generator(device="cpu").manual_seed(seed)
    width = heads * head_dim
    gaps = gap_layout(n, seed) if gap_mask is None else gap_mask
    gap_t = torch.from_numpy(gaps)
    cached = torch.randn(n, width, generator=g)
    cached[gap_t] = 0
    sigma = 0.02 * torch.exp(torch.randn(n, 1, generator=g))
    fresh = cached + sigma * torch.randn(n, width, generator=g)
    fresh[gap_t] = torch.randn(int(gaps.sum()), width, generator=g)
    return (
        fresh.to(dtype).to(device),
        cached.to(dtype).to(device),
        gap_t.to(device),
    )


def paged_pool(num_blocks: int, block_size: int, heads: int, head_dim: int, dtype, device,
               seed: int = 0) -> torch.Tensor:
    """One merged_first layer ``[2, NB, bs, H, D]`` with N(0, 1) values."""
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randn((2, num_blocks, block_size, heads, head_dim), generator=g, device=device,
                       dtype=torch.float32).to(dtype)


def block_slots(block_ids: torch.Tensor, block_size: int, tokens: int) -> torch.Tensor:
    """``block * bs + offset`` for consecutive tokens over ``block_ids``
    (the connector's slot mapping, reference connector.py:42-45)."""
    offsets = torch.arange(block_size, dtype=torch.long)
    return (block_ids.long()[:, None] * block_size + offsets[None, :]).reshape(-1)[:tokens]


def sparse_q_layout(context: int, queries: int, seed: int, max_gap: int = 511,
                    hit_chunk: int = 256) -> np.ndarray:
    """Boolean query (gap) mask over ``context`` tokens holding exactly
    ``queries`` gap tokens in runs of 1..max_gap, separated by hit runs of
    ``hit_chunk`` multiples, the last run ending at the last token."""
    rng = np.random.default_rng(seed)
    runs = []
    left = queries
    while left > 0:
        g = min(left, int(rng.integers(1, max_gap + 1)))
        runs.append(g)
        left -= g
    hit_chunks = (context - queries) // hit_chunk
    extra = context - queries - hit_chunks * hit_chunk
    split = rng.multinomial(hit_chunks, np.full(len(runs), 1.0 / len(runs)))
    mask = np.zeros(context, dtype=bool)
    pos = extra
    for g, h in zip(runs, split):
        pos += int(h) * hit_chunk
        mask[pos: pos + g] = True
        pos += g
    assert pos == context and int(mask.sum()) == queries
    return mask
