"""Side-forward attention of the selected queries on MI355X.

``blend_attention`` keeps the signature of ``Qwen3BlendExecutor._attention``
(cacheblend_vllm/ascend.py:798-846): queries ``[Nq, Hq, D]`` at absolute
positions ``q_positions`` attend causally (key ``k`` visible iff ``k <=
q_positions[i]``) to the layer buffer's keys/values ``[Nk, Hkv, D]`` with GQA
head sharing. It runs in ``cbk_blend_attention``: a flash-style MFMA kernel
that evaluates the mask in place (so the reference's cached
``[1, 1, Nq, Nk]`` mask, ``state.attention_mask``, is never built) and rounds
the logits as the reference's bf16/f16 einsum and ``* scale`` do.
"""

from __future__ import annotations

import torch

from . import _native


def blend_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    q_positions: torch.Tensor,
    scale: float,
    state=None,
) -> torch.Tensor:
    """Reference ascend.py:798-846 (``state`` is accepted for the signature;
    the mask needs no cache here). Returns ``[Nq, Hq, D]`` in the input dtype."""
    for name, t in (("query", query), ("key", key), ("value", value)):
        _native.require_device(t, name)
        if t.dim() != 3:
            raise ValueError(f"{name} must be [tokens, heads, head_size]")
        if t.stride(2) != 1 or t.stride(1) != t.shape[2]:
            raise ValueError(f"{name} rows must hold contiguous heads")
    nq, hq, d = query.shape
    nk, hkv, dk = key.shape
    if value.shape != key.shape or dk != d:
        raise ValueError("key/value shapes do not match the query head size")
    if key.dtype != query.dtype or value.dtype != query.dtype:
        raise ValueError("query, key and value must share a dtype")
    if query.dtype not in _native.DTYPE_CODES:
        raise ValueError(f"dtype {query.dtype} is not supported")
    if hq % hkv:
        raise ValueError(f"query heads ({hq}) must be divisible by KV heads ({hkv})")
    if q_positions.numel() != nq:
        raise ValueError(f"{q_positions.numel()} positions for {nq} queries")
    if q_positions.device.type == "cpu" and nq:
        lo, hi = int(q_positions.min()), int(q_positions.max())
        if lo < 0 or hi >= nk:
            raise IndexError(f"query positions in [{lo}, {hi}] outside the {nk} keys")
    pos = q_positions.to(device=query.device, dtype=torch.int64).contiguous()
    out = torch.empty((nq, hq, d), dtype=query.dtype, device=query.device)
    if nq == 0:
        return out
    rc = _native.load().cbk_blend_attention(
        query.data_ptr(), query.stride(0), pos.data_ptr(), nq,
        key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0), nk, hq, hkv, d,
        float(scale), _native.DTYPE_CODES[query.dtype], out.data_ptr(), out.stride(0),
        _native.stream_handle(query.device),
    )
    _native.check(rc, "blend_attention")
    return out
