"""RoPE relocation of cached keys on MI355X.

``relocate_key`` and ``validate_rope_support`` keep the reference's signatures
and errors (cacheblend_vllm/ascend.py:52-158). Relocation runs in the gfx950
blend-assembly kernel (cbk_blend_assemble, K plane only) and is bit-identical
to the reference's torch arithmetic: the ``cos_sin_cache`` is cast to the key
dtype, then every product, sum and difference is rounded to the key dtype.
"""

from __future__ import annotations

import threading
import weakref

import torch

from . import _native

# (id(cos_sin_cache), dtype, device) -> (weakref to that cache, its _version,
# converted table). The weakref guards against a new cache object reusing the
# id -- or the address -- of a freed one.
_tables: dict[tuple[int, torch.dtype, torch.device], tuple[weakref.ref, int, torch.Tensor]] = {}
_tables_lock = threading.Lock()


def rope_style(rotary_emb) -> tuple[int, bool]:
    """(head_size, neox) of a vLLM RotaryEmbedding-like object."""
    return int(rotary_emb.head_size), bool(rotary_emb.is_neox_style)


def cos_sin_table(rotary_emb, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """``rotary_emb.cos_sin_cache`` on ``device`` in ``dtype`` (cached per source
    tensor, so layers sharing one cache convert it once)."""
    cache = getattr(rotary_emb, "cos_sin_cache", None)
    if not isinstance(cache, torch.Tensor) or cache.ndim != 2:
        raise ValueError("CacheBlend requires a two-dimensional RoPE cos_sin_cache")
    key = (id(cache), dtype, torch.device(device))
    with _tables_lock:
        hit = _tables.get(key)
        if hit is not None and hit[0]() is cache and hit[1] == cache._version:
            return hit[2]
    table = cache.to(device=device, dtype=dtype).contiguous()
    if table is cache:
        return table  # nothing converted; holding it would keep the cache alive
    with _tables_lock:
        for k in [k for k, v in _tables.items() if v[0]() is None]:
            del _tables[k]
        _tables[key] = (weakref.ref(cache), cache._version, table)
    return table


def relocate_key(
    rotary_emb,
    old_positions: torch.Tensor,
    new_positions: torch.Tensor,
    key: torch.Tensor,
) -> torch.Tensor:
    """Apply ``R(new) R(old)^-1`` to already RoPE-encoded keys ``[T, H*D]``.

    Drop-in for reference ascend.py:52-103 (cos_sin_cache form). Returns
    ``key`` itself when every old position equals its new one.
    """
    if old_positions.shape == new_positions.shape and torch.equal(
        old_positions.to(new_positions.device), new_positions
    ):
        return key
    head_size, neox = rope_style(rotary_emb)
    rotary_dim = int(getattr(rotary_emb, "rotary_dim", head_size))
    if rotary_dim != head_size:
        raise ValueError(
            "CacheBlend requires rotary_dim == head_size; "
            f"got rotary_dim={rotary_dim}, head_size={head_size}"
        )
    _native.require_device(key, "key")
    if key.dtype not in _native.DTYPE_CODES:
        raise ValueError(f"key dtype {key.dtype} is not supported")
    tokens = key.shape[0]
    flat = key.reshape(tokens, -1)
    if flat.shape[1] % head_size:
        raise ValueError(f"key width {flat.shape[1]} is not a multiple of head_size {head_size}")
    if flat.stride(1) != 1:
        flat = flat.contiguous()
    table = cos_sin_table(rotary_emb, key.dtype, key.device)
    old = old_positions.reshape(-1).to(device=key.device, dtype=torch.int32)
    new = new_positions.reshape(-1).to(device=key.device, dtype=torch.int32)
    if old.numel() != tokens or new.numel() != tokens:
        raise ValueError("positions must have one entry per key row")
    out = torch.empty_like(flat)
    src_map = torch.arange(tokens, dtype=torch.int32, device=key.device)
    es = key.element_size()
    bad = torch.zeros(1, dtype=torch.int32, device=key.device)
    rc = _native.load().cbk_blend_assemble(
        None, None, src_map.data_ptr(), tokens,
        flat.data_ptr(), None, flat.stride(0) * es, tokens,
        old.data_ptr(), new.data_ptr(), table.data_ptr(), table.stride(0), table.shape[0],
        flat.shape[1] // head_size, head_size, 1, int(neox), _native.DTYPE_CODES[key.dtype],
        out.data_ptr(), None, out.stride(0) * es, bad.data_ptr(),
        _native.stream_handle(key.device),
    )
    _native.check(rc, "relocate_key")
    if int(bad.item()):
        raise IndexError("relocation position outside the RoPE cos_sin_cache")
    return out.reshape(key.shape)


def validate_rope_support(model, rotary_emb) -> None:
    """Fail closed for RoPE variants relocation does not cover.

    Same checks and messages as reference ascend.py:106-158: full rotary
    dimension, no rope_scaling, partial_rotary_factor 1, a 2-D non-empty
    cos_sin_cache of width rotary_dim with unit-norm (cos, sin) samples.
    """
    head_size = int(rotary_emb.head_size)
    rotary_dim = int(getattr(rotary_emb, "rotary_dim", head_size))
    if rotary_dim != head_size:
        raise ValueError(
            "CacheBlend requires rotary_dim == head_size; "
            f"got rotary_dim={rotary_dim}, head_size={head_size}"
        )
    config = getattr(model, "config", None)
    if getattr(config, "rope_scaling", None):
        raise ValueError("CacheBlend does not support rope_scaling")
    factor = getattr(config, "partial_rotary_factor", 1.0)
    factor = 1.0 if factor is None else float(factor)
    if factor != 1.0:
        raise ValueError(f"CacheBlend requires partial_rotary_factor=1.0; got {factor}")
    cache = getattr(rotary_emb, "cos_sin_cache", None)
    if not isinstance(cache, torch.Tensor) or cache.ndim != 2:
        raise ValueError("CacheBlend requires a two-dimensional RoPE cos_sin_cache")
    if cache.shape[0] == 0:
        raise ValueError("CacheBlend requires a non-empty RoPE cos_sin_cache")
    if cache.shape[-1] != rotary_dim:
        raise ValueError(
            "CacheBlend RoPE cache width does not match rotary_dim: "
            f"cache={cache.shape[-1]}, rotary_dim={rotary_dim}"
        )
    rows = sorted({0, max(0, cache.shape[0] - 1)})
    sample = cache[rows].float()
    cos, sin = sample.chunk(2, dim=-1)
    err = float((cos.square() + sin.square() - 1.0).abs().max())
    if err > 0.05:
        raise ValueError(
            f"CacheBlend requires unit-norm, unscaled RoPE; maximum sampled norm error is {err:.4f}"
        )
