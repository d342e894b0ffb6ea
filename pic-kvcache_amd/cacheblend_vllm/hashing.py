"""Token-window hashes of the blend lookup (reference cacheblend_vllm/hashing.py).

A chunk's identity is the polynomial hash of its tokens,
``H(t_0..t_{w-1}) = sum_j (t_j + 1) * 1_000_003^(w-1-j) mod 2^64``
(reference hashing.py:10-22). ``rolling_hash_values`` returns H at every
window start of a prompt; the library computes it with the O(1) rolling
update instead of the reference's O(n * w) sliding-window product
(hashing.py:42-53), bit for bit the same values. Tokens must fit int64
(vocabulary ids do).
"""

from __future__ import annotations

import array
from collections.abc import Iterator, Sequence

import numpy as np

from . import _native

MASK64 = (1 << 64) - 1
POLY_BASE = 1_000_003


def as_token_array(tokens) -> np.ndarray:
    """Contiguous int64 view or copy of a token sequence (list, tuple, numpy
    array or CPU tensor)."""
    if hasattr(tokens, "detach"):  # torch tensor
        tokens = tokens.detach().cpu().numpy()
    elif isinstance(tokens, (list, tuple)):
        # array.array converts a list of ints faster than numpy does
        return np.frombuffer(array.array("q", tokens), dtype=np.int64) if tokens else np.empty(0, np.int64)
    return np.ascontiguousarray(np.asarray(tokens, dtype=np.int64).reshape(-1))


def rolling_hash_values(tokens: Sequence[int], window: int) -> np.ndarray:
    """Every full-window hash as a contiguous uint64 array (reference
    hashing.py:42-53); empty when ``len(tokens) < window``."""
    if window <= 0:
        raise ValueError("window must be positive")
    values = as_token_array(tokens)
    n = values.shape[0]
    if n < window:
        return np.empty(0, dtype=np.uint64)
    out = np.empty(n - window + 1, dtype=np.uint64)
    _native.check(
        _native.load().cbk_rolling_hashes(values.ctypes.data, n, window, out.ctypes.data),
        "rolling_hash_values",
    )
    return out


def content_hash(tokens: Sequence[int]) -> int:
    """Hash of one token sequence (reference hashing.py:18-22)."""
    values = as_token_array(tokens)
    if values.shape[0] == 0:
        return 0
    return int(rolling_hash_values(values, values.shape[0])[0])


def rolling_hashes(tokens: Sequence[int], window: int) -> Iterator[tuple[int, int]]:
    """``(start, hash)`` for every full window (reference hashing.py:35-39)."""
    for start, value in enumerate(rolling_hash_values(tokens, window)):
        yield start, int(value)
