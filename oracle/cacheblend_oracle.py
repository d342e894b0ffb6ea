"""CPU restatement of CacheBlend's KV data-movement and selection semantics.

TEST INFRASTRUCTURE ONLY -- the oracle the tests compare against, never the product.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it.

Every function restates one piece of the reference (zoudinghong2000/PIC-KVCache,
a pure-Python vLLM connector) in numpy, citing the file:line it follows. Arrays
are numpy; bf16 data is carried as ``uint16`` bit patterns (``bf16_to_f32`` /
``f32_to_bf16``) because numpy has no bf16 dtype.

Contract differences from the reference, on purpose:

* ``select`` breaks ties at the top-k boundary toward the LOWER index. The
  reference calls ``torch.topk`` (cacheblend_vllm/ascend.py:792), whose choice
  among equal scores is implementation-defined; the lower-index rule is the
  build's contract.
* ``kdev_scores`` sums in float64 and rounds once to float32. The reference
  sums in torch float32 (ascend.py:535-538); the two differ only by float32
  summation-order noise.

Pinning (what checks each function, all in tests/test_oracle.py):

* slot_mapping, gather/scatter, layout dispatch: reference known answers
  (tests/test_connector_scheduler.py:58-90, tests/test_kv_layout.py:8-40),
  brute-force loops, round trips.
* select / budget: reference known answers (tests/test_ascend.py:144-154,
  256-267), brute force over every subset order on tiny inputs, tie cases.
* dilate / sparse_q_masks: reference known answers (tests/test_ascend.py:
  215-253), brute-force window scan.
* sparse_q_full_scores: reference closed-form test (tests/test_ascend.py:
  157-212), float64 dense softmax, column sums equal query count (softmax rows
  sum to one); the bf16 and f16 logit rounding, placed before the scale, to
  within float32 summation noise of torch's CPU kernels run in the order of
  ascend.py:688-698 at scale 0.37 (rounding after the scale, or no rounding,
  is far off).
* kdev_scores: float64 closed form on integer-valued data where float32 is
  exact, zero on identical inputs.
* relocate_key: reference known answer against fresh RoPE
  (tests/test_ascend.py:52-60), group property R(a)R(b)^-1; the bf16 path
  bit-exact against torch's CPU bf16 elementwise kernels run in the order
  of ascend.py:76-103 (the reference's third-party arithmetic).
* loader_assemble / loader_commit: reference known answer
  (tests/test_ascend.py:96-141).
* blend_attention: float64 closed forms -- identical keys give the mean of
  the visible values, a one-key context returns that value, uniform logits
  average the visible rows, two visible keys weigh sigmoid(scale * (q.k1 -
  q.k0)); a float64 brute-force per-(query, head) causal softmax with
  non-constant logits and scales 0.37 and 1.7; the bf16 and f16 rounding
  sequence bit-exact against torch's CPU kernels run in the order of
  ascend.py:834-846.
* content_hash / window_hashes / match_tokens: reference known answers
  (tests/test_matcher.py:6-31), closed forms of one- and two-token hashes,
  the wrap at 2^64, window hashes equal the Horner hash at every offset, and
  brute-force properties of matches on tiny vocabularies (sorted,
  non-overlapping, every match verified, no unmatched registered window left
  between matches).
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np

__all__ = [
    "bf16_to_f32",
    "f32_to_bf16",
    "round_bf16",
    "slot_mapping",
    "kv_planes",
    "gather_paged_kv",
    "scatter_paged_kv",
    "kdev_scores",
    "select_budget",
    "float_order_keys",
    "select",
    "dilate",
    "sparse_q_masks",
    "sparse_q_full_scores",
    "sparse_q_scores",
    "relocate_key",
    "loader_assemble",
    "loader_commit",
    "round_f16",
    "blend_attention",
    "content_hash",
    "window_hashes",
    "match_tokens",
]


# ---------------------------------------------------------------------------
# bf16 helpers (round-to-nearest-even, as torch's float->bfloat16 cast)
# ---------------------------------------------------------------------------


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Widen bf16 bit patterns (uint16/int16) to float32 exactly."""
    u = np.asarray(bits).view(np.uint16).astype(np.uint32) << np.uint32(16)
    return u.view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 to bf16 bit patterns, nearest-even; NaN stays NaN."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    rounded = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        rounded = rounded.copy()
        rounded[nan] = ((u[nan] >> np.uint64(16)) | np.uint64(0x40)).astype(np.uint16)
    return rounded


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 -> float32."""
    return bf16_to_f32(f32_to_bf16(x))


# ---------------------------------------------------------------------------
# Slots and paged layouts
# ---------------------------------------------------------------------------


def slot_mapping(block_ids: Sequence[int], block_size: int, token_count: int) -> np.ndarray:
    """``slot[i] = block_ids[i // bs] * bs + i % bs``, truncated.

    Follows cacheblend_vllm/connector.py:42-45.
    """
    blocks = np.asarray(block_ids, dtype=np.int64)
    offsets = np.arange(block_size, dtype=np.int64)
    return (blocks[:, None] * block_size + offsets[None, :]).reshape(-1)[:token_count]


def kv_planes(kv_layer) -> tuple[np.ndarray, np.ndarray]:
    """Return writable ``(K, V)`` views shaped ``[num_blocks, block_size, ...]``.

    Layout detection follows cacheblend_vllm/kv_layout.py:12-20 (separate
    pair), 113 (``shape[0] == 2`` -> merged_first ``[2, NB, bs, ...]``, tested
    first), 115 (``ndim >= 4 and shape[1] == 2`` -> merged_block
    ``[NB, 2, bs, ...]``) and 118 (anything else is rejected).
    """
    if isinstance(kv_layer, (list, tuple)):
        if len(kv_layer) != 2:
            raise ValueError(f"separate KV layout requires two tensors, got {len(kv_layer)}")
        key, value = kv_layer
        if not isinstance(key, np.ndarray) or not isinstance(value, np.ndarray):
            raise TypeError("separate KV layout must contain tensors")
        return key, value
    if kv_layer.shape[0] == 2:
        return kv_layer[0], kv_layer[1]
    if kv_layer.ndim >= 4 and kv_layer.shape[1] == 2:
        return kv_layer[:, 0], kv_layer[:, 1]
    raise ValueError(f"unsupported vLLM KV layout {tuple(kv_layer.shape)}")


def gather_paged_kv(kv_layer, slots: np.ndarray, block_size: int) -> np.ndarray:
    """``out[c, t] = plane_c[slot_t // bs, slot_t % bs]``, c in (K, V).

    Follows cacheblend_vllm/kv_layout.py:90-122 (torch advanced indexing).
    Slots must lie in ``[0, num_blocks * block_size)``; the reference's torch
    indexing would wrap negative slots, the build rejects them.
    """
    key, value = kv_planes(kv_layer)
    slots = np.asarray(slots, dtype=np.int64)
    _check_slots(slots, key.shape[0] * block_size)
    blocks, offsets = slots // block_size, slots % block_size
    return np.stack((key[blocks, offsets], value[blocks, offsets]), axis=0)


def scatter_paged_kv(contiguous: np.ndarray, kv_layer, slots: np.ndarray, block_size: int) -> None:
    """In place: ``plane_c[slot_t // bs, slot_t % bs] = contiguous[c, t]``.

    Follows cacheblend_vllm/kv_layout.py:125-161. Duplicate slots have no
    defined winner in the reference (torch ``index_put_``); callers never emit
    them and tests do not use them.
    """
    if contiguous.shape[0] != 2:
        raise ValueError("contiguous KV must have K/V as its first dimension")
    key, value = kv_planes(kv_layer)
    slots = np.asarray(slots, dtype=np.int64)
    _check_slots(slots, key.shape[0] * block_size)
    blocks, offsets = slots // block_size, slots % block_size
    key[blocks, offsets] = contiguous[0]
    value[blocks, offsets] = contiguous[1]


def _check_slots(slots: np.ndarray, num_slots: int) -> None:
    if slots.size and (slots.min() < 0 or slots.max() >= num_slots):
        raise IndexError(f"slot out of range [0, {num_slots})")


# ---------------------------------------------------------------------------
# K-deviation selection
# ---------------------------------------------------------------------------


def kdev_scores(fresh: np.ndarray, cached: np.ndarray) -> np.ndarray:
    """``s[i] = sum_j (fresh[i, j] - cached[i, j])**2`` over the flattened row.

    Follows cacheblend_vllm/ascend.py:534-538, where ``cached`` is
    ``flat_old_k[absolute_indices]`` and both operands are widened to float32
    before the difference. Inputs are float32 arrays (bf16 callers widen with
    ``bf16_to_f32`` first, which is exact).
    """
    f = np.asarray(fresh, dtype=np.float32).reshape(fresh.shape[0], -1)
    c = np.asarray(cached, dtype=np.float32).reshape(cached.shape[0], -1)
    diff = (f - c).astype(np.float64)  # float32 difference, as the reference
    return np.sum(diff * diff, axis=1).astype(np.float32)


def select_budget(n: int, gap_count: int, base_count: int, ratio: float) -> int:
    """Top-k budget of ``_select``.

    Follows cacheblend_vllm/ascend.py:775-785: ``topk = int(cached * ratio)``
    (Python float64 then truncation), at least one and at most ``available``
    when both are non-zero, else zero.
    """
    cached = n - gap_count
    topk = int(cached * ratio)
    available = n - base_count
    if cached and available:
        return min(max(topk, 1), available)
    return 0


def float_order_keys(scores: np.ndarray) -> np.ndarray:
    """Map float32 to uint32 keys whose unsigned order is torch.topk's order.

    NaN is canonicalised to the largest key (torch.topk ranks NaN above every
    number) and -0.0 to +0.0 (they compare equal, so they tie).
    """
    s = np.array(scores, dtype=np.float32, copy=True)
    s[np.isnan(s)] = np.float32(np.nan)
    s[s == 0] = np.float32(0.0)
    u = s.view(np.uint32)
    neg = (u >> np.uint32(31)).astype(bool)
    keys = np.where(neg, ~u, u | np.uint32(0x80000000)).astype(np.uint32)
    keys[np.isnan(s)] = np.uint32(0xFFFFFFFF)
    return keys


def select(
    scores: np.ndarray,
    gap_mask: np.ndarray,
    ratio: float,
    forced_mask: np.ndarray | None = None,
) -> np.ndarray:
    """Sorted int64 indices of ``gap | forced | top-k(scores masked to -inf)``.

    Follows Qwen3BlendExecutor._select, cacheblend_vllm/ascend.py:757-796, at
    TP1: ``base = gap | forced`` (770-774); budget (775-785); top-k over ALL
    tokens of ``scores.masked_fill(base, -inf)`` (791-792); the union with
    ``base`` in ascending index order (789-793). Ties at the boundary go to
    the lower index (the build's contract, see the module docstring).
    """
    scores = np.asarray(scores, dtype=np.float32)
    gap = np.asarray(gap_mask, dtype=bool)
    n = scores.shape[0]
    base = gap.copy()
    if forced_mask is not None:
        forced = np.asarray(forced_mask, dtype=bool)
        if forced.shape != gap.shape:
            raise ValueError("forced selection mask must match the active token shape")
        base |= forced
    topk = select_budget(n, int(gap.sum()), int(base.sum()), ratio)
    selected = base.copy()
    if topk:
        masked = np.where(base, np.float32(-np.inf), scores)
        keys = float_order_keys(masked).astype(np.int64)
        order = np.lexsort((np.arange(n), -keys))
        selected[order[:topk]] = True
    return np.flatnonzero(selected).astype(np.int64)


def dilate(gap_mask: np.ndarray, radius: int) -> np.ndarray:
    """``out[i] = any(gap[max(0, i - r) : min(n, i + r + 1)])``.

    Follows the prefix-sum window of cacheblend_vllm/ascend.py:662-671 (a
    token-distance window, not block aligned).
    """
    gap = np.asarray(gap_mask, dtype=bool)
    n = gap.shape[0]
    prefix = np.concatenate(([0], np.cumsum(gap.astype(np.int64))))
    pos = np.arange(n)
    left = np.clip(pos - radius, 0, None)
    right = np.clip(pos + radius + 1, None, n)
    return prefix[right] > prefix[left]


# ---------------------------------------------------------------------------
# Sparse-Q
# ---------------------------------------------------------------------------


def sparse_q_masks(
    gap_mask: np.ndarray, tail_query_tokens: int, radius: int
) -> tuple[np.ndarray, np.ndarray, bool]:
    """``(query_mask, forced_mask, tail_fallback)`` of ``_sparse_q_scores``.

    Follows cacheblend_vllm/ascend.py:652-671. Without gaps the last
    ``min(tail, N)`` tokens become queries and are forced (note Python's
    ``x[-0:]`` is the whole array, kept as is). With gaps and ``radius > 0``
    the forced set is dilated by ``radius`` tokens.
    """
    gap = np.asarray(gap_mask, dtype=bool)
    query = gap.copy()
    forced = gap.copy()
    has_gap = bool(gap.any())
    if not has_gap:
        tail = min(tail_query_tokens, gap.shape[0])
        query[-tail:] = True
        forced[-tail:] = True
    if radius and has_gap:
        forced |= dilate(gap, radius)
    return query, forced, not has_gap


def sparse_q_full_scores(
    query: np.ndarray,
    key: np.ndarray,
    query_positions: np.ndarray,
    scale: float,
    round_logits_bf16: bool,
    chunk: int = 8,
    *,
    logit_dtype: str | None = None,
    round_after_scale: bool = False,
) -> np.ndarray:
    """Per-key causal attention mass summed over heads and queries.

    Follows cacheblend_vllm/ascend.py:683-698. ``query`` is ``[Q, Hq, D]``
    float32 (the selected sparse queries), ``key`` is ``[K, Hkv, D]`` float32.
    Query head ``h`` reads KV head ``h // (Hq // Hkv)`` (692). Logits are the
    matmul output rounded to the input dtype (694: a bf16 or f16 ``matmul``
    then ``.float()``; ``logit_dtype`` "bf16" or "f16", or
    ``round_logits_bf16``; no rounding for float32 inputs), then ``* scale``
    in float32 (695), then keys ``k > position_q`` are set to
    ``finfo(float32).min`` (696-697), then a float32 softmax over all K keys,
    summed over (kv head, group, query) (698). Returns ``full_scores[K]``
    float32. ``round_after_scale`` swaps the rounding and the scale -- not
    what the reference does; it exists so a test can show that the rounding
    position is pinned.
    """
    if logit_dtype is None and round_logits_bf16:
        logit_dtype = "bf16"
    rnd = {None: None, "bf16": round_bf16, "f16": round_f16}[logit_dtype]
    q = np.asarray(query, dtype=np.float32)
    k = np.asarray(key, dtype=np.float32)
    nq, hq, d = q.shape
    nk, hkv, _ = k.shape
    if hq % hkv:
        raise ValueError(
            "Sparse-Q requires query heads to be divisible by KV heads; "
            f"got {hq} and {hkv}"
        )
    groups = hq // hkv
    pos = np.asarray(query_positions, dtype=np.int64)
    key_pos = np.arange(nk)
    full = np.zeros(nk, dtype=np.float32)
    kt = np.ascontiguousarray(k.transpose(1, 2, 0))  # [Hkv, D, K]
    s32 = np.float32(scale)
    fmin = np.finfo(np.float32).min
    for start in range(0, nq, chunk):
        end = min(start + chunk, nq)
        qc = q[start:end].reshape(end - start, hkv, groups, d).transpose(1, 2, 0, 3)
        logits = np.matmul(qc, kt[:, None]).astype(np.float32)  # [Hkv, G, c, K]
        if round_after_scale:
            logits = logits * s32
        if rnd is not None:
            logits = rnd(logits)
        if not round_after_scale:
            logits = logits * s32
        mask = pos[start:end, None] < key_pos[None, :]
        logits = np.where(mask[None, None], fmin, logits).astype(np.float32)
        row_max = logits.max(axis=-1, keepdims=True)
        e = np.exp(logits - row_max, dtype=np.float32)
        probs = e / e.sum(axis=-1, keepdims=True, dtype=np.float32)
        full += probs.sum(axis=(0, 1, 2), dtype=np.float32)
    return full


def sparse_q_scores(
    query: np.ndarray,
    key: np.ndarray,
    absolute_indices: np.ndarray,
    gap_mask: np.ndarray,
    scale: float,
    *,
    block_size: int,
    overflow_blocks: int,
    tail_query_tokens: int,
    chunk: int = 8,
    round_logits_bf16: bool = False,
    logit_dtype: str | None = None,
) -> tuple[np.ndarray, np.ndarray, dict]:
    """``(scores[N], forced[N], stats)`` of ``_sparse_q_scores``.

    Follows cacheblend_vllm/ascend.py:638-711: masks (652-671), sparse query
    rows and their absolute positions (673-675), full scores (683-698),
    indexed by ``absolute_indices`` (700-701), statistics (702-710).
    """
    gap = np.asarray(gap_mask, dtype=bool)
    radius = overflow_blocks * block_size
    qmask, forced, tail_fallback = sparse_q_masks(gap, tail_query_tokens, radius)
    sparse = np.flatnonzero(qmask)
    absolute = np.asarray(absolute_indices, dtype=np.int64)
    full = sparse_q_full_scores(
        np.asarray(query)[sparse],
        key,
        absolute[sparse],
        scale,
        round_logits_bf16,
        chunk,
        logit_dtype=logit_dtype,
    )
    gap_count = int(gap.sum())
    stats = {
        "active_tokens": int(query.shape[0]),
        "gap_tokens": gap_count,
        "cached_tokens": int(query.shape[0]) - gap_count,
        "sparse_query_tokens": int(sparse.size),
        "tail_fallback": tail_fallback,
        "overflow_blocks": overflow_blocks,
    }
    return full[absolute], forced, stats


# ---------------------------------------------------------------------------
# RoPE relocation and the layerwise blend buffer
# ---------------------------------------------------------------------------


def relocate_key(
    cos_sin_cache: np.ndarray,
    old_positions: np.ndarray,
    new_positions: np.ndarray,
    key: np.ndarray,
    head_size: int,
    neox: bool,
    bf16: bool,
) -> np.ndarray:
    """Apply the delta rotation ``R(new) R(old)^-1`` to RoPE-encoded keys.

    Follows cacheblend_vllm/ascend.py:64-103 with ``rotary_dim == head_size``
    (validate_rope_support, ascend.py:115-119, rejects anything else). ``key``
    is float32 ``[T, H * head_size]``. With ``bf16`` every elementwise result
    is rounded to bf16 exactly as torch's eager bf16 kernels do (the cache is
    cast to the key dtype first, ascend.py:76); otherwise float32 throughout.
    Identity when every old position equals its new position (64-65).
    """
    old = np.asarray(old_positions, dtype=np.int64)
    new = np.asarray(new_positions, dtype=np.int64)
    key = np.asarray(key, dtype=np.float32)
    if old.shape == new.shape and np.array_equal(old, new):
        return key.copy()
    rnd = round_bf16 if bf16 else (lambda a: np.asarray(a, dtype=np.float32))
    cache = rnd(np.asarray(cos_sin_cache, dtype=np.float32))
    half = cache.shape[-1] // 2
    oc, os_ = cache[old, :half], cache[old, half:]
    nc, ns = cache[new, :half], cache[new, half:]
    dcos = rnd(rnd(nc * oc) + rnd(ns * os_))
    dsin = rnd(rnd(ns * oc) - rnd(nc * os_))
    shaped = key.reshape(key.shape[0], -1, head_size)
    dcos = dcos[:, None, :]
    dsin = dsin[:, None, :]
    if neox:
        first, second = shaped[..., :half], shaped[..., half:]
    else:
        first, second = shaped[..., 0::2], shaped[..., 1::2]
    out_first = rnd(rnd(first * dcos) - rnd(second * dsin))
    out_second = rnd(rnd(second * dcos) + rnd(first * dsin))
    out = np.empty_like(shaped)
    if neox:
        out[..., :half], out[..., half:] = out_first, out_second
    else:
        out[..., 0::2], out[..., 1::2] = out_first, out_second
    return out.reshape(key.shape)


def loader_assemble(
    kv_layer,
    slots: np.ndarray,
    block_size: int,
    apc_prefix_tokens: int,
    allocation_end: int,
    segments: Sequence[tuple[int, int, np.ndarray]],
    relocate=None,
) -> np.ndarray:
    """The blend buffer ``[2, allocation_end, ...]`` one layer's prefetch builds.

    Follows PagedBlendLoader.prefetch/_zero_gaps/_load_segments_fused,
    cacheblend_vllm/ascend.py:230-253, 280-287, 313-370: ``[0, apc)`` is
    gathered from the pages through ``slots``; every gap is zero; each hit
    segment ``(source_start, target_start, host[2, L, ...])`` lands at
    ``[target_start, target_start + L)``. ``relocate(old_pos, new_pos, k)``
    (optional) rewrites the concatenated hit K, as ascend.py:357 does.
    """
    key, _ = kv_planes(kv_layer)
    row_shape = key.shape[2:]
    buf = np.zeros((2, allocation_end, *row_shape), dtype=key.dtype)
    if apc_prefix_tokens:
        buf[:, :apc_prefix_tokens] = gather_paged_kv(
            kv_layer, np.asarray(slots)[:apc_prefix_tokens], block_size
        )
    if segments:
        hosts = [np.asarray(h) for _, _, h in segments]
        hit = np.concatenate(hosts, axis=1)
        old = np.concatenate([np.arange(s, s + h.shape[1]) for (s, _, _), h in zip(segments, hosts)])
        new = np.concatenate([np.arange(t, t + h.shape[1]) for (_, t, _), h in zip(segments, hosts)])
        if relocate is not None:
            hit = hit.copy()
            hit[0] = relocate(old, new, hit[0])
        buf[:, new] = hit
    return buf


def loader_commit(
    contiguous: np.ndarray,
    kv_layer,
    slots: np.ndarray,
    block_size: int,
    apc_prefix_tokens: int,
    allocation_end: int,
) -> None:
    """Scatter ``contiguous[:, apc:]`` into the pages through ``slots[apc:]``.

    Follows PagedBlendLoader.commit, cacheblend_vllm/ascend.py:385-396: the
    APC prefix pages are never written.
    """
    start = apc_prefix_tokens
    if start >= allocation_end:
        return
    scatter_paged_kv(
        contiguous[:, start:allocation_end],
        kv_layer,
        np.asarray(slots)[start:allocation_end],
        block_size,
    )


# ---------------------------------------------------------------------------
# Side-forward attention of the selected queries
# ---------------------------------------------------------------------------


def round_f16(x: np.ndarray) -> np.ndarray:
    """float32 -> float16 (round to nearest even) -> float32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def blend_attention(
    query: np.ndarray,
    key: np.ndarray,
    value: np.ndarray,
    q_positions: np.ndarray,
    scale: float,
    rounding: str | None = "bf16",
    chunk: int = 64,
    return_mass: bool = False,
):
    """``out[q, h] = sum_k softmax_k(w[h, q, :])[k] * value[k, h // G]`` with
    ``w = r(r(query[q, h] . key[k, h // G]) * scale)`` and keys ``k >
    q_positions[q]`` masked out, G = Hq / Hkv.

    Follows cacheblend_vllm/ascend.py:798-846 (the einsum path of
    ``Qwen3BlendExecutor._attention``): the score einsum and the ``* scale``
    are rounded to the input dtype (``r``: bf16 or f16, none for float32),
    the softmax is float32 over all keys with masked entries at the dtype's
    minimum (exactly zero weight), the probabilities are rounded to the input
    dtype, and the value einsum accumulates them in float32 before rounding
    the output to the input dtype. Inputs are float32 arrays holding the
    dtype's values; returns float32 ``[Nq, Hq, D]`` -- and, with
    ``return_mass``, also ``sum_k p[k] * |value[k]|`` per output element, the
    L1 size of the terms each output sums (rounding errors of the
    probabilities scale with it, not with a possibly cancelled output).
    """
    r = {"bf16": round_bf16, "f16": round_f16, None: lambda x: np.asarray(x, np.float32)}[rounding]
    q = np.asarray(query, dtype=np.float32)
    k = np.asarray(key, dtype=np.float32)
    v = np.asarray(value, dtype=np.float32)
    nq, hq, d = q.shape
    nk, hkv, _ = k.shape
    if hq % hkv:
        raise ValueError("query heads must be divisible by KV heads")
    g = hq // hkv
    pos = np.asarray(q_positions, dtype=np.int64)
    out = np.empty((nq, hq, d), dtype=np.float32)
    mass = np.empty((nq, hq, d), dtype=np.float64) if return_mass else None
    keys = np.arange(nk)
    for c0 in range(0, nq, chunk):
        qc = q[c0:c0 + chunk]
        mask = pos[c0:c0 + chunk, None] < keys[None, :]                  # [c, nk]
        for h in range(hq):
            kh, vh = k[:, h // g, :], v[:, h // g, :]
            w = r(r(qc[:, h, :].astype(np.float64) @ kh.T.astype(np.float64)) * np.float32(scale))
            w = np.where(mask, -np.inf, w.astype(np.float64))
            w = w - w.max(axis=1, keepdims=True)
            e = np.exp(w)
            p = r(e / e.sum(axis=1, keepdims=True))
            out[c0:c0 + chunk, h, :] = r(p.astype(np.float64) @ vh.astype(np.float64))
            if mass is not None:
                mass[c0:c0 + chunk, h, :] = p.astype(np.float64) @ np.abs(vh.astype(np.float64))
    return (out, mass) if return_mass else out


# ---------------------------------------------------------------------------
# token-range matching (reference cacheblend_vllm/hashing.py, matcher.py)
# ---------------------------------------------------------------------------

MASK64 = (1 << 64) - 1
POLY_BASE = 1_000_003


def content_hash(tokens: Sequence[int]) -> int:
    """Horner evaluation of sum_j (t_j + 1) * B^(w-1-j) mod 2^64 with Python
    integers (reference hashing.py:14-22)."""
    value = 0
    for token in tokens:
        value = (value * POLY_BASE + ((int(token) + 1) & MASK64)) & MASK64
    return value


def window_hashes(tokens: Sequence[int], window: int) -> np.ndarray:
    """Hash of every full window, each evaluated on its own as a dot product
    with the power vector B^(w-1) .. B^0 in wrapping uint64 arithmetic
    (reference hashing.py:25-53)."""
    if window <= 0:
        raise ValueError("window must be positive")
    values = np.asarray(tokens, dtype=np.int64).astype(np.uint64) + np.uint64(1)
    if values.shape[0] < window:
        return np.empty(0, dtype=np.uint64)
    powers = np.array([pow(POLY_BASE, e, 1 << 64) for e in range(window - 1, -1, -1)], dtype=np.uint64)
    windows = np.lib.stride_tricks.sliding_window_view(values, window)
    return windows @ powers


def match_tokens(records: Sequence[tuple[str, int, tuple[int, ...]]], scope: str,
                 tokens: Sequence[int], start_offset: int, chunk_size: int) -> list[tuple[int, int]]:
    """Leftmost-greedy, non-overlapping exact matches (reference
    matcher.py:80-125). ``records`` are ``(scope, hash, tokens)`` in
    registration order; returns ``(target_start, record_index)`` pairs, the
    record being the first registered one of that scope and window hash whose
    tokens equal the window."""
    if start_offset < 0 or start_offset > len(tokens):
        raise ValueError("start_offset is outside the token sequence")
    by_hash: dict[int, list[int]] = {}
    for index, (s, h, _) in enumerate(records):
        if s == scope:
            by_hash.setdefault(int(h), []).append(index)
    if not by_hash:
        return []
    hashes = window_hashes(list(tokens)[start_offset:], chunk_size)
    out: list[tuple[int, int]] = []
    next_allowed = start_offset
    for rel, value in enumerate(hashes):
        target = start_offset + rel
        if target < next_allowed or int(value) not in by_hash:
            continue
        window = tuple(int(t) for t in tokens[target:target + chunk_size])
        for index in by_hash[int(value)]:
            if tuple(records[index][2]) == window:
                out.append((target, index))
                next_allowed = target + chunk_size
                break
    return out
