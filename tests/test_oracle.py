"""Pins the CPU oracle before any GPU result is compared against it.

Each oracle function is checked against the reference's own known answers
(tests/golden/reference_known_answers.json), against brute force on tiny
inputs, and against closed forms, chosen so that a dropped term, a wrong sign
or an off-by-one fails at least one check.
"""

import itertools
import math

import numpy as np
import pytest
import torch

import oracle as O


def _arange_base(shape):
    return np.arange(int(np.prod(shape)), dtype=np.float32).reshape(shape)


def _layout(base, layout):
    if layout == "merged_first":
        return base.copy()
    if layout == "merged_block":
        return np.ascontiguousarray(base.transpose(1, 0, 2, 3))
    return [base[0].copy(), base[1].copy()]


# ---------------------------------------------------------------- paged layouts


@pytest.mark.parametrize("layout", ["merged_first", "merged_block", "separate"])
def test_gather_scatter_known_answer(golden, layout):
    case = golden["kv_layout_round_trip"]
    base = _arange_base(case["base_shape"])
    paged = _layout(base, layout)
    got = O.gather_paged_kv(paged, np.array(case["slots"]), case["block_size"])
    np.testing.assert_array_equal(got, np.array(case["expected_gather"], dtype=np.float32))
    replacement = np.full_like(got, case["scatter_value"])
    O.scatter_paged_kv(replacement, paged, np.array(case["slots"]), case["block_size"])
    np.testing.assert_array_equal(
        O.gather_paged_kv(paged, np.array(case["slots"]), case["block_size"]), replacement
    )


def test_unknown_layout_rejected(golden):
    case = golden["kv_layout_unknown"]
    with pytest.raises(ValueError, match=case["match"]):
        O.gather_paged_kv(np.empty(case["shape"]), np.array(case["slots"]), case["block_size"])


def test_out_known_answer(golden):
    case = golden["kv_layout_out"]
    paged = _arange_base(case["paged_shape"])
    got = O.gather_paged_kv(paged, np.array(case["slots"]), case["block_size"])
    np.testing.assert_array_equal(got, np.array(case["expected"], dtype=np.float32))


@pytest.mark.parametrize("layout", ["merged_first", "merged_block", "separate"])
def test_gather_matches_brute_force_loop(layout):
    rng = np.random.default_rng(1)
    nb, bs, h, d = 7, 4, 3, 5
    base = rng.standard_normal((2, nb, bs, h, d)).astype(np.float32)
    if layout == "merged_first":
        paged = base.copy()
    elif layout == "merged_block":
        paged = np.ascontiguousarray(base.transpose(1, 0, 2, 3, 4))
    else:
        paged = [base[0].copy(), base[1].copy()]
    slots = rng.permutation(nb * bs)[:17]
    got = O.gather_paged_kv(paged, slots, bs)
    for t, s in enumerate(slots):
        for c in range(2):
            np.testing.assert_array_equal(got[c, t], base[c, s // bs, s % bs])
    # scatter is the inverse on the touched slots and leaves the rest alone
    fresh = rng.standard_normal(got.shape).astype(np.float32)
    before = O.gather_paged_kv(paged, np.arange(nb * bs), bs)
    O.scatter_paged_kv(fresh, paged, slots, bs)
    after = O.gather_paged_kv(paged, np.arange(nb * bs), bs)
    untouched = np.setdiff1d(np.arange(nb * bs), slots)
    np.testing.assert_array_equal(after[:, untouched], before[:, untouched])
    np.testing.assert_array_equal(after[:, slots], fresh)


def test_negative_or_large_slots_rejected():
    paged = np.zeros((2, 3, 2, 1, 1), dtype=np.float32)
    with pytest.raises(IndexError):
        O.gather_paged_kv(paged, np.array([-1]), 2)
    with pytest.raises(IndexError):
        O.gather_paged_kv(paged, np.array([6]), 2)


def test_slot_mapping_known_answers(golden):
    for case in golden["slot_mapping"]["cases"]:
        got = O.slot_mapping(case["block_ids"], case["block_size"], case["token_count"])
        assert got.tolist() == case["expected"]


def test_slot_mapping_brute_force():
    ids = [9, 2, 4]
    got = O.slot_mapping(ids, 4, 10)
    assert got.tolist() == [ids[i // 4] * 4 + i % 4 for i in range(10)]


# ------------------------------------------------------------------- bf16 bits


def test_bf16_round_trip_and_rne():
    # exact values survive; halfway cases round to even
    vals = np.array([1.0, -2.5, 0.0, 3.140625], dtype=np.float32)
    np.testing.assert_array_equal(O.round_bf16(vals), vals)
    one = np.float32(1.0).view(np.uint32)
    halfway_even = np.array([one + 0x8000], dtype=np.uint32).view(np.float32)  # 1 + 2^-8
    halfway_odd = np.array([one + 0x18000], dtype=np.uint32).view(np.float32)
    assert O.round_bf16(halfway_even)[0] == np.float32(1.0)
    assert O.round_bf16(halfway_odd)[0] == np.array([one + 0x20000], dtype=np.uint32).view(np.float32)[0]
    assert np.isnan(O.round_bf16(np.array([np.nan], dtype=np.float32)))[0]


# ------------------------------------------------------------------- selection


def test_select_known_answers(golden):
    case = golden["select_keeps_gaps"]
    got = O.select(np.array(case["scores"]), np.array(case["gap"]), case["ratio"])
    assert got.tolist() == case["expected"]
    case = golden["select_forced_not_budgeted"]
    got = O.select(
        np.array(case["scores"]), np.array(case["gap"]), case["ratio"], np.array(case["forced"])
    )
    assert got.tolist() == case["expected"]


def _brute_select(scores, gap, ratio, forced=None):
    n = len(scores)
    base = list(gap) if forced is None else [g or f for g, f in zip(gap, forced)]
    cached = n - sum(gap)
    topk = int(cached * ratio)
    available = n - sum(base)
    topk = min(max(topk, 1), available) if cached and available else 0
    masked = [(-math.inf if b else float(s)) for s, b in zip(scores, base)]
    # python's sort is stable: sort by -score, ties keep ascending index
    order = sorted(range(n), key=lambda i: -masked[i])
    chosen = set(i for i in range(n) if base[i]) | set(order[:topk])
    return sorted(chosen)


def test_select_brute_force_with_ties():
    rng = np.random.default_rng(7)
    for trial in range(300):
        n = int(rng.integers(1, 12))
        scores = rng.integers(0, 4, n).astype(np.float32)  # many exact ties
        gap = rng.random(n) < 0.3
        forced = rng.random(n) < 0.2 if trial % 2 else None
        ratio = float(rng.choice([0.0, 0.15, 0.5, 0.99, 1.0]))
        got = O.select(scores, gap, ratio, forced)
        assert got.tolist() == _brute_select(scores, gap, ratio, forced), (scores, gap, forced, ratio)


def test_select_lower_index_wins_ties():
    scores = np.zeros(10, dtype=np.float32)
    gap = np.zeros(10, dtype=bool)
    assert O.select(scores, gap, 0.3).tolist() == [0, 1, 2]
    scores[7] = 1.0
    assert O.select(scores, gap, 0.3).tolist() == [0, 1, 7]


def test_select_budget_floor_and_minimum():
    # int() truncation of the float64 product, minimum one, capped by available
    assert O.select_budget(512, 0, 0, 0.15) == 76
    assert O.select_budget(65536, 13107, 13107, 0.15) == int(52429 * 0.15) == 7864
    assert O.select_budget(10, 0, 0, 0.01) == 1
    assert O.select_budget(10, 10, 10, 0.5) == 0
    assert O.select_budget(10, 2, 9, 0.9) == 1


def test_float_order_keys_total_order():
    vals = np.array([-np.inf, -3.0, -1e-30, -0.0, 0.0, 1e-30, 2.0, np.inf, np.nan], dtype=np.float32)
    keys = O.float_order_keys(vals)
    assert np.all(np.diff(keys[:3].astype(np.int64)) > 0)
    assert keys[3] == keys[4]  # -0.0 ties +0.0
    assert np.all(np.diff(keys[4:].astype(np.int64)) > 0)  # NaN ranks highest


def test_dilate_brute_force():
    rng = np.random.default_rng(3)
    for _ in range(200):
        n = int(rng.integers(1, 40))
        gap = rng.random(n) < 0.1
        r = int(rng.integers(0, 6))
        want = [any(gap[max(0, i - r) : min(n, i + r + 1)]) for i in range(n)]
        assert O.dilate(gap, r).tolist() == want


def test_sparse_q_masks_known_answers(golden):
    case = golden["sparse_q_overflow_and_tail"]
    radius = case["overflow_blocks"] * case["block_size"]
    for sub in case["cases"]:
        _, forced, tail = O.sparse_q_masks(np.array(sub["gap"]), case["tail_query_tokens"], radius)
        assert forced.tolist() == sub["expected_forced"]
        assert tail == sub["expected_tail_fallback"]


def test_sparse_q_scores_known_answers(golden):
    case = golden["sparse_q_closed_form"]
    q1 = np.array(case["query_one_head"], dtype=np.float32)
    query = np.concatenate([q1, q1[..., ::-1]], axis=1)
    key = np.array(case["key"], dtype=np.float32)
    scores, forced, stats = O.sparse_q_scores(
        query,
        key,
        np.array(case["absolute"]),
        np.array(case["gap"]),
        case["scale"],
        block_size=case["block_size"],
        overflow_blocks=case["overflow_blocks"],
        tail_query_tokens=case["tail_query_tokens"],
        chunk=case["query_score_chunk_size"],
    )
    np.testing.assert_allclose(scores, case["expected_scores"], rtol=1e-6)
    assert forced.tolist() == case["expected_forced"]
    assert stats["sparse_query_tokens"] == case["expected_sparse_query_tokens"]
    assert stats["tail_fallback"] == case["expected_tail_fallback"]

    sub = golden["sparse_q_overflow_and_tail"]
    for c in sub["cases"]:
        _, forced, stats = O.sparse_q_scores(
            np.ones((6, 1, 2), np.float32),
            np.ones((6, 1, 2), np.float32),
            np.array(sub["absolute"]),
            np.array(c["gap"]),
            sub["scale"],
            block_size=sub["block_size"],
            overflow_blocks=sub["overflow_blocks"],
            tail_query_tokens=sub["tail_query_tokens"],
            chunk=sub["query_score_chunk_size"],
        )
        assert forced.tolist() == c["expected_forced"]
        if "expected_sparse_query_tokens" in c:
            assert stats["sparse_query_tokens"] == c["expected_sparse_query_tokens"]


def test_sparse_q_matches_float64_dense_softmax_and_mass():
    rng = np.random.default_rng(11)
    nq, hq, hkv, d, nk = 9, 4, 2, 8, 23
    q = rng.standard_normal((nq, hq, d)).astype(np.float32)
    k = rng.standard_normal((nk, hkv, d)).astype(np.float32)
    pos = np.sort(rng.choice(nk, nq, replace=False))
    got = O.sparse_q_full_scores(q, k, pos, 0.3, round_logits_bf16=False, chunk=4)
    want = np.zeros(nk)
    for h in range(hq):
        kv = h // (hq // hkv)
        for i in range(nq):
            logits = np.array([q[i, h].astype(np.float64) @ k[j, kv] * 0.3 for j in range(pos[i] + 1)])
            p = np.exp(logits - logits.max())
            want[: pos[i] + 1] += p / p.sum()
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=1e-7)
    # every softmax row sums to one: total mass = queries x heads
    assert abs(float(got.sum()) - nq * hq) < 1e-3
    # chunking does not change the result beyond float32 noise
    np.testing.assert_allclose(
        O.sparse_q_full_scores(q, k, pos, 0.3, False, chunk=1), got, rtol=1e-6, atol=1e-7
    )


def test_sparse_q_bf16_logit_rounding_is_applied():
    # logits 1 + 2^-8 (halfway) round to 1.0 in bf16; softmax sees equal logits
    q = np.array([[[1.0 + 2.0**-8]]], dtype=np.float32)
    k = np.array([[[1.0]], [[1.0]]], dtype=np.float32)
    k[1] = 1.0 / (1.0 + 2.0**-8)
    pos = np.array([1])
    rounded = O.sparse_q_full_scores(q, k, pos, 1.0, round_logits_bf16=True)
    np.testing.assert_allclose(rounded, [0.5, 0.5], rtol=1e-6)
    exact = O.sparse_q_full_scores(q, k, pos, 1.0, round_logits_bf16=False)
    assert exact[0] > 0.5


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_sparse_q_logit_rounding_order_matches_torch_cpu_chain(dtype):
    """ascend.py:688-698 run on torch's CPU kernels -- a 16-bit ``matmul``,
    ``.float()``, ``mul_(scale)``, the causal ``masked_fill_``, ``softmax``,
    the sum -- at scale 0.37 against the oracle: the rounding to the input
    dtype sits before the scale. Rounding after the scale, or not rounding,
    moves most columns by far more than the float32 summation noise the
    oracle shows."""
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16}[dtype]
    g = torch.Generator().manual_seed(3)
    nq, hq, hkv, d, nk, scale = 24, 8, 2, 64, 300, 0.37
    q = (torch.randn(nq, hq, d, generator=g) * 0.6).to(tdt)
    k = (torch.randn(nk, hkv, d, generator=g) * 0.6).to(tdt)
    pos = torch.sort(torch.randperm(nk, generator=g)[:nq]).values
    groups = hq // hkv
    kt = k.permute(1, 2, 0).contiguous()
    full = torch.zeros(nk)
    key_pos = torch.arange(nk)
    for start in range(0, nq, 8):
        end = min(start + 8, nq)
        qc = q[start:end].view(end - start, hkv, groups, d).permute(1, 2, 0, 3).contiguous()
        logits = torch.matmul(qc, kt[:, None]).float()
        logits.mul_(scale)
        logits.masked_fill_((pos[start:end, None] < key_pos[None, :])[None, None],
                            torch.finfo(logits.dtype).min)
        full.add_(torch.softmax(logits, dim=-1).sum(dim=(0, 1, 2)))
    want = full.numpy()
    live = int(pos.max()) + 1  # keys past the last query carry no mass
    assert np.all(want[live:] == 0) and np.all(want[:live] > 0)
    qf, kf = q.float().numpy(), k.float().numpy()

    def rel(got):
        assert np.all(got[live:] == 0)
        return np.abs(got[:live] - want[:live]) / want[:live]

    oracle = O.sparse_q_full_scores(qf, kf, pos.numpy(), scale, False, logit_dtype=dtype)
    assert rel(oracle).max() < 2e-6
    after = O.sparse_q_full_scores(qf, kf, pos.numpy(), scale, False, logit_dtype=dtype,
                                   round_after_scale=True)
    unrounded = O.sparse_q_full_scores(qf, kf, pos.numpy(), scale, False)
    for wrong in (after, unrounded):
        assert (rel(wrong) > 1e-5).mean() > 0.5


def test_kdev_scores_closed_form():
    rng = np.random.default_rng(5)
    a = rng.integers(-8, 8, (33, 40)).astype(np.float32)
    b = rng.integers(-8, 8, (33, 40)).astype(np.float32)
    want = ((a.astype(np.int64) - b.astype(np.int64)) ** 2).sum(axis=1)
    np.testing.assert_array_equal(O.kdev_scores(a, b), want.astype(np.float32))
    assert np.all(O.kdev_scores(a, a) == 0)
    # sign of the difference does not matter, magnitude does
    np.testing.assert_array_equal(O.kdev_scores(a, b), O.kdev_scores(b, a))


# ----------------------------------------------------------- relocation/loader


class _FakeRope:
    """Closed-form RoPE with one angle per position (tests/test_ascend.py:17-42)."""

    def __init__(self, neox, angle):
        self.neox, self.angle = neox, angle

    def __call__(self, positions, value):
        shaped = value.reshape(value.shape[0], -1, 4)
        ang = positions.astype(np.float32).reshape(-1, 1, 1) * np.float32(self.angle)
        c, s = np.cos(ang), np.sin(ang)
        if self.neox:
            f, sec = shaped[..., :2], shaped[..., 2:]
            out = np.concatenate((f * c - sec * s, sec * c + f * s), axis=-1)
        else:
            f, sec = shaped[..., 0::2], shaped[..., 1::2]
            out = np.stack((f * c - sec * s, sec * c + f * s), axis=-1).reshape(shaped.shape)
        return out.reshape(value.shape).astype(np.float32)


@pytest.mark.parametrize("neox", [False, True])
def test_relocate_key_matches_fresh_rope(golden, neox):
    case = golden["relocate_key_matches_fresh_rope"]
    rope = _FakeRope(neox, case["angle_per_position"])
    raw = np.random.default_rng(0).standard_normal((case["key_rows"], case["key_width"])).astype(np.float32)
    old = np.array(case["old_positions"])
    new = np.array(case["new_positions"])
    positions = np.arange(16)
    ang = positions[:, None].astype(np.float32) * np.float32(case["angle_per_position"])
    cache = np.concatenate([np.cos(ang), np.cos(ang), np.sin(ang), np.sin(ang)], axis=1)
    got = O.relocate_key(cache, old, new, rope(old, raw), case["head_size"], neox, bf16=False)
    np.testing.assert_allclose(got, rope(new, raw), atol=case["atol"], rtol=case["rtol"])


def test_relocate_group_property_and_identity():
    rng = np.random.default_rng(2)
    pos = np.arange(64)
    inv = 1.0 / (10000 ** (np.arange(0, 8, 2) / 8))
    ang = (pos[:, None] * inv[None, :]).astype(np.float32)
    cache = np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)
    key = rng.standard_normal((5, 16)).astype(np.float32)
    a, b, c = rng.integers(0, 64, 5), rng.integers(0, 64, 5), rng.integers(0, 64, 5)
    for neox in (False, True):
        two = O.relocate_key(cache, b, c, O.relocate_key(cache, a, b, key, 8, neox, False), 8, neox, False)
        one = O.relocate_key(cache, a, c, key, 8, neox, False)
        np.testing.assert_allclose(two, one, atol=2e-5)
        back = O.relocate_key(cache, b, a, O.relocate_key(cache, a, b, key, 8, neox, False), 8, neox, False)
        np.testing.assert_allclose(back, key, atol=2e-5)
        np.testing.assert_array_equal(O.relocate_key(cache, a, a, key, 8, neox, True), key)


def test_loader_known_answer(golden):
    case = golden["loader_prefix_gaps_suffix"]
    paged = _arange_base(case["paged_shape"])
    seg = case["segment"]
    host = np.array([case["host_k"], case["host_v"]], dtype=np.float32).reshape(2, seg["length"], 1, 1)
    buf = O.loader_assemble(
        paged,
        np.array(case["slots"]),
        case["block_size"],
        case["apc_prefix_tokens"],
        case["allocation_end"],
        [(seg["source_start"], seg["target_start"], host)],
    )
    assert buf[0].reshape(-1).tolist() == case["expected_buffer_k"]
    assert buf[1].reshape(-1).tolist() == case["expected_buffer_v"]
    lo, hi = case["commit_fill_range"]
    buf[:, lo:hi] = case["commit_fill"]
    O.loader_commit(
        buf, paged, np.array(case["slots"]), case["block_size"],
        case["apc_prefix_tokens"], case["allocation_end"],
    )
    assert paged[0].reshape(2, -1).tolist() == case["expected_pages_after_commit_k"]
    assert paged[1].reshape(2, -1).tolist() == case["expected_pages_after_commit_v"]


def test_select_exhaustive_permutations_tiny():
    # every ordering of distinct scores picks exactly the k largest
    for perm in itertools.permutations(range(5)):
        scores = np.array(perm, dtype=np.float32)
        gap = np.array([False, True, False, False, False])
        got = O.select(scores, gap, 0.5)
        cached = [i for i in range(5) if not gap[i]]
        top = sorted(cached, key=lambda i: -scores[i])[:2]
        assert got.tolist() == sorted({1, *top})


# ---- blend_attention (side-forward attention of the selected queries) ----

def test_blend_attention_single_visible_key_returns_its_value_per_kv_head():
    rng = np.random.default_rng(11)
    q = rng.standard_normal((3, 4, 16)).astype(np.float32)
    k = rng.standard_normal((6, 2, 16)).astype(np.float32)
    v = O.round_bf16(rng.standard_normal((6, 2, 16)))
    out = O.blend_attention(q, k, v, np.zeros(3, dtype=np.int64), 0.25, "bf16")
    for h in range(4):  # GQA: heads 0,1 read KV head 0, heads 2,3 read KV head 1
        np.testing.assert_array_equal(out[:, h, :], np.broadcast_to(v[0, h // 2], (3, 16)))


def test_blend_attention_identical_keys_average_the_visible_values():
    rng = np.random.default_rng(12)
    q = rng.standard_normal((4, 2, 8)).astype(np.float32)
    k = np.broadcast_to(rng.standard_normal((1, 1, 8)), (10, 1, 8)).astype(np.float32)
    v = rng.standard_normal((10, 1, 8)).astype(np.float32)
    pos = np.array([0, 3, 9, 5])
    out = O.blend_attention(q, k, v, pos, 0.5, None)
    for i, p in enumerate(pos):
        np.testing.assert_allclose(out[i], np.broadcast_to(v[: p + 1, 0].mean(axis=0), (2, 8)), rtol=1e-6)


def test_blend_attention_zero_query_is_uniform_and_rounding_is_bounded():
    rng = np.random.default_rng(13)
    k = rng.standard_normal((50, 2, 32)).astype(np.float32)
    v = O.round_bf16(rng.standard_normal((50, 2, 32)))
    pos = np.array([49, 20])
    zero = O.blend_attention(np.zeros((2, 2, 32), np.float32), k, v, pos, 1.0, None)
    np.testing.assert_allclose(zero[0], v[:, :, :].mean(axis=0), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(zero[1], v[:21].mean(axis=0), rtol=1e-5, atol=1e-7)
    q = O.round_bf16(rng.standard_normal((40, 4, 32)))
    pos2 = np.arange(40) % 50
    exact = O.blend_attention(q, k, v, pos2, 32 ** -0.5, None)
    rounded = O.blend_attention(q, k, v, pos2, 32 ** -0.5, "bf16")
    diff = np.abs(rounded - exact)
    assert diff.max() < 3e-2 * np.abs(v).max()  # bf16 rounding of logits, probabilities and output
    assert diff.max() > 0                        # ... which does change the result


def test_blend_attention_rejects_non_divisible_heads():
    with pytest.raises(ValueError, match="divisible"):
        O.blend_attention(np.zeros((1, 3, 4)), np.zeros((2, 2, 4)), np.zeros((2, 2, 4)), np.zeros(1), 1.0)


# ---------------------------------------------------------------- token matching


def test_content_hash_closed_forms_and_wrap():
    assert O.content_hash([]) == 0
    assert O.content_hash([0]) == 1
    assert O.content_hash([41]) == 42
    assert O.content_hash([2, 5]) == 3 * 1_000_003 + 6
    assert O.content_hash([-1]) == 0  # token + 1 wraps to zero
    big = [2**40] * 9  # overflows 64 bits: the sum of powers, reduced once
    assert O.content_hash(big) == sum((2**40 + 1) * 1_000_003 ** (8 - j) for j in range(9)) % 2**64


def test_window_hashes_reference_known_answer(golden):
    case = golden["rolling_hash_every_offset"]
    tokens, w = case["tokens"], case["window"]
    got = O.window_hashes(tokens, w)
    assert [int(v) for v in got] == [O.content_hash(tokens[i:i + w]) for i in range(len(tokens) - w + 1)]
    assert O.window_hashes(tokens[:2], w).shape == (0,)
    with pytest.raises(ValueError):
        O.window_hashes(tokens, 0)


def test_window_hashes_long_windows_wrap_like_horner():
    rng = np.random.default_rng(3)
    tokens = rng.integers(0, 150_000, size=600).tolist()
    got = O.window_hashes(tokens, 256)
    for i in (0, 1, 17, 344):
        assert int(got[i]) == O.content_hash(tokens[i:i + 256])


def _records(case):
    return [(s, O.content_hash(t), tuple(t)) for s, _, t in case["register"]]


def test_match_tokens_reference_known_answers(golden):
    case = golden["matcher_offsets_and_overlaps"]
    records = _records(case)
    got = O.match_tokens(records, "m", case["query"], case["start_offset"], case["chunk_size"])
    sources = [r[1] for r in case["register"]]
    assert [[t, sources[i]] for t, i in got] == case["expected_target_source"]
    assert O.match_tokens(records, "other", case["query"], 0, 4) == []
    col = golden["matcher_collision_verified"]
    fake = [(col["fake_record"]["scope"], O.content_hash(col["fake_record"]["hash_of"]),
             tuple(col["fake_record"]["tokens"]))]
    assert O.match_tokens(fake, "m", col["query"], 0, col["chunk_size"]) == col["expected"]
    with pytest.raises(ValueError):
        O.match_tokens(records, "m", [1, 2], 3, 4)


def test_match_tokens_brute_force_properties():
    """Tiny vocabularies: matches are sorted, non-overlapping, verified, and
    greedy -- no registered chunk occurs at a start between matches that the
    scan could have taken."""
    rng = np.random.default_rng(11)
    for trial in range(300):
        w = int(rng.integers(1, 4))
        tokens = rng.integers(0, 3, size=int(rng.integers(0, 24))).tolist()
        chunks = {tuple(rng.integers(0, 3, size=w).tolist()) for _ in range(int(rng.integers(1, 5)))}
        records = [("m", O.content_hash(c), c) for c in sorted(chunks)]
        start = int(rng.integers(0, len(tokens) + 1))
        got = O.match_tokens(records, "m", tokens, start, w)
        # brute force: walk positions, take every registered window greedily
        expect, p = [], start
        while p + w <= len(tokens):
            window = tuple(tokens[p:p + w])
            if window in chunks:
                expect.append((p, sorted(chunks).index(window)))
                p += w
            else:
                p += 1
        assert got == expect, (trial, tokens, chunks, start)


def _attention_brute_force(q, k, v, pos, scale):
    """Per-(query, head) causal softmax in float64 with Python scalars."""
    nq, hq, d = q.shape
    nk, hkv, _ = k.shape
    g = hq // hkv
    out = np.zeros((nq, hq, d))
    for i in range(nq):
        for h in range(hq):
            kvh = h // g
            logits = [scale * math.fsum(float(q[i, h, j]) * float(k[t, kvh, j]) for j in range(d))
                      for t in range(int(pos[i]) + 1)]
            top = max(logits)
            w = [math.exp(x - top) for x in logits]
            total = math.fsum(w)
            for j in range(d):
                out[i, h, j] = math.fsum(w[t] * float(v[t, kvh, j]) for t in range(len(w))) / total
    return out


def test_blend_attention_scaled_softmax_brute_force():
    """Non-constant logits, scale not in {0, 1}, GQA 3 query heads per KV head,
    positions that cut the context at different keys (ascend.py:827-846)."""
    rng = np.random.default_rng(21)
    q = rng.standard_normal((5, 6, 8)).astype(np.float32)
    k = rng.standard_normal((9, 2, 8)).astype(np.float32)
    v = rng.standard_normal((9, 2, 8)).astype(np.float32)
    pos = np.array([0, 8, 3, 6, 1])
    for scale in (0.37, 1.7):
        got = O.blend_attention(q, k, v, pos, scale, None)
        want = _attention_brute_force(q, k, v, pos, scale)
        np.testing.assert_allclose(got, want, rtol=2e-5, atol=1e-6)
    # the scale matters: the result at 0.37 is not the result at 1.7 or at 1
    assert np.abs(O.blend_attention(q, k, v, pos, 0.37, None)
                  - O.blend_attention(q, k, v, pos, 1.0, None)).max() > 1e-2


def test_blend_attention_two_key_closed_form():
    """A query at position 1 sees keys 0 and 1 only; the weight on key 1 is
    sigmoid(scale * (q.k1 - q.k0)) and the output is v0 + w1 (v1 - v0)."""
    rng = np.random.default_rng(22)
    q = rng.standard_normal((1, 2, 16)).astype(np.float32)
    k = rng.standard_normal((4, 1, 16)).astype(np.float32)
    k[2:] *= 50.0  # keys past the query position would dominate if not masked
    v = rng.standard_normal((4, 1, 16)).astype(np.float32)
    scale = 0.61
    got = O.blend_attention(q, k, v, np.array([1]), scale, None)
    for h in range(2):
        diff = float(np.dot(q[0, h].astype(np.float64), (k[1, 0] - k[0, 0]).astype(np.float64)))
        w1 = 1.0 / (1.0 + math.exp(-scale * diff))
        want = v[0, 0].astype(np.float64) + w1 * (v[1, 0].astype(np.float64) - v[0, 0])
        np.testing.assert_allclose(got[0, h], want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("rounding", ["bf16", "f16"])
def test_blend_attention_rounding_sequence_matches_torch_cpu(rounding):
    """The rounded path against torch's own CPU kernels run in the order the
    reference's einsum path uses (ascend.py:834-846): einsum in the input
    dtype, ``* scale`` in the input dtype, masked_fill with the dtype's
    minimum, float32 softmax cast back to the input dtype, einsum. Query and
    key values are multiples of 1/8 so the score sums are exact in float32
    and only the roundings under test can differ."""
    torch = pytest.importorskip("torch")
    dt = {"bf16": torch.bfloat16, "f16": torch.float16}[rounding]
    rng = np.random.default_rng(23)
    nq, hq, hkv, nk, d = 6, 4, 2, 11, 16
    q = (rng.integers(-12, 13, (nq, hq, d)) / 8.0).astype(np.float32)
    k = (rng.integers(-12, 13, (nk, hkv, d)) / 8.0).astype(np.float32)
    v = O.round_bf16(rng.standard_normal((nk, hkv, d))) if rounding == "bf16" else \
        O.round_f16(rng.standard_normal((nk, hkv, d)))
    pos = np.array([10, 0, 4, 7, 2, 9])
    scale = 0.3
    tq, tk, tv = (torch.from_numpy(x).to(dt) for x in (q, k, v))
    g = hq // hkv
    tk = tk[:, :, None].expand(-1, -1, g, -1).reshape(nk, hq, d)
    tv = tv[:, :, None].expand(-1, -1, g, -1).reshape(nk, hq, d)
    mask = torch.from_numpy(pos)[:, None] < torch.arange(nk)[None, :]
    w = torch.einsum("qhd,khd->hqk", tq, tk) * scale
    w = w.masked_fill(mask[None], torch.finfo(w.dtype).min)
    p = torch.softmax(w.float(), dim=-1).to(dt)
    want = torch.einsum("hqk,khd->qhd", p, tv).float().numpy()
    got = O.blend_attention(q, k, v, pos, scale, rounding)
    np.testing.assert_array_equal(got, want)
    # a rounding dropped anywhere in the chain is visible at these inputs
    assert not np.array_equal(O.blend_attention(q, k, v, pos, scale, None), want)


@pytest.mark.parametrize("neox", [False, True])
def test_relocate_key_bf16_matches_torch_cpu_bf16_ops(neox):
    """relocate_key(bf16=True) against torch's CPU bf16 elementwise kernels run
    in the order of ascend.py:76-103 (cache cast to the key dtype, index,
    delta cos/sin, rotation; every product, sum and difference rounded to
    bf16 by torch). Elementwise ops round per element, so equality is exact."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(24)
    head, heads, rows, max_pos = 16, 3, 40, 300
    inv = 1.0 / (10000 ** (np.arange(0, head, 2) / head))
    ang = np.arange(max_pos)[:, None] * inv[None, :]
    cache = np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)
    key = O.round_bf16(rng.standard_normal((rows, heads * head)))
    old = rng.integers(0, max_pos, rows)
    new = rng.integers(0, max_pos, rows)
    tcache = torch.from_numpy(cache).to(torch.bfloat16)
    oc, os_ = tcache.index_select(0, torch.from_numpy(old)).chunk(2, dim=-1)
    nc, ns = tcache.index_select(0, torch.from_numpy(new)).chunk(2, dim=-1)
    dcos = (nc * oc + ns * os_).unsqueeze(1)
    dsin = (ns * oc - nc * os_).unsqueeze(1)
    shaped = torch.from_numpy(key).to(torch.bfloat16).reshape(rows, heads, head)
    if neox:
        first, second = torch.chunk(shaped, 2, dim=-1)
        want = torch.cat((first * dcos - second * dsin, second * dcos + first * dsin), dim=-1)
    else:
        first, second = shaped[..., ::2], shaped[..., 1::2]
        want = torch.stack((first * dcos - second * dsin, second * dcos + first * dsin), dim=-1).flatten(-2)
    want = want.reshape(rows, heads * head).float().numpy()
    got = O.relocate_key(cache, old, new, key, head, neox, bf16=True)
    np.testing.assert_array_equal(got, want)
    # float32 arithmetic rounded once at the end is not the same thing
    once = O.round_bf16(O.relocate_key(cache, old, new, key, head, neox, bf16=False))
    assert not np.array_equal(once, want)
