"""GPU parity: Sparse-Q attention-mass scores and selection.

Scores must match the oracle within 1e-2 relative (the stated tolerance of the path;
the observed error is printed and is far smaller). Index sets are compared
outside an epsilon band around the k-th score: keys whose scores differ from
the boundary by more than the largest observed score difference must agree.
"""

import numpy as np
import pytest
import torch

import oracle as O
from cacheblend_vllm import selection as S
from cacheblend_vllm import synthetic
from cacheblend_vllm.config import CacheBlendConfig

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
RTOL = 1e-2
# logits are rounded to the input dtype before the scale (ascend.py:694-695)
LOGIT_DTYPE = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: None}


def test_reference_closed_form_known_answer(golden):
    case = golden["sparse_q_closed_form"]
    q1 = torch.tensor(case["query_one_head"])
    query = torch.cat((q1, q1.flip(-1)), dim=1).to(DEV)
    key = torch.tensor(case["key"]).to(DEV)
    sel = S.BlendSelector(CacheBlendConfig.from_extra_config({
        "selection_strategy": "sparse_q", "check_layers": [1],
        "query_score_chunk_size": case["query_score_chunk_size"],
        "overflow_blocks": case["overflow_blocks"], "tail_query_tokens": case["tail_query_tokens"],
        "strict_version_check": False}), case["block_size"])
    scores, forced, stats = sel._sparse_q_scores(
        query, key, torch.tensor(case["absolute"], device=DEV),
        torch.tensor(case["gap"], device=DEV), case["scale"])
    np.testing.assert_allclose(scores.cpu().numpy(), case["expected_scores"], rtol=1e-5)
    assert forced.tolist() == case["expected_forced"]
    assert stats["sparse_query_tokens"] == case["expected_sparse_query_tokens"]
    assert stats["tail_fallback"] == case["expected_tail_fallback"]


def test_reference_overflow_and_tail_known_answers(golden):
    case = golden["sparse_q_overflow_and_tail"]
    sel = S.BlendSelector(CacheBlendConfig.from_extra_config({
        "chunk_size": 2, "selection_strategy": "sparse_q", "check_layers": [1],
        "query_score_chunk_size": case["query_score_chunk_size"],
        "overflow_blocks": case["overflow_blocks"], "tail_query_tokens": case["tail_query_tokens"],
        "strict_version_check": False}), case["block_size"])
    ones = torch.ones(6, 1, 2, device=DEV)
    for sub in case["cases"]:
        _, forced, stats = sel._sparse_q_scores(ones, ones, torch.tensor(case["absolute"], device=DEV),
                                                torch.tensor(sub["gap"], device=DEV), case["scale"])
        assert forced.tolist() == sub["expected_forced"]
        assert stats["tail_fallback"] == sub["expected_tail_fallback"]
        if "expected_sparse_query_tokens" in sub:
            assert stats["sparse_query_tokens"] == sub["expected_sparse_query_tokens"]
    with pytest.raises(ValueError, match="divisible by KV heads"):
        sel._sparse_q_scores(torch.ones(6, 3, 2, device=DEV), torch.ones(6, 2, 2, device=DEV),
                             torch.arange(6, device=DEV), torch.zeros(6, dtype=torch.bool, device=DEV), 1.0)


def _inputs(n_active, prefix, hq, hkv, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    nk = prefix + n_active
    q = (torch.randn(n_active, hq, d, generator=g) / d ** 0.5).to(dtype)
    k = (torch.randn(nk, hkv, d, generator=g) / d ** 0.5).to(dtype)
    gap = torch.from_numpy(synthetic.gap_layout(n_active, seed, hit_chunk=64, max_hit_chunks=5, max_gap=63))
    absolute = torch.arange(prefix, nk)
    return q, k, gap, absolute


@pytest.mark.parametrize("dtype,d,hq,hkv", [
    (torch.bfloat16, 128, 32, 4),
    (torch.bfloat16, 64, 8, 8),
    (torch.float16, 128, 16, 2),
    (torch.float32, 32, 4, 2),
    # column-pass units of 4 consecutive (tile, head) rows that span two
    # tiles (3, 6) or four (1), and four 4-head units per tile (16, also the
    # widest row-statistics path)
    (torch.bfloat16, 128, 12, 4),
    (torch.bfloat16, 64, 24, 4),
    (torch.float16, 64, 4, 4),
    (torch.bfloat16, 128, 16, 1),
    # 9-15 heads per KV head: the 32x32 row pass with head slots past the
    # group; 12 leaves each wave's second pair tile half used, 9 leaves it
    # unused on three of the four waves (skipped)
    (torch.bfloat16, 128, 24, 2),
    (torch.bfloat16, 64, 9, 1),
    (torch.float16, 128, 12, 1),
    # row-pass tile grouping: 1-4 heads per KV head take four tiles per
    # workgroup (2 and 3 here, 1 and 4 above), 5-7 two tiles with head slots
    # past the group (5, 7)
    (torch.bfloat16, 128, 8, 4),
    (torch.bfloat16, 64, 6, 2),
    (torch.bfloat16, 128, 20, 4),
    (torch.float16, 64, 14, 2),
])
def test_sparse_q_scores_vs_oracle(dtype, d, hq, hkv):
    n_active, prefix = 1200 if dtype != torch.float32 else 300, 500
    q, k, gap, absolute = _inputs(n_active, prefix, hq, hkv, d, dtype, seed=d + hq)
    rows = torch.nonzero(gap).flatten()
    print(f"dtype={dtype} d={d} hq={hq} hkv={hkv} queries={rows.numel()} keys={k.shape[0]}", flush=True)
    scale = d ** -0.5
    got, full = S.sparse_q_full_scores(q.to(DEV), k.to(DEV), rows, absolute, scale,
                                       out_index=absolute, want_full=True)
    qf, kf = q.float().numpy(), k.float().numpy()
    want_full = O.sparse_q_full_scores(qf[rows.numpy()], kf, absolute.numpy()[rows.numpy()], scale, False,
                                       logit_dtype=LOGIT_DTYPE[dtype])
    full = full.cpu().numpy()
    err = np.max(np.abs(full - want_full) / np.maximum(np.abs(want_full), 1e-30))
    print(f"max relative score error {err:.3e}", flush=True)
    np.testing.assert_allclose(full, want_full, rtol=RTOL, atol=1e-6)
    np.testing.assert_allclose(got.cpu().numpy(), want_full[absolute.numpy()], rtol=RTOL, atol=1e-6)
    # softmax mass: every (query, head) row sums to one
    assert abs(full.sum() - rows.numel() * hq) < 1e-3 * rows.numel() * hq
    # deterministic
    _, again = S.sparse_q_full_scores(q.to(DEV), k.to(DEV), rows, absolute, scale, want_full=True)
    assert np.array_equal(again.cpu().numpy(), full)


def test_sparse_q_select_matches_oracle_outside_epsilon_band():
    hq, hkv, d = 32, 4, 128
    q, k, gap, absolute = _inputs(2000, 1000, hq, hkv, d, torch.bfloat16, seed=3)
    cfg = CacheBlendConfig.from_extra_config({"selection_strategy": "sparse_q", "check_layers": [1]})
    sel = S.BlendSelector(cfg, 16)
    selected, stats = sel.sparse_q_select(q.to(DEV), k.to(DEV), absolute.to(DEV), gap.to(DEV), d ** -0.5, 1)
    scores, forced, stats2 = sel._sparse_q_scores(q.to(DEV), k.to(DEV), absolute.to(DEV), gap.to(DEV), d ** -0.5)
    want_scores, want_forced, want_stats = O.sparse_q_scores(
        q.float().numpy(), k.float().numpy(), absolute.numpy(), gap.numpy(), d ** -0.5,
        block_size=16, overflow_blocks=1, tail_query_tokens=64, round_logits_bf16=True)
    assert forced.cpu().numpy().tolist() == want_forced.tolist()
    for key in ("active_tokens", "gap_tokens", "cached_tokens", "sparse_query_tokens", "tail_fallback"):
        assert stats[key] == want_stats[key]
    got_scores = scores.cpu().numpy()
    eps = float(np.max(np.abs(got_scores - want_scores)))
    # the GPU selection on the GPU's own scores is exact
    np.testing.assert_array_equal(selected.cpu().numpy(), O.select(got_scores, gap.numpy(), 0.15, want_forced))
    # against the oracle's scores: equal outside the epsilon band at the k-th score
    want_sel = O.select(want_scores, gap.numpy(), 0.15, want_forced)
    base = gap.numpy() | want_forced
    k_budget = O.select_budget(len(gap), int(gap.sum()), int(base.sum()), 0.15)
    cand = np.sort(want_scores[~base])[::-1]
    kth = cand[k_budget - 1]
    band = np.abs(want_scores - kth) <= 2 * eps
    a, b = set(selected.cpu().tolist()), set(want_sel.tolist())
    disagree = np.array(sorted(a ^ b), dtype=np.int64)
    print(f"eps={eps:.3e} band={int(band.sum())} disagreements={disagree.size}", flush=True)
    assert np.all(band[disagree])


def test_sparse_q_tail_fallback_no_gaps():
    hq, hkv, d = 8, 2, 64
    q, k, _, absolute = _inputs(700, 300, hq, hkv, d, torch.bfloat16, seed=9)
    gap = torch.zeros(700, dtype=torch.bool)
    cfg = CacheBlendConfig.from_extra_config({"selection_strategy": "sparse_q", "check_layers": [1],
                                              "tail_query_tokens": 64})
    sel = S.BlendSelector(cfg, 16)
    scores, forced, stats = sel._sparse_q_scores(q.to(DEV), k.to(DEV), absolute.to(DEV), gap.to(DEV), d ** -0.5)
    want, want_forced, want_stats = O.sparse_q_scores(
        q.float().numpy(), k.float().numpy(), absolute.numpy(), gap.numpy(), d ** -0.5,
        block_size=16, overflow_blocks=1, tail_query_tokens=64, round_logits_bf16=True)
    assert stats["tail_fallback"] and stats["sparse_query_tokens"] == 64
    assert forced.cpu().numpy().tolist() == want_forced.tolist()
    np.testing.assert_allclose(scores.cpu().numpy(), want, rtol=RTOL, atol=1e-6)


def test_sparse_q_full_layer6_vs_oracle_and_properties():
    """The layer-6 Sparse-Q shape: 4096 gap queries over a 98,304-key causal
    context, 32 query heads on 4 KV heads of 128 bf16.

    * 96 of the gap queries (the last one, at position 98,303, among them)
      against the oracle at the full context: all 98,304 column sums within
      1e-2 relative;
    * linearity at the full 4096 queries: the scores of all of them equal
      the scores of those 96 plus the scores of the other 4000 (column sums
      add over queries), so a key range or workspace offset that goes wrong
      only at the full query count shows;
    * the column sums add up to queries x heads (every softmax row sums to
      one), scores are finite and non-negative, keys after the last query
      get nothing, and the launch is deterministic."""
    nk, hq, hkv, d, nq = 98304, 32, 4, 128, 4096
    scale = d ** -0.5
    g = torch.Generator(device=DEV).manual_seed(0)
    query = (torch.randn((nk, hq, d), generator=g, device=DEV) / d ** 0.5).to(torch.bfloat16)
    key = (torch.randn((nk, hkv, d), generator=g, device=DEV) / d ** 0.5).to(torch.bfloat16)
    gap = synthetic.sparse_q_layout(nk, nq, seed=0)
    all_rows = np.flatnonzero(gap)
    assert all_rows[-1] == nk - 1
    rng = np.random.default_rng(6)
    pick = np.sort(np.concatenate(([nq - 1], rng.choice(nq - 1, 95, replace=False))))
    sub_rows, rest_rows = all_rows[pick], np.delete(all_rows, pick)
    absolute = torch.arange(nk, device=DEV)

    def scores(rows):
        _, full = S.sparse_q_full_scores(query, key, torch.from_numpy(rows).to(DEV), absolute, scale,
                                         want_full=True)
        return full.cpu().numpy()

    full = scores(all_rows)
    sub = scores(sub_rows)
    rest = scores(rest_rows)
    print(f"full-context oracle check: {sub_rows.size} queries at {sub_rows.min()}..{sub_rows.max()}",
          flush=True)
    want = O.sparse_q_full_scores(query[torch.from_numpy(sub_rows).to(DEV)].float().cpu().numpy(),
                                  key.float().cpu().numpy(), sub_rows, scale, True)
    err = np.max(np.abs(sub - want) / np.maximum(want, 1e-30))
    print(f"max relative score error over {nk} keys: {err:.3e}", flush=True)
    np.testing.assert_allclose(sub, want, rtol=RTOL, atol=1e-6)
    # the selection over all 98,304 tokens on these scores (top 15% of the
    # cached keys, gaps and 16-token overflow forced): the GPU's index set
    # equals the oracle's outside the epsilon band at the k-th score
    forced = O.dilate(gap, 16)
    got_sel = S.select(torch.from_numpy(sub).to(DEV), torch.from_numpy(gap).to(DEV), 0.15,
                       torch.from_numpy(forced).to(DEV)).cpu().numpy()
    want_sel = O.select(want, gap, 0.15, forced)
    base = gap | forced
    k_budget = O.select_budget(nk, int(gap.sum()), int(base.sum()), 0.15)
    kth = np.sort(want[~base])[::-1][k_budget - 1]
    eps = float(np.max(np.abs(sub - want)[~base]))
    band = ~base & (np.abs(want - kth) <= 2 * eps)
    disagree = np.setxor1d(got_sel, want_sel)
    print(f"full-context selection: {got_sel.size} selected, band {int(band.sum())}, "
          f"disagreements {disagree.size}", flush=True)
    assert got_sel.size == want_sel.size
    assert np.all(band[disagree])
    # linearity over the query set at the full size
    np.testing.assert_allclose(full, sub + rest, rtol=1e-4, atol=1e-6)
    full64 = full.astype(np.float64)
    assert np.isfinite(full64).all() and (full64 >= 0).all()
    assert abs(full64.sum() - nq * hq) < 1e-3 * nq * hq
    assert (full[all_rows.max() + 1:] == 0).all()
    assert np.array_equal(scores(all_rows), full)


@pytest.mark.parametrize("hq", [2, 4, 6, 8, 10, 16])
@pytest.mark.parametrize("n_active,prefix,d", [(1, 0, 128), (5, 0, 64), (17, 40, 128), (63, 1, 64),
                                                (64, 0, 128), (65, 63, 128), (200, 3, 64)])
def test_sparse_q_small_contexts(n_active, prefix, d, hq):
    """1 to 265 keys and 1 to 200 queries: partial 64-key blocks (rows past
    the context repeat the last key and are masked), single and partial
    16-query tiles (rows past the queries are zeros, masked in the column
    pass). 16 query heads over 2 KV heads take the row pass that pairs
    adjacent tiles: 1 and 5 tiles leave the last pair's second tile empty;
    2 to 8 heads take four tiles per row-pass workgroup (1 to 5 tiles: empty
    tiles in the last group), and 2 or 4 heads (1 or 2 per KV head) also
    column-pass units of four or two tiles, whose last unit holds empty
    tiles; 6 and 10 heads (3 and 5 per KV head) take column-pass units of
    four consecutive (tile, head) rows across tile boundaries, the last of
    which reaches rows past the last tile."""
    hkv = 2
    g = torch.Generator().manual_seed(n_active * 7 + prefix)
    nk = prefix + n_active
    q = (torch.randn(n_active, hq, d, generator=g) / d ** 0.5).to(torch.bfloat16)
    k = (torch.randn(nk, hkv, d, generator=g) / d ** 0.5).to(torch.bfloat16)
    absolute = torch.arange(prefix, nk)
    rows = torch.arange(0, n_active, 1 if n_active < 20 else 3)
    print(f"queries={rows.numel()} keys={nk} d={d}", flush=True)
    _, full = S.sparse_q_full_scores(q.to(DEV), k.to(DEV), rows, absolute, d ** -0.5, want_full=True)
    want = O.sparse_q_full_scores(q.float().numpy()[rows.numpy()], k.float().numpy(),
                                  absolute.numpy()[rows.numpy()], d ** -0.5, True)
    np.testing.assert_allclose(full.cpu().numpy(), want, rtol=RTOL, atol=1e-6)
    assert abs(float(full.sum()) - rows.numel() * hq) < 1e-3 * rows.numel() * hq


@pytest.mark.parametrize("big_key", [330, 256, 1990])
def test_sparse_q_rows_far_above_their_first_block(big_key):
    """Row statistics are summed against the first key block of each key
    range (the row pass splits a tile's blocks into up to 8 equal ranges:
    here 3 tiles at positions 1992-2031, 32 blocks each, ranges of 4
    blocks); rows with a logit more than 127 (log2 units) above that
    reference overflow the sum and are recomputed with online maxima. One key
    carries logits ~350 log2 units above every other for a third of the
    queries -- inside a range (330: block 5 of [4, 8)), at a range's first
    block (256: block 4), in the last block (1990: block 31 of [28, 32)) --
    and every score must still match the oracle."""
    g = torch.Generator().manual_seed(7)
    n_active, prefix, hq, hkv, d = 300, 1800, 8, 2, 64
    nk = prefix + n_active
    q = torch.randn(n_active, hq, d, generator=g) / d ** 0.5
    k = torch.randn(nk, hkv, d, generator=g) / d ** 0.5
    q[::3] = 1.0
    k[big_key] = 30.0
    q, k = q.to(torch.bfloat16), k.to(torch.bfloat16)
    gap = torch.from_numpy(synthetic.gap_layout(n_active, 7, hit_chunk=64, max_hit_chunks=3, max_gap=63))
    absolute = torch.arange(prefix, nk)
    rows = torch.nonzero(gap).flatten()
    scale = d ** -0.5
    _, full = S.sparse_q_full_scores(q.to(DEV), k.to(DEV), rows, absolute, scale, want_full=True)
    want = O.sparse_q_full_scores(q.float().numpy()[rows.numpy()], k.float().numpy(),
                                  absolute.numpy()[rows.numpy()], scale, True)
    full = full.cpu().numpy()
    assert np.all(np.isfinite(full))
    np.testing.assert_allclose(full, want, rtol=RTOL, atol=1e-6)
    rr = rows.numpy()
    seen = int((absolute.numpy()[rr[rr % 3 == 0]] >= big_key).sum())
    assert seen > 0
    print(f"big key {big_key}: {seen} of every third query see it; score {full[big_key]:.1f}", flush=True)
    assert full[big_key] > 0.8 * seen * hq   # the big key takes most of those rows' mass


@pytest.mark.parametrize("seed", range(24))
def test_sparse_q_random_shapes(seed):
    """Seeded random shapes: 1-16 query heads per KV head over 1-4 KV heads,
    head_dim 64 or 128, bf16 or f16, 1-600 queries picked anywhere in a
    context of up to 2500 keys, an arbitrary first absolute position."""
    rng = np.random.default_rng(700 + seed)
    hkv = int(rng.integers(1, 5))
    hq = hkv * int(rng.integers(1, 17))
    d = int(rng.choice([64, 128]))
    dtype = [torch.bfloat16, torch.float16][seed % 2]
    prefix = int(rng.integers(0, 1000))
    n_active = int(rng.integers(1, 1501))
    nk = prefix + n_active
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(n_active, hq, d, generator=g) / d ** 0.5).to(dtype)
    k = (torch.randn(nk, hkv, d, generator=g) / d ** 0.5).to(dtype)
    absolute = torch.arange(prefix, nk)
    n_rows = int(rng.integers(1, min(n_active, 600) + 1))
    rows = torch.from_numpy(np.sort(rng.choice(n_active, n_rows, replace=False))).long()
    label = f"seed={seed} hq={hq} hkv={hkv} d={d} {dtype} keys={nk} queries={n_rows}"
    print(label, flush=True)
    _, full = S.sparse_q_full_scores(q.to(DEV), k.to(DEV), rows, absolute, d ** -0.5, want_full=True)
    qf, kf = q.float().numpy(), k.float().numpy()
    want = O.sparse_q_full_scores(qf[rows.numpy()], kf, absolute.numpy()[rows.numpy()], d ** -0.5, False,
                                  logit_dtype=LOGIT_DTYPE[dtype])
    np.testing.assert_allclose(full.cpu().numpy(), want, rtol=RTOL, atol=1e-6)
    assert abs(float(full.sum()) - n_rows * hq) < 1e-3 * n_rows * hq
