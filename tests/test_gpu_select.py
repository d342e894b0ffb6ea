"""GPU parity: K-deviation scores and budgeted selection against the oracle.

Index sets are bit-exact for identical scores (the selection is integer work
on float keys). K-deviation scores match within 1e-5 relative (the float32
summation order differs); at the headline size the index set computed from
GPU scores equals the oracle's bit for bit, with the epsilon band around the
k-th score shown to hold the k-th alone.
"""

import numpy as np
import pytest
import torch

import oracle as O
from cacheblend_vllm import _native
from cacheblend_vllm import kv_layout as KL
from cacheblend_vllm import selection as S
from cacheblend_vllm import synthetic
from cacheblend_vllm.config import CacheBlendConfig

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
SCORE_RTOL = 1e-5


def test_reference_known_answers(golden):
    case = golden["select_keeps_gaps"]
    got = S.select(torch.tensor(case["scores"], device=DEV), torch.tensor(case["gap"], device=DEV), case["ratio"])
    assert got.tolist() == case["expected"]
    case = golden["select_forced_not_budgeted"]
    got = S.select(
        torch.tensor(case["scores"], device=DEV),
        torch.tensor(case["gap"], device=DEV),
        case["ratio"],
        torch.tensor(case["forced"], device=DEV),
    )
    assert got.tolist() == case["expected"]
    sel = S.BlendSelector(CacheBlendConfig.from_extra_config({"recompute_ratios": [0.5]}), 16)
    got = sel._select(torch.tensor(case["scores"], device=DEV), torch.tensor(case["gap"], device=DEV),
                      forced_mask=torch.tensor(case["forced"], device=DEV))
    assert got.tolist() == case["expected"]


@pytest.mark.parametrize("n", [1, 2, 7, 1023, 1024, 1025, 4095, 4096, 4097, 8193, 65536, 200000])
def test_select_bit_exact_vs_oracle_random(n):
    rng = np.random.default_rng(n)
    for trial in range(3):
        print(f"n={n} trial={trial}", flush=True)
        if trial == 0:
            scores = rng.standard_normal(n).astype(np.float32) ** 2
        elif trial == 1:
            scores = rng.integers(0, 5, n).astype(np.float32)  # heavy ties
        else:
            scores = rng.standard_normal(n).astype(np.float32)
            scores[rng.random(n) < 0.05] = 0.0
            scores[rng.random(n) < 0.01] = -0.0
        gap = rng.random(n) < 0.2
        forced = (rng.random(n) < 0.05) if trial != 1 else None
        ratio = [0.15, 0.5, 0.01][trial]
        radius = [0, 16, 3][trial]
        fc = forced
        if radius:
            fc = O.dilate(gap, radius) | (forced if forced is not None else False)
        want = O.select(scores, gap, ratio, fc)
        got = S.select(
            torch.from_numpy(scores).to(DEV),
            torch.from_numpy(gap).to(DEV),
            ratio,
            None if forced is None else torch.from_numpy(forced).to(DEV),
            radius=radius,
        )
        np.testing.assert_array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("n", [300, 5000, 70000])
def test_select_budget_reaching_minus_inf_ties_with_base(n):
    """The k-th largest score is -inf, the key base tokens carry too: ties
    then include base tokens and are taken in index order across tiles (the
    tile counts come from a token-by-token pass)."""
    rng = np.random.default_rng(n + 1)
    scores = np.full(n, -np.inf, dtype=np.float32)
    finite = rng.random(n) < 0.3
    scores[finite] = rng.random(int(finite.sum())).astype(np.float32)
    gap = rng.random(n) < 0.2
    forced = rng.random(n) < 0.05
    for ratio, radius in ((0.9, 0), (0.6, 4), (0.31, 0)):
        fc = forced | (O.dilate(gap, radius) if radius else False)
        want = O.select(scores, gap, ratio, fc)
        got = S.select(torch.from_numpy(scores).to(DEV), torch.from_numpy(gap).to(DEV), ratio,
                       torch.from_numpy(forced).to(DEV), radius=radius)
        np.testing.assert_array_equal(got.cpu().numpy(), want, err_msg=f"ratio {ratio} radius {radius}")


def test_select_dilation_equals_forced_mask_composition():
    # cbk_select(radius=r) == _select(gap, forced=dilate(gap, r))
    rng = np.random.default_rng(9)
    n = 5000
    scores = rng.random(n).astype(np.float32)
    gap = synthetic.gap_layout(n, seed=4)
    for r in (1, 16, 64, 4096):
        forced = O.dilate(gap, r)
        want = O.select(scores, gap, 0.15, forced)
        got = S.select(torch.from_numpy(scores).to(DEV), torch.from_numpy(gap).to(DEV), 0.15, radius=r)
        np.testing.assert_array_equal(got.cpu().numpy(), want)
        dil = S.dilate(torch.from_numpy(gap).to(DEV), r)
        np.testing.assert_array_equal(dil.cpu().numpy(), forced)


def test_select_edge_cases():
    # no cached tokens -> only gaps; nothing available -> only base; empty
    all_gap = torch.ones(10, dtype=torch.bool, device=DEV)
    assert S.select(torch.rand(10, device=DEV), all_gap, 0.5).tolist() == list(range(10))
    gap = torch.zeros(10, dtype=torch.bool, device=DEV)
    forced = torch.ones(10, dtype=torch.bool, device=DEV)
    assert S.select(torch.rand(10, device=DEV), gap, 0.5, forced).tolist() == list(range(10))
    empty = S.select(torch.empty(0, device=DEV), torch.empty(0, dtype=torch.bool, device=DEV), 0.5)
    assert empty.numel() == 0
    # NaN ranks highest, -inf never beats a finite score
    s = torch.tensor([1.0, float("nan"), 3.0, float("-inf"), 2.0], device=DEV)
    assert S.select(s, torch.zeros(5, dtype=torch.bool, device=DEV), 0.4).tolist() == [1, 2]
    with pytest.raises(ValueError, match="forced selection mask"):
        S.select(s, torch.zeros(5, dtype=torch.bool, device=DEV), 0.4, torch.zeros(4, dtype=torch.bool, device=DEV))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_kdev_scores_vs_oracle(dtype):
    fresh, cached, gap = synthetic.kdev_inputs(3000, 4, 128, dtype, DEV, seed=1)
    got = S.kdev_scores(fresh, cached)
    f = fresh.float().cpu().numpy()
    c = cached.float().cpu().numpy()
    want = O.kdev_scores(f, c)
    np.testing.assert_allclose(got.cpu().numpy(), want, rtol=SCORE_RTOL, atol=0)
    # gathered cached rows through absolute indices (ascend.py:536)
    idx = torch.randperm(3000)[:1000]
    got = S.kdev_scores(fresh[:1000], cached, idx.to(DEV))
    np.testing.assert_allclose(got.cpu().numpy(), O.kdev_scores(f[:1000], c[idx.numpy()]), rtol=SCORE_RTOL)


@pytest.mark.parametrize("kv_heads,n", [(1, 1001), (2, 3001), (2, 5), (8, 999)])
def test_kdev_scores_short_rows_share_a_wave(kv_heads, n):
    """Rows of 1 or 2 KV heads x 128 bf16 (16 or 32 lanes' loads) take four
    or two rows per wave pass; odd counts leave the last wave partly empty;
    8 heads take two passes per row. Against the oracle, with gathered rows."""
    fresh, cached, _ = synthetic.kdev_inputs(n, kv_heads, 128, torch.bfloat16, DEV, seed=kv_heads + n)
    f = fresh.float().cpu().numpy()
    c = cached.float().cpu().numpy()
    got = S.kdev_scores(fresh, cached)
    np.testing.assert_allclose(got.cpu().numpy(), O.kdev_scores(f, c), rtol=SCORE_RTOL, atol=0)
    idx = torch.randperm(n)[: max(1, n // 3)]
    got = S.kdev_scores(fresh[: idx.numel()], cached, idx.to(DEV))
    np.testing.assert_allclose(got.cpu().numpy(), O.kdev_scores(f[: idx.numel()], c[idx.numpy()]),
                               rtol=SCORE_RTOL, atol=0)


def test_kdev_odd_width_and_strided_rows():
    torch.manual_seed(5)
    fresh = torch.randn(100, 77, device=DEV).to(torch.bfloat16)
    cached = torch.randn(120, 80, device=DEV).to(torch.bfloat16)[:, :77]
    got = S.kdev_scores(fresh, cached, None, row0=20)
    want = O.kdev_scores(fresh.float().cpu().numpy(), cached[20:120].float().cpu().numpy())
    np.testing.assert_allclose(got.cpu().numpy(), want, rtol=SCORE_RTOL)


@pytest.mark.parametrize("overflow_blocks", [0, 1])
def test_kdev_select_full_size_index_set(overflow_blocks):
    """K-deviation selection at its headline size: 65,536 tokens, 4 KV heads x
    128 bf16, 20% gaps, ratio 0.15, 16-token blocks."""
    n, bs = 65536, 16
    fresh, cached, gap = synthetic.kdev_inputs(n, 4, 128, torch.bfloat16, DEV, seed=0)
    radius = overflow_blocks * bs
    selected, scores = S.kdev_select(fresh, cached, None, gap, 0.15, radius=radius)
    gap_np = gap.cpu().numpy()
    # selection is bit-exact on the GPU's own scores
    forced = O.dilate(gap_np, radius) if radius else None
    want_same = O.select(scores.cpu().numpy(), gap_np, 0.15, forced)
    np.testing.assert_array_equal(selected.cpu().numpy(), want_same)
    # oracle scores agree within tolerance ...
    got_scores = scores.cpu().numpy()
    want_scores = O.kdev_scores(fresh.float().cpu().numpy(), cached.float().cpu().numpy())
    np.testing.assert_allclose(got_scores, want_scores, rtol=SCORE_RTOL)
    # ... and, on these fixed inputs, the index set is the oracle's bit for
    # bit. Measured on the CPU: the k-th candidate score is 2332 float32 ulps
    # (overflow 0) and 51 ulps (overflow 1) from its neighbours, while the
    # float32 summation order moves a score by at most a few ulps; so the
    # band of candidates within twice the largest relative score error of
    # the k-th holds the k-th alone.
    want = O.select(want_scores, gap_np, 0.15, forced)
    base = gap_np | (forced if forced is not None else False)
    cand = np.sort(want_scores[~base])[::-1]
    k = O.select_budget(n, int(gap_np.sum()), int(base.sum()), 0.15)
    kth = cand[k - 1]
    live = ~base & (want_scores > 0)
    rel_err = float(np.max(np.abs(got_scores[live] - want_scores[live]) / want_scores[live]))
    band = ~base & (np.abs(want_scores - kth) <= 2 * rel_err * kth)
    disagree = np.setxor1d(selected.cpu().numpy(), want)
    print(f"k={k} kth={kth:.7g} max rel score error {rel_err:.3e} band={int(band.sum())} "
          f"disagreements={disagree.size}", flush=True)
    assert int(band.sum()) == 1
    assert disagree.size == 0
    np.testing.assert_array_equal(selected.cpu().numpy(), want)
    # determinism run to run
    again, _ = S.kdev_select(fresh, cached, None, gap, 0.15, radius=radius)
    assert torch.equal(again, selected)


@pytest.mark.parametrize("n", [1000, 4097, 65536])
def test_one_launch_select_gives_up_cleanly_then_falls_back(n):
    """The one-launch select's bounded wait made to give up from the host
    (CBK_SELECT_TEST_GIVE_UP: the first barrier expects one arrival more than
    the grid makes and polls zero times, so every workgroup exits normally):
    the count comes back -1 with no index written, and ``select`` /
    ``kdev_select`` then run the multi-launch select, whose result is the
    oracle's bit for bit."""
    rng = np.random.default_rng(900 + n)
    scores = (rng.standard_normal(n) ** 2).astype(np.float32)
    gap = rng.random(n) < 0.2
    want = O.select(scores, gap, 0.15, O.dilate(gap, 16))
    s_dev, g_dev = torch.from_numpy(scores).to(DEV), torch.from_numpy(gap).to(DEV)
    # through the C ABI, with the outputs prefilled: -1 and no index written
    lib = _native.load()
    out = torch.full((n,), -5, dtype=torch.long, device=DEV)
    count = torch.full((1,), -7, dtype=torch.long, device=DEV)
    ws = torch.empty(lib.cbk_select_workspace_bytes(n), dtype=torch.uint8, device=DEV)
    rc = lib.cbk_select_ex(s_dev.data_ptr(), g_dev.view(torch.uint8).data_ptr(), None, n, 16, 0.15,
                           out.data_ptr(), count.data_ptr(), ws.data_ptr(), ws.numel(),
                           _native.SELECT_TEST_GIVE_UP, _native.stream_handle(DEV))
    _native.check(rc, "select_ex")
    torch.cuda.synchronize()
    assert int(count.item()) == -1
    assert bool((out == -5).all())
    got = S.select(s_dev, g_dev, 0.15, radius=16, flags=_native.SELECT_TEST_GIVE_UP)
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    multi, mcount = S.select_async(s_dev, g_dev, 0.15, radius=16, flags=_native.SELECT_MULTI_LAUNCH)
    np.testing.assert_array_equal(multi[: int(mcount.item())].cpu().numpy(), want)
    fresh, cached, kgap = synthetic.kdev_inputs(n, 4, 128, torch.bfloat16, DEV, seed=n)
    sel_fb, sc_fb = S.kdev_select(fresh, cached, None, kgap, 0.15, radius=16, flags=_native.SELECT_TEST_GIVE_UP)
    kgap_np = kgap.cpu().numpy()
    np.testing.assert_array_equal(sel_fb.cpu().numpy(),
                                  O.select(sc_fb.cpu().numpy(), kgap_np, 0.15, O.dilate(kgap_np, 16)))
    sel, sc = S.kdev_select(fresh, cached, None, kgap, 0.15, radius=16)
    assert torch.equal(sc.view(torch.int32), sc_fb.view(torch.int32))
    assert torch.equal(sel, sel_fb)


def test_select_flag_checks():
    s_dev = torch.rand(100, device=DEV)
    g_dev = torch.zeros(100, dtype=torch.bool, device=DEV)
    with pytest.raises(ValueError, match="unknown select flags"):
        S.select_async(s_dev, g_dev, 0.15, flags=8)
    with pytest.raises(ValueError, match="needs the one-launch select"):
        S.select_async(s_dev, g_dev, 0.15, flags=_native.SELECT_TEST_GIVE_UP | _native.SELECT_MULTI_LAUNCH)


def test_selector_kv_deviation_block_matches_reference_composition():
    cfg = CacheBlendConfig.from_extra_config({"check_layers": [1], "recompute_ratios": [0.15]})
    sel = S.BlendSelector(cfg, 16)
    fresh, cached, gap = synthetic.kdev_inputs(5000, 4, 128, torch.bfloat16, DEV, seed=2)
    absolute = torch.arange(100, 5100, device=DEV)
    pool = torch.cat([torch.zeros(100, 512, dtype=torch.bfloat16, device=DEV), cached])
    got = sel.kv_deviation_select(fresh, pool, absolute, gap, layer_id=1)
    scores = S.kdev_scores(fresh, pool, absolute)
    want = O.select(scores.cpu().numpy(), gap.cpu().numpy(), 0.15)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


def test_cpu_plumbing_kdev_leg_exact_zero_ties():
    """The K-deviation leg of the fp32 plumbing case: separate K/V caches
    [64 blocks, 16, 2, 64] ~ N(0, 1), a randomly permuted block table, the
    first 512 tokens gathered through it; fresh K = cached K + N(0, 0.05) on
    a random 10% (51) of the tokens, no gaps, ratio 0.15, so topk =
    int(512 * 0.15) = 76 of which 25 fall among exactly-zero scores and go to
    the lowest indices (reference ascend.py:534-543, 757-796)."""
    g = torch.Generator().manual_seed(0)
    k_cache = torch.randn(64, 16, 2, 64, generator=g)
    v_cache = torch.randn(64, 16, 2, 64, generator=g)
    table = torch.randperm(64, generator=g)
    slots = synthetic.block_slots(table, 16, 512)
    kv = KL.gather_paged_kv([k_cache.to(DEV), v_cache.to(DEV)], slots.to(DEV), 16)
    assert kv.shape == (2, 512, 2, 64) and kv.dtype == torch.float32
    cached = kv[0].reshape(512, 128)
    noisy = torch.randperm(512, generator=g)[:51]
    fresh = cached.clone()
    fresh[noisy.to(DEV)] += (0.05 * torch.randn(51, 128, generator=g)).to(DEV)
    gap = torch.zeros(512, dtype=torch.bool, device=DEV)

    scores = S.kdev_scores(fresh, cached)
    want_scores = O.kdev_scores(fresh.cpu().numpy(), cached.cpu().numpy())
    np.testing.assert_allclose(scores.cpu().numpy(), want_scores, rtol=SCORE_RTOL, atol=0)
    assert int((scores == 0).sum()) == 512 - 51          # untouched rows score exactly zero

    sel = S.BlendSelector(CacheBlendConfig.from_extra_config({}), 16)
    got = sel.kv_deviation_select(fresh, cached, torch.arange(512, device=DEV), gap, layer_id=1)
    assert got.dtype == torch.int64
    want = O.select(want_scores, gap.cpu().numpy(), 0.15)
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    # closed form: every noisy token, then the 25 lowest-index zero-score tokens
    rest = np.setdiff1d(np.arange(512), noisy.numpy())[:76 - 51]
    np.testing.assert_array_equal(got.cpu().numpy(), np.union1d(noisy.numpy(), rest))


@pytest.mark.parametrize("n, case", [
    (65536, "one_bin"),        # every key shares the first 12-bit digit: second digit narrows
    (65536, "two_values"),     # two distinct keys: the last digit fixes the k-th key, index ties
    (1_500_000, "normal"),     # 4096-token tiles, 367 blocks
    (3_000_000, "normal"),     # past the 4096-token tiles' capacity: 8192-token tiles
    (5_000_000, "normal"),     # more tiles than fit at once: the multi-launch pipeline
])
def test_select_narrowing_paths_and_sizes(n, case):
    """Selection paths the k-th key's neighbourhood decides: few keys in its
    12-bit bin (candidates finished in LDS), a crowded bin narrowed by the
    next 12 bits, a crowded 24-bit prefix (ties resolved by index), and
    spans larger than one cooperative launch holds."""
    rng = np.random.default_rng(n + len(case))
    if case == "one_bin":
        scores = (1.0 + rng.random(n) / 8.5).astype(np.float32)   # all in [1, 1.125)
    elif case == "two_values":
        scores = np.where(rng.random(n) < 0.5, 2.0, 3.0).astype(np.float32)
    else:
        scores = rng.standard_normal(n).astype(np.float32)
    gap = rng.random(n) < 0.1
    forced = rng.random(n) < 0.02
    for ratio, radius in ((0.15, 16), (0.6, 0)):
        print(f"n={n} case={case} ratio={ratio} radius={radius}", flush=True)
        fc = forced | (O.dilate(gap, radius) if radius else False)
        want = O.select(scores, gap, ratio, fc)
        got = S.select(torch.from_numpy(scores).to(DEV), torch.from_numpy(gap).to(DEV), ratio,
                       torch.from_numpy(forced).to(DEV), radius=radius)
        np.testing.assert_array_equal(got.cpu().numpy(), want)


def _fuzz_scores(rng, n, kind):
    if kind == "normal":
        return rng.standard_normal(n).astype(np.float32)
    if kind == "lognormal":
        return rng.lognormal(0.0, 1.5, n).astype(np.float32)
    if kind == "few_values":  # masses of exact ties
        return rng.choice(np.array([0.0, 0.5, 1.0, 2.0], np.float32), n)
    if kind == "narrow":  # one 12-bit bin, a few 24-bit prefixes
        return (1.0 + rng.integers(0, 64, n) * 2.0 ** -20).astype(np.float32)
    s = rng.standard_normal(n).astype(np.float32)  # "specials": -inf, NaN, -0.0, +0.0
    pick = rng.random(n)
    s[pick < 0.05] = -np.inf
    s[(pick >= 0.05) & (pick < 0.07)] = np.nan
    s[(pick >= 0.07) & (pick < 0.10)] = -0.0
    s[(pick >= 0.10) & (pick < 0.13)] = 0.0
    return s


@pytest.mark.parametrize("seed", range(40))
def test_select_seeded_random_configurations(seed):
    """Seeded random selections against the oracle, bit for bit: sizes across
    the tile and launch-capacity edges, score distributions with ties,
    -inf, NaN and signed zeros, dilation radii on the register path (<= 24)
    and the LDS prefix path, forced masks, ratios near 0 and 1."""
    rng = np.random.default_rng(1000 + seed)
    sizes = [1, 63, 4095, 4096, 4097, 8191, 8193, 65535, 65536, 65537, 131072, 262143]
    n = int(sizes[seed % len(sizes)] if seed < 24 else rng.integers(1, 300_000))
    kind = ["normal", "lognormal", "few_values", "narrow", "specials"][seed % 5]
    scores = _fuzz_scores(rng, n, kind)
    gap = rng.random(n) < rng.uniform(0.0, 0.5)
    forced = (rng.random(n) < rng.uniform(0.0, 0.1)) if seed % 3 else None
    radius = int([0, 1, 16, 24, 25, 300][seed % 6])
    ratio = float([0.001, 0.15, 0.5, 0.99, 1.0, rng.uniform(0.0, 1.0)][seed % 6])
    print(f"seed={seed} n={n} kind={kind} radius={radius} ratio={ratio:.4f} forced={forced is not None}",
          flush=True)
    fc = forced
    if radius:
        fc = O.dilate(gap, radius) | (forced if forced is not None else False)
    want = O.select(scores, gap, ratio, fc)
    got = S.select(torch.from_numpy(scores).to(DEV), torch.from_numpy(gap).to(DEV), ratio,
                   None if forced is None else torch.from_numpy(forced).to(DEV), radius=radius)
    np.testing.assert_array_equal(got.cpu().numpy(), want)
