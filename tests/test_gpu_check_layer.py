"""GPU parity: row write-back (block-size-1, K-only descriptors) and the check
layer's selection block in its three strategies, against the oracle."""

import json

import numpy as np
import pytest
import torch

import oracle as O
from cacheblend_vllm import synthetic
from cacheblend_vllm.config import CacheBlendConfig
from cacheblend_vllm.kv_layout import write_back_kv, write_rows
from cacheblend_vllm.selection import BlendSelector
from cacheblend_vllm.trace import PipelineTracer

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _bits(t):
    t = t.detach().cpu()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_write_rows_matches_row_assignment(dtype):
    g = torch.Generator().manual_seed(1)
    dst = torch.randn(3000, 4, 128, generator=g).to(dtype).to(DEV)
    idx = torch.randperm(3000, generator=g)[:777]
    src = torch.randn(777, 512, generator=g).to(dtype).to(DEV)
    want = _bits(dst).copy()
    want[idx.numpy()] = _bits(src).reshape(777, 4, 128)
    write_rows(dst, idx, src)  # host indices: range-checked, uploaded
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(dst), want)
    with pytest.raises(IndexError):
        write_rows(dst, torch.tensor([0, 3000]), src[:2])


def test_write_back_kv_from_strided_qkv_views():
    g = torch.Generator().manual_seed(2)
    A, T, H, D = 4096, 1000, 4, 128
    old_kv = torch.randn(2, A, H, D, generator=g).to(torch.bfloat16).to(DEV)
    qkv = torch.randn(T, 32 * D + 2 * H * D, generator=g).to(torch.bfloat16).to(DEV)
    q, k, v = qkv.split([32 * D, H * D, H * D], dim=-1)  # row stride 5120 elements
    idx = (torch.arange(T) * 3 + 17).to(DEV)  # device indices, not read back
    want = _bits(old_kv).copy()
    want[0, idx.cpu().numpy()] = _bits(k).reshape(T, H, D)
    want[1, idx.cpu().numpy()] = _bits(v).reshape(T, H, D)
    write_back_kv(old_kv, idx, k, v)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(old_kv), want)


def _check_inputs(seed, n_active=1500, prefix=700, hq=16, hkv=4, d=128):
    g = torch.Generator().manual_seed(seed)
    nk = prefix + n_active
    flat_old_k = (torch.randn(nk, hkv * d, generator=g) / d ** 0.5).to(torch.bfloat16)
    noise = 0.02 * torch.exp(torch.randn(n_active, 1, generator=g)) * torch.randn(n_active, hkv * d, generator=g)
    k = (flat_old_k[prefix:].float() + noise / d ** 0.5).to(torch.bfloat16)
    q = (torch.randn(n_active, hq * d, generator=g) / d ** 0.5).to(torch.bfloat16)
    gap = torch.from_numpy(synthetic.gap_layout(n_active, seed, hit_chunk=64, max_hit_chunks=5, max_gap=63))
    absolute = torch.arange(prefix, nk)
    return q, k, flat_old_k, absolute, gap


def test_check_layer_kv_deviation_matches_oracle():
    q, k, old, absolute, gap = _check_inputs(5)
    sel = BlendSelector(CacheBlendConfig.from_extra_config({"check_layers": [1]}), 16)
    res = sel.check_layer(q.to(DEV), k.to(DEV), old.to(DEV), absolute.to(DEV), gap.to(DEV), 1, 128 ** -0.5,
                          16, 4, 128, strategy="kv_deviation")
    assert res.sparse_q_selected is None
    scores = O.kdev_scores(k.float().numpy(), old.float().numpy()[absolute.numpy()])
    want = O.select(scores, gap.numpy(), 0.15)
    np.testing.assert_array_equal(res.deviation_selected.cpu().numpy(), want)


@pytest.mark.parametrize("strategy", ["sparse_q", "compare"])
def test_check_layer_sparse_q_overwrites_and_selects(strategy, tmp_path, monkeypatch):
    q, k, old, absolute, gap = _check_inputs(7)
    old_dev = old.to(DEV)
    monkeypatch.setenv("CACHEBLEND_TRACE_DIR", str(tmp_path))
    tracer = PipelineTracer("worker")
    sel = BlendSelector(CacheBlendConfig.from_extra_config(
        {"check_layers": [1], "selection_strategy": "sparse_q"}), 16)
    res = sel.check_layer(q.to(DEV), k.to(DEV), old_dev, absolute.to(DEV), gap.to(DEV), 1, 128 ** -0.5,
                          16, 4, 128, strategy=strategy, tracer=tracer, request_id="r")
    tracer.close()
    score_keys = old.clone()
    score_keys[absolute] = k
    # sparse_q aliases flat_old_k (written in place); compare scores a copy
    np.testing.assert_array_equal(_bits(old_dev), _bits(score_keys if strategy == "sparse_q" else old))
    want_scores, want_forced, want_stats = O.sparse_q_scores(
        q.float().numpy().reshape(-1, 16, 128), score_keys.float().numpy().reshape(-1, 4, 128),
        absolute.numpy(), gap.numpy(), 128 ** -0.5, block_size=16, overflow_blocks=1,
        tail_query_tokens=64, round_logits_bf16=True)
    for key in ("sparse_query_tokens", "tail_fallback", "gap_tokens"):
        assert res.sparse_q_stats[key] == want_stats[key]
    got = set(res.sparse_q_selected.cpu().tolist())
    want = set(O.select(want_scores, gap.numpy(), 0.15, want_forced).tolist())
    base = gap.numpy() | want_forced
    kb = O.select_budget(len(gap), int(gap.sum()), int(base.sum()), 0.15)
    kth = np.sort(want_scores[~base])[::-1][kb - 1]
    band = np.abs(want_scores - kth) <= 1e-2 * abs(kth)
    disagree = np.array(sorted(got ^ want), dtype=np.int64)
    print(f"{strategy}: selected {len(got)} disagreements {disagree.size} band {int(band.sum())}", flush=True)
    assert np.all(band[disagree])
    if strategy == "compare":
        dev_want = O.select(O.kdev_scores(k.float().numpy(), old.float().numpy()[absolute.numpy()]),
                            gap.numpy(), 0.15)
        np.testing.assert_array_equal(res.deviation_selected.cpu().numpy(), dev_want)
    events = [json.loads(line) for f in tmp_path.iterdir() for line in f.read_text().splitlines()]
    names = [e["event"] for e in events]
    if strategy == "compare":
        assert "selection_compared" in names and "selection_finished" not in names
    else:
        # reference ascend.py:627-635: the Sparse-Q set and its stats
        (done,) = [e for e in events if e["event"] == "selection_finished"]
        assert done["request_id"] == "r" and done["layer_id"] == 1 and done["strategy"] == "sparse_q"
        assert done["selected_tokens"] == len(got)
        for key in ("active_tokens", "gap_tokens", "cached_tokens", "sparse_query_tokens",
                    "tail_fallback", "overflow_blocks"):
            assert done[key] == res.sparse_q_stats[key], key


@pytest.mark.parametrize("seed", range(12))
def test_check_layer_random_configurations(seed):
    """Seeded random check layers: 1-8 query heads per KV head over 1-4 KV
    heads, head_dim 64 or 128, 1-2000 active tokens at sorted random
    positions of a larger context, gap layouts (none: the tail fallback),
    ratios 0.05-0.6, block sizes 8 / 16 / 32, overflow radii of 0-2 blocks,
    every strategy. K-deviation sets equal the oracle's; Sparse-Q sets
    agree outside the epsilon band of the k-th score; the Sparse-Q strategy
    writes the fresh K rows into the cache (compare leaves it alone)."""
    rng = np.random.default_rng(3000 + seed)
    hkv = int(rng.choice([1, 2, 4]))
    hq = hkv * int(rng.choice([1, 2, 4, 8]))
    d = int(rng.choice([64, 128]))
    n = int(rng.integers(1, 2001))
    nk = n + int(rng.integers(0, 1500))
    absolute = np.sort(rng.choice(nk, n, replace=False))
    if rng.random() < 0.25:
        gap = np.zeros(n, dtype=bool)
    else:
        gap = synthetic.gap_layout(n, seed, hit_chunk=int(rng.choice([16, 64])), max_hit_chunks=4, max_gap=40)
    strategy = ["kv_deviation", "sparse_q", "compare"][int(rng.integers(3))]
    ratio = float(rng.uniform(0.05, 0.6))
    bs = int(rng.choice([8, 16, 32]))
    overflow = int(rng.integers(0, 3))
    tail = int(rng.integers(1, 100))
    scale = d ** -0.5
    print(f"seed={seed} hq={hq} hkv={hkv} d={d} n={n} nk={nk} gaps={int(gap.sum())} {strategy} "
          f"ratio={ratio:.3f} bs={bs} overflow={overflow} tail={tail}", flush=True)
    g = torch.Generator().manual_seed(seed)
    old = (torch.randn(nk, hkv * d, generator=g) / d ** 0.5).to(torch.bfloat16)
    abs_t = torch.from_numpy(absolute)
    noise = 0.02 * torch.exp(torch.randn(n, 1, generator=g)) * torch.randn(n, hkv * d, generator=g)
    k = (old[abs_t].float() + noise / d ** 0.5).to(torch.bfloat16)
    q = (torch.randn(n, hq * d, generator=g) / d ** 0.5).to(torch.bfloat16)
    config = CacheBlendConfig.from_extra_config({
        "check_layers": [1], "recompute_ratios": [ratio], "overflow_blocks": overflow,
        "tail_query_tokens": tail,
        "selection_strategy": "kv_deviation" if strategy == "kv_deviation" else "sparse_q"})
    old_dev = old.to(DEV)
    res = BlendSelector(config, bs).check_layer(
        q.to(DEV), k.to(DEV), old_dev, abs_t.to(DEV), torch.from_numpy(gap).to(DEV), 1, scale, hq, hkv, d,
        strategy=strategy)
    if strategy in ("kv_deviation", "compare"):
        want = O.select(O.kdev_scores(k.float().numpy(), old.float().numpy()[absolute]), gap, ratio)
        np.testing.assert_array_equal(res.deviation_selected.cpu().numpy(), want)
    if strategy == "kv_deviation":
        return
    score_keys = old.clone()
    score_keys[abs_t] = k
    np.testing.assert_array_equal(_bits(old_dev), _bits(score_keys if strategy == "sparse_q" else old))
    scores, forced, stats = O.sparse_q_scores(
        q.float().numpy().reshape(n, hq, d), score_keys.float().numpy().reshape(nk, hkv, d), absolute, gap,
        scale, block_size=bs, overflow_blocks=overflow, tail_query_tokens=tail, round_logits_bf16=True)
    for key in ("sparse_query_tokens", "tail_fallback", "gap_tokens"):
        assert res.sparse_q_stats[key] == stats[key]
    got = set(res.sparse_q_selected.cpu().tolist())
    want = set(O.select(scores, gap, ratio, forced).tolist())
    base = gap | forced
    disagree = np.array(sorted(got ^ want), dtype=np.int64)
    if disagree.size:
        kb = O.select_budget(n, int(gap.sum()), int(base.sum()), ratio)
        kth = np.sort(scores[~base])[::-1][kb - 1]
        band = np.abs(scores - kth) <= 1e-2 * abs(kth)
        assert np.all(band[disagree]), disagree[:10]


def test_k_only_gather_through_row_table():
    import ctypes

    from cacheblend_vllm import _native

    g = torch.Generator().manual_seed(3)
    table = torch.randn(500, 256, generator=g).to(DEV)
    idx = torch.randperm(500, generator=g)[:123].to(DEV)
    out = torch.empty(123, 256, device=DEV)
    desc = _native.KVDesc(table.data_ptr(), None, 500, 1, 1024, 1024, 1024)
    rc = _native.load().cbk_paged_gather(ctypes.byref(desc), idx.data_ptr(), 123, out.data_ptr(), None, 1024,
                                         None, _native.stream_handle(DEV))
    _native.check(rc, "gather K only")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), table.cpu().numpy()[idx.cpu().numpy()])
    # a V plane on one side only is an error, not a silent K-only copy
    rc = _native.load().cbk_paged_gather(ctypes.byref(desc), idx.data_ptr(), 123, out.data_ptr(),
                                         out.data_ptr(), 1024, None, _native.stream_handle(DEV))
    assert rc != 0
