"""CPU-side checks: the C ABI library loads and exports what the header
declares, host-side argument validation, and the Python boundary's layout
dispatch and error behaviour. No kernel is launched here."""

import ctypes
import os
import re

import pytest
import torch

from cacheblend_vllm import _native
from cacheblend_vllm.config import CacheBlendConfig
from cacheblend_vllm.kv_layout import gather_paged_kv, kv_planes, scatter_paged_kv
from cacheblend_vllm.types import BlendPlan, BlendSegment, SegmentId

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", f) for f in os.listdir(os.path.join(ROOT, "include"))]


def _declared_symbols():
    names = set()
    for path in HEADERS:
        text = open(path).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(cbk_[a-z0-9_]+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_native.LIB_PATH)
    declared = _declared_symbols()
    assert declared, "no declarations found"
    for name in sorted(declared):
        assert hasattr(lib, name), name
    assert declared == set(_native.EXPORTED_SYMBOLS)


def test_library_host_only_calls():
    lib = _native.load()
    assert lib.cbk_abi_version() == _native.ABI_VERSION
    assert lib.cbk_error_string(-1) == b"invalid argument"
    assert lib.cbk_select_workspace_bytes(65536) >= 65536 * 5
    assert lib.cbk_select_workspace_bytes(65536) % 256 == 0


def test_native_argument_validation_fails_before_any_launch():
    lib = _native.load()
    # NULL descriptor / pointers are rejected on the host
    rc = lib.cbk_paged_gather(None, None, 4, None, None, 16, None, None)
    assert rc == _native.CBK_ERR_INVALID
    assert b"NULL" in lib.cbk_last_error()
    desc = _native.KVDesc(0x1000, 0x2000, 4, 16, 16 * 256, 256, 256)
    rc = lib.cbk_paged_gather(desc, 0x3000, 8, 0x4000, 0x5000, 128, None, None)
    assert rc == _native.CBK_ERR_INVALID  # output token stride smaller than a row
    rc = lib.cbk_select(None, None, None, 10, 5000, 0.15, None, None, None, 0, None)
    assert rc == _native.CBK_ERR_INVALID  # radius above the supported maximum
    rc = lib.cbk_select(0x10, 0x20, None, 100, 0, 0.15, 0x30, 0x40, 0x50, 16, None)
    assert rc == _native.CBK_ERR_WORKSPACE
    rc = lib.cbk_kdev_scores(0x10, 8, 0x20, 8, 10, None, 0, 10, 8, 7, 0x30, None)
    assert rc == _native.CBK_ERR_UNSUPPORTED  # unknown dtype code
    with pytest.raises(ValueError, match="invalid argument|NULL"):
        _native.check(lib.cbk_paged_gather(None, None, 4, None, None, 16, None, None), "gather")


def test_layout_dispatch_matches_reference_rules():
    # reference tests/test_kv_layout.py:27-29
    with pytest.raises(ValueError, match="unsupported"):
        gather_paged_kv(torch.empty(3, 4, 5), torch.tensor([0]), 2)
    with pytest.raises(ValueError, match="requires two tensors"):
        gather_paged_kv([torch.empty(2, 2, 1)] * 3, torch.tensor([0]), 2)
    with pytest.raises(TypeError, match="must contain tensors"):
        gather_paged_kv([torch.empty(2, 2, 1), "x"], torch.tensor([0]), 2)
    with pytest.raises(ValueError, match="K/V as its first dimension"):
        scatter_paged_kv(torch.empty(3, 1, 1), torch.empty(2, 2, 2, 1), torch.tensor([0]), 2)
    first = torch.empty(2, 5, 4, 3)
    k, v = kv_planes(first)
    assert k.shape == (5, 4, 3) and v.data_ptr() > k.data_ptr()
    block = torch.empty(5, 2, 4, 3)
    k, v = kv_planes(block)
    assert k.stride(0) == 2 * 4 * 3


def test_cpu_tensors_have_no_fallback():
    paged = torch.zeros(2, 3, 2, 2)
    with pytest.raises(RuntimeError, match="ROCm device tensor"):
        gather_paged_kv(paged, torch.tensor([0, 3, 4]), 2)
    with pytest.raises(RuntimeError, match="ROCm device tensor"):
        scatter_paged_kv(torch.zeros(2, 3, 2), paged, torch.tensor([0, 3, 4]), 2)


def test_sparse_q_query_rows_match_nonzero():
    # the query-row compaction sized from the gap count, without a host read
    # of its own, against torch.nonzero on the masks of reference
    # ascend.py:652-671 (gaps; no gaps with a tail shorter, longer, and 0)
    from cacheblend_vllm.selection import sparse_q_masks, sparse_q_query_rows

    g = torch.Generator().manual_seed(0)
    cases = [(torch.rand(257, generator=g) < 0.2, 16), (torch.zeros(40, dtype=torch.bool), 7),
             (torch.zeros(5, dtype=torch.bool), 9), (torch.zeros(6, dtype=torch.bool), 0),
             (torch.ones(6, dtype=torch.bool), 3)]
    for gap, tail in cases:
        count = int(gap.sum())
        query_mask, _, has_gap = sparse_q_masks(gap, tail, 0, gap_count=count)
        assert has_gap == bool(gap.any())
        rows = sparse_q_query_rows(query_mask, has_gap, count, tail)
        assert torch.equal(rows, torch.nonzero(query_mask).flatten())


def test_config_matches_reference_rules():
    # reference tests/test_config_registry.py behaviour: unknown fields fail
    with pytest.raises(ValueError, match="Unknown CacheBlend config fields"):
        CacheBlendConfig.from_extra_config({"bogus": 1})
    cfg = CacheBlendConfig.from_extra_config({"check_layers": 2, "recompute_ratios": 0.2})
    assert cfg.check_layers == (2,) and cfg.recompute_ratios == (0.2,)
    with pytest.raises(ValueError, match="exactly one check layer"):
        CacheBlendConfig.from_extra_config({"selection_strategy": "sparse_q", "check_layers": [1, 2]})
    with pytest.raises(ValueError, match="tail_query_tokens > 0"):
        CacheBlendConfig.from_extra_config({"selection_strategy": "sparse_q", "tail_query_tokens": 0})
    cfg = CacheBlendConfig.from_extra_config({"check_layers": [1, 5], "recompute_ratios": [0.1, 0.3]})
    assert cfg.ratio_for(5) == 0.3 and cfg.ratio_for(1) == 0.1 and cfg.ratio_for(None) == 0.1


def test_config_fields_are_the_reference_fields_and_staging_depth_is_an_env_knob(monkeypatch):
    """The field table is reference config.py:10-35 exactly, so a config that
    names the loader's ring depth is rejected by both; the depth comes from
    CACHEBLEND_LOAD_STAGING_LAYERS instead."""
    from dataclasses import fields

    from cacheblend_vllm.config import LOAD_STAGING_LAYERS_ENV, load_staging_layers

    assert [f.name for f in fields(CacheBlendConfig)] == [
        "chunk_size", "local_cpu_gb", "min_retrieve_tokens", "min_hit_ratio", "min_saved_tokens",
        "max_apc_prefix_to_hit_ratio", "check_layers", "recompute_ratios", "selection_strategy",
        "query_score_chunk_size", "overflow_blocks", "tail_query_tokens", "save_decode_cache",
        "tp_global_selection", "event_pipeline", "fused_segment_copy", "cache_attention_mask",
        "lookup_timeout_ms", "store_workers", "max_inflight_store_batches", "strict_version_check",
        "ipc_root", "model_scope"]
    with pytest.raises(ValueError, match="Unknown CacheBlend config fields"):
        CacheBlendConfig.from_extra_config({"load_staging_layers": 3})
    monkeypatch.delenv(LOAD_STAGING_LAYERS_ENV, raising=False)
    assert load_staging_layers() == 4
    monkeypatch.setenv(LOAD_STAGING_LAYERS_ENV, "7")
    assert load_staging_layers() == 7
    for bad in ("1", "x"):
        monkeypatch.setenv(LOAD_STAGING_LAYERS_ENV, bad)
        with pytest.raises(ValueError, match=LOAD_STAGING_LAYERS_ENV):
            load_staging_layers()


def test_plan_invariants_and_gap_runs():
    sid = lambda start, n: SegmentId("m", start, start, n)  # noqa: E731
    plan = BlendPlan(2, 20, 6, (BlendSegment(sid(0, 4), 4), BlendSegment(sid(8, 2), 12)))
    assert plan.gap_tokens == 12
    assert plan.gap_runs() == [(2, 4), (8, 12), (14, 20)]
    with pytest.raises(ValueError, match="overlap"):
        BlendPlan(0, 20, 8, (BlendSegment(sid(0, 4), 2), BlendSegment(sid(8, 4), 4)))
    with pytest.raises(ValueError, match="after the APC prefix"):
        BlendPlan(4, 20, 4, (BlendSegment(sid(0, 4), 2),))
    with pytest.raises(ValueError, match="hit_tokens"):
        BlendPlan(0, 20, 5, (BlendSegment(sid(0, 4), 2),))
    assert BlendPlan.from_dict(plan.to_dict()) == plan


def test_cos_sin_table_cache_tracks_object_and_version():
    from types import SimpleNamespace

    from cacheblend_vllm.rope import cos_sin_table

    a = SimpleNamespace(cos_sin_cache=torch.ones(8, 4))
    t1 = cos_sin_table(a, torch.bfloat16, torch.device("cpu"))
    assert t1.dtype == torch.bfloat16 and cos_sin_table(a, torch.bfloat16, torch.device("cpu")) is t1
    a.cos_sin_cache.mul_(2)  # in-place update: version bump, table rebuilt
    assert float(cos_sin_table(a, torch.bfloat16, torch.device("cpu"))[0, 0]) == 2.0
    for _ in range(8):  # freed caches whose id or address is reused never hit a stale table
        b = SimpleNamespace(cos_sin_cache=torch.full((8, 4), 3.0))
        assert float(cos_sin_table(b, torch.bfloat16, torch.device("cpu"))[0, 0]) == 3.0
        del b
    same = torch.ones(8, 4, dtype=torch.bfloat16)
    assert cos_sin_table(SimpleNamespace(cos_sin_cache=same), torch.bfloat16, torch.device("cpu")) is same


def test_layer_chunk_addresses_requires_pins_and_addressable_chunks():
    from cacheblend_vllm.host_store import PinnedChunkStore
    from cacheblend_vllm.types import BlendSegment

    store = PinnedChunkStore(4, 1 << 20)
    sid = store.begin_put("m", 0, [1, 2, 3, 4], num_layers=1)
    store.put_layer_host(sid, 0, torch.zeros(2, 4, 2, 8))  # pageable: not kernel-addressable
    seg = BlendSegment(sid, 0)
    with pytest.raises(RuntimeError, match="not pinned"):
        store.layer_chunk_addresses("r", [seg], 0)
    store.pin("r", [seg])
    assert store.layer_chunk_addresses("r", [seg], 0) is None
    assert store.get_layer("r", seg, 0).shape == (2, 4, 2, 8)
    store.release("r")
    with pytest.raises(RuntimeError, match="not pinned"):
        store.get_layer("r", seg, 0)


def _slot_layout_runs(n, plane, slot_pitch, base=1 << 32):
    """The loader's hit run table for n full chunks whose [2, chunk, H, D]
    slots start slot_pitch bytes apart: K planes, then V planes."""
    import numpy as np

    k = base + np.arange(n, dtype=np.uint64) * np.uint64(slot_pitch)
    dst = np.arange(2 * n, dtype=np.uint64) * np.uint64(plane)
    return dst, np.concatenate((k, k + np.uint64(plane))), np.full(2 * n, plane, dtype=np.uint64)


def test_memcpy_runs_commands_known_answers():
    """How many DMA commands cbk_memcpy_runs folds a run table into (host
    arithmetic, no GPU call): runs adjacent on both sides make one copy,
    equal runs at constant ascending pitches >= their size one 2D copy."""
    import numpy as np

    from cacheblend_vllm import _native

    u = lambda *v: np.array(v, dtype=np.uint64)  # noqa: E731
    count = _native.memcpy_commands
    assert count(u(), u(), u()) == 0
    assert count(u(64), u(128), u(0)) == 0  # zero-byte runs are skipped
    assert count(u(64), u(128), u(32)) == 1
    # adjacent on both sides, sizes differ: one copy
    assert count(u(0, 10, 40, 41), u(100, 110, 140, 141), u(10, 30, 1, 7)) == 1
    # adjacent in dst only: not a chain, and unequal sizes: one copy each
    assert count(u(0, 10), u(100, 200), u(10, 30)) == 2
    # the store's layout: consecutive slots (pitch 2 planes) -> one 2D copy per plane
    for n in (1, 2, 5, 109):
        assert count(*_slot_layout_runs(n, 4096, 8192)) == (1 if n == 1 else 2)
        assert count(*_slot_layout_runs(n, 4096, 48 * 8192)) == (1 if n == 1 else 2)
    # slots back to back with the K and V planes of each slot contiguous in the
    # destination too ([2, T] host views of one tensor): one copy in all
    k = u(*range(0, 8 * 1000, 1000))
    assert count(np.concatenate((k, k + 8000)), np.concatenate((k, k + 8000)) + 7, np.full(16, 1000, np.uint64)) == 1
    # a pitch below the size (rows would overlap) or a backward step never folds
    assert count(u(0, 100, 200), u(0, 50, 100), u(80, 80, 80)) == 3
    assert count(u(200, 100, 0), u(0, 100, 200), u(80, 80, 80)) == 3
    # pitches beyond 2^31 are issued row by row
    far = np.uint64(1 << 32)
    assert count(u(0, 1 << 32, 2 << 32), u(0, 100, 200), u(80, 80, 80)) == 3
    assert count(u(0, 100, 200), np.array([0, far, 2 * far], dtype=np.uint64), u(80, 80, 80)) == 3
    # a group ends where the size or a pitch changes, or at a zero-byte run
    assert count(u(0, 100, 200, 300, 400), u(0, 200, 400, 600, 900), u(50, 50, 50, 50, 50)) == 2
    assert count(u(0, 100, 200, 300), u(0, 200, 400, 600), u(50, 50, 60, 50)) == 3
    assert count(u(0, 100, 200, 300, 400), u(0, 200, 400, 600, 800), u(50, 50, 0, 50, 50)) == 2
    with pytest.raises(ValueError, match="one length"):
        count(u(0, 1), u(0), u(8))
