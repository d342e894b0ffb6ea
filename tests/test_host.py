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


def test_loader_address_runs_join_adjacent_segments():
    """The loader's run search over host chunk addresses: segments join a
    run exactly when both their K and V planes follow the previous
    segment's (checked against a direct scan on random layouts)."""
    import types

    import numpy as np

    from cacheblend_vllm.loader import PagedBlendLoader

    rng = np.random.default_rng(4)
    row = 1024
    for _ in range(200):
        lengths = rng.integers(1, 5, size=int(rng.integers(1, 12))) * 16
        k = v = None
        flat = []
        for i, n in enumerate(lengths):
            if i and rng.random() < 0.6:  # continue both planes
                k, v = k + prev * row, v + prev * row
            elif i and rng.random() < 0.5:  # only K continues
                k, v = k + prev * row, v + 4096 * row
            else:
                k, v = int(rng.integers(1, 1 << 30)) * 64, int(rng.integers(1, 1 << 30)) * 64
            flat += [k, v]
            prev = int(n)
        fake = types.SimpleNamespace(_seg_plane_bytes=lengths.astype(np.int64) * row,
                                     _seg_row_off=np.concatenate(([0], np.cumsum(lengths))))
        got = PagedBlendLoader._address_runs(fake, flat, row)
        want, off = [], 0
        for i, n in enumerate(lengths.tolist()):
            kk, vv = flat[2 * i], flat[2 * i + 1]
            if want and kk == want[-1][2] + want[-1][1] * row and vv == want[-1][3] + want[-1][1] * row:
                want[-1][1] += n
            else:
                want.append([off, n, kk, vv])
            off += n
        assert got == [tuple(w) for w in want]
