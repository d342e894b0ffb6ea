"""GPU: the allocation-free K-deviation selection entry point.

cbk_kdev_select_noalloc (static device scratch, no workspace argument) is
checked against cbk_kdev_select (caller workspace) through the C ABI: the
same scores bit for bit, the same index set and count, on two calls in a
row with the second smaller; sizes beyond its maximum are rejected before
anything runs.
"""

import ctypes

import pytest
import torch

from cacheblend_vllm import _native, synthetic

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
MAX_TOKENS = 1048576  # CBK_NOALLOC_SELECT_MAX_TOKENS


def _call(lib, fresh, cached, gap, ratio, radius, workspace=None):
    n, width = fresh.shape
    scores = torch.full((n,), float("nan"), device=DEV)
    out = torch.full((max(n, 1),), -7, dtype=torch.long, device=DEV)
    count = torch.full((1,), -7, dtype=torch.long, device=DEV)
    args = [fresh.data_ptr(), fresh.stride(0), cached.data_ptr(), cached.stride(0), cached.shape[0],
            None, 0, n, width, _native.DTYPE_CODES[fresh.dtype], gap.data_ptr(), None, radius, ratio,
            scores.data_ptr(), out.data_ptr(), count.data_ptr()]
    stream = _native.stream_handle(DEV)
    if workspace is None:
        rc = lib.cbk_kdev_select_noalloc(*args, stream)
    else:
        rc = lib.cbk_kdev_select(*args, workspace.data_ptr(), workspace.numel(), stream)
    _native.check(rc, "kdev select")
    torch.cuda.synchronize()
    k = int(count.item())
    return scores, out[:k].clone(), k


def test_noalloc_select_matches_workspace_entry_point():
    lib = _native.load()
    for n, seed, ratio, radius in ((65536, 0, 0.15, 16), (5000, 1, 0.3, 0)):  # second call smaller
        print(f"noalloc kdev select n={n} seed={seed}", flush=True)
        fresh, cached, gap = synthetic.kdev_inputs(n, 4, 128, torch.bfloat16, DEV, seed=seed)
        gap_u8 = gap.view(torch.uint8)
        workspace = torch.empty(lib.cbk_select_workspace_bytes(n), dtype=torch.uint8, device=DEV)
        want_scores, want_idx, want_k = _call(lib, fresh, cached, gap_u8, ratio, radius, workspace)
        got_scores, got_idx, got_k = _call(lib, fresh, cached, gap_u8, ratio, radius)
        assert torch.equal(got_scores.view(torch.int32), want_scores.view(torch.int32))
        assert got_k == want_k > 0
        assert torch.equal(got_idx, want_idx)
        assert bool((got_idx[1:] > got_idx[:-1]).all())
        assert bool(gap[got_idx].sum() == gap.sum())   # every gap token is selected


def test_noalloc_select_at_its_maximum_size():
    """Exactly the largest accepted span (the static scratch's whole layout in
    use; one head of 8 dims keeps the inputs at 16 MB), then a smaller call
    on the same scratch: both equal the workspace entry point bit for bit."""
    lib = _native.load()
    for n, seed in ((MAX_TOKENS, 5), (4097, 6)):
        print(f"noalloc kdev select n={n} seed={seed}", flush=True)
        fresh, cached, gap = synthetic.kdev_inputs(n, 1, 8, torch.bfloat16, DEV, seed=seed)
        gap_u8 = gap.view(torch.uint8)
        workspace = torch.empty(lib.cbk_select_workspace_bytes(n), dtype=torch.uint8, device=DEV)
        want_scores, want_idx, want_k = _call(lib, fresh, cached, gap_u8, 0.15, 16, workspace)
        got_scores, got_idx, got_k = _call(lib, fresh, cached, gap_u8, 0.15, 16)
        assert torch.equal(got_scores.view(torch.int32), want_scores.view(torch.int32))
        assert got_k == want_k > 0
        assert torch.equal(got_idx, want_idx)
        assert bool(gap[got_idx].sum() == gap.sum())


def test_noalloc_select_rejects_sizes_beyond_its_scratch():
    lib = _native.load()
    tiny = torch.zeros(8, dtype=torch.uint8, device=DEV)
    rc = lib.cbk_kdev_select_noalloc(tiny.data_ptr(), 1, tiny.data_ptr(), 1, 1, None, 0, MAX_TOKENS + 1, 1,
                                     _native.DTYPE_CODES[torch.float32], tiny.data_ptr(), None, 0, 0.15,
                                     tiny.data_ptr(), tiny.data_ptr(), tiny.data_ptr(),
                                     _native.stream_handle(DEV))
    assert rc == -1  # CBK_ERR_INVALID
    assert b"static scratch maximum of 1048576" in lib.cbk_last_error()


def test_noalloc_select_replays_in_a_hip_graph():
    """The caller the entry point is for: HIP graph capture. One capture
    (after an eager warm-up), then replays with the program's own eager work
    in between -- another allocation-free select on other data, which leaves
    its own contents in the shared scratch -- and every replay must equal
    the eager result bit for bit."""
    lib = _native.load()
    n, ratio, radius = 65536, 0.15, 16
    fresh, cached, gap = synthetic.kdev_inputs(n, 4, 128, torch.bfloat16, DEV, seed=3)
    other = synthetic.kdev_inputs(20000, 4, 128, torch.bfloat16, DEV, seed=4)
    gap_u8 = gap.view(torch.uint8)
    want_scores, want_idx, want_k = _call(lib, fresh, cached, gap_u8, ratio, radius)
    scores = torch.full((n,), float("nan"), device=DEV)
    out = torch.full((n,), -7, dtype=torch.long, device=DEV)
    count = torch.full((1,), -7, dtype=torch.long, device=DEV)
    args = [fresh.data_ptr(), fresh.stride(0), cached.data_ptr(), cached.stride(0), cached.shape[0],
            None, 0, n, fresh.shape[1], _native.DTYPE_CODES[fresh.dtype], gap_u8.data_ptr(), None,
            radius, ratio, scores.data_ptr(), out.data_ptr(), count.data_ptr()]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.cbk_kdev_select_noalloc(*args, _native.stream_handle(DEV))
    _native.check(rc, "kdev select (captured)")
    for rep in range(4):
        print(f"graph replay {rep}", flush=True)
        scores.fill_(float("nan"))
        out.fill_(-7)
        count.fill_(-7)
        _, _, k_other = _call(lib, other[0], other[1], other[2].view(torch.uint8), 0.3, 0)
        assert k_other > 0
        graph.replay()
        torch.cuda.synchronize()
        assert int(count.item()) == want_k
        assert torch.equal(scores.view(torch.int32), want_scores.view(torch.int32))
        assert torch.equal(out[:want_k], want_idx)
