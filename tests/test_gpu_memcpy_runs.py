"""cbk_memcpy_runs on the GPU: run tables that fold into one copy, into 2D
copies (the slab's chunk-slot layouts) or stay one copy per run, in every
direction between pinned host memory (torch's and the slab's) and HBM.
Bit-exact: every destination byte equals a byte-by-byte copy made with
numpy, and bytes outside the runs keep their fill."""

import numpy as np
import pytest
import torch

from cacheblend_vllm import _native
from cacheblend_vllm.host_store import PinnedChunkSlab

pytestmark = pytest.mark.gpu

HOST_BYTES = 8 << 20
DEV_BYTES = 8 << 20


def _tables(kind, rng):
    """(dst offsets, src offsets, sizes) within [0, 8 MiB); dst runs disjoint."""
    if kind in ("slots", "slots_strided", "slots_odd"):
        n = int(rng.integers(2, 20))
        plane = 1000 if kind == "slots_odd" else 16384
        pitch = 2 * plane * (5 if kind == "slots_strided" else 1)
        k = np.arange(n) * pitch + 64
        return (np.arange(2 * n) * plane, np.concatenate((k, k + plane)), np.full(2 * n, plane))
    if kind == "permuted":  # slots in random order: mostly one copy per run
        n, plane = 24, 8192
        k = rng.permutation(n) * 2 * plane
        return (np.arange(2 * n) * plane, np.concatenate((k, k + plane)), np.full(2 * n, plane))
    if kind == "chain":  # adjacent on both sides, ragged sizes
        sizes = rng.integers(1, 40000, size=30)
        off = np.concatenate(([0], np.cumsum(sizes)[:-1]))
        return off + 4096, off + 123, sizes
    # mixed: pitched groups, ragged singles and zero-byte runs in one table
    dst, src, nb, d, s = [], [], [], 0, 0
    for _ in range(40):
        r = rng.random()
        if r < 0.4:
            w, rows = int(rng.integers(1, 5000)), int(rng.integers(2, 6))
            dp, sp = w + int(rng.integers(0, 300)), w + int(rng.integers(0, 9000))
            for i in range(rows):
                dst.append(d + i * dp), src.append(s + i * sp), nb.append(w)
            d += rows * dp
            s += rows * sp
        elif r < 0.5:
            dst.append(d), src.append(s), nb.append(0)
        else:
            w = int(rng.integers(1, 20000))
            dst.append(d), src.append(s), nb.append(w)
            d += w + int(rng.integers(0, 2)) * 512
            s += w + int(rng.integers(0, 2)) * 700
    return np.array(dst), np.array(src), np.array(nb)


def _check(kind, direction, seed, host_slab=None):
    rng = np.random.default_rng(seed)
    dst_off, src_off, nbytes = (np.asarray(a, dtype=np.int64) for a in _tables(kind, rng))
    assert (nbytes >= 0).all()
    live = nbytes > 0
    src_len = HOST_BYTES if direction in ("h2d", "h2h") else DEV_BYTES
    dst_len = DEV_BYTES if direction in ("h2d", "d2d") else HOST_BYTES
    assert (src_off[live] + nbytes[live]).max() <= src_len and (dst_off[live] + nbytes[live]).max() <= dst_len
    order = np.argsort(dst_off[live])  # destination runs must not overlap
    ends = (dst_off[live] + nbytes[live])[order]
    assert (dst_off[live][order][1:] >= ends[:-1]).all()

    gen = torch.Generator().manual_seed(seed)
    src_bytes = torch.randint(0, 256, (src_len,), dtype=torch.uint8, generator=gen)
    fill = torch.full((dst_len,), 0xA5, dtype=torch.uint8)
    if direction == "h2d":
        src_t = host_slab if host_slab is not None else torch.empty(src_len, dtype=torch.uint8, pin_memory=True)
        src_t.copy_(src_bytes)
        dst_t = fill.cuda()
    elif direction == "d2h":
        src_t = src_bytes.cuda()
        dst_t = host_slab if host_slab is not None else torch.empty(dst_len, dtype=torch.uint8, pin_memory=True)
        dst_t.copy_(fill)
    else:
        src_t, dst_t = src_bytes.cuda(), fill.cuda()
    torch.cuda.synchronize()
    print(f"memcpy_runs case kind={kind} direction={direction} seed={seed} runs={len(nbytes)} "
          f"commands={_native.memcpy_commands(dst_off, src_off, nbytes)}", flush=True)
    _native.memcpy_runs(dst_off.astype(np.uint64) + np.uint64(dst_t.data_ptr()),
                        src_off.astype(np.uint64) + np.uint64(src_t.data_ptr()),
                        nbytes, _native.stream_handle(torch.device("cuda")), "test runs")
    torch.cuda.synchronize()
    want = fill.numpy().copy()
    src_np = src_bytes.numpy()
    for d, s, n in zip(dst_off.tolist(), src_off.tolist(), nbytes.tolist()):
        want[d:d + n] = src_np[s:s + n]
    got = dst_t.cpu().numpy()
    assert np.array_equal(got, want), (kind, direction, seed)


@pytest.mark.parametrize("kind", ["slots", "slots_strided", "slots_odd", "permuted", "chain", "mixed"])
@pytest.mark.parametrize("direction", ["h2d", "d2h", "d2d"])
def test_memcpy_runs_bit_exact(kind, direction):
    for seed in range(3):
        _check(kind, direction, seed)


def test_memcpy_runs_folds_store_layout_into_two_commands():
    dst, src, nb = _tables("slots", np.random.default_rng(0))
    assert _native.memcpy_commands(dst, src, nb) == 2


@pytest.mark.parametrize("direction", ["h2d", "d2h"])
def test_memcpy_runs_on_slab_memory(direction):
    """The slab's arenas are fine-grained coherent pinned memory: the same
    tables, read from or written to a slab slot."""
    slab = PinnedChunkSlab((HOST_BYTES,), torch.uint8, chunks_per_arena=1)
    try:
        (slot,) = slab.alloc_run(1)
        for kind in ("slots", "mixed"):
            _check(kind, direction, 11, host_slab=slot)
        slab.free(slot)
    finally:
        slab.close()


@pytest.mark.parametrize("direction", ["h2d", "d2h"])
def test_memcpy_runs_group_across_two_allocations(direction):
    """Two equal runs whose host sides are two separate pinned allocations
    (slab arenas of one slot each) at a pitch that merely lines up, their
    device sides adjacent: the planner folds them into one 2D command, which
    the runtime rejects for reaching across allocations; the runs then go out
    one by one, and every byte arrives."""
    w = 4096
    slab = PinnedChunkSlab((w,), torch.uint8, chunks_per_arena=1)
    try:
        (first,) = slab.alloc_run(1)
        (second,) = slab.alloc_run(1)
        lo, hi = sorted((first, second), key=lambda t: t.data_ptr())
        if not w <= hi.data_ptr() - lo.data_ptr() <= (1 << 31):
            pytest.skip("the two arenas are not at a foldable pitch on this box")
        dev = torch.empty(2 * w, dtype=torch.uint8, device="cuda")
        rng = np.random.default_rng(3)
        host_addr = np.array([lo.data_ptr(), hi.data_ptr()], dtype=np.uint64)
        dev_addr = np.array([dev.data_ptr(), dev.data_ptr() + w], dtype=np.uint64)
        sizes = np.full(2, w, dtype=np.uint64)
        if direction == "h2d":
            for t in (lo, hi):
                t.copy_(torch.from_numpy(rng.integers(0, 256, w, dtype=np.uint8)))
            dst, src = dev_addr, host_addr
        else:
            dev.copy_(torch.from_numpy(rng.integers(0, 256, 2 * w, dtype=np.uint8)))
            dst, src = host_addr, dev_addr
        assert _native.memcpy_commands(dst, src, sizes) == 1
        stream = torch.cuda.current_stream()
        _native.memcpy_runs(dst, src, sizes, stream.cuda_stream, "runs across two allocations")
        torch.cuda.synchronize()
        assert torch.equal(dev.cpu(), torch.cat((lo, hi)))
        slab.free(first)
        slab.free(second)
    finally:
        slab.close()


def test_memcpy_runs_rejects_bad_tables():
    with pytest.raises(ValueError, match="NULL"):
        _native.memcpy_runs(np.array([0], np.uint64), np.array([64], np.uint64), np.array([8], np.uint64),
                            _native.stream_handle(torch.device("cuda")), "null dst")
    with pytest.raises(ValueError, match="one length"):
        _native.memcpy_runs(np.zeros(2, np.uint64), np.zeros(1, np.uint64), np.zeros(2, np.uint64), 0, "bad")
