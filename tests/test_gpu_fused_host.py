"""GPU: the fused host paths -- pinned chunk slab, gather straight into host
chunks (store) and assembly reading host chunks (load) -- bit-exact."""

import numpy as np
import pytest
import torch

import oracle as O
from cacheblend_vllm import _native, synthetic
from cacheblend_vllm.config import CacheBlendConfig
from cacheblend_vllm.host_store import PinnedChunkSlab, PinnedChunkStore
from cacheblend_vllm.kv_layout import scatter_chunks
from cacheblend_vllm.loader import PagedBlendLoader
from cacheblend_vllm.store_path import RequestMetadata, StoreStreamWriter
from cacheblend_vllm.types import BlendPlan, BlendSegment

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def test_slab_slots_are_pinned_recycled_and_bounded():
    slab = PinnedChunkSlab((2, 256, 4, 128), torch.bfloat16, chunks_per_arena=4, max_bytes=8 * 512 * 1024)
    slots = [slab.alloc() for _ in range(6)]
    assert all(_native.host_accessible(s) for s in slots)
    assert _native.host_accessible(torch.ones(64).pin_memory())
    assert not _native.host_accessible(torch.ones(64))
    assert all(s.data_ptr() % 256 == 0 for s in slots)
    assert len({s.data_ptr() for s in slots}) == 6
    st = slab.stats()
    assert st["arenas"] == 2 and st["live"] == 6 and st["free"] == 2
    ev = torch.cuda.Event()
    ev.record()
    freed = slots.pop()
    slab.free(freed, ev)
    torch.cuda.synchronize()
    again = slab.alloc()  # the fenced slot comes back once its event completed
    assert again.data_ptr() == freed.data_ptr()
    slots.append(again)
    slots += [slab.alloc(), slab.alloc()]
    with pytest.raises(RuntimeError, match="exceed"):
        slab.alloc()  # a third arena would pass max_bytes
    for s in slots:
        slab.free(s)
    with pytest.raises(ValueError, match="not a live slot"):
        slab.free(slots[0])
    del slots, again, freed
    slab.close()


def test_slab_runs_are_consecutive_and_fall_back_when_fragmented():
    slab = PinnedChunkSlab((2, 16, 2, 64), torch.bfloat16, chunks_per_arena=8)
    stride = slab.chunk_bytes
    run = slab.alloc_run(5)
    assert [t.data_ptr() - run[0].data_ptr() for t in run] == [i * stride for i in range(5)]
    other = slab.alloc_run(3)  # fills the arena
    assert other[0].data_ptr() == run[-1].data_ptr() + stride
    for t in run[1::2]:
        slab.free(t)  # arena 0 now has free slots 1 and 3 only
    run2 = slab.alloc_run(4)  # no run of 4 there: a fresh arena holds it
    assert slab.stats()["arenas"] == 2
    assert [t.data_ptr() - run2[0].data_ptr() for t in run2] == [i * stride for i in range(4)]
    single = slab.alloc_run(2)  # the two free slots of arena 0 are not adjacent: first run in arena 1
    assert single[1].data_ptr() == single[0].data_ptr() + stride
    live = run[0::2] + other + run2 + single
    assert slab.stats()["live"] == len(live)
    big = slab.alloc_run(10)  # longer than an arena: scattered lowest slots, new arenas as needed
    assert len({t.data_ptr() for t in big}) == 10
    for t in live + big:
        slab.free(t)
    st = slab.stats()
    assert st["live"] == 0 and st["free"] == 8 * st["arenas"]
    slab.close()


def _raw(t):
    t = t.detach().cpu()
    return t.view(torch.int32).numpy() if t.dtype == torch.float32 else t.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("seed", range(12))
def test_store_random_requests_bit_exact(seed):
    """Seeded random stores over two layers: block sizes 8-32, head shapes
    (80-dim rows included), bf16 / f16 / float32, chunk sizes 16-128, both
    page layouts, every transfer mode (slab by DMA, slab written by the
    gather, the reference's per-layer pinned batch), slab arenas of 1-5 slots
    (runs broken at arena ends). Three requests per save: A, then B sharing
    A's first chunks (same tokens at the same positions: those are stored
    once, so B's pending chunks are a subset) and its own after them, then C;
    each request's last partial chunk is not stored. Every stored chunk
    equals the oracle's gather from the request that stored it, and A's
    chunks, reloaded in place from the store into fresh random blocks,
    equal the oracle's scatter."""
    rng = np.random.default_rng(2000 + seed)
    L = 2
    bs = int(rng.choice([8, 16, 32]))
    H, D = [(1, 64), (2, 128), (4, 128), (8, 128), (3, 80)][int(rng.integers(5))]
    dtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(3))]
    CH = int(rng.choice([16, 32, 64, 128]))
    transfer = ["dma", "host_write", None][int(rng.integers(3))]
    layout = ["merged_first", "merged_block"][int(rng.integers(2))]
    per_arena = int(rng.integers(1, 6))
    workgroups = int(rng.choice([16, 64, 256]))
    na = CH * int(rng.integers(1, 5)) + int(rng.integers(0, CH))
    shared = int(rng.integers(0, na // CH + 1))  # full chunks of A that B repeats
    nb_ = shared * CH + CH * int(rng.integers(0, 4)) + int(rng.integers(0, CH))
    nc = int(rng.integers(0, 4 * CH))
    base = 100_000 * (seed + 1)
    tokens = {"A": list(range(base, base + na)),
              "B": list(range(base, base + shared * CH)) + list(range(base + 50_000, base + 50_000 + nb_ - shared * CH)),
              "C": list(range(base + 80_000, base + 80_000 + nc))}
    blocks = {r: (len(t) + bs - 1) // bs for r, t in tokens.items()}
    NB = sum(blocks.values()) + 8
    print(f"seed={seed} bs={bs} H={H} D={D} {dtype} CH={CH} transfer={transfer} layout={layout} "
          f"per_arena={per_arena} workgroups={workgroups} tokens A={na} B={nb_} (shared {shared}) C={nc}",
          flush=True)
    pools = [synthetic.paged_pool(NB, bs, H, D, dtype, DEV, seed=60 + seed + l) for l in range(L)]
    layers = pools if layout == "merged_first" else [p.transpose(0, 1).contiguous() for p in pools]
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(seed))
    slots, b0 = {}, 0
    for r in ("A", "B", "C"):
        slots[r] = synthetic.block_slots(perm[b0:b0 + blocks[r]], bs, len(tokens[r]))
        b0 += blocks[r]
    slab = None if transfer is None else PinnedChunkSlab((2, CH, H, D), dtype, chunks_per_arena=per_arena)
    store = PinnedChunkStore(CH, 1 << 34, on_release=None if slab is None else slab.free)
    writer = StoreStreamWriter(store, bs, CH, L, "m", slab=slab, max_workgroups=workgroups,
                               slab_transfer=transfer or "dma")
    requests = [RequestMetadata(r, tokens[r], slots[r], None, True, len(tokens[r])) for r in ("A", "B", "C")]
    for l in range(L):
        writer.save_layer(l, layers[l], requests)
    writer.wait_for_save()
    want = {}  # segment id -> (request, start) of the request that stored it
    for r in ("A", "B", "C"):
        starts = [s for s, _ in writer._chunk_ids.get(r, [])]
        assert starts == list(range(0, len(tokens[r]) // CH * CH, CH)), r
        for start, sid in writer._chunk_ids.get(r, []):
            want.setdefault(sid, (r, start))
    assert len(want) == na // CH + nb_ // CH - shared + nc // CH
    for sid, (r, start) in want.items():
        assert store.is_committed(sid)
        for l in range(L):
            expect = O.gather_paged_kv(_raw(pools[l]), slots[r][start:start + CH].numpy(), bs)
            np.testing.assert_array_equal(_raw(store._entries[sid].layers[l]), expect,
                                          err_msg=f"request {r} chunk {start} layer {l}")
    # reload: A's stored chunks, read in place from the store, into fresh
    # random blocks of another pool
    a_ids = [sid for _, sid in writer._chunk_ids.get("A", [])]
    if a_ids:
        chunks = [store._entries[sid].layers[1] for sid in a_ids]
        fresh = synthetic.paged_pool(NB, bs, H, D, dtype, DEV, seed=90 + seed)
        new_slots = synthetic.block_slots(torch.randperm(NB, generator=torch.Generator().manual_seed(seed + 7))
                                          [: (len(a_ids) * CH + bs - 1) // bs], bs, len(a_ids) * CH)
        expect_pool = _raw(fresh).copy()
        O.scatter_paged_kv(np.concatenate([_raw(c) for c in chunks], axis=1), expect_pool, new_slots.numpy(), bs)
        scatter_chunks(chunks, fresh, new_slots.to(DEV), bs)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_raw(fresh), expect_pool, err_msg="reload of A's chunks")
    store.clear()
    writer.close()
    if slab is not None:
        assert slab.stats()["live"] == 0
        slab.close()


@pytest.mark.parametrize("transfer", ["dma", "host_write"])
def test_store_and_reload_more_chunks_than_one_launch(transfer):
    """A launch carries at most 64 chunk addresses: a 2080-token request in
    16-token chunks is 130 chunks, three launches each way. Every stored
    chunk equals the oracle's gather, and the reload of all 130 chunks in
    place into fresh blocks equals the oracle's scatter."""
    NB, BS, H, D, CH, T = 160, 16, 2, 64, 16, 2080
    pool = synthetic.paged_pool(NB, BS, H, D, torch.bfloat16, DEV, seed=77)
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(77))
    slots = synthetic.block_slots(perm[:T // BS], BS, T)
    slab = PinnedChunkSlab((2, CH, H, D), torch.bfloat16, chunks_per_arena=48)
    store = PinnedChunkStore(CH, 1 << 34, on_release=slab.free)
    writer = StoreStreamWriter(store, BS, CH, 1, "m", slab=slab, slab_transfer=transfer)
    writer.save_layer(0, pool, [RequestMetadata("big", list(range(T)), slots, None, True, T)])
    writer.wait_for_save()
    ids = writer._chunk_ids["big"]
    assert len(ids) == T // CH == 130
    chunks = []
    for start, sid in ids:
        got = store._entries[sid].layers[0]
        np.testing.assert_array_equal(_bits(got), O.gather_paged_kv(_bits(pool), slots[start:start + CH].numpy(), BS),
                                      err_msg=f"chunk {start}")
        chunks.append(got)
    fresh = synthetic.paged_pool(NB, BS, H, D, torch.bfloat16, DEV, seed=78)
    new_slots = synthetic.block_slots(torch.randperm(NB, generator=torch.Generator().manual_seed(78))[:T // BS],
                                      BS, T)
    expect = _bits(fresh).copy()
    O.scatter_paged_kv(np.concatenate([_bits(c) for c in chunks], axis=1), expect, new_slots.numpy(), BS)
    scatter_chunks(chunks, fresh, new_slots.to(DEV), BS)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(fresh), expect)
    store.clear()
    writer.close()
    slab.close()


@pytest.mark.parametrize("transfer", ["dma", "host_write"])
@pytest.mark.parametrize("layout", ["merged_first", "merged_block"])
def test_fused_store_writes_chunks_bit_exact(layout, transfer):
    L, NB, BS, H, D, CH, T = 3, 128, 16, 8, 128, 256, 1000
    pools = [synthetic.paged_pool(NB, BS, H, D, torch.bfloat16, DEV, seed=40 + l) for l in range(L)]
    layers = pools if layout == "merged_first" else [p.transpose(0, 1).contiguous() for p in pools]
    slots = synthetic.block_slots(torch.randperm(NB)[: (T + BS - 1) // BS], BS, T)
    slab = PinnedChunkSlab((2, CH, H, D), torch.bfloat16, chunks_per_arena=8)
    store = PinnedChunkStore(CH, 1 << 34, on_release=slab.free)
    writer = StoreStreamWriter(store, BS, CH, L, "m", slab=slab, max_workgroups=32, slab_transfer=transfer)
    request = RequestMetadata("a", list(range(T)), slots, None, True, T)  # 3 full chunks of 256
    for l in range(L):
        writer.save_layer(l, layers[l], [request])
    writer.wait_for_save()
    segs = writer._chunk_ids["a"]
    assert [s for s, _ in segs] == [0, 256, 512]
    for start, sid in segs:
        assert store.is_committed(sid)
        for l in range(L):
            got = store._entries[sid].layers[l]
            assert _native.host_accessible(got)
            want = O.gather_paged_kv(_bits(pools[l]), slots[start:start + CH].numpy(), BS)
            np.testing.assert_array_equal(_bits(got), want, err_msg=f"chunk {start} layer {l}")
    assert slab.stats()["live"] == 3 * L
    store.clear()  # release hook returns every slot
    assert slab.stats()["live"] == 0
    writer.close()
    slab.close()


@pytest.mark.parametrize("order,zero_copy", [("apart", "auto"), ("apart", False), ("adjacent", False)])
def test_fused_store_then_load_round_trip(order, zero_copy):
    """Store with the fused gather, blend-load (host reads, or DMA of the
    run table -- segments in adjacent slab slots fold into one 2D copy per
    plane) with RoPE relocation, commit: every stage bit-exact against the
    oracle."""
    L, NB, BS, H, D, CH = 2, 192, 16, 4, 128, 256
    layers = [synthetic.paged_pool(NB, BS, H, D, torch.bfloat16, DEV, seed=60 + l) for l in range(L)]
    perm = torch.randperm(NB)
    slots = synthetic.block_slots(perm[:64], BS, 1024)
    slab = PinnedChunkSlab((2, CH, H, D), torch.bfloat16)
    store = PinnedChunkStore(CH, 1 << 34, on_release=slab.free)
    writer = StoreStreamWriter(store, BS, CH, L, "m", slab=slab)
    writer.save_layer(0, layers[0], [RequestMetadata("a", list(range(1024)), slots, None, True, 1024)])
    writer.save_layer(1, layers[1], [RequestMetadata("a", list(range(1024)), slots, None, True, 1024)])
    writer.wait_for_save()
    segs = writer._chunk_ids["a"]
    src = (3, 1) if order == "apart" else (1, 2)  # chunks 1 and 2 sit in consecutive slots
    blend = [BlendSegment(segs[src[0]][1], 260), BlendSegment(segs[src[1]][1], 700)]
    store.pin("b", blend)
    plan = BlendPlan(40, 1100, 512, tuple(blend))
    new_slots = synthetic.block_slots(perm[64:64 + 70], BS, 1100)

    class Rope:
        head_size = rotary_dim = D
        is_neox_style = True
        inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
        ang = torch.arange(4096, dtype=torch.float32)[:, None] * inv[None, :]
        cos_sin_cache = torch.cat([ang.cos(), ang.sin()], dim=-1).to(DEV)

    rope = Rope()
    cache = rope.cos_sin_cache.cpu().numpy()

    def reloc(old, new, k_bits):
        k = O.bf16_to_f32(k_bits).reshape(k_bits.shape[0], -1)
        return O.f32_to_bf16(O.relocate_key(cache, old, new, k, D, True, bf16=True)).reshape(k_bits.shape)

    before = [_bits(l) for l in layers]
    loader = PagedBlendLoader(layers, store, "b", plan, new_slots, BS, CacheBlendConfig.from_extra_config({}),
                              zero_copy=zero_copy)
    loader.prefetch(0, rope)
    for l in range(L):
        buf = loader.get(l)
        loader.prefetch(l + 1, rope)
        hosts = [(256 * c, t, O.gather_paged_kv(before[l], slots[256 * c:256 * c + 256].numpy(), BS))
                 for c, t in zip(src, (260, 700))]
        want = O.loader_assemble(before[l], new_slots.numpy(), BS, 40, 1100, hosts, relocate=reloc)
        np.testing.assert_array_equal(_bits(buf), want, err_msg=f"layer {l}")
        loader.commit(l, buf)
        torch.cuda.synchronize()
        expect = before[l].copy()
        O.loader_commit(want, expect, new_slots.numpy(), BS, 40, 1100)
        np.testing.assert_array_equal(_bits(layers[l]), expect)
    assert loader._zc_layers == ({0, 1} if zero_copy == "auto" else set())
    store.release("b")
    store.clear()
    writer.close()
    slab.close()


@pytest.mark.parametrize("where", ["slab", "device"])
@pytest.mark.parametrize("layout", ["merged_first", "merged_block", "separate"])
def test_scatter_chunks_round_trip_bit_exact(layout, where):
    """Chunks gathered from one set of blocks scatter back into fresh random
    blocks: the pages equal the oracle's scatter of the concatenated chunks
    (ragged last chunk, other pages intact); an out-of-range slot raises
    before anything moves."""
    from cacheblend_vllm.kv_layout import scatter_chunks

    NB, BS, H, D, CH, T = 96, 16, 4, 64, 64, 200  # 4 chunks, the last one ragged
    base = synthetic.paged_pool(NB, BS, H, D, torch.float16, DEV, seed=70)
    if layout == "merged_first":
        kv = base
    elif layout == "merged_block":
        kv = base.transpose(0, 1).contiguous()
    else:
        kv = [base[0].clone(), base[1].clone()]
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(3))
    src_slots = synthetic.block_slots(perm[:13], BS, T)
    chunks = []
    for c in range(4):
        rows = O.gather_paged_kv(_bits(base), src_slots[c * CH:(c + 1) * CH].numpy(), BS)
        full = np.zeros((2, CH, H, D), dtype=np.uint16)
        full[:, :rows.shape[1]] = rows
        t = torch.from_numpy(full.view(np.int16)).view(torch.float16)
        if where == "slab":
            slot = torch.empty((2, CH, H, D), dtype=torch.float16, pin_memory=True)
            slot.copy_(t)
            assert _native.host_accessible(slot)
            chunks.append(slot)
        else:
            chunks.append(t.to(DEV))
    dst_slots = synthetic.block_slots(perm[13:26], BS, T)
    expect = _bits(base).copy()
    flat = np.concatenate([_bits(c) for c in chunks], axis=1)[:, :T]
    O.scatter_paged_kv(flat, expect, dst_slots.numpy(), BS)
    bad = dst_slots.clone()
    bad[7] = NB * BS + 5
    with pytest.raises(IndexError):  # as the reference's index_put_ would
        scatter_chunks(chunks, kv, bad, BS)
    scatter_chunks(chunks, kv, dst_slots, BS, max_workgroups=32)
    torch.cuda.synchronize()
    if layout == "merged_first":
        got = _bits(kv)
    elif layout == "merged_block":
        got = _bits(kv.transpose(0, 1))
    else:
        got = np.stack([_bits(kv[0]), _bits(kv[1])])
    np.testing.assert_array_equal(got, expect)
    # device slots are not range-checked on the host: the kernel skips the
    # out-of-range token and moves the rest
    keep = np.ones(T, dtype=bool)
    keep[7] = False
    fresh = synthetic.block_slots(perm[26:39], BS, T).clone()
    O.scatter_paged_kv(flat[:, keep], expect, fresh.numpy()[keep], BS)
    fresh[7] = NB * BS + 5
    scatter_chunks(chunks, kv, fresh.to(DEV), BS)
    torch.cuda.synchronize()
    if layout == "merged_first":
        got = _bits(kv)
    elif layout == "merged_block":
        got = _bits(kv.transpose(0, 1))
    else:
        got = np.stack([_bits(kv[0]), _bits(kv[1])])
    np.testing.assert_array_equal(got, expect)


def test_scatter_chunks_rejects_pageable_and_short_inputs():
    from cacheblend_vllm.kv_layout import scatter_chunks

    kv = synthetic.paged_pool(8, 16, 2, 64, torch.bfloat16, DEV, seed=1)
    slots = torch.arange(40)
    pageable = [torch.zeros(2, 32, 2, 64, dtype=torch.bfloat16) for _ in range(2)]
    with pytest.raises(ValueError, match="page-locked"):
        scatter_chunks(pageable, kv, slots, 16)
    with pytest.raises(ValueError, match="need 2 chunks"):
        scatter_chunks(pageable[:1], kv, slots, 16)
    with pytest.raises(ValueError, match="expected"):
        scatter_chunks([torch.zeros(2, 32, 2, 32, dtype=torch.bfloat16, device=DEV)] * 2, kv, slots, 16)
    scatter_chunks([], kv, slots[:0], 16)  # nothing to move
