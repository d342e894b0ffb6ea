"""GPU: the worker connector driven exactly as vLLM drives it.

register_kv_caches(kv_caches) -> save_kv_layer(layer_name, kv_layer,
attn_metadata) per layer -> wait_for_save() -> start_load_kv(forward_context)
-> wait_for_layer_load(layer_name) -> get_finished(ids), with the layerwise
executor found through the model registry (reference connector.py:168-276).
The blended pages are compared bit for bit with the oracle; a second test
checks that chunks evicted after a load are not reused while the load may
still read them.
"""

import json
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle as O
from cacheblend_vllm import registry, synthetic
from cacheblend_vllm.connector import CacheBlendConnectorV1, KVConnectorRole
from cacheblend_vllm.store_path import CacheBlendConnectorMetadata, RequestMetadata
from cacheblend_vllm.types import BlendPlan

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
BS, H, D, CH, NB, L = 16, 2, 64, 64, 64, 3


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


class Rope:
    def __init__(self, head_size, max_pos):
        self.head_size = self.rotary_dim = head_size
        self.is_neox_style = True
        inv = 1.0 / (1e4 ** (torch.arange(0, head_size, 2, dtype=torch.float32) / head_size))
        ang = torch.arange(max_pos, dtype=torch.float32)[:, None] * inv[None, :]
        self.cos_sin_cache = torch.cat([ang.cos(), ang.sin()], dim=-1).to(DEV)


class CommitExecutor:
    """A layerwise executor without model math: each layer's assembled buffer
    is committed as loaded. Moves the forward context's cursors to check that
    the connector restores them."""

    def __init__(self, rope, delay_cycles=0):
        self.rope, self.delay_cycles, self.runs = rope, delay_cycles, []

    def run(self, request_id, tokens, plan, loader):
        self.runs.append((request_id, plan))
        if self.delay_cycles:  # hold the Load and Copy streams: the host reads stay in flight
            for stream in (loader._load_stream, loader._copy_stream):
                with torch.cuda.stream(stream):
                    torch.cuda._sleep(self.delay_cycles)
        n = len(loader.kv_caches)
        loader.prefetch(0, self.rope)
        for layer in range(n):
            buf = loader.get(layer)
            if layer + 1 < n:
                loader.prefetch(layer + 1, self.rope)
            loader.commit(layer, buf)


def _vllm_config(engine, local_cpu_gb=1.0):
    return SimpleNamespace(
        kv_transfer_config=SimpleNamespace(
            kv_connector_extra_config={"chunk_size": CH, "local_cpu_gb": local_cpu_gb},
            engine_id=engine, kv_load_failure_policy=None),
        cache_config=SimpleNamespace(block_size=BS),
        parallel_config=SimpleNamespace(pipeline_parallel_size=1, tensor_parallel_size=1),
        model_config=SimpleNamespace(model="test-model"),
    )


def _layers(seed):
    # vLLM's names, registered out of order: the connector sorts by layer index
    return {f"model.layers.{i}.self_attn.attn": synthetic.paged_pool(NB, BS, H, D, torch.bfloat16, DEV,
                                                                     seed=seed + i)
            for i in (2, 0, 1)}


def _save(conn, kv, request):
    conn.bind_connector_metadata(CacheBlendConnectorMetadata([request]))
    for name in sorted(kv, key=lambda n: int(n.split(".")[2])):
        conn.save_kv_layer(name, kv[name], None)
    conn.wait_for_save()
    conn.clear_connector_metadata()


def test_connector_drop_in_save_then_blend_load(monkeypatch, tmp_path):
    monkeypatch.setenv("CACHEBLEND_TRACE_DIR", str(tmp_path))
    registry.clear_for_test()
    rope = Rope(D, 4096)
    executor = CommitExecutor(rope)
    registry.register_model("drop-in", executor)
    conn = CacheBlendConnectorV1(_vllm_config("drop-in"), KVConnectorRole.WORKER)
    kv = _layers(20)
    conn.register_kv_caches(kv)
    ordered = [kv[f"model.layers.{i}.self_attn.attn"] for i in range(L)]
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(3))

    # save a 256-token prompt (4 chunks) from blocks perm[:16]
    prompt = list(range(1000, 1256))
    slots = synthetic.block_slots(perm[:16], BS, 256)
    _save(conn, kv, RequestMetadata("a", prompt, slots, None, True, 256))
    chunk_ids = conn._writer._chunk_ids["a"]
    assert all(conn._store.is_committed(sid) for _, sid in chunk_ids)

    # a new prompt reuses chunks 3 and 1 at other offsets behind a 32-token APC prefix
    new_prompt = list(range(50, 82)) + prompt[192:256] + list(range(7, 47)) + prompt[64:128] + [5] * 20
    segments = conn._store.match(conn.model_scope, new_prompt, 32)
    assert [(s.source_start, s.target_start) for s in segments] == [(192, 32), (64, 136)]
    assert conn._store.pin("b", segments) == segments   # what the lookup server does
    plan = BlendPlan(32, len(new_prompt), 128, segments)
    new_slots = synthetic.block_slots(perm[16:16 + 14], BS, len(new_prompt))
    before = [_bits(t) for t in ordered]
    ctx = SimpleNamespace(layer_idx=7, moe_layer_index=3)
    conn.bind_connector_metadata(CacheBlendConnectorMetadata(
        [RequestMetadata("b", new_prompt, new_slots, plan, False, 0)]))
    conn.start_load_kv(ctx)
    for name in kv:
        conn.wait_for_layer_load(name)
    torch.cuda.synchronize()
    assert (ctx.layer_idx, ctx.moe_layer_index) == (7, 3)
    assert executor.runs == [("b", plan)]

    cache = rope.cos_sin_cache.cpu().numpy()

    def reloc(old, new, k_bits):
        k = O.bf16_to_f32(k_bits).reshape(k_bits.shape[0], -1)
        return O.f32_to_bf16(O.relocate_key(cache, old, new, k, D, True, bf16=True)).reshape(k_bits.shape)

    for layer in range(L):
        hosts = [(192, 32, O.gather_paged_kv(before[layer], slots[192:256].numpy(), BS)),
                 (64, 136, O.gather_paged_kv(before[layer], slots[64:128].numpy(), BS))]
        buf = O.loader_assemble(before[layer], new_slots.numpy(), BS, 32, len(new_prompt), hosts,
                                relocate=reloc)
        want = before[layer].copy()
        O.loader_commit(buf, want, new_slots.numpy(), BS, 32, len(new_prompt))
        np.testing.assert_array_equal(_bits(ordered[layer]), want, err_msg=f"layer {layer}")

    assert conn.get_finished({"a", "b"}) == (None, None)
    assert conn.get_block_ids_with_load_errors() == set()
    conn.close()
    registry.clear_for_test()
    events = [json.loads(line)["event"] for f in tmp_path.iterdir() for line in f.read_text().splitlines()]
    for name in ("worker_registered", "save_store_enqueued", "save_store_finished",
                 "save_store_wait_finished", "blend_started", "loader_initialized",
                 "layer_committed", "blend_finished"):
        assert name in events, name


@pytest.mark.parametrize("seed", range(6))
def test_connector_random_reuse(seed):
    """Seeded random reuse through the connector: two saved prompts of 2-4
    chunks, then a prompt built from randomly chosen stored chunks (either
    prompt, any order, adjacent or separated by fresh filler) behind a random
    APC prefix. The store's matcher finds exactly the placed chunks, and the
    pages after the blend load equal the oracle's assembly (relocated K) and
    commit."""
    rng = np.random.default_rng(4000 + seed)
    registry.clear_for_test()
    rope = Rope(D, 4096)
    executor = CommitExecutor(rope)
    registry.register_model(f"random-{seed}", executor)
    conn = CacheBlendConnectorV1(_vllm_config(f"random-{seed}"), KVConnectorRole.WORKER)
    kv = _layers(30 + seed)
    conn.register_kv_caches(kv)
    ordered = [kv[f"model.layers.{i}.self_attn.attn"] for i in range(L)]
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(seed))
    saved, b0 = {}, 0
    for r, base in (("a", 1_000_000), ("b", 2_000_000)):
        n = CH * int(rng.integers(2, 5))
        tokens = [base + int(t) for t in rng.permutation(n)]
        slots = synthetic.block_slots(perm[b0:b0 + n // BS], BS, n)
        b0 += n // BS
        _save(conn, kv, RequestMetadata(r, tokens, slots, None, True, n))
        saved[r] = (tokens, slots)
    apc = int(rng.integers(0, 33))
    prompt = [3_000_000 + i for i in range(apc)]
    placed = []  # (request, source_start, target_start)
    fresh = 4_000_000
    while len(prompt) < 300:
        if rng.random() < 0.4:
            gap = int(rng.integers(1, 41))
            prompt += list(range(fresh, fresh + gap))
            fresh += gap
        r = "ab"[int(rng.integers(2))]
        src = CH * int(rng.integers(len(saved[r][0]) // CH))
        placed.append((r, src, len(prompt)))
        prompt += saved[r][0][src:src + CH]
    prompt += list(range(fresh, fresh + int(rng.integers(0, 20))))
    print(f"seed={seed} apc={apc} prompt={len(prompt)} placed={placed}", flush=True)
    segments = conn._store.match(conn.model_scope, prompt, apc)
    assert [(s.source_start, s.target_start) for s in segments] == [(s, t) for _, s, t in placed]
    assert conn._store.pin("new", segments) == segments
    plan = BlendPlan(apc, len(prompt), CH * len(placed), segments)
    new_slots = synthetic.block_slots(perm[b0:b0 + (len(prompt) + BS - 1) // BS], BS, len(prompt))
    before = [_bits(t) for t in ordered]
    conn.bind_connector_metadata(CacheBlendConnectorMetadata(
        [RequestMetadata("new", prompt, new_slots, plan, False, 0)]))
    conn.start_load_kv(SimpleNamespace())
    for name in kv:
        conn.wait_for_layer_load(name)
    torch.cuda.synchronize()
    cache = rope.cos_sin_cache.cpu().numpy()

    def reloc(old, new, k_bits):
        k = O.bf16_to_f32(k_bits).reshape(k_bits.shape[0], -1)
        return O.f32_to_bf16(O.relocate_key(cache, old, new, k, D, True, bf16=True)).reshape(k_bits.shape)

    for layer in range(L):
        # the stored chunks hold the pages as they were when saved (loads
        # write only the new prompt's blocks)
        hosts = [(s, t, O.gather_paged_kv(before[layer], saved[r][1][s:s + CH].numpy(), BS))
                 for r, s, t in placed]
        buf = O.loader_assemble(before[layer], new_slots.numpy(), BS, apc, len(prompt), hosts, relocate=reloc)
        want = before[layer].copy()
        O.loader_commit(buf, want, new_slots.numpy(), BS, apc, len(prompt))
        np.testing.assert_array_equal(_bits(ordered[layer]), want, err_msg=f"layer {layer}")
    conn.close()
    registry.clear_for_test()


def _sleep_cycles_per_ms():
    torch.cuda._sleep(1000)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    torch.cuda._sleep(5_000_000)
    e1.record()
    e1.synchronize()
    return 5_000_000 / e0.elapsed_time(e1)


def test_evicted_chunks_wait_for_in_flight_loads():
    """The store is full; a load's host reads are held in flight on the Load
    and Copy streams; its request is released and new chunks, written by
    the host into fresh slab slots, evict the loaded ones. Their slots must
    stay out of circulation until the load's reads are done (else the host
    writes would land in memory the load still reads), and the load must
    still be bit-exact."""
    registry.clear_for_test()
    rope = Rope(D, 4096)
    executor = CommitExecutor(rope, delay_cycles=int(300 * _sleep_cycles_per_ms()))
    registry.register_model("evict", executor)
    chunk_layer_bytes = 2 * CH * H * D * 2
    cap_gb = 4 * L * chunk_layer_bytes / 2**30        # room for exactly 4 chunks of every layer
    conn = CacheBlendConnectorV1(_vllm_config("evict", cap_gb), KVConnectorRole.WORKER)
    kv = _layers(40)
    conn.register_kv_caches(kv)
    ordered = [kv[f"model.layers.{i}.self_attn.attn"] for i in range(L)]
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(4))
    prompt = list(range(3000, 3256))
    slots = synthetic.block_slots(perm[:16], BS, 256)
    _save(conn, kv, RequestMetadata("a", prompt, slots, None, True, 256))
    loaded = {sid for _, sid in conn._writer._chunk_ids["a"]}
    loaded_ptrs = {t.data_ptr() for sid in loaded for t in conn._store._entries[sid].layers.values()}
    assert conn._store.current_bytes == conn._store.max_bytes

    segments = conn._store.match(conn.model_scope, prompt, 0)
    assert len(segments) == 4
    conn._store.pin("b", segments)
    plan = BlendPlan(0, 256, 256, segments)
    new_slots = synthetic.block_slots(perm[16:32], BS, 256)
    before = [_bits(t) for t in ordered]
    conn.bind_connector_metadata(CacheBlendConnectorMetadata(
        [RequestMetadata("b", prompt, new_slots, plan, False, 0)]))
    conn.start_load_kv(SimpleNamespace())   # returns with the loads still held on the Load stream
    conn.get_finished({"a"})

    # new chunks written by the host evict every loaded chunk while the loads are held
    other = list(range(9000, 9256))
    for sid in conn._store.begin_put_chunks(conn.model_scope, other, 0, 256, L):
        for layer in range(L):
            slot = conn._slab.alloc()
            slot.fill_(-1.0)
            conn._store.put_layer_host(sid, layer, slot)
    assert not any(sid in conn._store._entries for sid in loaded)
    held = conn._slab.stats()["pending"]
    in_use = {t.data_ptr() for e in conn._store._entries.values() for t in e.layers.values()}
    print(f"pending slots while loads in flight: {held}", flush=True)
    assert held == len(loaded_ptrs)
    assert not (in_use & loaded_ptrs)
    torch.cuda.synchronize()
    for layer in range(L):
        hosts = [(s.source_start, s.target_start,
                  O.gather_paged_kv(before[layer], slots[s.source_start:s.source_start + CH].numpy(), BS))
                 for s in segments]
        buf = O.loader_assemble(before[layer], new_slots.numpy(), BS, 0, 256, hosts)
        want = before[layer].copy()
        O.loader_commit(buf, want, new_slots.numpy(), BS, 0, 256)
        np.testing.assert_array_equal(_bits(ordered[layer]), want, err_msg=f"layer {layer}")
    conn._slab.alloc()                      # reclaims the slots whose loads finished
    assert conn._slab.stats()["pending"] == 0
    conn.close()
    registry.clear_for_test()
