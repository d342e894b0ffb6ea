"""GPU end to end: save pipeline -> pinned store -> blend loader -> commit.

A prompt's KV is saved layerwise through the Store stream (gather + pinned
D2H + publication), then loaded back as blend segments at other target
positions (RoPE relocation) and committed into fresh pages; every stage is
compared bit for bit with the oracle.
"""

import numpy as np
import pytest
import torch
from types import SimpleNamespace

import oracle as O
from cacheblend_vllm import registry, synthetic
from cacheblend_vllm.config import CacheBlendConfig
from cacheblend_vllm.connector import CacheBlendConnectorV1, KVConnectorRole
from cacheblend_vllm.host_store import PinnedChunkStore
from cacheblend_vllm.loader import PagedBlendLoader
from cacheblend_vllm.store_path import CacheBlendConnectorMetadata, RequestMetadata, StoreStreamWriter
from cacheblend_vllm.types import BlendPlan, BlendSegment

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


class Rope:
    def __init__(self, head_size, max_pos, neox=True):
        self.head_size = self.rotary_dim = head_size
        self.is_neox_style = neox
        inv = 1.0 / (1e6 ** (torch.arange(0, head_size, 2, dtype=torch.float32) / head_size))
        ang = torch.arange(max_pos, dtype=torch.float32)[:, None] * inv[None, :]
        self.cos_sin_cache = torch.cat([ang.cos(), ang.sin()], dim=-1).to(DEV)


def test_save_then_blend_load_round_trip():
    L, NB, BS, H, D, CH = 4, 256, 16, 8, 128, 256
    tokens = 1024
    layers = [synthetic.paged_pool(NB, BS, H, D, torch.bfloat16, DEV, seed=10 + l) for l in range(L)]
    perm = torch.randperm(NB)
    slots = synthetic.block_slots(perm[: tokens // BS], BS, tokens)
    store = PinnedChunkStore(CH, 1 << 34)
    writer = StoreStreamWriter(store, BS, CH, L, "m")
    request = RequestMetadata("a", list(range(5000, 5000 + tokens)), slots, None, True, tokens)
    for l in range(L):
        writer.save_layer(l, layers[l], [request])
    writer.wait_for_save()
    segs = writer._chunk_ids["a"]
    assert [s for s, _ in segs] == [0, 256, 512, 768]
    for start, sid in segs:
        assert store.is_committed(sid)
        for l in range(L):
            store_bits = _bits(store._entries[sid].layers[l])
            want = O.gather_paged_kv(_bits(layers[l]), slots[start:start + CH].numpy(), BS)
            np.testing.assert_array_equal(store_bits, want)

    # blend: chunks 2 and 0 reused at new positions behind a 100-token APC prefix
    blend = [BlendSegment(segs[2][1], 300), BlendSegment(segs[0][1], 700)]
    store.pin("b", blend)
    plan = BlendPlan(100, 1000, 512, tuple(blend))
    new_slots = synthetic.block_slots(perm[tokens // BS: tokens // BS + 63], BS, 1000)
    rope = Rope(D, 4096)
    loader = PagedBlendLoader(layers, store, "b", plan, new_slots, BS,
                              CacheBlendConfig.from_extra_config({}))
    cache = rope.cos_sin_cache.cpu().numpy()

    def reloc(old, new, k_bits):
        k = O.bf16_to_f32(k_bits).reshape(k_bits.shape[0], -1)
        return O.f32_to_bf16(O.relocate_key(cache, old, new, k, D, True, bf16=True)).reshape(k_bits.shape)

    loader.prefetch(0, rope)
    for l in range(L):
        pages_before = _bits(layers[l])
        buf = loader.get(l)
        loader.prefetch(l + 1, rope)
        hosts = [(512, 300, O.gather_paged_kv(pages_before, slots[512:768].numpy(), BS)),
                 (0, 700, O.gather_paged_kv(pages_before, slots[0:256].numpy(), BS))]
        want = O.loader_assemble(pages_before, new_slots.numpy(), BS, 100, 1000, hosts, relocate=reloc)
        np.testing.assert_array_equal(_bits(buf), want, err_msg=f"layer {l}")
        loader.commit(l, buf)
        torch.cuda.synchronize()
        expect = pages_before.copy()
        O.loader_commit(want, expect, new_slots.numpy(), BS, 100, 1000)
        np.testing.assert_array_equal(_bits(layers[l]), expect, err_msg=f"commit layer {l}")
    store.release("b")
    writer.close()


def test_connector_worker_save_and_load_with_failure_policy():
    cfg = SimpleNamespace(
        kv_transfer_config=SimpleNamespace(
            kv_connector_extra_config={"chunk_size": 64, "local_cpu_gb": 1},
            engine_id="e", kv_load_failure_policy="recompute"),
        cache_config=SimpleNamespace(block_size=16),
        parallel_config=SimpleNamespace(pipeline_parallel_size=1, tensor_parallel_size=1),
        model_config=SimpleNamespace(model="test-model"),
    )
    conn = CacheBlendConnectorV1(cfg, KVConnectorRole.WORKER)
    layers = {f"model.layers.{i}.self_attn.attn": synthetic.paged_pool(32, 16, 2, 64, torch.bfloat16, DEV, seed=i)
              for i in (1, 0)}

    class Executor:
        def __init__(self):
            self.calls = 0

        def run(self, request_id, tokens, plan, loader):
            self.calls += 1
            raise RuntimeError("model failure")

    executor = Executor()
    registry.clear_for_test()
    registry.register_model("e", executor)
    conn.register_kv_caches(layers)
    slots = synthetic.block_slots(torch.arange(8), 16, 128)
    req = RequestMetadata("r", list(range(128)), slots, None, True, 128)
    conn.bind_connector_metadata(CacheBlendConnectorMetadata([req]))
    for name in layers:
        conn.save_kv_layer(name, layers[name], None)
    conn.wait_for_save()
    segs = conn._writer._chunk_ids["r"]
    assert all(conn._store.is_committed(sid) for _, sid in segs)
    # a failing load reports exactly the blocks of the external span
    plan = BlendPlan(16, 128, 64, (BlendSegment(segs[1][1], 64),))
    conn._store.pin("r2", plan.segments)
    load_req = RequestMetadata("r2", list(range(128)), slots, plan, False, 0)
    conn.bind_connector_metadata(CacheBlendConnectorMetadata([load_req]))
    conn.start_load_kv(None)
    assert executor.calls == 1
    assert conn.get_block_ids_with_load_errors() == set(range(1, 8))
    with pytest.raises(NotImplementedError, match="control plane"):
        conn.build_connector_meta(None)
    conn.close()
    registry.clear_for_test()
