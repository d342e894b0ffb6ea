"""GPU parity: blend loader (fused assembly + commit) and RoPE relocation.

Buffers and pages are compared bit for bit with the oracle, including the
RoPE-relocated K rows (the kernel rounds every elementwise result to the key
dtype, as the reference's torch arithmetic does).
"""

import numpy as np
import pytest
import torch

import oracle as O
from cacheblend_vllm import synthetic
from cacheblend_vllm.config import CacheBlendConfig
from cacheblend_vllm.host_store import PinnedChunkStore
from cacheblend_vllm.loader import PagedBlendLoader, build_source_map
from cacheblend_vllm.rope import relocate_key, validate_rope_support
from cacheblend_vllm.types import BlendPlan, BlendSegment

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


class Rope:
    """vLLM-style RotaryEmbedding stand-in: a [max_pos, D] cos|sin cache."""

    def __init__(self, head_size: int, max_pos: int, neox: bool, base: float = 10000.0):
        self.head_size = head_size
        self.rotary_dim = head_size
        self.is_neox_style = neox
        inv = 1.0 / (base ** (torch.arange(0, head_size, 2, dtype=torch.float32) / head_size))
        ang = torch.arange(max_pos, dtype=torch.float32)[:, None] * inv[None, :]
        self.cos_sin_cache = torch.cat([ang.cos(), ang.sin()], dim=-1).to(DEV)


def _cfg(**kw):
    return CacheBlendConfig.from_extra_config({"strict_version_check": False, **kw})


def test_reference_known_answer(golden):
    case = golden["loader_prefix_gaps_suffix"]
    for pipeline in (False, True):
        paged = torch.arange(16, dtype=torch.float32).reshape(case["paged_shape"]).to(DEV)
        store = PinnedChunkStore(2, 1 << 20)
        seg = case["segment"]
        sid = store.begin_put("m", seg["source_start"], [7, 8], num_layers=1)
        parent = torch.zeros(2, 4, 1, 1)
        parent[0, 1:3, 0, 0] = torch.tensor(case["host_k"])
        parent[1, 1:3, 0, 0] = torch.tensor(case["host_v"])
        host = parent[:, 1:3]
        assert not host.is_contiguous()
        store.put_layer_host(sid, 0, host)
        segment = BlendSegment(sid, target_start=seg["target_start"])
        store.pin("r", [segment])
        plan = BlendPlan(case["apc_prefix_tokens"], case["allocation_end"], seg["length"], (segment,))
        loader = PagedBlendLoader([paged], store, "r", plan, torch.tensor(case["slots"]),
                                  case["block_size"], _cfg(chunk_size=2, event_pipeline=pipeline))
        loader.prefetch(0, Rope(2, 16, True))
        buf = loader.get(0)
        assert buf[0].reshape(-1).tolist() == case["expected_buffer_k"]
        assert buf[1].reshape(-1).tolist() == case["expected_buffer_v"]
        lo, hi = case["commit_fill_range"]
        buf[:, lo:hi].fill_(case["commit_fill"])
        loader.commit(0, buf)
        torch.cuda.synchronize()
        assert paged[0].reshape(2, -1).tolist() == case["expected_pages_after_commit_k"]
        assert paged[1].reshape(2, -1).tolist() == case["expected_pages_after_commit_v"]


# head_dim 128 / 64: one 16-byte vector per lane with lane exchange for NeoX
# pairs, rows of 0.75-4 KiB (1, 2 and 4 passes of 1 KiB); 80: heads straddle
# 1 KiB passes, so the per-pair path runs
@pytest.mark.parametrize("head_dim,heads", [(128, 4), (64, 6), (80, 3), (128, 6), (128, 8)])
@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_relocate_key_bit_exact_vs_oracle(neox, dtype, head_dim, heads):
    rope = Rope(head_dim, 4096, neox)
    torch.manual_seed(0)
    key = torch.randn(300, heads * head_dim, device=DEV).to(dtype)
    old = torch.randint(0, 4096, (300,))
    new = torch.randint(0, 4096, (300,))
    got = relocate_key(rope, old, new, key)
    cache = rope.cos_sin_cache.cpu().numpy()
    want = O.relocate_key(cache if dtype != torch.float16 else cache.astype(np.float16).astype(np.float32),
                          old.numpy(), new.numpy(), key.float().cpu().numpy(), head_dim, neox,
                          bf16=dtype == torch.bfloat16)
    if dtype == torch.float16:
        # the oracle's rounding helper is bf16-only: compare within one f16 ulp
        np.testing.assert_allclose(got.float().cpu().numpy(), want, rtol=2e-3, atol=2e-3)
    else:
        np.testing.assert_array_equal(got.float().cpu().numpy(), want)
    # identity when positions are unchanged (reference ascend.py:64-65)
    assert relocate_key(rope, old, old.clone(), key) is key


@pytest.mark.parametrize("neox", [False, True])
def test_relocate_key_known_answer_matches_fresh_rope(golden, neox):
    case = golden["relocate_key_matches_fresh_rope"]
    rope = Rope(4, 16, neox)
    ang = torch.arange(16, dtype=torch.float32)[:, None] * case["angle_per_position"]
    rope.cos_sin_cache = torch.cat([ang.cos(), ang.cos(), ang.sin(), ang.sin()], dim=1).to(DEV)

    def fresh(positions, value):
        shaped = value.reshape(value.shape[0], -1, 4)
        a = positions.float().reshape(-1, 1, 1) * case["angle_per_position"]
        c, s = torch.cos(a), torch.sin(a)
        if neox:
            f, sec = shaped[..., :2], shaped[..., 2:]
            out = torch.cat((f * c - sec * s, sec * c + f * s), dim=-1)
        else:
            f, sec = shaped[..., 0::2], shaped[..., 1::2]
            out = torch.stack((f * c - sec * s, sec * c + f * s), dim=-1).reshape_as(shaped)
        return out.reshape_as(value)

    raw = torch.randn(case["key_rows"], case["key_width"], generator=torch.Generator().manual_seed(0))
    old = torch.tensor(case["old_positions"])
    new = torch.tensor(case["new_positions"])
    got = relocate_key(rope, old, new, fresh(old, raw).to(DEV))
    assert torch.allclose(got.cpu(), fresh(new, raw), atol=case["atol"], rtol=case["rtol"])


def test_validate_rope_support_rules():
    from types import SimpleNamespace

    model = SimpleNamespace(config=SimpleNamespace(rope_scaling=None, partial_rotary_factor=1.0))
    rope = Rope(4, 8, True)
    validate_rope_support(model, rope)
    model.config.rope_scaling = {"type": "linear"}
    with pytest.raises(ValueError, match="rope_scaling"):
        validate_rope_support(model, rope)
    model.config.rope_scaling = None
    rope.cos_sin_cache = torch.ones(8, 4)
    with pytest.raises(ValueError, match="unit-norm"):
        validate_rope_support(model, rope)


def _blend_setup(num_layers, nb, bs, heads, dim, apc, segments, alloc_end, dtype, chunk, seed=0):
    """Pages, a pinned store holding each segment run contiguously per layer,
    and the plan. ``segments`` = list of (source_start, target_start, length)."""
    torch.manual_seed(seed)
    layers = [synthetic.paged_pool(nb, bs, heads, dim, dtype, DEV, seed=seed + l) for l in range(num_layers)]
    store = PinnedChunkStore(chunk, 1 << 40)
    blend_segments = []
    hosts = {}  # (seg_index, layer) -> host run [2, len, H, D]
    for i, (src, tgt, n) in enumerate(segments):
        for l in range(num_layers):
            hosts[i, l] = torch.randn(2, n, heads, dim).to(dtype).pin_memory()
        for c0 in range(0, n, chunk):
            tokens = list(range(src + c0 + 1000 * i, src + c0 + 1000 * i + chunk))
            sid = store.begin_put("m", src + c0, tokens, num_layers)
            for l in range(num_layers):
                store.put_layer_host(sid, l, hosts[i, l][:, c0 : c0 + chunk])
            blend_segments.append(BlendSegment(sid, tgt + c0))
    store.pin("req", blend_segments)
    hit = sum(n for _, _, n in segments)
    plan = BlendPlan(apc, alloc_end, hit, tuple(blend_segments))
    perm = torch.randperm(nb)
    slots = synthetic.block_slots(perm[: (alloc_end + bs - 1) // bs], bs, alloc_end)
    return layers, store, plan, slots, hosts


@pytest.mark.parametrize("zero_copy", [True, False])
@pytest.mark.parametrize("neox", [True, False])
def test_loader_bf16_relocation_bit_exact_vs_oracle(neox, zero_copy):
    heads, dim, bs, chunk = 4, 128, 16, 64
    segs = [(0, 100, 128), (512, 300, 64), (64, 400, 192)]  # source != target: relocate
    layers, store, plan, slots, hosts = _blend_setup(3, 200, bs, heads, dim, 37, segs, 700,
                                                     torch.bfloat16, chunk)
    rope = Rope(dim, 2048, neox)
    loader = PagedBlendLoader(layers, store, "req", plan, slots, bs, _cfg(chunk_size=chunk),
                              zero_copy=zero_copy)
    cache = rope.cos_sin_cache.cpu().numpy()

    def reloc(old, new, k_bits):
        k = O.bf16_to_f32(k_bits).reshape(k_bits.shape[0], -1)
        out = O.relocate_key(cache, old, new, k, dim, neox, bf16=True)
        return O.f32_to_bf16(out).reshape(k_bits.shape)

    loader.prefetch(0, rope)
    for l in range(3):
        buf = loader.get(l)
        loader.prefetch(l + 1, rope)
        want = O.loader_assemble(
            _bits(layers[l]), slots.numpy(), bs, plan.apc_prefix_tokens, plan.allocation_end,
            [(s, t, _bits(hosts[i, l])) for i, (s, t, _) in enumerate(segs)], relocate=reloc,
        )
        np.testing.assert_array_equal(_bits(buf), want, err_msg=f"layer {l}")
        # commit writes [apc:] into the pages, the prefix pages stay
        expect_pages = _bits(layers[l]).copy()
        fresh = torch.randn_like(buf, dtype=torch.float32).to(torch.bfloat16)
        O.loader_commit(_bits(fresh), expect_pages, slots.numpy(), bs, plan.apc_prefix_tokens,
                        plan.allocation_end)
        buf.copy_(fresh)
        loader.commit(l, buf)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bits(layers[l]), expect_pages, err_msg=f"commit layer {l}")
    # the pinned chunks took the host-read path exactly when asked to
    assert (len(loader._zc_layers) > 0) == zero_copy


@pytest.mark.parametrize("ring_slots", [2, 3, 7])
def test_loader_dma_ring_wraps_bit_exact(ring_slots):
    """DMA path with a hit ring shorter than the layer count: slots are
    refilled after the host-side fence on the assembly that last read them;
    every layer still equals the oracle."""
    heads, dim, bs, chunk, L = 4, 128, 16, 64, 7
    segs = [(0, 100, 128), (512, 300, 64), (64, 400, 192)]
    layers, store, plan, slots, hosts = _blend_setup(L, 200, bs, heads, dim, 37, segs, 700,
                                                     torch.bfloat16, chunk, seed=11)
    rope = Rope(dim, 2048, True)
    loader = PagedBlendLoader(layers, store, "req", plan, slots, bs, _cfg(chunk_size=chunk),
                              zero_copy=False, dma_staging_layers=ring_slots)
    cache = rope.cos_sin_cache.cpu().numpy()

    def reloc(old, new, k_bits):
        k = O.bf16_to_f32(k_bits).reshape(k_bits.shape[0], -1)
        return O.f32_to_bf16(O.relocate_key(cache, old, new, k, dim, True, bf16=True)).reshape(k_bits.shape)

    loader.prefetch(0, rope)
    for l in range(L):
        buf = loader.get(l)
        loader.prefetch(l + 1, rope)
        want = O.loader_assemble(
            _bits(layers[l]), slots.numpy(), bs, plan.apc_prefix_tokens, plan.allocation_end,
            [(s, t, _bits(hosts[i, l])) for i, (s, t, _) in enumerate(segs)], relocate=reloc,
        )
        np.testing.assert_array_equal(_bits(buf), want, err_msg=f"layer {l}")
        loader.commit(l, buf)
    torch.cuda.synchronize()
    assert loader._hit_ring.shape[0] == min(ring_slots, L) and not loader._zc_layers


@pytest.mark.parametrize("seed", range(16))
def test_loader_random_plans_bit_exact_vs_oracle(seed):
    """Seeded random blend plans over two layers: block sizes 8-32, head
    shapes (the 80-dim per-pair path included), chunk sizes 16-64, an APC
    prefix of 0-3 blocks, 1-5 segments with 0-69-token gaps, an allocation
    end not aligned to the block size, RoPE relocation (NeoX or interleaved)
    in bf16, float32 and f16, every transfer mode. Each assembled buffer and
    the pages after each commit equal the oracle's bit for bit, except the
    relocated f16 K rows: the oracle rounds once, at the end, where the
    kernel rounds every elementwise step to f16 as torch does, so those rows
    agree within 2e-3."""
    rng = np.random.default_rng(1000 + seed)
    bs = int(rng.choice([8, 16, 32]))
    heads, dim = [(1, 64), (2, 128), (4, 128), (8, 64), (3, 80)][int(rng.integers(5))]
    dtype = [torch.bfloat16, torch.float32, torch.float16][int(rng.integers(3))]
    chunk = int(rng.choice([16, 32, 64]))
    moved = rng.random() < 0.8
    neox = bool(rng.integers(2))
    zero_copy = ["auto", True, False][int(rng.integers(3))]
    apc = int(rng.integers(0, 3 * bs + 1))
    segs, pos = [], apc
    for _ in range(int(rng.integers(1, 6))):
        pos += int(rng.integers(0, 70))
        n = chunk * int(rng.integers(1, 5))
        segs.append((int(rng.integers(0, 600)) if moved else pos, pos, n))
        pos += n
    alloc_end = pos + int(rng.integers(0, 2 * bs + 2))
    nb = (alloc_end + bs - 1) // bs + 8
    print(f"seed={seed} bs={bs} heads={heads} dim={dim} {dtype} chunk={chunk} moved={moved} neox={neox} "
          f"zero_copy={zero_copy} apc={apc} segs={segs} alloc_end={alloc_end}", flush=True)
    layers, store, plan, slots, hosts = _blend_setup(2, nb, bs, heads, dim, apc, segs, alloc_end, dtype,
                                                     chunk, seed=seed)
    rope = Rope(dim, 2048, neox)
    cache = rope.cos_sin_cache.cpu().numpy()

    def reloc(old, new, k_bits):
        if dtype == torch.bfloat16:
            k = O.bf16_to_f32(k_bits).reshape(k_bits.shape[0], -1)
            out = O.relocate_key(cache, old, new, k, dim, neox, bf16=True)
            return O.f32_to_bf16(out).reshape(k_bits.shape)
        if dtype == torch.float16:
            k = k_bits.view(np.float16).astype(np.float32).reshape(k_bits.shape[0], -1)
            out = O.relocate_key(cache16, old, new, k, dim, neox, bf16=False)
            return out.astype(np.float16).view(np.uint16).reshape(k_bits.shape)
        k = k_bits.reshape(k_bits.shape[0], -1)
        return O.relocate_key(cache, old, new, k, dim, neox, bf16=False).reshape(k_bits.shape)

    cache16 = cache.astype(np.float16).astype(np.float32)
    relocated = np.zeros(alloc_end, dtype=bool)  # K rows whose positions move
    for s, t, n in segs:
        relocated[t:t + n] |= s != t
    loader = PagedBlendLoader(layers, store, "req", plan, slots, bs, _cfg(chunk_size=chunk),
                              zero_copy=zero_copy)
    loader.prefetch(0, rope)
    for l in range(2):
        buf = loader.get(l)
        loader.prefetch(l + 1, rope)
        want = O.loader_assemble(
            _bits(layers[l]), slots.numpy(), bs, apc, alloc_end,
            [(s, t, _bits(hosts[i, l])) for i, (s, t, _) in enumerate(segs)],
            relocate=reloc if moved else None,
        )
        got = _bits(buf)
        if dtype == torch.float16 and moved:
            np.testing.assert_array_equal(got[1], want[1], err_msg=f"V layer {l}")
            np.testing.assert_array_equal(got[0][~relocated], want[0][~relocated], err_msg=f"K layer {l}")
            np.testing.assert_allclose(got[0][relocated].view(np.float16).astype(np.float32),
                                       want[0][relocated].view(np.float16).astype(np.float32),
                                       rtol=2e-3, atol=2e-3, err_msg=f"relocated K layer {l}")
        else:
            np.testing.assert_array_equal(got, want, err_msg=f"layer {l}")
        expect_pages = _bits(layers[l]).copy()
        fresh = torch.randn(buf.shape, dtype=torch.float32).to(dtype).to(DEV)
        O.loader_commit(_bits(fresh), expect_pages, slots.numpy(), bs, apc, alloc_end)
        buf.copy_(fresh)
        loader.commit(l, buf)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bits(layers[l]), expect_pages, err_msg=f"commit layer {l}")


def test_loader_without_relocation_is_a_bit_copy():
    heads, dim, bs, chunk = 2, 64, 16, 32
    segs = [(40, 40, 64), (200, 200, 32)]  # source == target
    layers, store, plan, slots, hosts = _blend_setup(1, 64, bs, heads, dim, 0, segs, 300,
                                                     torch.float16, chunk, seed=3)
    src_map, old, relocate = build_source_map(plan)
    assert not relocate and (src_map[:40] == -1).all()
    loader = PagedBlendLoader(layers, store, "req", plan, slots, bs, _cfg(chunk_size=chunk))
    loader.prefetch(0, Rope(dim, 512, True))
    buf = loader.get(0)
    want = O.loader_assemble(_bits(layers[0]), slots.numpy(), bs, 0, 300,
                             [(s, t, _bits(hosts[i, 0])) for i, (s, t, _) in enumerate(segs)])
    np.testing.assert_array_equal(_bits(buf), want)


def _full_blend_span(allocation_end=32767, apc=2048, seed=0):
    """The Qwen3-30B-A3B blend span: 12 reused segments of 256-token
    multiples after a 2048-token APC prefix, separated by 1-511-token gaps,
    the rest of the span a trailing gap. (source_start, target_start, length)."""
    rng = np.random.default_rng(seed)
    gaps = rng.integers(1, 512, 12)
    chunks_total = (allocation_end - apc - int(gaps.sum())) // 256
    lens = 1 + rng.multinomial(chunks_total - 12, np.full(12, 1 / 12))
    segs, pos, src = [], apc, 0
    for g, m in zip(gaps, lens):
        pos += int(g)
        segs.append((src, pos, 256 * int(m)))
        src += 256 * int(m) + 512
        pos += 256 * int(m)
    return segs


def test_loader_blend_load_full_span_both_paths():
    """The whole Qwen3-30B-A3B blend span (allocation_end 32767, 2048-token
    APC prefix, 12 hit segments, 4 KV heads x 128 bf16, 16-token blocks) over
    2 layers, on both transfer paths: DMA into the hit ring ("auto" picks it,
    each segment's plane is one host run of >= 256 KiB) and the assembly
    reading the pinned chunks in place. Every assembled buffer and the pages
    after each commit equal the oracle's, bit for bit."""
    A, APC, bs = 32767, 2048, 16
    segs = _full_blend_span(A, APC)
    assert segs[-1][1] + segs[-1][2] < A and sum(n for *_, n in segs) > 25000
    nb = (A + bs - 1) // bs + 64
    layers, store, plan, slots, hosts = _blend_setup(2, nb, bs, 4, 128, APC, segs, A,
                                                     torch.bfloat16, 256, seed=5)
    rope = Rope(128, 65536, True, base=1e6)
    cache = rope.cos_sin_cache.cpu().numpy()

    def reloc(old, new, k_bits):
        k = O.bf16_to_f32(k_bits).reshape(k_bits.shape[0], -1)
        return O.f32_to_bf16(O.relocate_key(cache, old, new, k, 128, True, bf16=True)).reshape(k_bits.shape)

    want = [O.loader_assemble(_bits(layers[l]), slots.numpy(), bs, APC, A,
                              [(s, t, _bits(hosts[i, l])) for i, (s, t, _) in enumerate(segs)],
                              relocate=reloc) for l in range(2)]
    # the commit writes [apc:] only, so a second load assembles the same buffers
    pages = [_bits(layers[l]).copy() for l in range(2)]
    for l in range(2):
        O.loader_commit(want[l], pages[l], slots.numpy(), bs, APC, A)
    for zero_copy in ("auto", True):
        loader = PagedBlendLoader(layers, store, "req", plan, slots, bs, _cfg(), zero_copy=zero_copy)
        loader.prefetch(0, rope)
        for l in range(2):
            buf = loader.get(l)
            loader.prefetch(l + 1, rope)
            np.testing.assert_array_equal(_bits(buf), want[l], err_msg=f"{zero_copy} layer {l}")
            loader.commit(l, buf)
        torch.cuda.synchronize()
        for l in range(2):
            np.testing.assert_array_equal(_bits(layers[l]), pages[l], err_msg=f"{zero_copy} commit {l}")
        # "auto" takes DMA for these runs; True reads the chunks in place
        assert (len(loader._zc_layers) > 0) == (zero_copy is True)
