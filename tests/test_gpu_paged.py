"""GPU parity: paged gather/scatter kernels against the oracle, bit-exact."""

import numpy as np
import pytest
import torch

import oracle as O
from cacheblend_vllm import kv_layout as KL
from cacheblend_vllm import synthetic

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _np(t: torch.Tensor) -> np.ndarray:
    """Bit pattern view on the host (bf16/f16 as uint16, 8-bit floats as
    uint8, f32 as f32)."""
    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.element_size() == 1 and t.dtype != torch.uint8:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def _layout(base: torch.Tensor, layout: str):
    if layout == "merged_first":
        return base.clone()
    if layout == "merged_block":
        return base.transpose(0, 1).contiguous()
    return [base[0].clone(), base[1].clone()]


def _oracle_layer(paged):
    if isinstance(paged, list):
        return [_np(p) for p in paged]
    return _np(paged)


@pytest.mark.parametrize("layout", ["merged_first", "merged_block", "separate"])
def test_reference_known_answer_round_trip(golden, layout):
    case = golden["kv_layout_round_trip"]
    base = torch.arange(24, dtype=torch.float32).reshape(case["base_shape"]).to(DEV)
    paged = _layout(base, layout)
    slots = torch.tensor(case["slots"])
    got = KL.gather_paged_kv(paged, slots, case["block_size"])
    assert got.cpu().tolist() == case["expected_gather"]
    replacement = torch.full_like(got, case["scatter_value"])
    KL.scatter_paged_kv(replacement, paged, slots, case["block_size"])
    assert torch.equal(KL.gather_paged_kv(paged, slots, case["block_size"]), replacement)


def test_reference_known_answer_out_is_filled_and_returned(golden):
    case = golden["kv_layout_out"]
    paged = torch.arange(24, dtype=torch.float32).reshape(case["paged_shape"]).to(DEV)
    out = torch.empty(case["out_shape"], device=DEV)
    result = KL.gather_paged_kv(paged, torch.tensor(case["slots"]), case["block_size"], out=out)
    assert result is out
    assert out.cpu().tolist() == case["expected"]


CASES = [
    # (layout, dtype, num_blocks, block_size, heads, head_dim, tokens)
    ("separate", torch.float32, 64, 16, 2, 64, 512),       # CPU-plumbing workload
    ("merged_first", torch.bfloat16, 512, 16, 8, 128, 2048),
    ("merged_block", torch.bfloat16, 300, 16, 4, 128, 1000),
    ("merged_first", torch.float16, 40, 16, 3, 5, 333),    # 30-byte rows -> 2-byte vectors
    ("separate", torch.bfloat16, 33, 32, 1, 64, 1),
    ("merged_first", torch.float32, 10, 8, 5, 7, 80),      # 140-byte rows -> 4-byte vectors
    # 1 KiB rows are whole waves (scalar slot loads); 3 and 37 tokens leave
    # dead waves in the last workgroup of both launch shapes
    ("merged_first", torch.bfloat16, 64, 16, 4, 128, 3),
    ("separate", torch.bfloat16, 40, 16, 8, 64, 37),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{str(c[1])[6:]}-{c[5]}x{c[4]}-T{c[6]}")
def test_gather_scatter_bit_exact_vs_oracle(case):
    layout, dtype, nb, bs, h, d, tokens = case
    torch.manual_seed(0)
    base = torch.randn(2, nb, bs, h, d, device=DEV).to(dtype)
    paged = _layout(base, layout)
    perm = torch.randperm(nb * bs)
    slots = perm[:tokens]
    print(f"case={case}", flush=True)

    got = KL.gather_paged_kv(paged, slots, bs)
    want = O.gather_paged_kv(_oracle_layer(paged), slots.numpy(), bs)
    np.testing.assert_array_equal(_np(got), want)

    # device-resident slots take the same path
    got_dev = KL.gather_paged_kv(paged, slots.to(DEV), bs)
    assert torch.equal(got_dev.view(torch.uint8), got.view(torch.uint8))

    # scatter fresh rows to a different set of slots, compare the whole cache
    fresh = torch.randn_like(got, dtype=torch.float32).to(dtype)
    new_slots = perm[-tokens:]
    expect = _oracle_layer(paged)
    O.scatter_paged_kv(_np(fresh), expect, new_slots.numpy(), bs)
    KL.scatter_paged_kv(fresh, paged, new_slots, bs)
    if isinstance(paged, list):
        for p, e in zip(paged, expect):
            np.testing.assert_array_equal(_np(p), e)
    else:
        np.testing.assert_array_equal(_np(paged), expect)


def test_empty_and_reusable_output():
    paged = torch.zeros(2, 4, 16, 2, 64, dtype=torch.bfloat16, device=DEV)
    empty = KL.gather_paged_kv(paged, torch.empty(0, dtype=torch.long), 16)
    assert empty.shape == (2, 0, 2, 64)
    KL.scatter_paged_kv(empty, paged, torch.empty(0, dtype=torch.long), 16)
    out = torch.empty(2, 5, 2, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="gather output has shape"):
        KL.gather_paged_kv(paged, torch.arange(4), 16, out=out)
    with pytest.raises(ValueError, match="dtype and device"):
        KL.gather_paged_kv(paged, torch.arange(5), 16, out=out.float())


def test_strided_output_goes_through_staging():
    torch.manual_seed(1)
    paged = torch.randn(2, 8, 16, 2, 64, device=DEV).to(torch.bfloat16)
    slots = torch.randperm(128)[:40]
    big = torch.zeros(2, 40, 2, 128, dtype=torch.bfloat16, device=DEV)
    out = big[..., :64]  # row not contiguous with the token stride
    KL.gather_paged_kv(paged, slots, 16, out=out)
    want = O.gather_paged_kv(_np(paged), slots.numpy(), 16)
    np.testing.assert_array_equal(_np(out.contiguous()), want)
    assert torch.count_nonzero(big[..., 64:]) == 0


def test_out_of_range_slots():
    paged = torch.ones(2, 4, 16, 1, 8, device=DEV)
    with pytest.raises(IndexError):
        KL.gather_paged_kv(paged, torch.tensor([0, 64]), 16)
    with pytest.raises(IndexError):
        KL.scatter_paged_kv(torch.zeros(2, 1, 1, 8, device=DEV), paged, torch.tensor([-1]), 16)
    # device slots are not read back: a bad row gathers zeros, never faults
    got = KL.gather_paged_kv(paged, torch.tensor([1, 99, 2], device=DEV), 16)
    assert got[:, 1].abs().sum().item() == 0 and got[:, 0].sum().item() == 16
    # the same with 1 KiB rows, whose slot is one wave-uniform load
    wide = torch.ones(2, 4, 16, 4, 128, dtype=torch.bfloat16, device=DEV)
    got = KL.gather_paged_kv(wide, torch.tensor([1, 99, 2, -5], device=DEV), 16)
    assert got[:, 1].abs().sum().item() == 0 and got[:, 3].abs().sum().item() == 0
    assert got[:, 0].float().sum().item() == 2 * 512 and got[:, 2].float().sum().item() == 2 * 512
    KL.scatter_paged_kv(torch.zeros(2, 2, 4, 128, dtype=torch.bfloat16, device=DEV), wide,
                        torch.tensor([3, 640], device=DEV), 16)
    flat = wide.view(2, 64, 512)
    assert flat[:, 3].abs().sum().item() == 0 and flat.float().sum().item() == 2 * 63 * 512


def test_multi_layer_gather_scatter_round_trip():
    torch.manual_seed(2)
    layers = [synthetic.paged_pool(256, 16, 8, 128, torch.bfloat16, DEV, seed=s) for s in range(5)]
    blocks = torch.randperm(256)
    slots = synthetic.block_slots(blocks[:64], 16, 1000)
    got = KL.gather_paged_kv_layers(layers, slots, 16)
    for i, layer in enumerate(layers):
        assert torch.equal(got[i].view(torch.int16), KL.gather_paged_kv(layer, slots, 16).view(torch.int16))
    new_slots = synthetic.block_slots(blocks[64:128], 16, 1000)
    KL.scatter_paged_kv_layers(got, layers, new_slots, 16)
    again = KL.gather_paged_kv_layers(layers, new_slots, 16)
    assert torch.equal(again.view(torch.int16), got.view(torch.int16))
    # scatter left the source blocks alone
    src = KL.gather_paged_kv_layers(layers, slots, 16)
    assert torch.equal(src.view(torch.int16), got.view(torch.int16))


@pytest.mark.parametrize("num_layers", [64, 65, 130])
def test_multi_layer_copies_across_launches(num_layers):
    """At most 64 layers go in one launch: 64 is one, 65 two, 130 three (the
    last one of 2 layers). Every layer of the gather equals the oracle's, and
    the scatter writes every layer's pages."""
    layers = [synthetic.paged_pool(24, 16, 1, 64, torch.bfloat16, DEV, seed=100 + s) for s in range(num_layers)]
    perm = torch.randperm(24, generator=torch.Generator().manual_seed(num_layers))
    slots = synthetic.block_slots(perm[:8], 16, 120)
    got = KL.gather_paged_kv_layers(layers, slots.to(DEV), 16)
    assert got.shape == (num_layers, 2, 120, 1, 64)
    for i, layer in enumerate(layers):
        np.testing.assert_array_equal(_np(got[i]), O.gather_paged_kv(_np(layer), slots.numpy(), 16),
                                      err_msg=f"layer {i}")
    fresh = torch.randn(got.shape, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(DEV)
    new_slots = synthetic.block_slots(perm[8:16], 16, 120)
    want = [_np(layer).copy() for layer in layers]
    for i in range(num_layers):
        O.scatter_paged_kv(_np(fresh[i]), want[i], new_slots.numpy(), 16)
    KL.scatter_paged_kv_layers(fresh, layers, new_slots.to(DEV), 16)
    torch.cuda.synchronize()
    for i, layer in enumerate(layers):
        np.testing.assert_array_equal(_np(layer), want[i], err_msg=f"scatter layer {i}")


def test_store_workload_round_trip_full_size():
    """Qwen3-8B store shape per layer: 4096-block pool, 8 KV heads x 128,
    an 8192-token prompt in random blocks, gathered and scattered back into
    fresh random blocks: the round trip must reproduce every bit."""
    pool = synthetic.paged_pool(4096, 16, 8, 128, torch.bfloat16, DEV, seed=3)
    perm = torch.randperm(4096)
    slots = synthetic.block_slots(perm[:512], 16, 8192)
    new_slots = synthetic.block_slots(perm[512:1024], 16, 8192)
    chunks = KL.gather_paged_kv(pool, slots, 16)
    host = torch.empty(chunks.shape, dtype=chunks.dtype, pin_memory=True)
    host.copy_(chunks, non_blocking=True)
    torch.cuda.synchronize()
    KL.scatter_paged_kv(host, pool, new_slots, 16)
    back = KL.gather_paged_kv(pool, new_slots, 16)
    assert torch.equal(back.view(torch.int16), chunks.view(torch.int16))
    # checksum of checksums against the oracle on a sample of tokens
    sample = torch.randperm(8192)[:256]
    want = O.gather_paged_kv(_np(pool), slots[sample].numpy(), 16)
    np.testing.assert_array_equal(_np(chunks[:, sample]), want)


_RANDOM_DTYPES = [torch.uint8, torch.bfloat16, torch.float16, torch.float32] + (
    [torch.float8_e4m3fn] if hasattr(torch, "float8_e4m3fn") else [])


@pytest.mark.parametrize("seed", range(12))
def test_gather_scatter_random_shapes(seed):
    """Seeded random layouts, dtypes (8-bit float KV caches included), block
    sizes, head shapes and token counts, with random bit patterns (NaNs
    included): the copies move bytes, bit-exact against the oracle."""
    rng = np.random.default_rng(1000 + seed)
    layout = ["merged_first", "merged_block", "separate"][int(rng.integers(3))]
    dtype = _RANDOM_DTYPES[seed % len(_RANDOM_DTYPES)]
    nb = int(rng.integers(2, 300))
    bs = int(rng.choice([1, 8, 16, 32]))
    h = int(rng.integers(1, 9))
    d = int(rng.choice([7, 64, 96, 128, 256]))
    tokens = int(rng.integers(1, min(nb * bs, 3000) + 1))
    print(f"seed={seed} layout={layout} dtype={dtype} nb={nb} bs={bs} h={h} d={d} tokens={tokens}", flush=True)
    g = torch.Generator().manual_seed(seed)
    es = torch.empty((), dtype=dtype).element_size()
    raw = torch.randint(0, 256, (2 * nb * bs * h * d * es,), dtype=torch.uint8, generator=g)
    base = raw.view(dtype).reshape(2, nb, bs, h, d).to(DEV)
    paged = _layout(base, layout)
    perm = torch.randperm(nb * bs, generator=g)
    slots = perm[:tokens]
    got = KL.gather_paged_kv(paged, slots.to(DEV), bs)
    want = O.gather_paged_kv(_oracle_layer(paged), slots.numpy(), bs)
    assert np.array_equal(_np(got).view(np.uint8), np.ascontiguousarray(want).view(np.uint8))
    fresh_raw = torch.randint(0, 256, (got.numel() * es,), dtype=torch.uint8, generator=g)
    fresh = fresh_raw.view(dtype).reshape(got.shape).to(DEV)
    new_slots = perm[-tokens:]
    expect = _oracle_layer(paged)
    O.scatter_paged_kv(_np(fresh), expect, new_slots.numpy(), bs)
    KL.scatter_paged_kv(fresh, paged, new_slots, bs)
    for p_, e in (zip(paged, expect) if isinstance(paged, list) else [(paged, expect)]):
        assert np.array_equal(_np(p_).view(np.uint8), np.ascontiguousarray(e).view(np.uint8))
