"""Pins the torch CPU restatement that bench.py times as the CPU baseline
against the numpy oracle, so the baseline runs the same work the GPU path
is checked against."""

import numpy as np
import torch

import oracle as O
from oracle import torch_cpu_path as ref


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_gather_scatter_kdev_select_dilate():
    g = torch.Generator().manual_seed(1)
    pages = torch.randn(2, 16, 4, 2, 8, generator=g).to(torch.bfloat16)
    slots = torch.randperm(64, generator=g)[:40]
    got = ref.gather(pages, slots, 4)
    np.testing.assert_array_equal(_bits(got), O.gather_paged_kv(_bits(pages), slots.numpy(), 4))
    dst = torch.randperm(64, generator=g)[:40]
    want = _bits(pages).copy()
    O.scatter_paged_kv(_bits(got), want, dst.numpy(), 4)
    ref.scatter(got, pages, dst, 4)
    np.testing.assert_array_equal(_bits(pages), want)
    fresh, cached = torch.randn(300, 64, generator=g), torch.randn(300, 64, generator=g)
    scores = ref.kdev_scores(fresh, cached)
    np.testing.assert_allclose(scores.numpy(), O.kdev_scores(fresh.numpy(), cached.numpy()), rtol=1e-5)
    gap = torch.rand(300, generator=g) < 0.2
    np.testing.assert_array_equal(ref.dilate(gap, 5).numpy(), O.dilate(gap.numpy(), 5))
    # distinct scores: torch.topk's choice is the oracle's
    forced = ref.dilate(gap, 5)
    np.testing.assert_array_equal(ref.select(scores, gap, 0.2, forced).numpy(),
                                  O.select(scores.numpy(), gap.numpy(), 0.2, forced.numpy()))


def _rope_cache(head, max_pos):
    inv = 1.0 / (10000 ** (np.arange(0, head, 2) / head))
    ang = np.arange(max_pos)[:, None] * inv[None, :]
    return np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)


def test_relocate_and_blend_load_layer_bit_exact_vs_oracle():
    g = torch.Generator().manual_seed(2)
    bs, nb, h, d = 4, 40, 2, 16
    pages = torch.randn(2, nb, bs, h, d, generator=g).to(torch.bfloat16)
    slots = torch.randperm(nb * bs, generator=g)
    cache = _rope_cache(d, 256)
    hosts_t = [(0, 10, torch.randn(2, 8, h, d, generator=g).to(torch.bfloat16)),
               (40, 25, torch.randn(2, 12, h, d, generator=g).to(torch.bfloat16))]
    apc, end = 6, 45
    before = _bits(pages).copy()
    for neox in (True, False):
        pages_n = pages.clone()
        buf = ref.blend_load_layer(pages_n, slots, bs, apc, end, hosts_t, torch.from_numpy(cache), d, neox)

        def reloc(old, new, k_bits):
            k = O.bf16_to_f32(k_bits).reshape(k_bits.shape[0], -1)
            return O.f32_to_bf16(O.relocate_key(cache, old, new, k, d, neox, bf16=True)).reshape(k_bits.shape)

        hosts = [(s, t, _bits(x)) for s, t, x in hosts_t]
        want = O.loader_assemble(before, slots.numpy(), bs, apc, end, hosts, relocate=reloc)
        np.testing.assert_array_equal(_bits(buf), want)
        expect = before.copy()
        O.loader_commit(want, expect, slots.numpy(), bs, apc, end)
        np.testing.assert_array_equal(_bits(pages_n), expect)


def test_sparse_q_full_scores_vs_oracle():
    g = torch.Generator().manual_seed(3)
    q = (torch.randn(20, 8, 32, generator=g) / 32 ** 0.5).to(torch.bfloat16)
    k = (torch.randn(300, 2, 32, generator=g) / 32 ** 0.5).to(torch.bfloat16)
    pos = torch.sort(torch.randperm(300, generator=g)[:20]).values
    got = ref.sparse_q_full_scores(q, k, pos, 32 ** -0.5, chunk=8)
    want = O.sparse_q_full_scores(q.float().numpy(), k.float().numpy(), pos.numpy(), 32 ** -0.5,
                                  round_logits_bf16=True, chunk=8)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-2, atol=1e-6)
    assert abs(float(got.sum()) - 20 * 8) < 1e-2      # every softmax row sums to one
