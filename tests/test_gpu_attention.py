"""GPU parity: side-forward attention of the selected queries against the
oracle: every output within 1e-2 of the L1 size of the terms it sums,
sum_k p_k |v_k| (the oracle returns it). The kernel rounds the unnormalized
probabilities of each key block to bf16 (flash style) where the reference
rounds the normalized ones; either rounding moves a term by up to 2^-9 of
itself, so the bound is relative to the terms, not to an output that may
have cancelled to near zero.

The parity cases use queries and keys with entries in {-1, 0, 1} / 8, whose
dot products are exact in float32 and in bf16/f16: the kernel and the oracle
then round identical logits, and what remains is float32 summation order and
the rounding of the probabilities. With N(0,1) inputs the dot products reach
~45, where a bf16 ulp is 0.25: a dot product within float32 accumulation
error of a rounding boundary can round either way (in the reference's own
torch matmul as well), moving that key's weight by ~2%. That case is checked
separately: each element within the tolerance plus the most such logits of
its row can move it."""

import numpy as np
import pytest
import torch

import oracle as O
from cacheblend_vllm.attention import blend_attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
RTOL = 1e-2


def _case(nq, nk, hq, hkv, d, dtype, seed, sorted_positions=True, exact_dots=True):
    g = torch.Generator().manual_seed(seed)
    if exact_dots:
        q = (torch.randint(-1, 2, (nq, hq, d), generator=g) / 8).to(dtype)
        k = (torch.randint(-1, 2, (nk, hkv, d), generator=g) / 8).to(dtype)
    else:
        q = torch.randn(nq, hq, d, generator=g).to(dtype)
        k = torch.randn(nk, hkv, d, generator=g).to(dtype)
    v = torch.randn(nk, hkv, d, generator=g).to(dtype)
    pos = torch.randperm(nk, generator=g)[:nq]
    if sorted_positions:
        pos = pos.sort().values
    return q, k, v, pos


def _oracle(q, k, v, pos, scale, rounding="bf16"):
    return O.blend_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), pos.numpy(), scale,
                             rounding, return_mass=True)


def _check(got, want_mass, label):
    want, mass = want_mass
    err = np.abs(got.float().cpu().numpy() - want)
    ratio = err / np.maximum(mass, 1e-30)
    print(f"{label}: max |err| / sum p|v| = {ratio.max():.3e}", flush=True)
    assert np.all(err <= RTOL * mass + 1e-7)


@pytest.mark.parametrize("dtype,hq,hkv,d", [
    (torch.bfloat16, 32, 4, 128),
    (torch.bfloat16, 8, 8, 64),
    (torch.float16, 16, 2, 128),
    (torch.bfloat16, 12, 4, 64),   # G = 3: row tiles straddle queries unevenly
    (torch.float16, 8, 2, 64),
])
def test_blend_attention_matches_oracle(dtype, hq, hkv, d):
    nq, nk = 300, 1500
    q, k, v, pos = _case(nq, nk, hq, hkv, d, dtype, seed=hq + d)
    scale = 1.5  # logits up to ~ +-3: peaked rows as well as flat ones
    got = blend_attention(q.to(DEV), k.to(DEV), v.to(DEV), pos, scale)
    want = _oracle(q, k, v, pos, scale, "bf16" if dtype == torch.bfloat16 else "f16")
    _check(got, want, f"{dtype} hq={hq} hkv={hkv} d={d}")


def test_blend_attention_unsorted_positions_strided_views_and_f32():
    # queries in any order; q/k/v as views of wider rows (qkv split / layer buffer)
    nq, nk, hq, hkv, d = 97, 777, 8, 2, 128
    q, k, v, pos = _case(nq, nk, hq, hkv, d, torch.bfloat16, seed=5, sorted_positions=False)
    qkv = torch.cat([q.reshape(nq, -1), torch.zeros(nq, 64, dtype=torch.bfloat16)], dim=1).to(DEV)
    buf = torch.stack([k, v]).to(DEV)  # [2, nk, hkv, d]
    got = blend_attention(qkv[:, : hq * d].view(nq, hq, d), buf[0], buf[1], pos.to(DEV), d ** -0.5)
    _check(got, _oracle(q, k, v, pos, d ** -0.5), "bf16 strided")
    q32, k32, v32, pos32 = _case(64, 300, 4, 2, 64, torch.float32, seed=6)
    got32 = blend_attention(q32.to(DEV), k32.to(DEV), v32.to(DEV), pos32, 0.125)
    want32 = O.blend_attention(q32.numpy(), k32.numpy(), v32.numpy(), pos32.numpy(), 0.125, None)
    np.testing.assert_allclose(got32.cpu().numpy(), want32, rtol=1e-4, atol=1e-5)


def test_blend_attention_closed_forms_and_errors():
    nk, hkv, d = 200, 2, 128
    g = torch.Generator().manual_seed(9)
    v = torch.randn(nk, hkv, d, generator=g).to(torch.bfloat16)
    k = torch.randn(nk, hkv, d, generator=g).to(torch.bfloat16)
    q = torch.randn(3, 8, d, generator=g).to(torch.bfloat16)
    pos = torch.tensor([0, 0, 0])  # one visible key: the output is that value row exactly
    got = blend_attention(q.to(DEV), k.to(DEV), v.to(DEV), pos, d ** -0.5)
    want = v[0].repeat_interleave(4, dim=0)  # head h reads KV head h // 4
    assert torch.equal(got.cpu(), want.expand(3, 8, d))
    with pytest.raises(IndexError):
        blend_attention(q.to(DEV), k.to(DEV), v.to(DEV), torch.tensor([0, 1, nk]), 1.0)
    with pytest.raises(ValueError, match="divisible"):
        blend_attention(q[:, :3].contiguous().to(DEV), k.to(DEV), v.to(DEV), pos, 1.0)
    assert blend_attention(q[:0].to(DEV), k.to(DEV), v.to(DEV), pos[:0], 1.0).shape == (0, 8, d)


def _rounding_allowance(q, k, v, pos, scale, mass):
    """Per output element, the most that logits whose bf16 rounding the inputs
    do not fix can move it. A logit is unfixed when its exact dot product lies
    within (D - 1) * 2^-24 * sum_i |q_i k_i| of a bf16 rounding midpoint -- the
    first-order error bound of any order of fp32 additions of the D exact bf16
    products -- so an fp32 sum in another order (the reference's torch matmul
    and the MFMA sum add in different orders) may land on either side. Flipping it moves the
    rounded dot by one bf16 ulp u, the logit w = r(r(dot) * scale) by at most
    u * scale + ulp(w), its probability p_k by a factor up to e^dw, and the
    other probabilities by the renormalisation; so an output element moves by
    at most sum_k p_k (e^dw_k - 1) (|v_k| + mass) over the row's unfixed keys."""
    qf, kf, vf = q.double().numpy(), k.double().numpy(), v.double().numpy()
    nq, hq, d = qf.shape
    g = hq // kf.shape[1]
    visible = pos.numpy()[:, None] >= np.arange(kf.shape[0])[None, :]
    allow = np.zeros((nq, hq, d))
    unfixed_rows = 0
    for h in range(hq):
        kh, vh = kf[:, h // g, :], np.abs(vf[:, h // g, :])
        dot = qf[:, h, :] @ kh.T
        err = (d - 1) * 2.0 ** -24 * (np.abs(qf[:, h, :]) @ np.abs(kh).T)
        bits = np.abs(dot).astype(np.float32).view(np.uint32) & np.uint32(0xFFFF0000)
        lo = bits.view(np.float32).astype(np.float64)
        ulp = (bits + np.uint32(0x10000)).view(np.float32).astype(np.float64) - lo
        unfixed = visible & (np.abs(np.abs(dot) - (lo + ulp / 2)) <= err)
        unfixed_rows += int(unfixed.any(axis=1).sum())
        w = O.round_bf16(O.round_bf16(dot) * np.float32(scale)).astype(np.float64)
        w = np.where(visible, w, -np.inf)
        e = np.exp(w - w.max(axis=1, keepdims=True))
        p = e / e.sum(axis=1, keepdims=True)
        ulp_w = np.abs(w) * 2.0 ** -7  # a bf16 ulp of the logit, at most
        dw = ulp * scale + np.where(visible, ulp_w, 0.0)
        move = np.where(unfixed, p * np.expm1(dw), 0.0)               # [nq, nk]
        allow[:, h, :] = move @ vh + move.sum(axis=1, keepdims=True) * mass[:, h, :]
    return allow, unfixed_rows


def test_blend_attention_gaussian_inputs_rounding_boundary_bound():
    """N(0,1) queries/keys (unscaled, |dot| up to ~45, where a bf16 ulp is
    0.25): every output element within the parity tolerance plus what the
    row's logits with an unfixed rounding can move it (_rounding_allowance)."""
    nq, nk, hq, hkv, d = 300, 1500, 32, 4, 128
    q, k, v, pos = _case(nq, nk, hq, hkv, d, torch.bfloat16, seed=21, exact_dots=False)
    got = blend_attention(q.to(DEV), k.to(DEV), v.to(DEV), pos, d ** -0.5).float().cpu().numpy()
    want, mass = _oracle(q, k, v, pos, d ** -0.5)
    allow, unfixed_rows = _rounding_allowance(q.float(), k.float(), v.float(), pos, d ** -0.5, mass)
    err = np.abs(got - want)
    ratio = err / np.maximum(mass, 1e-30)
    outside = err > RTOL * mass + 1e-7
    print(f"gaussian: {int(outside.sum())} elements outside the tolerance, {unfixed_rows} of "
          f"{nq * hq} rows with an unfixed rounding, max ratio {ratio.max():.3e}", flush=True)
    assert np.all(err <= RTOL * mass + allow + 1e-7)
    assert ratio.max() < 5e-2


def test_blend_attention_full_blend_layer_properties():
    """The blend-layer shape (7000 selected queries over 32,767 keys, 32 query
    heads on 4 KV heads of 128 bf16): with every key's value equal to one
    vector c per KV head, each output row is c exactly (the probabilities sum
    to one); with values +c / -c split by key parity the output stays within
    [-|c|, |c|]; and the launch is deterministic."""
    nq, nk, hq, hkv, d = 7000, 32767, 32, 4, 128
    g = torch.Generator(device=DEV).manual_seed(5)
    q = (torch.randn((nq, hq, d), generator=g, device=DEV) / d ** 0.25).to(torch.bfloat16)
    k = (torch.randn((nk, hkv, d), generator=g, device=DEV) / d ** 0.25).to(torch.bfloat16)
    pos = torch.from_numpy(np.sort(np.random.default_rng(5).choice(np.arange(2048, nk), nq, replace=False))).to(DEV)
    c = (torch.randn((hkv, d), generator=g, device=DEV)).to(torch.bfloat16)
    v = c[None].expand(nk, hkv, d).contiguous()
    out = blend_attention(q, k, v, pos, d ** -0.5)
    want = c.repeat_interleave(hq // hkv, dim=0)[None].expand(nq, hq, d)
    assert torch.equal(out, want)
    sign = torch.where(torch.arange(nk, device=DEV) % 2 == 0, 1.0, -1.0).to(torch.bfloat16)
    v2 = (v * sign[:, None, None]).contiguous()
    out2 = blend_attention(q, k, v2, pos, d ** -0.5)
    bound = want.float().abs() * (1 + 2 ** -7)
    assert bool((out2.float().abs() <= bound).all())
    assert torch.equal(out2, blend_attention(q, k, v2, pos, d ** -0.5))


@pytest.mark.parametrize("nq,nk,d", [(1, 1, 128), (3, 5, 64), (20, 31, 128), (40, 32, 128), (50, 33, 64),
                                     (64, 65, 128), (7, 97, 64)])
def test_blend_attention_partial_key_blocks(nq, nk, d):
    """Contexts of 1 to 97 keys: the last 32-key block is partial, its rows
    past the context repeat the last key in LDS and must stay masked."""
    hq, hkv = 8, 2
    q, k, v, pos = _case(min(nq, nk), nk, hq, hkv, d, torch.bfloat16, seed=nq * 131 + nk)
    print(f"nq={q.shape[0]} nk={nk} d={d}", flush=True)
    got = blend_attention(q.to(DEV), k.to(DEV), v.to(DEV), pos, 0.7)
    _check(got, _oracle(q, k, v, pos, 0.7, "bf16"), f"nq={q.shape[0]} nk={nk} d={d}")


@pytest.mark.parametrize("nk,d", [(31, 128), (33, 64), (97, 128)])
def test_blend_attention_device_positions_past_the_context(nk, d):
    """Positions on the device are not checked on the host: one at or past
    the last key sees every key, as the reference's mask (key <= position
    over the nk keys) has it -- the last block's rows past nk, which repeat
    its last key in LDS, stay masked."""
    hq, hkv = 8, 2
    q, k, v, _ = _case(6, nk, hq, hkv, d, torch.bfloat16, seed=nk + d)
    pos = torch.tensor([nk - 1, nk, nk + 5, 1 << 20, 0, nk // 2])
    got = blend_attention(q.to(DEV), k.to(DEV), v.to(DEV), pos.to(DEV), 0.7)
    _check(got, _oracle(q, k, v, pos, 0.7, "bf16"), f"nk={nk} d={d} positions past the context")
    same = blend_attention(q.to(DEV), k.to(DEV), v.to(DEV), pos.clamp(max=nk - 1).to(DEV), 0.7)
    assert torch.equal(got, same)


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float16, 128), (torch.bfloat16, 64)])
@pytest.mark.parametrize("slope", [4.0, 2.0])
def test_blend_attention_rising_row_maxima(dtype, d, slope):
    """Logits that rise along the keys: the running maximum is raised block
    after block (every block over the first 320 keys, every few blocks over
    the next 512), then stays; half of the heads see the logits falling
    instead (a maximum in the first block, never raised). Exact dots: q is
    +-1/8 in every dim, key j is t_j / 8 in every dim, so q.k_j = +-d t_j / 64
    (scale 64 slope / d: logits +-slope t_j at both head sizes). At slope 4 the
    rising rows climb 112 above their first block (161 in log2 units): their
    terms overflow the first block's reference and the kernel recomputes them
    with the lazy rescaling; at slope 2 they climb 81 log2 units and stay on
    the fixed reference, with terms up to 2^81."""
    nq, nk, hq, hkv = 200, 1200, 8, 2
    g = torch.Generator().manual_seed(77)
    j = torch.arange(nk)
    t = torch.where(j < 320, j // 16 - 16, 4 + (j - 320) // 64)
    t = torch.where(j < 832, t, torch.randint(-16, 13, (nk,), generator=g))
    k = (t[:, None, None] / 8).expand(nk, hkv, d).to(dtype)
    sign = torch.tensor([1.0, -1.0]).repeat(hq // 2)
    q = (sign[None, :, None] / 8).expand(nq, hq, d).to(dtype)
    v = torch.randn(nk, hkv, d, generator=g).to(dtype)
    pos = torch.randperm(nk, generator=g)[:nq].sort().values
    scale = 64.0 * slope / d  # the same logits at both head sizes
    got = blend_attention(q.to(DEV), k.to(DEV), v.to(DEV), pos, scale)
    rounding = "bf16" if dtype == torch.bfloat16 else "f16"
    _check(got, _oracle(q, k, v, pos, scale, rounding), f"rising maxima {dtype} d={d} slope={slope}")


@pytest.mark.parametrize("seed", range(24))
def test_blend_attention_random_shapes(seed):
    """Seeded random shapes: 1-200 queries at sorted or unsorted positions
    over 1-1500 keys, 1-8 query heads per KV head, head_dim 64 or 128, bf16
    or f16, scales from 0.05 to 2."""
    rng = np.random.default_rng(500 + seed)
    nk = int(rng.integers(1, 1501))
    nq = int(rng.integers(1, min(nk, 200) + 1))
    hkv = int(rng.choice([1, 2, 4]))
    hq = hkv * int(rng.choice([1, 2, 3, 4, 8]))
    d = int(rng.choice([64, 128]))
    dtype = [torch.bfloat16, torch.float16][seed % 2]
    scale = float(rng.uniform(0.05, 2.0))
    sorted_positions = bool(rng.integers(2))
    q, k, v, pos = _case(nq, nk, hq, hkv, d, dtype, seed=seed, sorted_positions=sorted_positions)
    label = f"seed={seed} nq={nq} nk={nk} hq={hq} hkv={hkv} d={d} {dtype} scale={scale:.3f} sorted={sorted_positions}"
    print(label, flush=True)
    got = blend_attention(q.to(DEV), k.to(DEV), v.to(DEV), pos, scale)
    _check(got, _oracle(q, k, v, pos, scale, "bf16" if dtype == torch.bfloat16 else "f16"), label)
