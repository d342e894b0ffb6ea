"""HIP graph capture of the per-layer kernels a serving loop repeats: the
Sparse-Q scores and the side-forward attention each captured once (after an
eager call), then replayed several times with other eager work of the same
kind in between, every replay equal to the eager result bit for bit (both
kernels sum in a fixed order, and none of their launches is a memset)."""

import pytest
import torch

from cacheblend_vllm import selection as S
from cacheblend_vllm.attention import blend_attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _replays(graph, outputs, want, other, reps=4):
    for rep in range(reps):
        print(f"graph replay {rep}", flush=True)
        for o in outputs:
            o.fill_(float("nan"))
        other()
        graph.replay()
        torch.cuda.synchronize()
        for o, w in zip(outputs, want):
            assert torch.equal(o, w), f"replay {rep} differs from the eager result"


def test_sparse_q_scores_replay_in_a_hip_graph():
    g = torch.Generator().manual_seed(11)
    nk, n_active, hq, hkv, d = 3000, 600, 8, 2, 128
    q = (torch.randn(n_active, hq, d, generator=g) / d ** 0.5).to(torch.bfloat16).to(DEV)
    k = (torch.randn(nk, hkv, d, generator=g) / d ** 0.5).to(torch.bfloat16).to(DEV)
    absolute = torch.arange(nk - n_active, nk, device=DEV)
    rows = torch.arange(0, n_active, 3, device=DEV)
    out_index = torch.arange(0, nk, 2, device=DEV)
    scale = d ** -0.5
    want = [t.clone() for t in S.sparse_q_full_scores(q, k, rows, absolute, scale, out_index, want_full=True)]
    q_other = q.flip(0).contiguous()
    rows_other = torch.arange(1, n_active, 2, device=DEV)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out, full = S.sparse_q_full_scores(q, k, rows, absolute, scale, out_index, want_full=True)
    _replays(graph, [out, full], want,
             lambda: S.sparse_q_full_scores(q_other, k, rows_other, absolute, scale, want_full=True))


def test_blend_attention_replays_in_a_hip_graph():
    g = torch.Generator().manual_seed(12)
    nq, nk, hq, hkv, d = 500, 4000, 16, 4, 128
    q = torch.randn(nq, hq, d, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(nk, hkv, d, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(nk, hkv, d, generator=g).to(torch.bfloat16).to(DEV)
    pos = torch.randperm(nk, generator=g)[:nq].sort().values.to(DEV)
    scale = d ** -0.5
    want = blend_attention(q, k, v, pos, scale).clone()
    q_other = q.flip(0).contiguous()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = blend_attention(q, k, v, pos, scale)
    _replays(graph, [out], [want], lambda: blend_attention(q_other, k, v, pos, scale))
