#!/usr/bin/env python3
"""Benchmark of the CacheBlend KV data-movement and selection path on one MI355X.

Headline workload (one "step"): the Qwen3-8B-shaped KV offload -- 36 layers,
8 KV heads x 128 bf16, vLLM block_size 16, a 4096-block merged_first pool
per layer, an 8192-token prompt in randomly permuted blocks. A step gathers
every layer's prompt KV into contiguous [layer, K/V, 8192, 8, 128] staging
(one launch) and scatters it back into freshly chosen random blocks (one
launch). Inputs are resident in HBM when the timed region starts.

  value   = algorithmic bytes per step / time per step   (GB/s)
            = (gather read + write + scatter read + write)
            = 4 x 1,207,959,552 B per step
  roofline: the gather kernel, HIP events on the launch stream, against
            8 TB/s HBM3E peak

Also reported (same JSON line): the per-layer launch form of the same copy
(the connector's save_kv_layer granularity), pinned-host D2H / H2D rates of
the staging (host link), the K-deviation selection latency over a 65,536-token
span (4 KV heads x 128 bf16, ratio 0.15, overflow 1 block), and the
reference's torch path timed on the host cores (cpu_baseline).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "pic-kvcache_amd"))

HBM_PEAK_GBPS = 8000.0
HOST_LINK_PEAK_GBPS = 64.0  # PCIe 5.0 x16 per direction


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--skip-cpu-baseline", action="store_true")
    p.add_argument("--skip-extras", action="store_true", help="only the headline copy step")
    p.add_argument("--profile", action="store_true",
                   help="run each kernel --steps times and exit (for rocprofv3 runs)")
    p.add_argument("--profile-store", action="store_true",
                   help="run the 36-layer store pipeline (dma mode) 4 times and exit "
                        "(for rocprofv3 timeline runs; CACHEBLEND_ROCTX=1 marks its phases)")
    return p.parse_args()


PROFILE_SUMMARY = os.path.join(ROOT, "profiles", "paged_copy_qwen3_8b_store.md")


def profiled_traffic() -> int | None:
    """HBM bytes per gather launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE x 2 + WRITE_SIZE, calibrated on a plain copy of known size)."""
    try:
        with open(PROFILE_SUMMARY) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        return None
    return None


def queued_time_ms(torch, fn, reps: int, cycles_per_us: float) -> tuple[float, float]:
    """(device ms per call, host enqueue ms per call) of ``reps`` calls of fn
    on the current stream. The calls are enqueued behind a spin kernel that
    outlasts their enqueueing, so the events time the device back to back
    from a full queue, whatever the host's speed."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    host_ms = (time.perf_counter() - t0) * 1e3
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int((2.0 * host_ms + 1.0) * 1e3 * cycles_per_us))
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / reps, host_ms / reps


def event_time_ms(torch, fn, reps: int) -> float:
    """Average device time of fn() measured with HIP events on the current stream."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / reps


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
            "(this path has no cross-GPU work: each GPU gathers/scatters its own KV shard)",
            file=sys.stderr,
        )
        return 2

    import torch

    from cacheblend_vllm import kv_layout as KL
    from cacheblend_vllm import selection as S
    from cacheblend_vllm import synthetic

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    L, NB, BS, H, D, T = 36, 4096, 16, 8, 128, 8192
    dtype = torch.bfloat16
    log(f"allocating {L} layers of [2,{NB},{BS},{H},{D}] bf16")
    layers = [synthetic.paged_pool(NB, BS, H, D, dtype, dev, seed=l) for l in range(L)]
    g = torch.Generator().manual_seed(0)
    perm = torch.randperm(NB, generator=g)
    src_slots = synthetic.block_slots(perm[:512], BS, T).to(dev)
    dst_slots = synthetic.block_slots(perm[512:1024], BS, T).to(dev)
    cache = KL.PagedKVCache(layers, BS)
    staging = torch.empty((L, 2, T, H, D), dtype=dtype, device=dev)
    layer_bytes = 2 * T * H * D * 2  # K+V of one layer
    copy_bytes = L * layer_bytes  # 1,207,959,552
    step_bytes = 4 * copy_bytes

    def step():
        cache.gather(src_slots, out=staging)
        cache.scatter(staging, dst_slots)

    if args.profile:
        return profile_run(torch, S, synthetic, cache, src_slots, dst_slots, staging, args, dev)
    if args.profile_store:
        return profile_store_run(torch, layers, cache, src_slots)

    # correctness guard on the real workload before timing: round trip
    step()
    torch.cuda.synchronize()
    check = cache.gather(dst_slots)
    if not torch.equal(check.view(torch.int16), staging.view(torch.int16)):
        log("round-trip mismatch: gather(new slots) != staged prompt KV")
        return 1
    del check

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed / args.steps * 1e3
    value = step_bytes / (elapsed / args.steps) / 1e9
    log(f"step: {ms_per_step:.3f} ms, {value:.1f} GB/s")

    # dominant kernel: the multi-layer gather, timed alone with HIP events
    gather_ms = event_time_ms(torch, lambda: cache.gather(src_slots, out=staging), args.steps)
    scatter_ms = event_time_ms(torch, lambda: cache.scatter(staging, dst_slots), args.steps)
    achieved = 2 * copy_bytes / (gather_ms / 1e3) / 1e9
    scatter_gbps = 2 * copy_bytes / (scatter_ms / 1e3) / 1e9
    log(f"gather kernel {gather_ms*1e3:.1f} us ({achieved:.0f} GB/s); scatter {scatter_ms*1e3:.1f} us ({scatter_gbps:.0f} GB/s)")

    result = {
        "metric": "paged KV gather/scatter GB/s (% HBM peak); K-deviation select us per 64K tokens",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) KV pool, random block permutation)",
        "config": {
            "workload": "Qwen3-8B-shaped KV offload: gather all layers of an 8192-token prompt "
                        "from random vLLM blocks into [layer,K/V,8192,8,128] staging, scatter into new random blocks",
            "layers": L, "kv_heads": H, "head_dim": D, "block_size": BS,
            "pool_blocks": NB, "prompt_tokens": T, "kv_layout": "merged_first [2,NB,bs,H,D]",
        },
        "roofline": {
            "kernel": "paged_copy_kernel<16,gather> (36 layers, one launch)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": profiled_traffic(),
            "traffic_source": "profiles/paged_copy_qwen3_8b_store.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE)",
            "launch_us": round(gather_ms * 1e3, 2),
            "algorithmic_bytes": 2 * copy_bytes,
        },
        "scatter_kernel": {"GBps": round(scatter_gbps, 1), "launch_us": round(scatter_ms * 1e3, 2),
                           "frac": round(scatter_gbps / HBM_PEAK_GBPS, 4)},
    }

    if not args.skip_extras:
        reload_slots = synthetic.block_slots(perm[1024:1536], BS, T).to(dev)
        result.update(extras(torch, KL, S, synthetic, layers, cache, src_slots, staging, args, dev,
                             reload_slots, (gather_ms, scatter_ms)))
        result.update(_headline_scalars(result))

    if not args.skip_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(torch, synthetic)
    print(json.dumps(result), flush=True)
    return 0


def extras(torch, KL, S, synthetic, layers, cache, src_slots, staging, args, dev, reload_slots,
           all_layer_ms):
    out = {}
    L = len(layers)
    BS = cache.block_size
    layer_bytes = staging[0].numel() * staging.element_size()

    # per-layer launches (the connector's granularity: save_kv_layer
    # gathers one layer, a reload or commit scatters one), device time per
    # layer, beside a plain device copy of the same bytes per launch (layer l
    # into layer l + L/2 of the staging, so every copy reads what was written
    # half a rotation, 1.2 GB, earlier: nothing comes from the 256 MB
    # last-level cache). Against the all-layer launch of the same kernel,
    # t(1 layer) = fixed + x and t(36 layers) = fixed + 36 x split each launch
    # into its fixed cost (ramp, drain, the gap to the next launch) and the
    # streaming rate between them
    def per_layer():
        for l in range(L):
            cache.gather(src_slots, out=staging[l:l + 1], layers=(l, l + 1))

    reps = max(3, args.steps // 4)
    ms = event_time_ms(torch, per_layer, reps)
    per_layer_scatter_slots = reload_slots

    def per_layer_scatter():
        for l in range(L):
            cache.scatter(staging[l:l + 1], per_layer_scatter_slots, layers=(l, l + 1))

    ms_s = event_time_ms(torch, per_layer_scatter, reps)

    def plain_copies():
        for l in range(L):
            staging[(l + L // 2) % L].copy_(staging[l])

    ms_c = event_time_ms(torch, plain_copies, reps)
    ceiling = 2 * L * layer_bytes / (ms_c / 1e3) / 1e9

    def per_layer_entry(ms_total, ms_all_layers):
        us1 = ms_total * 1e3 / L
        stream_us = (ms_all_layers * 1e3 - us1) / (L - 1)
        gb = 2 * layer_bytes / (us1 / 1e6) / 1e9
        return {"GBps": round(gb, 1), "us_per_layer": round(us1, 2),
                "frac_of_hbm_peak": round(gb / HBM_PEAK_GBPS, 4),
                "frac_of_same_size_copy": round(gb / ceiling, 4),
                "launch_fixed_us": round(us1 - stream_us, 2),
                "streaming_GBps": round(2 * layer_bytes / (stream_us / 1e6) / 1e9, 1)}

    out["per_layer_gather"] = per_layer_entry(ms, all_layer_ms[0])
    out["per_layer_scatter"] = per_layer_entry(ms_s, all_layer_ms[1])
    out["per_layer_plain_copy"] = {"GBps": round(ceiling, 1), "us_per_copy": round(ms_c * 1e3 / L, 2),
                                   "bytes_per_copy": 2 * layer_bytes}
    log(f"per-layer gather: {out['per_layer_gather']}, scatter {out['per_layer_scatter']}, "
        f"plain copy {out['per_layer_plain_copy']}")

    # host link: pinned D2H / H2D of the whole staging (1.2 GB)
    host = torch.empty(staging.shape, dtype=staging.dtype, pin_memory=True)
    d2h_ms = event_time_ms(torch, lambda: host.copy_(staging, non_blocking=True), 3)
    h2d_ms = event_time_ms(torch, lambda: staging.copy_(host, non_blocking=True), 3)
    nbytes = staging.numel() * staging.element_size()
    d2h = nbytes / (d2h_ms / 1e3) / 1e9
    h2d = nbytes / (h2d_ms / 1e3) / 1e9
    out["host_link"] = {"d2h_GBps": round(d2h, 2), "h2d_GBps": round(h2d, 2),
                        "peak_GBps": HOST_LINK_PEAK_GBPS,
                        "d2h_frac": round(d2h / HOST_LINK_PEAK_GBPS, 4),
                        "h2d_frac": round(h2d / HOST_LINK_PEAK_GBPS, 4), "bytes": nbytes}
    log(f"host link: {out['host_link']}")
    del host

    # K-deviation selection: 65,536 tokens, 4 KV heads x 128 bf16, 20% gaps
    n = 65536
    fresh, cached, gap = synthetic.kdev_inputs(n, 4, 128, torch.bfloat16, dev, seed=0)
    lib_sel = lambda: S.kdev_select(fresh, cached, None, gap, 0.15, radius=16)  # noqa: E731
    selected, _ = lib_sel()
    reps = 50
    dev_ms, enqueue_ms = queued_time_ms(torch, lambda: _kdev_async(torch, S, fresh, cached, gap), reps,
                                        _sleep_cycles_per_us(torch))
    t0 = time.perf_counter()
    for _ in range(reps):
        lib_sel()
    wall_ms = (time.perf_counter() - t0) / reps * 1e3
    read_bytes = 2 * n * 512 * 2
    score_ms = event_time_ms(torch, lambda: S.kdev_scores(fresh, cached), reps)
    out["kdev_select"] = {
        "us_per_64k_tokens": round(dev_ms * 1e3, 2),
        "host_enqueue_us": round(enqueue_ms * 1e3, 2),
        "wall_us_with_count_readback": round(wall_ms * 1e3, 2),
        "score_kernel_us": round(score_ms * 1e3, 2),
        "score_kernel_GBps": round(read_bytes / (score_ms / 1e3) / 1e9, 1),
        "selected": int(selected.numel()),
        "tokens": n, "ratio": 0.15, "overflow_radius": 16,
    }
    log(f"kdev select: {out['kdev_select']}")
    del fresh, cached, gap

    out["sparse_q"] = sparse_q(torch, S, synthetic, dev)
    log(f"sparse_q: {out['sparse_q']}")
    out["blend_attention"] = blend_attention_bench(torch, dev)
    log(f"blend attention: {out['blend_attention']}")
    out["store_pipeline"] = store_pipeline(torch, layers, cache, src_slots, args, reload_slots)
    log(f"store pipeline: {out['store_pipeline']}")
    out["blend_load"] = blend_load(torch, synthetic, dev, args)
    log(f"blend load: {out['blend_load']}")
    out["token_matcher"] = token_matcher_bench(args)
    log(f"token matcher: {out['token_matcher']}")
    return out


def _headline_scalars(r: dict) -> dict:
    """Each configuration's headline figure as a top-level scalar (readers of
    the JSON line that keep scalars only still see them)."""
    out = {}

    def put(name, *path):
        node = r
        for key in path:
            if not isinstance(node, dict) or key not in node:
                return
            node = node[key]
        out[name] = node

    put("scatter_frac", "scatter_kernel", "frac")
    put("per_layer_gather_frac", "per_layer_gather", "frac_of_hbm_peak")
    put("per_layer_scatter_frac", "per_layer_scatter", "frac_of_hbm_peak")
    put("host_link_d2h_frac", "host_link", "d2h_frac")
    put("host_link_h2d_frac", "host_link", "h2d_frac")
    put("kdev_us_per_64k", "kdev_select", "us_per_64k_tokens")
    put("kdev_score_kernel_us", "kdev_select", "score_kernel_us")
    put("sparse_q_ms", "sparse_q", "score_ms")
    put("sparse_q_ms_min", "sparse_q", "score_ms_min")
    put("sparse_q_mfma_frac", "sparse_q", "mfma_frac_of_bf16_peak")
    put("sparse_q_qwen3_8b_ms", "sparse_q", "other_group_sizes", "qwen3_8b_32q_8kv", "ms")
    put("sparse_q_qwen3_14b_ms", "sparse_q", "other_group_sizes", "qwen3_14b_40q_8kv", "ms")
    put("attention_ms", "blend_attention", "ms")
    put("attention_ms_min", "blend_attention", "ms_min")
    put("attention_mfma_frac", "blend_attention", "mfma_frac_of_bf16_peak")
    # the store's default transfer (StoreStreamWriter slab_transfer="dma")
    put("store_d2h_GBps", "store_pipeline", "dma", "d2h_GBps")
    put("store_d2h_GBps_mean", "store_pipeline", "dma", "d2h_GBps_mean")
    put("store_host_link_frac", "store_pipeline", "dma", "host_link_frac")
    put("store_hidden_frac", "store_pipeline", "with_gemm_compute", "dma", "store_hidden_frac")
    put("reload_h2d_GBps", "store_pipeline", "reload_h2d", "h2d_GBps")
    put("reload_host_link_frac", "store_pipeline", "reload_h2d", "host_link_frac")
    put("blend_load_h2d_GBps", "blend_load", "dma", "h2d_GBps")
    put("blend_load_host_link_frac", "blend_load", "dma", "host_link_frac")
    put("blend_load_hidden_frac", "blend_load", "dma", "busy_wait", "load_hidden_frac")
    put("commit_scatter_frac", "blend_load", "commit_scatter", "frac_of_hbm_peak")
    return out


def token_matcher_bench(args, n_tokens=131072, n_chunks=512, chunk=256):
    """Scheduler lookup (host code): find 256-token stored chunks at any
    offset of a 128K-token prompt, half of it made of registered chunks
    placed at unaligned offsets. The oracle's leg evaluates every window
    hash on its own (the reference's sliding-window product) and verifies
    candidates in Python."""
    import numpy as np

    from cacheblend_vllm.matcher import TokenRangeMatcher

    rng = np.random.default_rng(0)
    prompt = rng.integers(0, 152_000, size=n_tokens)
    chunks = rng.integers(0, 152_000, size=(n_chunks, chunk))
    matcher = TokenRangeMatcher(chunk)
    for i in range(n_chunks):
        matcher.register(matcher.make_record("bench", i * chunk, chunks[i].tolist()))
    at = 17
    for i in range(0, n_chunks, 2):  # every other chunk, 3 tokens apart
        if at + chunk > n_tokens:
            break
        prompt[at:at + chunk] = chunks[i]
        at += chunk + 3 + chunk
    tokens = prompt.tolist()  # the scheduler holds prompt ids as a Python list
    found = matcher.match("bench", tokens)
    reps = 20
    t0 = time.perf_counter()
    for _ in range(reps):
        matcher.match("bench", tokens)
    ms = (time.perf_counter() - t0) / reps * 1e3
    t0 = time.perf_counter()
    for _ in range(reps):
        matcher.match("bench", prompt)
    ms_array = (time.perf_counter() - t0) / reps * 1e3
    out = {"prompt_tokens": n_tokens, "registered_chunks": n_chunks, "chunk": chunk,
           "matches": len(found), "ms_per_lookup": round(ms, 3),
           "ms_per_lookup_int64_array": round(ms_array, 3)}
    if not args.skip_cpu_baseline:
        import oracle as O

        records = [("bench", O.content_hash(c), tuple(int(t) for t in c)) for c in chunks]
        t0 = time.perf_counter()
        ref = O.match_tokens(records, "bench", tokens, 0, chunk)
        out["cpu_baseline_ms"] = round((time.perf_counter() - t0) * 1e3, 3)
        out["cpu_baseline_kind"] = "port"
        if [(s, i) for s, i in ref] != [(m.target_start, m.source_start // chunk) for m in found]:
            raise RuntimeError("token matcher disagrees with the oracle")
    return out


def sparse_q(torch, S, synthetic, dev):
    """Sparse-Q scoring at Qwen3-30B-A3B layer 6: 32 query heads over 4 KV
    heads x 128 bf16, Q/K ~ N(0,1)/sqrt(128); 4096 non-reused query tokens in
    gap runs over a 98,304-token causal key context (the last run ends at the
    last token); per-key attention mass summed over heads, then the top 15% of
    cached keys plus gaps and overflow blocks."""
    from cacheblend_vllm.config import CacheBlendConfig

    nk, hq, hkv, d, nq = 98304, 32, 4, 128, 4096
    g = torch.Generator(device=dev).manual_seed(0)
    query = (torch.randn((nk, hq, d), generator=g, device=dev) / d ** 0.5).to(torch.bfloat16)
    key = (torch.randn((nk, hkv, d), generator=g, device=dev) / d ** 0.5).to(torch.bfloat16)
    gap_np = synthetic.sparse_q_layout(nk, nq, seed=0)
    gap = torch.from_numpy(gap_np).to(dev)
    absolute = torch.arange(nk, device=dev)
    rows = torch.nonzero(gap).flatten()
    pos = np.flatnonzero(gap_np)
    flops_pass = 2.0 * d * hq * float((pos + 1).sum())
    scale = d ** -0.5
    fn = lambda: S.sparse_q_full_scores(query, key, rows, absolute, scale, out_index=absolute)  # noqa: E731
    # steady state: after 8 calls (the first rounds after only two ran up to
    # 9% slower), the mean of 5 rounds of 3 calls, the fastest round beside it
    for _ in range(8):
        fn()
    rounds = [event_time_ms(torch, fn, 3) for _ in range(5)]
    ms, ms_min = statistics.fmean(rounds), min(rounds)
    sel = S.BlendSelector(CacheBlendConfig.from_extra_config(
        {"selection_strategy": "sparse_q", "check_layers": [1]}), 16)
    sel.sparse_q_select(query, key, absolute, gap, scale, 1)  # first call: workspaces, code loading
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        selected, stats = sel.sparse_q_select(query, key, absolute, gap, scale, 1)
    torch.cuda.synchronize()
    total_ms = (time.perf_counter() - t0) / 3 * 1e3
    # algorithmic work: one Q.K^T over the unmasked logits (2 D Hq sum(pos+1));
    # the kernel pair computes the logits twice (row statistics, then column
    # sums), reported separately as executed work
    achieved = flops_pass / (ms / 1e3) / 1e12
    # the same positions at other query-head groupings of Qwen3 layers (a
    # kernel variant per group size): 4 query heads per KV head (Qwen3-8B,
    # 32 over 8), 5 (Qwen3-14B, 40 over 8), 2 (Qwen3-1.7B, 16 over 8)
    del query, key
    other_groups = {}
    for name, ghq, ghkv in (("qwen3_8b_32q_8kv", 32, 8), ("qwen3_14b_40q_8kv", 40, 8),
                            ("qwen3_1p7b_16q_8kv", 16, 8)):
        gq = (torch.randn((nk, ghq, d), generator=g, device=dev) / d ** 0.5).to(torch.bfloat16)
        gk = (torch.randn((nk, ghkv, d), generator=g, device=dev) / d ** 0.5).to(torch.bfloat16)
        gfn = lambda: S.sparse_q_full_scores(gq, gk, rows, absolute, scale, out_index=absolute)  # noqa: E731
        for _ in range(8):
            gfn()
        gms = statistics.fmean([event_time_ms(torch, gfn, 3) for _ in range(3)])
        gflops = 2.0 * d * ghq * float((pos + 1).sum())
        other_groups[name] = {"ms": round(gms, 3),
                              "mfma_frac_of_bf16_peak": round(gflops / (gms / 1e3) / 1e12 / 2500.0, 4)}
        del gq, gk
    return {
        "queries": nq, "keys": nk, "q_heads": hq, "kv_heads": hkv, "head_dim": d,
        "score_ms": round(ms, 3),
        "score_ms_min": round(ms_min, 3),
        "score_ms_rounds": [round(r, 3) for r in rounds],
        "algorithmic_flops": flops_pass,
        "TFLOPs": round(achieved, 1),
        "mfma_frac_of_bf16_peak": round(achieved / 2500.0, 4),
        "mfma_frac_of_bf16_peak_min_time": round(flops_pass / (ms_min / 1e3) / 1e12 / 2500.0, 4),
        "executed_two_pass_TFLOPs": round(2 * achieved, 1),
        "exp_per_s": round(2 * hq * float((pos + 1).sum()) / (ms / 1e3), 1),
        "select_total_ms_with_masks_and_sync": round(total_ms, 3),
        "selected": int(selected.numel()),
        "other_group_sizes": other_groups,
    }


def _attention_inputs(torch, dev, nq=7000, nk=32767):
    """Qwen3-30B-A3B blend layer after selection: 7000 selected queries (about
    the gaps plus 15% of the cached tokens of the blend-load prompt) at
    sorted uniform positions in [2048, 32767), 32 query heads over the layer
    buffer's 32767 keys of 4 KV heads x 128 bf16; Q, K ~ N(0,1)/128^(1/4)."""
    hq, hkv, d = 32, 4, 128
    g = torch.Generator(device=dev).manual_seed(0)
    q = (torch.randn((nq, hq, d), generator=g, device=dev) / d ** 0.25).to(torch.bfloat16)
    k = (torch.randn((nk, hkv, d), generator=g, device=dev) / d ** 0.25).to(torch.bfloat16)
    v = torch.randn((nk, hkv, d), generator=g, device=dev).to(torch.bfloat16)
    pos = np.sort(np.random.default_rng(0).choice(np.arange(2048, nk), nq, replace=False))
    return q, k, v, torch.from_numpy(pos).to(dev), pos


def blend_attention_bench(torch, dev):
    """Side-forward attention of the selected queries (_attention_inputs):
    QK^T and PV flops = 4 * D * Hq * sum(pos + 1) over the causal logits."""
    from cacheblend_vllm.attention import blend_attention

    q, k, v, pos, pos_np = _attention_inputs(torch, dev)
    d, hq = q.shape[2], q.shape[1]
    flops = 4.0 * d * hq * float((pos_np + 1).sum())
    fn = lambda: blend_attention(q, k, v, pos, d ** -0.5)  # noqa: E731
    # steady state: after 8 calls, the mean of 5 rounds of 3 calls, the
    # fastest round beside it
    for _ in range(8):
        fn()
    rounds = [event_time_ms(torch, fn, 3) for _ in range(5)]
    ms, ms_min = statistics.fmean(rounds), min(rounds)
    achieved = flops / (ms / 1e3) / 1e12
    return {"queries": q.shape[0], "keys": k.shape[0], "q_heads": hq, "kv_heads": k.shape[1], "head_dim": d,
            "ms": round(ms, 3), "ms_min": round(ms_min, 3), "ms_rounds": [round(r, 3) for r in rounds],
            "flops": flops, "TFLOPs": round(achieved, 1),
            "mfma_frac_of_bf16_peak": round(achieved / 2500.0, 4),
            "mfma_frac_of_bf16_peak_min_time": round(flops / (ms_min / 1e3) / 1e12 / 2500.0, 4)}


def store_pipeline(torch, layers, cache, src_slots, args, reload_slots):
    """Qwen3-8B layerwise store: save_kv_layer for all 36 layers of the
    8192-token prompt (32 chunks of 256) through the Store stream, timed from
    the first save to the end of wait_for_save (publication of every chunk
    into the host store included), in three modes:
    host_write -- pinned slab slots allocated as consecutive runs, written by
                  the gather kernel directly over the host link;
    dma        -- (the writer's default) the same slots; gather into a
                  chunk-major device staging, then (copier thread, Copy
                  stream) one copy command per run of slots;
    reference  -- gather into device staging + one D2H into a freshly pinned
                  per-layer batch (the reference's scheme).
    One store and writer per mode serve every repetition, as the connector
    keeps its writer for the life of the process (the first repetition
    starts the writer's copier and publisher threads and is reported apart).
    Also timed with the saves interleaved with bf16 GEMMs on the serving
    stream (about 1.5x the per-layer transfer time per layer), as a prefill
    would interleave them. Then the reload: the stored chunks scattered back
    over the host link into fresh random blocks (``reload_slots``), one
    ``scatter_chunks`` launch per layer, checked bit-exact."""
    from cacheblend_vllm.host_store import PinnedChunkSlab, PinnedChunkStore
    from cacheblend_vllm.store_path import RequestMetadata, StoreStreamWriter

    L = len(layers)
    T = src_slots.numel()
    slots_cpu = src_slots.cpu()
    H, D = cache.row_shape
    nbytes = L * 2 * T * H * D * 2
    slab = PinnedChunkSlab((2, 256, H, D), torch.bfloat16, chunks_per_arena=128)
    a = torch.randn(4096, 4096, device=layers[0].device, dtype=torch.bfloat16)
    b = torch.randn_like(a)
    c = torch.empty_like(a)
    rep_id = [0]

    writers = {}  # one store and writer per mode for the whole run, as a connector keeps them

    def once(mode, gemms=0):
        use_slab = mode != "reference"
        if mode not in writers:
            store = PinnedChunkStore(256, 1 << 40, on_release=slab.free if use_slab else None)
            writers[mode] = (store, StoreStreamWriter(store, cache.block_size, 256, L, "bench", store_workers=2,
                                                      slab=slab if use_slab else None,
                                                      slab_transfer=mode if use_slab else "dma"))
        store, writer = writers[mode]
        r = rep_id[0]
        rep_id[0] += 1
        request = RequestMetadata(f"{mode}{r}", list(range(r * T, r * T + T)), slots_cpu, None, True, T)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for l in range(L):
            for _ in range(gemms):
                torch.mm(a, b, out=c)
            writer.save_layer(l, layers[l], [request])
        writer.wait_for_save()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        committed = sum(store.is_committed(sid) for _, sid in writer._chunk_ids[request.request_id])
        store.clear()
        return elapsed, committed

    result = {"layers": L, "tokens": T, "bytes_d2h": nbytes}
    for mode in ("host_write", "dma", "reference"):
        times = [once(mode) for _ in range(4)]
        steady = [t for t, _ in times[1:]]  # rep 0 also pins the slab's arenas / warms the pools
        best, mean = min(steady), statistics.fmean(steady)
        result[mode] = {"ms": round(best * 1e3, 3), "mean_ms": round(mean * 1e3, 3),
                        "first_rep_ms": round(times[0][0] * 1e3, 3),
                        "chunks_committed": times[-1][1], "d2h_GBps": round(nbytes / best / 1e9, 2),
                        "d2h_GBps_mean": round(nbytes / mean / 1e9, 2),
                        "host_link_frac": round(nbytes / best / 1e9 / HOST_LINK_PEAK_GBPS, 4),
                        "host_link_frac_mean": round(nbytes / mean / 1e9 / HOST_LINK_PEAK_GBPS, 4)}
    # overlap with compute
    torch.mm(a, b, out=c)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        torch.mm(a, b, out=c)
    torch.cuda.synchronize()
    gemm_s = (time.perf_counter() - t0) / 20
    per_layer = result["host_write"]["ms"] / 1e3 / L
    reps = max(1, int(round(1.5 * per_layer / gemm_s)))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(L * reps):
        torch.mm(a, b, out=c)
    torch.cuda.synchronize()
    compute_s = time.perf_counter() - t0
    result["with_gemm_compute"] = {"compute_only_ms": round(compute_s * 1e3, 3),
                                   "compute_per_layer": f"{reps} x bf16 GEMM 4096^3"}
    for mode in ("host_write", "dma"):
        once(mode, reps)
        total = min(once(mode, reps)[0] for _ in range(2))
        alone = result[mode]["ms"] / 1e3
        result["with_gemm_compute"][mode] = {
            "total_ms": round(total * 1e3, 3),
            "store_hidden_frac": round(1.0 - max(0.0, total - compute_s) / alone, 4)}
    for _, writer in writers.values():
        writer.close()
    # reload: the stored chunks (pinned slab slots) scattered back over the
    # host link into fresh random blocks, one scatter_chunks launch per layer
    from cacheblend_vllm.kv_layout import scatter_chunks
    from cacheblend_vllm.types import BlendSegment

    store = PinnedChunkStore(256, 1 << 40, on_release=slab.free)
    writer = StoreStreamWriter(store, cache.block_size, 256, L, "bench", store_workers=2, slab=slab)
    request = RequestMetadata("reload", list(range(10**6, 10**6 + T)), slots_cpu, None, True, T)
    for l in range(L):
        writer.save_layer(l, layers[l], [request])
    writer.wait_for_save()
    segments = [BlendSegment(sid, start) for start, sid in writer._chunk_ids["reload"]]
    store.pin("reload", segments)
    chunks = [[store.get_layer("reload", seg, l) for seg in segments] for l in range(L)]

    def reload():
        for l in range(L):
            scatter_chunks(chunks[l], layers[l], reload_slots, cache.block_size)

    reload()
    torch.cuda.synchronize()
    same = all(torch.equal(cache.gather(reload_slots, layers=(l, l + 1)).view(torch.int16),
                           cache.gather(src_slots, layers=(l, l + 1)).view(torch.int16)) for l in (0, L - 1))
    if not same:
        raise RuntimeError("reload round trip is not bit-exact")
    times = []
    for _ in range(3):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        reload()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    best, mean = min(times), statistics.fmean(times)
    result["reload_h2d"] = {"ms": round(best * 1e3, 3), "mean_ms": round(mean * 1e3, 3),
                            "h2d_GBps": round(nbytes / best / 1e9, 2),
                            "h2d_GBps_mean": round(nbytes / mean / 1e9, 2),
                            "host_link_frac": round(nbytes / best / 1e9 / HOST_LINK_PEAK_GBPS, 4),
                            "launches": L, "bit_exact_layers_checked": [0, L - 1]}
    store.release("reload")
    writer.close()
    store.clear()
    result["slab"] = slab.stats()
    slab.close()
    return result


def _sleep_cycles_per_us(torch) -> float:
    """Clock rate of torch.cuda._sleep's spin kernel, measured."""
    torch.cuda._sleep(1000)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    torch.cuda._sleep(20_000_000)
    e1.record()
    e1.synchronize()
    return 20_000_000 / (e0.elapsed_time(e1) * 1e3)


def _c3_segments(allocation_end: int = 32767, apc: int = 2048) -> list[tuple[int, int, int]]:
    """The Qwen3-30B-A3B blend-load plan: 12 reused segments of 256-token
    multiples after the APC prefix, separated by 1-511-token gaps, the rest of
    the span a trailing gap. Returns (source_start, target_start, length)."""
    rng = np.random.default_rng(0)
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


def blend_load(torch, synthetic, dev, args):
    """Qwen3-30B-A3B blend load: 48 layers, 4 KV heads x 128 bf16, 16-token
    blocks; 32768-token prompt, 2048-token APC prefix, 12 reused segments of
    256-multiples separated by 1-511-token gaps (allocation_end 32767). The
    hit chunks of each layer live in one pinned [2, hit, 4, 128] host tensor.
    Per layer: hits cross the host link, the fused assembly relocates RoPE,
    the commit scatters into the pages. Timed alone and overlapped with a
    per-layer compute on the serving stream of 1.5x the per-layer load time,
    either a busy-wait (one spinning wave) or bf16 GEMMs (every CU busy).
    Both transfer modes are timed -- DMA of the coalesced runs (what "auto"
    picks here) and in-place host reads -- and, for chunks scattered over
    pinned slab slots (what the fused store produces), the "auto" choice."""
    import numpy as np

    from cacheblend_vllm.config import CacheBlendConfig
    from cacheblend_vllm.host_store import PinnedChunkSlab, PinnedChunkStore
    from cacheblend_vllm.loader import PagedBlendLoader
    from cacheblend_vllm.types import BlendPlan, BlendSegment

    L, BS, H, D, A, APC = 48, 16, 4, 128, 32767, 2048
    segs = _c3_segments(A, APC)
    hit = sum(n for _, _, n in segs)
    nb = (A + BS - 1) // BS + 8
    layers = [synthetic.paged_pool(nb, BS, H, D, torch.bfloat16, dev, seed=100 + l) for l in range(L)]
    hosts = [torch.empty((2, hit, H, D), dtype=torch.bfloat16, pin_memory=True) for _ in range(L)]
    for h in hosts:
        h.copy_(torch.randn(h.shape, device=dev, dtype=torch.bfloat16))
    slab = PinnedChunkSlab((2, 256, H, D), torch.bfloat16, chunks_per_arena=256)

    def make_store(layout):
        """layout "views": per-layer [2, hit] host tensors sliced per chunk;
        "slab_runs": one slab run per layer over all chunks, as the store
        path allocates a layer's chunks (consecutive slots); "slab_chunks":
        one slab slot per (chunk, layer) in chunk-major order, so a layer's
        chunks lie 48 slots apart and break at every arena."""
        store = PinnedChunkStore(256, 1 << 40, on_release=None if layout == "views" else slab.free)
        runs = [slab.alloc_run(hit // 256) for _ in range(L)] if layout == "slab_runs" else None
        blend_segments = []
        off = 0
        k = 0
        for i, (s0, t0, n) in enumerate(segs):
            for c in range(0, n, 256):
                sid = store.begin_put("bench", s0 + c, list(range(s0 + c + 7 * i, s0 + c + 7 * i + 256)), L)
                for l in range(L):
                    view = hosts[l][:, off + c : off + c + 256]
                    if layout != "views":
                        slot = runs[l][k] if runs is not None else slab.alloc()
                        slot.copy_(view)
                        view = slot
                    store.put_layer_host(sid, l, view)
                blend_segments.append(BlendSegment(sid, t0 + c))
                k += 1
            off += n
        store.pin("blend", blend_segments)
        return store, BlendPlan(APC, A, hit, tuple(blend_segments))

    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(1))
    slots = synthetic.block_slots(perm[: (A + BS - 1) // BS], BS, A)

    class Rope:
        head_size = rotary_dim = D
        is_neox_style = True
        inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
        cos_sin_cache = torch.cat([(torch.arange(65536, dtype=torch.float32)[:, None] * inv).cos(),
                                   (torch.arange(65536, dtype=torch.float32)[:, None] * inv).sin()], -1).to(dev)

    rope = Rope()
    cfg = CacheBlendConfig.from_extra_config({})
    h2d_bytes = L * hit * 2 * H * D * 2

    def run(store, plan, zero_copy, compute=None):
        loader = PagedBlendLoader(layers, store, "blend", plan, slots, BS, cfg, zero_copy=zero_copy)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        loader.prefetch(0, rope)
        for l in range(L):
            buf = loader.get(l)
            loader.prefetch(l + 1, rope)
            if compute is not None:
                compute()
            loader.commit(l, buf)
        torch.cuda.synchronize()
        return time.perf_counter() - t0, len(loader._zc_layers) == L

    def best(store, plan, zero_copy, compute=None, reps=2):
        run(store, plan, zero_copy, compute)
        results = [run(store, plan, zero_copy, compute) for _ in range(reps)]
        return min(r[0] for r in results), results[0][1]

    contiguous, plan_c = make_store("views")
    dma_s, dma_host_read = best(contiguous, plan_c, "auto")
    read_s, _ = best(contiguous, plan_c, True)
    assert not dma_host_read
    per_layer = dma_s / L

    cycles_per_us = _sleep_cycles_per_us(torch)
    delay_cycles = int(1.5 * per_layer * 1e6 * cycles_per_us)

    def busy():
        torch.cuda._sleep(delay_cycles)

    a = torch.randn(4096, 4096, device=dev, dtype=torch.bfloat16)
    b = torch.randn(4096, 4096, device=dev, dtype=torch.bfloat16)
    c = torch.empty(4096, 4096, device=dev, dtype=torch.bfloat16)
    torch.mm(a, b, out=c)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        torch.mm(a, b, out=c)
    torch.cuda.synchronize()
    reps = max(1, int(round(1.5 * per_layer / ((time.perf_counter() - t0) / 20))))

    def gemms():
        for _ in range(reps):
            torch.mm(a, b, out=c)

    def alone(fn):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(L):
            fn()
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    def overlap(load_s, total_s, compute_s):
        return {"overlapped_ms": round(total_s * 1e3, 3), "compute_only_ms": round(compute_s * 1e3, 3),
                "load_hidden_frac": round(1.0 - max(0.0, total_s - compute_s) / load_s, 4),
                "h2d_GBps_while_hidden": round(h2d_bytes / max(total_s, 1e-9) / 1e9, 2)}

    busy_s, gemm_s = alone(busy), alone(gemms)
    out = {
        "layers": L, "allocation_end": A, "apc_prefix": APC, "hit_tokens": hit, "segments": len(segs),
        "h2d_bytes": h2d_bytes,
        "dma": {"load_only_ms": round(dma_s * 1e3, 3), "h2d_GBps": round(h2d_bytes / dma_s / 1e9, 2),
                "host_link_frac": round(h2d_bytes / dma_s / 1e9 / HOST_LINK_PEAK_GBPS, 4),
                "busy_wait": overlap(dma_s, best(contiguous, plan_c, "auto", busy)[0], busy_s),
                "gemm": overlap(dma_s, best(contiguous, plan_c, "auto", gemms)[0], gemm_s)},
        "host_read": {"load_only_ms": round(read_s * 1e3, 3), "h2d_GBps": round(h2d_bytes / read_s / 1e9, 2),
                      "host_link_frac": round(h2d_bytes / read_s / 1e9 / HOST_LINK_PEAK_GBPS, 4),
                      "busy_wait": overlap(read_s, best(contiguous, plan_c, True, busy)[0], busy_s),
                      "gemm": overlap(read_s, best(contiguous, plan_c, True, gemms)[0], gemm_s)},
        "compute_per_layer": {"busy_wait_us": round(1.5 * per_layer * 1e6, 1),
                              "gemm": f"{reps} x bf16 GEMM 4096^3"},
    }
    contiguous.release("blend")
    del contiguous
    for layout in ("slab_runs", "slab_chunks"):
        store, plan_s = make_store(layout)
        auto_s, auto_host_read = best(store, plan_s, "auto")
        dma_s2, _ = best(store, plan_s, False)
        read_s2, _ = best(store, plan_s, True)
        out[layout] = {
            "auto_mode": "host_read" if auto_host_read else "dma",
            "load_only_ms": round(auto_s * 1e3, 3), "h2d_GBps": round(h2d_bytes / auto_s / 1e9, 2),
            "host_link_frac": round(h2d_bytes / auto_s / 1e9 / HOST_LINK_PEAK_GBPS, 4),
            "dma_GBps": round(h2d_bytes / dma_s2 / 1e9, 2),
            "host_read_GBps": round(h2d_bytes / read_s2 / 1e9, 2),
            "busy_wait": overlap(auto_s, best(store, plan_s, "auto", busy)[0], busy_s),
            "gemm": overlap(auto_s, best(store, plan_s, "auto", gemms)[0], gemm_s),
        }
        log(f"blend load {layout}: {out[layout]}")
        store.release("blend")
        store.clear()
    slab.close()

    # the commit's device scatter alone (loader.commit: [2, apc:A] of the
    # layer buffer into the pages), one launch per layer as the loader issues
    # it, timed with HIP events over back-to-back C-ABI calls
    from cacheblend_vllm import _native
    from cacheblend_vllm.kv_layout import kv_desc

    buf = torch.randn((2, A, H, D), device=dev).to(torch.bfloat16)
    src = buf[:, APC:]
    commit_slots = slots[APC:].to(dev)
    n = commit_slots.numel()
    lib = _native.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    descs = [kv_desc(layers[l], BS)[0] for l in range(L)]
    es = buf.element_size()

    calls = [(src[0].data_ptr(), src[1].data_ptr(), src.stride(1) * es, descs[l], commit_slots.data_ptr(), n,
              None, stream) for l in range(L)]
    scatter = lib.cbk_paged_scatter

    def commit_all():
        for c in calls:
            if scatter(*c):
                _native.check(scatter(*c), "commit scatter")

    ms = event_time_ms(torch, commit_all, 5)
    commit_bytes = 2 * 2 * n * H * D * es  # read + written, K and V
    # a plain device copy of the same bytes per launch, layer l's pool into
    # layer l + 24's (after every check above), so each copy reads a pool
    # last written 1.5 GB earlier
    elems = commit_bytes // 2 // es
    flat = [layer.view(-1) for layer in layers]

    def plain_copies():
        for l in range(L):
            flat[(l + L // 2) % L][:elems].copy_(flat[l][:elems])

    ms_c = event_time_ms(torch, plain_copies, 5)
    gb = L * commit_bytes / (ms / 1e3) / 1e9
    ceiling = L * commit_bytes / (ms_c / 1e3) / 1e9
    out["commit_scatter"] = {"tokens_per_layer": n, "us_per_layer": round(ms * 1e3 / L, 2),
                             "GBps": round(gb, 1), "frac_of_hbm_peak": round(gb / HBM_PEAK_GBPS, 4),
                             "plain_copy_same_bytes_GBps": round(ceiling, 1),
                             "frac_of_same_size_copy": round(gb / ceiling, 4)}
    return out


def profile_store_run(torch, layers, cache, src_slots) -> int:
    """The Qwen3-8B layerwise store of ``store_pipeline`` in its default dma
    mode, 4 repetitions on one writer (the first pins the slab's arenas and
    starts the writer's threads), each from the first save_layer to the end
    of wait_for_save; the stored chunks of the last repetition are checked
    against a gather."""
    from cacheblend_vllm.host_store import PinnedChunkSlab, PinnedChunkStore
    from cacheblend_vllm.kv_layout import gather_paged_kv
    from cacheblend_vllm.store_path import RequestMetadata, StoreStreamWriter
    from cacheblend_vllm.types import BlendSegment

    L, T = len(layers), src_slots.numel()
    H, D = cache.row_shape
    slots_cpu = src_slots.cpu()
    nbytes = L * 2 * T * H * D * 2
    slab = PinnedChunkSlab((2, 256, H, D), torch.bfloat16, chunks_per_arena=128)
    store = PinnedChunkStore(256, 1 << 40, on_release=slab.free)
    writer = StoreStreamWriter(store, cache.block_size, 256, L, "bench", store_workers=2, slab=slab)
    for rep in range(4):
        request = RequestMetadata(f"p{rep}", list(range(rep * T, rep * T + T)), slots_cpu, None, True, T)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for l in range(L):
            writer.save_layer(l, layers[l], [request])
        writer.wait_for_save()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        log(f"store pipeline rep {rep}: {elapsed * 1e3:.3f} ms, {nbytes / elapsed / 1e9:.2f} GB/s")
        if rep == 3:
            segments = [BlendSegment(sid, start) for start, sid in writer._chunk_ids[request.request_id]]
            store.pin("check", segments)
            for l in (0, L - 1):
                want = gather_paged_kv(layers[l], src_slots, cache.block_size).cpu()
                for seg in segments:
                    got = store.get_layer("check", seg, l)
                    if not torch.equal(got, want[:, seg.target_start:seg.target_start + 256]):
                        log(f"stored chunk at {seg.target_start} of layer {l} differs from the gather")
                        return 1
            store.release("check")
        store.clear()
    writer.close()
    return 0


def profile_run(torch, S, synthetic, cache, src_slots, dst_slots, staging, args, dev):
    """Each kernel --steps times, nothing timed here: rocprofv3 measures.
    The plain device copy of the staging (torch's copy kernel, 1,207,959,552 B
    read + written) calibrates the HBM counters."""
    copy_dst = torch.empty_like(staging)
    fresh, cached, gap = synthetic.kdev_inputs(65536, 4, 128, torch.bfloat16, dev, seed=0)
    for _ in range(args.steps):
        cache.gather(src_slots, out=staging)
    for _ in range(args.steps):
        cache.scatter(staging, dst_slots)
    for _ in range(args.steps):
        copy_dst.copy_(staging)
    for _ in range(args.steps):
        _kdev_async(torch, S, fresh, cached, gap)
    del copy_dst, fresh, cached
    # one-layer launches, as the connector issues them: save_kv_layer's
    # gather of one layer, a reload's scatter of one layer (36 of each per step)
    for _ in range(args.steps):
        for l in range(staging.shape[0]):
            cache.gather(src_slots, out=staging[l:l + 1], layers=(l, l + 1))
        for l in range(staging.shape[0]):
            cache.scatter(staging[l:l + 1], dst_slots, layers=(l, l + 1))
    _profile_commit(torch, synthetic, args, dev)
    nk, hq, hkv, d = 98304, 32, 4, 128
    g = torch.Generator(device=dev).manual_seed(0)
    query = (torch.randn((nk, hq, d), generator=g, device=dev) / d ** 0.5).to(torch.bfloat16)
    key = (torch.randn((nk, hkv, d), generator=g, device=dev) / d ** 0.5).to(torch.bfloat16)
    rows = torch.from_numpy(np.flatnonzero(synthetic.sparse_q_layout(nk, 4096, seed=0))).to(dev)
    absolute = torch.arange(nk, device=dev)
    # 8 warm-up calls, then the steady-state calls (the bench line times the
    # same sequence: 8 calls, then its timed rounds)
    for _ in range(8 + max(5, args.steps // 2)):
        S.sparse_q_full_scores(query, key, rows, absolute, d ** -0.5, out_index=absolute)
    del query, key
    from cacheblend_vllm.attention import blend_attention

    aq, ak, av, apos, _ = _attention_inputs(torch, dev)
    for _ in range(8 + max(5, args.steps // 2)):
        blend_attention(aq, ak, av, apos, 128 ** -0.5)
    del aq, ak, av
    _profile_host_link(torch, synthetic, cache, src_slots, args, dev)
    torch.cuda.synchronize()
    log(f"profile run done: {args.steps} x (gather, scatter, plain copy, kdev select, one-layer "
        "gathers and scatters, C3 commits, store gather into host chunks, blend assembly from "
        "host chunks), sparse_q, attention")
    return 0


def _profile_commit(torch, synthetic, args, dev):
    """The blend loader's commit at the Qwen3-30B-A3B blend span: the
    [2, 32767, 4, 128] bf16 layer buffer's rows past the 2048-token APC prefix
    (30,719 tokens) scattered into one layer's pages, 8 layers' pools in turn
    (537 MB, past the last-level cache), 8 launches per step."""
    from cacheblend_vllm import kv_layout as KL

    A, APC, BS, H, D = 32767, 2048, 16, 4, 128
    nb = (A + BS - 1) // BS + 8
    pools = [synthetic.paged_pool(nb, BS, H, D, torch.bfloat16, dev, seed=200 + l) for l in range(8)]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(1))
    slots = synthetic.block_slots(perm[: (A + BS - 1) // BS], BS, A).to(dev)
    buf = torch.randn(2, A, H, D, device=dev).to(torch.bfloat16)
    for _ in range(args.steps):
        for pool in pools:
            KL.scatter_paged_kv(buf[:, APC:], pool, slots[APC:], BS)
    torch.cuda.synchronize()


def _profile_host_link(torch, synthetic, cache, src_slots, args, dev):
    """Host-link kernels, --steps launches each:
    gather_chunks_kernel -- one Qwen3-8B layer of the 8192-token prompt
        (32 chunks, 33,554,432 B) written into pinned slab slots;
    assemble_rows_kernel -- one Qwen3-30B-A3B-shaped blend layer: 27,904 hit
        rows (57,147,392 B) read in place from 109 pinned chunks, RoPE
        relocation, APC prefix gather, gap zeroing (allocation_end 32767)."""
    import ctypes

    from cacheblend_vllm import _native
    from cacheblend_vllm.config import CacheBlendConfig
    from cacheblend_vllm.host_store import PinnedChunkSlab, PinnedChunkStore
    from cacheblend_vllm.kv_layout import kv_desc
    from cacheblend_vllm.loader import PagedBlendLoader
    from cacheblend_vllm.types import BlendPlan, BlendSegment

    H, D = cache.row_shape
    slab = PinnedChunkSlab((2, 256, H, D), torch.bfloat16, chunks_per_arena=32)
    slots_dev = src_slots.to(dev)
    desc, _ = kv_desc(cache.kv_layers[0], cache.block_size)
    chunks = slab.alloc_run(32)
    plane = 256 * desc.row_bytes
    k_ptrs = (ctypes.c_void_p * 32)(*[c.data_ptr() for c in chunks])
    v_ptrs = (ctypes.c_void_p * 32)(*[c.data_ptr() + plane for c in chunks])
    lib = _native.load()
    for _ in range(args.steps):
        _native.check(lib.cbk_paged_gather_chunks(desc, slots_dev.data_ptr(), src_slots.numel(), 256, k_ptrs,
                                                  v_ptrs, desc.row_bytes, 256, None,
                                                  _native.stream_handle(dev)), "profile gather_chunks")
    torch.cuda.synchronize()
    for c in chunks:
        slab.free(c)
    slab.close()

    L, BS, H3, A, APC = 1, 16, 4, 32767, 2048
    rng = np.random.default_rng(0)
    gaps = rng.integers(1, 512, 12)
    total = (A - APC - int(gaps.sum())) // 256
    lens = 1 + rng.multinomial(total - 12, np.full(12, 1 / 12))
    nb = (A + BS - 1) // BS + 8
    pages = synthetic.paged_pool(nb, BS, H3, D, torch.bfloat16, dev, seed=5)
    slab3 = PinnedChunkSlab((2, 256, H3, D), torch.bfloat16, chunks_per_arena=128)
    store = PinnedChunkStore(256, 1 << 40, on_release=slab3.free)
    segments, pos, src = [], APC, 0
    for i, (g, m) in enumerate(zip(gaps, lens)):
        pos += int(g)
        for c in range(int(m)):
            sid = store.begin_put("p", src + 256 * c, list(range(src + 256 * c + 7 * i, src + 256 * c + 7 * i + 256)), L)
            slot = slab3.alloc()
            slot.copy_(torch.randn(slot.shape, dtype=torch.float32).to(torch.bfloat16))
            store.put_layer_host(sid, 0, slot)
            segments.append(BlendSegment(sid, pos + 256 * c))
        src += 256 * int(m) + 512
        pos += 256 * int(m)
    store.pin("p", segments)
    plan = BlendPlan(APC, A, sum(s.length for s in segments), tuple(segments))
    slots = synthetic.block_slots(torch.randperm(nb, generator=torch.Generator().manual_seed(1))[: (A + BS - 1) // BS],
                                  BS, A)

    class Rope:
        head_size = rotary_dim = D
        is_neox_style = True
        inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
        ang = torch.arange(65536, dtype=torch.float32)[:, None] * inv
        cos_sin_cache = torch.cat([ang.cos(), ang.sin()], -1).to(dev)

    rope = Rope()
    cfg = CacheBlendConfig.from_extra_config({})
    for _ in range(args.steps):
        loader = PagedBlendLoader([pages], store, "p", plan, slots, BS, cfg, zero_copy=True)
        loader.prefetch(0, rope)
        loader.get(0)
    torch.cuda.synchronize()
    store.release("p")
    store.clear()
    slab3.close()


def _kdev_async(torch, S, fresh, cached, gap):
    """cbk_kdev_select without the count readback (device time only)."""
    from cacheblend_vllm import _native

    n = fresh.shape[0]
    lib = _native.load()
    nbytes = lib.cbk_select_workspace_bytes(n)
    ws = _native.workspace(fresh.device, nbytes)
    scores = _kdev_async.scores
    if scores is None or scores.numel() != n:
        _kdev_async.scores = scores = torch.empty(n, dtype=torch.float32, device=fresh.device)
        _kdev_async.out = torch.empty(n, dtype=torch.long, device=fresh.device)
        _kdev_async.count = torch.empty(1, dtype=torch.long, device=fresh.device)
        _kdev_async.gap = gap.view(torch.uint8)
    rc = lib.cbk_kdev_select(
        fresh.data_ptr(), fresh.stride(0), cached.data_ptr(), cached.stride(0), cached.shape[0],
        None, 0, n, fresh.shape[1], 1, _kdev_async.gap.data_ptr(), None, 16, 0.15,
        scores.data_ptr(), _kdev_async.out.data_ptr(), _kdev_async.count.data_ptr(),
        ws.data_ptr(), ws.numel(), _native.stream_handle(fresh.device),
    )
    _native.check(rc, "kdev_select")


_kdev_async.scores = None


def _host_cpu() -> dict:
    """Host CPU identity from /proc/cpuinfo and the threads this process may use."""
    fields = {}
    logical = 0
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, value = line.partition(":")
                key = key.strip()
                if key == "processor":
                    logical += 1
                elif key in ("model name", "vendor_id", "cpu family", "model", "stepping") and key not in fields:
                    fields[key] = value.strip()
    except OSError:
        pass
    name = fields.get("model name", "unknown")
    model = (f"{name} (vendor {fields.get('vendor_id', '?')}, family {fields.get('cpu family', '?')}, "
             f"model {fields.get('model', '?')}, stepping {fields.get('stepping', '?')})")
    affinity = len(os.sched_getaffinity(0))
    return {"cpu_model": model, "host_cpu_count": os.cpu_count(), "cpuinfo_processors": logical,
            "affinity_cpus": affinity}


def _median_time(fn, min_runs: int, max_runs: int, budget_s: float) -> tuple[float, int]:
    for _ in range(2):  # warm-up
        fn()
    times = []
    stop = time.perf_counter() + budget_s
    while len(times) < min_runs or (time.perf_counter() < stop and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline(torch, synthetic):
    """The reference's torch path (the build's restatement in
    oracle/torch_cpu_path.py, pinned against the oracle) on the host cores,
    on bounded samples of each workload:
      C2 (headline): 4 of 36 layers of the 8192-token prompt gathered and
          scattered back with advanced indexing / index_put_;
      C1: the fp32 plumbing case end to end;
      C3: 2 of 48 layers of the blend load (APC gather, gap zeroing, per
          segment plane copies, bf16 K relocation, index scatter, commit);
      C4: K-deviation scores + top-k selection over 65,536 tokens;
      C5: 16 of the 512 eight-query chunks of the Sparse-Q loop (the
          reference's loop is dense over the whole key context, so a chunk
          costs the same wherever it sits), scaled to all 512."""
    sys.path.insert(0, ROOT)
    from oracle import torch_cpu_path as ref

    host = _host_cpu()
    # the box allots each GPU job a share of the host (OMP_NUM_THREADS);
    # without one, every CPU this process may run on
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = min(host["affinity_cpus"], share) if share > 0 else host["affinity_cpus"]
    torch.set_num_threads(threads)
    NB, BS, H, D, T, LS = 4096, 16, 8, 128, 8192, 4
    # filled (not torch.zeros, whose untouched pages all map the shared zero
    # page and would make gathers read from cache)
    layers = [torch.full((2, NB, BS, H, D), float(i + 1), dtype=torch.bfloat16) for i in range(LS)]
    g = torch.Generator().manual_seed(0)
    perm = torch.randperm(NB, generator=g)
    src = synthetic.block_slots(perm[:512], BS, T)
    dst = synthetic.block_slots(perm[512:1024], BS, T)

    def c2():
        for layer in layers:
            chunk = ref.gather(layer, src, BS).contiguous()
            ref.scatter(chunk, layer, dst, BS)

    med, runs = _median_time(c2, 10, 40, 15.0)
    value = 4 * LS * 2 * T * H * D * 2 / med / 1e9
    del layers
    log(f"cpu baseline C2: {value:.2f} GB/s on {threads} threads")

    # C1: fp32 separate K/V [64, 16, 2, 64], 512 tokens -> two 256-token chunks
    # -> scatter to a fresh permutation; K-deviation top 15% over the 512 tokens
    g1 = torch.Generator().manual_seed(0)
    k1, v1 = torch.randn(64, 16, 2, 64, generator=g1), torch.randn(64, 16, 2, 64, generator=g1)
    kv1 = torch.stack((k1, v1))
    s1 = synthetic.block_slots(torch.randperm(64, generator=g1)[:32], 16, 512)
    d1 = synthetic.block_slots(torch.randperm(64, generator=g1)[:32], 16, 512)
    noisy = torch.randperm(512, generator=g1)[:51]
    gap1 = torch.zeros(512, dtype=torch.bool)

    def c1():
        chunks = [ref.gather(kv1, s1[i:i + 256], 16).contiguous() for i in (0, 256)]
        for i, c in zip((0, 256), chunks):
            ref.scatter(c, kv1, d1[i:i + 256], 16)
        cached = torch.cat([c[0] for c in chunks]).reshape(512, 128)
        fresh = cached.clone()
        fresh[noisy] += 0.05
        ref.select(ref.kdev_scores(fresh, cached), gap1, 0.15)

    c1_med, _ = _median_time(c1, 10, 200, 2.0)

    # C3: 2 sampled layers of the 48-layer blend load
    A, APC, H3 = 32767, 2048, 4
    segs = _c3_segments(A, APC)
    hit = sum(n for _, _, n in segs)
    nb3 = (A + BS - 1) // BS + 8
    pages3 = [torch.full((2, nb3, BS, H3, D), 0.5 * (i + 1), dtype=torch.bfloat16) for i in range(2)]
    slots3 = synthetic.block_slots(torch.randperm(nb3, generator=g)[: (A + BS - 1) // BS], BS, A)
    hosts3 = [[(s0, t0, torch.full((2, n, H3, D), 0.25 * (i + 1), dtype=torch.bfloat16)) for s0, t0, n in segs]
              for i in range(2)]
    inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    ang = torch.arange(65536, dtype=torch.float32)[:, None] * inv
    rope_cache = torch.cat([ang.cos(), ang.sin()], -1)
    bufs = [torch.empty((2, A, H3, D), dtype=torch.bfloat16) for _ in range(2)]

    def c3():
        for i in range(2):
            ref.blend_load_layer(pages3[i], slots3, BS, APC, A, hosts3[i], rope_cache, D, True, bufs[i])

    c3_med, c3_runs = _median_time(c3, 3, 10, 10.0)
    c3_layer_s = c3_med / 2
    del pages3, hosts3, bufs
    log(f"cpu baseline C3: {c3_layer_s * 1e3:.1f} ms per layer")

    # C4: K-deviation selection at 65,536 tokens
    fresh, cached, gap = synthetic.kdev_inputs(65536, 4, 128, torch.bfloat16, "cpu", seed=0)
    c4_med, _ = _median_time(lambda: ref.select(ref.kdev_scores(fresh, cached), gap, 0.15,
                                                ref.dilate(gap, 16)), 6, 20, 5.0)
    del fresh, cached, gap

    # C5: 16 of 512 eight-query chunks over the 98,304-key context
    nk, hq, hkv = 98304, 32, 4
    g5 = torch.Generator().manual_seed(0)
    key5 = (torch.randn((nk, hkv, D), generator=g5) / D ** 0.5).to(torch.bfloat16)
    qpos = torch.from_numpy(np.flatnonzero(synthetic.sparse_q_layout(nk, 4096, seed=0)))
    picks = torch.linspace(0, 511, 16).long()
    sample_pos = torch.cat([qpos[8 * c: 8 * c + 8] for c in picks.tolist()])
    q5 = (torch.randn((sample_pos.numel(), hq, D), generator=g5) / D ** 0.5).to(torch.bfloat16)
    c5_med, _ = _median_time(lambda: ref.sparse_q_full_scores(q5, key5, sample_pos, D ** -0.5, 8), 2, 5, 10.0)
    c5_chunk_s = c5_med / 16
    log(f"cpu baseline C5: {c5_chunk_s * 1e3:.1f} ms per 8-query chunk")

    return {
        "value": round(value, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"4 of 36 layers, 8192-token prompt, gather+scatter with the reference's torch ops "
                  f"(advanced indexing / index_put_), median of {runs} runs",
        "threads_note": "threads = the host share this process is given (OMP_NUM_THREADS where set, "
                        "else its CPU affinity)",
        **host,
        "c1_plumbing_us": round(c1_med * 1e6, 1),
        "c3_ms_per_layer": round(c3_layer_s * 1e3, 2),
        "c3_hit_GBps": round(hit * 2 * H3 * D * 2 / c3_layer_s / 1e9, 3),
        "c3_est_48_layers_ms": round(48 * c3_layer_s * 1e3, 1),
        "c3_sample": f"2 of 48 layers, median of {c3_runs} runs",
        "kdev_select_us_per_64k_tokens": round(c4_med * 1e6, 1),
        "c5_ms_per_chunk": round(c5_chunk_s * 1e3, 2),
        "c5_est_full_ms": round(512 * c5_chunk_s * 1e3, 1),
        "c5_sample": "16 of 512 chunks of 8 queries (evenly spaced), scaled x32",
    }


if __name__ == "__main__":
    sys.exit(main())
