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
    return p.parse_args()


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
            "traffic": None,
            "launch_us": round(gather_ms * 1e3, 2),
            "algorithmic_bytes": 2 * copy_bytes,
        },
        "scatter_kernel": {"GBps": round(scatter_gbps, 1), "launch_us": round(scatter_ms * 1e3, 2),
                           "frac": round(scatter_gbps / HBM_PEAK_GBPS, 4)},
    }

    if not args.skip_extras:
        result.update(extras(torch, KL, S, synthetic, layers, cache, src_slots, staging, args, dev))

    if not args.skip_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(torch, synthetic)
    print(json.dumps(result), flush=True)
    return 0


def extras(torch, KL, S, synthetic, layers, cache, src_slots, staging, args, dev):
    out = {}
    L = len(layers)
    BS = cache.block_size
    layer_bytes = staging[0].numel() * staging.element_size()

    # per-layer launches (save_kv_layer granularity), device time per layer
    def per_layer():
        for l in range(L):
            cache.gather(src_slots, out=staging[l:l + 1], layers=(l, l + 1))

    ms = event_time_ms(torch, per_layer, max(3, args.steps // 4))
    out["per_layer_gather"] = {"GBps": round(2 * L * layer_bytes / (ms / 1e3) / 1e9, 1),
                               "us_per_layer": round(ms * 1e3 / L, 2)}
    log(f"per-layer gather: {out['per_layer_gather']}")

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
    dev_ms = event_time_ms(torch, lambda: _kdev_async(torch, S, fresh, cached, gap), reps)
    t0 = time.perf_counter()
    for _ in range(reps):
        lib_sel()
    wall_ms = (time.perf_counter() - t0) / reps * 1e3
    read_bytes = 2 * n * 512 * 2
    score_ms = event_time_ms(torch, lambda: S.kdev_scores(fresh, cached), reps)
    out["kdev_select"] = {
        "us_per_64k_tokens": round(dev_ms * 1e3, 2),
        "wall_us_with_count_readback": round(wall_ms * 1e3, 2),
        "score_kernel_us": round(score_ms * 1e3, 2),
        "score_kernel_GBps": round(read_bytes / (score_ms / 1e3) / 1e9, 1),
        "selected": int(selected.numel()),
        "tokens": n, "ratio": 0.15, "overflow_radius": 16,
    }
    log(f"kdev select: {out['kdev_select']}")
    return out


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
    torch.cuda.synchronize()
    log(f"profile run done: {args.steps} x (gather, scatter, plain copy, kdev select)")
    return 0


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


def cpu_baseline(torch, synthetic):
    """The reference's torch path on the host cores, on a bounded sample:
    4 of the 36 layers (full 8192-token prompt) gathered and scattered back."""
    sys.path.insert(0, ROOT)
    from oracle import torch_cpu_path as ref

    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    NB, BS, H, D, T, LS = 4096, 16, 8, 128, 8192, 4
    # filled (not torch.zeros, whose untouched pages all map the shared zero
    # page and would make gathers read from cache)
    layers = [torch.full((2, NB, BS, H, D), float(i + 1), dtype=torch.bfloat16) for i in range(LS)]
    g = torch.Generator().manual_seed(0)
    perm = torch.randperm(NB, generator=g)
    src = synthetic.block_slots(perm[:512], BS, T)
    dst = synthetic.block_slots(perm[512:1024], BS, T)

    def run():
        for layer in layers:
            chunk = ref.gather(layer, src, BS).contiguous()
            ref.scatter(chunk, layer, dst, BS)

    for _ in range(2):
        run()
    times = []
    budget = time.perf_counter() + 15.0
    while len(times) < 10 or (time.perf_counter() < budget and len(times) < 40):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > budget + 15.0:
            break
    med = statistics.median(times)
    nbytes = 4 * LS * 2 * T * H * D * 2
    value = nbytes / med / 1e9
    # K-deviation selection at 65,536 tokens on the host
    fresh, cached, gap = synthetic.kdev_inputs(65536, 4, 128, torch.bfloat16, "cpu", seed=0)
    ktimes = []
    for i in range(8):
        t0 = time.perf_counter()
        scores = ref.kdev_scores(fresh, cached)
        ref.select(scores, gap, 0.15, ref.dilate(gap, 16))
        if i >= 2:
            ktimes.append(time.perf_counter() - t0)
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(value, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"4 of 36 layers, 8192-token prompt, gather+scatter with the reference's torch ops "
                  f"(advanced indexing / index_put_), median of {len(times)} runs",
        "kdev_select_us_per_64k_tokens": round(statistics.median(ktimes) * 1e6, 1),
        "cpu_model": cpu,
    }


if __name__ == "__main__":
    sys.exit(main())
