"""GPU: the side streams run concurrently with the serving stream and with
each other (spins on two streams overlap instead of adding up)."""

import time

import pytest
import torch

from cacheblend_vllm.streams import COPY, LOAD, STORE, STORE_COPY, side_stream

pytestmark = pytest.mark.gpu


def _cycles_per_ms():
    torch.cuda._sleep(1000)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    torch.cuda._sleep(5_000_000)
    e1.record()
    e1.synchronize()
    return 5_000_000 / e0.elapsed_time(e1)


def _pair_ms(a, b, cycles):
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(a):
        torch.cuda._sleep(cycles)
    with torch.cuda.stream(b):
        torch.cuda._sleep(cycles)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3


def test_side_streams_overlap_serving_and_each_other():
    streams = [side_stream(r) for r in (LOAD, COPY, STORE)]
    assert len({s.cuda_stream for s in streams}) == 3
    assert side_stream(LOAD) is streams[0]  # picked once, then reused
    # with the box's 4 hardware queues the store's copies share the
    # loader's copy stream rather than a queue of the serving stream
    store_copy = side_stream(STORE_COPY)
    assert store_copy is streams[1] or store_copy.cuda_stream not in {s.cuda_stream for s in streams}
    cycles = int(10 * _cycles_per_ms())  # 10 ms spins
    serving = torch.cuda.current_stream()
    pairs = [(serving, s) for s in streams] + [(streams[0], streams[1]), (streams[0], streams[2]),
                                               (streams[1], streams[2])]
    for a, b in pairs:
        ms = _pair_ms(a, b, cycles)
        print(f"{a.cuda_stream:#x} + {b.cuda_stream:#x}: {ms:.1f} ms", flush=True)
        assert ms < 15.0, "two 10 ms spins did not overlap"
