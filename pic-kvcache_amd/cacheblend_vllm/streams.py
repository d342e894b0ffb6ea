"""Side streams for the layerwise pipelines that really run beside compute.

HIP maps streams onto a few hardware queues per process (GPU_MAX_HW_QUEUES,
4 by default) round-robin in creation order, and streams that share a queue
execute in order. A Load or Store stream that happens to share the serving
stream's queue would serialize every transfer with the model's compute, and
which queue a new stream gets depends on every stream created before it. So
the side streams are picked by measurement (``cbk_side_streams``): new
non-blocking streams are kept only when a short spin on each overlaps spins
on the serving stream and on the others. The reference simply creates its
Load and Store streams (cacheblend_vllm/connector.py:198-199, ascend.py:212).
"""

from __future__ import annotations

import ctypes
import logging
import os
import threading

import torch

from . import _native

logger = logging.getLogger(__name__)

# roles, in the order the streams are picked: the loader's assembly (LOAD)
# and its H2D copies (COPY), the store's gathers (STORE) and its D2H copies
# (STORE_COPY)
LOAD, COPY, STORE, STORE_COPY = 0, 1, 2, 3
_ROLES = 4
# a role left without a hardware queue of its own shares this role's stream
# (a fresh stream could land on the serving stream's queue); with the
# default 4 queues the store's copies share the loader's copy stream
_SHARE = {STORE_COPY: COPY}

_picked: dict[tuple[int, int], list] = {}
_lock = threading.Lock()


def side_stream(role: int, device: torch.device | int | None = None):
    """The side stream for ``role`` (LOAD, COPY, STORE or STORE_COPY) on ``device``,
    concurrent with the device's current stream; picked once per (device,
    serving stream) and kept for the life of the process."""
    device = torch.device("cuda", torch.cuda.current_device() if device is None else
                          (device if isinstance(device, int) else device.index or 0))
    serving = torch.cuda.current_stream(device)
    key = (device.index, serving.cuda_stream)
    with _lock:
        streams = _picked.get(key)
        if streams is None:
            streams = _pick(device, serving)
            _picked[key] = streams
    return streams[role]


def _pick(device: torch.device, serving) -> list:
    # one queue per process goes to the serving stream; asking for more
    # streams than the other queues can hold only lengthens the search
    queues = int(os.environ.get("GPU_MAX_HW_QUEUES", "4"))
    want = max(1, min(_ROLES, queues - 1))
    out = (ctypes.c_void_p * want)()
    found = ctypes.c_int32()
    with torch.cuda.device(device):
        _native.check(_native.load().cbk_side_streams(serving.cuda_stream, want, 24, 0.5, out,
                                                      ctypes.byref(found)), "side streams")
    streams = [torch.cuda.ExternalStream(out[i], device=device) for i in range(found.value)]
    missing = [r for r in range(len(streams), _ROLES) if _SHARE.get(r, _ROLES) >= len(streams)]
    if missing:
        logger.warning("only %d side streams run concurrently with the serving stream; roles %s "
                       "share hardware queues (raise GPU_MAX_HW_QUEUES)", len(streams), missing)
    while len(streams) < _ROLES:
        role = len(streams)
        shared = _SHARE.get(role)
        streams.append(streams[shared] if shared is not None and shared < len(streams)
                       else torch.cuda.Stream(device))
    return streams
