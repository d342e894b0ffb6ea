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
import threading

import torch

from . import _native

logger = logging.getLogger(__name__)

# roles, in the order the streams are picked
LOAD, COPY, STORE = 0, 1, 2
_ROLES = 3

_picked: dict[tuple[int, int], list] = {}
_lock = threading.Lock()


def side_stream(role: int, device: torch.device | int | None = None):
    """The side stream for ``role`` (LOAD, COPY or STORE) on ``device``,
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
    out = (ctypes.c_void_p * _ROLES)()
    found = ctypes.c_int32()
    with torch.cuda.device(device):
        _native.check(_native.load().cbk_side_streams(serving.cuda_stream, _ROLES, 24, 0.5, out,
                                                      ctypes.byref(found)), "side streams")
    streams = [torch.cuda.ExternalStream(out[i], device=device) for i in range(found.value)]
    if len(streams) < _ROLES:
        logger.warning("only %d of %d side streams run concurrently with the serving stream; "
                       "the rest share hardware queues (raise GPU_MAX_HW_QUEUES)", len(streams), _ROLES)
        streams += [torch.cuda.Stream(device) for _ in range(_ROLES - len(streams))]
    return streams
