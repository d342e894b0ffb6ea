"""Opt-in JSONL pipeline trace, switched on by ``CACHEBLEND_TRACE_DIR``.

The record format is the reference tracer's (cacheblend_vllm/trace.py:19-64),
so its trace analysis reads these files unchanged: one file per process and
component, ``<dir>/<component>-pid-<pid>.jsonl``, opened for append and
line-buffered; each line a compact, key-sorted JSON object with
``timestamp_ns``, ``monotonic_ns``, ``pid``, ``thread_id``, ``component``,
``event``, an optional ``request_id`` and the event's own fields; the first
line of a tracer is ``trace_started``. Timestamps are taken on the host when
the event is emitted; tracing never synchronises a device.

``roctx_range(name)`` marks a host-side phase (a layer's load enqueue, its
commit, a layer's save, the check layer's selection) as a roctx range when
``CACHEBLEND_ROCTX`` is set, so ``rocprofv3 --marker-trace`` shows the
phases beside the kernels; otherwise it is a shared no-op context.
"""

from __future__ import annotations

import functools
import json
import os
import threading
import time
from typing import Any, TextIO

TRACE_DIR_ENV = "CACHEBLEND_TRACE_DIR"
ROCTX_ENV = "CACHEBLEND_ROCTX"
_encode = json.JSONEncoder(sort_keys=True, separators=(",", ":")).encode
_roctx_on = os.environ.get(ROCTX_ENV, "") not in ("", "0")


class _NoRange:
    __slots__ = ()

    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NO_RANGE = _NoRange()


class _RoctxRange:
    __slots__ = ("name",)

    def __init__(self, name: str):
        self.name = name

    def __enter__(self):
        import torch

        torch.cuda.nvtx.range_push(self.name)  # roctx on ROCm builds of torch
        return None

    def __exit__(self, *exc):
        import torch

        torch.cuda.nvtx.range_pop()
        return False


def roctx_range(name: str):
    """A roctx range around a host-side phase when ``CACHEBLEND_ROCTX`` is
    set, else a no-op context."""
    return _RoctxRange(name) if _roctx_on else _NO_RANGE


def roctx_phase(name: str):
    """Decorator: the call runs inside ``roctx_range(name)``."""

    def wrap(fn):
        @functools.wraps(fn)
        def inner(*args, **kwargs):
            if not _roctx_on:
                return fn(*args, **kwargs)
            with _RoctxRange(name):
                return fn(*args, **kwargs)

        return inner

    return wrap


def _open_trace_file(component: str) -> TextIO | None:
    directory = os.environ.get(TRACE_DIR_ENV)
    if not directory:
        return None
    os.makedirs(directory, exist_ok=True)
    path = os.path.join(directory, f"{component}-pid-{os.getpid()}.jsonl")
    return open(path, "a", encoding="utf-8", buffering=1)


class PipelineTracer:
    """Event sink of one pipeline component. When tracing is off, ``emit``
    returns at its first test and ``enabled`` lets callers skip building
    event fields at all."""

    __slots__ = ("component", "_sink", "_guard")

    def __init__(self, component: str):
        self.component = component
        self._guard = threading.Lock()
        self._sink = _open_trace_file(component)
        if self._sink is not None:
            self.emit("trace_started")

    @property
    def enabled(self) -> bool:
        return self._sink is not None

    def emit(self, event: str, request_id: str | None = None, **fields: Any) -> None:
        if self._sink is None:
            return
        head = {"timestamp_ns": time.time_ns(), "monotonic_ns": time.monotonic_ns(),
                "pid": os.getpid(), "thread_id": threading.get_ident(),
                "component": self.component, "event": event}
        if request_id is not None:
            head["request_id"] = request_id
        text = _encode({**head, **fields}) + "\n"
        with self._guard:
            sink = self._sink
            if sink is not None:
                sink.write(text)

    def close(self) -> None:
        with self._guard:
            sink, self._sink = self._sink, None
        if sink is not None:
            sink.close()
