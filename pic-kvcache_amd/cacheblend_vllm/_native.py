"""ctypes binding of libcacheblend_hip.so (the gfx950 kernels' C ABI).

The declarations mirror include/cacheblend_hip.h one for one. Loading fails
loudly: there is no CPU or torch fallback for any kernel in this package.
"""

from __future__ import annotations

import ctypes
import os
import threading

import numpy as np
import torch

LIB_NAME = "libcacheblend_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 1

CBK_OK = 0
CBK_ERR_INVALID = -1
CBK_ERR_UNSUPPORTED = -2
CBK_ERR_LAUNCH = -3
CBK_ERR_WORKSPACE = -4

DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
MAX_DILATION_RADIUS = 4096
SELECT_MULTI_LAUNCH = 1  # CBK_SELECT_MULTI_LAUNCH
SELECT_TEST_GIVE_UP = 2  # CBK_SELECT_TEST_GIVE_UP

c_i64 = ctypes.c_int64
c_i32 = ctypes.c_int32
c_u64 = ctypes.c_uint64
c_vp = ctypes.c_void_p


class KVDesc(ctypes.Structure):
    """``cbk_kv_desc``: one paged KV layer (base pointers, geometry in bytes)."""

    _fields_ = [
        ("k_base", c_vp),
        ("v_base", c_vp),
        ("num_blocks", c_i64),
        ("block_size", c_i64),
        ("block_stride", c_i64),
        ("token_stride", c_i64),
        ("row_bytes", c_i64),
    ]


# name -> (restype, argtypes)
_SIGNATURES = {
    "cbk_abi_version": (ctypes.c_int, []),
    "cbk_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "cbk_last_error": (ctypes.c_char_p, []),
    "cbk_paged_gather": (
        ctypes.c_int,
        [ctypes.POINTER(KVDesc), c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_vp],
    ),
    "cbk_paged_scatter": (
        ctypes.c_int,
        [c_vp, c_vp, c_i64, ctypes.POINTER(KVDesc), c_vp, c_i64, c_vp, c_vp],
    ),
    "cbk_paged_gather_layers": (
        ctypes.c_int,
        [ctypes.POINTER(KVDesc), c_i32, c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp],
    ),
    "cbk_paged_scatter_layers": (
        ctypes.c_int,
        [c_vp, c_i64, c_i64, c_i64, ctypes.POINTER(KVDesc), c_i32, c_vp, c_i64, c_vp, c_vp],
    ),
    "cbk_kdev_scores": (
        ctypes.c_int,
        [c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_i64, c_i32, c_vp, c_vp],
    ),
    "cbk_select_workspace_bytes": (ctypes.c_size_t, [c_i64]),
    "cbk_select": (
        ctypes.c_int,
        [c_vp, c_vp, c_vp, c_i64, c_i64, ctypes.c_double, c_vp, c_vp, c_vp, ctypes.c_size_t, c_vp],
    ),
    "cbk_kdev_select": (
        ctypes.c_int,
        [
            c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_i64, c_i32,
            c_vp, c_vp, c_i64, ctypes.c_double, c_vp, c_vp, c_vp, c_vp, ctypes.c_size_t, c_vp,
        ],
    ),
    "cbk_select_ex": (
        ctypes.c_int,
        [c_vp, c_vp, c_vp, c_i64, c_i64, ctypes.c_double, c_vp, c_vp, c_vp, ctypes.c_size_t,
         ctypes.c_uint32, c_vp],
    ),
    "cbk_kdev_select_ex": (
        ctypes.c_int,
        [
            c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_i64, c_i32,
            c_vp, c_vp, c_i64, ctypes.c_double, c_vp, c_vp, c_vp, c_vp, ctypes.c_size_t,
            ctypes.c_uint32, c_vp,
        ],
    ),
    "cbk_kdev_select_noalloc": (
        ctypes.c_int,
        [
            c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_i64, c_i32,
            c_vp, c_vp, c_i64, ctypes.c_double, c_vp, c_vp, c_vp, c_vp,
        ],
    ),
    "cbk_dilate": (ctypes.c_int, [c_vp, c_i64, c_i64, c_vp, c_vp]),
    "cbk_blend_assemble": (
        ctypes.c_int,
        [
            ctypes.POINTER(KVDesc), c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_vp,
            c_i64, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_vp, c_vp, c_i64, c_vp, c_vp,
        ],
    ),
    "cbk_paged_gather_chunks": (
        ctypes.c_int,
        [ctypes.POINTER(KVDesc), c_vp, c_i64, c_i64, c_vp, c_vp, c_i64, c_i32, c_vp, c_vp],
    ),
    "cbk_paged_scatter_chunks": (
        ctypes.c_int,
        [c_vp, c_vp, c_i64, c_i64, ctypes.POINTER(KVDesc), c_vp, c_i64, c_i32, c_vp, c_vp],
    ),
    "cbk_slab_create": (ctypes.c_int, [ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, ctypes.POINTER(c_vp)]),
    "cbk_slab_alloc": (ctypes.c_int, [c_vp, ctypes.POINTER(c_vp)]),
    "cbk_slab_alloc_run": (ctypes.c_int, [c_vp, c_i64, ctypes.POINTER(c_vp)]),
    "cbk_slab_free": (ctypes.c_int, [c_vp, c_vp]),
    "cbk_slab_stats": (
        ctypes.c_int,
        [c_vp, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)],
    ),
    "cbk_slab_destroy": (ctypes.c_int, [c_vp]),
    "cbk_host_accessible": (ctypes.c_int, [c_vp, ctypes.c_size_t, ctypes.POINTER(c_i32)]),
    "cbk_memcpy_runs": (ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp]),
    "cbk_memcpy_runs_commands": (ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, ctypes.POINTER(c_i64)]),
    "cbk_side_streams": (ctypes.c_int, [c_vp, c_i32, c_i32, ctypes.c_float, ctypes.POINTER(c_vp),
                                        ctypes.POINTER(c_i32)]),
    "cbk_stream_destroy": (ctypes.c_int, [c_vp]),
    "cbk_blend_assemble_chunks": (
        ctypes.c_int,
        [
            ctypes.POINTER(KVDesc), c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_i64,
            c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_vp, c_vp, c_i64, c_vp, c_i32, c_vp,
        ],
    ),
    "cbk_blend_attention": (
        ctypes.c_int,
        [c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_float,
         c_i32, c_vp, c_i64, c_vp],
    ),
    "cbk_rolling_hashes": (ctypes.c_int, [c_vp, c_i64, c_i64, c_vp]),
    "cbk_matcher_create": (ctypes.c_int, [c_i64, ctypes.POINTER(c_vp)]),
    "cbk_matcher_destroy": (ctypes.c_int, [c_vp]),
    "cbk_matcher_register": (ctypes.c_int, [c_vp, c_u64, c_u64, c_u64, c_vp]),
    "cbk_matcher_unregister": (ctypes.c_int, [c_vp, c_u64]),
    "cbk_matcher_size": (c_i64, [c_vp]),
    "cbk_matcher_match": (ctypes.c_int, [c_vp, c_u64, c_vp, c_i64, c_i64, c_vp, c_vp, c_i64,
                                         ctypes.POINTER(c_i64)]),
    "cbk_sparse_q_workspace_bytes": (ctypes.c_size_t, [c_i64, c_i64, c_i64, c_i64]),
    "cbk_sparse_q_scores": (
        ctypes.c_int,
        [
            c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64,
            ctypes.c_float, c_i32, c_i32, c_vp, c_i64, c_vp, c_vp, c_vp, ctypes.c_size_t, c_vp,
        ],
    ),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib: ctypes.PyDLL | None = None


def load() -> ctypes.PyDLL:
    """Load the HIP library once; raise if it is missing or mismatched.

    Loaded as a PyDLL: calls keep the GIL. Every entry point is a short
    enqueue (or a rare set-up call), and a ctypes call that released the
    GIL would, on return, wait out another Python thread's switch interval
    (5 ms by default) -- with the store publisher threads busy in Python,
    that stalled each save_kv_layer by milliseconds."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_NAME} is not built at {LIB_PATH}; run `make -C pic-kvcache_amd/csrc` "
                "(hipcc --offload-arch=gfx950). cacheblend_vllm has no CPU fallback."
            )
        lib = ctypes.PyDLL(LIB_PATH)
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.cbk_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{LIB_NAME} ABI {version} != expected {ABI_VERSION}; rebuild it")
        _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    """Raise the Python exception matching a CBK_* return code."""
    if rc == CBK_OK:
        return
    message = load().cbk_last_error().decode(errors="replace")
    text = f"{what}: {message}" if message else what
    if rc == CBK_ERR_INVALID:
        raise ValueError(text)
    if rc == CBK_ERR_UNSUPPORTED:
        raise NotImplementedError(text)
    raise RuntimeError(f"{text} ({load().cbk_error_string(rc).decode()})")


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def require_device(tensor: torch.Tensor, what: str) -> None:
    if tensor.device.type != "cuda":
        raise RuntimeError(
            f"{what} must be a ROCm device tensor (got {tensor.device}); "
            "cacheblend_vllm runs its kernels only on the GPU"
        )


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()


def _run_table(dst: np.ndarray, src: np.ndarray, nbytes: np.ndarray) -> tuple[np.ndarray, ...]:
    tables = tuple(np.ascontiguousarray(a, dtype=np.uint64) for a in (dst, src, nbytes))
    if not tables[0].shape == tables[1].shape == tables[2].shape or tables[0].ndim != 1:
        raise ValueError("dst, src and bytes must be 1-D tables of one length")
    return tables


def memcpy_runs(dst: np.ndarray, src: np.ndarray, nbytes: np.ndarray, stream: int, what: str) -> None:
    """cbk_memcpy_runs over uint64 tables (addresses and sizes in bytes)."""
    d, s, b = _run_table(dst, src, nbytes)
    check(load().cbk_memcpy_runs(d.ctypes.data, s.ctypes.data, b.ctypes.data, d.shape[0], stream), what)


def memcpy_commands(dst: np.ndarray, src: np.ndarray, nbytes: np.ndarray) -> int:
    """DMA commands cbk_memcpy_runs would issue for these runs."""
    d, s, b = _run_table(dst, src, nbytes)
    out = c_i64()
    check(load().cbk_memcpy_runs_commands(d.ctypes.data, s.ctypes.data, b.ctypes.data, d.shape[0],
                                           ctypes.byref(out)), "memcpy_runs_commands")
    return out.value


_workspaces: dict[tuple[int, int], torch.Tensor] = {}


def host_accessible(tensor: torch.Tensor) -> bool:
    """Whether the kernels can address ``tensor``'s bytes in host memory
    directly (page-locked, mapped at the host address)."""
    if tensor.device.type != "cpu" or tensor.numel() == 0:
        return False
    span = sum((n - 1) * abs(st) for n, st in zip(tensor.shape, tensor.stride()))
    nbytes = (span + 1) * tensor.element_size()
    out = ctypes.c_int32()
    check(load().cbk_host_accessible(tensor.data_ptr(), nbytes, ctypes.byref(out)), "host_accessible")
    return bool(out.value)


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A reusable uint8 device workspace of at least ``nbytes`` for the
    current stream of ``device`` (kernels on one stream are ordered, so one
    buffer per stream is never used by two calls at once)."""
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           stream_handle(device))
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _workspaces[key] = buf
    return buf
