"""The reference's store under its own module and class name.

``LocalPinnedCPUStore(chunk_size, max_bytes, pin_memory=True)`` keeps the
constructor of the reference store (cacheblend_vllm/storage.py:35-45) over
``host_store.PinnedChunkStore``: the same methods and properties
(``begin_put``, ``reserve_layer``, ``cancel_layer``, ``put_layer``,
``put_layer_host``, ``abort_put``, ``match``, ``validate``, ``pin``,
``release``, ``get_layer``, ``clear``, ``current_bytes``,
``committed_entries``), the same errors, and ``pin_memory`` deciding whether
``put_layer`` page-locks its host copies. Code that builds the store itself
(the reference connector does, connector.py:182-186) switches by import.
"""

from __future__ import annotations

from .host_store import PinnedChunkStore

__all__ = ["LocalPinnedCPUStore"]


class LocalPinnedCPUStore(PinnedChunkStore):
    def __init__(self, chunk_size: int, max_bytes: int, pin_memory: bool = True):
        super().__init__(chunk_size, max_bytes)
        self.pin_memory = bool(pin_memory)
