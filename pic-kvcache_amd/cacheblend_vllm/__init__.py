"""CacheBlend KV data movement and selection on MI355X (gfx950).

Keeps the import paths of the reference vLLM connector package
(zoudinghong2000/PIC-KVCache ``cacheblend_vllm``) for its hot path:

* ``cacheblend_vllm.kv_layout``  gather_paged_kv / scatter_paged_kv
* ``cacheblend_vllm.selection``  K-deviation, budgeted top-k, Sparse-Q
* ``cacheblend_vllm.loader``     PagedBlendLoader (layerwise H2D + scatter)
* ``cacheblend_vllm.store_path`` the connector's Store-stream save pipeline
* ``cacheblend_vllm.storage``    LocalPinnedCPUStore (the pinned chunk store)

Every kernel lives in ``libcacheblend_hip.so`` (HIP, gfx950); there is no CPU
fallback.
"""

__version__ = "0.1.0"
