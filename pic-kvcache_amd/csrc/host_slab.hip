// Pinned host chunk slab: fixed-size chunk slots carved from large pinned,
// fine-grained (coherent) host arenas, recycled through a free list.
//
// The save path writes every 256-token chunk of every layer straight into a
// slot with a GPU kernel, and the load path reads it back the same way, so
// a slot must be GPU-addressable host memory (hipHostMalloc) whose GPU
// accesses stay coherent with the host (hipHostMallocCoherent). Pinning is
// paid once per arena instead of once per layer batch (the reference pins a
// fresh batch per layer, connector.py:421-426).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <unordered_set>
#include <vector>

#include "cbk_common.hpp"

namespace {

struct Slab {
  std::mutex mu;
  size_t chunk_bytes = 0;
  size_t per_arena = 0;
  size_t max_bytes = 0;
  std::vector<void*> arenas;
  std::vector<void*> free_list;
  std::unordered_set<void*> live;
};

}  // namespace

extern "C" {

int cbk_slab_create(size_t chunk_bytes, size_t chunks_per_arena, size_t max_bytes, void** out_handle) {
  cbk::clear_error();
  CBK_REQUIRE(out_handle != nullptr, "out_handle is NULL");
  CBK_REQUIRE(chunk_bytes > 0 && chunks_per_arena > 0, "chunk_bytes and chunks_per_arena must be positive");
  CBK_REQUIRE(chunk_bytes % 256 == 0, "chunk_bytes must be a multiple of 256");
  Slab* s = new Slab;
  s->chunk_bytes = chunk_bytes;
  s->per_arena = chunks_per_arena;
  s->max_bytes = max_bytes;
  *out_handle = s;
  return CBK_OK;
}

int cbk_slab_alloc(void* handle, void** out_chunk) {
  cbk::clear_error();
  CBK_REQUIRE(handle != nullptr && out_chunk != nullptr, "NULL argument");
  Slab* s = static_cast<Slab*>(handle);
  std::lock_guard<std::mutex> lock(s->mu);
  if (s->free_list.empty()) {
    const size_t bytes = s->chunk_bytes * s->per_arena;
    const size_t total = bytes * (s->arenas.size() + 1);
    if (s->max_bytes && total > s->max_bytes)
      return cbk::set_error(CBK_ERR_WORKSPACE, "pinned slab would exceed %zu bytes", s->max_bytes);
    void* arena = nullptr;
    hipError_t err = hipHostMalloc(&arena, bytes, hipHostMallocCoherent | hipHostMallocPortable);
    if (err != hipSuccess || arena == nullptr)
      return cbk::set_error(CBK_ERR_LAUNCH, "hipHostMalloc(%zu): %s", bytes, hipGetErrorString(err));
    s->arenas.push_back(arena);
    for (size_t i = s->per_arena; i-- > 0;)
      s->free_list.push_back(static_cast<char*>(arena) + i * s->chunk_bytes);
  }
  void* chunk = s->free_list.back();
  s->free_list.pop_back();
  s->live.insert(chunk);
  *out_chunk = chunk;
  return CBK_OK;
}

int cbk_slab_free(void* handle, void* chunk) {
  cbk::clear_error();
  CBK_REQUIRE(handle != nullptr, "NULL handle");
  Slab* s = static_cast<Slab*>(handle);
  std::lock_guard<std::mutex> lock(s->mu);
  CBK_REQUIRE(s->live.erase(chunk) == 1, "chunk %p is not a live slot of this slab", chunk);
  s->free_list.push_back(chunk);
  return CBK_OK;
}

int cbk_slab_stats(void* handle, size_t* arenas, size_t* free_chunks, size_t* live_chunks) {
  cbk::clear_error();
  CBK_REQUIRE(handle != nullptr, "NULL handle");
  Slab* s = static_cast<Slab*>(handle);
  std::lock_guard<std::mutex> lock(s->mu);
  if (arenas) *arenas = s->arenas.size();
  if (free_chunks) *free_chunks = s->free_list.size();
  if (live_chunks) *live_chunks = s->live.size();
  return CBK_OK;
}

int cbk_slab_destroy(void* handle) {
  cbk::clear_error();
  if (handle == nullptr) return CBK_OK;
  Slab* s = static_cast<Slab*>(handle);
  int rc = CBK_OK;
  for (void* a : s->arenas) {
    if (hipHostFree(a) != hipSuccess) rc = cbk::set_error(CBK_ERR_LAUNCH, "hipHostFree failed");
  }
  delete s;
  return rc;
}

int cbk_memcpy_runs(const uint64_t* dst, const uint64_t* src, const uint64_t* bytes, int64_t n,
                    cbk_stream_t stream) {
  cbk::clear_error();
  CBK_REQUIRE(n >= 0, "negative run count");
  if (n == 0) return CBK_OK;
  CBK_REQUIRE(dst != nullptr && src != nullptr && bytes != nullptr, "NULL run table");
  for (int64_t i = 0; i < n; ++i) {
    if (bytes[i] == 0) continue;
    CBK_REQUIRE(dst[i] != 0 && src[i] != 0, "run %lld has a NULL address", (long long)i);
    const hipError_t err = hipMemcpyAsync(reinterpret_cast<void*>(dst[i]), reinterpret_cast<const void*>(src[i]),
                                          size_t(bytes[i]), hipMemcpyDefault, static_cast<hipStream_t>(stream));
    if (err != hipSuccess)
      return cbk::set_error(CBK_ERR_LAUNCH, "hipMemcpyAsync of run %lld: %s", (long long)i, hipGetErrorString(err));
  }
  return CBK_OK;
}

int cbk_host_accessible(const void* ptr, size_t bytes, int* accessible) {
  cbk::clear_error();
  CBK_REQUIRE(accessible != nullptr, "accessible is NULL");
  *accessible = 0;
  if (ptr == nullptr || bytes == 0) return CBK_OK;
  // both ends of the range must lie in page-locked host memory that the GPU
  // addresses at the host address (hipHostMalloc under unified addressing)
  const char* ends[2] = {static_cast<const char*>(ptr), static_cast<const char*>(ptr) + bytes - 1};
  for (const char* p : ends) {
    hipPointerAttribute_t attr{};
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
      (void)hipGetLastError();  // plain pageable memory: not an error for the caller
      return CBK_OK;
    }
    if (attr.type != hipMemoryTypeHost || attr.devicePointer == nullptr ||
        attr.devicePointer != attr.hostPointer)
      return CBK_OK;
  }
  *accessible = 1;
  return CBK_OK;
}

}  // extern "C"
