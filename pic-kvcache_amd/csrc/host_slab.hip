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
#include <cstdint>
#include <map>
#include <mutex>
#include <set>
#include <unordered_set>
#include <vector>

#include "cbk_common.hpp"

namespace {

struct Arena {
  char* base = nullptr;
  std::set<uint32_t> free;  // free slot indices, ascending
};

struct Slab {
  std::mutex mu;
  size_t chunk_bytes = 0;
  size_t per_arena = 0;
  size_t max_bytes = 0;
  size_t free_count = 0;
  std::vector<Arena> arenas;
  std::map<uintptr_t, size_t> by_base;  // arena base -> index
  std::unordered_set<void*> live;

  int grow() {
    const size_t bytes = chunk_bytes * per_arena;
    if (max_bytes && bytes * (arenas.size() + 1) > max_bytes)
      return cbk::set_error(CBK_ERR_WORKSPACE, "pinned slab would exceed %zu bytes", max_bytes);
    void* mem = nullptr;
    const hipError_t err = hipHostMalloc(&mem, bytes, hipHostMallocCoherent | hipHostMallocPortable);
    if (err != hipSuccess || mem == nullptr)
      return cbk::set_error(CBK_ERR_LAUNCH, "hipHostMalloc(%zu): %s", bytes, hipGetErrorString(err));
    Arena arena;
    arena.base = static_cast<char*>(mem);
    for (uint32_t i = 0; i < per_arena; ++i) arena.free.insert(arena.free.end(), i);
    by_base[reinterpret_cast<uintptr_t>(mem)] = arenas.size();
    arenas.push_back(std::move(arena));
    free_count += per_arena;
    return CBK_OK;
  }

  void take(size_t a, uint32_t first, size_t n, void** out) {
    Arena& arena = arenas[a];
    for (size_t k = 0; k < n; ++k) {
      arena.free.erase(first + uint32_t(k));
      void* slot = arena.base + (first + k) * chunk_bytes;
      live.insert(slot);
      out[k] = slot;
    }
    free_count -= n;
  }

  // first run of n free, consecutive slots (lowest arena, lowest index)
  bool find_run(size_t n, size_t* arena_out, uint32_t* first_out) const {
    for (size_t a = 0; a < arenas.size(); ++a) {
      const std::set<uint32_t>& f = arenas[a].free;
      if (f.size() < n) continue;
      uint32_t start = 0, prev = 0;
      size_t len = 0;
      for (uint32_t i : f) {
        if (len && i == prev + 1) {
          ++len;
        } else {
          start = i;
          len = 1;
        }
        prev = i;
        if (len == n) {
          *arena_out = a;
          *first_out = start;
          return true;
        }
      }
    }
    return false;
  }
};

}  // namespace

extern "C" {

int cbk_slab_create(size_t chunk_bytes, size_t chunks_per_arena, size_t max_bytes, void** out_handle) {
  cbk::clear_error();
  CBK_REQUIRE(out_handle != nullptr, "out_handle is NULL");
  CBK_REQUIRE(chunk_bytes > 0 && chunks_per_arena > 0, "chunk_bytes and chunks_per_arena must be positive");
  CBK_REQUIRE(chunk_bytes % 256 == 0, "chunk_bytes must be a multiple of 256");
  CBK_REQUIRE(chunks_per_arena < (size_t(1) << 31), "chunks_per_arena too large");
  Slab* s = new Slab;
  s->chunk_bytes = chunk_bytes;
  s->per_arena = chunks_per_arena;
  s->max_bytes = max_bytes;
  *out_handle = s;
  return CBK_OK;
}

int cbk_slab_alloc_run(void* handle, int64_t n, void** out_chunks) {
  cbk::clear_error();
  CBK_REQUIRE(handle != nullptr && out_chunks != nullptr, "NULL argument");
  CBK_REQUIRE(n > 0, "n must be positive");
  Slab* s = static_cast<Slab*>(handle);
  std::lock_guard<std::mutex> lock(s->mu);
  size_t a = 0;
  uint32_t first = 0;
  if (size_t(n) <= s->per_arena) {
    if (!s->find_run(size_t(n), &a, &first)) {
      // a fresh arena holds the run whole; without room for one, fall back
      // to scattered slots below
      if (s->grow() == CBK_OK) {
        a = s->arenas.size() - 1;
        first = 0;
      } else {
        cbk::clear_error();
        a = SIZE_MAX;
      }
    }
    if (a != SIZE_MAX) {
      s->take(a, first, size_t(n), out_chunks);
      return CBK_OK;
    }
  }
  while (s->free_count < size_t(n)) {
    const int rc = s->grow();
    if (rc != CBK_OK) return rc;  // nothing taken
  }
  int64_t k = 0;
  for (size_t i = 0; i < s->arenas.size() && k < n; ++i) {
    while (!s->arenas[i].free.empty() && k < n) {
      const uint32_t idx = *s->arenas[i].free.begin();
      s->take(i, idx, 1, out_chunks + k);
      ++k;
    }
  }
  return CBK_OK;
}

int cbk_slab_alloc(void* handle, void** out_chunk) {
  return cbk_slab_alloc_run(handle, 1, out_chunk);
}

int cbk_slab_free(void* handle, void* chunk) {
  cbk::clear_error();
  CBK_REQUIRE(handle != nullptr, "NULL handle");
  Slab* s = static_cast<Slab*>(handle);
  std::lock_guard<std::mutex> lock(s->mu);
  CBK_REQUIRE(s->live.erase(chunk) == 1, "chunk %p is not a live slot of this slab", chunk);
  auto it = s->by_base.upper_bound(reinterpret_cast<uintptr_t>(chunk));
  --it;  // a live slot lies in some arena at or below its address
  Arena& arena = s->arenas[it->second];
  arena.free.insert(uint32_t((static_cast<char*>(chunk) - arena.base) / s->chunk_bytes));
  ++s->free_count;
  return CBK_OK;
}

int cbk_slab_stats(void* handle, size_t* arenas, size_t* free_chunks, size_t* live_chunks) {
  cbk::clear_error();
  CBK_REQUIRE(handle != nullptr, "NULL handle");
  Slab* s = static_cast<Slab*>(handle);
  std::lock_guard<std::mutex> lock(s->mu);
  if (arenas) *arenas = s->arenas.size();
  if (free_chunks) *free_chunks = s->free_count;
  if (live_chunks) *live_chunks = s->live.size();
  return CBK_OK;
}

int cbk_slab_destroy(void* handle) {
  cbk::clear_error();
  if (handle == nullptr) return CBK_OK;
  Slab* s = static_cast<Slab*>(handle);
  int rc = CBK_OK;
  for (Arena& a : s->arenas) {
    if (hipHostFree(a.base) != hipSuccess) rc = cbk::set_error(CBK_ERR_LAUNCH, "hipHostFree failed");
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
