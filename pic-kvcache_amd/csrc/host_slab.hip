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

// One DMA command of a run table: `rows` copies of `width` bytes whose
// destinations and sources advance by dpitch and spitch bytes (rows == 1: a
// plain copy of width bytes).
struct CopyCommand {
  uint64_t dst, src, width, rows, dpitch, spitch;
};

// Farthest row pitch folded into one 2D copy.
constexpr uint64_t kMaxCopyPitch = uint64_t(1) << 31;

// The command that starts at run i (bytes[i] > 0) and the number of runs it
// covers. Each DMA command costs the engine about as long as moving 0.5 MB,
// so runs are folded: runs that each start where the previous one ends, in
// dst and in src, become one copy; failing that, runs of one size whose dst
// and src both advance by a constant pitch no smaller than that size (rows
// that cannot overlap) become one 2D copy, which the engine runs as a single
// command -- e.g. one layer's chunks in consecutive [2, chunk, H, D] slab
// slots, whose K planes lie one slot apart.
int64_t next_command(const uint64_t* dst, const uint64_t* src, const uint64_t* bytes, int64_t n, int64_t i,
                     CopyCommand* cmd) {
  int64_t j = i + 1;
  uint64_t total = bytes[i];
  while (j < n && dst[j] == dst[j - 1] + bytes[j - 1] && src[j] == src[j - 1] + bytes[j - 1]) total += bytes[j++];
  if (j - i >= 2) {
    *cmd = {dst[i], src[i], total, 1, 0, 0};
    return j - i;
  }
  const uint64_t w = bytes[i];
  if (i + 1 < n && bytes[i + 1] == w) {
    // unsigned differences: a backward step wraps far above kMaxCopyPitch
    const uint64_t dp = dst[i + 1] - dst[i], sp = src[i + 1] - src[i];
    if (dp >= w && sp >= w && dp <= kMaxCopyPitch && sp <= kMaxCopyPitch) {
      j = i + 2;
      while (j < n && bytes[j] == w && dst[j] - dst[j - 1] == dp && src[j] - src[j - 1] == sp) ++j;
      *cmd = {dst[i], src[i], w, uint64_t(j - i), dp, sp};
      return j - i;
    }
  }
  *cmd = {dst[i], src[i], w, 1, 0, 0};
  return 1;
}

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
  for (int64_t i = 0; i < n; ++i)
    CBK_REQUIRE(bytes[i] == 0 || (dst[i] != 0 && src[i] != 0), "run %lld has a NULL address", (long long)i);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  for (int64_t i = 0; i < n;) {
    if (bytes[i] == 0) {
      ++i;
      continue;
    }
    CopyCommand c;
    const int64_t covered = next_command(dst, src, bytes, n, i, &c);
    void* d = reinterpret_cast<void*>(c.dst);
    const void* from = reinterpret_cast<const void*>(c.src);
    hipError_t err = c.rows == 1
                         ? hipMemcpyAsync(d, from, size_t(c.width), hipMemcpyDefault, s)
                         : hipMemcpy2DAsync(d, size_t(c.dpitch), from, size_t(c.spitch), size_t(c.width),
                                            size_t(c.rows), hipMemcpyDefault, s);
    if (err == hipErrorInvalidValue && covered > 1) {
      // Folded runs can lie in different allocations whose addresses merely
      // happen to line up (two pinned tensors, two slab arenas); the runtime
      // checks a command's whole extent against one allocation and rejects
      // it before enqueueing anything. Each run lies in one allocation, so
      // the group goes out run by run.
      (void)hipGetLastError();
      err = hipSuccess;
      for (int64_t j = i; j < i + covered && err == hipSuccess; ++j) {
        if (bytes[j] == 0) continue;
        err = hipMemcpyAsync(reinterpret_cast<void*>(dst[j]), reinterpret_cast<const void*>(src[j]),
                             size_t(bytes[j]), hipMemcpyDefault, s);
      }
    }
    if (err != hipSuccess)
      return cbk::set_error(CBK_ERR_LAUNCH, "copy of runs %lld..%lld: %s", (long long)i,
                            (long long)(i + covered - 1), hipGetErrorString(err));
    i += covered;
  }
  return CBK_OK;
}

int cbk_memcpy_runs_commands(const uint64_t* dst, const uint64_t* src, const uint64_t* bytes, int64_t n,
                             int64_t* commands) {
  cbk::clear_error();
  CBK_REQUIRE(commands != nullptr, "commands is NULL");
  CBK_REQUIRE(n >= 0, "negative run count");
  *commands = 0;
  if (n == 0) return CBK_OK;
  CBK_REQUIRE(dst != nullptr && src != nullptr && bytes != nullptr, "NULL run table");
  for (int64_t i = 0; i < n;) {
    if (bytes[i] == 0) {
      ++i;
      continue;
    }
    CopyCommand c;
    i += next_command(dst, src, bytes, n, i, &c);
    ++*commands;
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
