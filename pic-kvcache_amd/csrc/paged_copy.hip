// Paged KV gather/scatter for gfx950: the bandwidth kernels behind
// gather_paged_kv / scatter_paged_kv (reference cacheblend_vllm/kv_layout.py).
//
// Work decomposition. A "row" is one token's [H, D] slice of one plane (K or
// V): row_bytes contiguous bytes on both the page side and the contiguous
// side. Rows are split into VEC-byte vectors (16 B when every pointer and
// stride allows it), and vector f of a launch is
//     row = f / row_vecs, j = f % row_vecs,
//     plane = row >= T, token = row - plane * T          (plane-major)
// so consecutive lanes walk consecutive 16 B of one row (fully coalesced
// 64-lane x 16 B = 1 KiB wavefront accesses), a wavefront covers whole
// (token, head) rows, and neighbouring workgroups touch neighbouring tokens
// of the same plane, i.e. the same 16-token page block (DRAM page locality;
// token-major interleaving of K and V measured ~5% slower). Each thread
// issues all its loads before its stores to keep bytes in flight per CU.
// Loads and stores are non-temporal: nothing is re-read, so the copy stays
// out of L2/MALL (+10% on gfx950 against plain accesses).
// blockIdx.y selects the layer, so one launch moves up to kMaxLayers layers;
// one-layer launches use a kernel with a small argument block.
#include "cbk_common.hpp"

namespace cbk {
namespace {

// Launch shapes from a sweep on the 36-layer, 8 KV-head store workload:
// gather 512 threads, scatter 256, one 16-byte vector per thread (more,
// smaller workgroups beat 2 vectors per thread by 2-3%; 8 per thread halves
// the scatter rate).
constexpr int kGatherThreads = 512;
constexpr int kScatterThreads = 256;
constexpr int kUnroll = 1;
constexpr int kMaxLayers = 64;

// Launch geometry shared by the single- and multi-layer kernels.
struct PagedGeom {
  char* c_base;             // contiguous side: layer 0, plane K, token 0
  int64_t c_layer_stride;   // bytes
  int64_t c_plane_stride;   // bytes (V minus K, may be negative)
  int64_t c_token_stride;   // bytes
  const int64_t* slots;
  int64_t block_stride;     // page side, bytes
  int64_t token_stride;     // page side, bytes
  int32_t* bad;             // optional out-of-range slot counter
  uint32_t num_tokens;
  uint32_t planes;          // 2: K and V; 1: K only
  uint32_t row_vecs;
  uint32_t num_slots;
  FastDiv row_div;          // by row_vecs
  FastDiv bs_div;           // by block_size
};

// Multi-layer launches carry the layers' base pointers in the arguments.
struct PagedArgs {
  const char* k_base[kMaxLayers];
  const char* v_base[kMaxLayers];
  PagedGeom g;
};

// kWaveRow: every row is a whole number of 64-lane waves (row_vecs % 64 ==
// 0), so a wave's token, plane and slot are wave-uniform: the slot comes
// through the scalar cache instead of a 64-lane vector load, which shortens
// the slot -> data dependent-load chain each one-shot wave waits on.
template <int VEC, bool GATHER, int kThreads, bool kWaveRow>
__device__ __forceinline__ void paged_copy_body(const PagedGeom& a, const char* kb, const char* vb, char* cb) {
  using V = typename Vec<VEC>::T;
  const uint32_t total = a.num_tokens * a.planes * a.row_vecs;
  const uint32_t f0 = blockIdx.x * uint32_t(kThreads * kUnroll) + threadIdx.x;

  const char* page[kUnroll];
  char* cont[kUnroll];
  bool valid[kUnroll];
  bool live[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const uint32_t f = f0 + uint32_t(u * kThreads);
    live[u] = f < total;
    valid[u] = false;
    page[u] = nullptr;
    cont[u] = nullptr;
    if (live[u]) {
      uint32_t row = a.row_div.div(f);
      const uint32_t j = f - row * a.row_vecs;
      // kWaveRow: f - lane is a multiple of 64 and so of row_vecs' factor
      // 64, so lane 0's row is every lane's
      if (kWaveRow) row = __builtin_amdgcn_readfirstlane(row);
      const uint32_t c = row >= a.num_tokens ? 1u : 0u;
      const uint32_t t = row - c * a.num_tokens;
      // a scalar load runs even where exec is 0: keep its address inside
      // slots[] for a dead wave past the end (t is in range for live ones)
      const int64_t slot = a.slots[kWaveRow ? min(t, a.num_tokens - 1) : t];
      valid[u] = slot >= 0 && slot < int64_t(a.num_slots);
      if (valid[u]) {
        const uint32_t s32 = uint32_t(slot);
        const uint32_t blk = a.bs_div.div(s32);
        const uint32_t off = s32 - blk * a.bs_div.d;
        page[u] = (c ? vb : kb) + int64_t(blk) * a.block_stride + int64_t(off) * a.token_stride +
                  int64_t(j) * VEC;
      } else if (a.bad != nullptr && c == 0 && j == 0) {
        atomicAdd(a.bad, 1);
      }
      cont[u] = cb + int64_t(c) * a.c_plane_stride + int64_t(t) * a.c_token_stride + int64_t(j) * VEC;
    }
  }
  V buf[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    if (GATHER) {
      buf[u] = V(0);
      if (valid[u]) buf[u] = __builtin_nontemporal_load(reinterpret_cast<const V*>(page[u]));
    } else if (live[u]) {
      buf[u] = __builtin_nontemporal_load(reinterpret_cast<const V*>(cont[u]));
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    if (GATHER) {
      if (live[u]) __builtin_nontemporal_store(buf[u], reinterpret_cast<V*>(cont[u]));
    } else if (valid[u]) {
      __builtin_nontemporal_store(buf[u], reinterpret_cast<V*>(const_cast<char*>(page[u])));
    }
  }
}

// blockIdx.y selects the layer
template <int VEC, bool GATHER, int kThreads, bool kWaveRow>
__global__ __launch_bounds__(kThreads) void paged_copy_kernel(const PagedArgs a) {
  const uint32_t layer = blockIdx.y;
  paged_copy_body<VEC, GATHER, kThreads, kWaveRow>(a.g, a.k_base[layer], a.v_base[layer],
                                                   a.g.c_base + int64_t(layer) * a.g.c_layer_stride);
}

// One layer: a ~100-byte argument block instead of the 1 KiB table, which
// every short-lived wave would otherwise fetch (measured 4% on a one-layer
// 30,719-token scatter).
template <int VEC, bool GATHER, int kThreads, bool kWaveRow>
__global__ __launch_bounds__(kThreads) void paged_copy1_kernel(const PagedGeom g, const char* kb, const char* vb) {
  paged_copy_body<VEC, GATHER, kThreads, kWaveRow>(g, kb, vb, g.c_base);
}

// Copies between pages and chunks: token t of a batch is row t % chunk_tokens
// of chunk t / chunk_tokens, each chunk plane being a [chunk_tokens, row]
// block at chunk_k[c] / chunk_v[c] (pinned host memory addressed over PCIe,
// or device memory). A bounded grid walks the batch with a stride; over the
// host link the rate grows with the CUs issuing (about 1.2-1.6 GB/s each),
// so the caller trades link rate against CUs left to the serving stream.
constexpr int kChunksPerLaunch = 64;
constexpr int kChunkThreads = 256;
constexpr int kChunkUnroll = 4;

struct ChunkArgs {
  char* chunk_k[kChunksPerLaunch];
  char* chunk_v[kChunksPerLaunch];
  const char* k_base;
  const char* v_base;
  const int64_t* slots;
  int64_t block_stride;
  int64_t token_stride;
  int64_t chunk_token_stride;  // bytes between tokens inside a chunk plane
  int32_t* bad;
  uint32_t num_tokens;         // tokens in this launch (<= 64 chunks)
  uint32_t row_vecs;
  uint32_t num_slots;
  FastDiv row_div;
  FastDiv bs_div;
  FastDiv chunk_div;
};

// One pass of the chunk copy. GATHER: page rows -> chunk rows (the store:
// chunks in pinned host memory are written over the host link; a token with
// an out-of-range slot gets a zero row). Scatter: chunk rows -> page rows
// (the reload: chunks are read over the host link; out-of-range slots are
// skipped). kChunkUnroll vectors per thread, all loads before the stores.
template <int VEC, bool GATHER>
__device__ __forceinline__ void chunks_body(const ChunkArgs& a) {
  using V = typename Vec<VEC>::T;
  const uint32_t total = a.num_tokens * 2u * a.row_vecs;
  const uint32_t stride = gridDim.x * uint32_t(kChunkThreads * kChunkUnroll);
  for (uint32_t base = blockIdx.x * uint32_t(kChunkThreads * kChunkUnroll) + threadIdx.x; base < total;
       base += stride) {
    V buf[kChunkUnroll];
    char* dst[kChunkUnroll];
#pragma unroll
    for (int u = 0; u < kChunkUnroll; ++u) {
      const uint32_t f = base + uint32_t(u * kChunkThreads);
      dst[u] = nullptr;
      buf[u] = V(0);
      if (f < total) {
        const uint32_t row = a.row_div.div(f);
        const uint32_t j = f - row * a.row_vecs;
        const uint32_t c = row >= a.num_tokens ? 1u : 0u;
        const uint32_t t = row - c * a.num_tokens;
        const uint32_t ck = a.chunk_div.div(t);
        const uint32_t r = t - ck * a.chunk_div.d;
        char* chunk = (c ? a.chunk_v[ck] : a.chunk_k[ck]) + int64_t(r) * a.chunk_token_stride + int64_t(j) * VEC;
        const int64_t slot = a.slots[t];
        const bool ok = slot >= 0 && slot < int64_t(a.num_slots);
        char* page = nullptr;
        if (ok) {
          const uint32_t s32 = uint32_t(slot);
          const uint32_t blk = a.bs_div.div(s32);
          const uint32_t off = s32 - blk * a.bs_div.d;
          page = const_cast<char*>(c ? a.v_base : a.k_base) + int64_t(blk) * a.block_stride +
                 int64_t(off) * a.token_stride + int64_t(j) * VEC;
        } else if (a.bad != nullptr && c == 0 && j == 0) {
          atomicAdd(a.bad, 1);
        }
        if (GATHER) {
          dst[u] = chunk;
          if (ok) buf[u] = __builtin_nontemporal_load(reinterpret_cast<const V*>(page));
        } else if (ok) {
          dst[u] = page;
          buf[u] = *reinterpret_cast<const V*>(chunk);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kChunkUnroll; ++u) {
      if (dst[u] == nullptr) continue;
      if (GATHER) *reinterpret_cast<V*>(dst[u]) = buf[u];
      else __builtin_nontemporal_store(buf[u], reinterpret_cast<V*>(dst[u]));
    }
  }
}

template <int VEC>
__global__ __launch_bounds__(kChunkThreads) void gather_chunks_kernel(const ChunkArgs a) {
  chunks_body<VEC, true>(a);
}

template <int VEC>
__global__ __launch_bounds__(kChunkThreads) void scatter_chunks_kernel(const ChunkArgs a) {
  chunks_body<VEC, false>(a);
}

int validate_desc(const cbk_kv_desc* kv, int planes = 2) {
  CBK_REQUIRE(kv != nullptr, "kv descriptor is NULL");
  CBK_REQUIRE(kv->k_base != nullptr && (kv->v_base != nullptr || planes == 1), "kv base pointer is NULL");
  CBK_REQUIRE(kv->num_blocks > 0 && kv->block_size > 0, "num_blocks and block_size must be positive");
  CBK_REQUIRE(kv->row_bytes > 0, "row_bytes must be positive");
  CBK_REQUIRE(kv->num_blocks * kv->block_size < (int64_t(1) << 32),
              "num_blocks * block_size must be below 2^32");
  CBK_REQUIRE(kv->token_stride >= kv->row_bytes, "token_stride smaller than a row");
  CBK_REQUIRE(kv->block_stride >= kv->token_stride * kv->block_size || kv->block_size == 1,
              "block_stride smaller than a block");
  return CBK_OK;
}

int launch_paged(bool gather, const cbk_kv_desc* kv, int32_t num_layers, const int64_t* slots,
                 int64_t num_tokens, char* c_base, int64_t c_layer_stride, int64_t c_plane_stride,
                 int64_t c_token_stride, int32_t* bad, hipStream_t stream, int planes = 2) {
  clear_error();
  if (int rc = validate_desc(kv, planes)) return rc;
  CBK_REQUIRE(num_layers >= 1, "num_layers must be >= 1");
  CBK_REQUIRE(num_tokens >= 0, "num_tokens must be >= 0");
  if (num_tokens == 0) return CBK_OK;
  CBK_REQUIRE(slots != nullptr && c_base != nullptr, "slots/contiguous pointer is NULL");
  CBK_REQUIRE(c_token_stride >= kv->row_bytes, "contiguous token stride smaller than a row");
  for (int32_t l = 1; l < num_layers; ++l) {
    CBK_REQUIRE(kv[l].num_blocks == kv[0].num_blocks && kv[l].block_size == kv[0].block_size &&
                    kv[l].block_stride == kv[0].block_stride &&
                    kv[l].token_stride == kv[0].token_stride && kv[l].row_bytes == kv[0].row_bytes,
                "layer %d geometry differs from layer 0", int(l));
    CBK_REQUIRE(kv[l].k_base != nullptr && kv[l].v_base != nullptr, "layer %d base is NULL", int(l));
  }

  // widest access that every address and stride allows
  int64_t align_vals[8] = {kv->row_bytes, kv->block_stride, kv->token_stride, c_token_stride,
                           c_plane_stride, c_layer_stride, int64_t(reinterpret_cast<uintptr_t>(c_base)),
                           0};
  int vec = common_vec_bytes(align_vals, 7);
  for (int32_t l = 0; l < num_layers; ++l) {
    int64_t p[2] = {int64_t(reinterpret_cast<uintptr_t>(kv[l].k_base)),
                    int64_t(reinterpret_cast<uintptr_t>(kv[l].v_base))};
    vec = std::min(vec, common_vec_bytes(p, 2));
  }
  const int64_t row_vecs = kv->row_bytes / vec;
  CBK_REQUIRE(num_tokens * planes * row_vecs < (int64_t(1) << 32),
              "too many vectors in one launch (%lld tokens)", (long long)num_tokens);

  PagedGeom g;
  g.c_base = c_base;
  g.c_layer_stride = c_layer_stride;
  g.c_plane_stride = c_plane_stride;
  g.c_token_stride = c_token_stride;
  g.slots = slots;
  g.block_stride = kv->block_stride;
  g.token_stride = kv->token_stride;
  g.bad = bad;
  g.num_tokens = uint32_t(num_tokens);
  g.planes = uint32_t(planes);
  g.row_vecs = uint32_t(row_vecs);
  g.num_slots = uint32_t(kv->num_blocks * kv->block_size);
  g.row_div = FastDiv::make(uint32_t(row_vecs));
  g.bs_div = FastDiv::make(uint32_t(kv->block_size));

  const uint64_t total = uint64_t(num_tokens) * uint64_t(planes) * uint64_t(row_vecs);
  const int threads = gather ? kGatherThreads : kScatterThreads;
  const uint32_t grid_x = uint32_t((total + threads * kUnroll - 1) / (threads * kUnroll));
  // whole waves per row (workgroups and unroll steps are whole waves)
  static_assert(kGatherThreads % 64 == 0 && kScatterThreads % 64 == 0, "threads in whole waves");
  const bool wave_row = row_vecs % 64 == 0;

  if (num_layers == 1) {
    const char* kb = static_cast<const char*>(kv->k_base);
    const char* vb = static_cast<const char*>(kv->v_base);
    dim3 grid(grid_x);
#define CBK_LAUNCH_PAGED1(V)                                                             \
  if (gather && wave_row)                                                                \
    hipLaunchKernelGGL((paged_copy1_kernel<V, true, kGatherThreads, true>), grid,        \
                       dim3(kGatherThreads), 0, stream, g, kb, vb);                      \
  else if (gather)                                                                       \
    hipLaunchKernelGGL((paged_copy1_kernel<V, true, kGatherThreads, false>), grid,       \
                       dim3(kGatherThreads), 0, stream, g, kb, vb);                      \
  else if (wave_row)                                                                     \
    hipLaunchKernelGGL((paged_copy1_kernel<V, false, kScatterThreads, true>), grid,      \
                       dim3(kScatterThreads), 0, stream, g, kb, vb);                     \
  else                                                                                   \
    hipLaunchKernelGGL((paged_copy1_kernel<V, false, kScatterThreads, false>), grid,     \
                       dim3(kScatterThreads), 0, stream, g, kb, vb);
    switch (vec) {
      case 16: CBK_LAUNCH_PAGED1(16); break;
      case 8: CBK_LAUNCH_PAGED1(8); break;
      case 4: CBK_LAUNCH_PAGED1(4); break;
      case 2: CBK_LAUNCH_PAGED1(2); break;
      default: CBK_LAUNCH_PAGED1(1); break;
    }
#undef CBK_LAUNCH_PAGED1
    return launch_status(gather ? "paged gather" : "paged scatter");
  }
  for (int32_t l0 = 0; l0 < num_layers; l0 += kMaxLayers) {
    const int32_t nl = std::min(kMaxLayers, num_layers - l0);
    PagedArgs al;
    for (int32_t i = 0; i < kMaxLayers; ++i) {
      const cbk_kv_desc& d = kv[l0 + (i < nl ? i : 0)];
      al.k_base[i] = static_cast<const char*>(d.k_base);
      al.v_base[i] = static_cast<const char*>(d.v_base);
    }
    al.g = g;
    al.g.c_base = c_base + int64_t(l0) * c_layer_stride;
    dim3 grid(grid_x, uint32_t(nl));
#define CBK_LAUNCH_PAGED(V)                                                              \
  if (gather && wave_row)                                                                \
    hipLaunchKernelGGL((paged_copy_kernel<V, true, kGatherThreads, true>), grid,         \
                       dim3(kGatherThreads), 0, stream, al);                             \
  else if (gather)                                                                       \
    hipLaunchKernelGGL((paged_copy_kernel<V, true, kGatherThreads, false>), grid,        \
                       dim3(kGatherThreads), 0, stream, al);                             \
  else if (wave_row)                                                                     \
    hipLaunchKernelGGL((paged_copy_kernel<V, false, kScatterThreads, true>), grid,       \
                       dim3(kScatterThreads), 0, stream, al);                            \
  else                                                                                   \
    hipLaunchKernelGGL((paged_copy_kernel<V, false, kScatterThreads, false>), grid,      \
                       dim3(kScatterThreads), 0, stream, al);
    switch (vec) {
      case 16: CBK_LAUNCH_PAGED(16); break;
      case 8: CBK_LAUNCH_PAGED(8); break;
      case 4: CBK_LAUNCH_PAGED(4); break;
      case 2: CBK_LAUNCH_PAGED(2); break;
      default: CBK_LAUNCH_PAGED(1); break;
    }
#undef CBK_LAUNCH_PAGED
    if (int rc = launch_status(gather ? "paged gather" : "paged scatter")) return rc;
  }
  return CBK_OK;
}

int launch_chunks(bool gather, const cbk_kv_desc* kv, const int64_t* slots, int64_t num_tokens,
                  int64_t chunk_tokens, void* const* chunk_k, void* const* chunk_v,
                  int64_t chunk_token_stride, int32_t max_workgroups, int32_t* bad,
                  hipStream_t stream) {
  clear_error();
  if (int rc = validate_desc(kv)) return rc;
  CBK_REQUIRE(num_tokens >= 0 && chunk_tokens > 0, "num_tokens/chunk_tokens invalid");
  if (num_tokens == 0) return CBK_OK;
  CBK_REQUIRE(slots && chunk_k && chunk_v, "NULL pointer");
  CBK_REQUIRE(chunk_token_stride >= kv->row_bytes, "chunk token stride smaller than a row");
  const int64_t nchunks = (num_tokens + chunk_tokens - 1) / chunk_tokens;
  int64_t align[6] = {kv->row_bytes, kv->block_stride, kv->token_stride, chunk_token_stride,
                      int64_t(reinterpret_cast<uintptr_t>(kv->k_base)),
                      int64_t(reinterpret_cast<uintptr_t>(kv->v_base))};
  int vec = common_vec_bytes(align, 6);
  for (int64_t c = 0; c < nchunks; ++c) {
    CBK_REQUIRE(chunk_k[c] && chunk_v[c], "chunk %lld destination is NULL", (long long)c);
    int64_t p[2] = {int64_t(reinterpret_cast<uintptr_t>(chunk_k[c])),
                    int64_t(reinterpret_cast<uintptr_t>(chunk_v[c]))};
    vec = std::min(vec, common_vec_bytes(p, 2));
  }
  const int64_t row_vecs = kv->row_bytes / vec;
  const int64_t per_launch = chunk_tokens * kChunksPerLaunch;
  CBK_REQUIRE(std::min(per_launch, num_tokens) * 2 * row_vecs < (int64_t(1) << 32), "launch too large");
  const uint32_t grid_cap = uint32_t(max_workgroups > 0 ? max_workgroups : 64);
  ChunkArgs a{};
  a.k_base = static_cast<const char*>(kv->k_base);
  a.v_base = static_cast<const char*>(kv->v_base);
  a.block_stride = kv->block_stride;
  a.token_stride = kv->token_stride;
  a.chunk_token_stride = chunk_token_stride;
  a.bad = bad;
  a.row_vecs = uint32_t(row_vecs);
  a.num_slots = uint32_t(kv->num_blocks * kv->block_size);
  a.row_div = FastDiv::make(uint32_t(row_vecs));
  a.bs_div = FastDiv::make(uint32_t(kv->block_size));
  a.chunk_div = FastDiv::make(uint32_t(chunk_tokens));
  for (int64_t t0 = 0; t0 < num_tokens; t0 += per_launch) {
    const int64_t n = std::min(per_launch, num_tokens - t0);
    const int64_t c0 = t0 / chunk_tokens;
    const int64_t nc = (n + chunk_tokens - 1) / chunk_tokens;
    for (int64_t c = 0; c < kChunksPerLaunch; ++c) {
      a.chunk_k[c] = static_cast<char*>(chunk_k[c0 + (c < nc ? c : 0)]);
      a.chunk_v[c] = static_cast<char*>(chunk_v[c0 + (c < nc ? c : 0)]);
    }
    a.slots = slots + t0;
    a.num_tokens = uint32_t(n);
    const uint64_t total = uint64_t(n) * 2 * uint64_t(row_vecs);
    const uint32_t grid = uint32_t(std::min<uint64_t>(
        grid_cap, (total + kChunkThreads * kChunkUnroll - 1) / (kChunkThreads * kChunkUnroll)));
#define CBK_LAUNCH_CHUNKS(V)                                                                          \
  if (gather)                                                                                         \
    hipLaunchKernelGGL(gather_chunks_kernel<V>, dim3(grid), dim3(kChunkThreads), 0, stream, a);       \
  else                                                                                                \
    hipLaunchKernelGGL(scatter_chunks_kernel<V>, dim3(grid), dim3(kChunkThreads), 0, stream, a);
    switch (vec) {
      case 16: CBK_LAUNCH_CHUNKS(16); break;
      case 8: CBK_LAUNCH_CHUNKS(8); break;
      case 4: CBK_LAUNCH_CHUNKS(4); break;
      case 2: CBK_LAUNCH_CHUNKS(2); break;
      default: CBK_LAUNCH_CHUNKS(1); break;
    }
#undef CBK_LAUNCH_CHUNKS
    if (int rc = launch_status(gather ? "paged gather to chunks" : "paged scatter from chunks")) return rc;
  }
  return CBK_OK;
}

// K plane only when the V pointers on both sides are NULL
int planes_of(const cbk_kv_desc* kv, const void* contiguous_v, int64_t num_tokens, int* planes) {
  *planes = 2;
  if (kv != nullptr && kv->v_base == nullptr && contiguous_v == nullptr) *planes = 1;
  else if (num_tokens > 0 && contiguous_v == nullptr)
    return set_error(CBK_ERR_INVALID, "V pointer is NULL while the descriptor has a V plane");
  return CBK_OK;
}

}  // namespace
}  // namespace cbk

extern "C" {

int cbk_paged_gather_chunks(const cbk_kv_desc* kv, const int64_t* slots_dev, int64_t num_tokens,
                            int64_t chunk_tokens, void* const* chunk_k, void* const* chunk_v,
                            int64_t chunk_token_stride, int32_t max_workgroups,
                            int32_t* bad_slots_dev, cbk_stream_t stream) {
  return cbk::launch_chunks(true, kv, slots_dev, num_tokens, chunk_tokens, chunk_k, chunk_v,
                            chunk_token_stride, max_workgroups, bad_slots_dev,
                            static_cast<hipStream_t>(stream));
}

int cbk_paged_scatter_chunks(const void* const* chunk_k, const void* const* chunk_v, int64_t chunk_tokens,
                             int64_t chunk_token_stride, const cbk_kv_desc* kv, const int64_t* slots_dev,
                             int64_t num_tokens, int32_t max_workgroups, int32_t* bad_slots_dev,
                             cbk_stream_t stream) {
  return cbk::launch_chunks(false, kv, slots_dev, num_tokens, chunk_tokens, const_cast<void* const*>(chunk_k),
                            const_cast<void* const*>(chunk_v), chunk_token_stride, max_workgroups,
                            bad_slots_dev, static_cast<hipStream_t>(stream));
}

int cbk_paged_gather(const cbk_kv_desc* kv, const int64_t* slots_dev, int64_t num_tokens,
                     void* out_k_dev, void* out_v_dev, int64_t out_token_stride,
                     int32_t* bad_slots_dev, cbk_stream_t stream) {
  if (num_tokens > 0 && out_k_dev == nullptr) return cbk::set_error(CBK_ERR_INVALID, "output pointer is NULL");
  int planes = 2;
  if (int rc = cbk::planes_of(kv, out_v_dev, num_tokens, &planes)) return rc;
  char* k = static_cast<char*>(out_k_dev);
  const int64_t plane = planes == 2 ? static_cast<char*>(out_v_dev) - k : 0;
  return cbk::launch_paged(true, kv, 1, slots_dev, num_tokens, k, 0, plane, out_token_stride,
                           bad_slots_dev, static_cast<hipStream_t>(stream), planes);
}

int cbk_paged_scatter(const void* in_k_dev, const void* in_v_dev, int64_t in_token_stride,
                      const cbk_kv_desc* kv, const int64_t* slots_dev, int64_t num_tokens,
                      int32_t* bad_slots_dev, cbk_stream_t stream) {
  if (num_tokens > 0 && in_k_dev == nullptr) return cbk::set_error(CBK_ERR_INVALID, "input pointer is NULL");
  int planes = 2;
  if (int rc = cbk::planes_of(kv, in_v_dev, num_tokens, &planes)) return rc;
  char* k = const_cast<char*>(static_cast<const char*>(in_k_dev));
  const int64_t plane = planes == 2 ? static_cast<const char*>(in_v_dev) - k : 0;
  return cbk::launch_paged(false, kv, 1, slots_dev, num_tokens, k, 0, plane, in_token_stride,
                           bad_slots_dev, static_cast<hipStream_t>(stream), planes);
}

int cbk_paged_gather_layers(const cbk_kv_desc* kv, int32_t num_layers, const int64_t* slots_dev,
                            int64_t num_tokens, void* out_dev, int64_t out_layer_stride,
                            int64_t out_plane_stride, int64_t out_token_stride,
                            int32_t* bad_slots_dev, cbk_stream_t stream) {
  return cbk::launch_paged(true, kv, num_layers, slots_dev, num_tokens, static_cast<char*>(out_dev),
                           out_layer_stride, out_plane_stride, out_token_stride, bad_slots_dev,
                           static_cast<hipStream_t>(stream));
}

int cbk_paged_scatter_layers(const void* in_dev, int64_t in_layer_stride, int64_t in_plane_stride,
                             int64_t in_token_stride, const cbk_kv_desc* kv, int32_t num_layers,
                             const int64_t* slots_dev, int64_t num_tokens, int32_t* bad_slots_dev,
                             cbk_stream_t stream) {
  return cbk::launch_paged(false, kv, num_layers, slots_dev, num_tokens,
                           const_cast<char*>(static_cast<const char*>(in_dev)), in_layer_stride,
                           in_plane_stride, in_token_stride, bad_slots_dev,
                           static_cast<hipStream_t>(stream));
}

}  // extern "C"
