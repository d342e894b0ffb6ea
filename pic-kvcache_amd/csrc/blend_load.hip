// Layerwise blend-buffer assembly for gfx950: one kernel builds the whole
// [2, allocation_end, H, D] buffer a layer's prefetch produces, replacing
// four passes of the reference loader (cacheblend_vllm/ascend.py):
//   APC prefix gather from the pages           (ascend.py:232-247)
//   zeroing of every gap                        (ascend.py:280-287)
//   placement of the H2D-staged hit rows        (ascend.py:358-370)
//   RoPE delta relocation of the hit K rows     (ascend.py:52-103, 357)
// Each buffer row p (per plane) has a source in src_map[p]:
//   >= 0  row of the hit staging (K relocated from old_pos[row] to new_pos[p])
//   -1    zero (gap)
//   -2    page slot slots[p] (APC prefix)
// One 64-lane wavefront handles one (plane, token) row at a time, 16-byte
// vectors across the row; a relocated K row is handled as rotation pairs.
//
// Relocation arithmetic reproduces torch's eager elementwise kernels in the
// key dtype: every product, sum and difference is computed in float32 and
// rounded to the key dtype (bf16/f16 round-to-nearest-even; float32 with no
// fused multiply-add), with the cos/sin table already in the key dtype, so
// the result is bit-identical to the reference's relocate_key on the same
// inputs.
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include "cbk_common.hpp"

// torch's eager float32 kernels round every product and sum separately; hipcc
// would otherwise fuse a*b - c*d into an FMA (-ffp-contract=fast). The
// operators below are written in this file so the pragma covers them.
#pragma clang fp contract(off)

namespace cbk {
namespace {

constexpr int kAsmThreads = 256;
constexpr int kRowsPerWave = 2;

struct AssembleArgs {
  char* out_k;
  char* out_v;               // nullptr: K plane only
  int64_t out_tok_stride;    // bytes
  const char* page_k;
  const char* page_v;
  int64_t block_stride;      // bytes
  int64_t token_stride;      // bytes
  uint32_t num_slots;
  FastDiv bs_div;
  const int64_t* slots;      // [num_tokens]
  const int32_t* src_map;    // [num_tokens]
  const char* hit_k;
  const char* hit_v;
  int64_t hit_tok_stride;    // bytes
  uint32_t hit_rows;
  const int32_t* old_pos;    // [hit_rows]
  const int32_t* new_pos;    // [num_tokens] or nullptr (= p)
  const char* cos_sin;       // [cs_rows, head_dim] in the key dtype
  int64_t cs_row_stride;     // elements
  uint32_t cs_rows;
  uint32_t num_tokens;
  uint32_t row_bytes;
  uint32_t head_dim;
  uint32_t heads;
  int32_t relocate;
  int32_t neox;
  int32_t* bad;
  // host-chunk source: hit row h lives in chunk h / chunk_tokens at row
  // h % chunk_tokens; hit_chunks[2 * c] / [2 * c + 1] are its K / V planes
  const uint64_t* hit_chunks;
  FastDiv chunk_div;
  int64_t chunk_tok_stride;
  int32_t rows_path;         // assemble_rows_kernel applies (P = rows_path KiB passes)
};

// Rounding to the key dtype after every elementwise op (torch eager semantics).
template <typename T> struct KeyMath;
template <> struct KeyMath<float> {
  static __device__ __forceinline__ float load(const char* p) { return *reinterpret_cast<const float*>(p); }
  static __device__ __forceinline__ void store(char* p, float v) { *reinterpret_cast<float*>(p) = v; }
  static __device__ __forceinline__ float r(float v) { return v; }
  static __device__ __forceinline__ float mul(float a, float b) { return a * b; }
  static __device__ __forceinline__ float add(float a, float b) { return a + b; }
  static __device__ __forceinline__ float sub(float a, float b) { return a - b; }
};
template <> struct KeyMath<__hip_bfloat16> {
  static __device__ __forceinline__ float load(const char* p) {
    return __uint_as_float(uint32_t(*reinterpret_cast<const uint16_t*>(p)) << 16);
  }
  static __device__ __forceinline__ void store(char* p, float v) {
    *reinterpret_cast<__hip_bfloat16*>(p) = __float2bfloat16(v);
  }
  static __device__ __forceinline__ float r(float v) { return __bfloat162float(__float2bfloat16(v)); }
  static __device__ __forceinline__ float mul(float a, float b) { return r(a * b); }
  static __device__ __forceinline__ float add(float a, float b) { return r(a + b); }
  static __device__ __forceinline__ float sub(float a, float b) { return r(a - b); }
};
template <> struct KeyMath<__half> {
  static __device__ __forceinline__ float load(const char* p) {
    return __half2float(*reinterpret_cast<const __half*>(p));
  }
  static __device__ __forceinline__ void store(char* p, float v) {
    *reinterpret_cast<__half*>(p) = __float2half(v);
  }
  static __device__ __forceinline__ float r(float v) { return __half2float(__float2half(v)); }
  static __device__ __forceinline__ float mul(float a, float b) { return r(a * b); }
  static __device__ __forceinline__ float add(float a, float b) { return r(a + b); }
  static __device__ __forceinline__ float sub(float a, float b) { return r(a - b); }
};

template <int VEC>
__device__ __forceinline__ void copy_row(char* dst, const char* src, uint32_t row_bytes, uint32_t lane) {
  using V = typename Vec<VEC>::T;
  for (uint32_t b = lane * VEC; b < row_bytes; b += 64 * VEC) {
    V v = src ? *reinterpret_cast<const V*>(src + b) : V(0);
    __builtin_nontemporal_store(v, reinterpret_cast<V*>(dst + b));
  }
}

// K row relocation: rotation pairs (neox: i and i + D/2; interleaved: 2i and
// 2i + 1) of every head, angle delta = new - old taken from the cos/sin table.
template <typename T>
__device__ __forceinline__ void relocate_row(char* dst, const char* src, const AssembleArgs& a,
                                             uint32_t oldp, uint32_t newp, uint32_t lane) {
  using M = KeyMath<T>;
  constexpr uint32_t es = sizeof(T);
  const uint32_t half = a.head_dim / 2;
  const uint32_t pairs = a.heads * half;
  const char* co = a.cos_sin + int64_t(oldp) * a.cs_row_stride * es;
  const char* cn = a.cos_sin + int64_t(newp) * a.cs_row_stride * es;
  for (uint32_t q = lane; q < pairs; q += 64) {
    const uint32_t h = q / half;
    const uint32_t i = q - h * half;
    const float oc = M::load(co + i * es), os = M::load(co + (half + i) * es);
    const float nc = M::load(cn + i * es), ns = M::load(cn + (half + i) * es);
    const float dc = M::add(M::mul(nc, oc), M::mul(ns, os));
    const float ds = M::sub(M::mul(ns, oc), M::mul(nc, os));
    const uint32_t e1 = h * a.head_dim + (a.neox ? i : 2 * i);
    const uint32_t e2 = a.neox ? e1 + half : e1 + 1;
    const float x1 = M::load(src + e1 * es);
    const float x2 = M::load(src + e2 * es);
    M::store(dst + e1 * es, M::sub(M::mul(x1, dc), M::mul(x2, ds)));
    M::store(dst + e2 * es, M::add(M::mul(x2, dc), M::mul(x1, ds)));
  }
}

// Relocation of the 16 bytes (E = 16 / sizeof(T) elements) one lane holds
// of a K row, with the lane's cos/sin vectors cs = {cos(old), sin(old),
// cos(new), sin(new)} at its pair indices. Interleaved pairs sit inside the
// lane; a NeoX pair (i, i + D/2) sits in lanes `partner` = D/2/E apart
// within the head, so every lane fetches its partner's vector with a lane
// exchange (the caller keeps the whole wave converged here). Per element the
// arithmetic is relocate_row's, in the same order.
template <typename T>
__device__ __forceinline__ Vec<16>::T rotate_lane(Vec<16>::T own, const Vec<16>::T* cs, bool neox,
                                                  bool first, uint32_t partner) {
  using M = KeyMath<T>;
  using V4 = Vec<16>::T;
  constexpr uint32_t es = sizeof(T);
  constexpr uint32_t E = 16 / es;
  V4 res;
  const char* x = reinterpret_cast<const char*>(&own);
  char* y = reinterpret_cast<char*>(&res);
  const char* oc = reinterpret_cast<const char*>(&cs[0]);
  const char* os = reinterpret_cast<const char*>(&cs[1]);
  const char* nc = reinterpret_cast<const char*>(&cs[2]);
  const char* ns = reinterpret_cast<const char*>(&cs[3]);
  if (neox) {
    V4 other;
#pragma unroll
    for (int w = 0; w < 4; ++w) other[w] = uint32_t(__shfl_xor(int(own[w]), int(partner)));
    const char* xo = reinterpret_cast<const char*>(&other);
#pragma unroll
    for (uint32_t j = 0; j < E; ++j) {
      const float c0 = M::load(oc + j * es), s0 = M::load(os + j * es);
      const float c1 = M::load(nc + j * es), s1 = M::load(ns + j * es);
      const float dc = M::add(M::mul(c1, c0), M::mul(s1, s0));
      const float ds = M::sub(M::mul(s1, c0), M::mul(c1, s0));
      const float mine = M::load(x + j * es), theirs = M::load(xo + j * es);
      // first half: x1 * dc - x2 * ds; second half: x2 * dc + x1 * ds
      M::store(y + j * es, first ? M::sub(M::mul(mine, dc), M::mul(theirs, ds))
                                 : M::add(M::mul(mine, dc), M::mul(theirs, ds)));
    }
  } else {
#pragma unroll
    for (uint32_t k = 0; k < E / 2; ++k) {
      const float c0 = M::load(oc + k * es), s0 = M::load(os + k * es);
      const float c1 = M::load(nc + k * es), s1 = M::load(ns + k * es);
      const float dc = M::add(M::mul(c1, c0), M::mul(s1, s0));
      const float ds = M::sub(M::mul(s1, c0), M::mul(c1, s0));
      const float x1 = M::load(x + 2 * k * es), x2 = M::load(x + (2 * k + 1) * es);
      M::store(y + 2 * k * es, M::sub(M::mul(x1, dc), M::mul(x2, ds)));
      M::store(y + (2 * k + 1) * es, M::add(M::mul(x2, dc), M::mul(x1, ds)));
    }
  }
  return res;
}

// Rows R at a time per wave, 16-byte vectors, rows of at most P KiB: every
// load of the R rows -- source tables, row data and, for relocated K rows,
// the cos/sin vectors -- is issued before any store, so one wave keeps R*P
// KiB of row data in flight. That lets a few workgroups saturate the host
// link when hit rows are read from pinned host memory, leaving the other
// CUs to the layer's compute. Relocation requires head bytes dividing 1 KiB
// (a lane's position within its head is the same in every pass), E | D/2
// for NeoX and 16-byte aligned cos/sin rows.
template <typename T, int R, int P>
__global__ __launch_bounds__(kAsmThreads) void assemble_rows_kernel(const AssembleArgs a) {
  using V4 = Vec<16>::T;
  using V2 = Vec<8>::T;
  constexpr uint32_t es = sizeof(T);
  constexpr uint32_t E = 16 / es;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = blockIdx.x * (kAsmThreads / 64) + (threadIdx.x >> 6);
  const uint32_t nwaves = gridDim.x * (kAsmThreads / 64);
  const uint32_t rows = (a.out_v ? 2u : 1u) * a.num_tokens;
  const uint32_t half = a.head_dim / 2;
  const uint32_t partner = a.head_dim / E / 2;
  const uint32_t d0 = (lane * E) % a.head_dim;  // lane's first element within its head
  const bool first = d0 < half;
  const uint32_t i0 = a.neox ? (first ? d0 : d0 - half) : d0 / 2;
  for (uint32_t row0 = wave * R; row0 < rows; row0 += nwaves * R) {
    V4 v[R][P];
    V4 cs[R][4];
    char* dst[R];
    bool rot[R];
    bool bad[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t row = row0 + r;
      const char* src = nullptr;
      dst[r] = nullptr;
      rot[r] = false;
      bad[r] = false;
      if (row < rows) {
        const uint32_t c = row >= a.num_tokens ? 1u : 0u;
        const uint32_t p = row - c * a.num_tokens;
        dst[r] = (c ? a.out_v : a.out_k) + int64_t(p) * a.out_tok_stride;
        const int32_t s = a.src_map[p];
        if (s >= 0) {
          if (uint32_t(s) >= a.hit_rows) {
            bad[r] = c == 0;
          } else {
            if (a.hit_chunks != nullptr) {
              const uint32_t ck = a.chunk_div.div(uint32_t(s));
              const uint32_t rr = uint32_t(s) - ck * a.chunk_div.d;
              src = reinterpret_cast<const char*>(a.hit_chunks[2 * ck + c]) + int64_t(rr) * a.chunk_tok_stride;
            } else {
              src = (c ? a.hit_v : a.hit_k) + int64_t(s) * a.hit_tok_stride;
            }
            if (c == 0 && a.relocate) {
              const int32_t oldp = a.old_pos[s];
              const int32_t newp = a.new_pos ? a.new_pos[p] : int32_t(p);
              if (oldp < 0 || newp < 0 || uint32_t(oldp) >= a.cs_rows || uint32_t(newp) >= a.cs_rows) {
                src = nullptr;
                bad[r] = true;
              } else {
                rot[r] = true;
                const char* co = a.cos_sin + int64_t(oldp) * a.cs_row_stride * es;
                const char* cn = a.cos_sin + int64_t(newp) * a.cs_row_stride * es;
                if (a.neox) {
                  cs[r][0] = *reinterpret_cast<const V4*>(co + i0 * es);
                  cs[r][1] = *reinterpret_cast<const V4*>(co + (half + i0) * es);
                  cs[r][2] = *reinterpret_cast<const V4*>(cn + i0 * es);
                  cs[r][3] = *reinterpret_cast<const V4*>(cn + (half + i0) * es);
                } else {
                  const V2 q0 = *reinterpret_cast<const V2*>(co + i0 * es);
                  const V2 q1 = *reinterpret_cast<const V2*>(co + (half + i0) * es);
                  const V2 q2 = *reinterpret_cast<const V2*>(cn + i0 * es);
                  const V2 q3 = *reinterpret_cast<const V2*>(cn + (half + i0) * es);
                  cs[r][0] = V4{q0[0], q0[1], 0u, 0u};
                  cs[r][1] = V4{q1[0], q1[1], 0u, 0u};
                  cs[r][2] = V4{q2[0], q2[1], 0u, 0u};
                  cs[r][3] = V4{q3[0], q3[1], 0u, 0u};
                }
              }
            }
          }
        } else if (s == -2) {
          const int64_t slot = a.slots[p];
          if (slot < 0 || slot >= int64_t(a.num_slots)) {
            bad[r] = c == 0;
          } else {
            const uint32_t s32 = uint32_t(slot);
            const uint32_t blk = a.bs_div.div(s32);
            const uint32_t off = s32 - blk * a.bs_div.d;
            src = (c ? a.page_v : a.page_k) + int64_t(blk) * a.block_stride + int64_t(off) * a.token_stride;
          }
        }
      }
#pragma unroll
      for (int j = 0; j < P; ++j) {
        const uint32_t b = uint32_t(j) * 1024u + lane * 16u;
        v[r][j] = (src != nullptr && b < a.row_bytes) ? *reinterpret_cast<const V4*>(src + b) : V4(0u);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (dst[r] == nullptr) continue;
      if (bad[r] && lane == 0 && a.bad) atomicAdd(a.bad, 1);
#pragma unroll
      for (int j = 0; j < P; ++j) {
        const uint32_t b = uint32_t(j) * 1024u + lane * 16u;
        V4 out = v[r][j];
        if (rot[r]) out = rotate_lane<T>(out, cs[r], a.neox != 0, first, partner);
        if (b < a.row_bytes) __builtin_nontemporal_store(out, reinterpret_cast<V4*>(dst[r] + b));
      }
    }
  }
}

template <typename T, int VEC>
__global__ __launch_bounds__(kAsmThreads) void assemble_kernel(const AssembleArgs a) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = blockIdx.x * (kAsmThreads / 64) + (threadIdx.x >> 6);
  const uint32_t nwaves = gridDim.x * (kAsmThreads / 64);
  const uint32_t planes = a.out_v ? 2u : 1u;
  const uint32_t rows = planes * a.num_tokens;
  for (uint32_t row = wave; row < rows; row += nwaves) {
    const uint32_t c = row >= a.num_tokens ? 1u : 0u;
    const uint32_t p = row - c * a.num_tokens;
    char* dst = (c ? a.out_v : a.out_k) + int64_t(p) * a.out_tok_stride;
    const int32_t src = a.src_map[p];
    if (src >= 0) {
      if (uint32_t(src) >= a.hit_rows) {
        copy_row<VEC>(dst, nullptr, a.row_bytes, lane);
        if (lane == 0 && c == 0 && a.bad) atomicAdd(a.bad, 1);
        continue;
      }
      const char* in;
      if (a.hit_chunks != nullptr) {
        const uint32_t ck = a.chunk_div.div(uint32_t(src));
        const uint32_t r = uint32_t(src) - ck * a.chunk_div.d;
        in = reinterpret_cast<const char*>(a.hit_chunks[2 * ck + c]) + int64_t(r) * a.chunk_tok_stride;
      } else {
        in = (c ? a.hit_v : a.hit_k) + int64_t(src) * a.hit_tok_stride;
      }
      if (c == 0 && a.relocate) {
        const int32_t oldp = a.old_pos[src];
        const int32_t newp = a.new_pos ? a.new_pos[p] : int32_t(p);
        if (oldp < 0 || newp < 0 || uint32_t(oldp) >= a.cs_rows || uint32_t(newp) >= a.cs_rows) {
          copy_row<VEC>(dst, nullptr, a.row_bytes, lane);
          if (lane == 0 && a.bad) atomicAdd(a.bad, 1);
          continue;
        }
        relocate_row<T>(dst, in, a, uint32_t(oldp), uint32_t(newp), lane);
      } else {
        copy_row<VEC>(dst, in, a.row_bytes, lane);
      }
    } else if (src == -2) {
      const int64_t slot = a.slots[p];
      if (slot < 0 || slot >= int64_t(a.num_slots)) {
        copy_row<VEC>(dst, nullptr, a.row_bytes, lane);
        if (lane == 0 && c == 0 && a.bad) atomicAdd(a.bad, 1);
        continue;
      }
      const uint32_t s32 = uint32_t(slot);
      const uint32_t blk = a.bs_div.div(s32);
      const uint32_t off = s32 - blk * a.bs_div.d;
      const char* in = (c ? a.page_v : a.page_k) + int64_t(blk) * a.block_stride + int64_t(off) * a.token_stride;
      copy_row<VEC>(dst, in, a.row_bytes, lane);
    } else {
      copy_row<VEC>(dst, nullptr, a.row_bytes, lane);
    }
  }
}

template <typename T>
int launch_assemble_t(const AssembleArgs& a, int vec, uint32_t max_workgroups, hipStream_t stream) {
  const uint32_t planes = a.out_v ? 2u : 1u;
  const uint64_t rows = uint64_t(planes) * a.num_tokens;
  const uint64_t waves = (rows + kRowsPerWave - 1) / kRowsPerWave;
  uint64_t blocks = (waves + kAsmThreads / 64 - 1) / (kAsmThreads / 64);
  if (max_workgroups > 0) blocks = std::min<uint64_t>(blocks, max_workgroups);
  if (a.rows_path) {
    const uint32_t P = uint32_t(a.rows_path);
    const uint32_t R = 8 / P;
    uint64_t wg = (rows + uint64_t(R) * (kAsmThreads / 64) - 1) / (uint64_t(R) * (kAsmThreads / 64));
    if (max_workgroups > 0) wg = std::min<uint64_t>(wg, max_workgroups);
    const dim3 g(static_cast<uint32_t>(wg));
    switch (P) {
      case 1: hipLaunchKernelGGL((assemble_rows_kernel<T, 8, 1>), g, dim3(kAsmThreads), 0, stream, a); break;
      case 2: hipLaunchKernelGGL((assemble_rows_kernel<T, 4, 2>), g, dim3(kAsmThreads), 0, stream, a); break;
      default: hipLaunchKernelGGL((assemble_rows_kernel<T, 2, 4>), g, dim3(kAsmThreads), 0, stream, a); break;
    }
    return launch_status("blend assemble");
  }
  const dim3 grid(static_cast<uint32_t>(blocks));
  switch (vec) {
    case 16: hipLaunchKernelGGL((assemble_kernel<T, 16>), grid, dim3(kAsmThreads), 0, stream, a); break;
    case 8: hipLaunchKernelGGL((assemble_kernel<T, 8>), grid, dim3(kAsmThreads), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((assemble_kernel<T, 4>), grid, dim3(kAsmThreads), 0, stream, a); break;
    default: hipLaunchKernelGGL((assemble_kernel<T, 2>), grid, dim3(kAsmThreads), 0, stream, a); break;
  }
  return launch_status("blend assemble");
}

}  // namespace
}  // namespace cbk

namespace cbk {
namespace {
int assemble_impl(const cbk_kv_desc* kv, const int64_t* slots_dev, const int32_t* src_map_dev,
                  int64_t num_tokens, const void* hit_k_dev, const void* hit_v_dev,
                  int64_t hit_token_stride, int64_t hit_rows, const uint64_t* hit_chunks_dev,
                  int64_t chunk_tokens, int64_t chunk_token_stride, const int32_t* old_pos_dev,
                  const int32_t* new_pos_dev, const void* cos_sin_dev, int64_t cos_sin_row_stride_elems,
                  int64_t cos_sin_rows, int64_t heads, int64_t head_dim, int32_t relocate, int32_t neox,
                  int32_t dtype, void* out_k_dev, void* out_v_dev, int64_t out_token_stride,
                  int32_t* bad_dev, int32_t max_workgroups, cbk_stream_t stream) {
  clear_error();
  CBK_REQUIRE(num_tokens >= 0 && num_tokens < (int64_t(1) << 30), "num_tokens out of range");
  if (num_tokens == 0) return CBK_OK;
  CBK_REQUIRE(src_map_dev && out_k_dev, "src_map/out_k is NULL");
  CBK_REQUIRE(hit_rows >= 0 && hit_rows < (int64_t(1) << 31), "hit_rows out of range");
  CBK_REQUIRE(heads > 0 && head_dim > 0, "heads/head_dim must be positive");
  CBK_REQUIRE(!relocate || head_dim % 2 == 0, "relocation needs an even head_dim");
  CBK_REQUIRE(dtype == CBK_DTYPE_F32 || dtype == CBK_DTYPE_BF16 || dtype == CBK_DTYPE_F16,
              "dtype %d", int(dtype));
  const int64_t es = dtype == CBK_DTYPE_F32 ? 4 : 2;
  const int64_t row_bytes = heads * head_dim * es;
  CBK_REQUIRE(out_token_stride >= row_bytes, "output token stride smaller than a row");
  if (hit_rows > 0 && hit_chunks_dev == nullptr) {
    CBK_REQUIRE(hit_k_dev && (hit_v_dev || !out_v_dev), "hit staging pointer is NULL");
    CBK_REQUIRE(hit_token_stride >= row_bytes, "hit token stride smaller than a row");
  }
  if (hit_chunks_dev != nullptr) {
    CBK_REQUIRE(chunk_tokens > 0 && chunk_token_stride >= row_bytes, "chunk geometry invalid");
    CBK_REQUIRE(chunk_token_stride % 16 == 0, "chunk token stride must be a multiple of 16 bytes");
  }
  if (relocate) {
    CBK_REQUIRE(cos_sin_dev && old_pos_dev && cos_sin_rows > 0, "relocation needs cos_sin and old_pos");
    CBK_REQUIRE(cos_sin_row_stride_elems >= head_dim, "cos_sin row stride smaller than head_dim");
  }
  AssembleArgs a{};
  a.out_k = static_cast<char*>(out_k_dev);
  a.out_v = static_cast<char*>(out_v_dev);
  a.out_tok_stride = out_token_stride;
  a.slots = slots_dev;
  a.src_map = src_map_dev;
  a.hit_k = static_cast<const char*>(hit_k_dev);
  a.hit_v = static_cast<const char*>(hit_v_dev);
  a.hit_tok_stride = hit_token_stride;
  a.hit_rows = uint32_t(hit_rows);
  a.old_pos = old_pos_dev;
  a.new_pos = new_pos_dev;
  a.cos_sin = static_cast<const char*>(cos_sin_dev);
  a.cs_row_stride = cos_sin_row_stride_elems;
  a.cs_rows = uint32_t(cos_sin_rows > 0 ? cos_sin_rows : 0);
  a.num_tokens = uint32_t(num_tokens);
  a.row_bytes = uint32_t(row_bytes);
  a.head_dim = uint32_t(head_dim);
  a.heads = uint32_t(heads);
  a.relocate = relocate ? 1 : 0;
  a.neox = neox ? 1 : 0;
  a.bad = bad_dev;
  a.hit_chunks = hit_chunks_dev;
  a.chunk_div = FastDiv::make(uint32_t(chunk_tokens > 0 ? chunk_tokens : 1));
  a.chunk_tok_stride = chunk_token_stride;
  int64_t align[12] = {row_bytes, out_token_stride, int64_t(reinterpret_cast<uintptr_t>(out_k_dev)),
                       int64_t(reinterpret_cast<uintptr_t>(out_v_dev)), 0, 0, 0, 0, 0, 0, 0, 0};
  int nalign = 4;
  if (hit_rows > 0 && hit_chunks_dev == nullptr) {
    align[nalign++] = hit_token_stride;
    align[nalign++] = int64_t(reinterpret_cast<uintptr_t>(hit_k_dev));
    align[nalign++] = int64_t(reinterpret_cast<uintptr_t>(hit_v_dev));
  }
  if (kv != nullptr) {
    CBK_REQUIRE(kv->k_base && kv->v_base && kv->num_blocks > 0 && kv->block_size > 0 &&
                    kv->num_blocks * kv->block_size < (int64_t(1) << 32),
                "invalid kv descriptor");
    CBK_REQUIRE(kv->row_bytes == row_bytes, "kv row_bytes %lld != heads*head_dim*elem %lld",
                (long long)kv->row_bytes, (long long)row_bytes);
    CBK_REQUIRE(slots_dev != nullptr, "slots are NULL while a page source is given");
    a.page_k = static_cast<const char*>(kv->k_base);
    a.page_v = static_cast<const char*>(kv->v_base);
    a.block_stride = kv->block_stride;
    a.token_stride = kv->token_stride;
    a.num_slots = uint32_t(kv->num_blocks * kv->block_size);
    a.bs_div = FastDiv::make(uint32_t(kv->block_size));
    align[nalign++] = kv->block_stride;
    align[nalign++] = kv->token_stride;
    align[nalign++] = int64_t(reinterpret_cast<uintptr_t>(kv->k_base));
    align[nalign++] = int64_t(reinterpret_cast<uintptr_t>(kv->v_base));
  } else {
    a.num_slots = 0;  // any -2 row is zeroed and counted as bad
    a.bs_div = FastDiv::make(1);
  }
  const int vec = common_vec_bytes(align, nalign);
  CBK_REQUIRE(vec >= es, "buffers are not aligned to the element size");
  {
    // the row-batched kernel: 16-byte vectors, rows up to 4 KiB, and for
    // relocation whole heads per 1 KiB pass with 16-byte aligned cos/sin rows
    const int64_t head_bytes = head_dim * es, lane_elems = 16 / es;
    const bool rope_ok = !relocate ||
        (1024 % head_bytes == 0 && head_dim % lane_elems == 0 &&
         (!neox || (head_dim / 2) % lane_elems == 0) &&
         (cos_sin_row_stride_elems * es) % 16 == 0 && reinterpret_cast<uintptr_t>(cos_sin_dev) % 16 == 0);
    const int64_t passes = (row_bytes + 1023) / 1024;
    a.rows_path = (vec == 16 && row_bytes <= 4096 && rope_ok) ? int32_t(passes == 3 ? 4 : passes) : 0;
  }
  const uint32_t cap = uint32_t(max_workgroups > 0 ? max_workgroups : 0);
  switch (dtype) {
    case CBK_DTYPE_F32: return launch_assemble_t<float>(a, vec, cap, static_cast<hipStream_t>(stream));
    case CBK_DTYPE_BF16: return launch_assemble_t<__hip_bfloat16>(a, vec, cap, static_cast<hipStream_t>(stream));
    default: return launch_assemble_t<__half>(a, vec, cap, static_cast<hipStream_t>(stream));
  }
}
}  // namespace
}  // namespace cbk

extern "C" int cbk_blend_assemble(
    const cbk_kv_desc* kv, const int64_t* slots_dev, const int32_t* src_map_dev, int64_t num_tokens,
    const void* hit_k_dev, const void* hit_v_dev, int64_t hit_token_stride, int64_t hit_rows,
    const int32_t* old_pos_dev, const int32_t* new_pos_dev, const void* cos_sin_dev,
    int64_t cos_sin_row_stride_elems, int64_t cos_sin_rows, int64_t heads, int64_t head_dim,
    int32_t relocate, int32_t neox, int32_t dtype, void* out_k_dev, void* out_v_dev,
    int64_t out_token_stride, int32_t* bad_dev, cbk_stream_t stream) {
  return cbk::assemble_impl(kv, slots_dev, src_map_dev, num_tokens, hit_k_dev, hit_v_dev,
                            hit_token_stride, hit_rows, nullptr, 0, 0, old_pos_dev, new_pos_dev,
                            cos_sin_dev, cos_sin_row_stride_elems, cos_sin_rows, heads, head_dim,
                            relocate, neox, dtype, out_k_dev, out_v_dev, out_token_stride, bad_dev, 0,
                            stream);
}

extern "C" int cbk_blend_assemble_chunks(
    const cbk_kv_desc* kv, const int64_t* slots_dev, const int32_t* src_map_dev, int64_t num_tokens,
    const uint64_t* hit_chunks_dev, int64_t chunk_tokens, int64_t chunk_token_stride, int64_t hit_rows,
    const int32_t* old_pos_dev, const void* cos_sin_dev, int64_t cos_sin_row_stride_elems,
    int64_t cos_sin_rows, int64_t heads, int64_t head_dim, int32_t relocate, int32_t neox,
    int32_t dtype, void* out_k_dev, void* out_v_dev, int64_t out_token_stride, int32_t* bad_dev,
    int32_t max_workgroups, cbk_stream_t stream) {
  if (hit_rows > 0 && hit_chunks_dev == nullptr)
    return cbk::set_error(CBK_ERR_INVALID, "hit chunk table is NULL");
  return cbk::assemble_impl(kv, slots_dev, src_map_dev, num_tokens, nullptr, nullptr, 0, hit_rows,
                            hit_chunks_dev, chunk_tokens, chunk_token_stride, old_pos_dev, nullptr,
                            cos_sin_dev, cos_sin_row_stride_elems, cos_sin_rows, heads, head_dim,
                            relocate, neox, dtype, out_k_dev, out_v_dev, out_token_stride, bad_dev,
                            max_workgroups, stream);
}
