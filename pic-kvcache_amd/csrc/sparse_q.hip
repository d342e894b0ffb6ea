// Sparse-Q attention-mass scores for gfx950 (the only MFMA kernel here).
//
// full[k] = sum_{h, q : pos_q >= k} softmax_k( r(Q[q,h] . K[k, h/G]) * scale )
// where r rounds the dot product to the input dtype (the reference's bf16
// matmul output, cacheblend_vllm/ascend.py:694) and the softmax runs over all
// keys of the context with keys k > pos_q masked (ascend.py:696-698).
//
// Two passes over Q.K^T on MFMA (v_mfma_f32_16x16x32_{bf16,f16}):
//   rowstats  one workgroup per (16-query tile, kv head): the G query heads
//             of the group x 16 queries against 64-key blocks staged in LDS,
//             online max / sum per row in the log2 domain, merged across
//             the 16 lanes that share a row -> (m, 1/l) per (head, query)
//   colsum    one workgroup per (256-key block, kv head): each wave keeps its
//             64 keys' K fragments in registers and streams the query tiles
//             (all G heads staged in LDS), accumulating exp2(x - m) / l per
//             key column in registers -> partial[kv head][key]; every key is
//             owned by exactly one wave, so the sum order is fixed and the
//             result is identical run to run (no float atomics)
//   gather    out[i] = sum over kv heads (fixed order) of partial[.][idx[i]]
// MFMA operand layout (checked on gfx950): A[i][k] in lane i + 16*(k/8),
// element k%8; B[k][j] in lane j + 16*(k/8); D[i][j] in lane j + 16*(i/4),
// register i%4. Q.K^T has both operands row-major in D, so A and B fragments
// are the same 16-byte loads of 8 consecutive dims.
//
// A float32 path (no MFMA, exact float32 dots) serves float32 inputs.
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include "cbk_common.hpp"

namespace cbk {
namespace {

typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kQTile = 16;
constexpr int kKeyBlock1 = 64;        // keys per LDS block in rowstats
constexpr int kColTiles = 4;          // 16-key column tiles per wave in colsum
constexpr int kKeyBlock2 = 4 * 16 * kColTiles;  // 256 keys per colsum workgroup
constexpr int kMaxHeadsInLds = 8;     // query heads staged per colsum LDS load
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

struct SqArgs {
  const char* q;          // [*, Hq, D] rows
  int64_t q_stride;       // elements between query rows
  const int64_t* q_index; // [nq] rows of q that are sparse queries (nullable: 0..nq-1)
  const int64_t* pos;     // [*] absolute position of every q row (indexed like q)
  const char* k;          // [nk, Hkv, D]
  int64_t k_stride;       // elements between key rows
  uint32_t nq, nk, hq, hkv, d, groups;
  float c2;               // scale * log2(e)
  int32_t round_mode;     // 0 none, 1 bf16, 2 f16
  float2* stats;          // [hq][nq_pad] (m2, 1/l)
  int32_t* tile_pos;      // [ntiles][2] (min, max) position per query tile
  float* partial;         // [hkv][nk]
  uint32_t nq_pad;
};

__device__ __forceinline__ float round_logit(float x, int mode) {
  if (mode == 1) return __bfloat162float(__float2bfloat16(x));
  if (mode == 2) return __half2float(__float2half(x));
  return x;
}

__device__ __forceinline__ int32_t query_pos(const SqArgs& a, uint32_t qi) {
  if (qi >= a.nq) return -1;
  const int64_t row = a.q_index ? a.q_index[qi] : int64_t(qi);
  return int32_t(a.pos[row]);
}

__device__ __forceinline__ const char* query_row(const SqArgs& a, uint32_t qi, uint32_t h, uint32_t es) {
  const int64_t row = a.q_index ? a.q_index[qi] : int64_t(qi);
  return a.q + (row * a.q_stride + int64_t(h) * a.d) * es;
}

// Online (max, sum) update in the log2 domain with -inf guards.
__device__ __forceinline__ void stats_merge(float& m, float& l, float m_o, float l_o) {
  const float mn = fmaxf(m, m_o);
  const float ms = mn == kNegInf ? 0.f : mn;
  l = l * __builtin_amdgcn_exp2f(m - ms) + l_o * __builtin_amdgcn_exp2f(m_o - ms);
  m = mn;
}

template <typename V>
__device__ __forceinline__ f32x4 mfma16(const V& a, const V& b, const f32x4& c);
template <>
__device__ __forceinline__ f32x4 mfma16<s16x8>(const s16x8& a, const s16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16<h16x8>(const h16x8& a, const h16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------ rowstats

template <typename V, int KSTEPS>
__global__ __launch_bounds__(kThreads) void sq_rowstats_kernel(const SqArgs a) {
  constexpr int D = 32 * KSTEPS;
  constexpr int LROW = D + 8;  // padded LDS row (elements) against bank conflicts
  constexpr int MAXT = 4;      // row tiles (heads) per wave: G <= 16
  __shared__ __attribute__((aligned(16))) uint16_t kblk[kKeyBlock1 * LROW];
  __shared__ int32_t s_pos[kQTile];
  __shared__ int32_t s_minmax[2];
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t qt = blockIdx.x, g = blockIdx.y;
  const uint32_t q0 = qt * kQTile;
  if (threadIdx.x < kQTile) s_pos[threadIdx.x] = query_pos(a, q0 + threadIdx.x);
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t lo = 0x7fffffff, hi = -1;
    for (int i = 0; i < kQTile; ++i) {
      if (q0 + i < a.nq) {
        lo = min(lo, s_pos[i]);
        hi = max(hi, s_pos[i]);
      }
    }
    s_minmax[0] = lo;
    s_minmax[1] = hi;
    if (g == 0) {
      a.tile_pos[2 * qt] = lo;
      a.tile_pos[2 * qt + 1] = hi;
    }
  }
  __syncthreads();
  const int32_t minpos = s_minmax[0], maxpos = min(s_minmax[1], int32_t(a.nk) - 1);
  const uint32_t col = lane & 15, rgrp = lane >> 4;
  int32_t rpos[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) rpos[i] = s_pos[4 * rgrp + i];
  const uint32_t qi = q0 + col;  // A row of this lane
  const uint32_t es = sizeof(uint16_t);

  V afrag[MAXT][KSTEPS];
  float m[MAXT][4], l[MAXT][4];
  const uint32_t ntiles_w = (a.groups > wave) ? (a.groups - wave + 3) / 4 : 0;
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) { m[t][i] = kNegInf; l[t][i] = 0.f; }
    if (t < int(ntiles_w)) {
      const uint32_t h = g * a.groups + wave + 4 * t;
      const char* row = qi < a.nq ? query_row(a, qi, h, es) : nullptr;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        if (row) {
          afrag[t][s] = *reinterpret_cast<const V*>(row + (32 * s + 8 * rgrp) * es);
        } else {
          afrag[t][s] = V(0);
        }
      }
    }
  }
  const int32_t nkb = maxpos < 0 ? 0 : maxpos / kKeyBlock1 + 1;
  for (int32_t kb = 0; kb < nkb; ++kb) {
    const int32_t k0 = kb * kKeyBlock1;
    __syncthreads();
    // stage 64 keys x D of kv head g: 16-byte pieces
    for (uint32_t p = threadIdx.x; p < kKeyBlock1 * (D / 8); p += kThreads) {
      const uint32_t kr = p / (D / 8), piece = p % (D / 8);
      const int32_t key = k0 + int32_t(kr);
      u32x4 v = u32x4(0);
      if (key < int32_t(a.nk))
        v = *reinterpret_cast<const u32x4*>(a.k + ((int64_t(key) * a.k_stride) + int64_t(g) * a.d + piece * 8) * es);
      *reinterpret_cast<u32x4*>(&kblk[kr * LROW + piece * 8]) = v;
    }
    __syncthreads();
    const bool need_mask = (k0 + kKeyBlock1 - 1 > minpos) || (k0 + kKeyBlock1 > int32_t(a.nk));
#pragma unroll
    for (int t = 0; t < MAXT; ++t) {
      if (t >= int(ntiles_w)) break;
      float x[kColTiles][4];
#pragma unroll
      for (int c = 0; c < kColTiles; ++c) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
          const V b = *reinterpret_cast<const V*>(&kblk[(c * 16 + col) * LROW + 32 * s + 8 * rgrp]);
          acc = mfma16<V>(afrag[t][s], b, acc);
        }
        const int32_t key = k0 + c * 16 + int32_t(col);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = round_logit(acc[i], a.round_mode) * a.c2;
          if (need_mask && (key > rpos[i] || key >= int32_t(a.nk))) v = kNegInf;
          x[c][i] = v;
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float bm = fmaxf(fmaxf(x[0][i], x[1][i]), fmaxf(x[2][i], x[3][i]));
        const float mn = fmaxf(m[t][i], bm);
        const float ms = mn == kNegInf ? 0.f : mn;
        float sum = 0.f;
#pragma unroll
        for (int c = 0; c < kColTiles; ++c) sum += __builtin_amdgcn_exp2f(x[c][i] - ms);
        l[t][i] = l[t][i] * __builtin_amdgcn_exp2f(m[t][i] - ms) + sum;
        m[t][i] = mn;
      }
    }
  }
  // merge the 16 lanes that hold the same rows, then publish (m2, 1/l)
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    if (t >= int(ntiles_w)) break;
    const uint32_t h = g * a.groups + wave + 4 * t;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float mm = m[t][i], ll = l[t][i];
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) {
        const float mo = __shfl_xor(mm, off, 64);
        const float lo = __shfl_xor(ll, off, 64);
        stats_merge(mm, ll, mo, lo);
      }
      const uint32_t q = q0 + 4 * rgrp + i;
      if (col == 0 && q < a.nq) a.stats[int64_t(h) * a.nq_pad + q] = make_float2(mm, ll > 0.f ? 1.f / ll : 0.f);
    }
  }
}

// -------------------------------------------------------------- colsum

template <typename V, int KSTEPS>
__global__ __launch_bounds__(kThreads) void sq_colsum_kernel(const SqArgs a) {
  constexpr int D = 32 * KSTEPS;
  constexpr int LROW = D + 8;
  __shared__ __attribute__((aligned(16))) uint16_t qblk[kMaxHeadsInLds * kQTile * LROW];
  __shared__ float2 s_stats[kMaxHeadsInLds][kQTile];
  __shared__ int32_t s_pos[kQTile];
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t g = blockIdx.y;
  const int32_t kw0 = int32_t(blockIdx.x) * kKeyBlock2 + int32_t(wave) * 16 * kColTiles;
  const int32_t kb0 = int32_t(blockIdx.x) * kKeyBlock2;
  const uint32_t col = lane & 15, rgrp = lane >> 4;
  const uint32_t es = sizeof(uint16_t);

  V bfrag[kColTiles][KSTEPS];
#pragma unroll
  for (int c = 0; c < kColTiles; ++c) {
    const int32_t key = kw0 + c * 16 + int32_t(col);
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      if (key < int32_t(a.nk)) {
        bfrag[c][s] = *reinterpret_cast<const V*>(
            a.k + ((int64_t(key) * a.k_stride) + int64_t(g) * a.d + 32 * s + 8 * rgrp) * es);
      } else {
        bfrag[c][s] = V(0);
      }
    }
  }
  float acc_col[kColTiles];
#pragma unroll
  for (int c = 0; c < kColTiles; ++c) acc_col[c] = 0.f;

  const uint32_t ntiles = (a.nq + kQTile - 1) / kQTile;
  for (uint32_t qt = 0; qt < ntiles; ++qt) {
    const int32_t tmax = a.tile_pos[2 * qt + 1];
    if (tmax < kb0) continue;  // no query of the tile sees any key of the block
    const int32_t tmin = a.tile_pos[2 * qt];
    const uint32_t q0 = qt * kQTile;
    for (uint32_t h0 = 0; h0 < a.groups; h0 += kMaxHeadsInLds) {
      const uint32_t nh = min(uint32_t(kMaxHeadsInLds), a.groups - h0);
      __syncthreads();
      for (uint32_t p = threadIdx.x; p < nh * kQTile * (D / 8); p += kThreads) {
        const uint32_t hl = p / (kQTile * (D / 8));
        const uint32_t rem = p % (kQTile * (D / 8));
        const uint32_t r = rem / (D / 8), piece = rem % (D / 8);
        u32x4 v = u32x4(0);
        if (q0 + r < a.nq)
          v = *reinterpret_cast<const u32x4*>(query_row(a, q0 + r, g * a.groups + h0 + hl, es) + piece * 8 * es);
        *reinterpret_cast<u32x4*>(&qblk[(hl * kQTile + r) * LROW + piece * 8]) = v;
      }
      for (uint32_t p = threadIdx.x; p < nh * kQTile; p += kThreads) {
        const uint32_t hl = p / kQTile, r = p % kQTile;
        s_stats[hl][r] = (q0 + r < a.nq) ? a.stats[int64_t(g * a.groups + h0 + hl) * a.nq_pad + q0 + r]
                                         : make_float2(0.f, 0.f);
      }
      if (threadIdx.x < kQTile) s_pos[threadIdx.x] = query_pos(a, q0 + threadIdx.x);
      __syncthreads();
      if (tmax < kw0) continue;  // this wave's keys are all after the tile's queries
      int32_t rpos[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) rpos[i] = s_pos[4 * rgrp + i];
      const bool need_mask = (kw0 + 16 * kColTiles - 1 > tmin) || (q0 + kQTile > a.nq);
      for (uint32_t hl = 0; hl < nh; ++hl) {
        V afrag[KSTEPS];
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s)
          afrag[s] = *reinterpret_cast<const V*>(&qblk[(hl * kQTile + col) * LROW + 32 * s + 8 * rgrp]);
        float2 st[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) st[i] = s_stats[hl][4 * rgrp + i];
#pragma unroll
        for (int c = 0; c < kColTiles; ++c) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < KSTEPS; ++s) acc = mfma16<V>(afrag[s], bfrag[c][s], acc);
          const int32_t key = kw0 + c * 16 + int32_t(col);
          float sum = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float x = round_logit(acc[i], a.round_mode) * a.c2;
            float p = __builtin_amdgcn_exp2f(x - st[i].x) * st[i].y;
            if (need_mask && key > rpos[i]) p = 0.f;
            sum += p;
          }
          acc_col[c] += sum;
        }
      }
    }
  }
  // column totals: the 4 lane groups hold the same column
#pragma unroll
  for (int c = 0; c < kColTiles; ++c) {
    float v = acc_col[c];
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    const int32_t key = kw0 + c * 16 + int32_t(col);
    if (rgrp == 0 && key < int32_t(a.nk)) a.partial[int64_t(g) * a.nk + key] = v;
  }
}

// ----------------------------------------------------------- float32 path

// rowstats: one wavefront per (query, head); lanes stride over keys.
__global__ __launch_bounds__(kThreads) void sq_rowstats_f32_kernel(const SqArgs a) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t item = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (item >= a.nq * a.hq) return;
  const uint32_t qi = item / a.hq, h = item % a.hq, g = h / a.groups;
  const int32_t pos = min(query_pos(a, qi), int32_t(a.nk) - 1);
  const float* qrow = reinterpret_cast<const float*>(query_row(a, qi, h, 4));
  float m = kNegInf, l = 0.f;
  for (int32_t key = int32_t(lane); key <= pos; key += 64) {
    const float* krow = reinterpret_cast<const float*>(a.k) + int64_t(key) * a.k_stride + int64_t(g) * a.d;
    float dot = 0.f;
    for (uint32_t e = 0; e < a.d; ++e) dot = fmaf(qrow[e], krow[e], dot);
    const float x = round_logit(dot, a.round_mode) * a.c2;
    stats_merge(m, l, x, 1.f);
  }
  for (int off = 1; off < 64; off <<= 1) {
    const float mo = __shfl_xor(m, off, 64), lo = __shfl_xor(l, off, 64);
    stats_merge(m, l, mo, lo);
  }
  if (lane == 0) a.stats[int64_t(h) * a.nq_pad + qi] = make_float2(m, l > 0.f ? 1.f / l : 0.f);
}

// colsum: one thread per (key, kv head), fixed query/head order.
__global__ __launch_bounds__(kThreads) void sq_colsum_f32_kernel(const SqArgs a) {
  const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
  if (t >= a.nk * a.hkv) return;
  const uint32_t key = t % a.nk, g = t / a.nk;
  const float* krow = reinterpret_cast<const float*>(a.k) + int64_t(key) * a.k_stride + int64_t(g) * a.d;
  float acc = 0.f;
  for (uint32_t qi = 0; qi < a.nq; ++qi) {
    if (query_pos(a, qi) < int32_t(key)) continue;
    for (uint32_t hl = 0; hl < a.groups; ++hl) {
      const uint32_t h = g * a.groups + hl;
      const float* qrow = reinterpret_cast<const float*>(query_row(a, qi, h, 4));
      float dot = 0.f;
      for (uint32_t e = 0; e < a.d; ++e) dot = fmaf(qrow[e], krow[e], dot);
      const float2 st = a.stats[int64_t(h) * a.nq_pad + qi];
      acc += __builtin_amdgcn_exp2f(round_logit(dot, a.round_mode) * a.c2 - st.x) * st.y;
    }
  }
  a.partial[int64_t(g) * a.nk + key] = acc;
}

// ---------------------------------------------------------------- gather

__global__ __launch_bounds__(kThreads) void sq_gather_kernel(const float* partial, uint32_t nk, uint32_t hkv,
                                                             const int64_t* index, uint32_t n,
                                                             float* out, float* full) {
  const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
  if (full != nullptr && i < nk) {
    float v = 0.f;
    for (uint32_t g = 0; g < hkv; ++g) v += partial[int64_t(g) * nk + i];
    full[i] = v;
  }
  if (out != nullptr && i < n) {
    const int64_t k = index ? index[i] : int64_t(i);
    float v = __uint_as_float(0x7fc00000u);
    if (k >= 0 && k < int64_t(nk)) {
      v = 0.f;
      for (uint32_t g = 0; g < hkv; ++g) v += partial[int64_t(g) * nk + k];
    }
    out[i] = v;
  }
}

__global__ void sq_zero_kernel(float* p, uint64_t n) {
  for (uint64_t i = blockIdx.x * uint64_t(kThreads) + threadIdx.x; i < n; i += uint64_t(gridDim.x) * kThreads)
    p[i] = 0.f;
}

struct SqLayout {
  uint32_t nq_pad, ntiles;
  uint64_t stats, tile_pos, partial, bytes;  // byte offsets
};

__host__ SqLayout sq_layout(int64_t nq, int64_t nk, int64_t hq, int64_t hkv) {
  SqLayout L;
  L.ntiles = uint32_t((nq + kQTile - 1) / kQTile);
  L.nq_pad = L.ntiles * kQTile;
  L.stats = 0;
  L.tile_pos = (L.stats + uint64_t(hq) * L.nq_pad * 8 + 255) & ~uint64_t(255);
  L.partial = (L.tile_pos + uint64_t(L.ntiles) * 8 + 255) & ~uint64_t(255);
  L.bytes = (L.partial + uint64_t(hkv) * nk * 4 + 255) & ~uint64_t(255);
  return L;
}

template <typename V>
int launch_mfma(const SqArgs& a, int ksteps, hipStream_t stream) {
  const dim3 g1((a.nq + kQTile - 1) / kQTile, a.hkv);
  const dim3 g2((a.nk + kKeyBlock2 - 1) / kKeyBlock2, a.hkv);
#define CBK_SQ(KS)                                                                        \
  hipLaunchKernelGGL((sq_rowstats_kernel<V, KS>), g1, dim3(kThreads), 0, stream, a);     \
  hipLaunchKernelGGL((sq_colsum_kernel<V, KS>), g2, dim3(kThreads), 0, stream, a)
  switch (ksteps) {
    case 2: CBK_SQ(2); break;
    case 4: CBK_SQ(4); break;
    default: return set_error(CBK_ERR_UNSUPPORTED, "head_dim %u", a.d);
  }
#undef CBK_SQ
  return launch_status("sparse_q mfma");
}

}  // namespace
}  // namespace cbk

extern "C" {

size_t cbk_sparse_q_workspace_bytes(int64_t nq, int64_t nk, int64_t hq, int64_t hkv) {
  if (nq < 0 || nk < 0 || hq <= 0 || hkv <= 0) return 0;
  return size_t(cbk::sq_layout(nq, nk, hq, hkv).bytes);
}

int cbk_sparse_q_scores(const void* q_dev, int64_t q_row_stride_elems, const int64_t* q_index_dev,
                        int64_t nq, const int64_t* positions_dev, const void* k_dev,
                        int64_t k_row_stride_elems, int64_t nk, int64_t hq, int64_t hkv,
                        int64_t head_dim, float scale, int32_t dtype, int32_t round_logits,
                        const int64_t* out_index_dev, int64_t n_out, float* out_scores_dev,
                        float* full_scores_dev, void* workspace_dev, size_t workspace_bytes,
                        cbk_stream_t stream) {
  using namespace cbk;
  clear_error();
  hipStream_t s = static_cast<hipStream_t>(stream);
  CBK_REQUIRE(nq >= 0 && nk >= 0 && n_out >= 0 && nq < (int64_t(1) << 30) && nk < (int64_t(1) << 30),
              "sizes out of range");
  CBK_REQUIRE(hq > 0 && hkv > 0 && hq % hkv == 0,
              "Sparse-Q requires query heads to be divisible by KV heads; got %lld and %lld",
              (long long)hq, (long long)hkv);
  CBK_REQUIRE(hq / hkv <= 16, "at most 16 query heads per KV head");
  CBK_REQUIRE(head_dim > 0 && q_row_stride_elems >= hq * head_dim && k_row_stride_elems >= hkv * head_dim,
              "row strides smaller than heads * head_dim");
  CBK_REQUIRE(round_logits >= 0 && round_logits <= 2, "round_logits must be 0, 1 or 2");
  if (nk == 0 || (out_scores_dev == nullptr && full_scores_dev == nullptr)) return CBK_OK;
  const SqLayout L = sq_layout(nq, nk, hq, hkv);
  if (workspace_bytes < L.bytes)
    return set_error(CBK_ERR_WORKSPACE, "sparse_q workspace %zu < %llu bytes", workspace_bytes,
                     (unsigned long long)L.bytes);
  CBK_REQUIRE(workspace_dev && (reinterpret_cast<uintptr_t>(workspace_dev) & 255) == 0,
              "workspace must be 256-byte aligned");
  CBK_REQUIRE(k_dev && (nq == 0 || (q_dev && positions_dev)), "NULL pointer");
  char* ws = static_cast<char*>(workspace_dev);
  SqArgs a{};
  a.q = static_cast<const char*>(q_dev);
  a.q_stride = q_row_stride_elems;
  a.q_index = q_index_dev;
  a.pos = positions_dev;
  a.k = static_cast<const char*>(k_dev);
  a.k_stride = k_row_stride_elems;
  a.nq = uint32_t(nq);
  a.nk = uint32_t(nk);
  a.hq = uint32_t(hq);
  a.hkv = uint32_t(hkv);
  a.d = uint32_t(head_dim);
  a.groups = uint32_t(hq / hkv);
  a.c2 = scale * kLog2e;
  a.round_mode = round_logits;
  a.stats = reinterpret_cast<float2*>(ws + L.stats);
  a.tile_pos = reinterpret_cast<int32_t*>(ws + L.tile_pos);
  a.partial = reinterpret_cast<float*>(ws + L.partial);
  a.nq_pad = L.nq_pad;
  if (nq == 0) {
    const uint64_t n = uint64_t(hkv) * nk;
    hipLaunchKernelGGL(sq_zero_kernel, dim3(uint32_t(std::min<uint64_t>((n + kThreads - 1) / kThreads, 4096))),
                       dim3(kThreads), 0, s, a.partial, n);
  } else if (dtype == CBK_DTYPE_F32) {
    const uint64_t items = uint64_t(nq) * hq;
    hipLaunchKernelGGL(sq_rowstats_f32_kernel, dim3(uint32_t((items + 3) / 4)), dim3(kThreads), 0, s, a);
    hipLaunchKernelGGL(sq_colsum_f32_kernel, dim3(uint32_t((uint64_t(nk) * hkv + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, s, a);
  } else {
    CBK_REQUIRE(dtype == CBK_DTYPE_BF16 || dtype == CBK_DTYPE_F16, "dtype %d", int(dtype));
    CBK_REQUIRE(head_dim % 32 == 0 && (head_dim == 64 || head_dim == 128),
                "MFMA path supports head_dim 64 or 128, got %lld", (long long)head_dim);
    CBK_REQUIRE(q_row_stride_elems % 8 == 0 && k_row_stride_elems % 8 == 0 &&
                    (reinterpret_cast<uintptr_t>(q_dev) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(k_dev) & 15) == 0,
                "q/k rows must be 16-byte aligned");
    const int ks = int(head_dim / 32);
    int rc = dtype == CBK_DTYPE_BF16 ? launch_mfma<s16x8>(a, ks, s) : launch_mfma<h16x8>(a, ks, s);
    if (rc) return rc;
  }
  if (int rc = launch_status("sparse_q")) return rc;
  const uint32_t n = uint32_t(std::max<int64_t>(full_scores_dev ? nk : 0, out_scores_dev ? n_out : 0));
  if (n > 0)
    hipLaunchKernelGGL(sq_gather_kernel, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, s,
                       a.partial, a.nk, a.hkv, out_index_dev, uint32_t(out_scores_dev ? n_out : 0),
                       out_scores_dev, full_scores_dev);
  return launch_status("sparse_q gather");
}

}  // extern "C"
