// Sparse-Q attention-mass scores for gfx950 (the only MFMA kernel here).
//
// full[k] = sum_{h, q : pos_q >= k} softmax_k( r(Q[q,h] . K[k, h/G]) * scale )
// where r rounds the dot product to the input dtype (the reference's bf16
// matmul output, cacheblend_vllm/ascend.py:694) and the softmax runs over all
// keys of the context with keys k > pos_q masked (ascend.py:696-698).
//
// Two passes over Q.K^T on MFMA (v_mfma_f32_16x16x32_{bf16,f16}; the row
// pass of 16-head groups on v_mfma_f32_32x32x16_{bf16,f16}):
//   rowstats  one workgroup per (1, 2 or 4 adjacent 16-query tiles, key
//             range, kv head): the G query heads of the group x 16 queries
//             of each tile against the range's
//             64-key blocks staged in LDS, sums of exp against the range's
//             first-block maximum (online max / sum where that does not
//             apply) in the log2 domain, merged across the 16 lanes that
//             share a row -> (m, l) per (range, head, query)
//   merge     the ranges' (m, l) of each row, in range order -> m + log2(l)
//   colsum    one workgroup per (256-key block, query-unit range, kv head):
//             each wave keeps its 64 keys' K fragments in registers and
//             streams the range's query tiles (all G heads staged in LDS),
//             accumulating exp2(x - m - log2 l) per key column in registers
//             -> partial[range][kv head][key]; every (key, range) is owned by
//             exactly one wave, so the sum order is fixed and the result is
//             identical run to run (no float atomics)
//   gather    out[i] = sum over ranges and kv heads (fixed order) of
//             partial[.][.][idx[i]]
// MFMA operand layout (checked on gfx950): A[i][k] in lane i + 16*(k/8),
// element k%8; B[k][j] in lane j + 16*(k/8); D[i][j] in lane j + 16*(i/4),
// register i%4; 32x32x16: A[i][k] in lane i + 32*(k/8), B[k][j] in lane
// j + 32*(k/8), element k%8; D[i][j] in lane j + 32*((i/4)%2), register
// 4*(i/8) + i%4. Q.K^T has both operands row-major in D, so A and B
// fragments are the same 16-byte loads of 8 consecutive dims.
//
// A float32 path (no MFMA, exact float32 dots) serves float32 inputs.
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "cbk_common.hpp"

namespace cbk {
namespace {

typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kQTile = 16;
constexpr int kTileWords = 32;        // per query tile: 16 positions, min, max, unused
constexpr int kKeyBlock1 = 64;        // keys per LDS block in rowstats
constexpr int kColTiles = 4;          // 16-key column tiles per wave in colsum
constexpr int kKeyBlock2 = 4 * 16 * kColTiles;  // 256 keys per colsum workgroup
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
  float2* stats;          // [hq][nq_pad] (m2 + log2(l), unused)
  float2* chunk_stats;    // [row_chunks][hq][nq_pad] (m2, l) of each key range, row_chunks > 1
  uint32_t row_chunks;    // key ranges per (query tile, kv head) in rowstats
  int32_t* tiles;         // [nq_pad / 16][32]: the 16 query positions (-1 past nq), min, max, unused
  float* partial;         // [hkv][nk]
  uint16_t* qdense;       // [hkv][nq_pad / 16][groups][16][D]: query rows in colsum's unit order
  uint32_t nq_pad;
  uint32_t col_splits;    // query-unit ranges per (key block, kv head) in colsum
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

// Published per (head, query) row: x = m + log2(l), so that a probability
// is the single exp2(logit * scale * log2(e) - x) (+inf: an empty row).
__device__ __forceinline__ float2 row_stats(float m, float l) {
  return make_float2(l > 0.f ? m + log2f(l) : __builtin_inff(), 0.f);
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

template <typename V>
__device__ __forceinline__ f32x16 mfma32(const V& a, const V& b, const f32x16& c);
template <>
__device__ __forceinline__ f32x16 mfma32<s16x8>(const s16x8& a, const s16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32<h16x8>(const h16x8& a, const h16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Rounds two logits to the input dtype, as a bf16/f16 matmul output would
// be (bf16: one instruction per logit).
template <int RMODE>
__device__ __forceinline__ void round_pair(float& x, float& y) {
  if constexpr (RMODE == 1) {
    x = bf16_round(x);
    y = bf16_round(y);
  } else if constexpr (RMODE == 2) {
    x = __half2float(__float2half(x));
    y = __half2float(__float2half(y));
  }
}

// ------------------------------------------------------------ rowstats

// One 64-key block against MAXT row tiles: MFMA, round, (mask), then the
// row statistics: online (max, sum) updates, or -- FIXED -- sums against the
// row's reference m, the maximum of its first key block (a logit of the row,
// hence at most its maximum: no term exceeds 2^(max - m); a row whose sum
// does not stay finite is recomputed online).
template <typename V, int KSTEPS, int MAXT, int RMODE, bool MASK, bool FIXED = false>
__device__ __forceinline__ void rowstats_block(const SqArgs& a, const uint16_t* blk, int32_t k0,
                                               const V (&afrag)[MAXT][KSTEPS], int ntiles_w,
                                               const int32_t (&rpos)[4], float (&m)[MAXT][4],
                                               float (&l)[MAXT][4], uint32_t col, uint32_t rgrp) {
  constexpr int D = 32 * KSTEPS;
  V bfrag[kColTiles][KSTEPS];
#pragma unroll
  for (int c = 0; c < kColTiles; ++c) {
    const uint32_t row = c * 16 + col;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
      bfrag[c][s] = *reinterpret_cast<const V*>(&blk[row * D + ((4 * s + rgrp) ^ lds_swizzle<D>(row)) * 8]);
  }
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    if (t >= ntiles_w) break;
    f32x4 acc[kColTiles];
#pragma unroll
    for (int c = 0; c < kColTiles; ++c) {
      acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) acc[c] = mfma16<V>(afrag[t][s], bfrag[c][s], acc[c]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float raw[kColTiles], r[kColTiles];
#pragma unroll
      for (int c = 0; c < kColTiles; ++c) {
        raw[c] = acc[c][i];
        if constexpr (MASK) {
          const int32_t key = k0 + c * 16 + int32_t(col);
          if (key > rpos[i] || key >= int32_t(a.nk)) raw[c] = kNegInf;
        }
      }
#pragma unroll
      for (int c = 0; c < kColTiles; c += 2) {
        r[c] = raw[c];
        r[c + 1] = raw[c + 1];
        round_pair<RMODE>(r[c], r[c + 1]);  // -inf stays -inf
      }
      if constexpr (FIXED) {
        float sum = __builtin_amdgcn_exp2f(fmaf(r[0], a.c2, -m[t][i]));
#pragma unroll
        for (int c = 1; c < kColTiles; ++c) sum += __builtin_amdgcn_exp2f(fmaf(r[c], a.c2, -m[t][i]));
        l[t][i] += sum;
        continue;
      }
      // online max / sum in the log2 domain; the max is taken on the
      // unrounded dots (canonical floats, no extra max(x, x); rounding is
      // monotonic, so exponents exceed 0 by at most a rounding step), and
      // scale > 0 preserves order
      const float bm2 = fmaxf(fmaxf(raw[0], raw[1]), fmaxf(raw[2], raw[3])) * a.c2;
      const float mn = fmaxf(m[t][i], bm2);
      // an unmasked block's dots are finite, so is its maximum
      const float ms = (MASK && mn == kNegInf) ? 0.f : mn;
      float sum = __builtin_amdgcn_exp2f(fmaf(r[0], a.c2, -ms));
#pragma unroll
      for (int c = 1; c < kColTiles; ++c) sum += __builtin_amdgcn_exp2f(fmaf(r[c], a.c2, -ms));
      l[t][i] = fmaf(l[t][i], __builtin_amdgcn_exp2f(m[t][i] - ms), sum);
      m[t][i] = mn;
    }
  }
}

// The same block on 32x32x16 MFMAs with the product transposed: S^T = K.Q^T,
// A = 32 keys of the block, B = a pair tile's 32 query rows (16 queries of
// two heads of the wave). Each lane then holds one row (its query column,
// lane % 32) and 16 keys of each 32-key half of the block: keys
// 8 * (r / 4) + 4 * (lane / 32) + r % 4 in register r. A row's statistics
// are one (max, sum) per lane, merged with the other half-wave at the end,
// so four head slots fit the register budget of three waves per SIMD.
// Pair tiles whose first slot is past the group (nslots) are skipped.
template <typename V, int D, int NT, int RMODE, bool MASK, bool FIXED>
__device__ __forceinline__ void rowstats_block_wide(const SqArgs& a, const uint16_t* blk, int32_t k0,
                                                    const V (&qfrag)[NT][D / 16], int nslots, int32_t rpos,
                                                    float (&m)[NT][1], float (&l)[NT][1], uint32_t lane) {
  constexpr int S = D / 16;
  const uint32_t kr = lane & 31, hi = lane >> 5;
  f32x16 acc[NT][2];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    const uint32_t row = kt * 32 + kr;
    V kfrag[S];
#pragma unroll
    for (int s = 0; s < S; ++s)
      kfrag[s] = *reinterpret_cast<const V*>(&blk[row * D + ((2 * s + hi) ^ lds_swizzle<D>(row)) * 8]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (2 * t >= nslots) break;
      acc[t][kt] = f32x16{};
#pragma unroll
      for (int s = 0; s < S; ++s) acc[t][kt] = mfma32<V>(kfrag[s], qfrag[t][s], acc[t][kt]);
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (2 * t >= nslots) break;
    float x[32];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        x[kt * 16 + r] = acc[t][kt][r];
        if constexpr (MASK) {
          const int32_t key = k0 + kt * 32 + 8 * (r / 4) + 4 * int32_t(hi) + (r % 4);
          if (key > rpos || key >= int32_t(a.nk)) x[kt * 16 + r] = kNegInf;
        }
      }
    float ms;
    if constexpr (FIXED) {
      ms = m[t][0];
    } else {
      // online max on the unrounded dots, as in the 16x16 block
      float bm = fmaxf(x[0], x[1]);
#pragma unroll
      for (int i = 2; i < 32; ++i) bm = fmaxf(bm, x[i]);
      const float mn = fmaxf(m[t][0], bm * a.c2);
      ms = (MASK && mn == kNegInf) ? 0.f : mn;
      l[t][0] *= __builtin_amdgcn_exp2f(m[t][0] - ms);
      m[t][0] = mn;
    }
#pragma unroll
    for (int i = 0; i < 32; i += 2) round_pair<RMODE>(x[i], x[i + 1]);  // -inf stays -inf
    float s0 = 0.f, s1 = 0.f;  // two chains of adds
#pragma unroll
    for (int i = 0; i < 32; i += 2) {
      s0 += __builtin_amdgcn_exp2f(fmaf(x[i], a.c2, -ms));
      s1 += __builtin_amdgcn_exp2f(fmaf(x[i + 1], a.c2, -ms));
    }
    l[t][0] += s0 + s1;
  }
}

// K blocks of 64 keys stream through three LDS buffers by DMA, as the query
// units do in colsum (see there for the wait and barrier scheme).
// FULL: the group is exactly (4 / TPW) * MAXT heads, so every wave has MAXT
// row tiles (a compile-time count: no branch between the tiles of a block).
// TPW: query tiles per workgroup (adjacent tiles of sorted queries: nearby
// positions), 4 / TPW waves per tile. With 2, two waves serve each of two
// tiles with twice the head slots, so each K fragment read from LDS serves
// 64 rows at 8 heads per KV head; with 4, each wave takes a whole tile's
// group (up to 4 heads), so a K block staged in LDS serves four tiles and
// no wave idles when the group is smaller than 4.
// Two waves per SIMD for paired tiles (238 registers at head_dim 128), for
// four head slots per wave at head_dim 128 (236 registers; three waves per
// SIMD spilled 224 bytes per lane), and for four tiles per workgroup at
// head_dim 128 or with 3-4 head slots (three waves per SIMD spill 87 bytes
// per lane at 3 slots; at head_dim 64 with 1-2 slots three waves measured
// 3% faster at one head per KV head); three waves per SIMD otherwise (two
// head slots at head_dim 128 spill 96 bytes per lane there, yet two waves
// per SIMD measured slower: 2.21-2.23 vs 1.99-2.00 ms at 5 heads per KV
// head, 1.35 vs 1.30 ms at 6, on 32K-key layers, with one tile per
// workgroup).
constexpr int rs_waves(int tpw, int maxt, int ksteps) {
  if (tpw == 2) return 2;
  if (tpw == 4) return (ksteps == 4 || maxt >= 3) ? 2 : 3;
  return (ksteps == 4 && maxt == 4) ? 2 : 3;
}
template <typename V, int KSTEPS, int MAXT, int RMODE, bool FULL, int TPW = 1>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(rs_waves(TPW, MAXT, KSTEPS), rs_waves(TPW, MAXT, KSTEPS))))
void sq_rowstats_kernel(const SqArgs a) {
  constexpr int D = 32 * KSTEPS;
  constexpr uint32_t P = D / 8;                   // 16-byte pieces per key row
  constexpr uint32_t kInsts = P / 4;              // requests per wave per block (1 KiB each)
  constexpr uint32_t kRowsPerInst = 64 / P;
  constexpr int kBuffers = 3;
  __shared__ __attribute__((aligned(16))) uint16_t kbuf[kBuffers][kKeyBlock1 * D];
  constexpr int WT = 4 / TPW;  // waves per query tile
  __shared__ int32_t s_pos[kQTile * TPW];
  __shared__ int32_t s_minmax[2];  // over the workgroup's tiles
  // the wave index in a scalar register: what derives from it stays scalar
  const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t ntiles = (a.nq + kQTile - 1) / kQTile;
  const uint32_t ngroups = (ntiles + TPW - 1) / TPW;  // workgroups' tile groups
  // tiles the column pass reads (its units of 2 or 4 tiles at 1-2 heads per
  // KV head end on a multiple of 4 tiles): their records and dense query
  // rows are written too, empty past the queries
  const uint32_t ntiles_pad = a.nq_pad / kQTile;
  // workgroup -> (tile, key range, kv head), the kv head fastest and the
  // latest tiles (most keys) first, so that workgroups are dispatched in
  // decreasing order of work across all heads
  // (a division by a runtime value runs on the VALU: readfirstlane brings
  // the results back to scalar registers)
  const uint32_t g = __builtin_amdgcn_readfirstlane(blockIdx.x % a.hkv);
  const uint32_t chunk = __builtin_amdgcn_readfirstlane((blockIdx.x / a.hkv) % a.row_chunks);
  const uint32_t qt_first = TPW * __builtin_amdgcn_readfirstlane(ngroups - 1 - blockIdx.x / (a.hkv * a.row_chunks));
  const uint32_t wt = wave / WT, wv = wave % WT;  // this wave's tile in the workgroup, its place there
  const uint32_t qt = qt_first + wt;               // this wave's tile (past ntiles: an odd last group)
  const bool tile_ok = qt < ntiles;
  const uint32_t q0 = qt * kQTile;
  if (threadIdx.x < kQTile * TPW) s_pos[threadIdx.x] = query_pos(a, qt_first * kQTile + threadIdx.x);
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t lo = 0x7fffffff, hi = -1;
    for (int u = 0; u < TPW; ++u) {
      int32_t tlo = 0x7fffffff, thi = -1;
      for (int i = 0; i < kQTile; ++i) {
        if ((qt_first + u) * kQTile + i < a.nq) {
          tlo = min(tlo, s_pos[u * kQTile + i]);
          thi = max(thi, s_pos[u * kQTile + i]);
        }
      }
      lo = min(lo, tlo);
      hi = max(hi, thi);
      if (g == 0 && chunk == 0 && qt_first + u < ntiles_pad) {
        a.tiles[kTileWords * (qt_first + u) + kQTile] = tlo;
        a.tiles[kTileWords * (qt_first + u) + kQTile + 1] = thi;
      }
    }
    s_minmax[0] = lo;
    s_minmax[1] = hi;
  }
  __syncthreads();
  // workgroup-uniform, and scalar: the key-block loop and its branches stay
  // uniform (an LDS value is per-lane to the compiler, which then keeps the
  // loop counter and every loop-carried value in vector registers)
  const int32_t minpos = __builtin_amdgcn_readfirstlane(s_minmax[0]);
  const int32_t maxpos = __builtin_amdgcn_readfirstlane(min(s_minmax[1], int32_t(a.nk) - 1));
  // Row tiles of a wave: its head slots are heads wave + 4 * slot of the
  // group. 16x16x32 (MAXT <= 2): one tile per slot, 4 rows per lane.
  // 32x32x16 (MAXT = 4): pair tiles of slots 2t and 2t + 1, one row per lane
  // (157 against 168 registers and half the spills of the 16x16 form there:
  // 16 heads per KV head 7% faster; at 8 heads the 16x16 form measured 1-3%
  // faster, the 32x32 form's busier co-execution lowering the clock that
  // the power limit allows). At head_dim 128, MAXT = 4 runs two waves per
  // SIMD: 236 registers and no spills, 3.26-3.28 -> 2.96-3.06 ms on a
  // 64-head, 32K-key layer against three waves with 224 bytes of spills.
  constexpr bool WIDE = MAXT == 4 && TPW == 1;
  constexpr int NT = WIDE ? MAXT / 2 : MAXT;    // row tiles
  constexpr int NR = WIDE ? 1 : 4;              // rows per lane and tile
  constexpr int NS = WIDE ? D / 16 : KSTEPS;    // MFMA steps over the head dim
  constexpr uint32_t kStepDims = WIDE ? 16 : 32;
  const uint32_t col = lane & 15, rgrp = lane >> 4;
  const uint32_t d0 = WIDE ? 8 * (lane >> 5) : 8 * rgrp;  // this lane's dims within a step
  int32_t rpos[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) rpos[i] = s_pos[wt * kQTile + (WIDE ? col : 4 * rgrp + i)];
  const uint32_t qi = q0 + col;

  V afrag[NT][NS];
  float m[NT][NR], l[NT][NR];
  const int nslots = FULL ? MAXT : (a.groups > wv) ? int((a.groups - wv + WT - 1) / WT) : 0;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int slot = WIDE ? 2 * t + int(rgrp & 1) : t;
    const char* row = (slot < nslots && qi < a.nq)
                          ? query_row(a, qi, g * a.groups + wv + WT * slot, 2) : nullptr;
#pragma unroll
    for (int s = 0; s < NS; ++s)
      afrag[t][s] = row ? *reinterpret_cast<const V*>(row + (kStepDims * s + d0) * 2) : V(0);
    // the dense copy colsum streams (zeros past nq)
    if (slot < nslots && chunk == 0 && qt < ntiles_pad) {
      uint16_t* dst = a.qdense + ((int64_t(g) * ntiles_pad + qt) * a.groups + wv + WT * slot) * (kQTile * D) + col * D;
#pragma unroll
      for (int s = 0; s < NS; ++s) *reinterpret_cast<V*>(dst + kStepDims * s + d0) = afrag[t][s];
    }
  }
  if (g == 0 && chunk == 0 && threadIdx.x < kQTile * TPW && qt_first + threadIdx.x / kQTile < ntiles_pad)
    a.tiles[kTileWords * (qt_first + threadIdx.x / kQTile) + threadIdx.x % kQTile] = s_pos[threadIdx.x];
  // the workgroup of the last tiles also writes the records past them, up
  // to 4 past the padded count, empty (positions -1, min above any, max -1):
  // the column pass's units of rows read their tiles' records whole
  if (blockIdx.x == 0) {
    const uint32_t t_end = ntiles_pad + 4;
    for (uint32_t w = ngroups * TPW * kTileWords + threadIdx.x; w < t_end * kTileWords; w += kThreads) {
      const uint32_t k = w % kTileWords;
      a.tiles[w] = k < kQTile ? -1 : k == kQTile ? 0x7fffffff : k == kQTile + 1 ? -1 : 0;
    }
  }
  // nothing of the compiler's own in flight once the requests start
  CBK_WAIT_VM_LGKM0(0);

  // this workgroup's key blocks: [kb_lo, kb_hi), an equal share of the tile's
  const int32_t nkb_tile = maxpos < 0 ? 0 : maxpos / kKeyBlock1 + 1;
  const int32_t kb_lo = __builtin_amdgcn_readfirstlane(int32_t(uint32_t(nkb_tile) * chunk / a.row_chunks));
  const int32_t kb_hi = __builtin_amdgcn_readfirstlane(int32_t(uint32_t(nkb_tile) * (chunk + 1) / a.row_chunks));
  // per-lane byte offsets of a block's requests (key row, swizzled piece)
  uint32_t koff[kInsts];
  uint32_t krow[kInsts];
#pragma unroll
  for (uint32_t j = 0; j < kInsts; ++j) {
    krow[j] = (wave * kInsts + j) * kRowsPerInst + lane / P;
    const uint32_t piece = (lane % P) ^ lds_swizzle<D>(krow[j]);
    koff[j] = (krow[j] * a.k_stride + g * a.d + piece * 8) * 2;
  }
  // block kb (clamped: a request past the range repeats its last block) into
  // buffer b; rows past nk of the last block read its last key (masked)
  auto request = [&](int32_t kb, int b) {
    kb = min(kb, kb_hi - 1);
    const int32_t k0 = kb * kKeyBlock1;
    const char* base = a.k + int64_t(k0) * a.k_stride * 2;
    const uint32_t lk = lds_address(kbuf[b]);
    if (k0 + kKeyBlock1 <= int32_t(a.nk)) {
#pragma unroll
      for (uint32_t j = 0; j < kInsts; ++j) lds_dma16(base, koff[j], lk + (wave * kInsts + j) * 1024);
    } else {
      const uint32_t last = uint32_t(int32_t(a.nk) - 1 - k0);
#pragma unroll
      for (uint32_t j = 0; j < kInsts; ++j) {
        const uint32_t r = min(krow[j], last);
        lds_dma16(base, koff[j] - (krow[j] - r) * a.k_stride * 2, lk + (wave * kInsts + j) * 1024);
      }
    }
  };
  // Row statistics against a fixed reference (the range's first block's
  // maximum) when that block is visible to every row of the tile, so every
  // lane's reference is a finite logit of its row; online (max, sum) updates
  // otherwise, and again from the start when a fixed-reference sum did not
  // stay finite (a logit over 127 above its row's reference, in log2 units).
  __shared__ uint32_t s_redo;
  // blocks [kb_lo, kb_m) are visible to every row of the tile and lie below
  // nk; the blocks from kb_m on are masked
  const int32_t kb_vis = int32_t(min((int64_t(minpos) + 1) / kKeyBlock1, int64_t(a.nk) / kKeyBlock1));
  const int32_t kb_m = min(max(kb_vis, kb_lo), kb_hi);
  bool fixed = kb_lo < kb_m;
  // one block: wait for it, request the block two ahead into the buffer
  // computed one block ago, then the block's statistics (each variant in a
  // loop of its own: no register copies between variants in the hot loop)
  auto step = [&](auto mask, auto fix, int32_t kb) {
    const int it = kb - kb_lo;
    CBK_WAIT_VM_LGKM0(kInsts);  // block kb has landed; the newest block may be pending
    asm volatile("s_barrier" ::: "memory");
    request(kb + 2, (it + 2) % kBuffers);
    if constexpr (WIDE)
      rowstats_block_wide<V, D, NT, RMODE, decltype(mask)::value, decltype(fix)::value>(
          a, kbuf[it % kBuffers], kb * kKeyBlock1, afrag, nslots, rpos[0], m, l, lane);
    else
      rowstats_block<V, KSTEPS, MAXT, RMODE, decltype(mask)::value, decltype(fix)::value>(
          a, kbuf[it % kBuffers], kb * kKeyBlock1, afrag, nslots, rpos, m, l, col, rgrp);
  };
  using yes = std::true_type;
  using no = std::false_type;
  for (;;) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < NR; ++i) { m[t][i] = kNegInf; l[t][i] = 0.f; }
    if (kb_hi > kb_lo) {
      request(kb_lo, 0);
      request(kb_lo + 1, 1);
      int32_t kb = kb_lo;
      if (fixed) {
        step(no(), no(), kb++);  // the reference block, online
        for (; kb < kb_m; ++kb) step(no(), yes(), kb);
        for (; kb < kb_hi; ++kb) step(yes(), yes(), kb);
      } else {
        for (; kb < kb_m; ++kb) step(no(), no(), kb);
        for (; kb < kb_hi; ++kb) step(yes(), no(), kb);
      }
      CBK_WAIT_VM_LGKM0(0);  // no LDS write in flight when the workgroup ends (or restarts)
    }
    if (!fixed) break;
    bool bad = false;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < NR; ++i) bad |= !(l[t][i] < 3.0e38f);
    if (threadIdx.x == 0) s_redo = 0;
    __syncthreads();
    if (bad) s_redo = 1;
    __syncthreads();
    if (!__builtin_amdgcn_readfirstlane(s_redo)) break;  // uniform: the loops stay scalar
    fixed = false;
  }
  // merge the lanes that hold the same rows (16 lanes, or the two half-waves
  // of the wide tiles), then publish m2 + log2(l), or this key range's
  // (m2, l) for sq_merge_kernel
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      float mm = m[t][i], ll = l[t][i];
#pragma unroll
      for (int off = WIDE ? 32 : 1; off < (WIDE ? 64 : 16); off <<= 1) {
        const float mo = __shfl_xor(mm, off, 64);
        const float lo = __shfl_xor(ll, off, 64);
        stats_merge(mm, ll, mo, lo);
      }
      const int slot = WIDE ? 2 * t + int(rgrp & 1) : t;
      const uint32_t h = g * a.groups + wv + WT * slot;
      const uint32_t q = q0 + (WIDE ? col : 4 * rgrp + i);  // rows past nq too: colsum reads whole tiles
      if ((WIDE ? lane < 32 : col == 0) && slot < nslots && tile_ok) {
        if (a.row_chunks == 1)
          a.stats[int64_t(h) * a.nq_pad + q] = row_stats(mm, ll);
        else
          a.chunk_stats[(int64_t(chunk) * a.hq + h) * a.nq_pad + q] = make_float2(mm, ll);
      }
    }
  }
}

// Merges the key ranges' (m2, l) of every (head, query) row in range order
// (the same result run to run) and publishes m2 + log2(l).
__global__ __launch_bounds__(kThreads) void sq_merge_kernel(const SqArgs a) {
  const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
  const uint32_t rows = a.hq * a.nq_pad;
  if (i >= rows) return;
  float m = kNegInf, l = 0.f;
  for (uint32_t c = 0; c < a.row_chunks; ++c) {
    const float2 p = a.chunk_stats[int64_t(c) * rows + i];
    stats_merge(m, l, p.x, p.y);
  }
  a.stats[i] = row_stats(m, l);
}

// -------------------------------------------------------------- colsum
//
// Query units (16-query tile x up to 4 heads of the KV head's group) stream
// through three LDS buffers filled by global_load_lds_dwordx4 from the dense
// copy rowstats wrote: one unit is computed while the next has landed and the
// one after is in flight, with no registers held for it. The DMA requests are
// inline asm, so the compiler adds no waits of its own for these LDS writes
// (it would wait for every request in flight before each read, not knowing
// which buffer a request fills); the kernel waits for them with explicit
// vmcnt counts, and the barrier is a plain s_barrier (a __syncthreads fence
// would wait for the request just issued). Vector memory ops complete in
// order, so the counts the compiler computes for its own loads stay safe.

constexpr int kHeadChunk = 4;  // query heads per unit
constexpr int kQBuffers = 3;   // units in LDS: computed, landed, requested

template <typename V, int KSTEPS>
__device__ __forceinline__ void colsum_mfma(const uint16_t* qlds, uint32_t hl, const V (&bfrag)[kColTiles][KSTEPS],
                                            f32x4 (&acc)[kColTiles], uint32_t col, uint32_t rgrp) {
  constexpr int D = 32 * KSTEPS;
  const uint32_t row = hl * kQTile + col;
  V afrag[KSTEPS];
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s)
    afrag[s] = *reinterpret_cast<const V*>(&qlds[row * D + ((4 * s + rgrp) ^ lds_swizzle<D>(row)) * 8]);
#pragma unroll
  for (int c = 0; c < kColTiles; ++c) {
    acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) acc[c] = mfma16<V>(afrag[s], bfrag[c][s], acc[c]);
  }
}

// Software-pipelined over the unit's 4 head slots: the MFMAs of head hl + 1
// are issued before the VALU work of head hl, which they do not depend on.
// FULL (every slot holds rows: chunks of 4 heads when the group is a
// multiple of 4, or four consecutive (tile, head) rows, T > 1; the kernel
// is launched with nothing else): no branch inside the unit, which the
// compiler then schedules as one block (without it, slots hl >= nh would be
// skipped). With T > 1 slot hl holds
// head (h0 + hl) mod G of the unit's tile (h0 + hl) / G (its first tile's
// heads from h0 on, then the next tile's; rows past the last query tile
// belong to empty tiles, whose positions are -1); MASK reads a slot's
// positions from its tile's record in LDS (trec), which keeps them out of
// the unmasked units' registers.
template <typename V, int KSTEPS, int RMODE, bool MASK, bool FULL, int T>
__device__ __forceinline__ void colsum_unit(const SqArgs& a, const uint16_t* qlds, const float2* st,
                                            uint32_t nh, int32_t kw0, const int32_t* trec, uint32_t grp,
                                            uint32_t h0,
                                            const V (&bfrag)[kColTiles][KSTEPS], float (&acc_col)[kColTiles],
                                            uint32_t col, uint32_t rgrp) {
  f32x4 acc[2][kColTiles];
  colsum_mfma<V, KSTEPS>(qlds, 0, bfrag, acc[0], col, rgrp);
#pragma unroll
  for (uint32_t hl = 0; hl < kHeadChunk; ++hl) {
    if (hl + 1 < kHeadChunk) colsum_mfma<V, KSTEPS>(qlds, hl + 1, bfrag, acc[(hl + 1) & 1], col, rgrp);
    if (FULL || hl < nh) {
      float mrow[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) mrow[i] = st[hl * kQTile + 4 * rgrp + i].x;
      int32_t rpos[4] = {0, 0, 0, 0};
      if constexpr (MASK) {
        uint32_t tix = 0;  // the slot's tile within the unit (uniform)
#pragma unroll
        for (int k = 1; k < T; ++k) tix += (h0 + hl >= uint32_t(k) * grp) ? 1u : 0u;
        const int4 rp = *reinterpret_cast<const int4*>(trec + kTileWords * tix + 4 * rgrp);
        rpos[0] = rp.x; rpos[1] = rp.y; rpos[2] = rp.z; rpos[3] = rp.w;
      }
#pragma unroll
      for (int c = 0; c < kColTiles; ++c) {
        const f32x4 v = acc[hl & 1][c];
        float r[4] = {v[0], v[1], v[2], v[3]};
        round_pair<RMODE>(r[0], r[1]);
        round_pair<RMODE>(r[2], r[3]);
        const int32_t key = kw0 + c * 16 + int32_t(col);
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[i] = __builtin_amdgcn_exp2f(fmaf(r[i], a.c2, -mrow[i]));
          if constexpr (MASK) p[i] = key > rpos[i] ? 0.f : p[i];
        }
        // a pair tree, not a chain of four adds into the column sum: 1-1.4%
        // off the C5 column pass (its sums on the matrix core, by an
        // identity-A 4x4x4 MFMA that adds a lane's four bf16 values to its
        // own accumulators, measured 3.7% slower: the matrix core's work grew
        // by 6% while the VALU's shrank by 10%)
        acc_col[c] += (p[0] + p[1]) + (p[2] + p[3]);
      }
    }
  }
}

// Three waves per SIMD: the LDS holds three workgroups' buffers. Units: T ==
// 1, a tile's chunk of up to 4 of its G heads (G a multiple of 4: every
// chunk whole); T > 1, four consecutive (tile, head) rows of the KV head's
// queries (row f is head f mod G of tile f / G), which span at most T tiles
// (T = 4 at one head per KV head, else 2), so that no head slot computes
// on rows that are never used when G is not a multiple of 4. G0: G known at
// compile time (1 or 2: the four rows are whole tiles, so every slot's tile
// and head are constants; 24-43 fewer spilled registers, 3-8% faster than
// the run-time mapping there), 0 for any G.
template <typename V, int KSTEPS, int RMODE, bool FULL, int T = 1, int G0 = 0>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3, 3))) void sq_colsum_kernel(
    const SqArgs a) {
  // every group size is launched with whole units: a multiple of 4 heads in
  // chunks of 4, any other in units of four rows
  static_assert(FULL && (T == 1 || T == 2 || T == 4), "units are whole");
  static_assert(G0 == 0 || G0 * T == kHeadChunk, "a compile-time group fills the unit's tiles");
  constexpr bool FLAT = T > 1;
  const uint32_t G = G0 ? uint32_t(G0) : a.groups;  // heads per KV head
  constexpr int D = 32 * KSTEPS;
  constexpr uint32_t P = D / 8;                   // 16-byte pieces per row
  constexpr uint32_t kInsts = P / 4;              // Q requests per wave per unit (1 KiB each)
  constexpr uint32_t kRowsPerInst = 64 / P;
  constexpr int kQElems = kHeadChunk * kQTile * D;
  __shared__ __attribute__((aligned(16))) uint16_t qbuf[kQBuffers][kQElems];
  __shared__ __attribute__((aligned(16))) float2 sbuf[kQBuffers][128];  // 64 used, lanes 32-63 repeat
  // tile records (T == 1: repeated; T == 4: two requests)
  __shared__ __attribute__((aligned(16))) int32_t tbuf[kQBuffers][T == 4 ? 128 : 64];
  const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // workgroup -> (key block, kv head), the kv head fastest: the earliest key
  // blocks (seen by the most queries) of every head are dispatched first
  // (a division by a runtime value runs on the VALU: readfirstlane brings
  // the results back to scalar registers)
  const uint32_t g = __builtin_amdgcn_readfirstlane(blockIdx.x % a.hkv);
  const uint32_t rest = __builtin_amdgcn_readfirstlane(blockIdx.x / a.hkv);
  const uint32_t split = __builtin_amdgcn_readfirstlane(rest % a.col_splits);
  const int32_t kb0 = __builtin_amdgcn_readfirstlane(int32_t(rest / a.col_splits) * kKeyBlock2);
  const int32_t kw0 = kb0 + int32_t(wave) * 16 * kColTiles;
  const uint32_t col = lane & 15, rgrp = lane >> 4;

  V bfrag[kColTiles][KSTEPS];
#pragma unroll
  for (int c = 0; c < kColTiles; ++c) {
    const int32_t key = kw0 + c * 16 + int32_t(col);
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
      bfrag[c][s] = key < int32_t(a.nk)
                        ? *reinterpret_cast<const V*>(a.k + ((int64_t(key) * a.k_stride) + int64_t(g) * a.d +
                                                             32 * s + 8 * rgrp) * 2)
                        : V(0);
  }
  float acc_col[kColTiles];
#pragma unroll
  for (int c = 0; c < kColTiles; ++c) acc_col[c] = 0.f;
  // the K fragments have landed before any request is issued (the compiler,
  // blind to the requests, would otherwise wait for everything in flight
  // wherever it first needs them)
  CBK_WAIT_VM_LGKM0(0);

  // Units: tiles from the last down to the lowest tile whose latest query
  // sees a key of this block (tiles in between that see none skip their
  // compute), each tile's head chunks in order. Latest tiles first: every key
  // block sees them, so the workgroups resident together stream the same
  // units at about the same time and find them in L2.
  const int32_t ntiles = int32_t((a.nq + kQTile - 1) / kQTile);
  const int32_t ntiles_pad = int32_t(a.nq_pad / kQTile);
  const uint32_t nflat = uint32_t(ntiles) * G;  // (tile, head) rows of the KV head
  // unit positions: tiles (each of nchunks units), or units of four rows
  const int32_t nunit_tiles = FLAT ? int32_t((nflat + 3) / 4) : ntiles;
  const uint32_t nchunks = FLAT ? 1u : (a.groups + kHeadChunk - 1) / kHeadChunk;
  int32_t tlo = ntiles;
  for (int32_t t0 = 0; t0 < ntiles; t0 += 64) {
    const int32_t u = t0 + int32_t(lane);
    const uint64_t hits = __ballot(u < ntiles && a.tiles[kTileWords * u + kQTile + 1] >= kb0);
    if (hits) {
      tlo = t0 + int32_t(__builtin_ctzll(hits));
      break;
    }
  }
  // this workgroup's share of the block's units: range `split` of
  // col_splits equal ranges, in unit order
  // the lowest unit holding a row of tile tlo
  const int32_t ulo = FLAT ? int32_t(uint32_t(tlo) * G / 4) : tlo;
  const uint32_t all_units = tlo < ntiles ? uint32_t(nunit_tiles - ulo) * nchunks : 0u;
  const uint32_t u_lo = all_units * split / a.col_splits;
  const int32_t nunits = int32_t(all_units * (split + 1) / a.col_splits - u_lo);

  // Per-lane byte offsets of the requests. A unit's Q rows are contiguous in
  // the dense copy; rows of heads past the group (a partial last chunk) read
  // the next rows, never used (the copy is padded by a unit at its end).
  uint32_t qoff[kInsts];
#pragma unroll
  for (uint32_t j = 0; j < kInsts; ++j) {
    const uint32_t row = (wave * kInsts + j) * kRowsPerInst + lane / P;
    qoff[j] = (row * D + ((lane % P) ^ lds_swizzle<D>(row)) * 8) * 2;
  }
  const uint32_t toff = (T == 1 ? lane % kTileWords : lane) * 4;
  // wave 0's statistics request: 8 lanes (128 bytes) per head slot of the
  // unit; for chunk units (T == 1) the lanes' offsets are the same each unit
  const uint32_t slot0 = (lane / 8) % kHeadChunk;
  const uint32_t soff_full = (slot0 * a.nq_pad + (lane % 8) * 2) * 8;
  // Issues unit qt (a tile's head chunk hc, or the four rows from 4 qt; a
  // request past the last unit repeats it, so every iteration issues the
  // same number of requests) into buffer B: the Q rows, and on wave 0 the
  // row statistics and the tile records. A unit's Q rows are contiguous in
  // the dense copy.
  auto request = [&](int32_t qt, uint32_t hc, auto bc) __attribute__((always_inline)) {
    constexpr int B = decltype(bc)::value;
    const uint32_t f0 = FLAT ? 4u * uint32_t(qt) : 0u;
    const int32_t t0 = FLAT ? int32_t(f0 / G) : qt;  // the unit's first tile
    const uint16_t* unit =
        FLAT ? a.qdense + (int64_t(g) * ntiles_pad * G + f0) * (kQTile * D)
             : a.qdense + ((int64_t(g) * ntiles_pad + t0) * a.groups + hc * kHeadChunk) * (kQTile * D);
    const uint32_t lq = lds_address(qbuf[B]);
#pragma unroll
    for (uint32_t j = 0; j < kInsts; ++j) lds_dma16(unit, qoff[j], lq + (wave * kInsts + j) * 1024);
    if (wave == 0) {
      const float2* st = a.stats + int64_t(g * G + hc * kHeadChunk) * a.nq_pad + t0 * kQTile;
      uint32_t soff = soff_full;
      if constexpr (FLAT) {
        // slot s: row f0 + s, head (h0 + s) mod G of tile t0 + (h0 + s) / G
        const uint32_t hs = f0 - uint32_t(t0) * G + slot0;
        uint32_t ts = 0;
#pragma unroll
        for (int k = 1; k < T; ++k) ts += hs >= uint32_t(k) * G ? 1u : 0u;
        soff = ((hs - ts * G) * a.nq_pad + ts * kQTile + (lane % 8) * 2) * 8;
      }
      lds_dma16(st, soff, lds_address(sbuf[B]));
      lds_dma4(a.tiles + kTileWords * t0, toff, lds_address(tbuf[B]));
      if constexpr (T == 4) lds_dma4(a.tiles + kTileWords * (t0 + 2), toff, lds_address(tbuf[B]) + 256);
    }
  };
  // units in order: the head chunks of tile ntiles - 1, then of the tile
  // below, down to tile tlo (stepped without divisions); with T > 1 the
  // units of four rows from the last down to the one holding tlo's first
  auto next = [&](int32_t& qt, uint32_t& hc) __attribute__((always_inline)) {
    if (++hc == nchunks) {
      hc = 0;
      --qt;
    }
  };
  if (nunits > 0) {
    // unit it, and the unit requested in iteration it: unit u of the block
    // is head chunk u % nchunks of tile nunit_tiles - 1 - u / nchunks (T > 1:
    // the rows of unit position nunit_tiles - 1 - u)
    int32_t qt_c = nunit_tiles - 1 - int32_t(u_lo / nchunks), qt_r = qt_c;
    uint32_t hc_c = u_lo % nchunks, hc_r = hc_c;
    const uint32_t u_last = u_lo + uint32_t(nunits) - 1;  // the range's last unit
    const int32_t qt_last = nunit_tiles - 1 - int32_t(u_last / nchunks);
    const uint32_t hc_last = u_last % nchunks;
    auto request_next = [&](int32_t i, auto bc) __attribute__((always_inline)) {
      if (i < nunits) {
        request(qt_r, hc_r, bc);
        next(qt_r, hc_r);
      } else {
        request(qt_last, hc_last, bc);
      }
    };
    request_next(0, std::integral_constant<int, 0>());
    request_next(1, std::integral_constant<int, 1>());
    // unit it in buffer B = it % 3, known at compile time in a loop of three
    // iterations: every LDS address is a lane's offset plus a constant
    auto iteration = [&](int32_t it, auto bc) __attribute__((always_inline)) {
      constexpr int B = decltype(bc)::value;
      // unit it has landed once at most the newest unit's requests are pending
      // (wave 0 also requests the statistics and one or two tile-record pieces)
      if (wave == 0)
        CBK_WAIT_VM_LGKM0(kInsts + (T == 4 ? 3 : 2));
      else
        CBK_WAIT_VM_LGKM0(kInsts);
      asm volatile("s_barrier" ::: "memory");
      request_next(it + 2, std::integral_constant<int, (B + 2) % kQBuffers>());  // the buffer computed one unit ago
      const int32_t qt = qt_c;
      const uint32_t hc = hc_c;
      next(qt_c, hc_c);
      // the unit's tiles t0 .. t0 + T - 1 (T > 1: all that its rows can
      // span; a tile it does not reach only widens the test below, and
      // those past the last query tile have empty records, which the row
      // pass writes) and their earliest and latest positions (uniform: scalar)
      const uint32_t f0 = FLAT ? 4u * uint32_t(qt) : 0u;
      const int32_t t0 = FLAT ? int32_t(f0 / G) : qt;
      const uint32_t h0 = f0 - uint32_t(t0) * G;  // the first row's head
      int32_t tmin = __builtin_amdgcn_readfirstlane(tbuf[B][kQTile]);
      int32_t tmax = __builtin_amdgcn_readfirstlane(tbuf[B][kQTile + 1]);
#pragma unroll
      for (int t = 1; t < T; ++t) {
        tmin = min(tmin, __builtin_amdgcn_readfirstlane(tbuf[B][kTileWords * t + kQTile]));
        tmax = max(tmax, __builtin_amdgcn_readfirstlane(tbuf[B][kTileWords * t + kQTile + 1]));
      }
      if (tmax >= kw0) {
        const uint32_t nh = min(uint32_t(kHeadChunk), a.groups - hc * kHeadChunk);
        // masked: some key of the wave past some query, or rows past nq in
        // the unit's tiles
        if (kw0 + 16 * kColTiles - 1 > tmin || uint32_t(t0 + T) * kQTile > a.nq)
          colsum_unit<V, KSTEPS, RMODE, true, FULL, T>(a, qbuf[B], sbuf[B], nh, kw0, tbuf[B], G, h0, bfrag,
                                                       acc_col, col, rgrp);
        else
          colsum_unit<V, KSTEPS, RMODE, false, FULL, T>(a, qbuf[B], sbuf[B], nh, kw0, tbuf[B], G, h0, bfrag,
                                                        acc_col, col, rgrp);
      }
    };
    int32_t it = 0;
    for (; it + 3 <= nunits; it += 3) {
      iteration(it, std::integral_constant<int, 0>());
      iteration(it + 1, std::integral_constant<int, 1>());
      iteration(it + 2, std::integral_constant<int, 2>());
    }
    if (it < nunits) iteration(it++, std::integral_constant<int, 0>());
    if (it < nunits) iteration(it++, std::integral_constant<int, 1>());
    CBK_WAIT_VM_LGKM0(0);  // no LDS write in flight when the workgroup ends
  }
  // column totals: the 4 lane groups hold the same column
#pragma unroll
  for (int c = 0; c < kColTiles; ++c) {
    float v = acc_col[c];
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    const int32_t key = kw0 + c * 16 + int32_t(col);
    if (rgrp == 0 && key < int32_t(a.nk)) a.partial[(int64_t(split) * a.hkv + g) * a.nk + key] = v;
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
  if (lane == 0) a.stats[int64_t(h) * a.nq_pad + qi] = row_stats(m, l);
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
      acc += __builtin_amdgcn_exp2f(round_logit(dot, a.round_mode) * a.c2 - st.x);
    }
  }
  a.partial[int64_t(g) * a.nk + key] = acc;
}

// ---------------------------------------------------------------- gather

// out / full = the sum over query-unit ranges and kv heads of the partial
// column sums [splits][hkv][nk], in that order.
__global__ __launch_bounds__(kThreads) void sq_gather_kernel(const float* partial, uint32_t nk, uint32_t hkv,
                                                             uint32_t splits, const int64_t* index, uint32_t n,
                                                             float* out, float* full) {
  const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
  const uint32_t parts = splits * hkv;
  if (full != nullptr && i < nk) {
    float v = 0.f;
    for (uint32_t p = 0; p < parts; ++p) v += partial[int64_t(p) * nk + i];
    full[i] = v;
  }
  if (out != nullptr && i < n) {
    const int64_t k = index ? index[i] : int64_t(i);
    float v = __uint_as_float(0x7fc00000u);
    if (k >= 0 && k < int64_t(nk)) {
      v = 0.f;
      for (uint32_t p = 0; p < parts; ++p) v += partial[int64_t(p) * nk + k];
    }
    out[i] = v;
  }
}

__global__ void sq_zero_kernel(float* p, uint64_t n) {
  for (uint64_t i = blockIdx.x * uint64_t(kThreads) + threadIdx.x; i < n; i += uint64_t(gridDim.x) * kThreads)
    p[i] = 0.f;
}

// Largest head_dim of the MFMA path: the dense query copy is sized for it.
constexpr int64_t kMaxHeadDim = 128;

// Key ranges a (query tile, kv head) of rowstats may be split into.
constexpr uint32_t kMaxRowChunks = 8;
// Query-unit ranges a (key block, kv head) of colsum may be split into.
constexpr uint32_t kMaxColSplits = 4;

struct SqLayout {
  uint32_t nq_pad, ntiles;
  uint64_t stats, tiles, partial, qdense, chunk_stats, bytes;  // byte offsets
};

__host__ SqLayout sq_layout(int64_t nq, int64_t nk, int64_t hq, int64_t hkv) {
  SqLayout L;
  L.ntiles = uint32_t((nq + kQTile - 1) / kQTile);
  // a multiple of 4 tiles: the column pass's units of 4 tiles (one head per
  // KV head) read whole groups of tile records, statistics and query rows
  L.nq_pad = (L.ntiles + 3) / 4 * 4 * kQTile;
  L.stats = 0;
  // (plus a tile of rows: the last unit of (tile, head) rows may reach the
  // rows of the tile past the last query tile, which it masks)
  L.tiles = (L.stats + (uint64_t(hq) * L.nq_pad + kQTile) * 8 + 255) & ~uint64_t(255);
  // (plus 4 records: a unit's requests read T records from its first tile)
  L.partial = (L.tiles + uint64_t(L.nq_pad / kQTile + 4) * kTileWords * 4 + 255) & ~uint64_t(255);
  L.qdense = (L.partial + uint64_t(kMaxColSplits) * hkv * nk * 4 + 255) & ~uint64_t(255);
  // padded by one unit: a partial head chunk's requests read past its group
  L.chunk_stats = (L.qdense + (uint64_t(L.nq_pad) * hq + 4 * kQTile) * kMaxHeadDim * 2 + 255) & ~uint64_t(255);
  L.bytes = (L.chunk_stats + uint64_t(kMaxRowChunks) * hq * L.nq_pad * 8 + 255) & ~uint64_t(255);
  return L;
}

// Compute units of the current device (cached per device).
int device_cus(int* cus) {
  static std::mutex mu;
  static int cached[64] = {};
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return set_error(CBK_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(err));
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= 0 && dev < 64 && cached[dev] > 0) {
    *cus = cached[dev];
    return CBK_OK;
  }
  err = hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (err != hipSuccess) return set_error(CBK_ERR_LAUNCH, "CU count: %s", hipGetErrorString(err));
  if (dev >= 0 && dev < 64) cached[dev] = *cus;
  return CBK_OK;
}

// Key ranges per (query tile, kv head) in rowstats: tiles differ in work by
// their positions (causal), and one workgroup per tile left the latest tiles
// running alone at the end; with ranges, about six workgroups per resident
// slot are dispatched in decreasing order of work (C5, same box: 3.525-3.530
// ms at 6 ranges against 3.557-3.583 at 3, 3.533 at 8, 3.556-3.579 at 12).
constexpr uint32_t kRowChunkTarget = 6;  // rowstats workgroups per resident slot (about)

// Query-unit ranges per (key block, kv head) in colsum: a block's work is
// the query units that see it (the earliest blocks: all of them), and the
// dispatch runs in decreasing order of work; with ranges, about four colsum
// workgroups per resident slot (three per CU): 2 ranges at C5 (3.521 ->
// 3.445-3.446 ms same box; 3 ranges 3.444-3.446, 4 ranges 3.449).
constexpr uint32_t kColSplitTarget = 4;

uint32_t col_splits(uint32_t units, int cus) {
  const uint32_t slots = 3u * uint32_t(cus);
  const uint32_t k = units ? (kColSplitTarget * slots + units - 1) / units : 1u;
  return std::max(1u, std::min(kMaxColSplits, k));
}

uint32_t row_chunks(uint32_t units, int cus, uint32_t per_cu) {
  const uint32_t slots = per_cu * uint32_t(cus);  // rowstats workgroups resident per CU
  const uint32_t k = units ? (kRowChunkTarget * slots + units - 1) / units : 1u;
  return std::max(1u, std::min(kMaxRowChunks, k));
}

// Sets the launch's key ranges in `a`.
template <typename V, int RMODE, int KS>
int launch_mfma_ks(SqArgs& a, int cus, hipStream_t stream) {
  const uint64_t ntiles = (a.nq + kQTile - 1) / kQTile;
  const uint64_t kblocks = (a.nk + kKeyBlock2 - 1) / kKeyBlock2;
  // Query tiles per row-pass workgroup by heads per KV head: up to 4, four
  // tiles, one wave per tile with the whole group; 5-8, two tiles, two waves
  // per tile with up to four head slots each; more, one tile (its 16 heads
  // on 32x32 MFMAs). Measured on 98,304-key layers of 4,096 sparse queries
  // (C5 positions, ms at head_dim 128 against one tile per workgroup, which
  // left waves without a head below 4): 1 head 13.83 -> 8.17, 2 heads 7.34 ->
  // 5.03, 3 heads 3.57 -> 2.96, 4 heads 4.19 -> 3.53, 5 heads 5.87 -> 5.34,
  // 6 heads 6.58 -> 5.71, 7 heads 3.49 -> 3.23 (28 query heads over 4).
  const uint32_t tpw = a.groups <= 4 ? 4u : a.groups <= 8 ? 2u : 1u;
  const uint64_t tgroups = (ntiles + tpw - 1) / tpw;
  const int waves = tpw == 4 ? ((KS == 4 || a.groups >= 3) ? 2 : 3) : tpw == 2 ? 2 : (a.groups > 8 && KS == 4) ? 2 : 3;
  a.row_chunks = row_chunks(uint32_t(tgroups * a.hkv), cus, uint32_t(waves));
  // one-dimensional grids (the kv head fastest): every launch within 2^32 threads
  CBK_REQUIRE(tgroups * a.hkv * a.row_chunks * kThreads < (uint64_t(1) << 32) &&
                  kblocks * a.hkv * kMaxColSplits * kThreads < (uint64_t(1) << 32) &&
                  uint64_t(a.hq) * a.nq_pad < (uint64_t(1) << 32),
              "sparse_q: %llu query tiles x %llu key blocks x %u kv heads exceed one launch",
              (unsigned long long)ntiles, (unsigned long long)kblocks, a.hkv);
  a.col_splits = col_splits(uint32_t(kblocks * a.hkv), cus);
  // units of four (tile, head) rows address a KV head's statistics with
  // per-lane 32-bit byte offsets
  CBK_REQUIRE(a.groups % kHeadChunk == 0 || uint64_t(a.groups) * a.nq_pad * 8 < (uint64_t(1) << 31),
              "sparse_q: %u heads per KV head x %u query rows exceed the column pass's offsets", a.groups,
              a.nq_pad);
  const dim3 g1(uint32_t(tgroups * a.hkv * a.row_chunks));
  const dim3 g2(uint32_t(kblocks * a.hkv * a.col_splits));
  if (a.groups == 1)
    hipLaunchKernelGGL((sq_rowstats_kernel<V, KS, 1, RMODE, true, 4>), g1, dim3(kThreads), 0, stream, a);
  else if (a.groups == 2)
    hipLaunchKernelGGL((sq_rowstats_kernel<V, KS, 2, RMODE, true, 4>), g1, dim3(kThreads), 0, stream, a);
  else if (a.groups == 3)
    hipLaunchKernelGGL((sq_rowstats_kernel<V, KS, 3, RMODE, true, 4>), g1, dim3(kThreads), 0, stream, a);
  else if (a.groups == 4)
    hipLaunchKernelGGL((sq_rowstats_kernel<V, KS, 4, RMODE, true, 4>), g1, dim3(kThreads), 0, stream, a);
  else if (a.groups == 8)
    hipLaunchKernelGGL((sq_rowstats_kernel<V, KS, 4, RMODE, true, 2>), g1, dim3(kThreads), 0, stream, a);
  else if (a.groups < 8)
    hipLaunchKernelGGL((sq_rowstats_kernel<V, KS, 4, RMODE, false, 2>), g1, dim3(kThreads), 0, stream, a);
  else if (a.groups == 16)
    hipLaunchKernelGGL((sq_rowstats_kernel<V, KS, 4, RMODE, true>), g1, dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((sq_rowstats_kernel<V, KS, 4, RMODE, false>), g1, dim3(kThreads), 0, stream, a);
  if (a.row_chunks > 1)
    hipLaunchKernelGGL(sq_merge_kernel, dim3((a.hq * a.nq_pad + kThreads - 1) / kThreads), dim3(kThreads), 0,
                       stream, a);
  // column-pass units: a tile's chunk of 4 heads when the group is a
  // multiple of 4, else four consecutive (tile, head) rows (spanning up to 4
  // tiles at one head per KV head, 2 otherwise); measured on 98,304-key
  // layers of 4,096 sparse queries at head_dim 128 against chunks whose
  // slots past the group computed unused rows: 1 head per KV head 8.05 ->
  // 5.21 ms, 2 heads 4.96 -> 4.16 ms (four rows of two tiles), 3 heads
  // 2.92 -> 2.78, 5 heads 5.27 -> 4.60, 6 heads 5.70 -> 5.31, 7 heads 3.24 ->
  // 3.20 ms
  if (a.groups % kHeadChunk == 0)
    hipLaunchKernelGGL((sq_colsum_kernel<V, KS, RMODE, true>), g2, dim3(kThreads), 0, stream, a);
  else if (a.groups == 1)
    hipLaunchKernelGGL((sq_colsum_kernel<V, KS, RMODE, true, 4, 1>), g2, dim3(kThreads), 0, stream, a);
  else if (a.groups == 2)
    hipLaunchKernelGGL((sq_colsum_kernel<V, KS, RMODE, true, 2, 2>), g2, dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((sq_colsum_kernel<V, KS, RMODE, true, 2>), g2, dim3(kThreads), 0, stream, a);
  return CBK_OK;
}

template <typename V, int RMODE>
int launch_mfma(SqArgs& a, int ksteps, hipStream_t stream) {
  int cus = 0;
  if (int rc = device_cus(&cus)) return rc;
  int rc = CBK_OK;
  switch (ksteps) {
    case 2: rc = launch_mfma_ks<V, RMODE, 2>(a, cus, stream); break;
    case 4: rc = launch_mfma_ks<V, RMODE, 4>(a, cus, stream); break;
    default: return set_error(CBK_ERR_UNSUPPORTED, "head_dim %u", a.d);
  }
  if (rc) return rc;
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
  a.tiles = reinterpret_cast<int32_t*>(ws + L.tiles);
  a.partial = reinterpret_cast<float*>(ws + L.partial);
  a.qdense = reinterpret_cast<uint16_t*>(ws + L.qdense);
  a.chunk_stats = reinterpret_cast<float2*>(ws + L.chunk_stats);
  a.row_chunks = 1;
  a.col_splits = 1;
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
    CBK_REQUIRE(round_logits == (dtype == CBK_DTYPE_BF16 ? 1 : 2),
                "the MFMA path rounds logits to the input dtype (round_logits %d)",
                dtype == CBK_DTYPE_BF16 ? 1 : 2);
    CBK_REQUIRE(scale > 0.f, "scale must be positive");
    // the DMA requests' per-lane 32-bit offsets span 64 key rows and 4 rows
    // of the statistics
    CBK_REQUIRE(nq <= (int64_t(1) << 26), "the MFMA path takes at most 2^26 queries, got %lld", (long long)nq);
    CBK_REQUIRE(k_row_stride_elems < (int64_t(1) << 24), "the MFMA path takes K row strides below 2^24 elements");
    const int ks = int(head_dim / 32);
    int rc = dtype == CBK_DTYPE_BF16 ? launch_mfma<s16x8, 1>(a, ks, s) : launch_mfma<h16x8, 2>(a, ks, s);
    if (rc) return rc;
  }
  if (int rc = launch_status("sparse_q")) return rc;
  const uint32_t n = uint32_t(std::max<int64_t>(full_scores_dev ? nk : 0, out_scores_dev ? n_out : 0));
  if (n > 0)
    hipLaunchKernelGGL(sq_gather_kernel, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, s,
                       a.partial, a.nk, a.hkv, a.col_splits, out_index_dev, uint32_t(out_scores_dev ? n_out : 0),
                       out_scores_dev, full_scores_dev);
  return launch_status("sparse_q gather");
}

}  // extern "C"
