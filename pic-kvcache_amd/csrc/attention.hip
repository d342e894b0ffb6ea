// Side-forward attention of the selected queries for gfx950 (the blend
// executor's attention over the layer buffer, cacheblend_vllm/ascend.py:
// 798-846):
//
//   out[i, h] = sum_{k <= pos_i} softmax_k( r(r(q[i, h] . key[k, h/G]) * scale) ) value[k, h/G]
//
// with r rounding to the input dtype (the reference's bf16/f16 einsum output
// and its "* scale"), the softmax in float32, G = Hq / Hkv.
//
// One workgroup (4 waves) per (128 rows of (query, group head), kv head):
// row r of the 128 is query r / G, head kv * G + r % G, so the K/V tiles
// staged in LDS serve all G heads of several queries. Per 32-key block:
//   S^T = K . Q^T   v_mfma_f32_16x16x32_{bf16,f16}: A = K rows, B = Q rows,
//                   both 16-byte loads of 8 consecutive dims; the result
//                   holds key 4*(lane/16)+i of row lane%16 in register i
//   softmax         per row in the log2 domain against a fixed reference:
//                   the maximum of the row's first block (a logit of the row,
//                   so no term exceeds 2^(max - m)); no per-logit maximum in
//                   the later blocks. A row whose sum outgrows it (2^100) is
//                   recomputed with online maxima (lazily rescaled, the row's
//                   32 keys of a block spread over its 4 lane groups)
//   O += P . V      v_mfma_f32_16x16x32_{bf16,f16}: the two halves' S^T
//                   registers, concatenated, are the A operand (row lane%16,
//                   keys 4*(lane/16)..+3 and 16+4*(lane/16)..+3: the
//                   contraction runs in that key order); B needs those keys
//                   of one dim, which two ds_read_tr16_b64 gather from the
//                   row-major V block
// software-pipelined: the step of block b issues S^T of block b+1 and P . V
// of block b-1 beside the softmax of block b. K/V blocks stream through
// rings of three LDS buffers by DMA (global_load_lds); the row tiles with the
// latest positions (most keys) are scheduled first.
// MFMA layout (checked on gfx950): 16x16x32 A[i][k] in lane i+16*(k/8)
// element k%8, B[k][j] in lane j+16*(k/8); D[i][j] in lane j+16*(i/4),
// register i%4.
//
// float32 inputs take an exact float32 path (one wave per (query, head)).
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <cmath>
#include <type_traits>

#include "cbk_common.hpp"

namespace cbk {
namespace {

typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 4 waves per workgroup, each with two 16-row tiles: every K and V fragment
// read from LDS serves 32 rows, a K/V block 128 (234 registers with the
// software pipeline: two waves per SIMD, two workgroups per CU at head_dim
// 128; 152-157 registers and three waves per SIMD at head_dim 64, which
// measured 1.28-1.31 ms against 1.44 ms at two on a 32-head, 8-KV-head,
// 32K-key layer). Measured against 8 waves of one tile (four waves per
// SIMD): 2.02-2.04 vs 2.12-2.15 ms per C3 layer.
constexpr int kWaves = 4;
constexpr int kRowTiles = 2;  // 16-row tiles per wave
constexpr int kKeyBlock = 32;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();
constexpr float kRescale = 8.f;  // log2 headroom of the lazy softmax rescaling

struct AttnArgs {
  const uint16_t* q;      // [nq, hq, d], row stride q_stride elements
  const int64_t* pos;     // [nq] key positions of the queries
  const uint16_t* k;      // [nk, hkv, d], row stride k_stride
  const uint16_t* v;      // [nk, hkv, d], row stride v_stride
  uint16_t* out;          // [nq, hq, d], row stride out_stride
  int64_t q_stride, k_stride, v_stride, out_stride;
  uint32_t nq, nk, hq, hkv, group, d;
  float scale;
};

template <bool F16> struct Ops;
template <> struct Ops<false> {  // bf16
  typedef s16x8 A8;
  typedef s16x4 A4;
  static __device__ __forceinline__ f32x4 mma32(const A8& a, const A8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  // two floats -> two bf16 (round to nearest even) packed low/high
  static __device__ __forceinline__ uint32_t pack(float x, float y) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){x, y}, b2));
  }
  static __device__ __forceinline__ float lo(uint32_t u) { return __uint_as_float(u << 16); }
  static __device__ __forceinline__ float hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
};
template <> struct Ops<true> {  // f16
  typedef h16x8 A8;
  typedef h16x4 A4;
  static __device__ __forceinline__ f32x4 mma32(const A8& a, const A8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float x, float y) {
    const __half2 h = __floats2half2_rn(x, y);
    return __builtin_bit_cast(uint32_t, h);
  }
  static __device__ __forceinline__ float lo(uint32_t u) {
    return __half2float(__builtin_bit_cast(__half, uint16_t(u & 0xffffu)));
  }
  static __device__ __forceinline__ float hi(uint32_t u) {
    return __half2float(__builtin_bit_cast(__half, uint16_t(u >> 16)));
  }
};

// Rounds a pair to the dtype and back (the dtype's matmul / multiply output;
// bf16: one instruction per value).
template <bool F16>
__device__ __forceinline__ void round2(float& x, float& y) {
  if constexpr (F16) {
    const uint32_t u = Ops<F16>::pack(x, y);
    x = Ops<F16>::lo(u);
    y = Ops<F16>::hi(u);
  } else {
    x = bf16_round(x);
    y = bf16_round(y);
  }
}

// bf16 / f16 1.0 in both halves of a word: the B operand of the "ones"
// column whose MFMA accumulates each row's sum of (rounded) probabilities
template <bool F16> constexpr uint32_t kOnesPair = F16 ? 0x3c003c00u : 0x3f803f80u;

// A lane's LDS read offsets within a K or V block, bytes, the same in every
// buffer: the K fragment of dim step st and the V transposing read of column
// tile c, both for the first 16-key half (the second half is 16 rows
// further: the swizzle of row 16 + r equals that of row r).
template <int D>
struct BlockOffsets {
  uint32_t k[D / 32];
  uint32_t v[D / 16];
  __device__ __forceinline__ explicit BlockOffsets(uint32_t lane) {
    const uint32_t row = lane & 15, grp = lane >> 4;
#pragma unroll
    for (int st = 0; st < D / 32; ++st) k[st] = (row * D + ((4 * st + grp) ^ lds_swizzle<D>(row)) * 8) * 2;
    // lane (row, grp) addresses key 4 grp + row / 4, dims 16c + 4 (row % 4) .. + 3
    // of the row-major V block
    const uint32_t vkey = 4 * grp + (row >> 2);
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      const uint32_t dim = 16 * c + 4 * (row & 3);
      v[c] = (vkey * D + ((dim / 8) ^ lds_swizzle<D>(vkey)) * 8 + (dim & 4)) * 2;
    }
  }
};

// S^T = K . Q^T of one block (K buffer ks) for every row tile; each K
// fragment is read from LDS once.
template <bool F16, int D, int RT>
__device__ __forceinline__ void qk_block(const uint16_t* ks, const BlockOffsets<D>& off,
                                         const typename Ops<F16>::A8 (&qf)[RT][D / 32], f32x4 (&s)[RT][2]) {
  using O = Ops<F16>;
  constexpr uint32_t kHalf = 16 * D * 2;  // bytes from a 16-key half to the next
#pragma unroll
  for (int t = 0; t < RT; ++t) s[t][0] = s[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < D / 32; ++st) {
    const char* kp = reinterpret_cast<const char*>(ks) + off.k[st];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const typename O::A8 kf = *reinterpret_cast<const typename O::A8*>(kp + h * kHalf);
#pragma unroll
      for (int t = 0; t < RT; ++t) s[t][h] = O::mma32(kf, qf[t][st], s[t][h]);
    }
  }
}

// The block's logits in place of its S^T: x = r(r(dot) * scale), as the
// dtype's einsum and multiply produce them (MASK: -inf past each row's
// position); lm[t] = this lane's maximum over its logits of row tile t, taken
// before the second rounding (rounding is monotonic, and the reference
// maximum only needs to bound the logits within the rescale headroom).
template <bool F16, int RT, bool MASK, bool WITH_MAX = true>
__device__ __forceinline__ void logits_block(f32x4 (&s)[RT][2], int32_t k0, float scale, const int32_t (&rpos)[RT],
                                             float (&lm)[RT], uint32_t grp) {
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    float y[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      y[h][0] = s[t][h][0]; y[h][1] = s[t][h][1]; y[h][2] = s[t][h][2]; y[h][3] = s[t][h][3];
      round2<F16>(y[h][0], y[h][1]);
      round2<F16>(y[h][2], y[h][3]);
      y[h][0] *= scale; y[h][1] *= scale; y[h][2] *= scale; y[h][3] *= scale;
      if constexpr (MASK) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (k0 + 16 * h + int32_t(4 * grp) + i > rpos[t]) y[h][i] = kNegInf;
      }
    }
    if constexpr (WITH_MAX)
      lm[t] = fmaxf(fmaxf(fmaxf(y[0][0], y[0][1]), fmaxf(y[0][2], y[0][3])),
                    fmaxf(fmaxf(y[1][0], y[1][1]), fmaxf(y[1][2], y[1][3])));
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      round2<F16>(y[h][0], y[h][1]);
      round2<F16>(y[h][2], y[h][3]);
      s[t][h] = f32x4{y[h][0], y[h][1], y[h][2], y[h][3]};
    }
  }
}

// p = 2^(x log2 e - m), rounded to the dtype: the A operand of P . V (the
// two 16-key halves' registers, concatenated); nms = -m (0 while m is -inf).
template <bool F16, int RT>
__device__ __forceinline__ void probs_block(const f32x4 (&x)[RT][2], const float (&nms)[RT],
                                            typename Ops<F16>::A8 (&pa)[RT]) {
  using O = Ops<F16>;
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    typename O::A4 ph[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(fmaf(x[t][h][i], kLog2e, nms[t]));
      const u32x2 pk = u32x2{O::pack(p[0], p[1]), O::pack(p[2], p[3])};
      ph[h] = __builtin_bit_cast(typename O::A4, pk);
    }
    pa[t] = __builtin_shufflevector(ph[0], ph[1], 0, 1, 2, 3, 4, 5, 6, 7);
  }
}

// O += P . V and the row sums l += P . 1, one 16x16x32 MFMA per 16-dim column
// tile for the block's 32 keys (two 16x16x16 MFMAs cost as much each). The
// contraction runs in this lane layout's key order: k-slot 8 grp + e holds
// key 4 grp + e for e < 4 and 16 + 4 grp + e - 4 after, in P (the S^T
// registers of the two 16-key halves, concatenated) and in V (two
// transposing reads, one per half, concatenated).
template <bool F16, int D, int RT>
__device__ __forceinline__ void pv_block(const uint16_t* vs, const BlockOffsets<D>& off,
                                         const typename Ops<F16>::A8 (&pa)[RT], f32x4 (&o)[RT][D / 16],
                                         f32x4 (&ol)[RT]) {
  using O = Ops<F16>;
  constexpr uint32_t kHalf = 16 * D * 2;
  typedef short s16x4v __attribute__((ext_vector_type(4)));
  const typename O::A8 ones = __builtin_bit_cast(
      typename O::A8, u32x4{kOnesPair<F16>, kOnesPair<F16>, kOnesPair<F16>, kOnesPair<F16>});
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
    // lane (row, grp) addresses key 16h + 4 grp + row / 4, dims 16c + 4 (row % 4) .. + 3 of
    // the row-major V block; ds_read_tr16_b64 hands lane j of each 16-lane group element i of
    // its group's lane 4i + j / 4, i.e. V[16h + 4 grp + i][16c + j]
    const char* vp = reinterpret_cast<const char*>(vs) + off.v[c];
    s16x4v w[2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
      w[h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4v*)((__attribute__((address_space(3))) const void*)(vp + h * kHalf)));
    const typename O::A8 vb =
        __builtin_bit_cast(typename O::A8, __builtin_shufflevector(w[0], w[1], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
    for (int t = 0; t < RT; ++t) o[t][c] = O::mma32(pa[t], vb, o[t][c]);
  }
#pragma unroll
  for (int t = 0; t < RT; ++t) ol[t] = O::mma32(pa[t], ones, ol[t]);
}

// K and V blocks of 32 keys stream through rings of three LDS buffers by DMA
// (global_load_lds, explicit vmcnt waits, plain s_barrier; see the LDS DMA
// helpers): K three blocks ahead of the step that reads it, V one.
template <bool F16, int D, int RT>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(D == 64 ? 3 : 2, D == 64 ? 3 : 2))) void attn_kernel(
    const AttnArgs a) {
  constexpr int W = kWaves;
  constexpr int kRows = W * 16 * RT;  // rows per workgroup
  constexpr uint32_t P = D / 8;                      // 16-byte pieces per key row
  constexpr uint32_t kInsts = kKeyBlock * P / 64 / W; // requests per wave per block, each of K and V
  constexpr uint32_t kRowsPerInst = 64 / P;
  constexpr int kBuffers = 3;
  static_assert(kInsts >= 1 && W * 16 * D <= 2 * kBuffers * kKeyBlock * D, "wave count vs block and staging");
  // K blocks, then V blocks; the output staging reuses the whole region
  __shared__ __attribute__((aligned(16))) uint16_t kvbuf[2][kBuffers][kKeyBlock * D];
  auto& kbuf = kvbuf[0];
  auto& vbuf = kvbuf[1];
  __shared__ int32_t s_max[W];
  using O = Ops<F16>;
  // wave-uniform values in scalar registers (readfirstlane: a division by a
  // runtime value runs on the VALU), so what derives from them stays scalar
  const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t row = lane & 15, grp = lane >> 4;
  // workgroup -> (row tile, kv head), the kv head fastest and the latest
  // tiles (most keys) first: work is dispatched in decreasing order across
  // all heads
  const uint32_t kvh = __builtin_amdgcn_readfirstlane(blockIdx.x % a.hkv);
  const uint32_t nrows = a.nq * a.group;
  const uint32_t ntiles = (nrows + kRows - 1) / kRows;
  const uint32_t tile = __builtin_amdgcn_readfirstlane(ntiles - 1 - blockIdx.x / a.hkv);
  const uint32_t r_wave = tile * kRows + wave * 16 * RT;

  // this lane's rows (one per row tile): (query, head) and their Q fragments
  typename O::A8 qf[RT][D / 32];
  int32_t rpos[RT];
  int32_t wmax = -1, wmin = 0x7fffffff;
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const uint32_t r = r_wave + 16 * t + row;
    const bool valid = r < nrows;
    const uint32_t qi = valid ? r / a.group : 0;
    const uint32_t qh = kvh * a.group + (valid ? r % a.group : 0);
    // a position at or past the context's end sees every key (the last
    // block's rows past nk repeat its last key and must stay masked)
    rpos[t] = valid ? int32_t(min(a.pos[qi], int64_t(a.nk) - 1)) : -1;
#pragma unroll
    for (int st = 0; st < D / 32; ++st) {
      u32x4 w = u32x4(0u);
      if (valid)
        w = *reinterpret_cast<const u32x4*>(a.q + int64_t(qi) * a.q_stride + int64_t(qh) * D + 32 * st + 8 * grp);
      qf[t][st] = __builtin_bit_cast(typename O::A8, w);
    }
    wmax = max(wmax, rpos[t]);
    if (valid) wmin = min(wmin, rpos[t]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    wmax = max(wmax, __shfl_xor(wmax, off));
    wmin = min(wmin, __shfl_xor(wmin, off));
  }
  if (lane == 0) s_max[wave] = wmax;
  __syncthreads();
  // workgroup-uniform: a scalar loop bound
  int32_t gm = s_max[0];
#pragma unroll
  for (int w = 1; w < W; ++w) gm = max(gm, s_max[w]);
  const int32_t gmax = __builtin_amdgcn_readfirstlane(gm);
  // blocks up to the latest position, within the context
  const int32_t nblocks =
      gmax < 0 ? 0 : min((gmax + kKeyBlock) / kKeyBlock, (int32_t(a.nk) + kKeyBlock - 1) / kKeyBlock);

  // per row tile: the reference max m (log2 units), -m for the exponents
  // (0 while m is -inf), and the logit above which m is raised,
  // (m + kRescale) ln 2 (all three change only when m is raised)
  float m[RT], nms[RT], thr[RT];
  f32x4 o[RT][D / 16], ol[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    m[t] = kNegInf;
    nms[t] = 0.f;
    thr[t] = kNegInf;
    ol[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < D / 16; ++c) o[t][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // nothing of the compiler's own in flight once the requests start
  CBK_WAIT_VM_LGKM0(0);

  // per-lane request offsets (key row of the block, swizzled piece), bytes
  uint32_t krow[kInsts], koff[kInsts], voff[kInsts];
#pragma unroll
  for (uint32_t j = 0; j < kInsts; ++j) {
    krow[j] = (wave * kInsts + j) * kRowsPerInst + lane / P;
    const uint32_t piece = (lane % P) ^ lds_swizzle<D>(krow[j]);
    koff[j] = uint32_t((krow[j] * a.k_stride + kvh * D + piece * 8) * 2);
    voff[j] = uint32_t((krow[j] * a.v_stride + kvh * D + piece * 8) * 2);
  }
  // K of block b into K buffer b % 3, V of block b into V buffer b % 3
  // (clamped: a request past the end repeats the last block); rows past nk
  // of the last block repeat its last key (masked)
  auto request = [&](int32_t b, const uint16_t* src, int64_t stride, const uint32_t (&offs)[kInsts],
                     uint16_t (&bufs)[kBuffers][kKeyBlock * D]) {
    const uint32_t l = lds_address(bufs[b % kBuffers]);
    b = min(b, nblocks - 1);
    const int32_t k0 = b * kKeyBlock;
    const uint16_t* base = src + int64_t(k0) * stride;
    if (k0 + kKeyBlock <= int32_t(a.nk)) {
#pragma unroll
      for (uint32_t j = 0; j < kInsts; ++j) lds_dma16(base, offs[j], l + (wave * kInsts + j) * 1024);
    } else {
      const uint32_t last = uint32_t(int32_t(a.nk) - 1 - k0);
#pragma unroll
      for (uint32_t j = 0; j < kInsts; ++j) {
        const uint32_t back = krow[j] - min(krow[j], last);  // rows to step back past nk
        lds_dma16(base, offs[j] - uint32_t(back * stride * 2), l + (wave * kInsts + j) * 1024);
      }
    }
  };
  const BlockOffsets<D> off(lane);
  // this wave's blocks: [0, b_m) are visible to all of its rows, [b_m, b_w)
  // masked, [b_w, nblocks) past its latest position (skipped; the wave still
  // takes its part in the requests and barriers).
  const int32_t wmin_s = __builtin_amdgcn_readfirstlane(wmin), wmax_s = __builtin_amdgcn_readfirstlane(wmax);
  const int32_t b_w = wmax_s < 0 ? 0 : min(wmax_s / kKeyBlock + 1, nblocks);
  const int32_t b_m = wmax_s < 0 ? 0 : min(int32_t((int64_t(wmin_s) + 1) / kKeyBlock), b_w);
  // Software pipeline: step b takes S^T of block b + 1 on the MFMAs while
  // the VALU turns block b's S^T into logits, then P . V of block b - 1
  // while the VALU turns block b's logits into probabilities: the matrix
  // cores and the VALU work on independent data in one instruction stream
  // (MFMA/VALU co-execution 23% -> 42% of the MFMA busy time; under the
  // power limit the clock fell 6%, so 2.11-2.12 -> 2.05-2.07 ms per C3 layer
  // in same-box runs). K(b + 1) and V(b - 1) are read in step b. The loops
  // take six steps at a time, so that the ring buffers and the register sets
  // of every step are known at compile time: no per-read address adds
  // (1.99 -> 1.93 ms per C3 layer in same-box runs).
  // Lazy rescaling: exponents stay relative to a reference max m that is
  // raised -- and O rescaled -- only when some lane sees a logit above
  // m + kRescale (log2 units); otherwise p <= 2^kRescale. The row max across
  // the row's 4 lane groups is only needed then. A raise found in step b
  // rescales O in step b + 1, between P . V of block b - 1 (relative to the
  // old m) and P . V of block b (relative to the new one): each step has one
  // uniform branch, between its two halves.
  bool pending = false;     // O still to be rescaled by alpha
  float alpha[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) alpha[t] = 1.f;
  auto rescale_o = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      float ao[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) ao[i] = __shfl(alpha[t], int(4 * grp + i));
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        o[t][c][0] *= ao[0]; o[t][c][1] *= ao[1]; o[t][c][2] *= ao[2]; o[t][c][3] *= ao[3];
      }
      ol[t][0] *= ao[0]; ol[t][1] *= ao[1]; ol[t][2] *= ao[2]; ol[t][3] *= ao[3];
    }
  };
  // The steps' request streams: K three blocks ahead of the step, V one,
  // clamped at the last block (every block before it is whole). Block j's K
  // goes to K buffer j % 3, its V to V buffer j % 3 (kVOffset bytes after
  // that K buffer).
  constexpr uint32_t kSlot = kKeyBlock * D * 2, kVOffset = kBuffers * kSlot;
  const int64_t kstep = int64_t(kKeyBlock) * a.k_stride * 2, vstep = int64_t(kKeyBlock) * a.v_stride * 2;
  const bool last_whole = nblocks * kKeyBlock <= int32_t(a.nk);
  const char* const kg0 = reinterpret_cast<const char*>(a.k) + int64_t(min(3, nblocks - 1)) * kstep;
  const char* const vg0 = reinterpret_cast<const char*>(a.v) + int64_t(min(1, nblocks - 1)) * vstep;
  const char* kg = kg0;
  const char* vg = vg0;
  auto stream = [&](int32_t j, const char*& g, int64_t stride_bytes, int64_t stride, const uint32_t (&offs)[kInsts],
                    uint32_t l) __attribute__((always_inline)) {
    const bool inner = j < nblocks - 1;
    if (inner || last_whole) {
#pragma unroll
      for (uint32_t i = 0; i < kInsts; ++i) lds_dma16(g, offs[i], l + (wave * kInsts + i) * 1024);
    } else {
      const uint32_t last = uint32_t(int32_t(a.nk) - 1 - (nblocks - 1) * kKeyBlock);
#pragma unroll
      for (uint32_t i = 0; i < kInsts; ++i) {
        const uint32_t back = krow[i] - min(krow[i], last);  // rows to step back past nk
        lds_dma16(g, offs[i] - uint32_t(back * stride * 2), l + (wave * kInsts + i) * 1024);
      }
    }
    if (inner) g += stride_bytes;
  };
  // KIND: 0 visible, 1 masked, 2 P . V of the wave's last block only, 3 no
  // work; FIRST: no block before; PHASE: b % 6 when known at compile time
  // (then every LDS address is a lane's offset plus a constant the DS
  // instruction's offset field carries), or -1. sc holds S^T of block b, pp
  // P of block b - 1; the step leaves S^T of block b + 1 in sn and P of
  // block b in pc (two register sets taken in turn: no copies between
  // steps).
  auto step = [&](auto kind, auto first, auto phase, auto fix, int32_t b, f32x4 (&sc)[RT][2],
                  f32x4 (&sn)[RT][2], typename O::A8 (&pp)[RT], typename O::A8 (&pc)[RT])
                  __attribute__((always_inline)) {
    constexpr int KIND = decltype(kind)::value;
    constexpr bool FIRST = decltype(first)::value;
    constexpr int PHASE = decltype(phase)::value;
    constexpr bool FIX = decltype(fix)::value;
    CBK_WAIT_VM_LGKM0(2 * kInsts);  // K(b + 1) and V(b - 1) have landed
    asm volatile("s_barrier" ::: "memory");
    uint32_t kb_addr, vb_addr, kw_addr, vw_addr;
    if constexpr (PHASE >= 0) {
      kw_addr = lds_address(kbuf[PHASE % 3]);
      vw_addr = lds_address(vbuf[(PHASE + 1) % 3]);
      kb_addr = lds_address(kbuf[(PHASE + 1) % 3]);
      vb_addr = lds_address(vbuf[(PHASE + 2) % 3]);
    } else {
      const uint32_t r = uint32_t(b) % 3;
      const uint32_t k0 = lds_address(kbuf[0]);
      kw_addr = k0 + r * kSlot;
      kb_addr = k0 + (r == 2 ? 0 : r + 1) * kSlot;
      vw_addr = kb_addr + kVOffset;
      vb_addr = k0 + (r == 0 ? 2 : r - 1) * kSlot + kVOffset;
      asm volatile("" : "+s"(kb_addr), "+s"(vb_addr));
    }
    stream(b + 3, kg, kstep, a.k_stride, koff, kw_addr);  // into the K buffer block b used
    stream(b + 1, vg, vstep, a.v_stride, voff, vw_addr);  // into the V buffer block b - 2 used
    if constexpr (KIND < 3) {
      const uint16_t* ks = (const uint16_t*)(__attribute__((address_space(3))) const uint16_t*)(size_t)kb_addr;
      const uint16_t* vs = (const uint16_t*)(__attribute__((address_space(3))) const uint16_t*)(size_t)vb_addr;
      if constexpr (KIND < 2 && FIX) {
        qk_block<F16, D, RT>(ks, off, qf, sn);
        float lm[RT];
        logits_block<F16, RT, KIND == 1, false>(sc, b * kKeyBlock, a.scale, rpos, lm, grp);
        probs_block<F16, RT>(sc, nms, pc);
        if constexpr (!FIRST) pv_block<F16, D, RT>(vs, off, pp, o, ol);
#pragma unroll
        for (int t = 0; t < RT; ++t) asm volatile("" : "+v"(pc[t]));
      } else if constexpr (KIND < 2) {
        qk_block<F16, D, RT>(ks, off, qf, sn);
        float lm[RT];
        logits_block<F16, RT, KIND == 1>(sc, b * kKeyBlock, a.scale, rpos, lm, grp);
        uint64_t over = 0;
#pragma unroll
        for (int t = 0; t < RT; ++t) over |= __ballot(lm[t] > thr[t]);
        if (pending || over != 0) {
          if (pending) rescale_o();
          pending = false;
#pragma unroll
          for (int t = 0; t < RT; ++t) {
            alpha[t] = 1.f;
            if (__any(lm[t] > thr[t])) {
              float bm = lm[t];
              bm = fmaxf(bm, __shfl_xor(bm, 16));
              bm = fmaxf(bm, __shfl_xor(bm, 32));
              const float mn = fmaxf(m[t], bm * kLog2e + 1.f);  // +1: covers the second rounding
              alpha[t] = mn == kNegInf ? 1.f : __builtin_amdgcn_exp2f(m[t] - mn);
              m[t] = mn;
              nms[t] = -mn;
              thr[t] = (mn + kRescale) * kLn2;
              pending = true;
            }
          }
        }
        probs_block<F16, RT>(sc, nms, pc);
        if constexpr (!FIRST) pv_block<F16, D, RT>(vs, off, pp, o, ol);
        // P of block b is computed here, beside P . V of block b - 1 (the
        // compiler would otherwise sink it to its use in the next step)
#pragma unroll
        for (int t = 0; t < RT; ++t) asm volatile("" : "+v"(pc[t]));
      } else if constexpr (!FIRST) {
        if constexpr (!FIX) {
          if (pending) rescale_o();
          pending = false;
        }
        pv_block<F16, D, RT>(vs, off, pp, o, ol);
      }
    }
  };
  using visible = std::integral_constant<int, 0>;
  using masked = std::integral_constant<int, 1>;
  using last = std::integral_constant<int, 2>;
  using none = std::integral_constant<int, 3>;
  using yes = std::true_type;
  using no = std::false_type;
  f32x4 sa[RT][2], sb[RT][2];
  typename O::A8 pa[RT], pb[RT];
  using any = std::integral_constant<int, -1>;
  // one step with its buffers chosen at run time, S^T of block b in sa and P
  // of block b - 1 in pa before and after
  auto single = [&](auto kind, auto fix, int32_t& b) __attribute__((always_inline)) {
    step(kind, no(), any(), fix, b++, sa, sb, pa, pb);
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      sa[t][0] = sb[t][0];
      sa[t][1] = sb[t][1];
      pa[t] = pb[t];
    }
  };
  // steps [b, end) of one kind: six at a time from a multiple of 6 (the
  // three-buffer rings and the two register sets back where they started),
  // single steps at the edges
  auto run = [&](auto kind, auto fix, int32_t& b, int32_t end) __attribute__((always_inline)) {
    while (b < end && b % 6 != 0) single(kind, fix, b);
    for (; b + 6 <= end; b += 6) {
      step(kind, no(), std::integral_constant<int, 0>(), fix, b, sa, sb, pa, pb);
      step(kind, no(), std::integral_constant<int, 1>(), fix, b + 1, sb, sa, pb, pa);
      step(kind, no(), std::integral_constant<int, 2>(), fix, b + 2, sa, sb, pa, pb);
      step(kind, no(), std::integral_constant<int, 3>(), fix, b + 3, sb, sa, pb, pa);
      step(kind, no(), std::integral_constant<int, 4>(), fix, b + 4, sa, sb, pa, pb);
      step(kind, no(), std::integral_constant<int, 5>(), fix, b + 5, sb, sa, pb, pa);
    }
    while (b < end) single(kind, fix, b);
  };
  // one pass over the blocks; the first step always takes the lazy path (it
  // sets each row's reference from block 0, where every row with a position
  // sees key 0 at least)
  auto pass = [&](auto fix) __attribute__((always_inline)) {
    // K of blocks 0-2 and V of block 0 ahead of step 0; then every wave
    // takes steps 0 .. nblocks (the requests and barriers of each)
    request(0, a.k, a.k_stride, koff, kbuf);
    request(1, a.k, a.k_stride, koff, kbuf);
    request(2, a.k, a.k_stride, koff, kbuf);
    request(0, a.v, a.v_stride, voff, vbuf);
    CBK_WAIT_VM_LGKM0(3 * kInsts);  // K(0) has landed
    asm volatile("s_barrier" ::: "memory");
    if (b_w > 0) {
      qk_block<F16, D, RT>((const uint16_t*)(__attribute__((address_space(3))) const uint16_t*)(size_t)lds_address(
                               kbuf[0]),
                           off, qf, sa);
    }
    int32_t b = 0;
    auto first = [&](auto kind) __attribute__((always_inline)) {
      step(kind, yes(), any(), no(), b++, sa, sb, pa, pb);
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        sa[t][0] = sb[t][0];
        sa[t][1] = sb[t][1];
        pa[t] = pb[t];
      }
    };
    if (b_m > 0)
      first(visible());
    else if (b_w > 0)
      first(masked());
    run(visible(), fix, b, b_m);
    run(masked(), fix, b, b_w);
    if (b_w > 0)
      step(last(), no(), any(), fix, b++, sa, sb, pa, pb);
    else
      step(none(), yes(), any(), fix, b++, sa, sb, pa, pb);
    for (; b <= nblocks; ++b) step(none(), no(), any(), fix, b, sa, sb, pa, pb);
    CBK_WAIT_VM_LGKM0(0);  // no LDS write in flight past this point
  };
  // Fixed reference: after block 0 every row keeps the reference its first
  // step set (a logit of the row, so p <= 2^(max - m)) -- no per-logit
  // maximum, no threshold ballot. A row whose terms outgrew it (its sum past
  // 2^100: a logit more than ~69 above the first block's maximum) or whose
  // output is not finite is recomputed, workgroup-wide, with the lazy
  // rescaling.
  __shared__ uint32_t s_redo;
  if (nblocks > 0) {
    pass(yes());
    bool bad = false;
#pragma unroll
    for (int t = 0; t < RT; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bad |= !(ol[t][i] < 0x1p100f);
#pragma unroll
        for (int c = 0; c < D / 16; ++c) bad |= !(fabsf(o[t][c][i]) < 3.0e38f);
      }
    }
    if (threadIdx.x == 0) s_redo = 0;
    __syncthreads();
    if (bad) s_redo = 1;
    __syncthreads();
    if (__builtin_amdgcn_readfirstlane(s_redo)) {  // uniform: the pass's loops stay scalar
      pending = false;
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        m[t] = kNegInf;
        nms[t] = 0.f;
        thr[t] = kNegInf;
        alpha[t] = 1.f;
        ol[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < D / 16; ++c) o[t][c] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      kg = kg0;
      vg = vg0;
      pass(no());
    }
  }
  __syncthreads();  // every wave is done with the K buffers the output staging reuses

  // normalize and write, one row tile at a time through the wave's LDS
  // staging area (the K buffers are free now): whole 16-byte pieces per row
  uint16_t* os = &kvbuf[0][0][0] + wave * 16 * D;
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    // row sums of the rounded probabilities, already in O's layout
    float lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) lo[i] = ol[t][i] > 0.f ? 1.f / ol[t][i] : 0.f;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      const uint32_t u01 = O::pack(o[t][c][0] * lo[0], o[t][c][1] * lo[1]);
      const uint32_t u23 = O::pack(o[t][c][2] * lo[2], o[t][c][3] * lo[3]);
      const uint32_t col = 16 * c + row;
      os[(4 * grp + 0) * D + col] = uint16_t(u01 & 0xffffu);
      os[(4 * grp + 1) * D + col] = uint16_t(u01 >> 16);
      os[(4 * grp + 2) * D + col] = uint16_t(u23 & 0xffffu);
      os[(4 * grp + 3) * D + col] = uint16_t(u23 >> 16);
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 16 * (D / 8) / 64; ++c) {
      const uint32_t idx = lane + 64 * c;
      const uint32_t orow = idx / (D / 8), chunk = idx % (D / 8);
      const uint32_t rr = r_wave + 16 * t + orow;
      if (rr < nrows) {
        const uint32_t oq = rr / a.group, oh = kvh * a.group + rr % a.group;
        *reinterpret_cast<u32x4*>(a.out + int64_t(oq) * a.out_stride + int64_t(oh) * D + chunk * 8) =
            *reinterpret_cast<const u32x4*>(&os[orow * D + chunk * 8]);
      }
    }
    __syncthreads();
  }
}

// float32: one wave per (query, head), exact float32 dots and accumulation,
// two dims per lane (D <= 128).
struct AttnArgsF32 {
  const float* q;
  const int64_t* pos;
  const float* k;
  const float* v;
  float* out;
  int64_t q_stride, k_stride, v_stride, out_stride;
  uint32_t nq, nk, hq, hkv, group, d;
  float scale;
};

__global__ __launch_bounds__(256) void attn_f32_kernel(const AttnArgsF32 a) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t job = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (job >= a.nq * a.hq) return;  // whole waves exit together
  const uint32_t qi = job / a.hq, h = job % a.hq, kvh = h / a.group;
  const float* q = a.q + int64_t(qi) * a.q_stride + int64_t(h) * a.d;
  const float q0 = lane < a.d ? q[lane] : 0.f;
  const float q1 = lane + 64 < a.d ? q[lane + 64] : 0.f;
  int64_t last = a.pos[qi];
  if (last >= int64_t(a.nk)) last = int64_t(a.nk) - 1;
  float m = kNegInf, l = 0.f, o0 = 0.f, o1 = 0.f;
  for (int64_t j = 0; j <= last; ++j) {
    const float* kr = a.k + j * a.k_stride + int64_t(kvh) * a.d;
    const float* vr = a.v + j * a.v_stride + int64_t(kvh) * a.d;
    float dot = (lane < a.d ? q0 * kr[lane] : 0.f) + (lane + 64 < a.d ? q1 * kr[lane + 64] : 0.f);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) dot += __shfl_xor(dot, off);
    const float x = dot * a.scale;
    const float mn = fmaxf(m, x);
    const float alpha = expf(m - mn);
    const float p = expf(x - mn);
    l = l * alpha + p;
    o0 = o0 * alpha + p * (lane < a.d ? vr[lane] : 0.f);
    o1 = o1 * alpha + p * (lane + 64 < a.d ? vr[lane + 64] : 0.f);
    m = mn;
  }
  float* out = a.out + int64_t(qi) * a.out_stride + int64_t(h) * a.d;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (lane < a.d) out[lane] = o0 * inv;
  if (lane + 64 < a.d) out[lane + 64] = o1 * inv;
}

}  // namespace
}  // namespace cbk

extern "C" int cbk_blend_attention(const void* q_dev, int64_t q_row_stride_elems, const int64_t* q_pos_dev,
                                   int64_t nq, const void* k_dev, int64_t k_row_stride_elems,
                                   const void* v_dev, int64_t v_row_stride_elems, int64_t nk, int64_t hq,
                                   int64_t hkv, int64_t head_dim, float scale, int32_t dtype, void* out_dev,
                                   int64_t out_row_stride_elems, cbk_stream_t stream) {
  using namespace cbk;
  clear_error();
  CBK_REQUIRE(nq >= 0 && nq < (int64_t(1) << 26), "nq out of range");
  if (nq == 0) return CBK_OK;
  CBK_REQUIRE(q_dev && q_pos_dev && k_dev && v_dev && out_dev, "NULL pointer");
  CBK_REQUIRE(nk > 0 && nk < (int64_t(1) << 31), "nk out of range");
  CBK_REQUIRE(hq > 0 && hkv > 0 && hq % hkv == 0, "query heads must be divisible by KV heads");
  CBK_REQUIRE(nq * hq < (int64_t(1) << 31), "nq * hq too large");
  CBK_REQUIRE(q_row_stride_elems >= hq * head_dim && out_row_stride_elems >= hq * head_dim &&
                  k_row_stride_elems >= hkv * head_dim && v_row_stride_elems >= hkv * head_dim,
              "row stride smaller than a row");
  CBK_REQUIRE(std::isfinite(scale), "scale must be finite");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == CBK_DTYPE_F32) {
    CBK_REQUIRE(head_dim > 0 && head_dim <= 128, "float32 path needs head_dim <= 128");
    AttnArgsF32 a;
    a.q = static_cast<const float*>(q_dev);
    a.pos = q_pos_dev;
    a.k = static_cast<const float*>(k_dev);
    a.v = static_cast<const float*>(v_dev);
    a.out = static_cast<float*>(out_dev);
    a.q_stride = q_row_stride_elems;
    a.k_stride = k_row_stride_elems;
    a.v_stride = v_row_stride_elems;
    a.out_stride = out_row_stride_elems;
    a.nq = uint32_t(nq);
    a.nk = uint32_t(nk);
    a.hq = uint32_t(hq);
    a.hkv = uint32_t(hkv);
    a.group = uint32_t(hq / hkv);
    a.d = uint32_t(head_dim);
    a.scale = scale;
    const uint64_t jobs = uint64_t(nq) * uint64_t(hq);
    hipLaunchKernelGGL(attn_f32_kernel, dim3(uint32_t((jobs + 3) / 4)), dim3(256), 0, s, a);
    return launch_status("blend attention f32");
  }
  CBK_REQUIRE(dtype == CBK_DTYPE_BF16 || dtype == CBK_DTYPE_F16, "dtype %d", int(dtype));
  CBK_REQUIRE(head_dim == 64 || head_dim == 128, "head_dim %lld: 64 or 128 supported", (long long)head_dim);
  const int64_t align[8] = {q_row_stride_elems * 2, k_row_stride_elems * 2, v_row_stride_elems * 2,
                            out_row_stride_elems * 2,
                            int64_t(reinterpret_cast<uintptr_t>(q_dev)), int64_t(reinterpret_cast<uintptr_t>(k_dev)),
                            int64_t(reinterpret_cast<uintptr_t>(v_dev)), int64_t(reinterpret_cast<uintptr_t>(out_dev))};
  CBK_REQUIRE(common_vec_bytes(align, 8) == 16, "q/k/v/out pointers and row strides must be 16-byte aligned");
  // the K/V requests' per-lane 32-bit byte offsets span a 32-key block
  CBK_REQUIRE(k_row_stride_elems < (int64_t(1) << 24) && v_row_stride_elems < (int64_t(1) << 24),
              "K/V row strides must stay below 2^24 elements");
  AttnArgs a;
  a.q = static_cast<const uint16_t*>(q_dev);
  a.pos = q_pos_dev;
  a.k = static_cast<const uint16_t*>(k_dev);
  a.v = static_cast<const uint16_t*>(v_dev);
  a.out = static_cast<uint16_t*>(out_dev);
  a.q_stride = q_row_stride_elems;
  a.k_stride = k_row_stride_elems;
  a.v_stride = v_row_stride_elems;
  a.out_stride = out_row_stride_elems;
  a.nq = uint32_t(nq);
  a.nk = uint32_t(nk);
  a.hq = uint32_t(hq);
  a.hkv = uint32_t(hkv);
  a.group = uint32_t(hq / hkv);
  a.d = uint32_t(head_dim);
  a.scale = scale;
  const uint64_t nrows = uint64_t(nq) * uint64_t(a.group);
  constexpr int RT = kRowTiles;
  const uint32_t waves = kWaves;
  const uint64_t rows_per_wg = 16 * RT * uint64_t(waves);
  const uint64_t groups = (nrows + rows_per_wg - 1) / rows_per_wg * uint64_t(hkv);
  CBK_REQUIRE(groups * 64 * waves < (uint64_t(1) << 32), "blend attention: %llu workgroups exceed one launch",
              (unsigned long long)groups);
  const dim3 grid(static_cast<uint32_t>(groups)), block(64 * waves);
  const bool f16 = dtype == CBK_DTYPE_F16;
  if (head_dim == 128) {
    if (f16) hipLaunchKernelGGL((attn_kernel<true, 128, RT>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((attn_kernel<false, 128, RT>), grid, block, 0, s, a);
  } else {
    if (f16) hipLaunchKernelGGL((attn_kernel<true, 64, RT>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((attn_kernel<false, 64, RT>), grid, block, 0, s, a);
  }
  return launch_status("blend attention");
}
