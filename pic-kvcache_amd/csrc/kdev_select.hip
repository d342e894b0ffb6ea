// K-deviation scores and budgeted top-k selection for gfx950.
//
// kdev: one 64-lane wavefront per token row (a 512-element bf16 row is one
// 16 B load per lane per operand), kRowsPerWave rows in flight per wave,
// float32 accumulation, cross-lane sum by shuffles.
//
// select: a multi-block radix select over order-preserving uint32 keys,
// with no host round trip and no float atomics:
//   zero    clears histograms and counters
//   prepare base = gap|forced|dilate(gap,r), key = base ? key(-inf) : key(s),
//           LDS histogram of key[31:20] -> global; the last block computes the
//           budget k and the bin holding the k-th largest key
//   pass2   histogram of key[19:8] inside that bin; last block narrows
//   pass3   histogram of key[7:0]; last block fixes the k-th key T exactly
//           and `need` = how many keys equal to T are taken (lowest index)
//   tiecount per-tile counts of key == T and of sure picks; last block:
//           tie offsets, output offsets, total
//   write   per-tile ordered compaction of selected indices
// (the fused K-deviation launch clears the counters in its first block, so
// the zero launch is skipped there)
// Every tile is 2048 consecutive tokens (8 per thread), so tile order is
// index order and ties resolve to the lower index deterministically.
#include <mutex>

#include "cbk_common.hpp"

namespace cbk {
namespace {

// ------------------------------------------------------------------ kdev

constexpr int kKdevThreads = 256;
constexpr int kRowsPerWave = 2;  // rows per wave: 2 edges out 4 (65.4 vs 66.5 us per 64K-token select) and 1, 8

template <typename T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) {
  return bf16_bits_to_float(v);
}
template <> __device__ __forceinline__ float to_f32<_Float16>(_Float16 v) { return float(v); }

// VE elements per load; T is the storage type (uint16_t carries bf16 bits).
template <typename T, int VE>
__global__ __launch_bounds__(kKdevThreads) void kdev_kernel(
    const T* __restrict__ fresh, int64_t fs, const T* __restrict__ cached, int64_t cs,
    int64_t cached_rows_total, const int64_t* __restrict__ rows, int64_t row0, uint32_t n,
    uint32_t width, float* __restrict__ scores, uint32_t* __restrict__ zero_words, uint32_t nzero) {
  typedef T VecT __attribute__((ext_vector_type(VE)));
  // the fused score + select launch: block 0 also clears the selection's
  // counters (the selection kernels run after this launch on the stream)
  if (zero_words != nullptr && blockIdx.x == 0)
    for (uint32_t i = threadIdx.x; i < nzero; i += kKdevThreads) zero_words[i] = 0u;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = blockIdx.x * (kKdevThreads / 64) + (threadIdx.x >> 6);
  const uint32_t r0 = wave * kRowsPerWave;
  if (r0 >= n) return;

  const T* fp[kRowsPerWave];
  const T* cp[kRowsPerWave];
  bool ok[kRowsPerWave];
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const uint32_t r = r0 + i;
    ok[i] = r < n;
    fp[i] = fresh;
    cp[i] = cached;
    if (ok[i]) {
      const int64_t cr = rows ? rows[r] : row0 + int64_t(r);
      ok[i] = cr >= 0 && cr < cached_rows_total;
      fp[i] = fresh + int64_t(r) * fs;
      cp[i] = cached + cr * cs;
    }
  }
  float acc[kRowsPerWave];
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) acc[i] = 0.f;

  for (uint32_t j = lane * VE; j < width; j += 64 * VE) {
    VecT a[kRowsPerWave], b[kRowsPerWave];
#pragma unroll
    for (int i = 0; i < kRowsPerWave; ++i) {
      if (ok[i]) {
        a[i] = *reinterpret_cast<const VecT*>(fp[i] + j);
        b[i] = *reinterpret_cast<const VecT*>(cp[i] + j);
      }
    }
#pragma unroll
    for (int i = 0; i < kRowsPerWave; ++i) {
      if (ok[i]) {
#pragma unroll
        for (int e = 0; e < VE; ++e) {
          const float d = to_f32<T>(a[i][e]) - to_f32<T>(b[i][e]);
          acc[i] = fmaf(d, d, acc[i]);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const float s = wave_sum(acc[i]);
    if (lane == 0 && r0 + i < n) scores[r0 + i] = ok[i] ? s : __uint_as_float(0x7fc00000u);
  }
}

template <typename T>
int launch_kdev_t(const void* fresh, int64_t fs, const void* cached, int64_t cs, int64_t total_rows,
                  const int64_t* rows, int64_t row0, int64_t n, int64_t width, float* scores,
                  uint32_t* zero_words, uint32_t nzero, hipStream_t stream) {
  const int64_t eb = sizeof(T);
  int64_t vals[5] = {fs * eb, cs * eb, width * eb, int64_t(reinterpret_cast<uintptr_t>(fresh)),
                     int64_t(reinterpret_cast<uintptr_t>(cached))};
  const int vec_bytes = common_vec_bytes(vals, 5);
  const int64_t waves = (n + kRowsPerWave - 1) / kRowsPerWave;
  const dim3 grid(uint32_t((waves + kKdevThreads / 64 - 1) / (kKdevThreads / 64)));
  const T* f = static_cast<const T*>(fresh);
  const T* c = static_cast<const T*>(cached);
#define CBK_KDEV(VE)                                                                        \
  hipLaunchKernelGGL((kdev_kernel<T, VE>), grid, dim3(kKdevThreads), 0, stream, f, fs, c, cs, \
                     total_rows, rows, row0, uint32_t(n), uint32_t(width), scores, zero_words, nzero)
  switch (vec_bytes / int(eb)) {
    case 8: CBK_KDEV(8); break;
    case 4: CBK_KDEV(4); break;
    case 2: CBK_KDEV(2); break;
    default: CBK_KDEV(1); break;
  }
#undef CBK_KDEV
  return launch_status("kdev scores");
}

int launch_kdev(const void* fresh, int64_t fs, const void* cached, int64_t cs, int64_t total_rows,
                const int64_t* rows, int64_t row0, int64_t n, int64_t width, int32_t dtype,
                float* scores, hipStream_t stream, uint32_t* zero_words = nullptr, uint32_t nzero = 0) {
  CBK_REQUIRE(n >= 0 && width >= 0, "n and width must be non-negative");
  CBK_REQUIRE(n < (int64_t(1) << 31) && width < (int64_t(1) << 31), "n or width too large");
  if (n == 0) return CBK_OK;
  CBK_REQUIRE(fresh && cached && scores, "NULL pointer");
  CBK_REQUIRE(fs >= width && cs >= width, "row stride smaller than width");
  CBK_REQUIRE(total_rows > 0, "cached tensor has no rows");
  switch (dtype) {
    case CBK_DTYPE_F32:
      return launch_kdev_t<float>(fresh, fs, cached, cs, total_rows, rows, row0, n, width, scores,
                                  zero_words, nzero, stream);
    case CBK_DTYPE_BF16:
      return launch_kdev_t<uint16_t>(fresh, fs, cached, cs, total_rows, rows, row0, n, width, scores,
                                     zero_words, nzero, stream);
    case CBK_DTYPE_F16:
      return launch_kdev_t<_Float16>(fresh, fs, cached, cs, total_rows, rows, row0, n, width, scores,
                                     zero_words, nzero, stream);
    default:
      return set_error(CBK_ERR_UNSUPPORTED, "dtype %d", int(dtype));
  }
}

// ---------------------------------------------------------------- select

constexpr int kSelThreads = 256;
constexpr int kSelItems = 8;   // 2048-token tiles: 66.5 us per 64K tokens (1024: 68.7, 4096: 75.4)
constexpr int kSelTile = kSelThreads * kSelItems;
constexpr uint32_t kKeyNegInf = 0x007FFFFFu;  // order key of -inf

// workspace layout, in uint32 words
constexpr uint32_t kH1 = 0;        // 4096 bins, key[31:20]
constexpr uint32_t kH2 = 4096;     // 4096 bins, key[19:8]
constexpr uint32_t kH3 = 8192;     // 256 bins, key[7:0]
constexpr uint32_t kCtrl = 8448;   // 64 counters
constexpr uint32_t kHeader = 8512; // words cleared by the zero kernel
// ctrl slots
enum : uint32_t {
  C_GAP = 0, C_BASE, C_T_PREP, C_T_P2, C_T_P3, C_T_TIES, C_T_COUNT,
  C_TOPK, C_PREFIX1, C_KREM1, C_PREFIX2, C_KREM2, C_THRESH, C_NEED, C_TOTAL
};

struct SelLayout {
  uint32_t nblocks;
  uint64_t blk_ties;  // word offset: per-tile tie count -> exclusive tie offset
  uint64_t blk_sel;   // word offset: per-tile selected count -> exclusive output offset
  uint64_t keys;      // word offset: n order keys
  uint64_t base;      // BYTE offset: n base flags
  uint64_t bytes;     // total
};

constexpr SelLayout sel_layout(int64_t n) {
  SelLayout L{};
  L.nblocks = uint32_t((n + kSelTile - 1) / kSelTile);
  const uint64_t nb4 = (uint64_t(L.nblocks) + 3) & ~uint64_t(3);
  L.blk_ties = kHeader;
  L.blk_sel = L.blk_ties + nb4;
  L.keys = L.blk_sel + nb4;
  L.base = (L.keys + uint64_t(n)) * 4;
  L.bytes = (L.base + uint64_t(n) + 255) & ~uint64_t(255);
  return L;
}

struct SelArgs {
  const float* scores;
  const uint8_t* gap;
  const uint8_t* forced;
  uint32_t n;
  int32_t radius;
  double ratio;
  uint32_t* ws;
  uint32_t nblocks;
  uint32_t* blk_ties;
  uint32_t* blk_sel;
  uint32_t* keys;
  uint8_t* base;
  int64_t* out_idx;
  int64_t* out_count;
};

__device__ __forceinline__ uint32_t order_key(float s) {
  if (s != s) return 0xFFFFFFFFu;  // NaN ranks above every number
  uint32_t u = __float_as_uint(s);
  if (s == 0.0f) u = 0u;           // -0 ties +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint32_t ld_acq(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Last-arriving block detection: every block publishes its global atomics,
// then takes a ticket; the block holding ticket nblocks-1 sees all of them.
__device__ __forceinline__ bool last_block(uint32_t* ticket, uint32_t nblocks, uint32_t* lds_flag) {
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) *lds_flag = (atomicAdd(ticket, 1u) == nblocks - 1) ? 1u : 0u;
  __syncthreads();
  const bool last = *lds_flag != 0;
  if (last) __threadfence();
  return last;
}

// Among bins scanned from the highest down, find the one holding the k-th
// largest key: cum(above) < k <= cum(above) + hist[bin].
template <int NBINS>
__device__ void find_bin_desc(const uint32_t* hist, uint32_t k, uint32_t* lds_scan,
                              uint32_t* out_bin, uint32_t* out_krem) {
  constexpr int PER = NBINS / kSelThreads;
  uint32_t c[PER];
  uint32_t s = 0;
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    c[p] = ld_acq(&hist[NBINS - 1 - threadIdx.x * PER - p]);
    s += c[p];
  }
  uint32_t total;
  const uint32_t above = block_exclusive_scan<kSelThreads>(s, lds_scan, &total);
  if (above < k && k <= above + s) {
    uint32_t run = above;
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      if (run < k && k <= run + c[p]) {
        *out_bin = NBINS - 1 - threadIdx.x * PER - p;
        *out_krem = k - run;
      }
      run += c[p];
    }
  }
}

__global__ __launch_bounds__(kSelThreads) void sel_zero_kernel(uint32_t* ws) {
  for (uint32_t i = threadIdx.x; i < kHeader; i += kSelThreads) ws[i] = 0u;
}

// base flags, keys, first-digit histogram, budget.
__global__ __launch_bounds__(kSelThreads) void sel_prepare_kernel(const SelArgs a) {
  extern __shared__ uint32_t smem[];
  uint32_t* hist = smem;                 // 4096
  uint32_t* scan = smem + 4096;          // 8
  uint32_t* flag = smem + 4096 + 8;      // 1
  uint32_t* window = smem + 4096 + 16;   // kSelTile + 2r (+1)
  const uint32_t tile0 = blockIdx.x * kSelTile;
  const int r = a.radius;

  for (uint32_t i = threadIdx.x; i < 4096; i += kSelThreads) hist[i] = 0u;
  if (r > 0) {
    // inclusive prefix count of gaps over [tile0 - r, tile0 + kSelTile + r)
    const uint32_t W = kSelTile + 2 * r;
    const uint32_t per = (W + kSelThreads - 1) / kSelThreads;
    const uint32_t beg = threadIdx.x * per;
    const uint32_t end = min(W, beg + per);
    uint32_t local = 0;
    for (uint32_t w = beg; w < end; ++w) {
      const int64_t g = int64_t(tile0) - r + w;
      local += (g >= 0 && g < int64_t(a.n) && a.gap[g]) ? 1u : 0u;
      window[w] = local;
    }
    uint32_t total;
    const uint32_t excl = block_exclusive_scan<kSelThreads>(local, scan, &total);
    for (uint32_t w = beg; w < end; ++w) window[w] += excl;
  }
  __syncthreads();

  uint32_t gap_cnt = 0, base_cnt = 0;
  const uint32_t i0 = tile0 + threadIdx.x * kSelItems;
#pragma unroll
  for (int e = 0; e < kSelItems; ++e) {
    const uint32_t i = i0 + e;
    if (i < a.n) {
      const bool g = a.gap[i] != 0;
      bool b = g || (a.forced != nullptr && a.forced[i] != 0);
      if (r > 0 && !b) {
        const uint32_t k = i - tile0 + r;  // window index of token i
        const uint32_t hi = window[k + r];
        const uint32_t lo = (k >= uint32_t(r) + 1) ? window[k - r - 1] : 0u;
        b = hi > lo;
      }
      const uint32_t key = b ? kKeyNegInf : order_key(a.scores[i]);
      a.keys[i] = key;
      a.base[i] = b ? 1 : 0;
      gap_cnt += g ? 1u : 0u;
      base_cnt += b ? 1u : 0u;
      atomicAdd(&hist[key >> 20], 1u);
    }
  }
  gap_cnt = wave_sum_u32(gap_cnt);
  base_cnt = wave_sum_u32(base_cnt);
  if ((threadIdx.x & 63) == 0) {
    if (gap_cnt) atomicAdd(&a.ws[kCtrl + C_GAP], gap_cnt);
    if (base_cnt) atomicAdd(&a.ws[kCtrl + C_BASE], base_cnt);
  }
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < 4096; i += kSelThreads) {
    if (hist[i]) atomicAdd(&a.ws[kH1 + i], hist[i]);
  }
  if (!last_block(&a.ws[kCtrl + C_T_PREP], a.nblocks, flag)) return;

  // budget: int(cached * ratio) as Python computes it, then [1, available]
  __shared__ uint32_t s_topk;
  if (threadIdx.x == 0) {
    const int64_t n = a.n;
    const int64_t gaps = ld_acq(&a.ws[kCtrl + C_GAP]);
    const int64_t bases = ld_acq(&a.ws[kCtrl + C_BASE]);
    const int64_t cached = n - gaps;
    int64_t topk = int64_t(double(cached) * a.ratio);
    const int64_t available = n - bases;
    if (cached && available) {
      topk = topk < 1 ? 1 : topk;
      topk = topk > available ? available : topk;
    } else {
      topk = 0;
    }
    a.ws[kCtrl + C_TOPK] = uint32_t(topk);
    s_topk = uint32_t(topk);
  }
  __syncthreads();
  if (s_topk == 0) return;
  find_bin_desc<4096>(a.ws + kH1, s_topk, scan, &a.ws[kCtrl + C_PREFIX1], &a.ws[kCtrl + C_KREM1]);
}

// Narrowing passes: histogram of the next digit among keys sharing the
// prefix fixed so far. PASS 2: key[19:8] under key[31:20]; PASS 3: key[7:0]
// under key[31:8].
template <int PASS>
__global__ __launch_bounds__(kSelThreads) void sel_pass_kernel(const SelArgs a) {
  constexpr int NBINS = PASS == 2 ? 4096 : 256;
  __shared__ uint32_t hist[NBINS];
  __shared__ uint32_t scan[8];
  __shared__ uint32_t flag;
  if (a.ws[kCtrl + C_TOPK] == 0) return;
  const uint32_t prefix = PASS == 2 ? a.ws[kCtrl + C_PREFIX1] : a.ws[kCtrl + C_PREFIX2];
  const uint32_t krem = PASS == 2 ? a.ws[kCtrl + C_KREM1] : a.ws[kCtrl + C_KREM2];
  for (uint32_t i = threadIdx.x; i < NBINS; i += kSelThreads) hist[i] = 0u;
  __syncthreads();
  const uint32_t i0 = blockIdx.x * kSelTile + threadIdx.x * kSelItems;
#pragma unroll
  for (int e = 0; e < kSelItems; ++e) {
    const uint32_t i = i0 + e;
    if (i < a.n) {
      const uint32_t key = a.keys[i];
      if (PASS == 2) {
        if ((key >> 20) == prefix) atomicAdd(&hist[(key >> 8) & 0xFFFu], 1u);
      } else {
        if ((key >> 8) == prefix) atomicAdd(&hist[key & 0xFFu], 1u);
      }
    }
  }
  __syncthreads();
  uint32_t* gh = a.ws + (PASS == 2 ? kH2 : kH3);
  for (uint32_t i = threadIdx.x; i < NBINS; i += kSelThreads) {
    if (hist[i]) atomicAdd(&gh[i], hist[i]);
  }
  if (!last_block(&a.ws[kCtrl + (PASS == 2 ? C_T_P2 : C_T_P3)], a.nblocks, &flag)) return;
  __shared__ uint32_t bin, rem;
  if (threadIdx.x == 0) { bin = 0; rem = 0; }
  __syncthreads();
  find_bin_desc<NBINS>(gh, krem, scan, &bin, &rem);
  __syncthreads();
  if (threadIdx.x == 0) {
    if (PASS == 2) {
      a.ws[kCtrl + C_PREFIX2] = (prefix << 12) | bin;
      a.ws[kCtrl + C_KREM2] = rem;
    } else {
      a.ws[kCtrl + C_THRESH] = (prefix << 8) | bin;
      a.ws[kCtrl + C_NEED] = rem;
    }
  }
}

struct SelState {
  uint32_t topk, thresh, need;
};

__device__ __forceinline__ SelState load_state(const SelArgs& a) {
  SelState s;
  s.topk = a.ws[kCtrl + C_TOPK];
  s.thresh = a.ws[kCtrl + C_THRESH];
  s.need = a.ws[kCtrl + C_NEED];
  return s;
}

// Tile b's selected flags for this thread, with the tile's first tie rank
// given; *ties_out receives the tile's tie count.
__device__ __forceinline__ uint32_t tile_selected_bits(const SelArgs& a, const SelState& st, uint32_t b,
                                                       uint32_t rank0, uint32_t* scan, uint32_t* ties_out) {
  const uint32_t i0 = b * kSelTile + threadIdx.x * kSelItems;
  uint32_t keys[kSelItems];
  uint32_t tie_bits = 0, ties = 0;
#pragma unroll
  for (int e = 0; e < kSelItems; ++e) {
    const uint32_t i = i0 + e;
    keys[e] = i < a.n ? a.keys[i] : 0u;
    if (st.topk && i < a.n && keys[e] == st.thresh) {
      tie_bits |= 1u << e;
      ++ties;
    }
  }
  uint32_t rank = rank0 + block_exclusive_scan<kSelThreads>(ties, scan, ties_out);
  uint32_t bits = 0;
#pragma unroll
  for (int e = 0; e < kSelItems; ++e) {
    const uint32_t i = i0 + e;
    if (i >= a.n) continue;
    bool sel = a.base[i] != 0;
    if (st.topk) {
      if (keys[e] > st.thresh) sel = true;
      if (tie_bits & (1u << e)) {
        if (rank < st.need) sel = true;
        ++rank;
      }
    }
    if (sel) bits |= 1u << e;
  }
  return bits;
}

// Per tile: the ties (key == T) and the tokens taken for sure (base, or key
// above T); the last block turns them into exclusive tie offsets and output
// offsets and the total. A tile takes its ties whose index-order rank is
// below `need`: clamp(need - tie_offset, 0, ties). Base tokens carry the key
// of -inf, so they tie only when T is that key; then the last block counts
// tile by tile, token by token.
__global__ __launch_bounds__(kSelThreads) void sel_tiecount_kernel(const SelArgs a) {
  __shared__ uint32_t scan[8];
  __shared__ uint32_t flag;
  const SelState st = load_state(a);
  uint32_t ties = 0, sure = 0;
  const uint32_t i0 = blockIdx.x * kSelTile + threadIdx.x * kSelItems;
#pragma unroll
  for (int e = 0; e < kSelItems; ++e) {
    const uint32_t i = i0 + e;
    if (i < a.n) {
      const uint32_t key = a.keys[i];
      if (st.topk && key == st.thresh) ++ties;
      if (a.base[i] != 0 || (st.topk && key > st.thresh)) ++sure;
    }
  }
  uint32_t tile_ties, tile_sure;
  block_exclusive_scan<kSelThreads>(ties, scan, &tile_ties);
  block_exclusive_scan<kSelThreads>(sure, scan, &tile_sure);
  if (threadIdx.x == 0) {
    a.blk_ties[blockIdx.x] = tile_ties;
    a.blk_sel[blockIdx.x] = tile_sure;
  }
  if (!last_block(&a.ws[kCtrl + C_T_TIES], a.nblocks, &flag)) return;
  uint32_t carry_t = 0, carry_s = 0;
  if (st.topk && st.thresh == kKeyNegInf) {
    for (uint32_t b = 0; b < a.nblocks; ++b) {
      uint32_t tt, ts;
      const uint32_t bits = tile_selected_bits(a, st, b, carry_t, scan, &tt);
      block_exclusive_scan<kSelThreads>(__popc(bits), scan, &ts);
      if (threadIdx.x == 0) {
        a.blk_ties[b] = carry_t;
        a.blk_sel[b] = carry_s;
      }
      carry_t += tt;
      carry_s += ts;
    }
  } else {
    for (uint32_t b0 = 0; b0 < a.nblocks; b0 += kSelThreads) {
      const uint32_t b = b0 + threadIdx.x;
      const uint32_t t = b < a.nblocks ? ld_acq(&a.blk_ties[b]) : 0u;
      const uint32_t su = b < a.nblocks ? ld_acq(&a.blk_sel[b]) : 0u;
      uint32_t chunk_t, chunk_s;
      const uint32_t tie_off = carry_t + block_exclusive_scan<kSelThreads>(t, scan, &chunk_t);
      const int64_t left = int64_t(st.need) - int64_t(tie_off);
      const uint32_t taken = !st.topk || left <= 0 ? 0u : (left < int64_t(t) ? uint32_t(left) : t);
      const uint32_t out_off = carry_s + block_exclusive_scan<kSelThreads>(su + taken, scan, &chunk_s);
      if (b < a.nblocks) {
        a.blk_ties[b] = tie_off;
        a.blk_sel[b] = out_off;
      }
      carry_t += chunk_t;
      carry_s += chunk_s;
    }
  }
  if (threadIdx.x == 0) {
    a.ws[kCtrl + C_TOTAL] = carry_s;
    *a.out_count = int64_t(carry_s);
  }
}

__global__ __launch_bounds__(kSelThreads) void sel_write_kernel(const SelArgs a) {
  __shared__ uint32_t scan[8];
  const SelState st = load_state(a);
  uint32_t tile_ties;
  const uint32_t bits = tile_selected_bits(a, st, blockIdx.x, a.blk_ties[blockIdx.x], scan, &tile_ties);
  uint32_t total;
  uint32_t pos = a.blk_sel[blockIdx.x] + block_exclusive_scan<kSelThreads>(__popc(bits), scan, &total);
  const uint32_t i0 = blockIdx.x * kSelTile + threadIdx.x * kSelItems;
#pragma unroll
  for (int e = 0; e < kSelItems; ++e) {
    if (bits & (1u << e)) a.out_idx[pos++] = int64_t(i0 + e);
  }
}

__global__ void write_zero_count_kernel(int64_t* out_count) { *out_count = 0; }

int check_select(const float* scores, const uint8_t* gap, int64_t n, int64_t radius, double ratio,
                 int64_t* out_idx, int64_t* out_count, void* ws, size_t ws_bytes) {
  CBK_REQUIRE(n >= 0 && n < (int64_t(1) << 31), "n out of range");
  CBK_REQUIRE(out_count != nullptr, "out_count is NULL");
  CBK_REQUIRE(radius >= 0 && radius <= CBK_MAX_DILATION_RADIUS,
              "dilation radius %lld outside [0, %d]", (long long)radius, CBK_MAX_DILATION_RADIUS);
  CBK_REQUIRE(ratio == ratio, "ratio is NaN");
  if (n == 0) return CBK_OK;
  CBK_REQUIRE(scores && gap && out_idx && ws, "NULL pointer");
  const SelLayout L = sel_layout(n);
  if (ws_bytes < L.bytes)
    return set_error(CBK_ERR_WORKSPACE, "select workspace %zu < %llu bytes", ws_bytes,
                     (unsigned long long)L.bytes);
  CBK_REQUIRE((reinterpret_cast<uintptr_t>(ws) & 15) == 0, "workspace must be 16-byte aligned");
  return CBK_OK;
}

// header_zeroed: an earlier launch on the stream cleared the kHeader counter
// words (the fused K-deviation launch does)
int launch_select(const float* scores, const uint8_t* gap, const uint8_t* forced, int64_t n,
                  int64_t radius, double ratio, int64_t* out_idx, int64_t* out_count, void* ws,
                  size_t ws_bytes, hipStream_t stream, bool header_zeroed = false) {
  if (int rc = check_select(scores, gap, n, radius, ratio, out_idx, out_count, ws, ws_bytes)) return rc;
  if (n == 0) {
    hipLaunchKernelGGL(write_zero_count_kernel, dim3(1), dim3(1), 0, stream, out_count);
    return launch_status("select (empty)");
  }
  const SelLayout L = sel_layout(n);
  SelArgs a;
  a.scores = scores;
  a.gap = gap;
  a.forced = forced;
  a.n = uint32_t(n);
  a.radius = int32_t(radius);
  a.ratio = ratio;
  a.ws = static_cast<uint32_t*>(ws);
  a.nblocks = L.nblocks;
  a.blk_ties = a.ws + L.blk_ties;
  a.blk_sel = a.ws + L.blk_sel;
  a.keys = a.ws + L.keys;
  a.base = static_cast<uint8_t*>(ws) + L.base;
  a.out_idx = out_idx;
  a.out_count = out_count;
  const dim3 grid(L.nblocks), block(kSelThreads);
  const size_t prep_lds = (4096 + 16 + kSelTile + 2 * size_t(radius) + 1) * sizeof(uint32_t);
  if (!header_zeroed) hipLaunchKernelGGL(sel_zero_kernel, dim3(1), block, 0, stream, a.ws);
  hipLaunchKernelGGL(sel_prepare_kernel, grid, block, prep_lds, stream, a);
  hipLaunchKernelGGL(sel_pass_kernel<2>, grid, block, 0, stream, a);
  hipLaunchKernelGGL(sel_pass_kernel<3>, grid, block, 0, stream, a);
  hipLaunchKernelGGL(sel_tiecount_kernel, grid, block, 0, stream, a);
  hipLaunchKernelGGL(sel_write_kernel, grid, block, 0, stream, a);
  return launch_status("select");
}

// ---------------------------------------------------------------- dilate

constexpr int kDilTile = 1024;

__global__ __launch_bounds__(256) void dilate_kernel(const uint8_t* gap, uint32_t n, int32_t r,
                                                      uint8_t* out) {
  extern __shared__ uint32_t win[];  // kDilTile + 2r prefix counts
  __shared__ uint32_t scan[8];
  const uint32_t tile0 = blockIdx.x * kDilTile;
  const uint32_t W = kDilTile + 2 * r;
  const uint32_t per = (W + 255) / 256;
  const uint32_t beg = threadIdx.x * per;
  const uint32_t end = min(W, beg + per);
  uint32_t local = 0;
  for (uint32_t w = beg; w < end; ++w) {
    const int64_t g = int64_t(tile0) - r + w;
    local += (g >= 0 && g < int64_t(n) && gap[g]) ? 1u : 0u;
    win[w] = local;
  }
  uint32_t total;
  const uint32_t excl = block_exclusive_scan<256>(local, scan, &total);
  for (uint32_t w = beg; w < end; ++w) win[w] += excl;
  __syncthreads();
  for (uint32_t t = threadIdx.x; t < kDilTile; t += 256) {
    const uint32_t i = tile0 + t;
    if (i >= n) break;
    const uint32_t k = t + r;
    const uint32_t hi = win[k + r];
    const uint32_t lo = (k >= uint32_t(r) + 1) ? win[k - r - 1] : 0u;
    out[i] = hi > lo ? 1 : 0;
  }
}

}  // namespace

// ------------------------------------------------ allocation-free selection
// cbk_kdev_select_noalloc takes its workspace from `scratch`, a file-scope
// device array sized for CBK_NOALLOC_SELECT_MAX_TOKENS tokens (5.04 MiB,
// held on every GPU the library runs on until the process ends). In host
// code `scratch` names a host-side stand-in, not device memory: its device
// address is looked up once per device (hipGetSymbolAddress, with that
// device current) and only that address is ever passed to kernels. Every
// call on one GPU shares the array; the counters that must start at zero
// are cleared by the call's own score launch, and calls that overlap on one
// GPU (two streams at once) race on it.
constexpr size_t kNoallocScratchBytes = size_t(sel_layout(CBK_NOALLOC_SELECT_MAX_TOKENS).bytes);
static __device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};
}  // namespace

// Device address of `scratch` on the device `stream` belongs to (the
// current device for the NULL stream).
static int noalloc_scratch(hipStream_t stream, void** out) {
  int current = -1;
  hipError_t err = hipGetDevice(&current);
  if (err != hipSuccess)
    return set_error(CBK_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(err));
  int device = current;
  if (stream != nullptr) {
    err = hipStreamGetDevice(stream, &device);
    if (err != hipSuccess)
      return set_error(CBK_ERR_LAUNCH, "hipStreamGetDevice: %s", hipGetErrorString(err));
  }
  if (device < 0 || device >= kMaxDevices)
    return set_error(CBK_ERR_UNSUPPORTED, "device %d beyond the %d the scratch table holds", device,
                     kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[device] == nullptr) {
    if (device != current && (err = hipSetDevice(device)) != hipSuccess)
      return set_error(CBK_ERR_LAUNCH, "hipSetDevice(%d): %s", device, hipGetErrorString(err));
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (device != current) hipSetDevice(current);
    if (err != hipSuccess || ptr == nullptr)
      return set_error(CBK_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", device,
                       hipGetErrorString(err));
    g_scratch_dev[device] = ptr;
  }
  *out = g_scratch_dev[device];
  return CBK_OK;
}

}  // namespace cbk

extern "C" {

int cbk_kdev_scores(const void* fresh_dev, int64_t fresh_row_stride_elems, const void* cached_dev,
                    int64_t cached_row_stride_elems, int64_t cached_num_rows,
                    const int64_t* cached_rows_dev, int64_t cached_row0, int64_t n, int64_t width,
                    int32_t dtype, float* scores_dev, cbk_stream_t stream) {
  cbk::clear_error();
  return cbk::launch_kdev(fresh_dev, fresh_row_stride_elems, cached_dev, cached_row_stride_elems,
                          cached_num_rows, cached_rows_dev, cached_row0, n, width, dtype,
                          scores_dev, static_cast<hipStream_t>(stream));
}

size_t cbk_select_workspace_bytes(int64_t n) {
  if (n <= 0) return 256;
  return size_t(cbk::sel_layout(n).bytes);
}

int cbk_select(const float* scores_dev, const uint8_t* gap_dev, const uint8_t* forced_dev,
               int64_t n, int64_t radius, double ratio, int64_t* out_idx_dev,
               int64_t* out_count_dev, void* workspace_dev, size_t workspace_bytes,
               cbk_stream_t stream) {
  cbk::clear_error();
  return cbk::launch_select(scores_dev, gap_dev, forced_dev, n, radius, ratio, out_idx_dev,
                            out_count_dev, workspace_dev, workspace_bytes,
                            static_cast<hipStream_t>(stream));
}

int cbk_kdev_select(const void* fresh_dev, int64_t fresh_row_stride_elems, const void* cached_dev,
                    int64_t cached_row_stride_elems, int64_t cached_num_rows,
                    const int64_t* cached_rows_dev, int64_t cached_row0, int64_t n, int64_t width,
                    int32_t dtype, const uint8_t* gap_dev, const uint8_t* forced_dev,
                    int64_t radius, double ratio, float* scores_dev, int64_t* out_idx_dev,
                    int64_t* out_count_dev, void* workspace_dev, size_t workspace_bytes,
                    cbk_stream_t stream) {
  cbk::clear_error();
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (int rc = cbk::check_select(scores_dev, gap_dev, n, radius, ratio, out_idx_dev, out_count_dev,
                                 workspace_dev, workspace_bytes))
    return rc;
  const bool zero = n > 0;  // the score launch clears the selection counters
  if (int rc = cbk::launch_kdev(fresh_dev, fresh_row_stride_elems, cached_dev,
                                cached_row_stride_elems, cached_num_rows, cached_rows_dev,
                                cached_row0, n, width, dtype, scores_dev, s,
                                zero ? static_cast<uint32_t*>(workspace_dev) : nullptr,
                                zero ? cbk::kHeader : 0u))
    return rc;
  return cbk::launch_select(scores_dev, gap_dev, forced_dev, n, radius, ratio, out_idx_dev,
                            out_count_dev, workspace_dev, workspace_bytes, s, zero);
}

int cbk_kdev_select_noalloc(const void* fresh_dev, int64_t fresh_row_stride_elems,
                            const void* cached_dev, int64_t cached_row_stride_elems,
                            int64_t cached_num_rows, const int64_t* cached_rows_dev,
                            int64_t cached_row0, int64_t n, int64_t width, int32_t dtype,
                            const uint8_t* gap_dev, const uint8_t* forced_dev, int64_t radius,
                            double ratio, float* scores_dev, int64_t* out_idx_dev,
                            int64_t* out_count_dev, cbk_stream_t stream) {
  cbk::clear_error();
  if (n > CBK_NOALLOC_SELECT_MAX_TOKENS)
    return cbk::set_error(CBK_ERR_INVALID,
                          "kdev_select_noalloc: %lld tokens exceed its static scratch maximum of %d",
                          (long long)n, CBK_NOALLOC_SELECT_MAX_TOKENS);
  void* scratch = nullptr;
  if (int rc = cbk::noalloc_scratch(static_cast<hipStream_t>(stream), &scratch)) return rc;
  return cbk_kdev_select(fresh_dev, fresh_row_stride_elems, cached_dev, cached_row_stride_elems,
                         cached_num_rows, cached_rows_dev, cached_row0, n, width, dtype, gap_dev,
                         forced_dev, radius, ratio, scores_dev, out_idx_dev, out_count_dev, scratch,
                         cbk::kNoallocScratchBytes, stream);
}

int cbk_dilate(const uint8_t* gap_dev, int64_t n, int64_t radius, uint8_t* forced_dev,
               cbk_stream_t stream) {
  cbk::clear_error();
  CBK_REQUIRE(n >= 0 && n < (int64_t(1) << 31), "n out of range");
  CBK_REQUIRE(radius >= 0 && radius <= CBK_MAX_DILATION_RADIUS,
              "dilation radius %lld outside [0, %d]", (long long)radius, CBK_MAX_DILATION_RADIUS);
  if (n == 0) return CBK_OK;
  CBK_REQUIRE(gap_dev && forced_dev, "NULL pointer");
  const uint32_t grid = uint32_t((n + cbk::kDilTile - 1) / cbk::kDilTile);
  const size_t lds = (cbk::kDilTile + 2 * size_t(radius)) * sizeof(uint32_t);
  hipLaunchKernelGGL(cbk::dilate_kernel, dim3(grid), dim3(256), lds, static_cast<hipStream_t>(stream),
                     gap_dev, uint32_t(n), int32_t(radius), forced_dev);
  return cbk::launch_status("dilate");
}

}  // extern "C"
