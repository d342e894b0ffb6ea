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
// SUB rows share a wave pass, 64 / SUB lanes each: rows of at most 32 or 16
// vectors (e.g. 2 KV heads x 128 bf16, a 4-KV-head layer split over two
// ranks) would otherwise leave half or three quarters of the lanes without
// a load (2 heads: 63% of 8 TB/s with one row per pass).
template <typename T, int VE, int SUB>
__global__ __launch_bounds__(kKdevThreads) void kdev_kernel(
    const T* __restrict__ fresh, int64_t fs, const T* __restrict__ cached, int64_t cs,
    int64_t cached_rows_total, const int64_t* __restrict__ rows, int64_t row0, uint32_t n,
    uint32_t width, float* __restrict__ scores, uint32_t* __restrict__ zero_words, uint32_t nzero) {
  typedef T VecT __attribute__((ext_vector_type(VE)));
  // the fused score + select launch: block 0 also clears the selection's
  // counters (the selection kernels run after this launch on the stream)
  if (zero_words != nullptr && blockIdx.x == 0)
    for (uint32_t i = threadIdx.x; i < nzero; i += kKdevThreads) zero_words[i] = 0u;
  constexpr uint32_t LPR = 64 / SUB;  // lanes per row
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t sub = lane / LPR, l = lane % LPR;
  const uint32_t wave = blockIdx.x * (kKdevThreads / 64) + (threadIdx.x >> 6);
  const uint32_t r0 = wave * kRowsPerWave * SUB;  // rows r0 + SUB i + sub
  if (r0 >= n) return;

  const T* fp[kRowsPerWave];
  const T* cp[kRowsPerWave];
  bool ok[kRowsPerWave];
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const uint32_t r = r0 + SUB * i + sub;
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

  for (uint32_t j = l * VE; j < width; j += LPR * VE) {
    VecT a[kRowsPerWave], b[kRowsPerWave];
    // read once: non-temporal loads (37.45-37.49 -> 37.09-37.39 us per
    // 64K-token select, same box)
#pragma unroll
    for (int i = 0; i < kRowsPerWave; ++i) {
      if (ok[i]) {
        a[i] = __builtin_nontemporal_load(reinterpret_cast<const VecT*>(fp[i] + j));
        b[i] = __builtin_nontemporal_load(reinterpret_cast<const VecT*>(cp[i] + j));
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
    float s = acc[i];
#pragma unroll
    for (uint32_t off = LPR / 2; off >= 1; off >>= 1) s += __shfl_xor(s, int(off), 64);
    const uint32_t r = r0 + SUB * i + sub;
    if (l == 0 && r < n) scores[r] = ok[i] ? s : __uint_as_float(0x7fc00000u);
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
  const int ve = vec_bytes / int(eb);
  // rows per wave pass: 4 for rows of at most 16 vectors, 2 for 32, else 1
  const int64_t row_vecs = (width + ve - 1) / ve;
  const int sub = row_vecs <= 16 ? 4 : row_vecs <= 32 ? 2 : 1;
  const int64_t waves = (n + kRowsPerWave * sub - 1) / (kRowsPerWave * sub);
  const dim3 grid(uint32_t((waves + kKdevThreads / 64 - 1) / (kKdevThreads / 64)));
  const T* f = static_cast<const T*>(fresh);
  const T* c = static_cast<const T*>(cached);
#define CBK_KDEV(VE, SUB)                                                                        \
  hipLaunchKernelGGL((kdev_kernel<T, VE, SUB>), grid, dim3(kKdevThreads), 0, stream, f, fs, c, cs, \
                     total_rows, rows, row0, uint32_t(n), uint32_t(width), scores, zero_words, nzero)
#define CBK_KDEV_SUB(VE)           \
  switch (sub) {                   \
    case 4: CBK_KDEV(VE, 4); break; \
    case 2: CBK_KDEV(VE, 2); break; \
    default: CBK_KDEV(VE, 1); break; \
  }
  switch (ve) {
    case 8: CBK_KDEV_SUB(8); break;
    case 4: CBK_KDEV_SUB(4); break;
    case 2: CBK_KDEV_SUB(2); break;
    default: CBK_KDEV_SUB(1); break;
  }
#undef CBK_KDEV_SUB
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
  C_TOPK, C_PREFIX1, C_KREM1, C_PREFIX2, C_KREM2, C_THRESH, C_NEED, C_TOTAL,
  // one-launch select: grid barrier arrivals (bit 31: the barrier failed),
  // candidates
  C_BAR = 16, C_GEN, C_CANDS
};
// candidates the one-launch select finishes in LDS (keys sharing the k-th
// key's 12- or 24-bit prefix)
constexpr uint32_t kCandCap = 8192;

struct SelLayout {
  uint32_t nblocks;
  uint64_t blk_ties;  // word offset: per-tile tie count -> exclusive tie offset
  uint64_t blk_sel;   // word offset: per-tile selected count -> exclusive output offset
  uint64_t tiles;     // word offset: 4 per-tile arrays of the one-launch select
  uint64_t cands;     // word offset: kCandCap candidate keys, then their indices
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
  L.tiles = L.blk_sel + nb4;
  L.cands = L.tiles + 4 * nb4;
  L.keys = L.cands + 2 * uint64_t(kCandCap);
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
  // one-launch select: per-tile base / sure / tie / selected counts and the
  // candidate list (keys, then indices with the base flag in bit 31)
  uint32_t* tile_base;
  uint32_t* tile_sure;
  uint32_t* tile_ties;
  uint32_t* tile_cnt;
  uint32_t* cand_key;
  uint32_t* cand_idx;
  uint32_t vec_ok;  // scores 16-byte and masks 8-byte aligned
  // grid barrier of the one-launch select: polls before giving up, and
  // arrivals expected beyond the grid's own (0; a test sets 1 with a spin
  // limit of 0 so every block gives up at once and exits normally)
  uint32_t spin_limit;
  uint32_t bar_extra;
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
// largest key: cum(above) < k <= cum(above) + hist[bin]. NT threads, PER
// bins each; threads past the last bin (NT > NBINS) read nothing.
template <int NBINS, int NT = kSelThreads>
__device__ void find_bin_desc(const uint32_t* hist, uint32_t k, uint32_t* lds_scan,
                              uint32_t* out_bin, uint32_t* out_krem, uint32_t* out_count = nullptr) {
  constexpr int PER = (NBINS + NT - 1) / NT;
  static_assert(NBINS % PER == 0, "bins split evenly over the threads that hold any");
  uint32_t c[PER];
  uint32_t s = 0;
  const uint32_t j0 = threadIdx.x * PER;  // this thread's bins: NBINS - 1 - (j0 .. j0 + PER - 1)
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    c[p] = j0 < NBINS ? ld_acq(&hist[NBINS - 1 - (j0 + p)]) : 0u;
    s += c[p];
  }
  uint32_t total;
  const uint32_t above = block_exclusive_scan<NT>(s, lds_scan, &total);
  if (j0 < NBINS && above < k && k <= above + s) {
    uint32_t run = above;
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      if (run < k && k <= run + c[p]) {
        *out_bin = NBINS - 1 - (j0 + p);
        *out_krem = k - run;
        if (out_count) *out_count = c[p];
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

// ---------------------------------------------------------------------
// One-launch selection (cooperative launch, every block co-resident).
//
// Block b owns tile b (NT * ITEMS tokens, ITEMS consecutive tokens
// per thread, kept in registers across the grid barriers):
//   P1  base flags (gap | forced | dilated gap), order keys, the tile's
//       12-bit first-digit histogram merged into H1; gap / base counts.
//   --  barrier
//   P2  every block finds the k-th key's first digit in H1 (the same answer
//       everywhere). If at most kCandCap keys share it, each block appends
//       its keys with that digit (key, index, base flag) to the candidate
//       list and publishes its count of tokens taken for sure (base, or a
//       higher digit); otherwise a second 12-bit digit narrows the prefix
//       (one more barrier), and if that still leaves more than kCandCap
//       keys the last 8 bits fix the k-th key exactly (ties path below).
//   --  barrier
//   P3  every block loads the candidates into LDS and finds the k-th
//       largest (key desc, index asc) among them: the threshold key T and
//       the largest index `cut` taken among keys equal to T. A token is
//       selected iff base, key > T, or key == T and index <= cut. Its
//       output offset is the sure counts of the earlier tiles plus the
//       selected non-base candidates below its first index.
// Ties path (more than kCandCap keys share the k-th key's 24-bit prefix,
// e.g. masses of equal scores): T and `need` come from the 8-bit digit,
// tiles publish their ties and sure counts, take ties in index order, and
// publish their selected counts before writing (three more barriers).
// ---------------------------------------------------------------------

constexpr uint32_t kBarrierSpins = 1u << 22;
constexpr uint32_t kBarrierFailed = 0x80000000u;

// Grid-wide barrier over `nblocks` co-resident blocks. C_BAR counts every
// block's arrivals over the launch (zeroed before it) in bits 0-30: barrier
// number `round` (1, 2, ...) is passed once the count reaches round *
// nblocks (+ bar_extra). Arrival is a posted atomic, so a block waits one
// round trip for the last arrival. A block that has polled spin_limit times
// without seeing the count complete marks the barrier failed (bit 31), by a
// compare-and-swap that succeeds only while the count is short. All blocks
// therefore agree: a block passes only on a count that reached the target
// with bit 31 clear, after which the mark can no longer be set; a block
// fails only on seeing the mark, after which the count can no longer pass
// (every later arrival and poll sees bit 31). Returns false on failure:
// the blocks were not all resident (or a test forced it), every block then
// writes a count of -1 and exits.
__device__ bool grid_barrier(uint32_t* ctrl, uint32_t nblocks, uint32_t round, const SelArgs& a,
                             uint32_t* lds_flag) {
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();  // this block's global writes before its arrival
    const uint32_t target = round * nblocks + a.bar_extra;
    uint32_t v = __hip_atomic_fetch_add(ctrl + C_BAR, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    uint32_t spins = 0;
    while (!(v & kBarrierFailed) && v < target) {
      if (spins++ >= a.spin_limit) {
        // give up: mark the barrier failed unless the count completes first
        while (!(v & kBarrierFailed) && v < target) {
          if (__hip_atomic_compare_exchange_strong(ctrl + C_BAR, &v, v | kBarrierFailed, __ATOMIC_RELAXED,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
            v |= kBarrierFailed;
          }
        }
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      v = __hip_atomic_load(ctrl + C_BAR, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __threadfence();  // the other blocks' writes after the barrier
    *lds_flag = (v & kBarrierFailed) ? 0u : 1u;
  }
  __syncthreads();
  return *lds_flag != 0;
}

__device__ __forceinline__ uint32_t ld_rlx(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS histogram `h` of NBINS bins: the bin holding the k-th largest
// (descending) or k-th smallest (ascending) element, and k's rank inside it.
template <int NT, int NBINS, bool DESC>
__device__ void lds_find_bin(const uint32_t* h, uint32_t k, uint32_t* scan, uint32_t* out_bin,
                             uint32_t* out_krem) {
  constexpr int PER = (NBINS + NT - 1) / NT;
  uint32_t c[PER];
  uint32_t s = 0;
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const int j = threadIdx.x * PER + p;
    const int bin = DESC ? NBINS - 1 - j : j;
    c[p] = j < NBINS ? h[bin] : 0u;
    s += c[p];
  }
  uint32_t total;
  const uint32_t before = block_exclusive_scan<NT>(s, scan, &total);
  if (before < k && k <= before + s) {
    uint32_t run = before;
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      if (run < k && k <= run + c[p]) {
        const int j = threadIdx.x * PER + p;
        *out_bin = DESC ? NBINS - 1 - j : j;
        *out_krem = k - run;
      }
      run += c[p];
    }
  }
  __syncthreads();
}

// Among the LDS candidates ck[0 .. cnt) whose top (32 - bits) key bits equal
// `prefix`, the key of the k-th largest: radix passes of up to 10 bits.
// Returns T; *need = k's rank among the candidates equal to T, *ties = their
// count.
template <int NT>
__device__ uint32_t cand_kth_key(const uint32_t* ck, uint32_t cnt, uint32_t prefix, int bits, uint32_t k,
                                 uint32_t* h, uint32_t* scan, uint32_t* sv, uint32_t* need,
                                 uint32_t* ties) {
  uint32_t pfx = prefix;
  uint32_t want = k;
  uint32_t last = cnt;
  while (bits > 0) {
    const int b = bits > 10 ? 10 : bits;
    bits -= b;
    for (uint32_t j = threadIdx.x; j < (1u << b); j += NT) h[j] = 0u;
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < cnt; j += NT) {
      const uint32_t key = ck[j];
      if ((key >> (bits + b)) == pfx) atomicAdd(&h[(key >> bits) & ((1u << b) - 1u)], 1u);
    }
    __syncthreads();
    if (b == 10) lds_find_bin<NT, 1024, true>(h, want, scan, &sv[0], &sv[1]);
    else if (b == 9) lds_find_bin<NT, 512, true>(h, want, scan, &sv[0], &sv[1]);
    else lds_find_bin<NT, 256, true>(h, want, scan, &sv[0], &sv[1]);  // b <= 8 here
    const uint32_t bin = sv[0];
    want = sv[1];
    last = h[bin];
    pfx = (pfx << b) | bin;
    __syncthreads();
  }
  *need = want;
  *ties = last;
  return pfx;
}

// The `need`-th smallest index among LDS candidates whose key equals T
// (indices < 2^31 in ci's low bits): radix passes of 11, 10 and 10 bits.
template <int NT>
__device__ uint32_t cand_kth_tie_index(const uint32_t* ck, const uint32_t* ci, uint32_t cnt, uint32_t T,
                                       uint32_t need, uint32_t* h, uint32_t* scan, uint32_t* sv) {
  uint32_t pfx = 0;
  uint32_t want = need;
  int done = 0;  // index bits fixed so far, from bit 30 down
  const int widths[3] = {11, 10, 10};
  for (int pass = 0; pass < 3; ++pass) {
    const int b = widths[pass];
    const int low = 31 - done - b;
    for (uint32_t j = threadIdx.x; j < (1u << b); j += NT) h[j] = 0u;
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < cnt; j += NT) {
      const uint32_t idx = ci[j] & 0x7FFFFFFFu;
      if (ck[j] == T && (idx >> (low + b)) == pfx) atomicAdd(&h[(idx >> low) & ((1u << b) - 1u)], 1u);
    }
    __syncthreads();
    if (b == 11) lds_find_bin<NT, 2048, false>(h, want, scan, &sv[0], &sv[1]);
    else lds_find_bin<NT, 1024, false>(h, want, scan, &sv[0], &sv[1]);
    pfx = (pfx << b) | sv[0];
    want = sv[1];
    done += b;
    __syncthreads();
  }
  return pfx;
}

// The bin of a global 4096-bin histogram (read after a grid barrier, so
// plain loads see every block's counts) holding the k-th largest element,
// scanning from the top bin down; thread t reads bins [4080 - 16t, 4096 -
// 16t) as four 16-byte loads. Outputs the bin, k's rank inside it and the
// bin's count; one block barrier.
template <int NT>
__device__ void find_bin_desc_4096(const uint32_t* hist, uint32_t k, uint32_t* lds, uint32_t* out_bin,
                                   uint32_t* out_krem, uint32_t* out_count) {
  constexpr int PER = 4096 / NT;  // 16 at 256 threads, 4 at 1024
  const uint32_t lo = 4096 - PER * (threadIdx.x + 1);
  uint32_t c[PER];
#pragma unroll
  for (int q = 0; q < PER / 4; ++q) {
    const uint4 v = *reinterpret_cast<const uint4*>(hist + lo + 4 * q);
    c[4 * q] = v.x; c[4 * q + 1] = v.y; c[4 * q + 2] = v.z; c[4 * q + 3] = v.w;
  }
  uint32_t s = 0;
#pragma unroll
  for (int p = 0; p < PER; ++p) s += c[p];
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t inc = wave_inclusive_scan(s);
  if (lane == 63) lds[wave] = inc;
  __syncthreads();
  uint32_t above = inc - s;  // bins above this thread's, within its wave
  for (uint32_t w = 0; w < wave; ++w) above += lds[w];
  if (above < k && k <= above + s) {
    uint32_t run = above;
#pragma unroll
    for (int p = PER - 1; p >= 0; --p) {  // descending bins: highest first
      if (run < k && k <= run + c[p]) {
        *out_bin = lo + p;
        *out_krem = k - run;
        *out_count = c[p];
      }
      run += c[p];
    }
  }
}

// Block-wide sums of K values per thread (two barriers, no atomics). `lds`
// holds K * NT / 64 words.
template <int NT, int K>
__device__ __forceinline__ void block_sums(uint32_t (&v)[K], uint32_t* lds) {
  constexpr int NW = NT / 64;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const uint32_t w = wave_sum_u32(v[k]);
    if ((threadIdx.x & 63) == 0) lds[k * NW + wave] = w;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < K; ++k) {
    uint32_t t = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) t += lds[k * NW + w];
    v[k] = t;
  }
  __syncthreads();
}

// Dilation radius the register path handles: a token's window lies inside
// the 56 gap flags [i0 - 24, i0 + 32) its thread loads.
constexpr int kRegDilation = 24;

template <int ITEMS, int NT>
__global__ __launch_bounds__(NT) void sel_onepass_kernel(const SelArgs a) {
  constexpr uint32_t TILE = NT * ITEMS;
  extern __shared__ uint32_t smem[];
  __shared__ uint32_t scan[NT / 64 + 16];
  __shared__ uint32_t red[4 * NT / 64];
  __shared__ uint32_t sv[4];
  __shared__ uint32_t flag;
  uint32_t* ctrl = a.ws + kCtrl;
  uint32_t bar_round = 0;
  const uint32_t ntiles = gridDim.x;
  const uint32_t tile = blockIdx.x;
  const uint32_t tile0 = tile * TILE;
  const uint32_t i0 = tile0 + threadIdx.x * ITEMS;
  const int r = a.radius;

  // ---------------------------------------------------------------- P1
  uint32_t* hist = smem;          // 4096
  uint32_t* window = smem + 4096;  // TILE + 2r
  // this thread's tokens: scores, gap and forced flags, all loads issued
  // before any is used (vector loads on a full tile)
  float sc[ITEMS];
  uint8_t gp[ITEMS], fc[ITEMS];
  if (a.vec_ok && i0 + ITEMS <= a.n) {
#pragma unroll
    for (int q = 0; q < ITEMS / 4; ++q) {
      const float4 v = *reinterpret_cast<const float4*>(a.scores + i0 + 4 * q);
      sc[4 * q] = v.x; sc[4 * q + 1] = v.y; sc[4 * q + 2] = v.z; sc[4 * q + 3] = v.w;
    }
#pragma unroll
    for (int q = 0; q < ITEMS / 8; ++q) {
      const uint64_t g8 = *reinterpret_cast<const uint64_t*>(a.gap + i0 + 8 * q);
      const uint64_t f8 = a.forced ? *reinterpret_cast<const uint64_t*>(a.forced + i0 + 8 * q) : 0ull;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        gp[8 * q + e] = uint8_t(g8 >> (8 * e));
        fc[8 * q + e] = uint8_t(f8 >> (8 * e));
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < ITEMS; ++e) {
      const uint32_t i = i0 + e;
      const bool in = i < a.n;
      sc[e] = in ? a.scores[i] : 0.f;
      gp[e] = in ? a.gap[i] : 0;
      fc[e] = in && a.forced ? a.forced[i] : 0;
    }
  }
  // dilation: with ITEMS == 8 and r <= kRegDilation each thread loads the
  // 56 gap flags [i0 - 24, i0 + 32) as seven 8-byte words into a bit mask;
  // otherwise the tile's window [tile0 - r, tile0 + TILE + r) becomes a
  // prefix count of gaps in LDS
  const bool reg_dil = ITEMS == 8 && r > 0 && r <= kRegDilation;
  uint64_t gmask = 0;
  if (reg_dil) {
#pragma unroll
    for (int q = 0; q < 7; ++q) {
      const int64_t g0 = int64_t(i0) - 24 + 8 * q;
      uint64_t w8 = 0;
      if (a.vec_ok && g0 >= 0 && g0 + 8 <= int64_t(a.n)) {
        w8 = *reinterpret_cast<const uint64_t*>(a.gap + g0);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int64_t g = g0 + e;
          w8 |= (g >= 0 && g < int64_t(a.n)) ? uint64_t(a.gap[g]) << (8 * e) : 0ull;
        }
      }
      uint64_t bits = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) bits |= ((w8 >> (8 * e)) & 0xFFull) ? (1ull << e) : 0ull;
      gmask |= bits << (8 * q);
    }
  }
#pragma unroll
  for (uint32_t q = 0; q < 4096 / (4 * NT); ++q)
    reinterpret_cast<uint4*>(hist)[threadIdx.x + q * NT] = make_uint4(0u, 0u, 0u, 0u);
  if (r > 0 && !reg_dil) {
    const uint32_t W = TILE + 2 * r;
    for (uint32_t w = threadIdx.x; w < W; w += NT) {
      const int64_t g = int64_t(tile0) - r + w;
      window[w] = (g >= 0 && g < int64_t(a.n) && a.gap[g]) ? 1u : 0u;
    }
    __syncthreads();
    const uint32_t per = (W + NT - 1) / NT;
    const uint32_t beg = threadIdx.x * per;
    const uint32_t end = min(W, beg + per);
    uint32_t local = 0;
    for (uint32_t w = beg; w < end; ++w) {
      local += window[w];
      window[w] = local;
    }
    uint32_t total;
    const uint32_t excl = block_exclusive_scan<NT>(local, scan, &total);
    for (uint32_t w = beg; w < end; ++w) window[w] += excl;
  }
  __syncthreads();
  // keys; base tokens (key of -inf) are counted, not histogrammed: their
  // count joins H1's -inf bin in the merge, which spares the LDS histogram
  // its most crowded bin
  uint32_t key[ITEMS];
  uint32_t base_bits = 0, valid_bits = 0, gap_cnt = 0, base_cnt = 0;
  const uint64_t dil_mask = reg_dil ? ((1ull << (2 * r + 1)) - 1ull) : 0ull;
#pragma unroll
  for (int e = 0; e < ITEMS; ++e) {
    const uint32_t i = i0 + e;
    key[e] = 0u;
    if (i < a.n) {
      const bool g = gp[e] != 0;
      bool b = g || fc[e] != 0;
      if (r > 0 && !b) {
        if (reg_dil) {
          b = (gmask >> (24 + e - r)) & dil_mask;
        } else {
          const uint32_t k = i - tile0 + r;  // window index of token i
          const uint32_t hi = window[k + r];
          const uint32_t lo = (k >= uint32_t(r) + 1) ? window[k - r - 1] : 0u;
          b = hi > lo;
        }
      }
      key[e] = b ? kKeyNegInf : order_key(sc[e]);
      valid_bits |= 1u << e;
      base_bits |= (b ? 1u : 0u) << e;
      gap_cnt += g ? 1u : 0u;
      base_cnt += b ? 1u : 0u;
      if (!b) atomicAdd(&hist[key[e] >> 20], 1u);
    }
  }
  uint32_t counts[2] = {gap_cnt, base_cnt};
  block_sums<NT>(counts, red);
  if (threadIdx.x == 0) {
    if (counts[0]) atomicAdd(&ctrl[C_GAP], counts[0]);
    if (counts[1]) atomicAdd(&ctrl[C_BASE], counts[1]);
    a.tile_base[tile] = counts[1];
  }
  for (uint32_t i = threadIdx.x; i < 4096; i += NT) {
    const uint32_t c = hist[i] + (i == (kKeyNegInf >> 20) ? counts[1] : 0u);
    if (c) atomicAdd(&a.ws[kH1 + i], c);
  }
  if (!grid_barrier(ctrl, ntiles, ++bar_round, a, &flag)) {
    if (threadIdx.x == 0) *a.out_count = -1;
    return;
  }

  // ---------------------------------------------------------------- P2
  // budget: int(cached * ratio) as Python computes it, then [1, available]
  const int64_t gaps = ld_rlx(&ctrl[C_GAP]);
  const int64_t bases = ld_rlx(&ctrl[C_BASE]);
  int64_t topk = 0;
  {
    const int64_t cached = int64_t(a.n) - gaps;
    const int64_t available = int64_t(a.n) - bases;
    if (cached && available) {
      topk = int64_t(double(cached) * a.ratio);
      topk = topk < 1 ? 1 : topk;
      topk = topk > available ? available : topk;
    }
  }
  uint32_t write_bits = base_bits;  // selected tokens of this thread
  uint32_t out_off = 0;
  if (topk == 0) {
    // only base tokens: the earlier tiles' base counts give the offset
    uint32_t before[1] = {0};
    for (uint32_t t = threadIdx.x; t < tile; t += NT) before[0] += a.tile_base[t];
    block_sums<NT>(before, red);
    out_off = before[0];
    if (tile == 0 && threadIdx.x == 0) *a.out_count = bases;
  } else {
    find_bin_desc_4096<NT>(a.ws + kH1, uint32_t(topk), scan, &sv[0], &sv[1], &sv[3]);
    __syncthreads();
    uint32_t prefix = sv[0];
    uint32_t krem = sv[1];
    uint32_t cnt = sv[3];
    int shift = 20;
    bool exact = false;  // the ties path: T fixed by all 32 bits
    if (cnt > kCandCap) {
      // second digit: key[19:8] among keys with key[31:20] == prefix
      __syncthreads();
      for (uint32_t i = threadIdx.x; i < 4096; i += NT) hist[i] = 0u;
      __syncthreads();
#pragma unroll
      for (int e = 0; e < ITEMS; ++e)
        if (((valid_bits >> e) & 1u) && (key[e] >> 20) == prefix) atomicAdd(&hist[(key[e] >> 8) & 0xFFFu], 1u);
      __syncthreads();
      for (uint32_t i = threadIdx.x; i < 4096; i += NT)
        if (hist[i]) atomicAdd(&a.ws[kH2 + i], hist[i]);
      if (!grid_barrier(ctrl, ntiles, ++bar_round, a, &flag)) {
        if (threadIdx.x == 0) *a.out_count = -1;
        return;
      }
      __syncthreads();
      find_bin_desc_4096<NT>(a.ws + kH2, krem, scan, &sv[0], &sv[1], &sv[3]);
      __syncthreads();
      prefix = (prefix << 12) | sv[0];
      krem = sv[1];
      cnt = sv[3];
      shift = 8;
      if (cnt > kCandCap) {
        // last digit: key[7:0] among keys with key[31:8] == prefix
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < 256; i += NT) hist[i] = 0u;
        __syncthreads();
#pragma unroll
        for (int e = 0; e < ITEMS; ++e)
          if (((valid_bits >> e) & 1u) && (key[e] >> 8) == prefix) atomicAdd(&hist[key[e] & 0xFFu], 1u);
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < 256; i += NT)
          if (hist[i]) atomicAdd(&a.ws[kH3 + i], hist[i]);
        if (!grid_barrier(ctrl, ntiles, ++bar_round, a, &flag)) {
          if (threadIdx.x == 0) *a.out_count = -1;
          return;
        }
        find_bin_desc<256, NT>(a.ws + kH3, krem, scan, &sv[0], &sv[1]);
        __syncthreads();
        prefix = (prefix << 8) | sv[0];
        krem = sv[1];
        shift = 0;
        exact = true;
      }
    }
    if (!exact) {
      // -------------------------------------------- candidate path
      uint32_t sure = 0, mine = 0;
#pragma unroll
      for (int e = 0; e < ITEMS; ++e) {
        if (!((valid_bits >> e) & 1u)) continue;
        const uint32_t d = key[e] >> shift;
        sure += (((base_bits >> e) & 1u) || d > prefix) ? 1u : 0u;
        mine += d == prefix ? 1u : 0u;
      }
      // candidate slots: wave scans, a wave offset from an LDS counter, the
      // block's range from one global counter
      const uint32_t lane = threadIdx.x & 63;
      const uint32_t inc = wave_inclusive_scan(mine);
      const uint32_t wave_total = __shfl(inc, 63, 64);
      const uint32_t sure_w = wave_sum_u32(sure);
      if (threadIdx.x == 0) { red[8] = 0; red[9] = 0; }
      __syncthreads();
      uint32_t wave_off = 0;
      if (lane == 63) {
        wave_off = atomicAdd(&red[8], wave_total);
        atomicAdd(&red[9], sure_w);
      }
      wave_off = __shfl(wave_off, 63, 64);
      __syncthreads();
      if (threadIdx.x == 0) {
        a.tile_sure[tile] = red[9];
        sv[2] = red[8] ? atomicAdd(&ctrl[C_CANDS], red[8]) : 0u;
      }
      __syncthreads();
      uint32_t pos = sv[2] + wave_off + inc - mine;
#pragma unroll
      for (int e = 0; e < ITEMS; ++e) {
        if (((valid_bits >> e) & 1u) && (key[e] >> shift) == prefix) {
          a.cand_key[pos] = key[e];
          a.cand_idx[pos] = (i0 + e) | (((base_bits >> e) & 1u) << 31);
          ++pos;
        }
      }
      if (!grid_barrier(ctrl, ntiles, ++bar_round, a, &flag)) {
        if (threadIdx.x == 0) *a.out_count = -1;
        return;
      }
      // ---------------------------------------------------------- P3
      uint32_t* ck = smem;
      uint32_t* ci = smem + kCandCap;
      uint32_t* h = smem + 2 * kCandCap;  // 2048
      // candidates written by every block before the barrier: 16-byte
      // loads, all issued before any is stored (capacity-padded, so a
      // partial last vector stays inside the candidate arrays)
      constexpr uint32_t kVecPerThread = kCandCap / (4 * NT);
      uint4 vk[kVecPerThread], vi[kVecPerThread];
#pragma unroll
      for (uint32_t q = 0; q < kVecPerThread; ++q) {
        const uint32_t j = 4 * (threadIdx.x + q * NT);
        if (j < cnt) {
          vk[q] = *reinterpret_cast<const uint4*>(a.cand_key + j);
          vi[q] = *reinterpret_cast<const uint4*>(a.cand_idx + j);
        }
      }
      // the tiles' sure counts, loaded with the candidates
      uint32_t sure_before = 0, sure_all = 0;
      for (uint32_t t = threadIdx.x; t < ntiles; t += NT) {
        const uint32_t v = a.tile_sure[t];
        sure_all += v;
        sure_before += t < tile ? v : 0u;
      }
#pragma unroll
      for (uint32_t q = 0; q < kVecPerThread; ++q) {
        const uint32_t j = 4 * (threadIdx.x + q * NT);
        if (j < cnt) {
          *reinterpret_cast<uint4*>(ck + j) = vk[q];
          *reinterpret_cast<uint4*>(ci + j) = vi[q];
        }
      }
      __syncthreads();
      // the k-th largest (key desc, index asc) among the candidates: with a
      // 20-bit remainder, one 11-bit LDS pass first; when at most 64
      // candidates then share the prefix, one wave ranks them directly,
      // else radix passes on the remaining key bits, then on the indices
      // of the keys equal to T
      uint32_t pfx = prefix, want = krem, rest = uint32_t(shift), m = cnt;
      if (rest == 20) {
        for (uint32_t j = threadIdx.x; j < 2048; j += NT) h[j] = 0u;
        __syncthreads();
        for (uint32_t j = threadIdx.x; j < cnt; j += NT) atomicAdd(&h[(ck[j] >> 9) & 2047u], 1u);
        __syncthreads();
        lds_find_bin<NT, 2048, true>(h, want, scan, &sv[0], &sv[1]);
        m = h[sv[0]];
        pfx = (pfx << 11) | sv[0];
        want = sv[1];
        rest = 9;
        __syncthreads();
      }
      uint32_t T, cut;
      if (m <= 64) {
        uint32_t* list = h;  // the m candidates sharing the prefix
        if (threadIdx.x == 0) sv[2] = 0;
        __syncthreads();
        for (uint32_t j = threadIdx.x; j < cnt; j += NT) {
          if ((ck[j] >> rest) == pfx) {
            const uint32_t slot = atomicAdd(&sv[2], 1u);
            list[2 * slot] = ck[j];
            list[2 * slot + 1] = ci[j] & 0x7FFFFFFFu;
          }
        }
        __syncthreads();
        if (threadIdx.x < 64) {
          const uint32_t lane = threadIdx.x;
          const bool have = lane < m;
          const uint32_t kk = have ? list[2 * lane] : 0u;
          const uint32_t ii = have ? list[2 * lane + 1] : 0xFFFFFFFFu;
          uint32_t rank = 0;
          for (uint32_t l = 0; l < m; ++l) {
            const uint32_t kl = __shfl(kk, int(l), 64);
            const uint32_t il = __shfl(ii, int(l), 64);
            rank += (kl > kk || (kl == kk && il < ii)) ? 1u : 0u;
          }
          if (have && rank == want - 1) {
            sv[0] = kk;
            sv[1] = ii;
          }
        }
        __syncthreads();
        T = sv[0];
        cut = sv[1];
      } else {
        uint32_t need, ties;
        T = cand_kth_key<NT>(ck, cnt, pfx, int(rest), want, h, scan, sv, &need, &ties);
        cut = need >= ties ? 0x7FFFFFFFu : cand_kth_tie_index<NT>(ck, ci, cnt, T, need, h, scan, sv);
      }
      uint32_t before = 0, taken = 0;
      for (uint32_t j = threadIdx.x; j < cnt; j += NT) {
        const uint32_t idx = ci[j] & 0x7FFFFFFFu;
        const bool sel = ck[j] > T || (ck[j] == T && idx <= cut);
        if (sel && !(ci[j] >> 31)) {
          ++taken;
          before += idx < tile0 ? 1u : 0u;
        }
      }
      uint32_t sums[4] = {taken, before, sure_before, sure_all};
      block_sums<NT>(sums, red);
      out_off = sums[2] + sums[1];
      if (tile == 0 && threadIdx.x == 0) *a.out_count = int64_t(sums[3]) + sums[0];
#pragma unroll
      for (int e = 0; e < ITEMS; ++e) {
        const uint32_t i = i0 + e;
        if ((valid_bits >> e) & 1u) {
          if (key[e] > T || (key[e] == T && i <= cut)) write_bits |= 1u << e;
        }
      }
    } else {
      // ------------------------------------------------ ties path
      const uint32_t T = prefix;
      const uint32_t need = krem;
      uint32_t ties = 0, sure = 0;
#pragma unroll
      for (int e = 0; e < ITEMS; ++e) {
        if (!((valid_bits >> e) & 1u)) continue;
        ties += key[e] == T ? 1u : 0u;
        sure += (((base_bits >> e) & 1u) || key[e] > T) ? 1u : 0u;
      }
      uint32_t tile_ties, tile_sure;
      uint32_t rank = block_exclusive_scan<NT>(ties, scan, &tile_ties);
      block_exclusive_scan<NT>(sure, scan, &tile_sure);
      if (threadIdx.x == 0) a.tile_ties[tile] = tile_ties;
      if (!grid_barrier(ctrl, ntiles, ++bar_round, a, &flag)) {
        if (threadIdx.x == 0) *a.out_count = -1;
        return;
      }
      uint32_t tb = 0;
      for (uint32_t t = threadIdx.x; t < tile; t += NT) tb += ld_rlx(&a.tile_ties[t]);
      uint32_t tie_off;
      block_exclusive_scan<NT>(tb, scan, &tie_off);
      const int64_t left = int64_t(need) - int64_t(tie_off);
      const uint32_t allow = left <= 0 ? 0u : (left < int64_t(tile_ties) ? uint32_t(left) : tile_ties);
      uint32_t count = 0;
#pragma unroll
      for (int e = 0; e < ITEMS; ++e) {
        if (!((valid_bits >> e) & 1u)) continue;
        bool sel = ((base_bits >> e) & 1u) || key[e] > T;
        if (key[e] == T) {
          sel = sel || rank < allow;
          ++rank;
        }
        if (sel) {
          write_bits |= 1u << e;
          ++count;
        }
      }
      uint32_t tile_count;
      block_exclusive_scan<NT>(count, scan, &tile_count);
      if (threadIdx.x == 0) a.tile_cnt[tile] = tile_count;
      if (!grid_barrier(ctrl, ntiles, ++bar_round, a, &flag)) {
        if (threadIdx.x == 0) *a.out_count = -1;
        return;
      }
      uint32_t cb = 0, ca = 0;
      for (uint32_t t = threadIdx.x; t < ntiles; t += NT) {
        const uint32_t v = ld_rlx(&a.tile_cnt[t]);
        ca += v;
        cb += t < tile ? v : 0u;
      }
      uint32_t sb, sa;
      block_exclusive_scan<NT>(cb, scan, &sb);
      block_exclusive_scan<NT>(ca, scan, &sa);
      out_off = sb;
      if (tile == 0 && threadIdx.x == 0) *a.out_count = sa;
    }
  }
  // ------------------------------------------------------------- write
  uint32_t total;
  uint32_t pos = out_off + block_exclusive_scan<NT>(__popc(write_bits), scan, &total);
#pragma unroll
  for (int e = 0; e < ITEMS; ++e) {
    if (((write_bits >> e) & 1u) && pos < a.n) a.out_idx[pos++] = int64_t(i0 + e);
  }
}

__global__ void write_zero_count_kernel(int64_t* out_count) { *out_count = 0; }

int check_select(const float* scores, const uint8_t* gap, int64_t n, int64_t radius, double ratio,
                 int64_t* out_idx, int64_t* out_count, void* ws, size_t ws_bytes, uint32_t flags) {
  CBK_REQUIRE((flags & ~uint32_t(CBK_SELECT_MULTI_LAUNCH | CBK_SELECT_TEST_GIVE_UP)) == 0,
              "unknown select flags 0x%x", unsigned(flags));
  CBK_REQUIRE((flags & CBK_SELECT_MULTI_LAUNCH) == 0 || (flags & CBK_SELECT_TEST_GIVE_UP) == 0,
              "CBK_SELECT_TEST_GIVE_UP needs the one-launch select");
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

constexpr int kNotLaunched = 1;
// Threads per block of the one-launch select at 8 tokens per thread: 4096-
// token tiles, 16 blocks at 64K tokens (38.0 us per K-deviation select
// against 40.0 at 256 threads and 41.0 at 1024, same box): fewer blocks
// shorten the histogram merge's contended adds and the barriers' arrival
// chains, while each thread keeps its 8 tokens (16 tokens per thread, 8192-
// token tiles, measured 40.9 us at 512 threads and 41.3 at 256).
constexpr int kOnepassThreads = 512;

// Blocks of sel_onepass_kernel<ITEMS, NT> with `lds` dynamic LDS bytes that the
// device can hold at once, per device (cached: the occupancy query is a
// runtime call).
template <int ITEMS, int NT>
int onepass_capacity(size_t lds, int* capacity) {
  static std::mutex mu;
  static int cached_dev[16] = {};
  static size_t cached_lds[16] = {};
  static int cached_cap[16] = {};
  static int used = 0;
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return set_error(CBK_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(err));
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i)
    if (cached_dev[i] == dev && cached_lds[i] == lds) {
      *capacity = cached_cap[i];
      return CBK_OK;
    }
  int per_cu = 0, cus = 0, coop = 0;
  err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, sel_onepass_kernel<ITEMS, NT>, NT, lds);
  if (err == hipSuccess) err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (err == hipSuccess) err = hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev);
  if (err != hipSuccess) return set_error(CBK_ERR_LAUNCH, "occupancy query: %s", hipGetErrorString(err));
  *capacity = coop ? per_cu * cus : 0;
  if (used < 16) {
    cached_dev[used] = dev;
    cached_lds[used] = lds;
    cached_cap[used] = *capacity;
    ++used;
  }
  return CBK_OK;
}

// kNotLaunched when the tiles do not fit on the device at once.
template <int ITEMS, int NT>
int launch_onepass(const SelArgs& a, int64_t n, int64_t radius, hipStream_t stream) {
  constexpr int64_t tile = int64_t(NT) * ITEMS;
  const int64_t grid = (n + tile - 1) / tile;
  const int64_t p1 = 4096 + tile + 2 * radius + 1;
  const int64_t p3 = 2 * int64_t(kCandCap) + 2048;
  const size_t lds = size_t(p1 > p3 ? p1 : p3) * sizeof(uint32_t);
  int capacity = 0;
  if (int rc = onepass_capacity<ITEMS, NT>(lds, &capacity)) return rc;
  if (grid > capacity) return kNotLaunched;
  hipLaunchKernelGGL((sel_onepass_kernel<ITEMS, NT>), dim3(uint32_t(grid)), dim3(NT), lds, stream, a);
  return launch_status("select (one launch)");
}

// header_zeroed: an earlier launch on the stream cleared the kHeader counter
// words (the fused K-deviation launch does). flags: CBK_SELECT_* bits.
int launch_select(const float* scores, const uint8_t* gap, const uint8_t* forced, int64_t n,
                  int64_t radius, double ratio, int64_t* out_idx, int64_t* out_count, void* ws,
                  size_t ws_bytes, hipStream_t stream, bool header_zeroed, uint32_t flags) {
  if (int rc = check_select(scores, gap, n, radius, ratio, out_idx, out_count, ws, ws_bytes, flags))
    return rc;
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
  a.tile_base = a.ws + L.tiles;
  a.tile_sure = a.tile_base + (L.cands - L.tiles) / 4;
  a.tile_ties = a.tile_sure + (L.cands - L.tiles) / 4;
  a.tile_cnt = a.tile_ties + (L.cands - L.tiles) / 4;
  a.cand_key = a.ws + L.cands;
  a.cand_idx = a.cand_key + kCandCap;
  a.vec_ok = (reinterpret_cast<uintptr_t>(scores) % 16 == 0 && reinterpret_cast<uintptr_t>(gap) % 8 == 0 &&
              reinterpret_cast<uintptr_t>(forced) % 8 == 0) ? 1u : 0u;
  const bool give_up = (flags & CBK_SELECT_TEST_GIVE_UP) != 0;
  a.spin_limit = give_up ? 0u : kBarrierSpins;
  a.bar_extra = give_up ? 1u : 0u;
  if (!header_zeroed) hipLaunchKernelGGL(sel_zero_kernel, dim3(1), dim3(kSelThreads), 0, stream, a.ws);
  // one launch when every tile's block can be resident at once
  if ((flags & CBK_SELECT_MULTI_LAUNCH) == 0) {
    int rc = launch_onepass<8, kOnepassThreads>(a, n, radius, stream);
    if (rc == kNotLaunched) rc = launch_onepass<32, kSelThreads>(a, n, radius, stream);
    if (rc != kNotLaunched) return rc;
  }
  const dim3 grid(L.nblocks), block(kSelThreads);
  const size_t prep_lds = (4096 + 16 + kSelTile + 2 * size_t(radius) + 1) * sizeof(uint32_t);
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
// device array sized for CBK_NOALLOC_SELECT_MAX_TOKENS tokens (5.11 MiB,
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
    if (device != current) (void)hipSetDevice(current);
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

int cbk_select_ex(const float* scores_dev, const uint8_t* gap_dev, const uint8_t* forced_dev,
                  int64_t n, int64_t radius, double ratio, int64_t* out_idx_dev,
                  int64_t* out_count_dev, void* workspace_dev, size_t workspace_bytes,
                  uint32_t flags, cbk_stream_t stream) {
  cbk::clear_error();
  return cbk::launch_select(scores_dev, gap_dev, forced_dev, n, radius, ratio, out_idx_dev,
                            out_count_dev, workspace_dev, workspace_bytes,
                            static_cast<hipStream_t>(stream), false, flags);
}

int cbk_select(const float* scores_dev, const uint8_t* gap_dev, const uint8_t* forced_dev,
               int64_t n, int64_t radius, double ratio, int64_t* out_idx_dev,
               int64_t* out_count_dev, void* workspace_dev, size_t workspace_bytes,
               cbk_stream_t stream) {
  return cbk_select_ex(scores_dev, gap_dev, forced_dev, n, radius, ratio, out_idx_dev,
                       out_count_dev, workspace_dev, workspace_bytes, 0u, stream);
}

int cbk_kdev_select(const void* fresh_dev, int64_t fresh_row_stride_elems, const void* cached_dev,
                    int64_t cached_row_stride_elems, int64_t cached_num_rows,
                    const int64_t* cached_rows_dev, int64_t cached_row0, int64_t n, int64_t width,
                    int32_t dtype, const uint8_t* gap_dev, const uint8_t* forced_dev,
                    int64_t radius, double ratio, float* scores_dev, int64_t* out_idx_dev,
                    int64_t* out_count_dev, void* workspace_dev, size_t workspace_bytes,
                    cbk_stream_t stream) {
  return cbk_kdev_select_ex(fresh_dev, fresh_row_stride_elems, cached_dev, cached_row_stride_elems,
                            cached_num_rows, cached_rows_dev, cached_row0, n, width, dtype, gap_dev,
                            forced_dev, radius, ratio, scores_dev, out_idx_dev, out_count_dev,
                            workspace_dev, workspace_bytes, 0u, stream);
}

int cbk_kdev_select_ex(const void* fresh_dev, int64_t fresh_row_stride_elems, const void* cached_dev,
                       int64_t cached_row_stride_elems, int64_t cached_num_rows,
                       const int64_t* cached_rows_dev, int64_t cached_row0, int64_t n, int64_t width,
                       int32_t dtype, const uint8_t* gap_dev, const uint8_t* forced_dev,
                       int64_t radius, double ratio, float* scores_dev, int64_t* out_idx_dev,
                       int64_t* out_count_dev, void* workspace_dev, size_t workspace_bytes,
                       uint32_t flags, cbk_stream_t stream) {
  cbk::clear_error();
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (int rc = cbk::check_select(scores_dev, gap_dev, n, radius, ratio, out_idx_dev, out_count_dev,
                                 workspace_dev, workspace_bytes, flags))
    return rc;
  const bool zero = n > 0;  // the score launch clears the selection counters
  if (int rc = cbk::launch_kdev(fresh_dev, fresh_row_stride_elems, cached_dev,
                                cached_row_stride_elems, cached_num_rows, cached_rows_dev,
                                cached_row0, n, width, dtype, scores_dev, s,
                                zero ? static_cast<uint32_t*>(workspace_dev) : nullptr,
                                zero ? cbk::kHeader : 0u))
    return rc;
  return cbk::launch_select(scores_dev, gap_dev, forced_dev, n, radius, ratio, out_idx_dev,
                            out_count_dev, workspace_dev, workspace_bytes, s, zero, flags);
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
