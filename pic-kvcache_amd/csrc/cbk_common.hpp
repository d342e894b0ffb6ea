// Shared helpers of the gfx950 CacheBlend kernels: error reporting, integer
// fast division, vector types and wavefront reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "cacheblend_hip.h"

namespace cbk {

// --------------------------------------------------------------- errors

int set_error(int code, const char* fmt, ...);
void clear_error();

#define CBK_REQUIRE(cond, ...)                                  \
  do {                                                          \
    if (!(cond)) return ::cbk::set_error(CBK_ERR_INVALID, __VA_ARGS__); \
  } while (0)

// Returns CBK_OK, or CBK_ERR_LAUNCH with the HIP error of the last launch.
int launch_status(const char* what);

// ---------------------------------------------------------- fast divide
// Unsigned 32-bit division by a runtime constant d >= 1 (Granlund-Montgomery
// round-up method): q = (umulhi(n, m) + n) >> s, exact for every n < 2^32.
struct FastDiv {
  uint32_t d;
  uint32_t m;
  uint32_t s;

  __host__ static FastDiv make(uint32_t divisor) {
    FastDiv f;
    f.d = divisor;
    uint32_t s = 0;
    while ((uint64_t(1) << s) < divisor) ++s;
    f.s = s;
    f.m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << s) - divisor)) / divisor + 1);
    return f;
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    uint64_t t = __umulhi(n, m);
    return uint32_t((t + n) >> s);
  }
};

// ------------------------------------------------------- vector types

template <int BYTES> struct Vec;
template <> struct Vec<16> { typedef uint32_t T __attribute__((ext_vector_type(4))); };
template <> struct Vec<8> { typedef uint32_t T __attribute__((ext_vector_type(2))); };
template <> struct Vec<4> { typedef uint32_t T; };
template <> struct Vec<2> { typedef uint16_t T; };
template <> struct Vec<1> { typedef uint8_t T; };

// Largest power-of-two access width (<= 16) dividing every value.
__host__ inline int common_vec_bytes(const int64_t* values, int count) {
  int vec = 16;
  for (int i = 0; i < count; ++i) {
    while (vec > 1 && (values[i] % vec) != 0) vec >>= 1;
  }
  return vec;
}

// ------------------------------------------- LDS DMA (global_load_lds)

// Tiles that the DMA below fills sit in LDS unpadded, D / 8 pieces of 16
// bytes per row of D 16-bit elements, piece p of row R at position
// p ^ swz(R): the 16 lanes that read one piece of 16 consecutive rows then
// hit distinct bank groups.
template <int D>
__device__ __forceinline__ uint32_t lds_swizzle(uint32_t row) {
  constexpr uint32_t P = D / 8;
  return (row / (16 / P)) % P;
}

// s_waitcnt vmcnt(n) lgkmcnt(0), expcnt untouched (gfx9 encoding)
#define CBK_WAIT_VM_LGKM0(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (((n) >> 4) << 14))

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}

// A wave-uniform 64-bit value in SGPRs (readfirstlane returns a signed int:
// each half is widened as unsigned).
__device__ __forceinline__ uint64_t uniform64(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(v))));
  const uint32_t hi = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(v >> 32))));
  return uint64_t(lo) | (uint64_t(hi) << 32);
}

// global_load_lds_dword{,x4}: lane l's 4 or 16 bytes at base + off land at
// LDS address lds + l * size (base and lds wave-uniform). The LDS address
// goes through M0, which the asm saves and restores. The compiler's hazard
// checks do not look inside inline asm, so the asm pads for them itself:
// s_nop 4 gives the 5 wait states a VMEM read of an SGPR needs after a VALU
// wrote it (the base and M0 come from v_readfirstlane) and the 1 an M0 write
// needs before an LDS DMA; s_nop 0 separates the DMA from the M0 restore.
#define CBK_LDS_DMA(op)                                                                           \
  "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 4\n\t" op " %1, %2\n\ts_nop 0\n\ts_mov_b32 m0, %0"
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t off, uint32_t lds) {
  uint32_t saved;
  asm volatile(CBK_LDS_DMA("global_load_lds_dwordx4")
               : "=&s"(saved)
               : "v"(off), "s"(uniform64(base)), "s"(__builtin_amdgcn_readfirstlane(int(lds)))
               : "memory");
}
__device__ __forceinline__ void lds_dma4(const void* base, uint32_t off, uint32_t lds) {
  uint32_t saved;
  asm volatile(CBK_LDS_DMA("global_load_lds_dword")
               : "=&s"(saved)
               : "v"(off), "s"(uniform64(base)), "s"(__builtin_amdgcn_readfirstlane(int(lds)))
               : "memory");
}

// ------------------------------------------------------- reductions

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Inclusive prefix sum over the 64 lanes of a wavefront.
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    uint32_t o = __shfl_up(v, off, 64);
    if (lane >= off) v += o;
  }
  return v;
}

// Exclusive block-wide scan for a block of NT threads (NT multiple of 64).
// `lds` needs NT/64 + 1 uint32 slots. Returns the exclusive prefix of `v`
// and writes the block total to *total.
template <int NT>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* lds, uint32_t* total) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t inc = wave_inclusive_scan(v);
  if (lane == 63) lds[wave] = inc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t run = 0;
    for (int w = 0; w < NW; ++w) {
      uint32_t t = lds[w];
      lds[w] = run;
      run += t;
    }
    lds[NW] = run;
  }
  __syncthreads();
  uint32_t result = lds[wave] + inc - v;
  *total = lds[NW];
  __syncthreads();
  return result;
}

// bf16 / f16 / f32 element loads widened to float.
__device__ __forceinline__ float bf16_bits_to_float(uint16_t b) {
  return __uint_as_float(uint32_t(b) << 16);
}

// x rounded to bf16 (nearest even; -inf, +inf and NaN stay what they are),
// as a float, in one instruction: v_cvt_pk_bf16_f32 with 0 for the low half
// leaves the rounded value in the high half and zeros below it, which is the
// float's bit pattern.
__device__ __forceinline__ float bf16_round(float x) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __uint_as_float(__builtin_bit_cast(uint32_t, __builtin_convertvector((f2){0.f, x}, b2)));
}

}  // namespace cbk
