// Shared device/host helpers of the gfx950 MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vmoe.h"

#define VMOE_CHECK_LAUNCH()                                   \
  do {                                                        \
    if (hipGetLastError() != hipSuccess) return VMOE_ERR_LAUNCH; \
  } while (0)

namespace vmoe {

constexpr int kWave = 64;

// bf16 <-> fp32 with the rounding of c10::BFloat16 (round to nearest even,
// NaN -> 0x7FC0), so a bf16 value produced here has the bits torch produces
// for the same fp32 value.
__device__ __forceinline__ float bf16_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if (f != f) return 0x7FC0u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

// Two bf16 halves of a 32-bit word.
__device__ __forceinline__ float lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f32(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
}

// Count of set bits of `mask` in lanes below the calling lane.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
}

__device__ __forceinline__ uint64_t ballot64(bool p) { return __ballot(p); }

// Inclusive scan across a 64-lane wave.
template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    T o = __shfl_up(v, off, kWave);
    if (lane >= off) v += o;
  }
  return v;
}

// Exclusive scan across the whole block (blockDim.x = NT, NT % 64 == 0).
// `smem` holds NT/64 + 1 values. Returns the exclusive prefix; *total gets
// the block sum. Contains two __syncthreads().
template <typename T, int NT>
__device__ __forceinline__ T block_exclusive_scan(T v, T* smem, T* total) {
  constexpr int NW = NT / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  T inc = wave_inclusive_scan(v);
  if (lane == kWave - 1) smem[wave] = inc;
  __syncthreads();
  if (wave == 0) {
    T s = lane < NW ? smem[lane] : T(0);
    T si = wave_inclusive_scan(s);
    if (lane < NW) smem[lane] = si - s;
    if (lane == NW - 1) smem[NW] = si;
  }
  __syncthreads();
  T excl = smem[wave] + inc - v;
  *total = smem[NW];
  return excl;
}

}  // namespace vmoe
