// Shared device/host helpers of the gfx950 MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

#include "vmoe.h"

#define VMOE_CHECK_LAUNCH()                                   \
  do {                                                        \
    if (hipGetLastError() != hipSuccess) return VMOE_ERR_LAUNCH; \
  } while (0)

namespace vmoe {

// Dispatch timing (vmoe_set_launch_timing, for measurement): while a stop
// event is set on the calling host thread, every launch goes through
// hipExtLaunchKernelGGL with the events bound to the dispatch itself; the
// first launch takes the start event, every launch the stop event, so the
// pair spans the kernels of one entry point without the event-record gaps
// around them.
struct LaunchTiming {
  hipEvent_t start;
  hipEvent_t stop;
};
extern thread_local LaunchTiming g_launch_timing;

// gemm.hip: between gemm_pair_begin() and gemm_pair_end(), the calling host
// thread's GEMM launches go out two at a time (those on one stream), each
// pair as one launch of grouped_gemm_pair_kernel with the CUs split between
// the two (dH with dW2, dX with dW1; other pairs launch one after the
// other). gemm_pair_end() launches a GEMM still held alone and returns its
// status.
void gemm_pair_begin();
int gemm_pair_end();

}  // namespace vmoe

#define VMOE_LAUNCH(K, G, B, SH, S, ...)                                                   \
  do {                                                                                     \
    if (::vmoe::g_launch_timing.stop) {                                                    \
      hipExtLaunchKernelGGL(K, G, B, SH, S, ::vmoe::g_launch_timing.start,                 \
                            ::vmoe::g_launch_timing.stop, 0, __VA_ARGS__);                 \
      ::vmoe::g_launch_timing.start = nullptr;                                             \
    } else {                                                                               \
      hipLaunchKernelGGL(K, G, B, SH, S, __VA_ARGS__);                                     \
    }                                                                                      \
  } while (0)

namespace vmoe {

constexpr int kWave = 64;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16 by the gfx950 conversion instruction (v_cvt_pk_bf16_f32, one
// instruction per pair): round to nearest even, denormals kept. For every
// non-NaN input this gives the bits of c10::BFloat16's rounding (checked on
// the device over all 2^32 fp32 patterns); a NaN input gives a quiet NaN
// whose payload may differ from torch's 0x7FC0.
__device__ __forceinline__ float bf16_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

typedef short i16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  // A vector-to-vector bit cast keeps the value in registers (a cast
  // straight to uint32_t can leave a stack temporary behind).
  const i16x2_t h = __builtin_bit_cast(i16x2_t, __builtin_convertvector(v, bf16x2_t));
  return (uint32_t)(uint16_t)h.x | ((uint32_t)(uint16_t)h.y << 16);
}

__device__ __forceinline__ uint32_t f32_to_bf16(float f) { return pack_bf16(f, 0.0f) & 0xFFFFu; }

// Two bf16 halves of a 32-bit word.
__device__ __forceinline__ float lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f32(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// v of the lane a DPP control selects (every lane active; quad_perm 0xB1 /
// 0x4E swap lanes 1 / 2 apart, row_half_mirror 0x141 reverses 8 lanes).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
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

// Routing tiles: vmoe_route counts the expert ids of every tile of
// kRouteTile consecutive assignments. Its workspace starts with those counts,
// expert-major int32 [E][tiles], followed by one bad-id flag per tile;
// vmoe_router_topk_hist writes the same two arrays.
constexpr int kRouteTile = 1024;
__host__ __device__ inline int64_t route_tiles(int64_t A) {
  return (A + kRouteTile - 1) / kRouteTile;
}

// Count columns per routing tile written by vmoe_router_topk_hist for T
// tokens, E experts and top_k k: each top-k workgroup counts S consecutive
// column blocks' worth of kRouteTile / S assignments (kRouteTile / (S k)
// tokens), S the power of two <= 8 that keeps the launch near 256
// workgroups; the counts array is then [E][tiles * S]. 0 where that launch
// does not apply: the grouped top-k kernel's experts (E % 8 == 0, E <= 128)
// and k <= 8 dividing kRouteTile, T > 0, at most 1024 workgroups, and E
// tiles S <= 65536 counts (what one placement workgroup sums).
inline int route_hist_split(int64_t T, int E, int k) {
  if (T <= 0 || E % 8 != 0 || E > 128 || k <= 0 || k > 8 || kRouteTile % k != 0) return 0;
  const int64_t nt = route_tiles(T * k);
  int S = 1;
  while (S < 8 && nt * S * 2 <= 256) S *= 2;
  if (nt * S > 1024 || (int64_t)E * nt * S > 65536) return 0;
  return S;
}

}  // namespace vmoe
