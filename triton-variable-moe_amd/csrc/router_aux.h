// The router's auxiliary-loss reduction as the device code of one 1024-thread
// workgroup. router_aux_kernel (router.hip) runs it as a launch of its own;
// route_small_kernel (route.hip) runs it in one extra workgroup beside the
// routing placement when the MoE layer asks for it, so the layer's forward
// has one launch fewer. Both run the same code with the same thread mapping,
// so the losses carry the same bits either way.
#pragma once

#include "vmoe_common.h"

namespace vmoe {

constexpr int kAuxThreads = 1024;
constexpr int kAuxWaves = kAuxThreads / kWave;

// Element type of the logits, the routing weights and the logit gradients:
// bf16 bit patterns (F32 = false, the module in bf16) or fp32 (the module in
// fp32). torch evaluates logsumexp and its square in the logits' dtype, so
// for bf16 each is rounded to bf16 once; for fp32 they stay fp32.
template <bool F32>
struct RtElt;
template <>
struct RtElt<false> {
  using T = uint16_t;
  __device__ static float ld(const T* p) { return bf16_to_f32(*p); }
  __device__ static T cvt(float v) { return (T)f32_to_bf16(v); }
  __device__ static float rnd(float v) { return bf16_to_f32(f32_to_bf16(v)); }
};
template <>
struct RtElt<true> {
  using T = float;
  __device__ static float ld(const T* p) { return *p; }
  __device__ static T cvt(float v) { return v; }
  __device__ static float rnd(float v) { return v; }
};

// Sums the top-k launch's per-workgroup partial rows ([nblk][E + 1]: the
// probability sums per expert, then the squared-logsumexp sum) in a fixed
// order and forms the losses of the reference (moe.py:253-303):
//   f_i = bf16(tpe / sum(tpe)), p_i = column / T, z_out = bf16(z column / T),
//   out_scalars[0] = sum_e coef_e f_e p_e (load balance),
//   out_scalars[1] = sum_e wn_e p_e (compute loss).
// Columns go 64 at a time (one per lane); wave w adds rows w, w + 16, ...
// with 8 independent loads in flight, then the 16 wave sums are added in
// wave order. `tokens_per_expert` may point to global memory or to LDS.
// Every thread of the (kAuxThreads-thread) workgroup must call it.
template <bool F32>
__device__ __forceinline__ void router_aux_block(
    const float* __restrict__ partial, int nblk, int64_t T, int E,
    const int32_t* tokens_per_expert, const float* __restrict__ coef,
    const float* __restrict__ wn, typename RtElt<F32>::T* __restrict__ f_i,
    float* __restrict__ f_i32, float* __restrict__ p_i, typename RtElt<F32>::T* __restrict__ z_out,
    float* __restrict__ out_scalars) {
  __shared__ float wsum[kAuxWaves][kWave];
  __shared__ long long sh_cnt[kAuxWaves];
  __shared__ float sh_z;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
  // total routed assignments
  long long cnt = 0;
  for (int e = tid; e < E; e += kAuxThreads) cnt += tokens_per_expert[e];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) cnt += __shfl_xor(cnt, off, kWave);
  if (lane == 0) sh_cnt[wv] = cnt;
  __syncthreads();
  long long total_i = 0;
#pragma unroll
  for (int w = 0; w < kAuxWaves; ++w) total_i += sh_cnt[w];
  const float total = (float)total_i;
  const float invT = T > 0 ? 1.0f / (float)T : 0.0f;
  float lb = 0.0f, cl = 0.0f;
  for (int c0 = 0; c0 <= E; c0 += kWave) {
    const int c = c0 + lane;
    float s = 0.0f;
    if (c <= E) {
      float acc[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
      int b = wv;
      for (; b + 7 * kAuxWaves < nblk; b += 8 * kAuxWaves) {
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += partial[(int64_t)(b + i * kAuxWaves) * (E + 1) + c];
      }
      for (int i = 0; b < nblk; b += kAuxWaves, ++i) acc[i] += partial[(int64_t)b * (E + 1) + c];
#pragma unroll
      for (int i = 0; i < 8; ++i) s += acc[i];
    }
    wsum[wv][lane] = s;
    __syncthreads();
    if (wv == 0 && c <= E) {
      float col = 0.0f;
#pragma unroll
      for (int w = 0; w < kAuxWaves; ++w) col += wsum[w][lane];
      if (c == E) {
        sh_z = col;
      } else {
        const float pe = col * invT;
        // f_i = (tpe.float() / tpe.sum()).to(dtype); 0 when nothing was routed
        const float fe =
            total_i > 0 ? RtElt<F32>::rnd((float)tokens_per_expert[c] / total) : 0.0f;
        f_i[c] = RtElt<F32>::cvt(fe);
        f_i32[c] = fe;
        p_i[c] = pe;
        lb += coef[c] * fe * pe;
        cl += wn[c] * pe;
      }
    }
    __syncthreads();
  }
  if (wv == 0) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      lb += __shfl_xor(lb, off, kWave);
      cl += __shfl_xor(cl, off, kWave);
    }
    if (lane == 0) {
      *z_out = RtElt<F32>::cvt(sh_z * invT);
      out_scalars[0] = lb;
      out_scalars[1] = cl;
    }
  }
}

// Operands of the auxiliary losses for route_small_kernel's extra workgroup
// (the bf16 layer path, vmoe_moe_forward); partial == nullptr: no losses.
struct RouteAux {
  const float* partial;  // [nblk][E + 1] of the top-k launch
  int nblk;
  int64_t T;
  const float* coef;
  const float* wn;
  uint16_t* f_i;
  float* f_i32;
  float* p_i;
  uint16_t* z;
  float* losses;
};

// vmoe_route_counted (route.hip) with the losses above folded into the
// routing launch where the E <= 64 placement kernel runs: then *aux_done is
// set and the caller skips its router_aux launch; otherwise *aux_done is
// left false and nothing of `aux` is touched.
int route_counted_aux(const void* sel, int32_t is64, int64_t A, int32_t E, int32_t top_k,
                      int32_t block, int32_t rounding, int32_t* bin_ids, int32_t* indices,
                      int32_t* tpe, int32_t* bins, int32_t* padded_bins, int32_t* row_src,
                      int32_t* gather_map, int32_t gather_map_pad, int64_t row_capacity,
                      int32_t* assignment_row, int32_t* info, int32_t* expert_offsets,
                      int32_t* padded_counts, const uint16_t* weights, float* row_weight,
                      void* workspace, size_t ws_bytes, vmoe_stream_t stream,
                      const RouteAux* aux, bool* aux_done);

}  // namespace vmoe
