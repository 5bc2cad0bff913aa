// Router front end on gfx950: sigmoid, top-k, weight normalisation and the
// auxiliary-loss reductions of TritonMoEMLP.forward, plus the gradient of
// the auxiliary losses with respect to the router logits.
//
// Semantics (triton_moe/moe.py:166-182, 253-303 of the reference):
//   p[t, e]   = sigmoid(float(L[t, e]))                    L = router logits (bf16)
//   (v, s)    = topk(p[t], k) in torch.topk's order on ROCm, ties included
//               (torch_topk_order below)
//   w[t, j]   = bf16(v_j / (sum_j v_j + 1e-20))  (norm) or bf16(v_j), the sum
//               in the order of torch's row reduction (torch_row_sum)
//   z_loss    = bf16(mean_t bf16(bf16(logsumexp_e L[t, e])^2))
//   p_i[e]    = mean_t p[t, e]
//   f_i[e]    = bf16(tokens_per_expert[e] / sum tokens_per_expert)
//   lb_loss   = sum_e coef[e] * f_i[e] * p_i[e]   (coef folds the reference's
//               uniform / ungrouped / grouped formulas, moe.py:276-303)
//   cl_loss   = sum_e wn[e] * p_i[e]  (= mean_t p[t] . wn, moe.py:266-268)
// Gradients (the weights w get none, as in the reference, scatter.py:176):
//   dL[t, e] = g_z * 2 lse_t softmax(L[t])[e] / T
//            + (g_lb coef[e] f_i[e] + g_cl wn[e]) / T * p (1 - p)
//
// One wave per token: lane l holds experts l, l + 64, ... (VPL of them), so
// the top-k is k rounds of a wave-wide arg-max over 64-bit keys
// (value bits << 32 | ~expert), and the per-expert column sums of p stay in
// registers until a fixed-order block reduction writes one partial row per
// workgroup. The final sums run over those rows in a fixed order, so every
// result is the same from run to run.

#include <algorithm>

#include "router_aux.h"
#include "vmoe_common.h"

namespace vmoe {
namespace {

constexpr int kRtThreads = 256;   // aux backward
constexpr int kRtWaves = kRtThreads / kWave;

// Top-k workgroup: 16 waves (many tokens in flight per CU) while a lane's
// experts fit in the 128 registers that leaves a wave; 4 waves beyond.
__host__ __device__ constexpr int topk_threads(int vpl) { return vpl <= 8 ? 1024 : 256; }
constexpr int kRtMaxExperts = 2048;
constexpr int kRtMaxBlocks = 1024;

// Tokens whose logits a wave loads together before working on them (their
// loads are in flight at once).
template <int VPL>
struct TokBatch {
  static constexpr int value = VPL >= 4 ? 1 : 2;
};

// Wave-wide reductions on DPP moves (no LDS round trip): xor 1 and xor 2
// inside quads, the half-row and row mirrors, then row broadcasts 15 and 31
// leave the full result in lane 63, which is read back for every lane.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp(uint32_t old, uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)x, CTRL, ROW_MASK, 0xF, false);
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;
constexpr int kDppBcast15 = 0x142;
constexpr int kDppBcast31 = 0x143;

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint64_t max_step_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  const uint64_t o = ((uint64_t)dpp<CTRL, ROW_MASK>(hi, hi) << 32) | dpp<CTRL, ROW_MASK>(lo, lo);
  return o > v ? o : v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = max_step_u64<kDppXor1>(v);
  v = max_step_u64<kDppXor2>(v);
  v = max_step_u64<kDppHalfMirror>(v);
  v = max_step_u64<kDppMirror>(v);
  v = max_step_u64<kDppBcast15, 0xA>(v);
  v = max_step_u64<kDppBcast31, 0xC>(v);
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, 63);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float fdpp(float v) {
  return __uint_as_float(dpp<CTRL, ROW_MASK>(__float_as_uint(v), __float_as_uint(v)));
}

__device__ __forceinline__ float wave_sum_f32(float v) {
  v += fdpp<kDppXor1>(v);
  v += fdpp<kDppXor2>(v);
  v += fdpp<kDppHalfMirror>(v);
  v += fdpp<kDppMirror>(v);
  // rows outside the mask keep their value and add 0
  v += __uint_as_float(dpp<kDppBcast15, 0xA>(0u, __float_as_uint(v)));
  v += __uint_as_float(dpp<kDppBcast31, 0xC>(0u, __float_as_uint(v)));
  return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 63));
}

__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, fdpp<kDppXor1>(v));
  v = fmaxf(v, fdpp<kDppXor2>(v));
  v = fmaxf(v, fdpp<kDppHalfMirror>(v));
  v = fmaxf(v, fdpp<kDppMirror>(v));
  v = fmaxf(v, fdpp<kDppBcast15, 0xA>(v));
  v = fmaxf(v, fdpp<kDppBcast31, 0xC>(v));
  return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 63));
}

// sigmoid as torch evaluates it for fp32 (1 / (1 + exp(-x)), precise exp).
__device__ __forceinline__ float sigmoidf(float x) { return 1.0f / (1.0f + expf(-x)); }


// ---- torch.topk's output order and torch.sum's order, for one token ----
//
// The reference takes torch.topk(sigmoid(L.float()), k) (moe.py:168-170).
// On ROCm (PyTorch 2.x, aten/src/ATen/native/cuda/TensorTopK.cu, Sort.cu,
// SortUtils.cuh) a row of up to a few thousand values goes through the
// single-block selection, which writes the values above the k-th largest in
// ascending index order and then the values equal to it, also by ascending
// index, until k are written; for 1 < k <= 32 an in-place 32-slot bitonic
// sort (descending, slots past k marked unused and sorted to the end) then
// orders them, and for k > 32 a stable radix sort does. The bitonic sort is
// not stable: equal values come out in the order its network leaves them,
// so that network is replayed here. Slots >= N (N = 8, 16 or 32, the
// smallest >= k) hold no entry through the whole network and a slot below N
// never swaps with one above, so N slots replay it exactly: the sizes 2 .. N
// with direction bit (pos & size), then one descending merge pass over the N
// slots for each wider size up to 32. An unused slot is key -1, below every
// probability's bits (p >= 0); such slots are interchangeable.
//
// Input: pb / ex hold the k largest values (float bits) and their expert
// indices in the selection order of this file's kernels (value descending,
// equal values by ascending index); entries at j >= k are ignored. Output:
// the same k entries in torch.topk's order.
__device__ __forceinline__ void cx_select(uint32_t& ka, int32_t& va, uint32_t& kb, int32_t& vb,
                                          bool swap) {
  const uint32_t k0 = ka, k1 = kb;
  const int32_t v0 = va, v1 = vb;
  ka = swap ? k1 : k0;
  kb = swap ? k0 : k1;
  va = swap ? v1 : v0;
  vb = swap ? v0 : v1;
}

template <int N>
__device__ __forceinline__ void torch_topk_order(uint32_t (&pb)[N], int32_t (&ex)[N], int k) {
  static_assert(N == 8 || N == 16 || N == 32, "N slots");
  uint32_t kth = pb[0];
#pragma unroll
  for (int j = 1; j < N; ++j)
    if (j == k - 1) kth = pb[j];
  // Selection order: ascending (value == kth, index); the index (< 65536)
  // stays in the low bits of the sort key, the value bits ride along.
  uint32_t ck[N];
#pragma unroll
  for (int j = 0; j < N; ++j)
    ck[j] = j < k ? ((pb[j] == kth ? 1u << 16 : 0u) | (uint32_t)ex[j]) : 0xFFFFFFFFu;
#pragma unroll
  for (int size = 2; size <= N; size *= 2)
#pragma unroll
    for (int stride = size / 2; stride > 0; stride /= 2)
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int l = i ^ stride;
        if (l > i) {
          const bool up = (i & size) == 0;
          const bool swap = up ? ck[i] > ck[l] : ck[i] < ck[l];
          const uint32_t c0 = ck[i], c1 = ck[l], p0 = pb[i], p1 = pb[l];
          ck[i] = swap ? c1 : c0;
          ck[l] = swap ? c0 : c1;
          pb[i] = swap ? p1 : p0;
          pb[l] = swap ? p0 : p1;
        }
      }
  // torch's network: swap when (key_a > key_b) == dir, keys signed.
  uint32_t key[N];
#pragma unroll
  for (int j = 0; j < N; ++j) {
    key[j] = j < k ? pb[j] : 0xFFFFFFFFu;  // -1 as int32
    ex[j] = (int32_t)(ck[j] & 0xFFFFu);
  }
#pragma unroll
  for (int size = 2; size <= 32; size *= 2) {
    // sizes above N: one descending pass with strides N / 2 .. 1
    const int smax = size <= N ? size / 2 : N / 2;
#pragma unroll
    for (int stride = smax; stride > 0; stride /= 2)
#pragma unroll
      for (int t = 0; t < N / 2; ++t) {
        const int pos = 2 * t - (t & (stride - 1));
        const bool dir = size <= N && (pos & size) != 0;
        const bool gt = (int32_t)key[pos] > (int32_t)key[pos + stride];
        cx_select(key[pos], ex[pos], key[pos + stride], ex[pos + stride], gt == dir);
      }
  }
#pragma unroll
  for (int j = 0; j < N; ++j) pb[j] = key[j];
}

// sum(dim=-1) of the k values as torch's reduction kernel orders it for a
// contiguous row of k: block width bw = the largest power of two <= k
// (k <= 64, the wave size), thread x adds x, x + bw (from 0), then the
// threads are combined by shfl_down with offsets 1, 2, .., bw / 2. Values
// at j >= k count as 0 (adding +0 to a non-negative sum is exact).
template <int BW, int N>
__device__ __forceinline__ float torch_tree_sum(const float (&v)[N]) {
  float acc[BW];
#pragma unroll
  for (int x = 0; x < BW; ++x) {
    acc[x] = v[x];
#pragma unroll
    for (int m = x + BW; m < N; m += BW) acc[x] += v[m];
  }
#pragma unroll
  for (int off = 1; off < BW; off *= 2)
#pragma unroll
    for (int x = 0; x < BW; x += 2 * off) acc[x] += acc[x + off];
  return acc[0];
}

template <int N>
__device__ __forceinline__ float torch_row_sum(const uint32_t (&pb)[N], int k) {
  float v[N];
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = j < k ? __uint_as_float(pb[j]) : 0.0f;
  if (k >= 32) return torch_tree_sum<(N < 32 ? N : 32), N>(v);
  if (k >= 16) return torch_tree_sum<(N < 16 ? N : 16), N>(v);
  if (k >= 8) return torch_tree_sum<8, N>(v);
  if (k >= 4) return torch_tree_sum<4, N>(v);
  if (k >= 2) return torch_tree_sum<2, N>(v);
  return v[0];
}

// Lane j < k holds the j-th selected entry (selection order); afterwards it
// holds torch.topk's j-th entry. Every lane replays the network on copies.
template <int N>
__device__ __forceinline__ void topk_order_lanes(float& my_v, int& my_e, int k, int lane) {
  uint32_t pb[N];
  int32_t ex[N];
#pragma unroll
  for (int j = 0; j < N; ++j) {
    pb[j] = __builtin_amdgcn_readlane(__float_as_uint(my_v), j);
    ex[j] = __builtin_amdgcn_readlane(my_e, j);
  }
  torch_topk_order<N>(pb, ex, k);
#pragma unroll
  for (int j = 0; j < N; ++j)
    if (lane == j) {
      my_v = __uint_as_float(pb[j]);
      my_e = ex[j];
    }
}

// Block b handles tokens [b * per, min(T, (b + 1) * per)); its waves take
// batches of TB consecutive tokens in turn. partial[b][e] = sum of p[t][e]
// over the block's tokens (e < E); partial[b][E] = sum of bf16(bf16(lse_t)^2).
template <int VPL, bool F32>
__global__ __launch_bounds__(topk_threads(VPL)) void router_topk_kernel(
    const typename RtElt<F32>::T* __restrict__ logits, int64_t ldl, int64_t T, int E, int k,
    int norm, typename RtElt<F32>::T* __restrict__ weights, int32_t* __restrict__ selected32,
    int64_t* __restrict__ selected64, float* __restrict__ probs, float* __restrict__ lse_out,
    float* __restrict__ partial, int64_t per) {
  constexpr int TB = TokBatch<VPL>::value;
  constexpr int NW = topk_threads(VPL) / kWave;
  extern __shared__ float red[];  // [NW][E + 1]
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
  float col[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) col[v] = 0.0f;
  float zsum = 0.0f;
  const int64_t t_beg = (int64_t)blockIdx.x * per, t_end = min(T, t_beg + per);
  for (int64_t tb = t_beg + (int64_t)wv * TB; tb < t_end; tb += (int64_t)NW * TB) {
    float lgb[TB][VPL];
#pragma unroll
    for (int u = 0; u < TB; ++u)
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const int e = lane + v * kWave;
        lgb[u][v] = (tb + u < t_end && e < E) ? RtElt<F32>::ld(logits + (tb + u) * ldl + e)
                                               : -INFINITY;
      }
#pragma unroll
    for (int u = 0; u < TB; ++u) {
      const int64_t t = tb + u;
      if (t >= t_end) break;
      float p[VPL];
      float m = -INFINITY;
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const int e = lane + v * kWave;
        m = fmaxf(m, lgb[u][v]);
        p[v] = e < E ? sigmoidf(lgb[u][v]) : 0.0f;
        col[v] += p[v];
        if (probs && e < E) probs[t * E + e] = p[v];
      }
      // logsumexp in fp32, rounded to bf16 as torch.logsumexp on bf16 logits.
      m = wave_max_f32(m);
      float se = 0.0f;
#pragma unroll
      for (int v = 0; v < VPL; ++v)
        if (lane + v * kWave < E) se += expf(lgb[u][v] - m);
      se = wave_sum_f32(se);
      const float lse = RtElt<F32>::rnd(logf(se) + m);
      if (lse_out && lane == 0) lse_out[t] = lse;
      zsum += RtElt<F32>::rnd(lse * lse);
      // top-k: k rounds of a wave arg-max; keys order by value, then by the
      // lower expert index. p >= 0, so its bits order like its value.
      uint32_t taken = 0;
      float my_v = 0.0f;
      int my_e = 0;
      for (int j = 0; j < k; ++j) {
        uint64_t best = 0;
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
          const int e = lane + v * kWave;
          if (e < E && !((taken >> v) & 1u)) {
            const uint64_t key = ((uint64_t)__float_as_uint(p[v]) << 32) | (uint32_t)(~e);
            best = key > best ? key : best;
          }
        }
        best = wave_max_u64(best);
        const int e_sel = (int)(~(uint32_t)best);
        const float v_sel = __uint_as_float((uint32_t)(best >> 32));
        if ((e_sel & (kWave - 1)) == lane) taken |= 1u << (e_sel / kWave);
        if (lane == j) {
          my_v = v_sel;
          my_e = e_sel;
        }
      }
      // sum in torch's order: lane x < bw adds lanes x and x + bw, then
      // shfl_down steps 1 .. bw / 2 (lane 0 ends with the total)
      int bw = 1;
      while (2 * bw <= k) bw *= 2;
      float part = lane < k ? my_v : 0.0f;
      const float upper = __shfl(part, (lane + bw) & (kWave - 1), kWave);
      if (lane + bw < k) part += upper;
      for (int off = 1; off < bw; off *= 2) part += __shfl_down(part, off, kWave);
      const float vsum = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(part), 0));
      if (k <= 8) {
        topk_order_lanes<8>(my_v, my_e, k, lane);
      } else if (k <= 16) {
        topk_order_lanes<16>(my_v, my_e, k, lane);
      } else if (k <= 32) {
        topk_order_lanes<32>(my_v, my_e, k, lane);
      }  // k > 32: a stable sort, the selection order
      if (lane < k) {
        const float wv_ = norm ? my_v / (vsum + 1e-20f) : my_v;
        weights[t * k + lane] = RtElt<F32>::cvt(wv_);
        if (selected32) selected32[t * k + lane] = my_e;
        if (selected64) selected64[t * k + lane] = my_e;
      }
    }
  }
  // Block partials: fixed order over waves.
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int e = lane + v * kWave;
    if (e < E) red[wv * (E + 1) + e] = col[v];
  }
  if (lane == 0) red[wv * (E + 1) + E] = zsum;
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += NW * kWave) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) s += red[w * (E + 1) + e];
    partial[(int64_t)blockIdx.x * (E + 1) + e] = s;
  }
}

// Top-k with G lanes per token, 8 experts per lane (E % 8 == 0, E <= 8 G,
// k <= 8): lane (s, r) of a wave holds experts 8r .. 8r + 7 of token slot s
// (one 16-byte load), so a wave works on 64 / G tokens at once instead of
// one. Each lane sorts its 8 keys with a 19-comparator network, then log2 G
// butterfly steps merge the sorted lists of partner lanes (the larger of
// A[j] and B[7 - j] is a bitonic sequence holding the top 8 of A and B; three
// half-cleaner stages sort it), after which every lane of the group holds the
// token's top 8, in the selection order, which torch_topk_order turns into
// torch.topk's. Keys, sigmoid, weights and output order are those of
// router_topk_kernel; logsumexp and the column sums reduce in a different
// fixed order.
constexpr int kGrpMaxExperts = 128;
constexpr int kGrpThreads = 1024;
constexpr int kGrpWaves = kGrpThreads / kWave;

__device__ __forceinline__ void cs_desc(uint64_t& a, uint64_t& b) {
  const uint64_t hi = a > b ? a : b, lo = a > b ? b : a;
  a = hi;
  b = lo;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, kWave);
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, kWave);
  return ((uint64_t)hi << 32) | lo;
}

template <int G, bool F32>
__global__ __launch_bounds__(kGrpThreads) void router_topk_group_kernel(
    const typename RtElt<F32>::T* __restrict__ logits, int64_t ldl, int64_t T, int E, int k,
    int norm, typename RtElt<F32>::T* __restrict__ weights, int32_t* __restrict__ selected32,
    int64_t* __restrict__ selected64, float* __restrict__ probs, float* __restrict__ lse_out,
    float* __restrict__ partial, int64_t per, int32_t* __restrict__ hist_counts,
    int32_t* __restrict__ hist_bad, int hist_cols) {
  constexpr int TPW = kWave / G;  // tokens per wave and batch
  __shared__ float red[kGrpWaves][kGrpMaxExperts + 1];
  // With hist_counts, the workgroup's per * k assignments are count column
  // blockIdx.x of the routing (kRouteTile / (per * k) columns per tile): its
  // expert histogram for vmoe_route_counted.
  __shared__ int32_t thist[kGrpMaxExperts];
  if (hist_counts) {
    for (int e = threadIdx.x; e < E; e += kGrpThreads) thist[e] = 0;
    __syncthreads();
  }
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
  const int r = lane & (G - 1), slot = lane / G;
  const int e0 = 8 * r;
  const bool part_ok = e0 < E;
  float col[8];
#pragma unroll
  for (int v = 0; v < 8; ++v) col[v] = 0.0f;
  float zsum = 0.0f;
  const int64_t t_beg = (int64_t)blockIdx.x * per, t_end = min(T, t_beg + per);
  for (int64_t tb = t_beg + (int64_t)wv * TPW; tb < t_end; tb += (int64_t)kGrpWaves * TPW) {
    const int64_t t = tb + slot;
    const bool ok = t < t_end && part_ok;
    float x[8];
    if (ok) {
      if constexpr (F32) {
        const float4 a = *reinterpret_cast<const float4*>(logits + t * ldl + e0);
        const float4 b = *reinterpret_cast<const float4*>(logits + t * ldl + e0 + 4);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
      } else {
        const uint4 raw = *reinterpret_cast<const uint4*>(logits + t * ldl + e0);
        const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          x[2 * v] = __uint_as_float(w4[v] << 16);
          x[2 * v + 1] = __uint_as_float(w4[v] & 0xFFFF0000u);
        }
      }
    } else {
#pragma unroll
      for (int v = 0; v < 8; ++v) x[v] = -INFINITY;
    }
    float p[8];
    float m = -INFINITY;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      m = fmaxf(m, x[v]);
      p[v] = ok ? sigmoidf(x[v]) : 0.0f;
      col[v] += p[v];
    }
    if (probs && ok) {
      float4* dst = reinterpret_cast<float4*>(probs + t * E + e0);
      dst[0] = make_float4(p[0], p[1], p[2], p[3]);
      dst[1] = make_float4(p[4], p[5], p[6], p[7]);
    }
    // logsumexp in fp32 over the group, rounded to bf16 as torch.logsumexp
    // on bf16 logits.
#pragma unroll
    for (int st = 1; st < G; st <<= 1) m = fmaxf(m, __shfl_xor(m, st, kWave));
    float se = 0.0f;
    if (ok) {
#pragma unroll
      for (int v = 0; v < 8; ++v) se += expf(x[v] - m);
    }
#pragma unroll
    for (int st = 1; st < G; st <<= 1) se += __shfl_xor(se, st, kWave);
    const float lse = RtElt<F32>::rnd(logf(se) + m);
    const bool tok = t < t_end;
    if (tok && r == 0) {
      if (lse_out) lse_out[t] = lse;
      zsum += RtElt<F32>::rnd(lse * lse);
    }
    // keys: value bits, then the lower expert index (p >= 0 orders like its
    // bits); 0 for no expert, below every real key.
    uint64_t key[8];
#pragma unroll
    for (int v = 0; v < 8; ++v)
      key[v] = ok ? ((uint64_t)__float_as_uint(p[v]) << 32) | (uint32_t)(~(e0 + v)) : 0ull;
    cs_desc(key[0], key[1]); cs_desc(key[2], key[3]); cs_desc(key[4], key[5]); cs_desc(key[6], key[7]);
    cs_desc(key[0], key[2]); cs_desc(key[1], key[3]); cs_desc(key[4], key[6]); cs_desc(key[5], key[7]);
    cs_desc(key[1], key[2]); cs_desc(key[5], key[6]);
    cs_desc(key[0], key[4]); cs_desc(key[1], key[5]); cs_desc(key[2], key[6]); cs_desc(key[3], key[7]);
    cs_desc(key[2], key[4]); cs_desc(key[3], key[5]);
    cs_desc(key[1], key[2]); cs_desc(key[3], key[4]); cs_desc(key[5], key[6]);
#pragma unroll
    for (int st = 1; st < G; st <<= 1) {
      uint64_t b[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) b[j] = shfl_xor_u64(key[j], st);
#pragma unroll
      for (int j = 0; j < 8; ++j) key[j] = key[j] > b[7 - j] ? key[j] : b[7 - j];
#pragma unroll
      for (int d = 4; d >= 1; d >>= 1)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if ((j & d) == 0) cs_desc(key[j], key[j + d]);
    }
    if (tok) {
      uint32_t pb[8];
      int32_t ex[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        pb[j] = (uint32_t)(key[j] >> 32);
        ex[j] = (int32_t)(~(uint32_t)key[j]);
      }
      const float vsum = torch_row_sum<8>(pb, k);
      torch_topk_order<8>(pb, ex, k);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j < k && (j & (G - 1)) == r) {
          const float v = __uint_as_float(pb[j]);
          weights[t * k + j] = RtElt<F32>::cvt(norm ? v / (vsum + 1e-20f) : v);
          if (selected32) selected32[t * k + j] = ex[j];
          if (selected64) selected64[t * k + j] = ex[j];
          if (hist_counts) atomicAdd(&thist[ex[j]], 1);
        }
      }
    }
  }
  // Column sums: lanes with the same r hold the same experts; add over the
  // token slots, then one partial row per workgroup in wave order.
#pragma unroll
  for (int st = G; st < kWave; st <<= 1)
#pragma unroll
    for (int v = 0; v < 8; ++v) col[v] += __shfl_xor(col[v], st, kWave);
  if (slot == 0 && part_ok) {
#pragma unroll
    for (int v = 0; v < 8; ++v) red[wv][e0 + v] = col[v];
  }
  zsum = wave_sum_f32(zsum);
  if (lane == 0) red[wv][E] = zsum;
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += kGrpThreads) {
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < kGrpWaves; ++w) sum += red[w][e];
    partial[(int64_t)blockIdx.x * (E + 1) + e] = sum;
  }
  if (hist_counts) {
    // Every written id is a real expert (E >= 8 >= k keys beat the empty
    // ones), so the tile's bad-id flag is 0.
    for (int e = threadIdx.x; e < E; e += kGrpThreads)
      hist_counts[(int64_t)e * hist_cols + blockIdx.x] = thist[e];
    if (threadIdx.x == 0) hist_bad[blockIdx.x] = 0;
  }
}

// One workgroup: the auxiliary losses (router_aux_block).
template <bool F32>
__global__ __launch_bounds__(kAuxThreads) void router_aux_kernel(
    const float* __restrict__ partial, int nblk, int64_t T, int E,
    const int32_t* __restrict__ tokens_per_expert, const float* __restrict__ coef,
    const float* __restrict__ wn, typename RtElt<F32>::T* __restrict__ f_i,
    float* __restrict__ f_i32, float* __restrict__ p_i, typename RtElt<F32>::T* __restrict__ z_out,
    float* __restrict__ out_scalars) {
  router_aux_block<F32>(partial, nblk, T, E, tokens_per_expert, coef, wn, f_i, f_i32, p_i, z_out,
                        out_scalars);
}

// dL for every logit (one wave per token).
template <int VPL, bool F32>
__global__ __launch_bounds__(kRtThreads) void router_aux_bwd_kernel(
    const typename RtElt<F32>::T* __restrict__ logits, int64_t ldl, int64_t T, int E,
    const float* __restrict__ lse, const float* __restrict__ f_i32,
    const float* __restrict__ coef, const float* __restrict__ wn,
    const float* __restrict__ g_z, const float* __restrict__ g_lb,
    const float* __restrict__ g_cl, typename RtElt<F32>::T* __restrict__ grad, int64_t ldg) {
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
  const float invT = 1.0f / (float)T;
  const float gz = g_z ? *g_z : 0.0f, glb = g_lb ? *g_lb : 0.0f, gcl = g_cl ? *g_cl : 0.0f;
  float ce[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int e = lane + v * kWave;
    ce[v] = e < E ? (glb * coef[e] * f_i32[e] + gcl * wn[e]) * invT : 0.0f;
  }
  for (int64_t t = (int64_t)blockIdx.x * kRtWaves + wv; t < T;
       t += (int64_t)gridDim.x * kRtWaves) {
    const float l = lse[t];
    const float zt = gz * 2.0f * l * invT;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const int e = lane + v * kWave;
      if (e >= E) continue;
      const float x = RtElt<F32>::ld(logits + t * ldl + e);
      const float p = sigmoidf(x);
      const float d = zt * expf(x - l) + ce[v] * p * (1.0f - p);
      grad[t * ldg + e] = RtElt<F32>::cvt(d);
    }
  }
}

// Gradient of the routing weights with respect to the logits (opt-in; the
// reference's weights get none, scatter.py:176), one wave per token, lane j
// < k holding slot j: p_j = sigmoid(float(L[t, s_j])) as in the forward,
// g_j = grad_w[t, j], then
//   normalised:   S = sum_j p_j + 1e-20, dp_j = (g_j - sum_i g_i p_i / S) / S
//   otherwise:    dp_j = g_j
// and grad[t, e] = bf16(dp_j p_j (1 - p_j)) for e = s_j, 0 for the other
// experts (torch.topk's backward scatters into zeros; sigmoid's is
// g y (1 - y)). The sums run in the DPP order of wave_sum_f32.
template <int VPL, bool F32>
__global__ __launch_bounds__(kRtThreads) void router_weight_bwd_kernel(
    const typename RtElt<F32>::T* __restrict__ logits, int64_t ldl, int64_t T, int E, int k,
    int norm, const int32_t* __restrict__ sel32, const int64_t* __restrict__ sel64,
    const typename RtElt<F32>::T* __restrict__ gw, int64_t ldgw,
    typename RtElt<F32>::T* __restrict__ grad, int64_t ldg) {
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
  for (int64_t t = (int64_t)blockIdx.x * kRtWaves + wv; t < T;
       t += (int64_t)gridDim.x * kRtWaves) {
    int e = -1;
    float p = 0.0f, g = 0.0f;
    if (lane < k) {
      e = sel32 ? sel32[t * k + lane] : (int)sel64[t * k + lane];
      if (e >= 0 && e < E) {
        p = sigmoidf(RtElt<F32>::ld(logits + t * ldl + e));
        g = RtElt<F32>::ld(gw + t * ldgw + lane);
      } else {
        e = -1;
      }
    }
    float dp = g;
    if (norm) {
      const float S = wave_sum_f32(p) + 1e-20f;
      const float gp = wave_sum_f32(g * p);
      dp = (g - gp / S) / S;
    }
    const float dl = dp * p * (1.0f - p);
    float val[VPL];
#pragma unroll
    for (int v = 0; v < VPL; ++v) val[v] = 0.0f;
    for (int j = 0; j < k; ++j) {
      const int ej = __shfl(e, j, kWave);
      const float dj = __shfl(dl, j, kWave);
#pragma unroll
      for (int v = 0; v < VPL; ++v)
        if (ej == lane + v * kWave) val[v] = dj;
    }
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const int ee = lane + v * kWave;
      if (ee < E) grad[t * ldg + ee] = RtElt<F32>::cvt(val[v]);
    }
  }
}

inline int vpl_of(int E) {
  int v = 1;
  while (v * kWave < E) v <<= 1;
  return v;
}

inline int group_size(int E) {
  int g = 1;
  while (8 * g < E) g <<= 1;
  return g;
}

// Workgroups of the top-k launch = partial rows for the aux kernel (both
// top-k kernels take any count; each workgroup handles a contiguous token
// range). Experts the grouped kernel can take: one token batch per wave
// (16 waves of 64 / G tokens), but at least min(256, T / (64 / G))
// workgroups so small T still spreads over the device. Otherwise about
// 2 tokens per wave. At most kRtMaxBlocks.
inline int router_blocks(int64_t T, int E) {
  int64_t b;
  if (E % 8 == 0 && E <= kGrpMaxExperts) {
    const int64_t tpw = kWave / group_size(E);
    b = (T + kGrpWaves * tpw - 1) / (kGrpWaves * tpw);
    b = std::max(b, std::min<int64_t>(256, (T + tpw - 1) / tpw));
  } else {
    const int per = 2 * topk_threads(vpl_of(E)) / kWave;
    b = (T + per - 1) / per;
  }
  return (int)std::max<int64_t>(1, std::min<int64_t>(b, kRtMaxBlocks));
}

// Workgroups of vmoe_router_topk_hist: S per routing tile (S =
// route_hist_split), kRouteTile / (S k) tokens each, on the grouped top-k
// kernel; 0 where that launch does not apply.
static_assert(kGrpMaxExperts == 128 && kRtMaxBlocks >= 1024, "route_hist_split's limits");
inline int router_hist_blocks(int64_t T, int E, int k) {
  const int S = route_hist_split(T, E, k);
  return S ? (int)(route_tiles(T * k) * S) : 0;
}

// The grouped top-k launch for G lanes per token (hist_counts nullable).
template <bool F32>
int topk_group_launch(int G, int nblk, hipStream_t s, const typename RtElt<F32>::T* logits,
                      int64_t ld, int64_t T, int E, int k, int norm,
                      typename RtElt<F32>::T* weights, int32_t* sel32, int64_t* sel64,
                      float* probs, float* lse, float* partial, int64_t per,
                      int32_t* hist_counts, int32_t* hist_bad) {
  switch (G) {
#define VMOE_RT_GRP(GG)                                                                        \
  case GG:                                                                                     \
    VMOE_LAUNCH((router_topk_group_kernel<GG, F32>), dim3(nblk), dim3(kGrpThreads), 0, \
                       s,                                                                      \
                       logits, ld, T, E, k, norm, weights, sel32, sel64, probs, lse, partial,   \
                       per, hist_counts, hist_bad, nblk);                                      \
    break;
    VMOE_RT_GRP(1)
    VMOE_RT_GRP(2)
    VMOE_RT_GRP(4)
    VMOE_RT_GRP(8)
    VMOE_RT_GRP(16)
#undef VMOE_RT_GRP
    default:
      return VMOE_ERR_UNSUPPORTED;
  }
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

// Shapes and layouts the grouped top-k kernel reads (16-byte logits rows).
bool group_kernel_ok(const void* logits, int64_t ld, int E, int k, const float* probs) {
  return E % 8 == 0 && E <= kGrpMaxExperts && k <= 8 && ld % 8 == 0 &&
         reinterpret_cast<uintptr_t>(logits) % 16 == 0 &&
         (!probs || reinterpret_cast<uintptr_t>(probs) % 16 == 0);
}

// Router logits L = bf16(x W^T) (nn.Linear without bias) for E <= 32 NT
// experts: a workgroup takes 32 tokens and its 4 waves split K into quarters.
// A wave walks its quarter in chunks of 64 k (one 128-byte line per row):
// global loads of 8 rows x 128 bytes per instruction (the next chunk's in
// registers while the current one is used), a wave-private swizzled LDS copy
// (chunk c of row r at c ^ ((r >> 1) & 7): conflict-free 16-lane phases both
// ways), then v_mfma_f32_32x32x16_bf16 with the expert rows as the first
// operand (each lane then holds 4 consecutive experts of one token). Rows
// past T or E read a valid row and their results are never stored. Waves 1-3
// leave their partial sums in LDS; wave 0 adds them in wave order and rounds
// once.
typedef __bf16 rl_bf16x8 __attribute__((ext_vector_type(8)));
typedef float rl_f32x16 __attribute__((ext_vector_type(16)));
constexpr int kRlThreads = 256;
constexpr int kRlWaves = kRlThreads / kWave;
constexpr int kRlTokens = 32;
constexpr int kRlChunk = 64;  // k per chunk: 128 bytes of a row
typedef __attribute__((address_space(3))) char rl_lds;
typedef uint32_t rl_u32x4 __attribute__((ext_vector_type(4)));

template <int NT>
__global__ __launch_bounds__(kRlThreads) void router_logits_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t T, int K, const uint16_t* __restrict__ w,
    int64_t ldw, int E, uint16_t* __restrict__ out, int64_t ldo) {
  constexpr int XI = kRlTokens / 8, WI = 32 * NT / 8;  // load instructions per chunk
  __shared__ __align__(16) char stage[kRlWaves][(kRlTokens + 32 * NT) * 128];
  __shared__ float red[kRlWaves - 1][NT][16][kWave];
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
  const int64_t t0 = (int64_t)blockIdx.x * kRlTokens;
  const int kq = K / kRlWaves;
  const int k0 = wv * kq;
  // Loads: instruction u covers rows 8u .. 8u + 7, lane -> (row 8u + lane/8, 16 bytes lane%8).
  const rl_u32x4* xs[XI];
  const rl_u32x4* ws[WI];
#pragma unroll
  for (int u = 0; u < XI; ++u) {
    const int64_t t = min(t0 + 8 * u + (lane >> 3), T - 1);
    xs[u] = reinterpret_cast<const rl_u32x4*>(x + t * ldx + k0) + (lane & 7);
  }
#pragma unroll
  for (int u = 0; u < WI; ++u) {
    const int e = min(8 * u + (lane >> 3), E - 1);
    ws[u] = reinterpret_cast<const rl_u32x4*>(w + (int64_t)e * ldw + k0) + (lane & 7);
  }
  // An LDS pointer, so the compiler knows these stores cannot touch the
  // lane's registers-in-memory (a generic pointer keeps xa / wa in scratch).
  rl_lds* st = (rl_lds*)stage[wv];
  auto spos = [](int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); };
  rl_f32x16 acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[j][v] = 0.0f;
  rl_u32x4 xa[XI], wa[WI];
#pragma unroll
  for (int u = 0; u < XI; ++u) xa[u] = xs[u][0];
#pragma unroll
  for (int u = 0; u < WI; ++u) wa[u] = ws[u][0];
  const int nch = kq / kRlChunk;
  for (int ch = 0; ch < nch; ++ch) {
    // the chunk into LDS, then the next chunk's loads
#pragma unroll
    for (int u = 0; u < XI; ++u)
      *reinterpret_cast<__attribute__((address_space(3))) rl_u32x4*>(st + spos(8 * u + (lane >> 3), lane & 7)) = xa[u];
#pragma unroll
    for (int u = 0; u < WI; ++u)
      *reinterpret_cast<__attribute__((address_space(3))) rl_u32x4*>(st + kRlTokens * 128 + spos(8 * u + (lane >> 3), lane & 7)) = wa[u];
    {
      // the last chunk reloads itself (unused) so the loads are unconditional
      const int off = min(ch + 1, nch - 1) * (kRlChunk / 8);  // uint4 per chunk of a row
#pragma unroll
      for (int u = 0; u < XI; ++u) xa[u] = xs[u][off];
#pragma unroll
      for (int u = 0; u < WI; ++u) wa[u] = ws[u][off];
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int s4 = 0; s4 < kRlChunk / 16; ++s4) {
      const int c = 2 * s4 + (lane >> 5);
      const rl_u32x4 a = *reinterpret_cast<const __attribute__((address_space(3))) rl_u32x4*>(st + spos(lane & 31, c));
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const rl_u32x4 b = *reinterpret_cast<const __attribute__((address_space(3))) rl_u32x4*>(
            st + kRlTokens * 128 + spos(32 * j + (lane & 31), c));
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(rl_bf16x8, b),
                                                         __builtin_bit_cast(rl_bf16x8, a), acc[j],
                                                         0, 0, 0);
      }
    }
    __builtin_amdgcn_wave_barrier();  // the next chunk overwrites the wave's stage
  }
  if (wv > 0) {
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) red[wv - 1][j][v][lane] = acc[j][v];
  }
  __syncthreads();
  const int64_t t = t0 + (lane & 31);
  if (wv != 0 || t >= T) return;
#pragma unroll
  for (int j = 0; j < NT; ++j) {
#pragma unroll
    for (int w2 = 0; w2 < kRlWaves - 1; ++w2)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[j][v] += red[w2][j][v][lane];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      // experts 32 j + 8 g + 4 (lane / 32) + r, r = 0..3
      const int e = 32 * j + 8 * g + 4 * (lane >> 5);
      if (e < E)
        *reinterpret_cast<uint2*>(out + t * ldo + e) =
            make_uint2(pack_bf16(acc[j][4 * g], acc[j][4 * g + 1]),
                       pack_bf16(acc[j][4 * g + 2], acc[j][4 * g + 3]));
    }
  }
}

}  // namespace
}  // namespace vmoe

using namespace vmoe;

extern "C" size_t vmoe_router_partial_floats(int64_t num_tokens, int32_t num_experts) {
  if (num_tokens < 0 || num_experts <= 0) return 0;
  return (size_t)router_blocks(num_tokens, num_experts) * (size_t)(num_experts + 1);
}

template <bool F32>
int router_topk_impl(const typename RtElt<F32>::T* logits, int64_t ld_logits, int64_t num_tokens,
                     int32_t num_experts, int32_t top_k, int32_t normalize,
                     typename RtElt<F32>::T* weights, int32_t* selected_i32,
                     int64_t* selected_i64, float* probs, float* lse, float* partial,
                     size_t partial_floats, int32_t* num_partial_rows, vmoe_stream_t stream) {
  if (num_tokens < 0 || num_experts <= 0 || top_k <= 0 || top_k > num_experts ||
      ld_logits < num_experts)
    return VMOE_ERR_INVALID_ARG;
  if (num_experts > kRtMaxExperts || top_k > kWave) return VMOE_ERR_UNSUPPORTED;
  // with no tokens only the partial rows (zeros) are written; empty outputs
  // may come as NULL
  if (!partial || (num_tokens > 0 && (!weights || !lse || (!selected_i32 && !selected_i64) ||
                                      !logits)))
    return VMOE_ERR_INVALID_ARG;
  const int nblk = router_blocks(num_tokens, num_experts);
  if (partial_floats < (size_t)nblk * (size_t)(num_experts + 1)) return VMOE_ERR_WORKSPACE;
  if (num_partial_rows) *num_partial_rows = nblk;
  const int64_t per = (num_tokens + nblk - 1) / nblk;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (group_kernel_ok(logits, ld_logits, num_experts, top_k, probs))
    return topk_group_launch<F32>(group_size(num_experts), nblk, s, logits, ld_logits,
                                  num_tokens, num_experts, top_k, normalize, weights,
                                  selected_i32, selected_i64, probs, lse, partial, per, nullptr,
                                  nullptr);
  const int vpl = vpl_of(num_experts);
  const size_t lds = sizeof(float) * (topk_threads(vpl) / kWave) * (num_experts + 1);
  switch (vpl) {
#define VMOE_RT_CASE(V)                                                                      \
  case V:                                                                                    \
    VMOE_LAUNCH((router_topk_kernel<V, F32>), dim3(nblk), dim3(topk_threads(V)), lds, \
                       s, logits, ld_logits, num_tokens, num_experts, top_k, normalize,       \
                       weights, selected_i32, selected_i64, probs, lse, partial, per);        \
    break;
    VMOE_RT_CASE(1)
    VMOE_RT_CASE(2)
    VMOE_RT_CASE(4)
    VMOE_RT_CASE(8)
    VMOE_RT_CASE(16)
    VMOE_RT_CASE(32)
#undef VMOE_RT_CASE
    default:
      return VMOE_ERR_UNSUPPORTED;
  }
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

template <bool F32>
int router_topk_hist_impl(const typename RtElt<F32>::T* logits, int64_t ld_logits,
                          int64_t num_tokens, int32_t num_experts, int32_t top_k,
                          int32_t normalize, typename RtElt<F32>::T* weights,
                          int32_t* selected_i32, int64_t* selected_i64, float* probs, float* lse,
                          float* partial, size_t partial_floats, int32_t* num_partial_rows,
                          void* route_workspace, size_t route_workspace_bytes,
                          vmoe_stream_t stream) {
  if (num_tokens < 0 || num_experts <= 0 || top_k <= 0 || top_k > num_experts ||
      ld_logits < num_experts)
    return VMOE_ERR_INVALID_ARG;
  if (!weights || !partial || !lse || !route_workspace || (!selected_i32 && !selected_i64) ||
      (num_tokens > 0 && !logits))
    return VMOE_ERR_INVALID_ARG;
  const int nblk = router_hist_blocks(num_tokens, num_experts, top_k);
  if (nblk == 0 || !group_kernel_ok(logits, ld_logits, num_experts, top_k, probs))
    return VMOE_ERR_UNSUPPORTED;
  if (partial_floats < (size_t)nblk * (size_t)(num_experts + 1) ||
      route_workspace_bytes < vmoe_route_counted_workspace_bytes(num_tokens, num_experts, top_k))
    return VMOE_ERR_WORKSPACE;
  if (num_partial_rows) *num_partial_rows = nblk;
  // counts [E][nblk] (one column per workgroup), then a bad-id flag per column
  const int S = route_hist_split(num_tokens, num_experts, top_k);
  int32_t* counts = static_cast<int32_t*>(route_workspace);
  return topk_group_launch<F32>(group_size(num_experts), nblk,
                                reinterpret_cast<hipStream_t>(stream), logits, ld_logits,
                                num_tokens, num_experts, top_k, normalize, weights, selected_i32,
                                selected_i64, probs, lse, partial, kRouteTile / (top_k * S),
                                counts, counts + (int64_t)num_experts * nblk);
}

template <bool F32>
int router_aux_impl(const float* partial, int32_t num_partial_rows, int64_t num_tokens,
                    int32_t num_experts, const int32_t* tokens_per_expert, const float* coef,
                    const float* widths_normalized, typename RtElt<F32>::T* f_i, float* f_i_f32,
                    float* p_i, typename RtElt<F32>::T* z_loss, float* losses,
                    vmoe_stream_t stream) {
  if (num_partial_rows <= 0 || num_tokens < 0 || num_experts <= 0) return VMOE_ERR_INVALID_ARG;
  if (!partial || !tokens_per_expert || !coef || !widths_normalized || !f_i || !f_i_f32 ||
      !p_i || !z_loss || !losses)
    return VMOE_ERR_INVALID_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  VMOE_LAUNCH(router_aux_kernel<F32>, dim3(1), dim3(kAuxThreads), 0, s, partial,
                     num_partial_rows, num_tokens, num_experts, tokens_per_expert, coef,
                     widths_normalized, f_i, f_i_f32, p_i, z_loss, losses);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

template <bool F32>
int router_aux_bwd_impl(const typename RtElt<F32>::T* logits, int64_t ld_logits,
                        int64_t num_tokens, int32_t num_experts, const float* lse,
                        const float* f_i_f32, const float* coef, const float* widths_normalized,
                        const float* grad_z, const float* grad_lb, const float* grad_cl,
                        typename RtElt<F32>::T* grad_logits, int64_t ld_grad,
                        vmoe_stream_t stream) {
  if (num_tokens < 0 || num_experts <= 0 || ld_logits < num_experts || ld_grad < num_experts)
    return VMOE_ERR_INVALID_ARG;
  if (num_experts > kRtMaxExperts) return VMOE_ERR_UNSUPPORTED;
  if (num_tokens == 0) return VMOE_OK;
  if (!logits || !lse || !f_i_f32 || !coef || !widths_normalized || !grad_logits)
    return VMOE_ERR_INVALID_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t g = std::min<int64_t>((num_tokens + kRtWaves - 1) / kRtWaves, 4096);
  switch (vpl_of(num_experts)) {
#define VMOE_RB_CASE(V)                                                                       \
  case V:                                                                                     \
    VMOE_LAUNCH((router_aux_bwd_kernel<V, F32>), dim3((unsigned)g), dim3(kRtThreads),   \
                       0, s, logits, ld_logits, num_tokens, num_experts, lse, f_i_f32, coef,   \
                       widths_normalized, grad_z, grad_lb, grad_cl, grad_logits, ld_grad);    \
    break;
    VMOE_RB_CASE(1)
    VMOE_RB_CASE(2)
    VMOE_RB_CASE(4)
    VMOE_RB_CASE(8)
    VMOE_RB_CASE(16)
    VMOE_RB_CASE(32)
#undef VMOE_RB_CASE
    default:
      return VMOE_ERR_UNSUPPORTED;
  }
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

template <bool F32>
int router_weight_bwd_impl(const typename RtElt<F32>::T* logits, int64_t ld_logits,
                           int64_t num_tokens, int32_t num_experts, int32_t top_k,
                           int32_t normalize, const int32_t* selected,
                           const int64_t* selected_i64,
                           const typename RtElt<F32>::T* grad_weights, int64_t ld_grad_weights,
                           typename RtElt<F32>::T* grad_logits, int64_t ld_grad,
                           vmoe_stream_t stream) {
  if (num_tokens < 0 || num_experts <= 0 || top_k <= 0 || top_k > num_experts ||
      ld_logits < num_experts || ld_grad < num_experts || ld_grad_weights < top_k)
    return VMOE_ERR_INVALID_ARG;
  if (num_experts > kRtMaxExperts || top_k > kWave) return VMOE_ERR_UNSUPPORTED;
  if (num_tokens == 0) return VMOE_OK;
  if (!logits || !grad_weights || !grad_logits || (!selected == !selected_i64))
    return VMOE_ERR_INVALID_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t g = std::min<int64_t>((num_tokens + kRtWaves - 1) / kRtWaves, 4096);
  switch (vpl_of(num_experts)) {
#define VMOE_RW_CASE(V)                                                                      \
  case V:                                                                                    \
    VMOE_LAUNCH((router_weight_bwd_kernel<V, F32>), dim3((unsigned)g),                 \
                       dim3(kRtThreads), 0, s, logits, ld_logits, num_tokens, num_experts,    \
                       top_k, normalize, selected, selected_i64, grad_weights,                \
                       ld_grad_weights, grad_logits, ld_grad);                                \
    break;
    VMOE_RW_CASE(1)
    VMOE_RW_CASE(2)
    VMOE_RW_CASE(4)
    VMOE_RW_CASE(8)
    VMOE_RW_CASE(16)
    VMOE_RW_CASE(32)
#undef VMOE_RW_CASE
    default:
      return VMOE_ERR_UNSUPPORTED;
  }
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

extern "C" int vmoe_router_topk(const uint16_t* logits, int64_t ld_logits, int64_t num_tokens,
                                int32_t num_experts, int32_t top_k, int32_t normalize,
                                uint16_t* weights, int32_t* selected_i32, int64_t* selected_i64,
                                float* probs, float* lse, float* partial, size_t partial_floats,
                                int32_t* num_partial_rows, vmoe_stream_t stream) {
  return router_topk_impl<false>(logits, ld_logits, num_tokens, num_experts, top_k, normalize,
                                 weights, selected_i32, selected_i64, probs, lse, partial,
                                 partial_floats, num_partial_rows, stream);
}

extern "C" int vmoe_router_topk_f32(const float* logits, int64_t ld_logits, int64_t num_tokens,
                                    int32_t num_experts, int32_t top_k, int32_t normalize,
                                    float* weights, int32_t* selected_i32, int64_t* selected_i64,
                                    float* probs, float* lse, float* partial,
                                    size_t partial_floats, int32_t* num_partial_rows,
                                    vmoe_stream_t stream) {
  return router_topk_impl<true>(logits, ld_logits, num_tokens, num_experts, top_k, normalize,
                                weights, selected_i32, selected_i64, probs, lse, partial,
                                partial_floats, num_partial_rows, stream);
}

extern "C" int vmoe_router_topk_hist_blocks(int64_t num_tokens, int32_t num_experts,
                                            int32_t top_k) {
  return router_hist_blocks(num_tokens, num_experts, top_k);
}

extern "C" int vmoe_router_topk_hist(const uint16_t* logits, int64_t ld_logits,
                                     int64_t num_tokens, int32_t num_experts, int32_t top_k,
                                     int32_t normalize, uint16_t* weights, int32_t* selected_i32,
                                     int64_t* selected_i64, float* probs, float* lse,
                                     float* partial, size_t partial_floats,
                                     int32_t* num_partial_rows, void* route_workspace,
                                     size_t route_workspace_bytes, vmoe_stream_t stream) {
  return router_topk_hist_impl<false>(logits, ld_logits, num_tokens, num_experts, top_k,
                                      normalize, weights, selected_i32, selected_i64, probs,
                                      lse, partial, partial_floats, num_partial_rows,
                                      route_workspace, route_workspace_bytes, stream);
}

extern "C" int vmoe_router_topk_hist_f32(const float* logits, int64_t ld_logits,
                                         int64_t num_tokens, int32_t num_experts, int32_t top_k,
                                         int32_t normalize, float* weights,
                                         int32_t* selected_i32, int64_t* selected_i64,
                                         float* probs, float* lse, float* partial,
                                         size_t partial_floats, int32_t* num_partial_rows,
                                         void* route_workspace, size_t route_workspace_bytes,
                                         vmoe_stream_t stream) {
  return router_topk_hist_impl<true>(logits, ld_logits, num_tokens, num_experts, top_k,
                                     normalize, weights, selected_i32, selected_i64, probs, lse,
                                     partial, partial_floats, num_partial_rows, route_workspace,
                                     route_workspace_bytes, stream);
}

extern "C" int vmoe_router_aux(const float* partial, int32_t num_partial_rows,
                               int64_t num_tokens, int32_t num_experts,
                               const int32_t* tokens_per_expert, const float* coef,
                               const float* widths_normalized, uint16_t* f_i, float* f_i_f32,
                               float* p_i, uint16_t* z_loss, float* losses,
                               vmoe_stream_t stream) {
  return router_aux_impl<false>(partial, num_partial_rows, num_tokens, num_experts,
                                tokens_per_expert, coef, widths_normalized, f_i, f_i_f32, p_i,
                                z_loss, losses, stream);
}

extern "C" int vmoe_router_aux_f32(const float* partial, int32_t num_partial_rows,
                                   int64_t num_tokens, int32_t num_experts,
                                   const int32_t* tokens_per_expert, const float* coef,
                                   const float* widths_normalized, float* f_i, float* f_i_f32,
                                   float* p_i, float* z_loss, float* losses,
                                   vmoe_stream_t stream) {
  return router_aux_impl<true>(partial, num_partial_rows, num_tokens, num_experts,
                               tokens_per_expert, coef, widths_normalized, f_i, f_i_f32, p_i,
                               z_loss, losses, stream);
}

extern "C" int vmoe_router_aux_bwd(const uint16_t* logits, int64_t ld_logits, int64_t num_tokens,
                                   int32_t num_experts, const float* lse, const float* f_i_f32,
                                   const float* coef, const float* widths_normalized,
                                   const float* grad_z, const float* grad_lb,
                                   const float* grad_cl, uint16_t* grad_logits, int64_t ld_grad,
                                   vmoe_stream_t stream) {
  return router_aux_bwd_impl<false>(logits, ld_logits, num_tokens, num_experts, lse, f_i_f32,
                                    coef, widths_normalized, grad_z, grad_lb, grad_cl,
                                    grad_logits, ld_grad, stream);
}

extern "C" int vmoe_router_aux_bwd_f32(const float* logits, int64_t ld_logits,
                                       int64_t num_tokens, int32_t num_experts, const float* lse,
                                       const float* f_i_f32, const float* coef,
                                       const float* widths_normalized, const float* grad_z,
                                       const float* grad_lb, const float* grad_cl,
                                       float* grad_logits, int64_t ld_grad,
                                       vmoe_stream_t stream) {
  return router_aux_bwd_impl<true>(logits, ld_logits, num_tokens, num_experts, lse, f_i_f32,
                                   coef, widths_normalized, grad_z, grad_lb, grad_cl,
                                   grad_logits, ld_grad, stream);
}

extern "C" int vmoe_router_weight_bwd(const uint16_t* logits, int64_t ld_logits,
                                      int64_t num_tokens, int32_t num_experts, int32_t top_k,
                                      int32_t normalize, const int32_t* selected,
                                      const int64_t* selected_i64, const uint16_t* grad_weights,
                                      int64_t ld_grad_weights, uint16_t* grad_logits,
                                      int64_t ld_grad, vmoe_stream_t stream) {
  return router_weight_bwd_impl<false>(logits, ld_logits, num_tokens, num_experts, top_k,
                                       normalize, selected, selected_i64, grad_weights,
                                       ld_grad_weights, grad_logits, ld_grad, stream);
}

extern "C" int vmoe_router_weight_bwd_f32(const float* logits, int64_t ld_logits,
                                          int64_t num_tokens, int32_t num_experts, int32_t top_k,
                                          int32_t normalize, const int32_t* selected,
                                          const int64_t* selected_i64, const float* grad_weights,
                                          int64_t ld_grad_weights, float* grad_logits,
                                          int64_t ld_grad, vmoe_stream_t stream) {
  return router_weight_bwd_impl<true>(logits, ld_logits, num_tokens, num_experts, top_k,
                                      normalize, selected, selected_i64, grad_weights,
                                      ld_grad_weights, grad_logits, ld_grad, stream);
}

extern "C" int vmoe_router_logits(const uint16_t* x, int64_t ldx, int64_t num_tokens,
                                  int64_t hidden, const uint16_t* weight, int64_t ldw,
                                  int32_t num_experts, uint16_t* logits, int64_t ld_logits,
                                  vmoe_stream_t stream) {
  if (num_tokens < 0 || hidden <= 0 || num_experts <= 0 || ldx < hidden || ldw < hidden ||
      ld_logits < num_experts)
    return VMOE_ERR_INVALID_ARG;
  if (num_tokens == 0) return VMOE_OK;
  if (!x || !weight || !logits) return VMOE_ERR_INVALID_ARG;
  if (num_experts > 4 * 32 || num_experts % 8 != 0 || hidden % (kRlChunk * kRlWaves) != 0 ||
      hidden > INT32_MAX || ldx % 8 != 0 || ldw % 8 != 0 || ld_logits % 4 != 0 ||
      reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(weight) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(logits) % 8 != 0)
    return VMOE_ERR_UNSUPPORTED;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((num_tokens + kRlTokens - 1) / kRlTokens));
  switch ((num_experts + 31) / 32) {
#define VMOE_RL_CASE(N)                                                                   \
  case N:                                                                                 \
    VMOE_LAUNCH(router_logits_kernel<N>, grid, dim3(kRlThreads), 0, s, x, ldx,      \
                       num_tokens, (int)hidden, weight, ldw, num_experts, logits, ld_logits); \
    break;
    VMOE_RL_CASE(1)
    VMOE_RL_CASE(2)
    VMOE_RL_CASE(3)
    VMOE_RL_CASE(4)
#undef VMOE_RL_CASE
    default:
      return VMOE_ERR_UNSUPPORTED;
  }
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}
