// Token permutation on gfx950: padded gather (plain and weighted) and the
// fused weighted combine. All three are HBM-bound row copies: each wave owns
// one row at a time and moves it with 16-byte vectors, every output row is
// written exactly once (pad rows get zeros in the same pass, so no memset of
// the output), and the combine sums the top_k rows of a token in fp32
// registers, so the [T, k, d] intermediate of the reference never exists.
//
// Numerics (bit-exact with the reference for the same inputs):
//   gather:    copy (triton_moe/kernels/gather.py:56-60)
//   weighted:  bf16(v * w), the product of two bf16 is exact in fp32 and is
//              rounded once (gather.py:170-174)
//   combine:   out = bf16(sum_j f32(bf16(y_j * w_j))), j ascending, as
//              padded_scatter's per-slot bf16 product followed by
//              intermediate.sum(dim=1) with fp32 accumulation
//              (triton_moe/kernels/scatter.py:61-69, 133)

#include <algorithm>

#include "vmoe_common.h"

namespace vmoe {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / kWave;

// VEC = 8: rows move as uint4 (8 bf16); VEC = 1: scalar fallback for
// unaligned shapes.
template <int VEC>
struct Vec;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <>
struct Vec<8> {
  using T = uint4;
  __device__ static T load(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
  __device__ static void store(uint16_t* p, T v) { *reinterpret_cast<uint4*>(p) = v; }
  // Streaming (non-temporal) forms, for data read or written once.
  __device__ static T load_nt(const uint16_t* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  }
  __device__ static void store_nt(uint16_t* p, T v) {
    const u32x4 o = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(p));
  }
  __device__ static T zero() { return make_uint4(0, 0, 0, 0); }
  __device__ static void to_f32(T v, float* f) {
    f[0] = lo_f32(v.x); f[1] = hi_f32(v.x); f[2] = lo_f32(v.y); f[3] = hi_f32(v.y);
    f[4] = lo_f32(v.z); f[5] = hi_f32(v.z); f[6] = lo_f32(v.w); f[7] = hi_f32(v.w);
  }
  __device__ static T from_f32(const float* f) {
    return make_uint4(pack_bf16(f[0], f[1]), pack_bf16(f[2], f[3]), pack_bf16(f[4], f[5]),
                      pack_bf16(f[6], f[7]));
  }
};
template <>
struct Vec<1> {
  using T = uint16_t;
  __device__ static T load(const uint16_t* p) { return *p; }
  __device__ static void store(uint16_t* p, T v) { *p = v; }
  __device__ static T zero() { return 0; }
  __device__ static void to_f32(T v, float* f) { f[0] = bf16_to_f32(v); }
  __device__ static T from_f32(const float* f) { return (uint16_t)f32_to_bf16(f[0]); }
};

// out[r] = x[row_src[r] / top_k] (* w[row_src[r]]), zeros for row_src < 0.
template <int VEC, bool WEIGHTED>
__global__ __launch_bounds__(kThreads) void gather_kernel(
    const uint16_t* __restrict__ x, int64_t x_rows, int64_t ldx,
    const int32_t* __restrict__ row_src, int top_k, const uint16_t* __restrict__ w,
    int64_t nw, uint16_t* __restrict__ out, int64_t ldo, int64_t num_rows,
    const int32_t* __restrict__ num_rows_dev, int64_t hidden) {
  using V = Vec<VEC>;
  const int lane = threadIdx.x & (kWave - 1);
  int64_t rows = num_rows;
  if (num_rows_dev) rows = min(rows, (int64_t)*num_rows_dev);
  const int64_t nvec = hidden / VEC;
  for (int64_t r = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave; r < rows;
       r += (int64_t)gridDim.x * kRowsPerBlock) {
    const int32_t s = row_src[r];
    const int64_t t = s >= 0 ? s / top_k : -1;
    const bool live = s >= 0 && t < x_rows && (!WEIGHTED || s < nw);
    uint16_t* orow = out + r * ldo;
    if (!live) {
      for (int64_t c = lane; c < nvec; c += kWave) V::store(orow + c * VEC, V::zero());
      continue;
    }
    const uint16_t* xrow = x + t * ldx;
    float scale = 1.0f;
    if (WEIGHTED) scale = bf16_to_f32(w[s]);
    for (int64_t c = lane; c < nvec; c += kWave) {
      typename V::T v = V::load(xrow + c * VEC);
      if (WEIGHTED) {
        float f[VEC];
        V::to_f32(v, f);
#pragma unroll
        for (int i = 0; i < VEC; ++i) f[i] *= scale;
        v = V::from_f32(f);
      }
      V::store(orow + c * VEC, v);
    }
  }
}

// Token-major form of the same gather: wave-blocks [0, tok_blocks) take
// tokens, read x[t] once and write it (times w[t*k+j] when weighted) to each
// of its rows assignment_row[t*k+j] < rows; the remaining blocks write zeros
// to the pad rows (row_src < 0), found 64 rows at a time with a wave ballot.
// x is read once instead of top_k times. CHUNKS 16-byte vectors per lane stay
// in registers between the top_k stores.
template <bool WEIGHTED, int CHUNKS>
__global__ __launch_bounds__(kThreads) void gather_tokens_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const int32_t* __restrict__ assignment_row,
    int64_t num_tokens, int top_k, const uint16_t* __restrict__ w,
    const int32_t* __restrict__ row_src, uint16_t* __restrict__ out, int64_t ldo,
    int64_t num_rows, const int32_t* __restrict__ num_rows_dev, int64_t hidden, int tok_blocks) {
  using V = Vec<8>;
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  int64_t rows = num_rows;
  if (num_rows_dev) rows = min(rows, (int64_t)*num_rows_dev);
  const int64_t nvec = hidden / 8;
  if ((int)blockIdx.x < tok_blocks) {
    for (int64_t t = (int64_t)blockIdx.x * kRowsPerBlock + wv; t < num_tokens;
         t += (int64_t)tok_blocks * kRowsPerBlock) {
      // Lane j < top_k holds the row (and weight) of slot j.
      const int64_t a0 = t * top_k;
      int32_t my_row = -1;
      float my_w = 1.0f;
      if (lane < top_k) {
        my_row = assignment_row[a0 + lane];
        if (WEIGHTED) my_w = bf16_to_f32(w[a0 + lane]);
      }
      const uint16_t* xrow = x + t * ldx;
      for (int64_t c0 = 0; c0 < nvec; c0 += (int64_t)CHUNKS * kWave) {
        V::T v[CHUNKS];
#pragma unroll
        for (int ch = 0; ch < CHUNKS; ++ch) {
          const int64_t c = c0 + ch * kWave + lane;
          v[ch] = c < nvec ? V::load(xrow + c * 8) : V::zero();
        }
        for (int j = 0; j < top_k; ++j) {
          const int32_t r = __shfl(my_row, j, kWave);
          if (r < 0 || r >= rows) continue;
          const float scale = WEIGHTED ? __shfl(my_w, j, kWave) : 1.0f;
          uint16_t* orow = out + (int64_t)r * ldo;
#pragma unroll
          for (int ch = 0; ch < CHUNKS; ++ch) {
            const int64_t c = c0 + ch * kWave + lane;
            if (c >= nvec) continue;
            typename V::T o = v[ch];
            if (WEIGHTED) {
              float f[8];
              V::to_f32(o, f);
#pragma unroll
              for (int i = 0; i < 8; ++i) f[i] *= scale;
              o = V::from_f32(f);
            }
            V::store(orow + c * 8, o);
          }
        }
      }
    }
    return;
  }
  const int pad_blocks = (int)gridDim.x - tok_blocks;
  for (int64_t r0 = ((int64_t)(blockIdx.x - tok_blocks) * kRowsPerBlock + wv) * kWave; r0 < rows;
       r0 += (int64_t)pad_blocks * kRowsPerBlock * kWave) {
    const int64_t r = r0 + lane;
    uint64_t pad = ballot64(r < rows && row_src[r] < 0);
    while (pad) {
      const int b = __builtin_ctzll(pad);
      pad &= pad - 1;
      uint16_t* orow = out + (r0 + b) * ldo;
      for (int64_t c = lane; c < nvec; c += kWave) V::store(orow + c * 8, V::zero());
    }
  }
}

// out[t] = bf16(sum_j f32(bf16(y[row(t,j)] * w[t*k+j]))). Each lane keeps up
// to CHUNKS vectors of the row in fp32 registers.
template <int VEC, bool WEIGHTED, int CHUNKS>
__global__ __launch_bounds__(kThreads) void combine_kernel(
    const uint16_t* __restrict__ y, int64_t y_rows, int64_t ldy,
    const int32_t* __restrict__ assignment_row, const uint16_t* __restrict__ w, int top_k,
    uint16_t* __restrict__ out, int64_t ldo, int64_t num_tokens, int64_t hidden) {
  using V = Vec<VEC>;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t nvec = hidden / VEC;
  for (int64_t t = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave; t < num_tokens;
       t += (int64_t)gridDim.x * kRowsPerBlock) {
    for (int64_t c0 = 0; c0 < nvec; c0 += (int64_t)CHUNKS * kWave) {
      float acc[CHUNKS][VEC];
#pragma unroll
      for (int ch = 0; ch < CHUNKS; ++ch)
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[ch][i] = 0.0f;
      for (int j = 0; j < top_k; ++j) {
        const int64_t a = t * top_k + j;
        const int32_t row = assignment_row[a];
        if (row < 0 || row >= y_rows) continue;
        const float scale = WEIGHTED ? bf16_to_f32(w[a]) : 1.0f;
        const uint16_t* yrow = y + (int64_t)row * ldy;
        typename V::T v[CHUNKS];
#pragma unroll
        for (int ch = 0; ch < CHUNKS; ++ch) {
          const int64_t c = c0 + ch * kWave + lane;
          v[ch] = c < nvec ? V::load(yrow + c * VEC) : V::zero();
        }
#pragma unroll
        for (int ch = 0; ch < CHUNKS; ++ch) {
          float f[VEC];
          V::to_f32(v[ch], f);
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            // Round the weighted slot value to bf16 before the sum, as the
            // reference's bf16 [T, k, d] intermediate does.
            const float p = WEIGHTED ? bf16_to_f32(f32_to_bf16(f[i] * scale)) : f[i];
            acc[ch][i] += p;
          }
        }
      }
#pragma unroll
      for (int ch = 0; ch < CHUNKS; ++ch) {
        const int64_t c = c0 + ch * kWave + lane;
        if (c < nvec) V::store(out + t * ldo + c * VEC, V::from_f32(acc[ch]));
      }
    }
  }
}

// The same combine for top_k <= KMAX on 16-byte vectors: lane j reads slot
// j's row index (and weight) once and the wave takes them by readlane, then
// every slot's loads are issued before any is summed, so a wave has k rows
// in flight instead of one. The sum is the same: slot order, invalid rows
// skipped. The slot rows (read once) are loaded and the token rows stored
// non-temporally, so this 300 MB stream does not evict what the GEMMs
// around it re-read (cfg3 step -3 %, measured against plain accesses).
template <int KMAX, bool WEIGHTED, int CHUNKS>
__global__ __launch_bounds__(kThreads) void combine_k_kernel(
    const uint16_t* __restrict__ y, int64_t y_rows, int64_t ldy,
    const int32_t* __restrict__ assignment_row, const uint16_t* __restrict__ w, int top_k,
    uint16_t* __restrict__ out, int64_t ldo, int64_t num_tokens, int64_t hidden) {
  using V = Vec<8>;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t nvec = hidden / 8;
  for (int64_t t = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave; t < num_tokens;
       t += (int64_t)gridDim.x * kRowsPerBlock) {
    int32_t my_row = -1;
    uint32_t my_w = 0;
    if (lane < top_k) {
      my_row = assignment_row[t * top_k + lane];
      if (WEIGHTED) my_w = __float_as_uint(bf16_to_f32(w[t * top_k + lane]));
    }
    int32_t rows[KMAX];
    bool ok[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      rows[j] = __builtin_amdgcn_readlane(my_row, j);
      ok[j] = j < top_k && rows[j] >= 0 && rows[j] < y_rows;
    }
    for (int64_t c0 = 0; c0 < nvec; c0 += (int64_t)CHUNKS * kWave) {
      V::T v[KMAX][CHUNKS];
#pragma unroll
      for (int j = 0; j < KMAX; ++j)
#pragma unroll
        for (int ch = 0; ch < CHUNKS; ++ch) {
          const int64_t c = c0 + ch * kWave + lane;
          v[j][ch] = ok[j] && c < nvec ? V::load_nt(y + (int64_t)rows[j] * ldy + c * 8) : V::zero();
        }
      float acc[CHUNKS][8];
#pragma unroll
      for (int ch = 0; ch < CHUNKS; ++ch)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[ch][i] = 0.0f;
#pragma unroll
      for (int j = 0; j < KMAX; ++j) {
        if (!ok[j]) continue;
        const float scale =
            WEIGHTED ? __uint_as_float(__builtin_amdgcn_readlane(my_w, j)) : 1.0f;
#pragma unroll
        for (int ch = 0; ch < CHUNKS; ++ch) {
          float f[8];
          V::to_f32(v[j][ch], f);
#pragma unroll
          for (int i = 0; i < 8; ++i)
            acc[ch][i] += WEIGHTED ? bf16_to_f32(f32_to_bf16(f[i] * scale)) : f[i];
        }
      }
#pragma unroll
      for (int ch = 0; ch < CHUNKS; ++ch) {
        const int64_t c = c0 + ch * kWave + lane;
        if (c < nvec) V::store_nt(out + t * ldo + c * 8, V::from_f32(acc[ch]));
      }
    }
  }
}

// Zero columns [widths[e], max_width) of expert e's rows [eto[e], eto[e+1]).
__global__ __launch_bounds__(kThreads) void zero_tail_kernel(
    uint16_t* __restrict__ buf, int64_t ld, const int32_t* __restrict__ eto,
    const int32_t* __restrict__ widths, int E, int64_t max_width, int64_t rows_bound) {
  const int lane = threadIdx.x & (kWave - 1);
  for (int64_t r = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave; r < rows_bound;
       r += (int64_t)gridDim.x * kRowsPerBlock) {
    // Last expert whose range starts at or before r (binary search on eto).
    int lo = 0, hi = E;  // answer in [0, E)
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if ((int64_t)eto[mid] <= r) lo = mid; else hi = mid;
    }
    if (r < eto[lo] || r >= eto[lo + 1]) continue;
    const int64_t w0 = max<int64_t>(0, widths[lo]);
    for (int64_t c = w0 + lane; c < max_width; c += kWave) buf[r * ld + c] = 0;
  }
}

// Routing-weight gradient of the weighted combine (opt-in; the reference
// returns None for the weights, triton_moe/kernels/scatter.py:176):
//   gw[t*k+j] = sum_c f32(g[t, c]) * f32(y[row(t, j), c]), 0 for slots with no row.
// The rounding to bf16 of each slot is taken as identity (straight-through),
// as for the other gradients. One wave per token; the token's gradient row is
// re-read per slot from cache, y rows once from HBM. Lane partial sums are
// added by a butterfly, so the result is fp32 with a fixed summation order.
template <int VEC>
__global__ __launch_bounds__(kThreads) void combine_wgrad_kernel(
    const uint16_t* __restrict__ g, int64_t ldg, const uint16_t* __restrict__ y, int64_t y_rows,
    int64_t ldy, const int32_t* __restrict__ assignment_row, int top_k,
    float* __restrict__ gw, int64_t num_tokens, int64_t hidden) {
  using V = Vec<VEC>;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t nvec = hidden / VEC;
  for (int64_t t = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave; t < num_tokens;
       t += (int64_t)gridDim.x * kRowsPerBlock) {
    const uint16_t* grow = g + t * ldg;
    for (int j = 0; j < top_k; ++j) {
      const int64_t a = t * top_k + j;
      const int32_t row = assignment_row[a];
      float s = 0.0f;
      if (row >= 0 && row < y_rows) {
        const uint16_t* yrow = y + (int64_t)row * ldy;
        for (int64_t c = lane; c < nvec; c += kWave) {
          float fg[VEC], fy[VEC];
          V::to_f32(V::load(grow + c * VEC), fg);
          V::to_f32(V::load(yrow + c * VEC), fy);
#pragma unroll
          for (int i = 0; i < VEC; ++i) s = fmaf(fg[i], fy[i], s);
        }
      }
#pragma unroll
      for (int off = kWave / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, kWave);
      if (lane == 0) gw[a] = s;
    }
  }
}

// Routing-weight gradient of the module path, whose up GEMM writes
// H' = bf16(w * relu(z)^2): dL/dw of a row is sum_c dL/dH'[c] * relu(z)[c]^2.
// The dH GEMM leaves row_dot[row][b] = sum over block b of
// bf16(w * dL/dH') * PRE^2 (vmoe_gemm_down_bwd_dh); here the blocks are
// summed in order and divided by w, one thread per assignment:
//   gw[a] = bf16(sum_b row_dot[row][b] / w[row]), row = assignment_row[a],
// 0 where row < 0 (a dropped assignment) or w[row] == 0.
// Routing weights below this magnitude (zero and every bf16 denormal among
// them) take the direct form of their gradient: the dH GEMM's row sums hold
// w * (G W2^T) * relu(z)^2 rounded through bf16(w * (G W2^T)), and dividing
// them by such a w is 0 / 0 at w = 0 and loses the gradient's bits below.
constexpr float kTinyWeight = 0x1p-64f;

__global__ __launch_bounds__(kThreads) void routing_wgrad_kernel(
    const float* __restrict__ row_dot, int64_t ld, int nblk, int64_t rows,
    const float* __restrict__ row_weight, const int32_t* __restrict__ assignment_row,
    int64_t A, uint16_t* __restrict__ gw) {
  for (int64_t a = (int64_t)blockIdx.x * kThreads + threadIdx.x; a < A;
       a += (int64_t)gridDim.x * kThreads) {
    const int32_t row = assignment_row[a];
    float g = 0.0f;
    if (row >= 0 && row < rows) {
      const float w = row_weight[row];
      if (!(fabsf(w) < kTinyWeight)) {
        const float* rd = row_dot + (int64_t)row * ld;
        float s = 0.0f;
        for (int b = 0; b < nblk; ++b) s += rd[b];
        g = s / w;
      }
    }
    gw[a] = (uint16_t)f32_to_bf16(g);
  }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// The gradient of the routing weights below kTinyWeight, from its definition
// dL/dw = sum_c (G[t] . W2[ewo[e] + c]) * pre[row][c]^2, G's row t = a / top_k
// and e the expert whose rows [eto[e], eto[e+1]) hold `row`. Each lane tests
// one assignment; the wave then works through the tiny ones it found (one
// fp32 dot of length hidden per column, summed across the wave), so the
// launch costs one read of assignment_row and row_weight when there are
// none. Only the tiny entries of gw are written.
__global__ __launch_bounds__(kThreads) void routing_wgrad_direct_kernel(
    const uint16_t* __restrict__ gy, int64_t ldgy, int64_t gy_rows,
    const uint16_t* __restrict__ grad_scale, const uint16_t* __restrict__ w2, int64_t ldw2,
    const uint16_t* __restrict__ pre,
    int64_t ldp, const float* __restrict__ row_weight,
    const int32_t* __restrict__ assignment_row, int64_t A, int top_k,
    const int32_t* __restrict__ eto, const int32_t* __restrict__ ewo,
    const int32_t* __restrict__ widths, int E, int64_t hidden, int64_t rows,
    uint16_t* __restrict__ gw) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t nwaves = (int64_t)gridDim.x * kRowsPerBlock;
  for (int64_t base = ((int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave) * kWave;
       base < A; base += nwaves * kWave) {
    const int64_t a = base + lane;
    int32_t row = -1;
    bool tiny = false;
    if (a < A) {
      row = assignment_row[a];
      tiny = row >= 0 && row < rows && fabsf(row_weight[row]) < kTinyWeight;
    }
    uint64_t mask = ballot64(tiny);
    while (mask) {
      const int src = __builtin_ctzll(mask);
      mask &= mask - 1;
      const int32_t r = __shfl(row, src);
      const int64_t aa = base + src;
      const int64_t tok = aa / top_k;
      int lo = 0, hi = E;  // eto[lo] <= r < eto[hi]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (eto[mid] <= r) lo = mid; else hi = mid;
      }
      const int width = widths[lo];
      const int64_t col0 = ewo[lo];
      float s = 0.0f;
      if (tok < gy_rows) {
        const uint16_t* g = gy + tok * ldgy;
        const uint16_t* p = pre + (int64_t)r * ldp;
        for (int c = 0; c < width; ++c) {
          const uint16_t* wr = w2 + (col0 + c) * ldw2;
          float d = 0.0f;
          for (int64_t j = lane; j < hidden; j += kWave) d += bf16_to_f32(g[j]) * bf16_to_f32(wr[j]);
          d = wave_sum(d);
          const float pc = bf16_to_f32(p[c]);
          s += d * (pc * pc);
        }
      }
      if (grad_scale) s *= bf16_to_f32(*grad_scale);
      if (lane == 0) gw[aa] = (uint16_t)f32_to_bf16(s);
    }
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

inline int row_grid(int64_t rows) {
  const int64_t g = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  return (int)std::max<int64_t>(1, std::min<int64_t>(g, 65536));
}

}  // namespace
}  // namespace vmoe

using namespace vmoe;

extern "C" int vmoe_gather(const uint16_t* x, int64_t x_rows, int64_t ldx,
                           const int32_t* row_src, int32_t top_k, const uint16_t* weights,
                           int64_t num_weights, uint16_t* out, int64_t ldo, int64_t num_rows,
                           const int32_t* num_rows_dev, int64_t hidden, vmoe_stream_t stream) {
  if (num_rows < 0 || hidden < 0 || x_rows < 0 || top_k <= 0 || ldx < 0 || ldo < hidden)
    return VMOE_ERR_INVALID_ARG;
  if (num_rows == 0 || hidden == 0) return VMOE_OK;
  if (!out || !row_src || (x_rows > 0 && !x) || (weights && num_weights < 0))
    return VMOE_ERR_INVALID_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool vec = hidden % 8 == 0 && ldx % 8 == 0 && ldo % 8 == 0 && aligned16(x) &&
                   aligned16(out);
  const dim3 grid(row_grid(num_rows)), block(kThreads);
  if (vec) {
    if (weights)
      VMOE_LAUNCH((gather_kernel<8, true>), grid, block, 0, s, x, x_rows, ldx, row_src,
                         top_k, weights, num_weights, out, ldo, num_rows, num_rows_dev, hidden);
    else
      VMOE_LAUNCH((gather_kernel<8, false>), grid, block, 0, s, x, x_rows, ldx, row_src,
                         top_k, weights, num_weights, out, ldo, num_rows, num_rows_dev, hidden);
  } else {
    if (weights)
      VMOE_LAUNCH((gather_kernel<1, true>), grid, block, 0, s, x, x_rows, ldx, row_src,
                         top_k, weights, num_weights, out, ldo, num_rows, num_rows_dev, hidden);
    else
      VMOE_LAUNCH((gather_kernel<1, false>), grid, block, 0, s, x, x_rows, ldx, row_src,
                         top_k, weights, num_weights, out, ldo, num_rows, num_rows_dev, hidden);
  }
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

extern "C" int vmoe_gather_tokens(const uint16_t* x, int64_t ldx,
                                  const int32_t* assignment_row, int64_t num_tokens,
                                  int32_t top_k, const uint16_t* weights,
                                  const int32_t* row_src, uint16_t* out, int64_t ldo,
                                  int64_t num_rows, const int32_t* num_rows_dev, int64_t hidden,
                                  vmoe_stream_t stream) {
  if (num_rows < 0 || hidden < 0 || num_tokens < 0 || top_k <= 0 || top_k > kWave || ldx < 0 ||
      ldo < hidden)
    return VMOE_ERR_INVALID_ARG;
  if (num_rows == 0 || hidden == 0) return VMOE_OK;
  if (!out || !row_src || (num_tokens > 0 && (!x || !assignment_row)))
    return VMOE_ERR_INVALID_ARG;
  if (hidden % 8 != 0 || ldx % 8 != 0 || ldo % 8 != 0 || !aligned16(x) || !aligned16(out))
    return VMOE_ERR_UNSUPPORTED;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int tok_blocks = num_tokens > 0 ? std::min(row_grid(num_tokens), 8192) : 0;
  const int pad_blocks = (int)std::min<int64_t>(
      1024, std::max<int64_t>(1, (num_rows + kRowsPerBlock * kWave - 1) / (kRowsPerBlock * kWave)));
  const dim3 grid(tok_blocks + pad_blocks), block(kThreads);
  if (weights)
    VMOE_LAUNCH((gather_tokens_kernel<true, 2>), grid, block, 0, s, x, ldx,
                       assignment_row, num_tokens, top_k, weights, row_src, out, ldo, num_rows,
                       num_rows_dev, hidden, tok_blocks);
  else
    VMOE_LAUNCH((gather_tokens_kernel<false, 2>), grid, block, 0, s, x, ldx,
                       assignment_row, num_tokens, top_k, weights, row_src, out, ldo, num_rows,
                       num_rows_dev, hidden, tok_blocks);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

extern "C" int vmoe_combine(const uint16_t* y, int64_t y_rows, int64_t ldy,
                            const int32_t* assignment_row, const uint16_t* weights,
                            int32_t top_k, uint16_t* out, int64_t ldo, int64_t num_tokens,
                            int64_t hidden, vmoe_stream_t stream) {
  if (num_tokens < 0 || hidden < 0 || y_rows < 0 || top_k <= 0 || ldy < 0 || ldo < hidden)
    return VMOE_ERR_INVALID_ARG;
  if (num_tokens == 0 || hidden == 0) return VMOE_OK;
  if (!out || !assignment_row || (y_rows > 0 && !y)) return VMOE_ERR_INVALID_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool vec = hidden % 8 == 0 && ldy % 8 == 0 && ldo % 8 == 0 && aligned16(y) &&
                   aligned16(out);
  const dim3 grid(row_grid(num_tokens)), block(kThreads);
  if (vec && top_k <= 2) {
    // (fewer slot registers: more waves in flight for the short sums)
    if (weights)
      VMOE_LAUNCH((combine_k_kernel<2, true, 2>), grid, block, 0, s, y, y_rows, ldy,
                         assignment_row, weights, top_k, out, ldo, num_tokens, hidden);
    else
      VMOE_LAUNCH((combine_k_kernel<2, false, 2>), grid, block, 0, s, y, y_rows, ldy,
                         assignment_row, weights, top_k, out, ldo, num_tokens, hidden);
  } else if (vec && top_k <= 8) {
    if (weights)
      VMOE_LAUNCH((combine_k_kernel<8, true, 2>), grid, block, 0, s, y, y_rows, ldy,
                         assignment_row, weights, top_k, out, ldo, num_tokens, hidden);
    else
      VMOE_LAUNCH((combine_k_kernel<8, false, 2>), grid, block, 0, s, y, y_rows, ldy,
                         assignment_row, weights, top_k, out, ldo, num_tokens, hidden);
  } else if (vec) {
    // Two 16-byte chunks per lane cover d <= 1024 in one pass.
    if (weights)
      VMOE_LAUNCH((combine_kernel<8, true, 2>), grid, block, 0, s, y, y_rows, ldy,
                         assignment_row, weights, top_k, out, ldo, num_tokens, hidden);
    else
      VMOE_LAUNCH((combine_kernel<8, false, 2>), grid, block, 0, s, y, y_rows, ldy,
                         assignment_row, weights, top_k, out, ldo, num_tokens, hidden);
  } else {
    if (weights)
      VMOE_LAUNCH((combine_kernel<1, true, 4>), grid, block, 0, s, y, y_rows, ldy,
                         assignment_row, weights, top_k, out, ldo, num_tokens, hidden);
    else
      VMOE_LAUNCH((combine_kernel<1, false, 4>), grid, block, 0, s, y, y_rows, ldy,
                         assignment_row, weights, top_k, out, ldo, num_tokens, hidden);
  }
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

extern "C" int vmoe_combine_weight_grad(const uint16_t* grad, int64_t ldg, const uint16_t* y,
                                        int64_t y_rows, int64_t ldy,
                                        const int32_t* assignment_row, int32_t top_k,
                                        float* grad_weights, int64_t num_tokens, int64_t hidden,
                                        vmoe_stream_t stream) {
  if (num_tokens < 0 || hidden < 0 || y_rows < 0 || top_k <= 0 || ldy < 0 || ldg < 0)
    return VMOE_ERR_INVALID_ARG;
  if (num_tokens == 0) return VMOE_OK;
  if (!grad_weights || !assignment_row || (hidden > 0 && (!grad || (y_rows > 0 && !y))))
    return VMOE_ERR_INVALID_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool vec = hidden % 8 == 0 && ldy % 8 == 0 && ldg % 8 == 0 && aligned16(y) &&
                   aligned16(grad);
  const dim3 grid(row_grid(num_tokens)), block(kThreads);
  if (vec)
    VMOE_LAUNCH((combine_wgrad_kernel<8>), grid, block, 0, s, grad, ldg, y, y_rows, ldy,
                       assignment_row, top_k, grad_weights, num_tokens, hidden);
  else
    VMOE_LAUNCH((combine_wgrad_kernel<1>), grid, block, 0, s, grad, ldg, y, y_rows, ldy,
                       assignment_row, top_k, grad_weights, num_tokens, hidden);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

extern "C" int vmoe_routing_weight_grad(const float* row_dot, int64_t ld_row_dot,
                                        int32_t num_blocks, int64_t rows,
                                        const float* row_weight, const int32_t* assignment_row,
                                        int64_t num_assignments, uint16_t* grad_weights,
                                        vmoe_stream_t stream) {
  if (num_assignments < 0 || rows < 0 || num_blocks < 0 || ld_row_dot < num_blocks)
    return VMOE_ERR_INVALID_ARG;
  if (num_assignments == 0) return VMOE_OK;
  if (!grad_weights || !assignment_row || (rows > 0 && (!row_weight || (num_blocks > 0 && !row_dot))))
    return VMOE_ERR_INVALID_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t g = std::min<int64_t>((num_assignments + kThreads - 1) / kThreads, 65536);
  VMOE_LAUNCH(routing_wgrad_kernel, dim3((unsigned)g), dim3(kThreads), 0, s, row_dot,
                     ld_row_dot, num_blocks, rows, row_weight, assignment_row, num_assignments,
                     grad_weights);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

extern "C" int vmoe_routing_weight_grad_direct(
    const uint16_t* grad_y, int64_t ldgy, int64_t gy_rows, const uint16_t* grad_scale,
    const uint16_t* w2, int64_t ldw2, const uint16_t* pre_act, int64_t ld_pre,
    const float* row_weight,
    const int32_t* assignment_row, int64_t num_assignments, int32_t top_k, const int32_t* eto,
    const int32_t* ewo, const int32_t* widths, int32_t num_experts, int64_t hidden, int64_t rows,
    uint16_t* grad_weights, vmoe_stream_t stream) {
  if (num_assignments < 0 || rows < 0 || top_k <= 0 || num_experts <= 0 || hidden < 0 ||
      gy_rows < 0 || ldgy < 0 || ldw2 < hidden || ld_pre < 0)
    return VMOE_ERR_INVALID_ARG;
  if (num_assignments == 0 || rows == 0) return VMOE_OK;
  if (!grad_weights || !assignment_row || !row_weight || !eto || !ewo || !widths || !pre_act ||
      (hidden > 0 && (!w2 || (gy_rows > 0 && !grad_y))))
    return VMOE_ERR_INVALID_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t g = std::min<int64_t>((num_assignments + kThreads - 1) / kThreads, 65536);
  VMOE_LAUNCH(routing_wgrad_direct_kernel, dim3((unsigned)g), dim3(kThreads), 0, s,
                     grad_y, ldgy, gy_rows, grad_scale, w2, ldw2, pre_act, ld_pre, row_weight,
                     assignment_row, num_assignments, top_k, eto, ewo, widths, num_experts,
                     hidden, rows, grad_weights);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

extern "C" int vmoe_zero_tail_cols(uint16_t* buf, int64_t ld, const int32_t* eto,
                                   const int32_t* widths, int32_t E, int64_t max_width,
                                   int64_t rows_bound, vmoe_stream_t stream) {
  if (E <= 0 || max_width < 0 || rows_bound < 0 || ld < max_width) return VMOE_ERR_INVALID_ARG;
  if (rows_bound == 0 || max_width == 0) return VMOE_OK;
  if (!buf || !eto || !widths) return VMOE_ERR_INVALID_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  VMOE_LAUNCH(zero_tail_kernel, dim3(row_grid(rows_bound)), dim3(kThreads), 0, s, buf,
                     ld, eto, widths, E, max_width, rows_bound);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}
