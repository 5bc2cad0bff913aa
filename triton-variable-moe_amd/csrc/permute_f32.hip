// fp32 token permutation for the module in float32 (the reference's kernels
// are dtype-generic; a float32 TritonMoEMLP gathers, scatters and
// differentiates in fp32): the combine with or without routing weights,
// the row gather of the output gradient (weighted: the reference's
// padded_scatter backward, scatter.py:141-189), and the weight gradient of
// the weighted combine. Sums run in fp32 in slot order, as the reference's
// intermediate.sum(dim=1) (scatter.py:61-69, 133); rows move as 4-float
// vectors when every row start is 16-byte aligned, as single floats
// otherwise. One wave per output row.

#include <algorithm>

#include "vmoe_common.h"

namespace vmoe {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / kWave;

template <int VEC>
struct F32Vec;
template <>
struct F32Vec<4> {
  using T = float4;
  __device__ static T load(const float* p) { return *reinterpret_cast<const float4*>(p); }
  __device__ static void store(float* p, T v) { *reinterpret_cast<float4*>(p) = v; }
  __device__ static T zero() { return make_float4(0.0f, 0.0f, 0.0f, 0.0f); }
  // acc + round(v * s): the product is rounded before the sum (contraction
  // into a fused multiply-add is off here), as the reference's fp32
  // [T, k, d] slot values are.
  __device__ static void axpy(T& acc, T v, float s) {
#pragma clang fp contract(off)
    acc.x += v.x * s; acc.y += v.y * s; acc.z += v.z * s; acc.w += v.w * s;
  }
  __device__ static T scale(T v, float s) { return make_float4(v.x * s, v.y * s, v.z * s, v.w * s); }
  __device__ static float dot(T a, T b, float s) {
    s = fmaf(a.x, b.x, s); s = fmaf(a.y, b.y, s); s = fmaf(a.z, b.z, s);
    return fmaf(a.w, b.w, s);
  }
};
template <>
struct F32Vec<1> {
  using T = float;
  __device__ static T load(const float* p) { return *p; }
  __device__ static void store(float* p, T v) { *p = v; }
  __device__ static T zero() { return 0.0f; }
  __device__ static void axpy(T& acc, T v, float s) {
#pragma clang fp contract(off)
    acc += v * s;
  }
  __device__ static T scale(T v, float s) { return v * s; }
  __device__ static float dot(T a, T b, float s) { return fmaf(a, b, s); }
};

// out[t] = sum_j y[row(t, j)] * w[t*k+j] (w == nullptr: weight 1), j
// ascending, rows outside [0, y_rows) skipped.
template <int VEC>
__global__ __launch_bounds__(kThreads) void combine_f32_kernel(
    const float* __restrict__ y, int64_t y_rows, int64_t ldy,
    const int32_t* __restrict__ assignment_row, const float* __restrict__ w, int top_k,
    float* __restrict__ out, int64_t ldo, int64_t num_tokens, int64_t hidden) {
  using V = F32Vec<VEC>;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t nvec = hidden / VEC;
  for (int64_t t = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave; t < num_tokens;
       t += (int64_t)gridDim.x * kRowsPerBlock) {
    for (int64_t c = lane; c < nvec; c += kWave) {
      typename V::T acc = V::zero();
      for (int j = 0; j < top_k; ++j) {
        const int64_t a = t * top_k + j;
        const int32_t row = assignment_row[a];
        if (row < 0 || row >= y_rows) continue;
        V::axpy(acc, V::load(y + (int64_t)row * ldy + c * VEC), w ? w[a] : 1.0f);
      }
      V::store(out + t * ldo + c * VEC, acc);
    }
  }
}

// out[r] = x[row_src[r] / top_k] * w[row_src[r]] (w == nullptr: weight 1),
// zeros where row_src[r] < 0 or the token is past x_rows; ldx = 0 reads one
// row for every token.
template <int VEC>
__global__ __launch_bounds__(kThreads) void gather_f32_kernel(
    const float* __restrict__ x, int64_t x_rows, int64_t ldx, const int32_t* __restrict__ row_src,
    int top_k, const float* __restrict__ w, int64_t nw, float* __restrict__ out, int64_t ldo,
    int64_t num_rows, const int32_t* __restrict__ num_rows_dev, int64_t hidden) {
  using V = F32Vec<VEC>;
  const int lane = threadIdx.x & (kWave - 1);
  int64_t rows = num_rows;
  if (num_rows_dev) rows = min(rows, (int64_t)*num_rows_dev);
  const int64_t nvec = hidden / VEC;
  for (int64_t r = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave; r < rows;
       r += (int64_t)gridDim.x * kRowsPerBlock) {
    const int32_t s = row_src[r];
    const int64_t t = s >= 0 ? s / top_k : -1;
    const bool live = s >= 0 && t < x_rows && (!w || s < nw);
    float* orow = out + r * ldo;
    if (!live) {
      for (int64_t c = lane; c < nvec; c += kWave) V::store(orow + c * VEC, V::zero());
      continue;
    }
    const float scale = w ? w[s] : 1.0f;
    const float* xrow = x + t * ldx;
    for (int64_t c = lane; c < nvec; c += kWave)
      V::store(orow + c * VEC, V::scale(V::load(xrow + c * VEC), scale));
  }
}

// gw[t*k+j] = sum_c g[t, c] * y[row(t, j), c] (fp32, each lane's columns in
// order, then a butterfly over the wave), 0 for slots with no row.
template <int VEC>
__global__ __launch_bounds__(kThreads) void combine_wgrad_f32_kernel(
    const float* __restrict__ g, int64_t ldg, const float* __restrict__ y, int64_t y_rows,
    int64_t ldy, const int32_t* __restrict__ assignment_row, int top_k, float* __restrict__ gw,
    int64_t num_tokens, int64_t hidden) {
  using V = F32Vec<VEC>;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t nvec = hidden / VEC;
  for (int64_t t = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave; t < num_tokens;
       t += (int64_t)gridDim.x * kRowsPerBlock) {
    const float* grow = g + t * ldg;
    for (int j = 0; j < top_k; ++j) {
      const int64_t a = t * top_k + j;
      const int32_t row = assignment_row[a];
      float s = 0.0f;
      if (row >= 0 && row < y_rows) {
        const float* yrow = y + (int64_t)row * ldy;
        for (int64_t c = lane; c < nvec; c += kWave)
          s = V::dot(V::load(grow + c * VEC), V::load(yrow + c * VEC), s);
      }
#pragma unroll
      for (int off = kWave / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, kWave);
      if (lane == 0) gw[a] = s;
    }
  }
}

inline bool vec4_ok(const float* p, int64_t ld, int64_t hidden) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && ld % 4 == 0 && hidden % 4 == 0;
}

inline int row_grid(int64_t rows) {
  const int64_t g = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  return (int)std::max<int64_t>(1, std::min<int64_t>(g, 65536));
}

}  // namespace
}  // namespace vmoe

using namespace vmoe;

extern "C" int vmoe_combine_f32(const float* y, int64_t y_rows, int64_t ldy,
                                const int32_t* assignment_row, const float* weights,
                                int32_t top_k, float* out, int64_t ldo, int64_t num_tokens,
                                int64_t hidden, vmoe_stream_t stream) {
  if (num_tokens < 0 || hidden < 0 || y_rows < 0 || top_k <= 0 || ldy < hidden || ldo < hidden)
    return VMOE_ERR_INVALID_ARG;
  if (num_tokens == 0 || hidden == 0) return VMOE_OK;
  if (!out || !assignment_row || (y_rows > 0 && !y)) return VMOE_ERR_INVALID_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(row_grid(num_tokens)), block(kThreads);
  if ((y_rows == 0 || vec4_ok(y, ldy, hidden)) && vec4_ok(out, ldo, hidden))
    VMOE_LAUNCH(combine_f32_kernel<4>, grid, block, 0, s, y, y_rows, ldy, assignment_row,
                       weights, top_k, out, ldo, num_tokens, hidden);
  else
    VMOE_LAUNCH(combine_f32_kernel<1>, grid, block, 0, s, y, y_rows, ldy, assignment_row,
                       weights, top_k, out, ldo, num_tokens, hidden);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

extern "C" int vmoe_gather_f32(const float* x, int64_t x_rows, int64_t ldx,
                               const int32_t* row_src, int32_t top_k, const float* weights,
                               int64_t num_weights, float* out, int64_t ldo, int64_t num_rows,
                               const int32_t* num_rows_dev, int64_t hidden,
                               vmoe_stream_t stream) {
  if (num_rows < 0 || hidden < 0 || x_rows < 0 || top_k <= 0 || ldx < 0 || ldo < hidden ||
      (weights && num_weights < 0))
    return VMOE_ERR_INVALID_ARG;
  if (num_rows == 0 || hidden == 0) return VMOE_OK;
  if (!out || !row_src || (x_rows > 0 && !x)) return VMOE_ERR_INVALID_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(row_grid(num_rows)), block(kThreads);
  if ((x_rows == 0 || vec4_ok(x, ldx, hidden)) && vec4_ok(out, ldo, hidden))
    VMOE_LAUNCH(gather_f32_kernel<4>, grid, block, 0, s, x, x_rows, ldx, row_src, top_k,
                       weights, num_weights, out, ldo, num_rows, num_rows_dev, hidden);
  else
    VMOE_LAUNCH(gather_f32_kernel<1>, grid, block, 0, s, x, x_rows, ldx, row_src, top_k,
                       weights, num_weights, out, ldo, num_rows, num_rows_dev, hidden);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

extern "C" int vmoe_combine_weight_grad_f32(const float* grad, int64_t ldg, const float* y,
                                            int64_t y_rows, int64_t ldy,
                                            const int32_t* assignment_row, int32_t top_k,
                                            float* grad_weights, int64_t num_tokens,
                                            int64_t hidden, vmoe_stream_t stream) {
  if (num_tokens < 0 || hidden < 0 || y_rows < 0 || top_k <= 0 || ldg < 0 || ldy < hidden)
    return VMOE_ERR_INVALID_ARG;
  if (num_tokens == 0) return VMOE_OK;
  if (!grad_weights || !assignment_row || (hidden > 0 && (!grad || (y_rows > 0 && !y))))
    return VMOE_ERR_INVALID_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(row_grid(num_tokens)), block(kThreads);
  if (vec4_ok(grad, ldg, hidden) && (y_rows == 0 || vec4_ok(y, ldy, hidden)))
    VMOE_LAUNCH(combine_wgrad_f32_kernel<4>, grid, block, 0, s, grad, ldg, y, y_rows, ldy,
                       assignment_row, top_k, grad_weights, num_tokens, hidden);
  else
    VMOE_LAUNCH(combine_wgrad_f32_kernel<1>, grid, block, 0, s, grad, ldg, y, y_rows, ldy,
                       assignment_row, top_k, grad_weights, num_tokens, hidden);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}
