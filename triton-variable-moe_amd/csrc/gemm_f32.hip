// fp32 grouped GEMMs: the float32 inputs of the public grouped-GEMM API.
//
// The reference's grouped-GEMM kernels take fp32 as well as bf16 operands
// (triton_moe/kernels/grouped_gemm.py:217-1162, dtype-generic tl.dot with an
// fp32 accumulator); its autograd tests and forward/backward benchmark run
// them in fp32 (tests/test_grouped_gemm_backward.py:151-208). The bf16 kernels
// of gemm.hip stage bf16 tiles for MFMA and cannot take fp32, so this file
// holds one LDS-tiled fp32 VALU kernel for all six forms (up forward with its
// activation, down forward, and both backward GEMMs of each). Every product
// is an fp32 fma in k order per output, outputs are stored in fp32, and the
// activation gradients (relu^2, SwiGLU's [dG | dU]) are formed from
// grad/pre/up as the operand tile is loaded, as the reference's backward
// kernels do (grouped_gemm.py:751-764, 914-927), so no launch sits between
// the GEMMs. This is the path for fp32 callers; the bf16 module path never
// uses it.
//
// Tiles: 64 x 64 outputs per 256-thread workgroup, 4 x 4 per thread (4
// consecutive rows by 4 consecutive columns), k steps of 16 staged in LDS, each thread loading runs of 4 consecutive elements
// (16-byte loads where the address is aligned and the run in range). Workgroups stride over the experts' tiles in order,
// read from the metadata on the device (no host sync).
#include <algorithm>

#include "vmoe_common.h"

namespace vmoe {
namespace {

enum F32Form { F_UP_FWD, F_DOWN_FWD, F_UP_DX, F_UP_DW, F_DOWN_DH, F_DOWN_DW };

constexpr int kT = 64;        // tile edge
constexpr int kBK = 16;       // k per LDS stage
constexpr int kThreads = 256;
constexpr int kPad = kT + 4;  // LDS row length (floats)

struct F32Args {
  // token-row operand: x (up forms), h (down forms) or grad_y (dH)
  const float* a;
  int64_t lda, a_rows;
  const int32_t* a_map;  // x rows through a gather map (up forms), may be null
  // weights: w1 or w2 (forward, dX and dH), or grad_y (down dW)
  const float* b;
  int64_t ldb;
  // gradient of the up projection's output with pre (relu(z) or the gate)
  // and up (SwiGLU), all [rows, max_width] with leading dimension ldg
  const float *g, *pre, *up;
  int64_t ldg;
  float *c, *c2, *c3;
  int64_t ldc;
  const int32_t *eto, *ewo, *widths, *tpe;
  int E, act;
  int64_t hidden, max_width, rows_bound;
};

struct F32Prob {
  int64_t M, N, K, t0, w0, w;
};

__device__ __forceinline__ int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Rows of expert e: [t0, t0 + rows), rows = min(tpe, eto[e+1] - eto[e]) and
// inside [0, rows_bound).
template <int F>
__device__ F32Prob f32_prob(const F32Args& p, int e) {
  F32Prob q;
  const int64_t t0 = p.eto[e];
  const int64_t t1 = min((int64_t)p.eto[e + 1], p.rows_bound);
  int64_t rows = min((int64_t)p.tpe[e], t1 - t0);
  if (t0 < 0 || rows < 0) rows = 0;
  const int64_t w = max((int64_t)0, min((int64_t)p.widths[e], p.max_width));
  // the SwiGLU backward GEMMs run over the expert's gate and up columns
  const int64_t wg = p.act == VMOE_ACT_SWIGLU ? 2 * w : w;
  q.t0 = t0;
  q.w0 = p.ewo[e];
  q.w = w;
  switch (F) {
    case F_UP_FWD: q.M = rows; q.N = w; q.K = p.hidden; break;
    case F_DOWN_FWD: q.M = rows; q.N = p.hidden; q.K = w; break;
    case F_UP_DX: q.M = rows; q.N = p.hidden; q.K = wg; break;
    case F_UP_DW: q.M = p.hidden; q.N = wg; q.K = rows; break;
    case F_DOWN_DH: q.M = rows; q.N = w; q.K = p.hidden; break;
    default: q.M = w; q.N = p.hidden; q.K = rows; break;  // F_DOWN_DW
  }
  return q;
}

__device__ __forceinline__ float sigmoid32(float v) { return 1.0f / (1.0f + expf(-v)); }

// The gradient w.r.t. the up projection's pre-activation at row r, column c
// (c < 2w for SwiGLU: c < w is the gate's, c >= w the up half's).
__device__ __forceinline__ float act_grad(const F32Args& p, int64_t r, int64_t c, int64_t w) {
  if (p.act == VMOE_ACT_SWIGLU) {
    const int64_t cc = c < w ? c : c - w;
    const int64_t o = r * p.ldg + cc;
    const float gr = p.g[o], gate = p.pre[o], s = sigmoid32(gate);
    return c < w ? gr * p.up[o] * s * (1.0f + gate * (1.0f - s)) : gr * gate * s;
  }
  const int64_t o = r * p.ldg + c;
  const float gr = p.g[o];
  if (p.act == VMOE_ACT_RELU_SQUARED) {
    const float pr = p.pre[o];
    return pr > 0.0f ? gr * 2.0f * pr : 0.0f;
  }
  return gr;
}

// x row of padded row r (through the gather map when there is one; a map
// entry outside [0, a_rows) reads zeros).
__device__ __forceinline__ const float* token_row(const F32Args& p, int64_t r) {
  if (!p.a_map) return p.a + r * p.lda;
  const int64_t s = p.a_map[r];
  return s >= 0 && s < p.a_rows ? p.a + s * p.lda : nullptr;
}

// A(m, k) of the tile's problem (0 outside M x K).
template <int F>
__device__ __forceinline__ float f32_a(const F32Args& p, const F32Prob& q, int64_t m, int64_t k) {
  if (m >= q.M || k >= q.K) return 0.0f;
  switch (F) {
    case F_UP_FWD: {
      const float* row = token_row(p, q.t0 + m);
      return row ? row[k] : 0.0f;
    }
    case F_DOWN_FWD:
    case F_DOWN_DH: return p.a[(q.t0 + m) * p.lda + k];
    case F_UP_DX: return act_grad(p, q.t0 + m, k, q.w);
    case F_UP_DW: {
      const float* row = token_row(p, q.t0 + k);
      return row ? row[m] : 0.0f;
    }
    default: return p.a[(q.t0 + k) * p.lda + m];  // F_DOWN_DW: h^T
  }
}

// B(k, n); `second` selects the SwiGLU up half of W1 in the up forward.
template <int F>
__device__ __forceinline__ float f32_b(const F32Args& p, const F32Prob& q, int64_t k, int64_t n,
                                       bool second) {
  if (k >= q.K || n >= q.N) return 0.0f;
  switch (F) {
    case F_UP_FWD: return p.b[k * p.ldb + q.w0 + (second ? q.w : 0) + n];
    case F_DOWN_FWD: return p.b[(q.w0 + k) * p.ldb + n];
    case F_UP_DX: return p.b[n * p.ldb + q.w0 + k];  // W1^T
    case F_UP_DW: return act_grad(p, q.t0 + k, n, q.w);
    case F_DOWN_DH: return p.b[(q.w0 + n) * p.ldb + k];  // W2^T
    default: return p.b[(q.t0 + k) * p.ldb + n];  // F_DOWN_DW: grad_y
  }
}

// Whether A / B are contiguous along k (decides which thread loads what).
template <int F>
constexpr bool a_k_contig() { return F == F_UP_FWD || F == F_DOWN_FWD || F == F_UP_DX || F == F_DOWN_DH; }
template <int F>
constexpr bool b_k_contig() { return F == F_UP_DX || F == F_DOWN_DH; }

// Four consecutive floats from ptr of which `valid` are in range (the rest
// read as 0): one 16-byte load when all four are and the address allows it.
__device__ __forceinline__ float4 load_run(const float* ptr, int64_t valid) {
  float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (!ptr || valid <= 0) return v;
  if (valid >= 4 && (reinterpret_cast<uintptr_t>(ptr) & 15) == 0)
    return *reinterpret_cast<const float4*>(ptr);
  v.x = ptr[0];
  if (valid > 1) v.y = ptr[1];
  if (valid > 2) v.z = ptr[2];
  if (valid > 3) v.w = ptr[3];
  return v;
}

// Four elements of A from (m, k) along its contiguous dimension (k for the
// K-contiguous forms, m otherwise); not for up dX, whose A is the
// activation gradient (stage_elem).
template <int F>
__device__ __forceinline__ float4 f32_a_run(const F32Args& p, const F32Prob& q, int64_t m,
                                            int64_t k) {
  const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  switch (F) {
    case F_UP_FWD: {
      if (m >= q.M) return z;
      const float* row = token_row(p, q.t0 + m);
      return load_run(row ? row + k : nullptr, q.K - k);
    }
    case F_DOWN_FWD:
    case F_DOWN_DH:
      return m < q.M ? load_run(p.a + (q.t0 + m) * p.lda + k, q.K - k) : z;
    case F_UP_DW: {
      if (k >= q.K) return z;
      const float* row = token_row(p, q.t0 + k);
      return load_run(row ? row + m : nullptr, q.M - m);
    }
    default:  // F_DOWN_DW: h^T
      return k < q.K ? load_run(p.a + (q.t0 + k) * p.lda + m, q.M - m) : z;
  }
}

// Four elements of B from (k, n) along its contiguous dimension (k for up dX
// and down dH, n otherwise); not for up dW, whose B is the activation
// gradient (stage_elem).
template <int F>
__device__ __forceinline__ float4 f32_b_run(const F32Args& p, const F32Prob& q, int64_t k,
                                            int64_t n, bool second) {
  const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  switch (F) {
    case F_UP_FWD:
      return k < q.K ? load_run(p.b + k * p.ldb + q.w0 + (second ? q.w : 0) + n, q.N - n) : z;
    case F_DOWN_FWD:
      return k < q.K ? load_run(p.b + (q.w0 + k) * p.ldb + n, q.N - n) : z;
    case F_UP_DX:  // W1^T
      return n < q.N ? load_run(p.b + n * p.ldb + q.w0 + k, q.K - k) : z;
    case F_DOWN_DH:  // W2^T
      return n < q.N ? load_run(p.b + (q.w0 + n) * p.ldb + k, q.K - k) : z;
    default:  // F_DOWN_DW: grad_y
      return k < q.K ? load_run(p.b + (q.t0 + k) * p.ldb + n, q.N - n) : z;
  }
}

// Loads a kBK x kT stage into lds[k][x] element by element, consecutive
// lanes along the operand's contiguous dimension (the activation-gradient
// operands, formed per element).
template <bool KCONTIG, typename Fn>
__device__ __forceinline__ void stage_elem(float (*lds)[kPad], Fn&& at) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int k, x;
    if (KCONTIG) {
      k = tid & (kBK - 1);
      x = (tid >> 4) + 16 * i;
    } else {
      x = tid & (kT - 1);
      k = (tid >> 6) + 4 * i;
    }
    lds[k][x] = at(k, x);
  }
}

// Loads a kBK x kT stage into lds[k][x]: one run of 4 elements per thread
// along the operand's contiguous dimension (k when KCONTIG, x otherwise).
template <bool KCONTIG, typename Fn>
__device__ __forceinline__ void stage(float (*lds)[kPad], Fn&& run) {
  const int tid = threadIdx.x;
  if (KCONTIG) {
    const int x = tid >> 2, k = (tid & 3) * 4;
    const float4 v = run(k, x);
    lds[k][x] = v.x;
    lds[k + 1][x] = v.y;
    lds[k + 2][x] = v.z;
    lds[k + 3][x] = v.w;
  } else {
    const int x = (tid & 15) * 4, k = tid >> 4;
    const float4 v = run(k, x);
    lds[k][x] = v.x;
    lds[k][x + 1] = v.y;
    lds[k][x + 2] = v.z;
    lds[k][x + 3] = v.w;
  }
}

// GLU: the SwiGLU up forward (a second accumulator over the up columns); its
// own instance, so the other forms do not carry its registers.
template <int F, bool GLU>
__global__ __launch_bounds__(kThreads) void grouped_gemm_f32_kernel(F32Args p) {
  __shared__ __align__(16) float As[kBK][kPad];
  __shared__ __align__(16) float Bs[kBK][kPad];
  __shared__ __align__(16) float Us[GLU ? kBK : 1][kPad];  // SwiGLU up half
  constexpr bool glu = GLU && F == F_UP_FWD;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  int e = 0;
  int64_t before = 0;  // tiles of experts < e
  F32Prob q{};
  int64_t tiles = 0, tn_count = 1;
  bool have = false;
  for (int64_t t = blockIdx.x;; t += gridDim.x) {
    // experts are visited in order and t only grows, so one pass over them
    while (true) {
      if (!have) {
        if (e >= p.E) break;
        q = f32_prob<F>(p, e);
        tn_count = cdiv64(q.N, kT);
        tiles = cdiv64(q.M, kT) * tn_count;
        have = true;
      }
      if (t < before + tiles) break;
      before += tiles;
      ++e;
      have = false;
    }
    if (!have) break;
    const int64_t local = t - before;
    const int64_t m0 = (local / tn_count) * kT, n0 = (local % tn_count) * kT;
    float acc[4][4] = {}, acc_up[glu ? 4 : 1][4] = {};
    for (int64_t k0 = 0; k0 < q.K; k0 += kBK) {
      if constexpr (F == F_UP_DX)
        stage_elem<true>(As, [&](int k, int x) { return f32_a<F>(p, q, m0 + x, k0 + k); });
      else
        stage<a_k_contig<F>()>(As, [&](int k, int x) { return f32_a_run<F>(p, q, m0 + x, k0 + k); });
      if constexpr (F == F_UP_DW)
        stage_elem<false>(Bs, [&](int k, int x) { return f32_b<F>(p, q, k0 + k, n0 + x, false); });
      else
        stage<b_k_contig<F>()>(Bs, [&](int k, int x) {
          return f32_b_run<F>(p, q, k0 + k, n0 + x, false);
        });
      if constexpr (glu)
        stage<false>(Us, [&](int k, int x) { return f32_b_run<F>(p, q, k0 + k, n0 + x, true); });
      __syncthreads();
#pragma unroll
      for (int k = 0; k < kBK; ++k) {
        // each thread's 4 rows / 4 columns are consecutive: one 16-byte LDS
        // read per operand (the 16 lanes of a row group read 256 contiguous
        // bytes of B, and share one address of A)
        const float4 av = *reinterpret_cast<const float4*>(&As[k][4 * ty]);
        const float4 bv = *reinterpret_cast<const float4*>(&Bs[k][4 * tx]);
        const float a[4] = {av.x, av.y, av.z, av.w};
        float b[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
        if constexpr (glu) {
          const float4 uv = *reinterpret_cast<const float4*>(&Us[k][4 * tx]);
          b[0] = uv.x; b[1] = uv.y; b[2] = uv.z; b[3] = uv.w;
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc_up[i][j] = fmaf(a[i], b[j], acc_up[i][j]);
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t m = m0 + 4 * ty + i;
      if (m >= q.M) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t n = n0 + 4 * tx + j;
        if (n >= q.N) continue;
        const float z = acc[i][j];
        if (F == F_UP_DW) {
          p.c[m * p.ldc + q.w0 + n] = z;
        } else if (F == F_DOWN_DW) {
          p.c[(q.w0 + m) * p.ldc + n] = z;
        } else {
          const int64_t o = (q.t0 + m) * p.ldc + n;
          if (F == F_UP_FWD && p.act == VMOE_ACT_RELU_SQUARED) {
            const float r = fmaxf(z, 0.0f);
            if (p.c2) p.c2[o] = r;
            p.c[o] = r * r;
          } else if constexpr (glu) {
            const float u = acc_up[i][j];
            if (p.c2) p.c2[o] = z;
            if (p.c3) p.c3[o] = u;
            if (p.c) p.c[o] = z * sigmoid32(z) * u;
          } else {
            p.c[o] = z;
          }
        }
      }
    }
  }
}

// Upper bound of the tiles of one launch (sizes the grid; workgroups past
// the real count leave at once).
int64_t tile_bound(int64_t E, int64_t m_bound, int64_t n_bound, bool rows_m) {
  const int64_t tn = (n_bound + kT - 1) / kT;
  const int64_t tm = rows_m ? (m_bound + kT - 1) / kT + E : E * ((m_bound + kT - 1) / kT);
  return tm * tn;
}

template <int F, bool GLU = false>
int f32_launch(const F32Args& p, int64_t bound, hipStream_t s) {
  if (bound <= 0 || p.rows_bound == 0 || p.max_width == 0) return VMOE_OK;  // no work
  const int64_t grid = bound < 2048 ? bound : 2048;
  VMOE_LAUNCH((grouped_gemm_f32_kernel<F, GLU>), dim3((unsigned)grid), dim3(kThreads), 0, s,
                     p);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

int f32_common(const int32_t* eto, const int32_t* ewo, const int32_t* widths,
               const int32_t* tpe, int32_t E, int64_t hidden, int64_t max_width,
               int64_t rows_bound) {
  if (!eto || !ewo || !widths || !tpe || E <= 0 || hidden <= 0 || max_width < 0 ||
      rows_bound < 0)
    return VMOE_ERR_INVALID_ARG;
  return VMOE_OK;
}

F32Args f32_args(const int32_t* eto, const int32_t* ewo, const int32_t* widths,
                 const int32_t* tpe, int32_t E, int64_t hidden, int64_t max_width,
                 int64_t rows_bound, int act) {
  F32Args p{};
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.act = act; p.hidden = hidden; p.max_width = max_width; p.rows_bound = rows_bound;
  return p;
}

bool act_ok(int act) {
  return act == VMOE_ACT_NONE || act == VMOE_ACT_RELU_SQUARED || act == VMOE_ACT_SWIGLU;
}

// grad/pre/up of the backward GEMMs: pre is needed for relu^2, pre and up
// for SwiGLU.
bool grad_ok(const float* g, const float* pre, const float* up, int64_t ldg, int64_t max_width,
             int act) {
  if (!g || ldg < max_width || ldg <= 0) return false;
  if (act == VMOE_ACT_RELU_SQUARED && !pre) return false;
  if (act == VMOE_ACT_SWIGLU && (!pre || !up)) return false;
  return true;
}

__global__ __launch_bounds__(256) void f32_relu2_grad_kernel(const float* g, const float* pre,
                                                             int64_t ld, float* ga, int64_t ldo,
                                                             int64_t rows, int64_t cols) {
  const int64_t n = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cols, c = i - r * cols;
    const float pr = pre[r * ld + c];
    ga[r * ldo + c] = pr > 0.0f ? g[r * ld + c] * 2.0f * pr : 0.0f;
  }
}

}  // namespace
}  // namespace vmoe

using namespace vmoe;

extern "C" int vmoe_f32_relu2_grad(const float* grad_h, const float* pre_act, int64_t ld,
                                   float* grad_act, int64_t ldo, int64_t rows, int64_t cols,
                                   vmoe_stream_t stream) {
  if (rows < 0 || cols < 0 || ld < cols || ldo < cols) return VMOE_ERR_INVALID_ARG;
  if (rows == 0 || cols == 0) return VMOE_OK;
  if (!grad_h || !pre_act || !grad_act) return VMOE_ERR_INVALID_ARG;
  const int64_t n = rows * cols;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 8192);
  VMOE_LAUNCH(f32_relu2_grad_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), grad_h, pre_act, ld, grad_act, ldo,
                     rows, cols);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

extern "C" int vmoe_gemm_f32_up_fwd(const float* x, int64_t ldx, int64_t x_rows,
                                    const int32_t* gather_map, const float* w1, int64_t ldw1,
                                    float* out, float* pre_act, float* up, int64_t ldo,
                                    int32_t activation, const int32_t* eto, const int32_t* ewo,
                                    const int32_t* widths, const int32_t* tpe, int32_t E,
                                    int64_t hidden, int64_t max_width, int64_t rows_bound,
                                    vmoe_stream_t stream) {
  int st = f32_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (!act_ok(activation) || !x || !w1 || x_rows < 0 || ldx < hidden || ldw1 <= 0 ||
      ldo < max_width || ldo <= 0)
    return VMOE_ERR_INVALID_ARG;
  if (!out && !(activation == VMOE_ACT_SWIGLU && (pre_act || up))) return VMOE_ERR_INVALID_ARG;
  F32Args p = f32_args(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound, activation);
  p.a = x; p.lda = ldx; p.a_rows = x_rows; p.a_map = gather_map;
  p.b = w1; p.ldb = ldw1;
  p.c = out; p.ldc = ldo;
  p.c2 = activation == VMOE_ACT_NONE ? nullptr : pre_act;
  p.c3 = activation == VMOE_ACT_SWIGLU ? up : nullptr;
  const int64_t bound = tile_bound(E, rows_bound, max_width, true);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  return activation == VMOE_ACT_SWIGLU ? f32_launch<F_UP_FWD, true>(p, bound, s)
                                       : f32_launch<F_UP_FWD>(p, bound, s);
}

extern "C" int vmoe_gemm_f32_down_fwd(const float* h, int64_t ldh, const float* w2, int64_t ldw2,
                                      float* y, int64_t ldy, const int32_t* eto,
                                      const int32_t* ewo, const int32_t* widths,
                                      const int32_t* tpe, int32_t E, int64_t hidden,
                                      int64_t max_width, int64_t rows_bound,
                                      vmoe_stream_t stream) {
  int st = f32_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (!h || !w2 || !y || ldh < max_width || ldh <= 0 || ldw2 < hidden || ldy < hidden)
    return VMOE_ERR_INVALID_ARG;
  F32Args p = f32_args(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound, VMOE_ACT_NONE);
  p.a = h; p.lda = ldh;
  p.b = w2; p.ldb = ldw2;
  p.c = y; p.ldc = ldy;
  return f32_launch<F_DOWN_FWD>(p, tile_bound(E, rows_bound, hidden, true),
                                reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vmoe_gemm_f32_up_bwd_dx(const float* grad_h, const float* pre_act,
                                       const float* up, int64_t ldg, int32_t activation,
                                       const float* w1, int64_t ldw1, float* grad_x,
                                       int64_t ldgx, const int32_t* eto, const int32_t* ewo,
                                       const int32_t* widths, const int32_t* tpe, int32_t E,
                                       int64_t hidden, int64_t max_width, int64_t rows_bound,
                                       vmoe_stream_t stream) {
  int st = f32_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (!act_ok(activation) || !grad_ok(grad_h, pre_act, up, ldg, max_width, activation) || !w1 ||
      ldw1 <= 0 || !grad_x || ldgx < hidden)
    return VMOE_ERR_INVALID_ARG;
  F32Args p = f32_args(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound, activation);
  p.g = grad_h; p.pre = pre_act; p.up = up; p.ldg = ldg;
  p.b = w1; p.ldb = ldw1;
  p.c = grad_x; p.ldc = ldgx;
  return f32_launch<F_UP_DX>(p, tile_bound(E, rows_bound, hidden, true),
                             reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vmoe_gemm_f32_up_bwd_dw(const float* x, int64_t ldx, int64_t x_rows,
                                       const int32_t* gather_map, const float* grad_h,
                                       const float* pre_act, const float* up, int64_t ldg,
                                       int32_t activation, float* grad_w1, int64_t ldgw,
                                       const int32_t* eto, const int32_t* ewo,
                                       const int32_t* widths, const int32_t* tpe, int32_t E,
                                       int64_t hidden, int64_t max_width, int64_t rows_bound,
                                       vmoe_stream_t stream) {
  int st = f32_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (!act_ok(activation) || !grad_ok(grad_h, pre_act, up, ldg, max_width, activation) || !x ||
      x_rows < 0 || ldx < hidden || !grad_w1 || ldgw <= 0)
    return VMOE_ERR_INVALID_ARG;
  F32Args p = f32_args(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound, activation);
  p.a = x; p.lda = ldx; p.a_rows = x_rows; p.a_map = gather_map;
  p.g = grad_h; p.pre = pre_act; p.up = up; p.ldg = ldg;
  p.c = grad_w1; p.ldc = ldgw;
  const int64_t n_bound = activation == VMOE_ACT_SWIGLU ? 2 * max_width : max_width;
  return f32_launch<F_UP_DW>(p, tile_bound(E, hidden, n_bound, false),
                             reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vmoe_gemm_f32_down_bwd_dh(const float* grad_y, int64_t ldgy, const float* w2,
                                         int64_t ldw2, float* grad_h, int64_t ldgh,
                                         const int32_t* eto, const int32_t* ewo,
                                         const int32_t* widths, const int32_t* tpe, int32_t E,
                                         int64_t hidden, int64_t max_width, int64_t rows_bound,
                                         vmoe_stream_t stream) {
  int st = f32_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (!grad_y || ldgy < hidden || !w2 || ldw2 < hidden || !grad_h || ldgh < max_width ||
      ldgh <= 0)
    return VMOE_ERR_INVALID_ARG;
  F32Args p = f32_args(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound, VMOE_ACT_NONE);
  p.a = grad_y; p.lda = ldgy;
  p.b = w2; p.ldb = ldw2;
  p.c = grad_h; p.ldc = ldgh;
  return f32_launch<F_DOWN_DH>(p, tile_bound(E, rows_bound, max_width, true),
                               reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vmoe_gemm_f32_down_bwd_dw(const float* h, int64_t ldh, const float* grad_y,
                                         int64_t ldgy, float* grad_w2, int64_t ldgw,
                                         const int32_t* eto, const int32_t* ewo,
                                         const int32_t* widths, const int32_t* tpe, int32_t E,
                                         int64_t hidden, int64_t max_width, int64_t rows_bound,
                                         vmoe_stream_t stream) {
  int st = f32_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (!h || ldh < max_width || ldh <= 0 || !grad_y || ldgy < hidden || !grad_w2 ||
      ldgw < hidden)
    return VMOE_ERR_INVALID_ARG;
  F32Args p = f32_args(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound, VMOE_ACT_NONE);
  p.a = h; p.lda = ldh;
  p.b = grad_y; p.ldb = ldgy;
  p.c = grad_w2; p.ldc = ldgw;
  return f32_launch<F_DOWN_DW>(p, tile_bound(E, max_width, hidden, false),
                               reinterpret_cast<hipStream_t>(stream));
}
