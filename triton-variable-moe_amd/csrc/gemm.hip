// Variable-width grouped GEMMs on gfx950 bf16 MFMA (v_mfma_f32_32x32x16_bf16).
//
// One kernel template serves the six GEMMs of the MoE MLP (up/down forward,
// their dX and dW backward). Each is C_e = A_e @ B_e per expert e with the
// operand placement given by the variant's traits below; the math is that of
// the reference kernels:
//   UP_FWD   _grouped_gemm_up_kernel                 (triton_moe/kernels/grouped_gemm.py:212-368)
//   DOWN_FWD _grouped_gemm_down_kernel               (grouped_gemm.py:480-583)
//   UP_DX    _grouped_gemm_up_backward_dx_kernel     (grouped_gemm.py:654-802)
//   UP_DW    _grouped_gemm_up_backward_dw_kernel     (grouped_gemm.py:805-967)
//   DOWN_DH  _grouped_gemm_down_backward_dintermediate_kernel (grouped_gemm.py:970-1063)
//   DOWN_DW  _grouped_gemm_down_backward_dw_kernel   (grouped_gemm.py:1066-1162)
//
// Design:
//  * Tile scheduler on the device: the grid is an upper bound of the tile
//    count; each workgroup scans the per-expert tile counts (from the same
//    metadata the reference reads) in LDS and finds its (expert, tile), so no
//    host sync is needed and empty experts cost nothing. Workgroup ids are
//    remapped so that consecutive tiles (same expert, same weight slice) run on
//    the same XCD and share its L2.
//  * 256 threads = 4 waves in a 2x2 grid, each wave owns a (BM/2)x(BN/2) block
//    of 32x32 MFMA accumulators (fp32).
//  * Operands are staged through double-buffered LDS in K-contiguous form,
//    which is what the MFMA fragments want (8 consecutive k per lane, one
//    ds_read_b128). K-contiguous sources are copied with 16-byte vectors;
//    M/N-contiguous sources (W1/W2 in the forward, both dW operands) are
//    transposed in registers (4x8 blocks) on their way into LDS.
//  * relu^2 gradient GA = bf16(pre > 0 ? 2 * grad * pre : 0) is formed on the
//    fly in the operand load (grouped_gemm.py:751-766, 914-928); relu / relu^2
//    are applied to the fp32 accumulator in the epilogue (grouped_gemm.py:336-346).

#include <algorithm>
#include <mutex>

#include "vmoe_common.h"

namespace vmoe {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;

enum Variant { UP_FWD = 0, DOWN_FWD, UP_DX, UP_DW, DOWN_DH, DOWN_DW };

struct Args {
  const uint16_t* a;    // A source
  const uint16_t* a2;   // pre_act, for the gradient prologue on A
  int64_t lda;
  const int32_t* a_map;  // row gather for A (UP_DW fused gather), nullable
  int64_t a_rows;        // rows of the gathered source
  const uint16_t* b;
  const uint16_t* b2;    // pre_act, for the gradient prologue on B
  int64_t ldb;
  uint16_t* c;
  uint16_t* c2;  // pre_act output (UP_FWD)
  int64_t ldc;
  const int32_t* eto;
  const int32_t* ewo;
  const int32_t* widths;
  const int32_t* tpe;
  int E;
  int hidden;
  int act;
  int64_t rows_bound;
  int kc;          // K rows per work item for the dW GEMMs (0 = whole K)
  float* partial;  // fp32 partial tiles of split work items
};

// Per-expert problem: valid extents and operand origins.
//   A K-contig:  A(m,k) = a[(ar + m) * lda + ac + k]
//   A MN-contig: A(m,k) = a[row(ar + k) * lda + ac + m]
//   B K-contig:  B(k,n) = b[(br + n) * ldb + bc + k]
//   B MN-contig: B(k,n) = b[(br + k) * ldb + bc + n]
//   C(m,n) = c[(cr + m) * ldc + cc + n]
struct Prob {
  int M, N, K;
  int64_t ar, ac, br, bc, cr, cc;
};

template <int V>
struct Traits;

__device__ __forceinline__ int clamp0(int64_t v) { return (int)max<int64_t>(0, v); }

template <>
struct Traits<UP_FWD> {
  static constexpr bool a_k = true, b_k = false, a_grad = false, b_grad = false;
  __device__ static void tile_dims(const Args& p, int e, int& mt, int& nt) {
    mt = p.tpe[e];
    nt = p.widths[e];
  }
  __device__ static Prob prob(const Args& p, int e) {
    const int64_t t0 = p.eto[e], t1 = min<int64_t>(p.eto[e + 1], p.rows_bound);
    Prob q;
    q.M = clamp0(min<int64_t>(p.tpe[e], t1 - t0));
    q.N = clamp0(p.widths[e]);
    q.K = p.hidden;
    q.ar = t0; q.ac = 0;
    q.br = 0; q.bc = p.ewo[e];
    q.cr = t0; q.cc = 0;
    return q;
  }
};

template <>
struct Traits<DOWN_FWD> {
  static constexpr bool a_k = true, b_k = false, a_grad = false, b_grad = false;
  __device__ static void tile_dims(const Args& p, int e, int& mt, int& nt) {
    mt = p.tpe[e];
    nt = p.hidden;
  }
  __device__ static Prob prob(const Args& p, int e) {
    const int64_t t0 = p.eto[e], t1 = min<int64_t>(p.eto[e + 1], p.rows_bound);
    Prob q;
    q.M = clamp0(min<int64_t>(p.tpe[e], t1 - t0));
    q.N = p.hidden;
    q.K = clamp0((int64_t)p.ewo[e + 1] - p.ewo[e]);
    q.ar = t0; q.ac = 0;
    q.br = p.ewo[e]; q.bc = 0;
    q.cr = t0; q.cc = 0;
    return q;
  }
};

template <>
struct Traits<UP_DX> {
  static constexpr bool a_k = true, b_k = true, a_grad = true, b_grad = false;
  __device__ static void tile_dims(const Args& p, int e, int& mt, int& nt) {
    mt = p.tpe[e];
    nt = p.hidden;
  }
  __device__ static Prob prob(const Args& p, int e) {
    const int64_t t0 = p.eto[e], t1 = min<int64_t>(p.eto[e + 1], p.rows_bound);
    Prob q;
    q.M = clamp0(min<int64_t>(p.tpe[e], t1 - t0));
    q.N = p.hidden;
    q.K = clamp0((int64_t)p.ewo[e + 1] - p.ewo[e]);
    q.ar = t0; q.ac = 0;
    q.br = 0; q.bc = p.ewo[e];  // B(k,n) = W1[n][ewo + k]
    q.cr = t0; q.cc = 0;
    return q;
  }
};

template <>
struct Traits<UP_DW> {
  static constexpr bool a_k = false, b_k = false, a_grad = false, b_grad = true;
  __device__ static void tile_dims(const Args& p, int e, int& mt, int& nt) {
    mt = p.hidden;
    nt = p.widths[e];
  }
  __device__ static Prob prob(const Args& p, int e) {
    const int64_t t0 = p.eto[e], t1 = min<int64_t>(p.eto[e + 1], p.rows_bound);
    Prob q;
    q.M = p.hidden;
    q.N = clamp0(p.widths[e]);
    q.K = clamp0(t1 - t0);
    q.ar = t0; q.ac = 0;  // A(m,k) = X[row(t0 + k)][m]
    q.br = t0; q.bc = 0;  // B(k,n) = GA[t0 + k][n]
    q.cr = 0; q.cc = p.ewo[e];
    return q;
  }
};

template <>
struct Traits<DOWN_DH> {
  static constexpr bool a_k = true, b_k = true, a_grad = false, b_grad = false;
  __device__ static void tile_dims(const Args& p, int e, int& mt, int& nt) {
    mt = p.tpe[e];
    nt = p.widths[e];
  }
  __device__ static Prob prob(const Args& p, int e) {
    const int64_t t0 = p.eto[e], t1 = min<int64_t>(p.eto[e + 1], p.rows_bound);
    Prob q;
    q.M = clamp0(min<int64_t>(p.tpe[e], t1 - t0));
    q.N = clamp0(p.widths[e]);
    q.K = p.hidden;
    q.ar = t0; q.ac = 0;
    q.br = p.ewo[e]; q.bc = 0;  // B(k,n) = W2[ewo + n][k]
    q.cr = t0; q.cc = 0;
    return q;
  }
};

template <>
struct Traits<DOWN_DW> {
  static constexpr bool a_k = false, b_k = false, a_grad = false, b_grad = false;
  __device__ static void tile_dims(const Args& p, int e, int& mt, int& nt) {
    mt = p.widths[e];
    nt = p.hidden;
  }
  __device__ static Prob prob(const Args& p, int e) {
    const int64_t t0 = p.eto[e], t1 = min<int64_t>(p.eto[e + 1], p.rows_bound);
    Prob q;
    q.M = clamp0(p.widths[e]);
    q.N = p.hidden;
    q.K = clamp0(t1 - t0);
    q.ar = t0; q.ac = 0;  // A(m,k) = H[t0 + k][m]
    q.br = t0; q.bc = 0;  // B(k,n) = GY[t0 + k][n]
    q.cr = p.ewo[e]; q.cc = 0;
    return q;
  }
};

__host__ __device__ constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }

// GA = bf16(pre > 0 ? 2 * g * pre : 0) for relu^2, else g; 8 values at once.
__device__ __forceinline__ uint4 relu2_grad(uint4 g, uint4 pre, int act) {
  if (act != VMOE_ACT_RELU_SQUARED) return g;
  uint32_t gw[4] = {g.x, g.y, g.z, g.w}, pw[4] = {pre.x, pre.y, pre.z, pre.w}, o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float pl = lo_f32(pw[i]), ph = hi_f32(pw[i]);
    const float vl = pl > 0.0f ? lo_f32(gw[i]) * 2.0f * pl : 0.0f;
    const float vh = ph > 0.0f ? hi_f32(gw[i]) * 2.0f * ph : 0.0f;
    o[i] = pack_bf16(vl, vh);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

__device__ __forceinline__ uint32_t half_of(const uint4& v, int i) {
  const uint32_t w = i < 2 ? (i == 0 ? v.x : v.y) : (i == 2 ? v.z : v.w);
  return w;
}

// Register transpose of a 4(k) x 8(mn) bf16 block into 8 rows of 4 k-values.
// in[kk] holds mn = 0..7 at k = kk; out[mm] = {k0|k1, k2|k3} at mn = mm.
__device__ __forceinline__ void transpose4x8(const uint4 in[4], uint2 out[8]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t a0 = half_of(in[0], w), a1 = half_of(in[1], w);
    const uint32_t a2 = half_of(in[2], w), a3 = half_of(in[3], w);
    // even mn = 2w: low halves; odd mn = 2w+1: high halves
    out[2 * w].x = (a0 & 0xFFFFu) | (a1 << 16);
    out[2 * w].y = (a2 & 0xFFFFu) | (a3 << 16);
    out[2 * w + 1].x = (a0 >> 16) | (a1 & 0xFFFF0000u);
    out[2 * w + 1].y = (a2 >> 16) | (a3 & 0xFFFF0000u);
  }
}

template <int V, int BM, int BN, int BK>
struct Gemm {
  using T = Traits<V>;
  static constexpr int LDK = BK + 8;  // LDS row pitch (bf16): 16-byte pad
  static constexpr int WM = BM / 2, WN = BN / 2;  // wave tile
  static constexpr int FM = WM / 32, FN = WN / 32;  // 32x32 blocks per wave
  static constexpr int A_ELEMS = BM * LDK, B_ELEMS = BN * LDK;
  static constexpr size_t LDS_BYTES = 2 * (A_ELEMS + B_ELEMS) * sizeof(uint16_t);

  // K-contig loader: 16-byte chunks, ROWS x BK tile.
  template <int ROWS>
  struct KLoad {
    static constexpr int CPR = BK / 8;  // chunks per row
    static constexpr int TOTAL = ROWS * CPR;
    static constexpr int N = cdiv(TOTAL, kThreads);
  };
  // MN-contig loader: 8(mn) x 4(k) blocks.
  template <int COLS>
  struct TLoad {
    static constexpr int KB = BK / 4, MB = COLS / 8;
    static constexpr int TOTAL = KB * MB;
    static constexpr int N = cdiv(TOTAL, kThreads);
  };

  static constexpr int NA = T::a_k ? KLoad<BM>::N : TLoad<BM>::N * 4;
  static constexpr int NB = T::b_k ? KLoad<BN>::N : TLoad<BN>::N * 4;

  struct Regs {
    uint4 a[NA];
    uint4 a2[T::a_grad ? NA : 1];
    uint4 b[NB];
    uint4 b2[T::b_grad ? NB : 1];
  };

  __device__ static void load_k(const uint16_t* src, const uint16_t* src2, int64_t ld,
                                const int32_t* map, int64_t map_rows, int64_t r0, int64_t c0,
                                int rows_valid, int k0, int K, uint4* dst, uint4* dst2,
                                bool two, int nchunks, int cpr, int total) {
    for (int i = 0; i < nchunks; ++i) {
      const int c = threadIdx.x + kThreads * i;
      const int row = c / cpr, kc = c % cpr;
      const int k = k0 + kc * 8;
      uint4 v = make_uint4(0, 0, 0, 0), v2 = v;
      int64_t srow = r0 + row;
      bool ok = c < total && row < rows_valid && k < K;
      if (ok && map) {
        srow = map[srow];
        ok = srow >= 0 && srow < map_rows;
      }
      if (ok) {
        const int64_t off = srow * ld + c0 + k;
        v = *reinterpret_cast<const uint4*>(src + off);
        if (two) v2 = *reinterpret_cast<const uint4*>(src2 + off);
      }
      dst[i] = v;
      if (two) dst2[i] = v2;
    }
  }

  __device__ static void load_t(const uint16_t* src, const uint16_t* src2, int64_t ld,
                                const int32_t* map, int64_t map_rows, int64_t r0, int64_t c0,
                                int cols_valid, int k0, int K, uint4* dst, uint4* dst2,
                                bool two, int nblocks, int kb_count, int total) {
    for (int i = 0; i < nblocks; ++i) {
      const int blk = threadIdx.x + kThreads * i;
      const int kb = blk % kb_count, mb = blk / kb_count;
      const bool col_ok = blk < total && mb * 8 < cols_valid;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int k = k0 + kb * 4 + kk;
        uint4 v = make_uint4(0, 0, 0, 0), v2 = v;
        if (col_ok && k < K) {
          int64_t row = r0 + k;
          bool ok = true;
          if (map) {
            row = map[row];
            ok = row >= 0 && row < map_rows;
          }
          if (ok) {
            const int64_t off = row * ld + c0 + mb * 8;
            v = *reinterpret_cast<const uint4*>(src + off);
            if (two) v2 = *reinterpret_cast<const uint4*>(src2 + off);
          }
        }
        dst[i * 4 + kk] = v;
        if (two) dst2[i * 4 + kk] = v2;
      }
    }
  }

  __device__ static void store_k(uint16_t* lds, const uint4* v, int nchunks, int cpr,
                                 int total) {
    for (int i = 0; i < nchunks; ++i) {
      const int c = threadIdx.x + kThreads * i;
      if (c >= total) break;
      const int row = c / cpr, kc = c % cpr;
      *reinterpret_cast<uint4*>(lds + row * LDK + kc * 8) = v[i];
    }
  }

  __device__ static void store_t(uint16_t* lds, const uint4* v, int nblocks, int kb_count,
                                 int total) {
    for (int i = 0; i < nblocks; ++i) {
      const int blk = threadIdx.x + kThreads * i;
      if (blk >= total) break;
      const int kb = blk % kb_count, mb = blk / kb_count;
      uint2 o[8];
      transpose4x8(v + i * 4, o);
#pragma unroll
      for (int mm = 0; mm < 8; ++mm)
        *reinterpret_cast<uint2*>(lds + (mb * 8 + mm) * LDK + kb * 4) = o[mm];
    }
  }

  __device__ static void load_tiles(const Args& p, const Prob& q, int m0, int n0, int k0,
                                    Regs& r) {
    if (T::a_k)
      load_k(p.a, p.a2, p.lda, p.a_map, p.a_rows, q.ar + m0, q.ac, q.M - m0, k0, q.K, r.a,
             r.a2, T::a_grad,
             KLoad<BM>::N, KLoad<BM>::CPR, KLoad<BM>::TOTAL);
    else
      load_t(p.a, p.a2, p.lda, p.a_map, p.a_rows, q.ar, q.ac + m0, q.M - m0, k0, q.K, r.a,
             r.a2, T::a_grad, TLoad<BM>::N, TLoad<BM>::KB, TLoad<BM>::TOTAL);
    if (T::b_k)
      load_k(p.b, p.b2, p.ldb, nullptr, 0, q.br + n0, q.bc, q.N - n0, k0, q.K, r.b, r.b2,
             T::b_grad,
             KLoad<BN>::N, KLoad<BN>::CPR, KLoad<BN>::TOTAL);
    else
      load_t(p.b, p.b2, p.ldb, nullptr, 0, q.br, q.bc + n0, q.N - n0, k0, q.K, r.b, r.b2,
             T::b_grad, TLoad<BN>::N, TLoad<BN>::KB, TLoad<BN>::TOTAL);
  }

  __device__ static void store_tiles(const Args& p, uint16_t* As, uint16_t* Bs, Regs& r) {
    if (T::a_grad) {
#pragma unroll
      for (int i = 0; i < NA; ++i) r.a[i] = relu2_grad(r.a[i], r.a2[i], p.act);
    }
    if (T::b_grad) {
#pragma unroll
      for (int i = 0; i < NB; ++i) r.b[i] = relu2_grad(r.b[i], r.b2[i], p.act);
    }
    if (T::a_k)
      store_k(As, r.a, KLoad<BM>::N, KLoad<BM>::CPR, KLoad<BM>::TOTAL);
    else
      store_t(As, r.a, TLoad<BM>::N, TLoad<BM>::KB, TLoad<BM>::TOTAL);
    if (T::b_k)
      store_k(Bs, r.b, KLoad<BN>::N, KLoad<BN>::CPR, KLoad<BN>::TOTAL);
    else
      store_t(Bs, r.b, TLoad<BN>::N, TLoad<BN>::KB, TLoad<BN>::TOTAL);
  }

  // Work items of expert e: its output tiles times its K chunks (chunks > 1
  // only for the split-K dW GEMMs, p.kc > 0).
  __device__ static void expert_work(const Args& p, int e, int& tiles, int& chunks) {
    int mt, nt;
    T::tile_dims(p, e, mt, nt);
    tiles = (mt > 0 && nt > 0) ? cdiv(mt, BM) * cdiv(nt, BN) : 0;
    chunks = 1;
    if (p.kc > 0 && tiles > 0) {
      const int K = T::prob(p, e).K;
      chunks = K > p.kc ? cdiv(K, p.kc) : 1;
    }
  }

  // Finds the expert owning index `id` in the concatenation of per-expert
  // ranges of size a_e (a block scan over experts), the offset inside that
  // range, and the exclusive prefix of a second per-expert count b_e.
  // MODE 0: a = items, b = split items (GEMM); MODE 1: a = tiles, b = split
  // items (reduce). Returns false when id is past the end.
  template <int MODE>
  __device__ static bool locate(const Args& p, int id, int& e_out, int& local_out,
                                int& bpre_out, int& chunks_out) {
    __shared__ long long scan[kThreads / kWave + 1];
    __shared__ int32_t s_e, s_local, s_bpre, s_chunks;
    if (threadIdx.x == 0) s_e = -1;
    long long base = 0;
    for (int e0 = 0; e0 < p.E; e0 += kThreads) {
      const int e = e0 + threadIdx.x;
      int tiles = 0, chunks = 1;
      if (e < p.E) expert_work(p, e, tiles, chunks);
      const int items = tiles * chunks;
      const int a = MODE == 0 ? items : tiles;
      const int b = chunks > 1 ? items : 0;
      const long long packed = ((long long)a << 32) | (long long)b;
      long long total;
      const long long ex = block_exclusive_scan<long long, kThreads>(packed, scan, &total);
      const long long pre = base + ex;
      const int a_pre = (int)(pre >> 32), b_pre = (int)(pre & 0xFFFFFFFFll);
      if (a > 0 && id >= a_pre && id < a_pre + a) {
        s_e = e;
        s_local = id - a_pre;
        s_bpre = b_pre;
        s_chunks = chunks;
      }
      base += total;
      __syncthreads();
      if (s_e >= 0 || (int)(base >> 32) > id) break;
    }
    e_out = s_e;
    local_out = s_local;
    bpre_out = s_bpre;
    chunks_out = s_chunks;
    return s_e >= 0;
  }

  __device__ static void run(const Args& p) {
    extern __shared__ __align__(16) uint16_t smem[];
    uint16_t* As = smem;                  // [2][BM][LDK]
    uint16_t* Bs = smem + 2 * A_ELEMS;    // [2][BN][LDK]

    // XCD-aware remap: hardware deals workgroup ids round-robin over the 8
    // XCDs; give each XCD a contiguous range of tiles (gridDim.x % 8 == 0).
    const int g = gridDim.x, b = blockIdx.x;
    const int bid = (b % 8) * (g / 8) + b / 8;

    int e, local, split_pre, chunks;
    if (!locate<0>(p, bid, e, local, split_pre, chunks)) return;
    int mt_dim, nt_dim;
    T::tile_dims(p, e, mt_dim, nt_dim);
    const int n_tiles = cdiv(nt_dim, BN);
    const int tile = local / chunks, chunk = local % chunks;
    const int m0 = (tile / n_tiles) * BM;
    const int n0 = (tile % n_tiles) * BN;
    Prob q = T::prob(p, e);
    // K range of this work item: [kbeg, q.K) after clamping q.K to the chunk.
    int kbeg = 0;
    if (chunks > 1) {
      kbeg = chunk * p.kc;
      q.K = min(q.K, kbeg + p.kc);
    }

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int wm = wave >> 1, wn = wave & 1;

    f32x16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int nk = q.K > kbeg ? cdiv(q.K - kbeg, BK) : 0;
    Regs regs;
    if (nk > 0) {
      load_tiles(p, q, m0, n0, kbeg, regs);
      store_tiles(p, As, Bs, regs);
    }
    __syncthreads();

    const int frag_row = lane & 31;
    const int frag_k = (lane >> 5) * 8;
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load_tiles(p, q, m0, n0, kbeg + (kt + 1) * BK, regs);
      const uint16_t* Ac = As + cur * A_ELEMS;
      const uint16_t* Bc = Bs + cur * B_ELEMS;
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        bf16x8_t af[FM], bfr[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          af[i] = *reinterpret_cast<const bf16x8_t*>(
              Ac + (wm * WM + i * 32 + frag_row) * LDK + ks * 16 + frag_k);
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bfr[j] = *reinterpret_cast<const bf16x8_t*>(
              Bc + (wn * WN + j * 32 + frag_row) * LDK + ks * 16 + frag_k);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            // Operands swapped: the accumulator holds C^T, so each lane owns
            // 4 consecutive n of one m and stores 8 bytes at a time.
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
      }
      if (kt + 1 < nk)
        store_tiles(p, As + (cur ^ 1) * A_ELEMS, Bs + (cur ^ 1) * B_ELEMS, regs);
      __syncthreads();
    }

    // Epilogue. acc[i][j][4*g + r] sits at m = wm*WM + i*32 + (lane & 31),
    // n = wn*WN + j*32 + 8*g + 4*(lane >> 5) + r.
    if (chunks > 1) {
      // Split-K item: the whole fp32 tile goes to its partial slot; the
      // reduce kernel sums the chunks in chunk order and rounds once.
      float* slot = p.partial + (int64_t)(split_pre + local) * (BM * BN);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int ml = wm * WM + i * 32 + (lane & 31);
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            const int nl = wn * WN + j * 32 + 8 * gq + 4 * (lane >> 5);
            *reinterpret_cast<float4*>(slot + ml * BN + nl) =
                make_float4(acc[i][j][4 * gq], acc[i][j][4 * gq + 1], acc[i][j][4 * gq + 2],
                            acc[i][j][4 * gq + 3]);
          }
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = m0 + wm * WM + i * 32 + (lane & 31);
      if (m >= q.M) continue;
      uint16_t* crow = p.c + (q.cr + m) * p.ldc + q.cc;
      uint16_t* crow2 = p.c2 ? p.c2 + (q.cr + m) * p.ldc + q.cc : nullptr;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int n = n0 + wn * WN + j * 32 + 8 * gq + 4 * (lane >> 5);
          if (n >= q.N) continue;
          float v0 = acc[i][j][4 * gq + 0], v1 = acc[i][j][4 * gq + 1];
          float v2 = acc[i][j][4 * gq + 2], v3 = acc[i][j][4 * gq + 3];
          if (V == UP_FWD && p.act == VMOE_ACT_RELU_SQUARED) {
            v0 = fmaxf(v0, 0.0f); v1 = fmaxf(v1, 0.0f);
            v2 = fmaxf(v2, 0.0f); v3 = fmaxf(v3, 0.0f);
            if (crow2)
              *reinterpret_cast<uint2*>(crow2 + n) =
                  make_uint2(pack_bf16(v0, v1), pack_bf16(v2, v3));
            v0 *= v0; v1 *= v1; v2 *= v2; v3 *= v3;
          }
          *reinterpret_cast<uint2*>(crow + n) = make_uint2(pack_bf16(v0, v1), pack_bf16(v2, v3));
        }
      }
    }
  }
};

template <int V, int BM, int BN, int BK>
__global__ __launch_bounds__(kThreads) void grouped_gemm_kernel(Args p) {
  Gemm<V, BM, BN, BK>::run(p);
}

// Sums the K-chunk partials of every split (expert, tile) in chunk order and
// stores the bf16 result. One workgroup per output tile; tiles of experts that
// were not split exit at once (their GEMM item stored bf16 directly).
template <int V, int BM, int BN, int BK>
__global__ __launch_bounds__(kThreads) void splitk_reduce_kernel(Args p) {
  using G = Gemm<V, BM, BN, BK>;
  const int g = gridDim.x, b = blockIdx.x;
  const int id = (b % 8) * (g / 8) + b / 8;
  int e, tile, split_pre, chunks;
  if (!G::template locate<1>(p, id, e, tile, split_pre, chunks)) return;
  if (chunks <= 1) return;
  int mt_dim, nt_dim;
  Traits<V>::tile_dims(p, e, mt_dim, nt_dim);
  const int n_tiles = cdiv(nt_dim, BN);
  const int m0 = (tile / n_tiles) * BM, n0 = (tile % n_tiles) * BN;
  const Prob q = Traits<V>::prob(p, e);
  const float* base = p.partial + (int64_t)(split_pre + tile * chunks) * (BM * BN);
  for (int idx = threadIdx.x * 4; idx < BM * BN; idx += kThreads * 4) {
    const int ml = idx / BN, nl = idx % BN;
    const int m = m0 + ml, n = n0 + nl;
    if (m >= q.M || n >= q.N) continue;
    float4 acc = *reinterpret_cast<const float4*>(base + idx);
    for (int c = 1; c < chunks; ++c) {
      const float4 v = *reinterpret_cast<const float4*>(base + (int64_t)c * (BM * BN) + idx);
      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
    *reinterpret_cast<uint2*>(p.c + (q.cr + m) * p.ldc + q.cc + n) =
        make_uint2(pack_bf16(acc.x, acc.y), pack_bf16(acc.z, acc.w));
  }
}

// Tile configuration (one for all variants for now).
constexpr int kBM = 128, kBN = 128, kBK = 32;

inline bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Compute units of the current device (cached per device id).
int cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// Split-K plan of a dW GEMM: K rows per work item, and the partial-tile
// capacity it can need. The chunk keeps a work item near a quarter of one
// CU's share of the whole dW (tiles_max * rows_bound row-tiles), so one
// heavily loaded expert is spread over many CUs; it never drops below 1024
// rows, so lightly loaded layers do not pay for partials.
struct SplitPlan {
  int kc;
  int64_t slots;  // partial tiles
};

SplitPlan split_plan(int64_t tiles_max, int64_t rows_bound) {
  const int64_t cus = cu_count();
  int64_t kc = (tiles_max * rows_bound) / (4 * cus);
  kc = std::max<int64_t>(1024, (kc + kBK - 1) / kBK * kBK);
  kc = std::min<int64_t>(kc, 1 << 30);
  SplitPlan sp;
  sp.kc = (int)kc;
  sp.slots = tiles_max * (2 * ((rows_bound + kc - 1) / kc) + 1);
  return sp;
}

template <int V>
int launch(const Args& p, int64_t grid_tiles, hipStream_t s) {
  using G = Gemm<V, kBM, kBN, kBK>;
  auto kern = grouped_gemm_kernel<V, kBM, kBN, kBK>;
  if (G::LDS_BYTES > 65536) {
    static std::once_flag once;
    static hipError_t attr_err = hipSuccess;
    std::call_once(once, [&] {
      attr_err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)G::LDS_BYTES);
    });
    if (attr_err != hipSuccess) return VMOE_ERR_LAUNCH;
  }
  if (grid_tiles <= 0) return VMOE_OK;
  int64_t g = (grid_tiles + 7) / 8 * 8;
  if (g > INT32_MAX) return VMOE_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(kern, dim3((unsigned)g), dim3(kThreads), G::LDS_BYTES, s, p);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

// dW GEMM with split-K: GEMM items, then the chunk reduction.
template <int V>
int launch_dw(Args p, int64_t tiles_max, void* ws, size_t ws_bytes, hipStream_t s) {
  const int64_t E = p.E;
  if (ws) {
    const SplitPlan sp = split_plan(tiles_max, p.rows_bound);
    if (ws_bytes < (size_t)sp.slots * kBM * kBN * sizeof(float)) return VMOE_ERR_WORKSPACE;
    p.kc = sp.kc;
    p.partial = reinterpret_cast<float*>(ws);
    const int64_t items = tiles_max * (E + p.rows_bound / sp.kc + 1);
    int st = launch<V>(p, items, s);
    if (st) return st;
    int64_t g = (E * tiles_max + 7) / 8 * 8;
    if (g > INT32_MAX) return VMOE_ERR_UNSUPPORTED;
    hipLaunchKernelGGL((splitk_reduce_kernel<V, kBM, kBN, kBK>), dim3((unsigned)g),
                       dim3(kThreads), 0, s, p);
    VMOE_CHECK_LAUNCH();
    return VMOE_OK;
  }
  p.kc = 0;
  p.partial = nullptr;
  return launch<V>(p, E * tiles_max, s);
}

// Shared argument checks. Every dimension the kernels vectorise over must be a
// multiple of 8 elements and every base 16-byte aligned.
inline int check_common(const int32_t* eto, const int32_t* ewo, const int32_t* widths,
                        const int32_t* tpe, int32_t E, int64_t hidden, int64_t max_width,
                        int64_t rows_bound) {
  if (!eto || !ewo || !widths || !tpe || E <= 0 || hidden <= 0 || max_width < 0 ||
      rows_bound < 0)
    return VMOE_ERR_INVALID_ARG;
  if (hidden % 8 != 0 || max_width % 8 != 0 || hidden > INT32_MAX / 2 ||
      rows_bound > INT32_MAX)
    return VMOE_ERR_UNSUPPORTED;
  return VMOE_OK;
}

inline bool ld_ok(int64_t ld) { return ld > 0 && ld % 8 == 0; }

inline int64_t rows_tiles(int64_t rows_bound, int E, int BM) {
  return (rows_bound + BM - 1) / BM + E;
}

}  // namespace
}  // namespace vmoe

using namespace vmoe;

extern "C" int vmoe_gemm_up_fwd(const uint16_t* x, int64_t ldx, int64_t x_rows,
                                const int32_t* gather_map, const uint16_t* w1, int64_t ldw1,
                                uint16_t* out, uint16_t* pre_act, int64_t ldo, int32_t activation,
                                const int32_t* eto, const int32_t* ewo, const int32_t* widths,
                                const int32_t* tpe, int32_t E, int64_t hidden, int64_t max_width,
                                int64_t rows_bound, vmoe_stream_t stream) {
  int st = check_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (activation != VMOE_ACT_NONE && activation != VMOE_ACT_RELU_SQUARED)
    return VMOE_ERR_INVALID_ARG;
  if (!x || !w1 || !out || x_rows < 0) return VMOE_ERR_INVALID_ARG;
  if (!ld_ok(ldx) || !ld_ok(ldw1) || !ld_ok(ldo) || ldx < hidden || ldo < max_width)
    return VMOE_ERR_UNSUPPORTED;
  if (!a16(x) || !a16(w1) || !a16(out) || (pre_act && !a16(pre_act)))
    return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = x; p.lda = ldx; p.a_map = gather_map; p.a_rows = gather_map ? x_rows : 0;
  p.b = w1; p.ldb = ldw1;
  p.c = out; p.c2 = activation == VMOE_ACT_RELU_SQUARED ? pre_act : nullptr; p.ldc = ldo;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = activation; p.rows_bound = rows_bound;
  const int64_t tiles = rows_tiles(rows_bound, E, kBM) * ((max_width + kBN - 1) / kBN);
  return launch<UP_FWD>(p, tiles, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vmoe_gemm_down_fwd(const uint16_t* h, int64_t ldh, const uint16_t* w2,
                                  int64_t ldw2, uint16_t* y, int64_t ldy, const int32_t* eto,
                                  const int32_t* ewo, const int32_t* widths, const int32_t* tpe,
                                  int32_t E, int64_t hidden, int64_t max_width,
                                  int64_t rows_bound, vmoe_stream_t stream) {
  int st = check_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (!h || !w2 || !y) return VMOE_ERR_INVALID_ARG;
  if (!ld_ok(ldh) || !ld_ok(ldw2) || !ld_ok(ldy) || ldw2 < hidden || ldy < hidden)
    return VMOE_ERR_UNSUPPORTED;
  if (!a16(h) || !a16(w2) || !a16(y)) return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = h; p.lda = ldh;
  p.b = w2; p.ldb = ldw2;
  p.c = y; p.ldc = ldy;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = VMOE_ACT_NONE; p.rows_bound = rows_bound;
  const int64_t tiles = rows_tiles(rows_bound, E, kBM) * ((hidden + kBN - 1) / kBN);
  return launch<DOWN_FWD>(p, tiles, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vmoe_gemm_up_bwd_dx(const uint16_t* grad_h, const uint16_t* pre_act, int64_t ldg,
                                   int32_t activation, const uint16_t* w1, int64_t ldw1,
                                   uint16_t* grad_x, int64_t ldgx, const int32_t* eto,
                                   const int32_t* ewo, const int32_t* widths, const int32_t* tpe,
                                   int32_t E, int64_t hidden, int64_t max_width,
                                   int64_t rows_bound, vmoe_stream_t stream) {
  int st = check_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (activation != VMOE_ACT_NONE && activation != VMOE_ACT_RELU_SQUARED)
    return VMOE_ERR_INVALID_ARG;
  if (!grad_h || !w1 || !grad_x || (activation == VMOE_ACT_RELU_SQUARED && !pre_act))
    return VMOE_ERR_INVALID_ARG;
  if (!ld_ok(ldg) || !ld_ok(ldw1) || !ld_ok(ldgx) || ldgx < hidden) return VMOE_ERR_UNSUPPORTED;
  if (!a16(grad_h) || !a16(w1) || !a16(grad_x) || (pre_act && !a16(pre_act)))
    return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = grad_h; p.a2 = pre_act ? pre_act : grad_h; p.lda = ldg;
  p.b = w1; p.ldb = ldw1;
  p.c = grad_x; p.ldc = ldgx;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = activation; p.rows_bound = rows_bound;
  const int64_t tiles = rows_tiles(rows_bound, E, kBM) * ((hidden + kBN - 1) / kBN);
  return launch<UP_DX>(p, tiles, reinterpret_cast<hipStream_t>(stream));
}

extern "C" size_t vmoe_gemm_dw_workspace_bytes(int32_t E, int64_t hidden, int64_t max_width,
                                               int64_t rows_bound) {
  if (E <= 0 || hidden <= 0 || max_width <= 0 || rows_bound <= 0) return 0;
  const int64_t up_tiles = ((hidden + kBM - 1) / kBM) * ((max_width + kBN - 1) / kBN);
  const int64_t down_tiles = ((max_width + kBM - 1) / kBM) * ((hidden + kBN - 1) / kBN);
  const SplitPlan a = split_plan(up_tiles, rows_bound), b = split_plan(down_tiles, rows_bound);
  return (size_t)std::max(a.slots, b.slots) * kBM * kBN * sizeof(float);
}

extern "C" int vmoe_gemm_up_bwd_dw(const uint16_t* x, int64_t ldx, int64_t x_rows,
                                   const int32_t* gather_map, const uint16_t* grad_h,
                                   const uint16_t* pre_act, int64_t ldg, int32_t activation,
                                   uint16_t* grad_w1, int64_t ldgw, const int32_t* eto,
                                   const int32_t* ewo, const int32_t* widths, const int32_t* tpe,
                                   int32_t E, int64_t hidden, int64_t max_width,
                                   int64_t rows_bound, void* workspace, size_t workspace_bytes,
                                   vmoe_stream_t stream) {
  int st = check_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (activation != VMOE_ACT_NONE && activation != VMOE_ACT_RELU_SQUARED)
    return VMOE_ERR_INVALID_ARG;
  if (!x || !grad_h || !grad_w1 || x_rows < 0 ||
      (activation == VMOE_ACT_RELU_SQUARED && !pre_act))
    return VMOE_ERR_INVALID_ARG;
  if (!ld_ok(ldx) || !ld_ok(ldg) || !ld_ok(ldgw) || ldx < hidden) return VMOE_ERR_UNSUPPORTED;
  if (!a16(x) || !a16(grad_h) || !a16(grad_w1) || (pre_act && !a16(pre_act)))
    return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = x; p.lda = ldx; p.a_map = gather_map; p.a_rows = gather_map ? x_rows : 0;
  p.b = grad_h; p.b2 = pre_act ? pre_act : grad_h; p.ldb = ldg;
  p.c = grad_w1; p.ldc = ldgw;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = activation; p.rows_bound = rows_bound;
  const int64_t tiles_max = ((hidden + kBM - 1) / kBM) * ((max_width + kBN - 1) / kBN);
  return launch_dw<UP_DW>(p, tiles_max, workspace, workspace_bytes,
                          reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vmoe_gemm_down_bwd_dh(const uint16_t* grad_y, int64_t ldgy, const uint16_t* w2,
                                     int64_t ldw2, uint16_t* grad_h, int64_t ldgh,
                                     const int32_t* eto, const int32_t* ewo,
                                     const int32_t* widths, const int32_t* tpe, int32_t E,
                                     int64_t hidden, int64_t max_width, int64_t rows_bound,
                                     vmoe_stream_t stream) {
  int st = check_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (!grad_y || !w2 || !grad_h) return VMOE_ERR_INVALID_ARG;
  if (!ld_ok(ldgy) || !ld_ok(ldw2) || !ld_ok(ldgh) || ldgy < hidden || ldw2 < hidden ||
      ldgh < max_width)
    return VMOE_ERR_UNSUPPORTED;
  if (!a16(grad_y) || !a16(w2) || !a16(grad_h)) return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = grad_y; p.lda = ldgy;
  p.b = w2; p.ldb = ldw2;
  p.c = grad_h; p.ldc = ldgh;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = VMOE_ACT_NONE; p.rows_bound = rows_bound;
  const int64_t tiles = rows_tiles(rows_bound, E, kBM) * ((max_width + kBN - 1) / kBN);
  return launch<DOWN_DH>(p, tiles, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vmoe_gemm_down_bwd_dw(const uint16_t* h, int64_t ldh, const uint16_t* grad_y,
                                     int64_t ldgy, uint16_t* grad_w2, int64_t ldgw,
                                     const int32_t* eto, const int32_t* ewo,
                                     const int32_t* widths, const int32_t* tpe, int32_t E,
                                     int64_t hidden, int64_t max_width, int64_t rows_bound,
                                     void* workspace, size_t workspace_bytes,
                                     vmoe_stream_t stream) {
  int st = check_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (!h || !grad_y || !grad_w2) return VMOE_ERR_INVALID_ARG;
  if (!ld_ok(ldh) || !ld_ok(ldgy) || !ld_ok(ldgw) || ldgy < hidden || ldgw < hidden)
    return VMOE_ERR_UNSUPPORTED;
  if (!a16(h) || !a16(grad_y) || !a16(grad_w2)) return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = h; p.lda = ldh;
  p.b = grad_y; p.ldb = ldgy;
  p.c = grad_w2; p.ldc = ldgw;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = VMOE_ACT_NONE; p.rows_bound = rows_bound;
  const int64_t tiles_max = ((max_width + kBM - 1) / kBM) * ((hidden + kBN - 1) / kBN);
  return launch_dw<DOWN_DW>(p, tiles_max, workspace, workspace_bytes,
                            reinterpret_cast<hipStream_t>(stream));
}
