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
//  * Tile scheduler on the device: the grid is an upper bound of the work
//    count; each workgroup scans the per-expert work counts (from the same
//    metadata the reference reads) and finds its (expert, tile, K chunk), so
//    no host sync is needed and empty experts cost nothing. Workgroup ids are
//    remapped so that consecutive tiles (same expert, same weight slice) run
//    on the same XCD and share its L2.
//  * 256 threads = 4 waves in a 2x2 grid; each wave owns (BM/2)x(BN/2) of
//    32x32 MFMA accumulators (fp32; 128x128 per wave for 256x256 tiles).
//  * Every operand tile goes global -> LDS by DMA (global_load_lds, 16 bytes
//    per lane), never through VGPRs, in a multi-stage ring: the loads of
//    tile k+STAGES-1 fly while tile k is multiplied.
//      - K-contiguous sources (activations in the forward, W in dX/dH) land
//        in "K-form": one 64-byte row per m (n), 16-byte chunk c of row r at
//        c ^ ((r >> 1) & 3); MFMA fragments are one ds_read_b128.
//      - M/N-contiguous sources (W1/W2 in the forward, both dW operands)
//        land as they are in memory ("T-form": one row per k), chunk c of
//        k-row k at c ^ 2(k & 3); fragments are two ds_read_b64_tr_b16,
//        the gfx950 LDS transpose read, so no operand is transposed in
//        registers. Both swizzles make the fragment reads bank-conflict free.
//  * Epilogues: relu and relu^2 of the fp32 accumulator (PRE, H) for the up
//    projection (grouped_gemm.py:336-346); for the down dH GEMM an optional
//    fused relu^2 gradient GA = bf16(pre > 0 ? 2 * bf16(acc) * pre : 0)
//    (grouped_gemm.py:751-766), so dX and dW read GA directly; split-K fp32
//    partial tiles for the dW GEMMs, summed in chunk order by a second pass.

#include <algorithm>

#include "vmoe_common.h"

namespace vmoe {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4;
typedef __attribute__((address_space(3))) bf16x8_t lds_bf16x8;

constexpr int kThreads = 256;
constexpr int kBK = 32;  // k per LDS stage: two 16-deep MFMA steps

enum Variant { UP_FWD = 0, DOWN_FWD, UP_DX, UP_DW, DOWN_DH, DOWN_DW };

struct Args {
  const uint16_t* a;     // A source
  int64_t lda;
  const int32_t* a_map;  // row gather for A (fused gather), nullable
  int64_t a_rows;        // rows of the gathered source
  const uint16_t* b;
  int64_t ldb;
  uint16_t* c;
  int64_t ldc;
  uint16_t* c2;          // UP_FWD: pre_act output (nullable)
  const uint16_t* pre;   // DOWN_DH: pre_act input -> fused relu^2 gradient (nullable)
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

__device__ __forceinline__ int clamp0(int64_t v) { return (int)max<int64_t>(0, v); }

template <int V>
struct Traits;

template <>
struct Traits<UP_FWD> {
  static constexpr bool t_map = false;
  static constexpr bool a_k = true, b_k = false;
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
    q.br = 0; q.bc = p.ewo[e];  // B(k,n) = W1[k][ewo + n]
    q.cr = t0; q.cc = 0;
    return q;
  }
};

template <>
struct Traits<DOWN_FWD> {
  static constexpr bool t_map = false;
  static constexpr bool a_k = true, b_k = false;
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
    q.br = p.ewo[e]; q.bc = 0;  // B(k,n) = W2[ewo + k][n]
    q.cr = t0; q.cc = 0;
    return q;
  }
};

template <>
struct Traits<UP_DX> {
  static constexpr bool t_map = false;
  static constexpr bool a_k = true, b_k = true;
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
    q.ar = t0; q.ac = 0;        // A(m,k) = GA[t0 + m][k]
    q.br = 0; q.bc = p.ewo[e];  // B(k,n) = W1[n][ewo + k]
    q.cr = t0; q.cc = 0;
    return q;
  }
};

template <>
struct Traits<UP_DW> {
  static constexpr bool a_k = false, b_k = false;
  static constexpr bool t_map = true;  // A rows may come through the gather map
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
  static constexpr bool t_map = false;
  static constexpr bool a_k = true, b_k = true;
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
  static constexpr bool t_map = false;
  static constexpr bool a_k = false, b_k = false;
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

// Tile shape per variant: 256x128 for the GEMMs tiled over rows (large M),
// 128x128 for the dW GEMMs (M, N are hidden x width; split-K supplies the
// parallelism, and smaller tiles keep partial tiles cheap).
template <int V>
struct Cfg {
  static constexpr bool dw = V == UP_DW || V == DOWN_DW;
  static constexpr int BM = dw ? 128 : 256;
  static constexpr int BN = 128;
  static constexpr int STAGES = 4;  // LDS ring: STAGES - 1 tiles in flight
};

__host__ __device__ constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without the release/acquire fences of __syncthreads(),
// which would drain every outstanding DMA (vmcnt(0)) and empty the LDS ring.
// LDS data are ordered explicitly instead: each wave waits for its own DMAs
// (wait_vmcnt) before the barrier, and its LDS reads of a buffer are consumed
// by MFMAs before it reaches the next barrier. The asm clobbers keep the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Buffer resource over [base, base + 2 GiB): word 3 = 0x00020000 is the raw
// 32-bit-dword format of the gfx9 family. A lane whose offset is kOob (past
// num_records) reads zeros, which is how every masked lane is handled.
constexpr uint32_t kOob = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  // The base is block-uniform; readfirstlane keeps the resource in SGPRs
  // (a VGPR resource would force a waterfall loop around every DMA).
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void* b = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(b, 0, 0x7FFFFFFF, 0x00020000);
}

// 16-byte DMA of the lane's source into LDS at dst + 16 * lane
// (buffer_load_dwordx4 ... lds, LDS base in M0). Issued as inline asm so the
// compiler does not track it: it would otherwise wait for every DMA before
// any LDS read it cannot prove disjoint (at the loop head it cannot), which
// empties the ring. The kernels order DMA completion themselves with
// wait_vmcnt + block_barrier, and nothing else in them uses M0.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, lds_char* dst) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(dst));
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :: "v"(voff), "s"(r), "s"(lds) : "memory");
}

template <int V, int BM, int BN, int STAGES>
struct Gemm {
  using T = Traits<V>;
  static constexpr int BK = kBK;
  static constexpr int WM = BM / 2, WN = BN / 2;    // wave tile
  static constexpr int FM = WM / 32, FN = WN / 32;  // 32x32 blocks per wave
  static constexpr int A_STAGE = BM * BK * 2, B_STAGE = BN * BK * 2;  // bytes
  static constexpr int STAGE = A_STAGE + B_STAGE;
  static constexpr int LDS_BYTES = STAGES * STAGE;
  // DMA instructions per wave per stage for an operand of R rows/cols.
  template <int R>
  struct Dma {
    static constexpr int INSTS = R * BK / 8 / 64;
    static constexpr int PW = INSTS / 4;
    static constexpr int LPR = R / 8;        // T-form: lanes per k-row
    static constexpr int RPI = 64 / LPR;     // T-form: k-rows per instruction
    static_assert(INSTS % 4 == 0 && PW >= 1, "tile too small for 4 waves");
  };
  static constexpr int PWA = Dma<BM>::PW, PWB = Dma<BN>::PW;

  __device__ static int kswz(int r) { return (r >> 1) & 3; }
  __device__ static int tswz(int k) { return (k & 3) << 1; }

  // Per-thread DMA state of one operand: a buffer resource over the
  // operand (rebased to the tile where no row map is used) and one 32-bit
  // byte offset per DMA instruction.
  template <int PW>
  struct Src {
    __amdgpu_buffer_rsrc_t rsrc;
    const int32_t* map;  // T-form row gather (nullable)
    int64_t map_rows;
    int64_t r0;          // T-form with map: source row of k = 0
    uint32_t ld2;        // leading dimension in bytes
    uint32_t off[PW];    // K-form: row + chunk; T-form: chunk column (+ k-row without map)
    int idx[PW];         // K-form: k of the lane's chunk; T-form: the lane's k-row
    bool ok[PW];         // K-form: row valid; T-form: column valid
  };

  // K-form setup: rows [0, R) of the tile (source rows r0 + row, or
  // map[r0 + row]), rows_valid of them real, k measured from column c0.
  template <int R, int PW>
  __device__ static void setup_k(Src<PW>& s, const uint16_t* base, int64_t ld,
                                 const int32_t* map, int64_t map_rows, int64_t r0, int64_t c0,
                                 int rows_valid) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // Without a map, rebase to the tile's first row so offsets stay small.
    const uint16_t* b = map ? base + c0 : base + r0 * ld + c0;
    s.rsrc = make_rsrc(b);
    s.map = nullptr;
    s.ld2 = (uint32_t)(ld * 2);
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int row = (wave * PW + i) * 16 + (lane >> 2);
      const int c = (lane & 3) ^ kswz(row);
      bool ok = row < rows_valid;
      int64_t srow = row;
      if (ok && map) {
        srow = map[r0 + row];
        ok = srow >= 0 && srow < map_rows;
      }
      s.ok[i] = ok;
      s.idx[i] = c * 8;
      s.off[i] = ok ? (uint32_t)((srow * ld + c * 8) * 2) : kOob;
    }
  }

  // K-form issue: stage tile k0 .. k0 + BK (k0 relative to the setup's c0).
  template <int R, int PW>
  __device__ static void issue_k(const Src<PW>& s, int k0, int K, lds_char* stage) {
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const bool v = s.ok[i] && k0 + s.idx[i] < K;
      dma16(s.rsrc, v ? s.off[i] + (uint32_t)(k0 * 2) : kOob, stage + (wave * PW + i) * 1024);
    }
  }

  // T-form setup: columns [0, R) of the tile starting at source column c0,
  // cols_valid of them real; source rows r0 + k, or map[r0 + k].
  template <int R, int PW>
  __device__ static void setup_t(Src<PW>& s, const uint16_t* base, int64_t ld,
                                 const int32_t* map, int64_t map_rows, int64_t r0, int64_t c0,
                                 int cols_valid) {
    constexpr int LPR = Dma<R>::LPR, RPI = Dma<R>::RPI;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint16_t* b = map ? base + c0 : base + r0 * ld + c0;
    s.rsrc = make_rsrc(b);
    s.map = map;
    s.map_rows = map_rows;
    s.r0 = r0;
    s.ld2 = (uint32_t)(ld * 2);
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int krow = (wave * PW + i) * RPI + lane / LPR;
      const int c = (lane % LPR) ^ tswz(krow);
      s.idx[i] = krow;
      s.ok[i] = c * 8 < cols_valid;
      s.off[i] = (uint32_t)(c * 16 + (map ? 0 : (int64_t)krow * ld * 2));
    }
  }

  template <int R, int PW>
  __device__ static void issue_t(const Src<PW>& s, int k0, int K, lds_char* stage) {
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int k = k0 + s.idx[i];
      bool v = s.ok[i] && k < K;
      uint32_t off;
      if (T::t_map && s.map) {
        int64_t row = v ? (int64_t)s.map[s.r0 + k] : -1;
        v = v && row >= 0 && row < s.map_rows;
        off = v ? s.off[i] + (uint32_t)row * s.ld2 : kOob;
      } else {
        off = v ? s.off[i] + (uint32_t)k0 * s.ld2 : kOob;
      }
      dma16(s.rsrc, off, stage + (wave * PW + i) * 1024);
    }
  }

  // MFMA fragment of rows [row0, row0 + 32) x k-step ks (16 deep).
  __device__ static bf16x8_t frag_k(const lds_char* stage, int row0, int ks) {
    const int lane = threadIdx.x & 63;
    const int row = row0 + (lane & 31);
    const int c = 2 * ks + (lane >> 5);
    return *reinterpret_cast<const lds_bf16x8*>(stage + row * 64 + ((c ^ kswz(row)) << 4));
  }

  template <int R>
  __device__ static bf16x8_t frag_t(const lds_char* stage, int col0, int ks) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, L = lane & 15;
    const int m = col0 + 16 * (g & 1) + 4 * (L & 3);
    const int kr = 16 * ks + 8 * (g >> 1) + (L >> 2);
    const int cpos = (((m >> 3) ^ tswz(kr)) << 4) + ((m & 7) << 1);
    const bf16x4_t lo =
        __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(stage + kr * (2 * R) + cpos));
    const bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
        (lds_bf16x4*)(stage + (kr + 4) * (2 * R) + cpos));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
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
  // items (reduce). `scratch` holds 16 longs of LDS. Returns false when id is
  // past the end.
  template <int MODE>
  __device__ static bool locate(const Args& p, int id, long long* scratch, int& e_out,
                                int& local_out, int& bpre_out, int& chunks_out) {
    long long* scan = scratch;                               // kThreads / 64 + 1 entries
    int32_t* sh = reinterpret_cast<int32_t*>(scratch + 8);  // e, local, bpre, chunks
    if (threadIdx.x == 0) sh[0] = -1;
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
        sh[0] = e;
        sh[1] = id - a_pre;
        sh[2] = b_pre;
        sh[3] = chunks;
      }
      base += total;
      __syncthreads();
      if (sh[0] >= 0 || (int)(base >> 32) > id) break;
    }
    // The values are block-uniform; readfirstlane tells the compiler so, and
    // everything derived from them (operand bases, buffer resources) stays in
    // scalar registers.
    e_out = __builtin_amdgcn_readfirstlane(sh[0]);
    local_out = __builtin_amdgcn_readfirstlane(sh[1]);
    bpre_out = __builtin_amdgcn_readfirstlane(sh[2]);
    chunks_out = __builtin_amdgcn_readfirstlane(sh[3]);
    __syncthreads();  // the scratch LDS is reused by the caller
    return e_out >= 0;
  }

  // One k-tile. Tiles kt+1 .. kt+STAGES-2 may still be in flight: wait until
  // only their DMAs are outstanding (DMA completes in order), sync, hand the
  // buffer read by the previous step to tile kt+STAGES-1, then multiply.
  // Every stage buffer is a distinct LDS object, so the compiler can tell the
  // DMAs into the other buffers from the reads of `cur` and adds no waits.
  template <class Issue>
  __device__ static void step(int kt, int nk, lds_char* cur, lds_char* refill, Issue& issue,
                              f32x16_t (&acc)[FM][FN]) {
    constexpr int PT = PWA + PWB;  // DMA instructions per tile per thread
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int after = min(nk - 1 - kt, STAGES - 2);
    if (STAGES > 3 && after >= 2)
      wait_vmcnt<(STAGES > 3 ? 2 : 0) * PT>();
    else if (STAGES > 2 && after >= 1)
      wait_vmcnt<(STAGES > 2 ? 1 : 0) * PT>();
    else
      wait_vmcnt<0>();
    block_barrier();
    if (kt + STAGES - 1 < nk) issue(kt + STAGES - 1, refill);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8_t af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = T::a_k ? frag_k(cur, wm * WM + i * 32, ks) : frag_t<BM>(cur, wm * WM + i * 32, ks);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = T::b_k ? frag_k(cur + A_STAGE, wn * WN + j * 32, ks)
                        : frag_t<BN>(cur + A_STAGE, wn * WN + j * 32, ks);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          // Operands swapped: the accumulator holds C^T, so each lane owns
          // 4 consecutive n of one m and stores 8 bytes at a time.
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
    }
  }

  __device__ static void run(const Args& p, lds_char* const (&st)[STAGES]) {
    // XCD-aware remap: hardware deals workgroup ids round-robin over the 8
    // XCDs; give each XCD a contiguous range of tiles (gridDim.x % 8 == 0).
    const int g = gridDim.x, b = blockIdx.x;
    const int bid = (b % 8) * (g / 8) + b / 8;

    int e, local, split_pre, chunks;
    if (!locate<0>(p, bid, reinterpret_cast<long long*>((char*)st[STAGES - 1]), e, local, split_pre,
                   chunks))
      return;
    int mt_dim, nt_dim;
    T::tile_dims(p, e, mt_dim, nt_dim);
    const int n_tiles = cdiv(nt_dim, BN);
    const int tile = local / chunks, chunk = local % chunks;
    const int m0 = (tile / n_tiles) * BM;
    const int n0 = (tile % n_tiles) * BN;
    Prob q = T::prob(p, e);
    int kbeg = 0;
    if (chunks > 1) {
      kbeg = chunk * p.kc;
      q.K = min(q.K, kbeg + p.kc);
    }
    const int nk = q.K > kbeg ? cdiv(q.K - kbeg, BK) : 0;
    const int klen = q.K - kbeg;  // k below is relative to kbeg

    Src<PWA> sa;
    Src<PWB> sb;
    if (T::a_k)
      setup_k<BM>(sa, p.a, p.lda, p.a_map, p.a_rows, q.ar + m0, q.ac + kbeg, q.M - m0);
    else
      setup_t<BM>(sa, p.a, p.lda, p.a_map, p.a_rows, q.ar + kbeg, q.ac + m0, q.M - m0);
    if (T::b_k)
      setup_k<BN>(sb, p.b, p.ldb, nullptr, 0, q.br + n0, q.bc + kbeg, q.N - n0);
    else
      setup_t<BN>(sb, p.b, p.ldb, nullptr, 0, q.br + kbeg, q.bc + n0, q.N - n0);

    auto issue = [&](int kt, lds_char* st) {
      const int k0 = kt * BK;
      if (T::a_k) issue_k<BM>(sa, k0, klen, st); else issue_t<BM>(sa, k0, klen, st);
      if (T::b_k) issue_k<BN>(sb, k0, klen, st + A_STAGE);
      else issue_t<BN>(sb, k0, klen, st + A_STAGE);
    };

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    f32x16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
      if (s < nk) issue(s, st[s]);
    // Groups of STAGES k-tiles with every step unconditional (so the
    // accumulators stay in their registers across the loop), then the tail.
    int kt = 0;
    for (; kt + STAGES - 1 < nk; kt += STAGES) {
#pragma unroll
      for (int j = 0; j < STAGES; ++j)
        step(kt + j, nk, st[j], st[(j + STAGES - 1) % STAGES], issue, acc);
    }
#pragma unroll
    for (int j = 0; j < STAGES - 1; ++j)
      if (kt + j < nk) step(kt + j, nk, st[j], st[(j + STAGES - 1) % STAGES], issue, acc);

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
      const int64_t roff = (q.cr + m) * p.ldc + q.cc;
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
            if (p.c2)
              *reinterpret_cast<uint2*>(p.c2 + roff + n) =
                  make_uint2(pack_bf16(v0, v1), pack_bf16(v2, v3));
            v0 *= v0; v1 *= v1; v2 *= v2; v3 *= v3;
          }
          if (V == DOWN_DH && p.pre) {
            // GA = bf16(pre > 0 ? 2 * GH * pre : 0), GH the bf16-rounded dH.
            const uint2 pr = *reinterpret_cast<const uint2*>(p.pre + roff + n);
            const float p0 = lo_f32(pr.x), p1 = hi_f32(pr.x), p2 = lo_f32(pr.y), p3 = hi_f32(pr.y);
            v0 = p0 > 0.0f ? bf16_to_f32(f32_to_bf16(v0)) * 2.0f * p0 : 0.0f;
            v1 = p1 > 0.0f ? bf16_to_f32(f32_to_bf16(v1)) * 2.0f * p1 : 0.0f;
            v2 = p2 > 0.0f ? bf16_to_f32(f32_to_bf16(v2)) * 2.0f * p2 : 0.0f;
            v3 = p3 > 0.0f ? bf16_to_f32(f32_to_bf16(v3)) * 2.0f * p3 : 0.0f;
          }
          *reinterpret_cast<uint2*>(p.c + roff + n) = make_uint2(pack_bf16(v0, v1), pack_bf16(v2, v3));
        }
      }
    }
  }
};

template <int V>
__global__ __launch_bounds__(kThreads) void grouped_gemm_kernel(Args p) {
  using G = Gemm<V, Cfg<V>::BM, Cfg<V>::BN, Cfg<V>::STAGES>;
  static_assert(Cfg<V>::STAGES == 4, "the ring below declares four stage buffers");
  // Stage buffers as distinct LDS objects (see Gemm::step).
  __shared__ __align__(16) char stage0[G::STAGE];
  __shared__ __align__(16) char stage1[G::STAGE];
  __shared__ __align__(16) char stage2[G::STAGE];
  __shared__ __align__(16) char stage3[G::STAGE];
  lds_char* const st[4] = {(lds_char*)stage0, (lds_char*)stage1, (lds_char*)stage2,
                           (lds_char*)stage3};
  G::run(p, st);
}

// Sums the K-chunk partials of every split (expert, tile) in chunk order and
// stores the bf16 result. One workgroup per output tile; tiles of experts that
// were not split exit at once (their GEMM item stored bf16 directly).
template <int V>
__global__ __launch_bounds__(kThreads) void splitk_reduce_kernel(Args p) {
  constexpr int BM = Cfg<V>::BM, BN = Cfg<V>::BN;
  using G = Gemm<V, BM, BN, Cfg<V>::STAGES>;
  __shared__ long long scratch[16];
  const int g = gridDim.x, b = blockIdx.x;
  const int id = (b % 8) * (g / 8) + b / 8;
  int e, tile, split_pre, chunks;
  if (!G::template locate<1>(p, id, scratch, e, tile, split_pre, chunks)) return;
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

// GA = bf16(pre > 0 ? 2 * grad_h * pre : 0) elementwise over [rows, cols]
// (the relu^2 derivative, grouped_gemm.py:751-766), for callers that hold
// grad_h and pre_act separately.
__global__ __launch_bounds__(256) void relu2_grad_kernel(const uint16_t* __restrict__ gh,
                                                          const uint16_t* __restrict__ pre,
                                                          int64_t ld, uint16_t* __restrict__ ga,
                                                          int64_t ldo, int64_t rows,
                                                          int64_t cols) {
  const int64_t vpr = cols / 8;
  const int64_t total = rows * vpr;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / vpr, c = (i % vpr) * 8;
    const uint4 g = *reinterpret_cast<const uint4*>(gh + r * ld + c);
    const uint4 pv = *reinterpret_cast<const uint4*>(pre + r * ld + c);
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, pw[4] = {pv.x, pv.y, pv.z, pv.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float pl = lo_f32(pw[j]), ph = hi_f32(pw[j]);
      const float vl = pl > 0.0f ? lo_f32(gw[j]) * 2.0f * pl : 0.0f;
      const float vh = ph > 0.0f ? hi_f32(gw[j]) * 2.0f * ph : 0.0f;
      o[j] = pack_bf16(vl, vh);
    }
    *reinterpret_cast<uint4*>(ga + r * ldo + c) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

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
int launch(const Args& p, int64_t grid_items, hipStream_t s) {
  if (grid_items <= 0) return VMOE_OK;
  int64_t g = (grid_items + 7) / 8 * 8;
  if (g > INT32_MAX) return VMOE_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(grouped_gemm_kernel<V>, dim3((unsigned)g), dim3(kThreads), 0, s, p);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

template <int V>
int64_t tiles_max(int64_t mmax, int64_t nmax) {
  return ((mmax + Cfg<V>::BM - 1) / Cfg<V>::BM) * ((nmax + Cfg<V>::BN - 1) / Cfg<V>::BN);
}

// Upper bound of the work items of a row-tiled GEMM: sum_e ceil(tpe_e / BM)
// <= rows_bound / BM + E row tiles, each with at most ceil(nmax / BN) tiles.
template <int V>
int64_t row_items(int64_t rows_bound, int E, int64_t nmax) {
  return ((rows_bound + Cfg<V>::BM - 1) / Cfg<V>::BM + E) *
         ((nmax + Cfg<V>::BN - 1) / Cfg<V>::BN);
}

// dW GEMM with split-K: GEMM items, then the chunk reduction.
template <int V>
int launch_dw(Args p, int64_t tmax, void* ws, size_t ws_bytes, hipStream_t s) {
  constexpr int BM = Cfg<V>::BM, BN = Cfg<V>::BN;
  const int64_t E = p.E;
  if (ws) {
    const SplitPlan sp = split_plan(tmax, p.rows_bound);
    if (ws_bytes < (size_t)sp.slots * BM * BN * sizeof(float)) return VMOE_ERR_WORKSPACE;
    p.kc = sp.kc;
    p.partial = reinterpret_cast<float*>(ws);
    const int64_t items = tmax * (E + p.rows_bound / sp.kc + 1);
    int st = launch<V>(p, items, s);
    if (st) return st;
    int64_t g = (E * tmax + 7) / 8 * 8;
    if (g > INT32_MAX) return VMOE_ERR_UNSUPPORTED;
    hipLaunchKernelGGL((splitk_reduce_kernel<V>), dim3((unsigned)g), dim3(kThreads), 0, s, p);
    VMOE_CHECK_LAUNCH();
    return VMOE_OK;
  }
  p.kc = 0;
  p.partial = nullptr;
  return launch<V>(p, E * tmax, s);
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

// DMA offsets are 31-bit byte offsets from an operand base (rebased to the
// tile where rows are not gathered): every source the kernels address by a
// row index must span less than 2 GiB.
inline bool span_ok(int64_t rows, int64_t ld) { return rows * ld * 2 < ((int64_t)1 << 31); }

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
  if ((gather_map && !span_ok(x_rows, ldx)) || !span_ok(hidden, ldw1))
    return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = x; p.lda = ldx; p.a_map = gather_map; p.a_rows = gather_map ? x_rows : 0;
  p.b = w1; p.ldb = ldw1;
  p.c = out; p.c2 = activation == VMOE_ACT_RELU_SQUARED ? pre_act : nullptr; p.ldc = ldo;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = activation; p.rows_bound = rows_bound;
  return launch<UP_FWD>(p, row_items<UP_FWD>(rows_bound, E, max_width),
                        reinterpret_cast<hipStream_t>(stream));
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
  if (!span_ok(max_width, ldw2)) return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = h; p.lda = ldh;
  p.b = w2; p.ldb = ldw2;
  p.c = y; p.ldc = ldy;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = VMOE_ACT_NONE; p.rows_bound = rows_bound;
  return launch<DOWN_FWD>(p, row_items<DOWN_FWD>(rows_bound, E, hidden),
                          reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vmoe_relu2_grad(const uint16_t* grad_h, const uint16_t* pre_act, int64_t ld,
                               uint16_t* grad_act, int64_t ldo, int64_t rows, int64_t cols,
                               vmoe_stream_t stream) {
  if (rows < 0 || cols < 0 || ld < cols || ldo < cols) return VMOE_ERR_INVALID_ARG;
  if (rows == 0 || cols == 0) return VMOE_OK;
  if (!grad_h || !pre_act || !grad_act) return VMOE_ERR_INVALID_ARG;
  if (cols % 8 || ld % 8 || ldo % 8 || !a16(grad_h) || !a16(pre_act) || !a16(grad_act))
    return VMOE_ERR_UNSUPPORTED;
  const int64_t n = rows * (cols / 8);
  const int64_t grid = std::min<int64_t>((n + 255) / 256, 65536);
  hipLaunchKernelGGL(relu2_grad_kernel, dim3((unsigned)grid), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), grad_h, pre_act, ld, grad_act, ldo,
                     rows, cols);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

extern "C" int vmoe_gemm_up_bwd_dx(const uint16_t* grad_act, int64_t ldg, const uint16_t* w1,
                                   int64_t ldw1, uint16_t* grad_x, int64_t ldgx,
                                   const int32_t* eto, const int32_t* ewo, const int32_t* widths,
                                   const int32_t* tpe, int32_t E, int64_t hidden,
                                   int64_t max_width, int64_t rows_bound, vmoe_stream_t stream) {
  int st = check_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (!grad_act || !w1 || !grad_x) return VMOE_ERR_INVALID_ARG;
  if (!ld_ok(ldg) || !ld_ok(ldw1) || !ld_ok(ldgx) || ldgx < hidden) return VMOE_ERR_UNSUPPORTED;
  if (!a16(grad_act) || !a16(w1) || !a16(grad_x)) return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = grad_act; p.lda = ldg;
  p.b = w1; p.ldb = ldw1;
  p.c = grad_x; p.ldc = ldgx;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = VMOE_ACT_NONE; p.rows_bound = rows_bound;
  return launch<UP_DX>(p, row_items<UP_DX>(rows_bound, E, hidden),
                       reinterpret_cast<hipStream_t>(stream));
}

extern "C" size_t vmoe_gemm_dw_workspace_bytes(int32_t E, int64_t hidden, int64_t max_width,
                                               int64_t rows_bound) {
  if (E <= 0 || hidden <= 0 || max_width <= 0 || rows_bound <= 0) return 0;
  const SplitPlan a = split_plan(tiles_max<UP_DW>(hidden, max_width), rows_bound);
  const SplitPlan b = split_plan(tiles_max<DOWN_DW>(max_width, hidden), rows_bound);
  const size_t tile_a = (size_t)Cfg<UP_DW>::BM * Cfg<UP_DW>::BN * sizeof(float);
  const size_t tile_b = (size_t)Cfg<DOWN_DW>::BM * Cfg<DOWN_DW>::BN * sizeof(float);
  return std::max((size_t)a.slots * tile_a, (size_t)b.slots * tile_b);
}

extern "C" int vmoe_gemm_up_bwd_dw(const uint16_t* x, int64_t ldx, int64_t x_rows,
                                   const int32_t* gather_map, const uint16_t* grad_act,
                                   int64_t ldg, uint16_t* grad_w1, int64_t ldgw,
                                   const int32_t* eto, const int32_t* ewo, const int32_t* widths,
                                   const int32_t* tpe, int32_t E, int64_t hidden,
                                   int64_t max_width, int64_t rows_bound, void* workspace,
                                   size_t workspace_bytes, vmoe_stream_t stream) {
  int st = check_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (!x || !grad_act || !grad_w1 || x_rows < 0) return VMOE_ERR_INVALID_ARG;
  if (!ld_ok(ldx) || !ld_ok(ldg) || !ld_ok(ldgw) || ldx < hidden) return VMOE_ERR_UNSUPPORTED;
  if (!a16(x) || !a16(grad_act) || !a16(grad_w1)) return VMOE_ERR_UNSUPPORTED;
  if (!span_ok(gather_map ? x_rows : rows_bound, ldx) || !span_ok(rows_bound, ldg))
    return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = x; p.lda = ldx; p.a_map = gather_map; p.a_rows = gather_map ? x_rows : 0;
  p.b = grad_act; p.ldb = ldg;
  p.c = grad_w1; p.ldc = ldgw;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = VMOE_ACT_NONE; p.rows_bound = rows_bound;
  return launch_dw<UP_DW>(p, tiles_max<UP_DW>(hidden, max_width), workspace, workspace_bytes,
                          reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vmoe_gemm_down_bwd_dh(const uint16_t* grad_y, int64_t ldgy, const uint16_t* w2,
                                     int64_t ldw2, const uint16_t* pre_act, uint16_t* grad_h,
                                     int64_t ldgh, const int32_t* eto, const int32_t* ewo,
                                     const int32_t* widths, const int32_t* tpe, int32_t E,
                                     int64_t hidden, int64_t max_width, int64_t rows_bound,
                                     vmoe_stream_t stream) {
  int st = check_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (!grad_y || !w2 || !grad_h) return VMOE_ERR_INVALID_ARG;
  if (!ld_ok(ldgy) || !ld_ok(ldw2) || !ld_ok(ldgh) || ldgy < hidden || ldw2 < hidden ||
      ldgh < max_width)
    return VMOE_ERR_UNSUPPORTED;
  if (!a16(grad_y) || !a16(w2) || !a16(grad_h) || (pre_act && !a16(pre_act)))
    return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = grad_y; p.lda = ldgy;
  p.b = w2; p.ldb = ldw2;
  p.c = grad_h; p.ldc = ldgh;
  p.pre = pre_act;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = VMOE_ACT_NONE; p.rows_bound = rows_bound;
  return launch<DOWN_DH>(p, row_items<DOWN_DH>(rows_bound, E, max_width),
                         reinterpret_cast<hipStream_t>(stream));
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
  if (!span_ok(rows_bound, ldh) || !span_ok(rows_bound, ldgy)) return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = h; p.lda = ldh;
  p.b = grad_y; p.ldb = ldgy;
  p.c = grad_w2; p.ldc = ldgw;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = VMOE_ACT_NONE; p.rows_bound = rows_bound;
  return launch_dw<DOWN_DW>(p, tiles_max<DOWN_DW>(max_width, hidden), workspace,
                            workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}
