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
//  * Persistent grid, one 768-thread workgroup per CU. Each workgroup builds
//    the per-expert work table (tiles x K chunks, exclusive prefix) in LDS
//    from the same metadata the reference reads, so no host sync is needed
//    and empty experts cost nothing. Row-tiled GEMMs: XCD x owns a
//    contiguous eighth of the work items (the tiles of one expert share that
//    XCD's L2) and its workgroups take every (grid / 8)-th item. dW GEMMs:
//    lanes of 4 or 8 workgroups (by shape, lane_shift) on one XCD take
//    contiguous item ranges (see item_range).
//  * 128x256 output tiles; 8 consumer waves in a 2x4 grid, 64x64 fp32
//    accumulators per wave (two consumer waves per SIMD), and 4 producer
//    waves that issue every DMA.
//  * Every operand tile goes global -> LDS by DMA (buffer_load ... lds, 16
//    bytes per lane), never through VGPRs, in a 4-stage ring; the k-tiles of
//    all items of a workgroup form one stream, so the next item's first
//    stages load while the current item finishes and stores its tile.
//      - K-contiguous sources (activations in the forward, W in dX/dH) land
//        in "K-form": one 64-byte row per m (n), 16-byte chunk c of row r at
//        c ^ ((r >> 2) & 3); MFMA fragments are one ds_read_b128.
//      - M/N-contiguous sources (W1/W2 in the forward, both dW operands)
//        land as they are in memory ("T-form": one row per k), chunk c of
//        k-row k at c ^ (4 (k & 3) | 2 ((k >> 3) & 1)); fragments are two
//        ds_read_b64_tr_b16, the gfx950 LDS transpose read, so no operand is
//        transposed in registers. Both swizzles make the fragment reads
//        bank-conflict free (64 banks of 4 bytes).
//  * Epilogues: relu and relu^2 of the fp32 accumulator (PRE, H) for the up
//    projection (grouped_gemm.py:336-346); for the down dH GEMM an optional
//    fused relu^2 gradient GA = bf16(pre > 0 ? 2 * bf16(acc) * pre : 0)
//    (grouped_gemm.py:751-766), so dX and dW read GA directly; split-K fp32
//    partial tiles for the dW GEMMs, summed in chunk order by the wave that
//    finishes a tile's last segment.

#include <algorithm>
#include <atomic>

#include "vmoe_common.h"

namespace vmoe {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4;
typedef __attribute__((address_space(3))) bf16x8_t lds_bf16x8;
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Workgroup roles: consumer waves (two per SIMD, so one hides the other's
// LDS latency) read the staged tiles, run the MFMAs and store the results;
// producer waves (one per SIMD) issue every DMA and do every wait on it.
// The wait counter of a wave (vmcnt) counts its loads and stores together,
// so keeping the DMAs out of the consumers means their stores never hold
// up the pipeline.
constexpr int kConsumers = 8;
constexpr int kProducers = 4;
constexpr int kWaves = kConsumers + kProducers;
constexpr int kThreads = kWaves * 64;
constexpr int kMaxExperts = 2048;  // per-expert work prefix held in LDS
constexpr int kRecExperts = 256;   // per-expert metadata also held in LDS up to this E
// dW GEMMs: the workgroups of one XCD that share each K chunk form a lane of
// 1 << p.lsh of them (lane_shift: 4, or 8 for large d x w tiles per expert)
constexpr int kMaxLaneShift = 3;
constexpr int kMaxLanes = 64;      // dW GEMMs: lanes (grid >> lsh) a launch may have
constexpr int kMaxDwGrid = kMaxLanes << 2;  // dW grid limit (lanes of 4 fill lane_beg)

enum Variant { UP_FWD = 0, DOWN_FWD, UP_DX, UP_DW, DOWN_DH, DOWN_DW, UP_GLU };

struct Args {
  const uint16_t* a;     // A source
  int64_t lda;
  const int32_t* a_map;  // row gather for A (fused gather), nullable
  int64_t a_rows;        // rows of the gathered source
  const uint16_t* b;
  int64_t ldb;
  uint16_t* c;
  int64_t ldc;
  uint16_t* c2;          // UP_FWD: pre_act output; UP_GLU: gate output (nullable)
  uint16_t* c3;          // UP_GLU: up output (nullable); c, c2 and c3 share ldc
  const uint16_t* pre;   // DOWN_DH: pre_act input -> fused relu^2 gradient (nullable)
  const int32_t* b_map;  // row gather for B (T-form; no variant uses it), nullable
  int64_t b_rows;        // rows of B's gathered source
  const float* row_scale;  // UP_FWD / DOWN_DH: per-row factor of the output (nullable)
  const uint16_t* gscale;  // DOWN_DH / DOWN_DW: bf16 scalar factor of the output (nullable)
  const int32_t* eto;
  const int32_t* ewo;
  const int32_t* widths;
  const int32_t* tpe;
  int E;
  int hidden;
  int act;
  int64_t rows_bound;
  int kc;          // K rows per work item for the dW GEMMs (0 = whole K)
  int lsh = 2;     // dW GEMMs: log2 of the workgroups per lane (lane_shift)
  float* partial;    // fp32 partial tiles of split tiles (2 slots per workgroup)
  uint32_t* arrive;  // split-K arrival words, kConsumers per workgroup (zero between launches)
  int grid;          // GEMM workgroups
  int paired;        // 1: one of the two GEMMs of grouped_gemm_pair_kernel (see vblock)
  float* row_dot;    // DOWN_DH with pre: per (row, 64-column block) sum of GH * PRE^2 (nullable)
  int64_t ld_rd;     // its leading dimension (floats)
};

// Metadata of one expert as the GEMMs read it: its row range [t0, t1) in
// the expert-sorted layout (t1 clipped to rows_bound), its routed-row count,
// its weight column range [ew0, ew1) and its width.
struct ExpertRec {
  int t0, t1, tpe, ew0, ew1, w;
};

// The same through the scalar cache, for a uniform e: a load from the
// constant address space at a uniform index compiles to s_load, which
// completes on lgkmcnt. Vector loads in a producer wave would make the
// compiler wait for them with vmcnt(0), which also drains the DMAs in flight
// (the compiler does not count them).
__device__ __forceinline__ int32_t sload(const int32_t* ptr, int idx) {
  typedef __attribute__((address_space(4))) const int32_t cint;
  return ((cint*)ptr)[__builtin_amdgcn_readfirstlane(idx)];
}

__device__ __forceinline__ ExpertRec rec_scalar(const Args& p, int e) {
  ExpertRec r;
  r.t0 = sload(p.eto, e);
  r.t1 = (int)min<int64_t>(sload(p.eto, e + 1), p.rows_bound);
  r.tpe = sload(p.tpe, e);
  r.ew0 = sload(p.ewo, e);
  r.ew1 = sload(p.ewo, e + 1);
  r.w = sload(p.widths, e);
  return r;
}

__device__ __forceinline__ ExpertRec rec_global(const Args& p, int e) {
  ExpertRec r;
  r.t0 = p.eto[e];
  r.t1 = (int)min<int64_t>(p.eto[e + 1], p.rows_bound);
  r.tpe = p.tpe[e];
  r.ew0 = p.ewo[e];
  r.ew1 = p.ewo[e + 1];
  r.w = p.widths[e];
  return r;
}

// Per-expert problem: valid extents and operand origins.
//   A K-contig:  A(m,k) = a[(ar + m) * lda + ac + k]
//   A MN-contig: A(m,k) = a[row(ar + k) * lda + ac + m]
//   B K-contig:  B(k,n) = b[(br + n) * ldb + bc + k]
//   B MN-contig: B(k,n) = b[(br + k) * ldb + bc + n]
//   C(m,n) = c[(cr + m) * ldc + cc + n]
struct Prob {
  int M, N, K;
  int ar, ac, br, bc, cr, cc;
};

__device__ __forceinline__ int clamp0(int v) { return max(0, v); }

template <int V>
struct Traits;

template <>
struct Traits<UP_FWD> {
  static constexpr bool k_map = true;  // A rows may come through the gather map
  static constexpr bool t_map = false, t_map_b = false;
  static constexpr bool a_k = true, b_k = false;
  __device__ static Prob prob(const Args& p, const ExpertRec& r) {
    Prob q;
    q.M = clamp0(min(r.tpe, r.t1 - r.t0));
    q.N = clamp0(r.w);
    q.K = p.hidden;
    q.ar = r.t0; q.ac = 0;
    q.br = 0; q.bc = r.ew0;  // B(k,n) = W1[k][ewo + n]
    q.cr = r.t0; q.cc = 0;
    return q;
  }
};

// SwiGLU up projection (the reference's ACTIVATION == 2 path,
// grouped_gemm.py:293-349): the B tile's 256 staged columns are the gate
// columns W1[:, ewo + n] and the up columns W1[:, ewo + w + n] of 128 output
// columns n, interleaved per 32 (setup_glu), so that each consumer wave
// holds gate and up of the same 32 outputs in its two accumulator blocks.
template <>
struct Traits<UP_GLU> : Traits<UP_FWD> {};

template <>
struct Traits<DOWN_FWD> {
  static constexpr bool k_map = false;
  static constexpr bool t_map = false, t_map_b = false;
  static constexpr bool a_k = true, b_k = false;
  __device__ static Prob prob(const Args& p, const ExpertRec& r) {
    Prob q;
    q.M = clamp0(min(r.tpe, r.t1 - r.t0));
    q.N = p.hidden;
    q.K = clamp0(r.ew1 - r.ew0);
    q.ar = r.t0; q.ac = 0;
    q.br = r.ew0; q.bc = 0;  // B(k,n) = W2[ewo + k][n]
    q.cr = r.t0; q.cc = 0;
    return q;
  }
};

template <>
struct Traits<UP_DX> {
  static constexpr bool k_map = false;
  static constexpr bool t_map = false, t_map_b = false;
  static constexpr bool a_k = true, b_k = true;
  __device__ static Prob prob(const Args& p, const ExpertRec& r) {
    Prob q;
    q.M = clamp0(min(r.tpe, r.t1 - r.t0));
    q.N = p.hidden;
    q.K = clamp0(r.ew1 - r.ew0);
    q.ar = r.t0; q.ac = 0;   // A(m,k) = GA[t0 + m][k]
    q.br = 0; q.bc = r.ew0;  // B(k,n) = W1[n][ewo + k]
    q.cr = r.t0; q.cc = 0;
    return q;
  }
};

template <>
struct Traits<UP_DW> {
  static constexpr bool k_map = false;
  static constexpr bool a_k = false, b_k = false;
  static constexpr bool t_map = true;  // A rows may come through the gather map
  static constexpr bool t_map_b = false;
  __device__ static Prob prob(const Args& p, const ExpertRec& r) {
    Prob q;
    q.M = p.hidden;
    q.N = clamp0(r.w);
    q.K = clamp0(r.t1 - r.t0);
    q.ar = r.t0; q.ac = 0;  // A(m,k) = X[row(t0 + k)][m]
    q.br = r.t0; q.bc = 0;  // B(k,n) = GA[t0 + k][n]
    q.cr = 0; q.cc = r.ew0;
    return q;
  }
};

template <>
struct Traits<DOWN_DH> {
  static constexpr bool k_map = true;  // A (the output gradient) may come through the map
  static constexpr bool t_map = false, t_map_b = false;
  static constexpr bool a_k = true, b_k = true;
  __device__ static Prob prob(const Args& p, const ExpertRec& r) {
    Prob q;
    q.M = clamp0(min(r.tpe, r.t1 - r.t0));
    q.N = clamp0(r.w);
    q.K = p.hidden;
    q.ar = r.t0; q.ac = 0;
    q.br = r.ew0; q.bc = 0;  // B(k,n) = W2[ewo + n][k]
    q.cr = r.t0; q.cc = 0;
    return q;
  }
};

template <>
// grad_w2 is computed transposed, C' = GY^T H (m over hidden, n over the
// expert's width), so the row-mapped operand is A, the narrower one (two
// DMAs per producer wave per stage instead of four), as in UP_DW; the
// epilogue stores C' transposed into grad_w2[ew0 + n][m].
struct Traits<DOWN_DW> {
  static constexpr bool k_map = false;
  static constexpr bool t_map = true;  // A (the output gradient) may come through the map
  static constexpr bool t_map_b = false;
  static constexpr bool a_k = false, b_k = false;
  __device__ static Prob prob(const Args& p, const ExpertRec& r) {
    Prob q;
    q.M = p.hidden;
    q.N = clamp0(r.w);
    q.K = clamp0(r.t1 - r.t0);
    q.ar = r.t0; q.ac = 0;  // A(m,k) = GY[row(t0 + k)][m]
    q.br = r.t0; q.bc = 0;  // B(k,n) = H[t0 + k][n]
    q.cr = r.ew0; q.cc = 0;  // C'(m,n) -> grad_w2[cr + n][cc + m]
    return q;
  }
};

// Tile shape: 128x256 output tiles, the 8 consumer waves in a 2 (m) x 4 (n)
// grid of 64x64 fp32 accumulators each (64 registers, so three waves fit a
// SIMD). N = 256 covers a whole 256-wide expert in the up projection. The
// dW GEMMs split their long K (the expert's rows) into chunks and accumulate
// a tile across consecutive chunks ("contig"); the row-tiled GEMMs deal
// items round-robin.
//
// k per LDS stage (BK) and ring depth. A K-contiguous ("K-form") operand row
// of a stage is BK * 2 bytes; 128-byte rows (BK = 64) would halve the L2
// requests per byte, but within the LDS budget they allow only a 2-deep
// ring of 48 KiB stages, and that measured slower on every variant than
// BK = 32 in a 4-deep ring of 24 KiB stages (the per-stage wait is exposed).
template <int V>
struct Cfg {
  static constexpr int BM = 128, BN = 256;
  static constexpr int WGM = 2, WGN = 4;
  static constexpr bool contig = V == UP_DW || V == DOWN_DW;
  static constexpr int BK = 32;
  static constexpr int STAGES = 4;
};

__host__ __device__ constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }

// Output columns of a tile: BN, except UP_GLU, whose BN staged columns are
// the gate and up halves of BN / 2 outputs.
template <int V>
__host__ __device__ constexpr int out_cols() { return V == UP_GLU ? Cfg<V>::BN / 2 : Cfg<V>::BN; }

// Split-K chunk of the dW GEMMs: K rows per work item (p.kc is 0 or this).
// Small chunks let the contiguous item ranges balance experts of very
// different row counts; the chunks of one tile inside one range accumulate
// in registers, so the chunk size does not change the partial traffic (at
// most two partial tiles per workgroup).
constexpr int kDwChunk = 512;

// Output tiles and K chunks of expert e (chunks > 1 only for the split-K dW
// GEMMs, p.kc > 0). Every divisor is a compile-time power of two.
template <int V>
__device__ __forceinline__ void expert_work(const Args& p, const Prob& q, int& tiles,
                                            int& chunks) {
  constexpr int BM = Cfg<V>::BM, BN = out_cols<V>();
  tiles = (q.M > 0 && q.N > 0) ? cdiv(q.M, BM) * cdiv(q.N, BN) : 0;
  chunks = (Cfg<V>::contig && p.kc > 0 && tiles > 0 && q.K > kDwChunk) ? cdiv(q.K, kDwChunk) : 1;
}

// x / d for 0 <= x < 2^22 and 1 <= d < 2^22: the float reciprocal estimate
// is within one of the quotient and one correction each way makes it exact
// (a 32-bit integer division is a long instruction sequence, and the work
// decoder runs on the critical path of every item).
__device__ __forceinline__ int udiv_small(int x, int d) {
  int q = (int)((float)x * __builtin_amdgcn_rcpf((float)d));
  q -= q * d > x ? 1 : 0;
  q += (q + 1) * d <= x ? 1 : 0;
  return q;
}

// sigmoid in fp32, 1 / (1 + exp(-x)) with the precise exp.
__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

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

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base,
                                                          int bytes = 0x7FFFFFFF) {
  // The base is block-uniform; readfirstlane keeps the resource in SGPRs
  // (a VGPR resource would force a waterfall loop around every DMA).
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void* b = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(b, 0, __builtin_amdgcn_readfirstlane(bytes),
                                           0x00020000);
}

// 16-byte DMA of the lane's source into LDS at lds + 16 * lane
// (buffer_load_dwordx4 ... lds; lds is a uniform LDS byte address, written to
// M0). Issued as inline asm so the
// compiler does not track it: it would otherwise wait for every DMA before
// any LDS read it cannot prove disjoint, which empties the ring. The kernels
// order DMA completion themselves with wait_vmcnt + block_barrier. The asm
// has no register outputs (the data goes to LDS), so no register is written
// behind the compiler's back; M0 is declared clobbered.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :: "v"(voff), "s"(r), "s"(lds) : "memory", "m0");
}

// 4-byte DMA of the lane's source into LDS at dst + 4 * lane (the row-map
// windows of the T-form gather), under the same rules as dma16.
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, uint32_t voff, lds_char* dst) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(dst));
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dword %0, %1, 0 offen lds"
               :: "v"(voff), "s"(r), "s"(lds) : "memory", "m0");
}

// Work items of an expert with `tiles` output tiles and `chunks` K chunks.
// Row-tiled GEMMs: one item per tile. dW GEMMs: the tiles form groups of
// 1 << lsh and an item is (tile group, chunk); the workgroups of a lane (all
// on one XCD) each take one tile of the group, so they read the same K chunk
// of the shared operand at the same time and it comes from HBM once.
template <int V>
__host__ __device__ __forceinline__ int work_items(int tiles, int chunks, int lsh) {
  return Cfg<V>::contig ? ((tiles + (1 << lsh) - 1) >> lsh) * chunks : tiles * chunks;
}

// Per-expert tables of a launch, built once per workgroup: the exclusive
// prefix of work items (pre[E] = total) and, for E <= kRecExperts, the
// expert records themselves.
struct Meta {
  int pre[kMaxExperts + 1];
  int rec[6][kRecExperts];
  // dW GEMMs: first item of each lane (lane_beg[NL] = total); row-tiled
  // GEMMs: first item of each XCD's range (lane_beg[8] = total)
  int lane_beg[kMaxLanes + 1];
};

// Work-item range of workgroup b. Round-robin: XCD x (hardware deals
// workgroup b to XCD b % 8) owns the contiguous range [lane_beg[x],
// lane_beg[x + 1]) of items, an eighth of the estimated cost (see
// build_meta), so the tiles of one expert share an L2, and its
// workgroups take every (grid / 8)-th item. Contig (lanes of L = 1 << lsh
// workgroups, grid a multiple of 8 L): the j-th workgroup of XCD x
// (j = b / 8) is slot j % L of lane l = x * (grid / 8 / L) + j / L; lane l
// owns items [lane_beg[l], lane_beg[l + 1]) of the NL = grid / L lanes
// (equal shares of the k-steps, see build_meta), and its slot s works on
// tile L * group + s of each. lin = L * l + s names the workgroup's split-K
// partial slots.
struct Range {
  int beg, end, stride, lin, slot;
};

// The workgroup's index among the p.grid workgroups of its GEMM. A paired
// launch (grouped_gemm_pair_kernel) deals consecutive groups of 8 workgroups
// to its two GEMMs in turn, so each GEMM holds p.grid = gridDim.x / 2 of them,
// the same number on every XCD, and its k-th workgroup still sits on XCD
// k mod 8.
__device__ __forceinline__ int vblock(const Args& p) {
  const int b = blockIdx.x;
  return p.paired ? ((b >> 4) << 3) | (b & 7) : b;
}

template <bool CONTIG>
__device__ __forceinline__ Range item_range(const Args& p, int total, const int* lane_beg) {
  const int G = p.grid, b = vblock(p);
  const int xcd = b & 7, per = G >> 3, j = b >> 3;
  Range r;
  r.lin = xcd * per + j;
  r.slot = 0;
  if (CONTIG) {
    const int NL = G >> p.lsh;
    const int lane = xcd * (NL >> 3) + (j >> p.lsh);
    r.slot = j & ((1 << p.lsh) - 1);
    r.lin = (lane << p.lsh) + r.slot;
    r.beg = lane_beg[lane];
    r.end = lane_beg[lane + 1];
    r.stride = 1;
  } else {
    r.beg = lane_beg[xcd] + j;
    r.end = lane_beg[xcd + 1];
    r.stride = per;
  }
  return r;
}

template <int V>
struct Gemm {
  using T = Traits<V>;
  static constexpr int BM = Cfg<V>::BM, BN = Cfg<V>::BN;
  static constexpr int WGM = Cfg<V>::WGM, WGN = Cfg<V>::WGN;
  static_assert(WGM * WGN == kConsumers, "one consumer wave per wave-grid cell");
  static constexpr int BK = Cfg<V>::BK, kStages = Cfg<V>::STAGES;
  static constexpr int WM = BM / WGM, WN = BN / WGN;  // wave tile
  static constexpr int FM = WM / 32, FN = WN / 32;    // 32x32 blocks per wave
  static constexpr int A_STAGE = BM * BK * 2, B_STAGE = BN * BK * 2;  // bytes
  static constexpr int STAGE = A_STAGE + B_STAGE;
  // The GEMMs that store a [rows, d] output (DOWN_FWD, UP_DX) stage their
  // K-contiguous A operand two k-steps at a time: one 128-byte request per
  // row instead of two 64-byte ones, which halves the address-queue slots
  // those loads take from the epilogue stores (2-3 us each at cfg3; the
  // other row-tiled GEMMs gain nothing from it). A pair slot holds blocks of 8 rows, each the 8 rows' 64 bytes of
  // the even k-step, then of the odd one; kPairSlots slots keep the ring's
  // lookahead (a pair is refilled kStages - 1 stages ahead, as one stage
  // is). Items then have an even number of k-steps (an odd one gets a k-step
  // of zeros), so pairs never straddle items. The ring is the A pair slots,
  // then kStages B stages; otherwise kStages stages of A then B.
  static constexpr bool PAIR_A = V == DOWN_FWD || V == UP_DX;
  static constexpr int kPairSlots = 3;
  static constexpr int A_RING = PAIR_A ? kPairSlots * 2 * A_STAGE : 0;
  static constexpr int RING = PAIR_A ? A_RING + kStages * B_STAGE : kStages * STAGE;
  template <typename P>
  __device__ static P* a_at(P* ring, int s) {
    return PAIR_A ? ring + ((s >> 1) % kPairSlots) * (2 * A_STAGE) : ring + (s % kStages) * STAGE;
  }
  template <typename P>
  __device__ static P* b_at(P* ring, int s) {
    return PAIR_A ? ring + A_RING + (s % kStages) * B_STAGE
                  : ring + (s % kStages) * STAGE + A_STAGE;
  }
  // DMA instructions per producer wave per stage for an operand of R rows/cols.
  template <int R>
  struct Dma {
    static constexpr int INSTS = R * BK * 2 / 1024;
    static constexpr int PW = INSTS / kProducers;
    static constexpr int LPR = R / 8;     // T-form: lanes per k-row
    static constexpr int RPI = 64 / LPR;  // T-form: k-rows per instruction
    static_assert(INSTS % kProducers == 0 && PW >= 1, "tile too small for the producers");
    static_assert(RPI >= 1, "T-form k-row wider than one DMA instruction");
  };
  static constexpr int PWA = Dma<BM>::PW, PWB = Dma<BN>::PW;
  static constexpr int PT = PWA + PWB;  // DMA instructions per stage per producer thread
  static constexpr int PWA_S = PAIR_A ? 2 * PWA : PWA;  // A DMAs per issue (a pair: two stages)
  __device__ static int pwave() { return (threadIdx.x >> 6) - kConsumers; }

  // LDS address of this wave's first DMA slot of an operand stage, uniform:
  // DMA i of the wave then writes at lds_slot + 1024 i (scalar adds). Every
  // vector instruction a producer issues between a barrier and its DMAs
  // competes with the consumers' MFMAs for the SIMD and delays the stage, so
  // the per-DMA work is one vector op (the offset) where possible.
  template <int PW>
  __device__ static uint32_t lds_slot(lds_char* stage) {
    return __builtin_amdgcn_readfirstlane(
        (uint32_t)reinterpret_cast<uintptr_t>(stage + pwave() * PW * 1024));
  }

  // LDS is 64 banks x 4 bytes; a ds_read_b128 serves 16 lanes per cycle and
  // a ds_read_b64_tr_b16 32 lanes per cycle. K-form: a row is KCH 16-byte
  // chunks and the 16 rows one phase reads share 256-byte bank lines
  // (KCH = 4: four rows per line; KCH = 8: two), so the chunk is XORed with
  // (row / (16 / KCH)) mod KCH to give the 16 rows distinct 16-byte slots.
  // T-form: one phase reads k-rows k..k+3 at two column offsets 32 bytes
  // apart, so the chunk is XORed with 4 * (k % 4) (distinct 64-byte slots
  // per k-row) and with 2 * ((k / 8) % 2) for the other phase's k-rows.
  static constexpr int KCH = BK * 2 / 16;  // 16-byte chunks per K-form row
  static constexpr int KRPI = 64 / KCH;    // K-form rows per DMA instruction
  static_assert(KCH == 4 || KCH == 8, "K-form rows of 64 or 128 bytes");
  __device__ static int kswz(int r) { return KCH == 4 ? (r >> 2) & 3 : (r >> 1) & 7; }
  __device__ static int tswz(int k) { return ((k & 3) << 2) | (((k >> 3) & 1) << 1); }
  static_assert(BM >= 128 && BN >= 128, "T-form swizzle needs 16 chunks per k-row");

  // Per-thread DMA state of one operand: a buffer resource over the
  // operand (rebased to the tile where no row map is used) and one 32-bit
  // byte offset per DMA instruction.
  template <int PW>
  struct Src {
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t ld2;        // leading dimension in bytes
    uint32_t off[PW];    // K-form: row + chunk; T-form: chunk column (+ k-row without map)
    int idx[PW];         // K-form: k of the lane's chunk; T-form: the lane's k-row
    bool ok[PW];         // K-form: row valid; T-form: column valid
  };
  // T-form row gather (the A operand of the up dW GEMM, B of the down dW
  // GEMM). Each producer wave stages the map entries of its k-rows for
  // kWinStages stages of an item in a 512-byte LDS window (lane l of window
  // DMA h fetches the entry of stage 8 h + l / 8, row 8 * wave + l % 8), by
  // DMA like the operand tiles, so the ring's vmcnt waits order it too. The
  // window of the next item loads while the current one streams (two windows
  // per wave); a scalar load of the entries instead waits on the scalar cache
  // once per stage. A split-K item (kDwChunk rows) fits one window: refilling
  // a window in the middle of an item has to drain every DMA in flight.
  static constexpr int kWinStages = 16;
  static constexpr int kWinBytes = kWinStages * 8 * 4;
  // Row factors of the output (UP_FWD, DOWN_DH): one slot of BM floats per
  // item. The producers set an item up right after issuing the previous
  // item's last stage, kStages - 1 stages ahead of the consumers, and every
  // item has at least one stage, so the slot of item n - kStages - 1 is the
  // newest one a consumer can still be reading.
  static constexpr bool kScaled = V == UP_FWD || V == UP_GLU || V == DOWN_DH;
  static constexpr int kScaleSlots = kStages + 1;
  struct TMap {
    __amdgpu_buffer_rsrc_t mrs;  // over the row map
    lds_char* win;               // this wave's window of the current item
    int64_t mbase;               // map index of the item's first k-row
    int klen;                    // k-rows of the item
    uint32_t rows;               // rows of the gathered source
    int pf_kt;                   // stage whose entries are in pf (-1: none)
    int32_t pf[4];               // the lane's entries of stage pf_kt, read a stage ahead
    bool on;
  };
  static_assert(BK / kProducers == 8 && kWinStages * 8 == 128,
                "window: 8 k-rows per producer wave per stage, two DMA instructions");

  // K-form setup: rows [0, R) of the tile (source rows r0 + row, or
  // map[r0 + row]), rows_valid of them real, k measured from column c0.
  template <int R, int PW, bool PAIR>
  __device__ static void setup_k(Src<PW>& s, const uint16_t* base, int64_t ld,
                                 const int32_t* map, int64_t map_rows, int64_t r0, int64_t c0,
                                 int rows_valid, const lds_char* win) {
    const int lane = threadIdx.x & 63, wave = pwave();
    // Without a map, rebase to the tile's first row so offsets stay small.
    if (!T::k_map) map = nullptr;
    const uint16_t* b = map ? base + c0 : base + r0 * ld + c0;
    s.rsrc = make_rsrc(b);
    s.ld2 = (uint32_t)(ld * 2);
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      // PAIR: instruction i covers rows 8 (wave PW + i) .. +7; lanes 0-31
      // the even k-step's 64 bytes of them, lanes 32-63 the odd one's.
      const int lr = PAIR ? i * 8 + ((lane & 31) >> 2) : i * KRPI + lane / KCH;  // wave-local row
      const int row = wave * (PAIR ? PW * 8 : PW * KRPI) + lr;
      const int c = PAIR ? (lane & 3) ^ ((row >> 2) & 3) : (lane % KCH) ^ kswz(row);
      const int k = PAIR ? (lane >> 5) * BK + c * 8 : c * 8;
      bool ok = row < rows_valid;
      int64_t srow = row;
      if (T::k_map && map && ok) {
        // One entry per lane, once per item (the K-form rows are fixed for
        // all of the item's k-tiles), from the wave's map window.
        srow = reinterpret_cast<const __attribute__((address_space(3))) int32_t*>(win)[lr];
        ok = srow >= 0 && srow < map_rows;
      }
      s.ok[i] = ok;
      s.idx[i] = k;
      s.off[i] = ok ? (uint32_t)((srow * ld + k) * 2) : kOob;
    }
  }

  // K-form issue: stage tile k0 .. k0 + BK (k0 relative to the setup's c0).
  // Invalid rows hold offset kOob, which stays out of range after adding k0
  // (offsets are below 2^31), so a stage inside K needs one add per DMA.
  template <int R, int PW, bool PAIR>
  __device__ static void issue_k(const Src<PW>& s, int k0, int K, lds_char* stage) {
    const uint32_t m0 = lds_slot<PW>(stage);
    if (k0 + (PAIR ? 2 * BK : BK) <= K) {
#pragma unroll
      for (int i = 0; i < PW; ++i) dma16(s.rsrc, s.off[i] + (uint32_t)(k0 * 2), m0 + i * 1024);
      return;
    }
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const bool v = s.ok[i] & (k0 + s.idx[i] < K);
      dma16(s.rsrc, v ? s.off[i] + (uint32_t)(k0 * 2) : kOob, m0 + i * 1024);
    }
  }

  // T-form setup: columns [0, R) of the tile starting at source column c0,
  // cols_valid of them real; source rows r0 + k, or map[r0 + k] (a map entry
  // outside [0, map_rows) reads zeros).
  template <int R, int PW, bool MAP>
  __device__ static void setup_t(Src<PW>& s, TMap& tm, const uint16_t* base, int64_t ld,
                                 const int32_t* map, int64_t map_rows, int64_t r0, int64_t c0,
                                 int cols_valid, int k_valid, bool owns_map = true) {
    constexpr int LPR = Dma<R>::LPR, RPI = Dma<R>::RPI;
    const int lane = threadIdx.x & 63, wave = pwave();
    if (!MAP) map = nullptr;
    s.rsrc = make_rsrc(map ? base + c0 : base + r0 * ld + c0);
    s.ld2 = (uint32_t)(ld * 2);
    if (owns_map) tm.on = MAP && map;
    if (MAP && map) {
      tm.mbase = r0;
      tm.klen = k_valid;
      tm.rows = (uint32_t)map_rows;
      tm.pf_kt = -1;
    }
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int krow = (wave * PW + i) * RPI + lane / LPR;
      const int c = (lane % LPR) ^ tswz(krow);
      s.idx[i] = krow;
      s.ok[i] = c * 8 < cols_valid;
      // Without a map an invalid column holds kOob (see issue_k); with one,
      // the column offset, to which the gathered row's offset is added.
      s.off[i] = map ? (uint32_t)(c * 16)
                     : (s.ok[i] ? (uint32_t)(c * 16 + (int64_t)krow * ld * 2) : kOob);
    }
  }

  // UP_GLU's B operand (T-form, no map): staged chunk q (8 columns) of a
  // k-row holds output columns 32 (q / 8) + 8 (q % 4) .. + 7 of the tile, from
  // the gate columns (c0 + n) for q % 8 < 4 and from the up columns
  // (c0 + up + n) otherwise; out_valid output columns are real.
  __device__ static void setup_glu(Src<PWB>& s, const uint16_t* base, int64_t ld, int64_t r0,
                                   int64_t c0, int up, int out_valid) {
    constexpr int LPR = Dma<BN>::LPR, RPI = Dma<BN>::RPI;
    const int lane = threadIdx.x & 63, wave = pwave();
    s.rsrc = make_rsrc(base + r0 * ld + c0);
    s.ld2 = (uint32_t)(ld * 2);
#pragma unroll
    for (int i = 0; i < PWB; ++i) {
      const int krow = (wave * PWB + i) * RPI + lane / LPR;
      const int c = (lane % LPR) ^ tswz(krow);
      const int oc = (c >> 3) * 4 + (c & 3);  // output chunk
      s.idx[i] = krow;
      s.ok[i] = oc * 8 < out_valid;
      s.off[i] = s.ok[i] ? (uint32_t)(oc * 16 + ((c >> 2) & 1) * up * 2 + (int64_t)krow * ld * 2)
                         : kOob;
    }
  }

  // DMA of this wave's map entries for stages [kw / BK, kw / BK + kWinStages)
  // of the item into window `win`; entries past the item's rows read 0.
  // K-form gather (A of UP_FWD and DOWN_DH): the window holds the entries of
  // the wave's PWA * KRPI tile rows instead (tm.klen = valid rows).
  __device__ static void load_window(const TMap& tm, int kw, lds_char* win) {
    const int lane = threadIdx.x & 63, wave = pwave();
    if constexpr (T::k_map) {
      static_assert(PWA * KRPI <= 64, "one 4-byte DMA covers the wave's tile rows");
      const int row = wave * PWA * KRPI + lane;
      const bool v = lane < PWA * KRPI && row < tm.klen;
      dma4(tm.mrs, v ? (uint32_t)((tm.mbase + row) * 4) : kOob, win);
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = kw + (8 * h + (lane >> 3)) * BK + wave * 8 + (lane & 7);
        dma4(tm.mrs, k < tm.klen ? (uint32_t)((tm.mbase + k) * 4) : kOob, win + h * 256);
      }
    }
  }

  // The lane's map entries (one per DMA instruction) of stage kt from the
  // current window.
  template <int R, int PW>
  __device__ static void window_rows(const TMap& tm, int kt, int32_t (&rows)[PW]) {
    constexpr int LPR = Dma<R>::LPR, RPI = Dma<R>::RPI;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < PW; ++i)
      rows[i] = reinterpret_cast<const __attribute__((address_space(3))) int32_t*>(
          tm.win)[(kt % kWinStages) * 8 + i * RPI + lane / LPR];
  }

  template <int R, int PW, bool MAP>
  __device__ static void issue_t(const Src<PW>& s, TMap& tm, int kt, int K, lds_char* stage) {
    const uint32_t m0 = lds_slot<PW>(stage);
    const int k0 = kt * BK;
    if constexpr (MAP) {
      static_assert(PW <= 4, "prefetched map entries per lane");
      if (tm.on) {
        if (kt > 0 && kt % kWinStages == 0) {
          // Items longer than the window (no split-K): refill it in place.
          load_window(tm, k0, tm.win);
          wait_vmcnt<0>();
          tm.pf_kt = -1;
        }
        // Entries of this stage, read from LDS during the previous stage's
        // issue when it was in the same window (the read's latency then
        // overlaps the wait for the ring), else now.
        int32_t rows[PW];
        if (tm.pf_kt == kt) {
#pragma unroll
          for (int i = 0; i < PW; ++i) rows[i] = tm.pf[i];
        } else {
          window_rows<R, PW>(tm, kt, rows);
        }
        const bool kin = k0 + BK <= K;  // uniform: every k-row of the stage is in K
#pragma unroll
        for (int i = 0; i < PW; ++i) {
          const bool v = s.ok[i] & (kin | (k0 + s.idx[i] < K)) & ((uint32_t)rows[i] < tm.rows);
          dma16(s.rsrc, v ? s.off[i] + (uint32_t)rows[i] * s.ld2 : kOob, m0 + i * 1024);
        }
        const int kn = kt + 1;
        tm.pf_kt = -1;
        if (kn * BK < K && kn % kWinStages != 0) {
          int32_t nx[PW];
          window_rows<R, PW>(tm, kn, nx);
#pragma unroll
          for (int i = 0; i < PW; ++i) tm.pf[i] = nx[i];
          tm.pf_kt = kn;
        }
        return;
      }
    }
    if (k0 + BK <= K) {
#pragma unroll
      for (int i = 0; i < PW; ++i)
        dma16(s.rsrc, s.off[i] + (uint32_t)k0 * s.ld2, m0 + i * 1024);
      return;
    }
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const bool v = s.ok[i] & (k0 + s.idx[i] < K);
      dma16(s.rsrc, v ? s.off[i] + (uint32_t)k0 * s.ld2 : kOob, m0 + i * 1024);
    }
  }

  // MFMA fragment of rows [row0, row0 + 32) x k-step ks (16 deep).
  // Fragment of rows [row0, row0 + 32) x k-step ks of half h of an A pair
  // slot (the layout setup_k's PAIR mapping writes).
  __device__ static bf16x8_t frag_kp(const lds_char* pair, int h, int row0, int ks) {
    const int lane = threadIdx.x & 63;
    const int row = row0 + (lane & 31);
    const int c = 2 * ks + (lane >> 5);
    return *reinterpret_cast<const lds_bf16x8*>(pair + (row >> 3) * 1024 + h * 512 +
                                                (row & 7) * 64 + ((c ^ ((row >> 2) & 3)) << 4));
  }

  __device__ static bf16x8_t frag_k(const lds_char* stage, int row0, int ks) {
    const int lane = threadIdx.x & 63;
    const int row = row0 + (lane & 31);
    const int c = 2 * ks + (lane >> 5);
    return *reinterpret_cast<const lds_bf16x8*>(stage + row * (BK * 2) +
                                                ((c ^ kswz(row)) << 4));
  }

  // Fragment of columns [col0, col0 + 32) x k-step ks from a T-form stage of
  // R columns: two transposing reads of k-rows kr and kr + 4.
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

  // Builds the per-expert tables (all threads; `scan` is 16 longs of LDS).
  // Returns the total number of work items.
  // Contig (dW) GEMMs also split the items into NL = grid >> lsh lane
  // ranges of equal estimated cost, in k-step units: an item costs its
  // chunk's k-steps (1 .. kDwChunk / BK) plus kItemCost for starting it, and
  // a tile group kEpiCost more for its epilogue (measured: an item start
  // about 2 k-steps, a tile's rounding and stores about 4). Equal item
  // counts left the lanes of large experts three times as busy as the
  // lanes of the many small ones. Lane l starts at the first item at or
  // after cumulative cost cost_total * l / NL. `cpre` is LDS scratch for
  // E + 1 ints (the ring, before its first use).
  // Row-tiled GEMMs split their items into the 8 XCDs' ranges the same way,
  // an item (a tile) costing its k-steps plus kTileCost: where K differs
  // between experts (K = w_e for the down projection and dX), equal item
  // counts gave the XCDs holding the widest experts several times the work
  // of the others (workgroups ending between 430 and 1225 us at cfg4).
  static constexpr int kItemCost = 2, kEpiCost = 4, kTileCost = 3;
  __device__ static int build_meta(const Args& p, Meta& mt, long long* scan,
                                   __attribute__((address_space(3))) int* cpre) {
    constexpr bool CONTIG = Cfg<V>::contig;
    long long base = 0, cbase = 0;
    for (int e0 = 0; e0 < p.E; e0 += kThreads) {
      const int e = e0 + threadIdx.x;
      int items = 0, cost = 0;
      if (e < p.E) {
        const ExpertRec r = rec_global(p, e);
        if (p.E <= kRecExperts) {
          mt.rec[0][e] = r.t0; mt.rec[1][e] = r.t1; mt.rec[2][e] = r.tpe;
          mt.rec[3][e] = r.ew0; mt.rec[4][e] = r.ew1; mt.rec[5][e] = r.w;
        }
        const Prob q = T::prob(p, r);
        int tiles, chunks;
        expert_work<V>(p, q, tiles, chunks);
        items = work_items<V>(tiles, chunks, p.lsh);
        if (CONTIG)
          cost = ((tiles + (1 << p.lsh) - 1) >> p.lsh) *
                 (cdiv(q.K, BK) + kItemCost * chunks + kEpiCost);
        else
          cost = items * (cdiv(q.K, BK) + kTileCost);
      }
      // One scan of (cost << 32 | items): both prefixes stay below 2^31.
      long long total;
      const long long ex = block_exclusive_scan<long long, kThreads>(
          ((long long)cost << 32) | (long long)items, scan, &total);
      if (e < p.E) {
        mt.pre[e] = (int)(base + (ex & 0xFFFFFFFFll));
        cpre[e] = (int)(cbase + (ex >> 32));
      }
      base += total & 0xFFFFFFFFll;
      cbase += total >> 32;
      __syncthreads();  // scan scratch reused by the next chunk
    }
    if (threadIdx.x == 0) {
      mt.pre[p.E] = (int)base;
      cpre[p.E] = (int)cbase;
    }
    __syncthreads();
    {
      const int NL = CONTIG ? p.grid >> p.lsh : 8;
      for (int l = threadIdx.x; l <= NL; l += kThreads) {
        int item = (int)base;
        if (l == 0 || cbase == 0) {
          item = l == NL ? (int)base : 0;
        } else if (l < NL) {
          // any monotone split will do: float, no 64-bit division
          const int target = min((int)cbase - 1, (int)((float)cbase * ((float)l / (float)NL)));
          // first expert e with cpre[e + 1] > target (zero-cost experts skipped)
          int lo = 0, hi = p.E - 1;
          while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (cpre[mid + 1] > target) hi = mid; else lo = mid + 1;
          }
          const int e = lo;
          const ExpertRec r = p.E <= kRecExperts
              ? ExpertRec{mt.rec[0][e], mt.rec[1][e], mt.rec[2][e], mt.rec[3][e], mt.rec[4][e],
                          mt.rec[5][e]}
              : rec_global(p, e);
          const Prob q = T::prob(p, r);
          int tiles, chunks;
          expert_work<V>(p, q, tiles, chunks);
          const int o = target - cpre[e];
          if (CONTIG) {
            const int gcost = cdiv(q.K, BK) + kItemCost * chunks + kEpiCost;
            const int g = udiv_small(o, gcost), rem = o - g * gcost;
            // first item of group g starting at or after rem: chunk c starts
            // at cost c * (kDwChunk / BK + kItemCost); past the last chunk,
            // the next group's first item
            item = mt.pre[e] + g * chunks + min(chunks, cdiv(rem, kDwChunk / BK + kItemCost));
          } else {
            // the first tile starting at or after the target
            const int tcost = cdiv(q.K, BK) + kTileCost;
            const int g = udiv_small(o, tcost);
            item = mt.pre[e] + min(tiles, g + (o - g * tcost > 0 ? 1 : 0));
          }
        }
        mt.lane_beg[l] = item;
      }
      __syncthreads();
    }
    return (int)base;
  }

  struct Work {
    int m0, n0, kbeg, klen, nk, chunk, chunks;
    bool skip;  // contig: the item's tile group has no tile for this slot
    Prob q;
  };

  // Work item `item` (ascending across calls with the same cursor): finds its
  // expert with a wave-wide search of the prefix table from the cursor, then
  // its tile (for contig, that of lane slot `slot`) and K chunk. Every field
  // is workgroup-uniform.
  __device__ static Work decode(const Args& p, const Meta& mt, int item, int& ecur, int slot) {
    const int lane = threadIdx.x & 63;
    int e = ecur;
    for (;;) {
      const int c = e + 1 + lane;
      const bool past = c > p.E || mt.pre[c] > item;
      const uint64_t mask = ballot64(past);
      if (mask) {
        e += __builtin_ctzll(mask);
        break;
      }
      e += 64;
    }
    e = __builtin_amdgcn_readfirstlane(e);
    ecur = e;
    ExpertRec r;
    if (p.E <= kRecExperts) {
      r.t0 = __builtin_amdgcn_readfirstlane(mt.rec[0][e]);
      r.t1 = __builtin_amdgcn_readfirstlane(mt.rec[1][e]);
      r.tpe = __builtin_amdgcn_readfirstlane(mt.rec[2][e]);
      r.ew0 = __builtin_amdgcn_readfirstlane(mt.rec[3][e]);
      r.ew1 = __builtin_amdgcn_readfirstlane(mt.rec[4][e]);
      r.w = __builtin_amdgcn_readfirstlane(mt.rec[5][e]);
    } else {
      r = rec_scalar(p, e);
    }
    Work w;
    w.q = T::prob(p, r);
    int tiles, chunks;
    expert_work<V>(p, w.q, tiles, chunks);
    const int local = item - __builtin_amdgcn_readfirstlane(mt.pre[e]);
    const int group = chunks == 1 ? local : udiv_small(local, chunks);
    const int chunk = local - group * chunks;
    const int tile = Cfg<V>::contig ? (group << p.lsh) + slot : group;
    w.skip = tile >= tiles;
    constexpr int BNO = out_cols<V>();
    const int n_tiles = cdiv(w.q.N, BNO);
    const int mt_idx = n_tiles == 1 ? tile : udiv_small(tile, n_tiles);
    w.m0 = mt_idx * BM;
    w.n0 = (tile - mt_idx * n_tiles) * BNO;
    w.kbeg = 0;
    w.chunk = chunk;
    w.chunks = chunks;
    int K = w.q.K;
    if (chunks > 1) {
      w.kbeg = chunk * p.kc;
      K = min(K, w.kbeg + p.kc);
    }
    w.klen = K - w.kbeg;
    w.nk = w.klen > 0 && !w.skip ? cdiv(w.klen, BK) : 0;
    if (PAIR_A) w.nk = (w.nk + 1) & ~1;  // pairs of k-steps
    return w;
  }

  // Map fields of work w for the gathered T-form operand (A of UP_DW, B of
  // DOWN_DW).
  __device__ static void setup_map(const Args& p, const Work& w, TMap& tm) {
    if constexpr (T::k_map) {
      tm.mbase = w.q.ar + w.m0;  // map index of the tile's first row
      tm.klen = w.q.M - w.m0;    // rows of the tile that exist
    } else {
      tm.mbase = (T::t_map_b ? w.q.br : w.q.ar) + w.kbeg;
      tm.klen = w.klen;
    }
    tm.rows = (uint32_t)(T::t_map_b ? p.b_rows : p.a_rows);
    tm.on = true;
  }

  __device__ static void setup(const Args& p, const Work& w, Src<PWA_S>& sa, Src<PWB>& sb,
                               TMap& tm) {
    const Prob& q = w.q;
    if constexpr (T::a_k)
      setup_k<BM, PWA_S, PAIR_A>(sa, p.a, p.lda, p.a_map, p.a_rows, q.ar + w.m0, q.ac + w.kbeg,
                                 q.M - w.m0, tm.win);
    else
      setup_t<BM, PWA, T::t_map>(sa, tm, p.a, p.lda, p.a_map, p.a_rows, q.ar + w.kbeg,
                                 q.ac + w.m0, q.M - w.m0, w.klen, !T::t_map_b);
    if (V == UP_GLU)
      setup_glu(sb, p.b, p.ldb, q.br + w.kbeg, q.bc + w.n0, q.N, q.N - w.n0);
    else if (T::b_k)
      setup_k<BN, PWB, false>(sb, p.b, p.ldb, nullptr, 0, q.br + w.n0, q.bc + w.kbeg, q.N - w.n0,
                              nullptr);
    else
      setup_t<BN, PWB, T::t_map_b>(sb, tm, p.b, p.ldb, p.b_map, p.b_rows, q.br + w.kbeg,
                                   q.bc + w.n0, q.N - w.n0, w.klen, T::t_map_b);
  }

  // Issues k-step kt of item w as global stage s (A of a pair: on even kt).
  __device__ static void issue(const Work& w, const Src<PWA_S>& sa, const Src<PWB>& sb,
                               TMap& tm, int kt, lds_char* ring, int s) {
    const int k0 = kt * BK;
    if constexpr (T::a_k) {
      if (!PAIR_A || (kt & 1) == 0) issue_k<BM, PWA_S, PAIR_A>(sa, k0, w.klen, a_at(ring, s));
    } else {
      issue_t<BM, PWA, T::t_map>(sa, tm, kt, w.klen, a_at(ring, s));
    }
    if (T::b_k) issue_k<BN, PWB, false>(sb, k0, w.klen, b_at(ring, s));
    else issue_t<BN, PWB, T::t_map_b>(sb, tm, kt, w.klen, b_at(ring, s));
  }

  // Multiplies one staged k-tile into the wave's accumulators.
  __device__ static void compute(const lds_char* ring, int s, f32x16_t (&acc)[FM][FN]) {
    const int wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const lds_char* ca = a_at(ring, s);
    const lds_char* cb = b_at(ring, s);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8_t af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = PAIR_A ? frag_kp(ca, s & 1, wm * WM + i * 32, ks)
                : T::a_k ? frag_k(ca, wm * WM + i * 32, ks) : frag_t<BM>(ca, wm * WM + i * 32, ks);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = T::b_k ? frag_k(cb, wn * WN + j * 32, ks) : frag_t<BN>(cb, wn * WN + j * 32, ks);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          // Operands swapped: the accumulator holds C^T, so each lane owns
          // 4 consecutive n of one m and stores 8 bytes at a time.
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
    }
  }

  // Epilogue. acc[i][j][4*g + r] sits at m = wm*WM + i*32 + (lane & 31),
  // n = wn*WN + j*32 + 8*g + 4*(lane >> 5) + r.
  //
  // Deferred stores: when a tile's last K chunk is done, each consumer wave
  // rounds its accumulators to packed bf16 in registers (the "pending"
  // tile, 32 registers per output) and goes on with the next item; the
  // pending tile is stored one 32x64 block at a time between the MFMA
  // k-steps of that next item. The stores of one tile thus overlap the
  // loads and MFMAs of the next instead of stalling the whole workgroup
  // (all consumer waves reach a tile end together). Split-K partial tiles
  // are stored at once in fp32.
  //
  // Store staging: a block goes through the wave's private 4 KiB LDS
  // scratch and is read back as 128-byte row segments, so a store
  // instruction writes 8 whole cache lines (the accumulator layout alone
  // gives 8 bytes per lane over 32 rows). Row r holds its 16 8-byte
  // half-chunks hc at position hc ^ (r & 15). ds_write_b64 serves 16
  // consecutive lanes per cycle over 32 dword banks (128 B; measured: a
  // (r >> 1) swizzle conflicts 2-way there and takes twice the cycles), and
  // 16 rows with one half-chunk then fill the 32 banks exactly; a 16-lane
  // ds_read_b128 phase covers two whole rows over all 64 banks.
  static constexpr int EPI_BYTES = 32 * 64 * 2;
  static_assert(WN == 64 && FN == 2 && FM == 2, "epilogue assumes 64x64 wave tiles");
  // UP_FWD with relu^2 stores PRE and H; UP_GLU [gate | up] blocks and H
  // (the right half of its H blocks is unused); every other variant one
  // output.
  static constexpr int NOUT = V == UP_FWD || V == UP_GLU ? 2 : 1;

  // Pending blocks are units u = out * FM + i (output-major, row block i);
  // every unit index is a compile-time constant where the block is used, so
  // the pending tile stays in registers.
  static constexpr int UNITS = NOUT * FM;
  struct Pending {
    uint32_t pk[NOUT][FM][FN][8];  // bf16 pairs of block (i, j): (g, half) -> 2 g + half
    int mb, nb;                    // first row / column of the wave tile in the problem
    int M, N, cr, cc;              // the tile's problem extents and output origin
    int mask;                      // bit u: unit u still to be stored
  };

  __device__ static int epi_off(int r, int hc) { return r * 128 + ((hc ^ (r & 15)) << 3); }

  // Packed block (out, i) into the wave's scratch: lane (r = lane & 31,
  // h = lane >> 5) holds for each (j, g) the 4 values at columns
  // 32j + 8g + 4h .. +3 of row r.
  template <int OUT, int I>
  __device__ __forceinline__ static void epi_write(lds_char* scr, const Pending& pd, int lane) {
    const int r = lane & 31, h = lane >> 5;
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const u32x2_t v = {pd.pk[OUT][I][j][2 * g], pd.pk[OUT][I][j][2 * g + 1]};
        *reinterpret_cast<__attribute__((address_space(3))) u32x2_t*>(
            scr + epi_off(r, 2 * (4 * j + g) + h)) = v;
      }
  }

  // Row 8q + (lane >> 3), columns 8 (lane & 7) .. +7 of the scratch block.
  __device__ __forceinline__ static uint4 epi_read(const lds_char* scr, int q, int lane) {
    const int r = 8 * q + (lane >> 3), c = lane & 7;
    const int f = r & 15;
    const u32x4_t v = *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(
        scr + r * 128 + ((((2 * c) ^ f) >> 1) << 4));
    // Half-chunks 2c and 2c + 1 sit swapped when f is odd.
    return (f & 1) ? make_uint4(v.z, v.w, v.x, v.y) : make_uint4(v.x, v.y, v.z, v.w);
  }

  // Rounds the finished tile of this wave into `pd` (the previous pending
  // tile must be fully stored): relu / relu^2 for the up projection
  // (PRE = bf16(relu(z)), H = bf16(relu(z)^2), grouped_gemm.py:336-346),
  // the accumulators as they are otherwise.
  __device__ __forceinline__ static void stash(const Args& p, const Work& w,
                                              const f32x16_t (&acc)[FM][FN], Pending& pd,
                                              const lds_char* scale) {
    const int wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    // Row factors (UP_FWD: the output H, not PRE; DOWN_DH: the gradient
    // before the relu^2 rule): acc row wm * WM + 32 i + (lane & 31).
    float sc[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) sc[i] = 1.0f;
    if constexpr (kScaled) {
      if (scale) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
          sc[i] = reinterpret_cast<const __attribute__((address_space(3))) float*>(scale)
              [wm * WM + i * 32 + (threadIdx.x & 31)];
      }
    }
    if constexpr (V == DOWN_DH || V == DOWN_DW) {
      // A broadcast output gradient c * ones: the GEMM read the ones row, c
      // scales the result here.
      if (p.gscale) {
        const float gs = bf16_to_f32(*p.gscale);
#pragma unroll
        for (int i = 0; i < FM; ++i) sc[i] *= gs;
      }
    }
    const Prob& q = w.q;
    if constexpr (V == DOWN_DW) {
      // Transposed store: for each (i, j, g, r) lanes 0-31 hold 32
      // consecutive m of column n and lanes 32-63 of column n + 4, i.e. two
      // 64-byte runs of output rows n and n + 4.
      pd.mask = 0;
      const int lane = threadIdx.x & 63;
      const int n0 = w.n0 + wn * WN + 4 * (lane >> 5);  // this lane's first column
      const int m0 = w.m0 + wm * WM + (lane & 31);
      // One buffer resource over the expert's rows of grad_w2, 32-bit byte
      // offsets per store.
      const auto rc = make_rsrc(p.c + (int64_t)q.cr * p.ldc + q.cc);
      const uint32_t ld2 = (uint32_t)p.ldc * 2;
      const uint32_t base = (uint32_t)n0 * ld2 + (uint32_t)m0 * 2;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int dn = j * 32 + 8 * g + r;
#pragma unroll
            for (int i = 0; i < FM; ++i) {
              const bool ok = n0 + dn < q.N && m0 + i * 32 < q.M;
              __builtin_amdgcn_raw_buffer_store_b16(
                  (uint16_t)f32_to_bf16(sc[i] * acc[i][j][4 * g + r]), rc,
                  ok ? base + (uint32_t)dn * ld2 + i * 64 : kOob, 0, 0);
            }
          }
      return;
    }
    pd.mb = w.m0 + wm * WM;
    pd.nb = w.n0 + wn * (V == UP_GLU ? WN / 2 : WN);
    pd.M = q.M; pd.N = q.N; pd.cr = q.cr; pd.cc = q.cc;
    if constexpr (V == UP_GLU) {
      // Block j = 0 holds the gate g, j = 1 the up projection u of the same
      // 32 outputs: gate and up (bf16) go to unit (0, i), H = bf16(g
      // sigmoid(g) u) (from the fp32 accumulators, times the row factor) to
      // unit (1, i).
      const int rows = pd.mb >= q.M ? 0 : (pd.mb + 32 >= q.M ? 1 : 3);
      pd.mask = (p.c ? rows << FM : 0) | (p.c2 || p.c3 ? rows : 0);
      if (pd.mask == 0) return;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const float ga = acc[i][0][4 * g + 2 * hh], gb = acc[i][0][4 * g + 2 * hh + 1];
            const float ua = acc[i][1][4 * g + 2 * hh], ub = acc[i][1][4 * g + 2 * hh + 1];
            pd.pk[0][i][0][2 * g + hh] = pack_bf16(ga, gb);
            pd.pk[0][i][1][2 * g + hh] = pack_bf16(ua, ub);
            pd.pk[1][i][0][2 * g + hh] =
                pack_bf16(sc[i] * ((ga * sigmoid_f32(ga)) * ua),
                          sc[i] * ((gb * sigmoid_f32(gb)) * ub));
            pd.pk[1][i][1][2 * g + hh] = 0u;
          }
      return;
    }
    const bool two = V == UP_FWD && p.act == VMOE_ACT_RELU_SQUARED && p.c2;
    // Row blocks starting inside the problem (wave-uniform): none, the first, or both.
    const int rows = pd.mb >= q.M ? 0 : (pd.mb + 32 >= q.M ? 1 : 3);
    pd.mask = (rows << (FM * (NOUT - 1))) | (two ? rows : 0);
    if (pd.mask == 0) return;
    // The activation is uniform, so it selects one of two straight-line
    // loops (per-element selects cost two VALU instructions per pair, and a
    // wave64 VALU instruction four cycles of the SIMD).
    if (NOUT == 2 && p.act == VMOE_ACT_RELU_SQUARED)
      stash_units<true>(acc, sc, pd);
    else
      stash_units<false>(acc, sc, pd);
  }

  // Packed bf16 units of the pending tile: PRE = relu(acc) and H = sc *
  // relu(acc)^2 (R2), or H = sc * acc. Every store goes to a fixed element,
  // which keeps the pending tile in registers.
  template <bool R2>
  __device__ __forceinline__ static void stash_units(const f32x16_t (&acc)[FM][FN],
                                                     const float (&sc)[FM], Pending& pd) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const float a = acc[i][j][4 * g + 2 * hh], b = acc[i][j][4 * g + 2 * hh + 1];
            if (NOUT == 2 && R2) {
              const float ra = fmaxf(a, 0.0f), rb = fmaxf(b, 0.0f);
              pd.pk[0][i][j][2 * g + hh] = pack_bf16(ra, rb);
              pd.pk[NOUT - 1][i][j][2 * g + hh] = pack_bf16(sc[i] * (ra * ra), sc[i] * (rb * rb));
            } else {
              // without relu^2 the up projection's PRE unit is never stored
              // (pd.mask), so its registers are left as they are
              pd.pk[NOUT - 1][i][j][2 * g + hh] = pack_bf16(sc[i] * a, sc[i] * b);
            }
          }
  }

  // DOWN_DH with pre: the PRE values unit I of the pending tile combines
  // with, loaded a few k-steps before its flush so the load latency does not
  // stall the wave (and with it the next barrier) at every flush.
  template <int I>
  __device__ __forceinline__ static void load_pre(const Args& p, const Pending& pd,
                                                  uint4 (&pr)[4]) {
    if constexpr (V == DOWN_DH) {
      if (!p.pre) return;
      int lane = threadIdx.x & 63;
      asm volatile("" : "+v"(lane));
      const int mb = pd.mb + I * 32;
      const int n = pd.nb + 8 * (lane & 7);
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int m = mb + 8 * qq + (lane >> 3);
        pr[qq] = make_uint4(0, 0, 0, 0);
        if (m < pd.M && n < pd.N)
          pr[qq] = *reinterpret_cast<const uint4*>(p.pre + ((int64_t)pd.cr + m) * p.ldc + pd.cc + n);
      }
    }
  }

  // Stores block (OUT, I) of the pending tile: rows pd.mb + 32 I .. +31.
  template <int OUT, int I>
  __device__ __forceinline__ static void flush_unit(const Args& p, const Pending& pd, lds_char* scr,
                                                    const uint4 (&pr)[4]) {
    // The lane index is made opaque so that this lane-only address math is
    // recomputed here instead of being hoisted out of the k-loop, where it
    // would stay live (and spill) across the MFMAs.
    int lane = threadIdx.x & 63;
    asm volatile("" : "+v"(lane));
    const int mb = pd.mb + I * 32;
    epi_write<OUT, I>(scr, pd, lane);
    const int n = pd.nb + 8 * (lane & 7);
    const bool n_ok = n < pd.N;
    if (V == DOWN_DH && p.pre) {
      // GA = bf16(pre > 0 ? 2 * GH * pre : 0), GH the bf16-rounded dH
      // (grouped_gemm.py:751-766), with PRE from load_pre. With row_dot, the
      // wave also sums GH * PRE^2 over each row's 64 columns (8 lanes of 8
      // columns, added with DPP moves in a fixed order): the gradient of the
      // row's routing weight is that sum over the row's blocks divided by
      // the weight (the module's H' is w * relu(z)^2).
      const bool dot = p.row_dot != nullptr;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const uint4 gh = epi_read(scr, qq, lane);
        const int m = mb + 8 * qq + (lane >> 3);
        float s = 0.0f;
        if (m < pd.M && n_ok) {
          const uint32_t gw[4] = {gh.x, gh.y, gh.z, gh.w};
          const uint32_t pw[4] = {pr[qq].x, pr[qq].y, pr[qq].z, pr[qq].w};
          uint32_t o[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float pl = lo_f32(pw[t]), ph = hi_f32(pw[t]);
            o[t] = pack_bf16(pl > 0.0f ? lo_f32(gw[t]) * 2.0f * pl : 0.0f,
                             ph > 0.0f ? hi_f32(gw[t]) * 2.0f * ph : 0.0f);
            if (dot) s += lo_f32(gw[t]) * (pl * pl) + hi_f32(gw[t]) * (ph * ph);
          }
          *reinterpret_cast<uint4*>(p.c + ((int64_t)pd.cr + m) * p.ldc + pd.cc + n) =
              make_uint4(o[0], o[1], o[2], o[3]);
        }
        if (dot) {
          s += dpp_f32<0xB1>(s);   // quad_perm [1, 0, 3, 2]
          s += dpp_f32<0x4E>(s);   // quad_perm [2, 3, 0, 1]
          s += dpp_f32<0x141>(s);  // row_half_mirror: the other quad of 8 lanes
          if ((lane & 7) == 0 && m < pd.M && pd.nb < pd.N)
            p.row_dot[((int64_t)pd.cr + m) * p.ld_rd + ((pd.cc + pd.nb) >> 6)] = s;
        }
      }
      return;
    }
    if constexpr (V == UP_GLU) {
      // Chunk c of a scratch row: unit 0 gate (c < 4) / up (c >= 4), unit 1
      // H (c < 4), at output column nb + 8 (c % 4).
      const int c = lane & 7;
      const int ng = pd.nb + 8 * (c & 3);
      uint16_t* go = OUT == 1 ? (c < 4 ? p.c : nullptr) : (c < 4 ? p.c2 : p.c3);
      const bool ok = go != nullptr && ng < pd.N;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const uint4 v = epi_read(scr, qq, lane);
        const int m = mb + 8 * qq + (lane >> 3);
        if (ok && m < pd.M)
          *reinterpret_cast<uint4*>(go + ((int64_t)pd.cr + m) * p.ldc + pd.cc + ng) = v;
      }
      return;
    }
    uint16_t* out = (NOUT == 2 && OUT == 0) ? p.c2 : p.c;
    // The [rows, d] outputs of DOWN_FWD and UP_DX (268 MB at cfg3), which
    // only the combine reads (itself with non-temporal loads), are stored
    // non-temporally so they do not evict the operands these GEMMs re-read
    // (cfg3: dX 135 -> 122 us, down fwd 128 -> 121 us; the combines read
    // them 7 us slower each, the step is ~1 % shorter); the other outputs
    // are read right after by the next GEMM.
    constexpr bool kStream = V == DOWN_FWD || V == UP_DX;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const uint4 v = epi_read(scr, qq, lane);
      const int m = mb + 8 * qq + (lane >> 3);
      if (m < pd.M && n_ok) {
        u32x4_t* dst = reinterpret_cast<u32x4_t*>(out + ((int64_t)pd.cr + m) * p.ldc + pd.cc + n);
        const u32x4_t val = {v.x, v.y, v.z, v.w};
        if (kStream)
          __builtin_nontemporal_store(val, dst);
        else
          *dst = val;
      }
    }
  }

  // Stores unit U of the pending tile if it is still pending.
  template <int U>
  __device__ __forceinline__ static void flush_slot(const Args& p, Pending& pd, lds_char* scr,
                                                    const uint4 (&pr)[4]) {
    if (pd.mask & (1 << U)) flush_unit<U / FM, U % FM>(p, pd, scr, pr);
  }

  // Partial tiles travel between XCDs, whose L2s are not coherent with one
  // another: they are written and read with device-scope cache policy (sc1),
  // so stores reach the device-coherent level and loads do not hit a stale
  // line, without flushing or invalidating a whole L2.
  static constexpr int kScDevice = 16;  // buffer cache policy: sc1

  // The accumulators as a partial sum over some of the tile's K chunks: the
  // wave's fp32 values go to partial slot `pslot` in the accumulator layout
  // (wave, i, j, g, lane: 1 KiB contiguous per store).
  __device__ __forceinline__ static void store_partial(const Args& p, int pslot,
                                                       const f32x16_t (&acc)[FM][FN]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const auto r = make_rsrc(p.partial + (int64_t)pslot * (BM * BN) + wave * (WM * WN));
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const u32x4_t v = {__float_as_uint(acc[i][j][4 * g]),
                             __float_as_uint(acc[i][j][4 * g + 1]),
                             __float_as_uint(acc[i][j][4 * g + 2]),
                             __float_as_uint(acc[i][j][4 * g + 3])};
          __builtin_amdgcn_raw_buffer_store_b128(v, r, (((i * FN + j) * 4 + g) * 64 + lane) << 4,
                                                 0, kScDevice);
        }
  }

  // Adds (FIRST: copies) the wave's values of partial slot `pslot` into acc,
  // one 32x32 block at a time to bound the registers in flight (two blocks
  // per round trip measured 20 % slower on the up-projection dW GEMM).
  template <bool FIRST>
  __device__ __forceinline__ static void add_partial(const Args& p, int pslot,
                                                     f32x16_t (&acc)[FM][FN]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const auto r = make_rsrc(p.partial + (int64_t)pslot * (BM * BN) + wave * (WM * WN));
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        // Keeps the next block's loads below this block's additions.
        asm volatile("" ::: "memory");
        u32x4_t v[4];
#pragma unroll
        for (int g = 0; g < 4; ++g)
          v[g] = __builtin_amdgcn_raw_buffer_load_b128(
              r, (((i * FN + j) * 4 + g) * 64 + lane) << 4, 0, kScDevice);
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const float x = __uint_as_float(v[g][c]);
            acc[i][j][4 * g + c] = FIRST ? x : acc[i][j][4 * g + c] + x;
          }
      }
  }

  // Split-K, per consumer wave. The K chunks [a, a + chunks) of a split tile
  // are segments of consecutive non-empty lane ranges L0, L0 + 1, ...; the
  // wave of each segment stores its fp32 partial (slot 2 lin for a range's
  // first segment, 2 lin + 1 for its last), waits until the stores are
  // complete and counts itself in the tile's arrival word with a wrapping
  // increment, which the last arrival puts back to zero. The last wave sums
  // the segments in lane order, s0 + s1 + s2 + ...; its own term comes from
  // registers when it is s0 or s1 (the first addition commutes), else from
  // its slot, so the sum does not depend on which wave arrives last. Returns
  // true for that wave: acc then holds the whole tile for the normal
  // epilogue. No wave waits for another.
  __device__ static bool split_arrive(const Args& p, const Meta& mt, const Range& rg, int a,
                                      int chunks, int seg_item, f32x16_t (&acc)[FM][FN]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int NL = p.grid >> p.lsh, me = rg.lin >> p.lsh, ts = rg.slot;
    const int* lb = mt.lane_beg;
    int L0 = me;
    while (L0 > 0 && lb[L0] > a) --L0;
    const bool l0_inside = lb[L0] != a;  // L0's segment starts mid-range
    store_partial(p, 2 * rg.lin + (seg_item == rg.beg ? 0 : 1), acc);
    int nseg = 0, own = 0;
    for (int l = L0; l < NL; ++l) {
      const int b0 = lb[l];
      if (b0 >= a + chunks) break;
      if (lb[l + 1] == b0) continue;  // empty range
      if (l == me) own = nseg;
      ++nseg;
    }
    wait_vmcnt<0>();  // the partial is at the device-coherent level
    uint32_t old = 0;
    if (lane == 0)
      old = __builtin_amdgcn_atomic_inc32(
          p.arrive + ((int64_t)((L0 << p.lsh) + ts) * kConsumers + wave), (uint32_t)(nseg - 1),
          __ATOMIC_RELAXED, "agent");
    old = __builtin_amdgcn_readfirstlane(old);
    if (old != (uint32_t)(nseg - 1)) return false;
    asm volatile("" ::: "memory");  // the loads below follow the arrival
    int t = 0;
    for (int l = L0; l < NL && t < nseg; ++l) {
      const int b0 = lb[l];
      if (lb[l + 1] == b0) continue;
      const int slot = 2 * ((l << p.lsh) + ts) + (l == L0 && l0_inside ? 1 : 0);
      // own >= 2: the sum is rebuilt from the slots, own included.
      if (own >= 2 && t == 0)
        add_partial<true>(p, slot, acc);
      else if (t != own || own >= 2)
        add_partial<false>(p, slot, acc);
      ++t;
    }
    return true;
  }


  // Producer waves: stage the k-tiles of all of the workgroup's items, in
  // item order, as one stream through the LDS ring (the first stages of the
  // next item load while the current one finishes), waiting for each stage
  // before the barrier that hands it to the consumers.
  //
  // Row-map windows (T-form gather): when an item starts, the window of the
  // next item with k-steps is requested into the wave's other window. The
  // wait before stage s's barrier completes every DMA issued before stage
  // s + 1's, so a window requested after stage j was issued is in LDS once
  // the loop has waited for stage j; an item that starts earlier than that
  // (an item of fewer stages than the ring is deep, or the first one)
  // waits for its window explicitly.
  __device__ static void run_producer(const Args& p, lds_char* ring, lds_char* wins,
                                      lds_char* scl, const Meta& mt, const Range& rg) {
    // The producer wave of each SIMD issues ahead of its two consumer waves
    // when both have an instruction ready: the DMAs are the stage's long pole
    // (s_setprio orders issue only; results do not change).
    __builtin_amdgcn_s_setprio(2);
    int ei = 0, ela = 0;
    Work wi;
    Src<PWA_S> sa;
    Src<PWB> sb;
    TMap tm;
    const bool mapped = ((T::t_map || T::k_map) && p.a_map) || (T::t_map_b && p.b_map);
    if (mapped) tm.mrs = make_rsrc(T::t_map_b ? p.b_map : p.a_map);
    const bool scaled = kScaled && p.row_scale;
    __amdgpu_buffer_rsrc_t srs;
    if (scaled) srs = make_rsrc(p.row_scale);
    int nbegun = 0;         // items begun (row factors go to slot nbegun % kScaleSlots)
    lds_char* const win0 = wins + pwave() * kWinBytes;
    lds_char* const win1 = win0 + kProducers * kWinBytes;
    int wcur = 0;           // window of the current item (0: win0, 1: win1)
    int la_item = -1;       // item whose window was requested into the other one
    int la_stage = 0;       // last stage issued before that request
    int win_stage = -2;     // the same for the current item's window
    int done = -2;          // every DMA issued before stage done + 1's is complete
    int issued = 0;         // stages issued
    int ikt = 0, inext = rg.beg, witem = rg.beg;
    Work wla;  // decode of la_item, reused when that item begins
    auto begin_item = [&]() {
      if (mapped) {
        if (la_item == witem) {
          wcur ^= 1;
          tm.win = wcur ? win1 : win0;
          win_stage = la_stage;
        } else {
          tm.win = wcur ? win1 : win0;
          setup_map(p, wi, tm);
          load_window(tm, 0, tm.win);
          wait_vmcnt<0>();
          win_stage = -2;
        }
        // The K-form gather reads its entries when the item is set up.
        if (T::k_map && win_stage > done) {
          wait_vmcnt<0>();
          win_stage = -2;
        }
      }
      setup(p, wi, sa, sb, tm);
      if (scaled && pwave() == 0) {
        // The tile's BM row factors into the item's slot; the consumers read
        // them when they round the tile, many barriers after this DMA.
        const int lane = threadIdx.x & 63;
        const int64_t r0 = (int64_t)wi.q.cr + wi.m0;
        lds_char* slot = scl + (nbegun % kScaleSlots) * (BM * 4);
#pragma unroll
        for (int h = 0; h < BM / 64; ++h) {
          const int m = wi.m0 + h * 64 + lane;
          dma4(srs, m < wi.q.M ? (uint32_t)((r0 + h * 64 + lane) * 4) : kOob, slot + h * 256);
        }
      }
      ++nbegun;
      if (!mapped) return;
      la_item = -1;
      for (int nx = witem + rg.stride; nx < rg.end; nx += rg.stride) {
        wla = decode(p, mt, nx, ela, rg.slot);
        if (wla.nk > 0) {
          TMap tn = tm;
          setup_map(p, wla, tn);
          load_window(tn, 0, wcur ? win0 : win1);
          la_item = nx;
          la_stage = issued - 1;
          break;
        }
      }
    };
    // Moves to the next item with k-steps and sets it up (decode, operand
    // offsets, row factors, the next map window); false at the range's end.
    auto advance = [&]() -> bool {
      while (inext < rg.end) {
        witem = inext;
        wi = inext == la_item ? wla : decode(p, mt, inext, ei, rg.slot);
        inext += rg.stride;
        if (wi.nk > 0) {
          ikt = 0;
          begin_item();
          return true;
        }
      }
      return false;
    };
    bool have = advance();
    // Issues the stream's next stage into `st`; after an item's last stage
    // the next item is set up right away, so that work runs before the next
    // wait instead of between a barrier and the DMAs it would delay.
    auto issue_one = [&]() {
      if (!have) return;
      if (mapped && ikt == 0 && win_stage > done) wait_vmcnt<0>();  // window not yet in LDS
      issue(wi, sa, sb, tm, ikt, ring, issued);
      ++issued;
      if (++ikt >= wi.nk) have = advance();
    };
#pragma unroll
    for (int s = 0; s < kStages - 1; ++s) issue_one();
    // One barrier per issued stage, as the consumers take one per stage.
    for (int s = 0; s < issued; ++s) {
      // Stages s+1 .. issued-1 may still be in flight: wait until only
      // their DMAs are outstanding (loads complete in order), sync (the
      // consumers then read stage s), and refill the buffer the consumers
      // read in the previous step, which every wave has left by now.
      // With A pairs an even stage issues 2 PWA + PWB DMAs and an odd one
      // PWB, so two consecutive stages still issue 2 PT.
      const int after = issued - 1 - s;
      if (after >= 2) {
        wait_vmcnt<2 * PT>();
      } else if (after == 1) {
        if (!PAIR_A)
          wait_vmcnt<PT>();
        else if ((s & 1) == 1)
          wait_vmcnt<2 * PWA + PWB>();  // stage s + 1 is even
        else
          wait_vmcnt<PWB>();
      } else {
        wait_vmcnt<0>();
      }
      done = s;
      block_barrier();
      issue_one();
    }
  }

  // Consumer waves: multiply each stage after the barrier that publishes it.
  // A tile is finished when its last K chunk in this workgroup is done; its
  // results become the pending tile, stored during the next item's k-steps
  // (spread evenly over them) or at the end. A contiguous range may start or
  // end inside a split tile; such a segment is a partial sum, and the wave
  // that completes the tile's last segment stores the tile (split_arrive).
  __device__ static void run_consumer(const Args& p, const lds_char* ring, const Meta& mt,
                                      const Range& rg, int total, lds_char* scr,
                                      const lds_char* scl) {
    int ec = 0;
    int s = 0;
    int nbegun = 0;  // items with k-steps so far (the producers' slot count)
    int seg_item = rg.beg, seg_chunk = -1;
    f32x16_t acc[FM][FN];
    Pending pd;
    pd.mask = 0;
    uint4 pr[4];  // DOWN_DH: PRE of the next unit to flush
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) pr[qq] = make_uint4(0, 0, 0, 0);
    // Units flush kLead k-steps after their PRE loads are issued.
    constexpr int kLead = V == DOWN_DH ? 2 : 0;
    for (int item = rg.beg; item < rg.end; item += rg.stride) {
      const Work w = decode(p, mt, item, ec, rg.slot);
      if (w.skip) continue;
      int slot = 0;
      if constexpr (kScaled) {
        slot = nbegun % kScaleSlots;
        if (w.nk > 0) ++nbegun;
      }
      if (seg_chunk < 0) {
        seg_item = item;
        seg_chunk = w.chunk;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
      }
      // Pending unit u goes out after k-step min(u * gap, nk - 1) of this item
      // (right away when the item has no k-steps), so the previous tile's
      // stores are spread over this item's MFMAs. The dW GEMMs finish few
      // tiles per workgroup and store them at once (pending stays empty),
      // which keeps their registers for the accumulators.
      const int gap = max(1, w.nk / UNITS);
      // The GEMMs with K = hidden (up fwd, dH) offset their flush k-steps by
      // (b / 8) mod gap, so that the chip's workgroups, which reach their
      // k-steps nearly together, do not all store in the same k-step
      // (measured at cfg3, same box, three runs: up fwd -6 us, dH -1.6 us;
      // on the down projection, with 8 k-steps per item, +14 us).
      const int stagger =
          (V == UP_FWD || V == UP_GLU || V == DOWN_DH) ? (int)((vblock(p) >> 3) % (unsigned)gap)
                                                       : 0;
      int kt = 0;
      if (pd.mask & 1) load_pre<0>(p, pd, pr);
#pragma unroll
      for (int u = 0; u < (Cfg<V>::contig ? 0 : UNITS); ++u) {
        const int at = min(u * gap + kLead + stagger, w.nk - 1);
        for (; kt <= at; ++kt, ++s) {
          block_barrier();
          compute(ring, s, acc);
        }
        if (u == 0) flush_slot<0>(p, pd, scr, pr);
        if (u == 1) flush_slot<1>(p, pd, scr, pr);
        if (u == 2) flush_slot<2 % UNITS>(p, pd, scr, pr);
        if (u == 3) flush_slot<3 % UNITS>(p, pd, scr, pr);
        if (V == DOWN_DH && u == 0 && (pd.mask & 2)) load_pre<1 % FM>(p, pd, pr);
      }
      pd.mask = 0;
      for (; kt < w.nk; ++kt, ++s) {
        block_barrier();
        compute(ring, s, acc);
      }
      const bool last_chunk = w.chunk == w.chunks - 1;
      if (rg.stride != 1 || last_chunk || item + 1 >= rg.end) {
        bool whole = true;
        if constexpr (Cfg<V>::contig) {
          if (w.chunks > 1 && !(seg_chunk == 0 && last_chunk))
            whole = split_arrive(p, mt, rg, item - w.chunk, w.chunks, seg_item, acc);
        }
        if (whole) {
          stash(p, w, acc, pd, kScaled && p.row_scale && w.nk > 0 ? scl + slot * (BM * 4)
                                                                  : nullptr);
          if (Cfg<V>::contig) {
            flush_slot<0>(p, pd, scr, pr);
            flush_slot<1>(p, pd, scr, pr);
            pd.mask = 0;
          }
        }
        seg_chunk = -1;
      }
    }
    // The last tile has no next item to hide behind.
    if (pd.mask & 1) load_pre<0>(p, pd, pr);
    flush_slot<0>(p, pd, scr, pr);
    if (V == DOWN_DH && (pd.mask & 2)) load_pre<1 % FM>(p, pd, pr);
    flush_slot<1>(p, pd, scr, pr);
    if (UNITS > 2) {
      flush_slot<2 % UNITS>(p, pd, scr, pr);
      flush_slot<3 % UNITS>(p, pd, scr, pr);
    }
  }

  __device__ static void run(const Args& p, lds_char* ring, Meta& mt, lds_char* epi,
                             lds_char* wins, lds_char* scl) {
    const int total = build_meta(p, mt, (long long*)(char*)ring,
                                 (__attribute__((address_space(3))) int*)(ring + 256));
    const Range rg = item_range<Cfg<V>::contig>(p, total, mt.lane_beg);
    if (rg.beg >= rg.end) return;
    const int wave = threadIdx.x >> 6;
    if (wave >= kConsumers)
      run_producer(p, ring, wins, scl, mt, rg);
    else
      run_consumer(p, ring, mt, rg, total, epi + wave * EPI_BYTES, scl);
  }
};

// LDS of one GEMM workgroup, carved from one buffer: the DMA ring, the
// consumers' epilogue scratch, the per-expert tables, the producers' row-map
// windows (two per wave, for the gathered operands) and the row-factor slots.
template <int V>
struct Lds {
  using G = Gemm<V>;
  static constexpr int WIN_BYTES =
      Traits<V>::t_map || Traits<V>::t_map_b || Traits<V>::k_map ? 2 * kProducers * G::kWinBytes
                                                                  : 16;
  static constexpr int SCL_BYTES = G::kScaled ? G::kScaleSlots * G::BM * 4 : 16;
  static constexpr int up16(int n) { return (n + 15) / 16 * 16; }
  static constexpr int RING = 0;
  static constexpr int EPI = RING + up16(G::RING);
  static constexpr int META = EPI + kConsumers * G::EPI_BYTES;
  static constexpr int WINS = META + up16((int)sizeof(Meta));
  static constexpr int SCL = WINS + WIN_BYTES;
  static constexpr int BYTES = SCL + SCL_BYTES;
  static_assert(BYTES <= 160 * 1024, "LDS budget of a gfx950 CU");
  static_assert(G::RING % 1024 == 0, "the ring's stages keep their 1 KiB alignment");

  __device__ static void run(const Args& p, char* lds) {
    G::run(p, (lds_char*)(lds + RING), *reinterpret_cast<Meta*>(lds + META),
           (lds_char*)(lds + EPI), (lds_char*)(lds + WINS), (lds_char*)(lds + SCL));
  }
};

template <int V>
__global__ __launch_bounds__(kThreads) void grouped_gemm_kernel(Args p) {
  __shared__ __align__(1024) char lds[Lds<V>::BYTES];
  Lds<V>::run(p, lds);
}

// Two independent GEMMs in one launch (the backward's dH with dW2, dX with
// dW1, on small problems): workgroups take the two in turn by groups of 8,
// so each GEMM runs on half of every XCD's CUs. Beside each other, the
// tiles left over by one GEMM's last round and the start and end of each
// launch overlap the other's work, which two launches on one stream leave
// idle, without the event hand-overs of a second stream.
template <int V1, int V2>
__global__ __launch_bounds__(kThreads) void grouped_gemm_pair_kernel(Args p1, Args p2) {
  constexpr int B = Lds<V1>::BYTES > Lds<V2>::BYTES ? Lds<V1>::BYTES : Lds<V2>::BYTES;
  __shared__ __align__(1024) char lds[B];
  if (((blockIdx.x >> 3) & 1) == 0)
    Lds<V1>::run(p1, lds);
  else
    Lds<V2>::run(p2, lds);
}

// SwiGLU (activation "swiglu"; the reference's forward epilogue
// silu(gate) * up, grouped_gemm.py:347-349, and an unfinished backward,
// :768-790): the forward is the UP_GLU GEMM; its derivative is
//   dG = bf16(gh * u * s * (1 + g (1 - s))), dU = bf16(gh * g * s),
//   s = sigmoid(g), from the bf16 gate g and up u the forward stored.

// SwiGLU backward into the layout of the fused up projection's backward
// GEMMs: for row r of expert e (eto[e] <= r < eto[e+1]) and c < w_e,
// grad_gu[r, c] = dG and grad_gu[r, w_e + c] = dU (formulas above), from
// grad_h, gate and up at [r, c]; rows r >= eto[e] + min(tpe[e], eto[e+1] -
// eto[e]) of the expert hold zeros there. [dG | dU] per row is then the A
// operand of one dX GEMM and one dW GEMM over the expert's 2 w_e contiguous
// W1 columns. One wave per row.
__global__ __launch_bounds__(256) void glu_grad_kernel(
    const uint16_t* __restrict__ gh, int64_t ldgh, const uint16_t* __restrict__ gate,
    const uint16_t* __restrict__ up, int64_t ld, uint16_t* __restrict__ ggu, int64_t ldo,
    const int32_t* __restrict__ eto, const int32_t* __restrict__ widths,
    const int32_t* __restrict__ tpe, int E, int64_t rows, int max_width) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows || r < eto[0] || r >= eto[E]) return;
  // the expert: the last e with eto[e] <= r (an empty expert before it has
  // a smaller index, one after it starts past r)
  int lo = 0, hi = E;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (eto[mid] <= r) lo = mid; else hi = mid;
  }
  const int e = lo, w = min(widths[e], max_width);
  const bool live = r - eto[e] < min(tpe[e], eto[e + 1] - eto[e]);
  for (int c = lane * 8; c < w; c += 64 * 8) {
    uint4 gv = make_uint4(0, 0, 0, 0), uv = gv, hv = gv;
    if (live) {
      gv = *reinterpret_cast<const uint4*>(gate + r * ld + c);
      uv = *reinterpret_cast<const uint4*>(up + r * ld + c);
      hv = *reinterpret_cast<const uint4*>(gh + r * ldgh + c);
    }
    const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
    const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
    uint32_t a[4], b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float ra[2], rb[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float g = h ? hi_f32(gw[j]) : lo_f32(gw[j]);
        const float u = h ? hi_f32(uw[j]) : lo_f32(uw[j]);
        const float d = h ? hi_f32(hw[j]) : lo_f32(hw[j]);
        const float sg = sigmoid_f32(g);
        ra[h] = d * u * sg * (1.0f + g * (1.0f - sg));
        rb[h] = d * g * sg;
      }
      a[j] = pack_bf16(ra[0], ra[1]);
      b[j] = pack_bf16(rb[0], rb[1]);
    }
    *reinterpret_cast<uint4*>(ggu + r * ldo + c) = make_uint4(a[0], a[1], a[2], a[3]);
    *reinterpret_cast<uint4*>(ggu + r * ldo + w + c) = make_uint4(b[0], b[1], b[2], b[3]);
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

// Compute units of the current device (cached per device id; host threads
// may race to fill an entry, and all of them store the same value).
int cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

static_assert(kDwChunk % Cfg<UP_DW>::BK == 0 &&
                  kDwChunk / Cfg<UP_DW>::BK <= Gemm<UP_DW>::kWinStages,
              "a split-K item fits one map window");

// Persistent grid: one workgroup per CU (the LDS ring and tables fill a CU),
// never more than there are work items; a multiple of 8 so every XCD gets
// the same number of workgroups.
int gemm_grid(int64_t items_bound) {
  const int64_t cus = std::max(8, cu_count() / 8 * 8);
  return (int)std::min<int64_t>(cus, (items_bound + 7) / 8 * 8);
}

// Grid of the dW GEMMs: whole lanes of either width on every XCD (a
// multiple of 8 << kMaxLaneShift), one workgroup per CU where the device
// allows, at most kMaxDwGrid (lanes of 4 then fill lane_beg[]).
constexpr int kLaneGridStep = 8 << kMaxLaneShift;
int lane_grid() {
  const int g = std::max(kLaneGridStep, cu_count() / kLaneGridStep * kLaneGridStep);
  return std::min(g, kMaxDwGrid);
}
static_assert(kMaxDwGrid % kLaneGridStep == 0, "whole lanes on every XCD");

// Workgroups per lane of a dW GEMM (as a shift), from its shape: lanes of 8
// where an expert's output has many tiles (d x max width >= 2^21, e.g.
// 2048 x 1024), else 4. Measured on whole steps against lanes of 4: the
// cfg4 shape (d 2048, widths up to 1024) 1.6 % faster (dW1 900 -> 842 us);
// d 1024 x 256 1 % slower, d 768 x 512 3.5-4 % slower.
int lane_shift(int64_t hidden, int64_t max_width) {
  return hidden * max_width >= (int64_t(1) << 21) ? 3 : 2;
}

// Paired launches (gemm_pair_begin / gemm_pair_end): while a pair is open on
// the calling host thread, the first GEMM launch is held and the second goes
// out with it as one grouped_gemm_pair_kernel, each on half of every XCD's
// CUs (pair_grid workgroups, whole dW lanes).
struct HeldGemm {
  int variant;
  Args p;
  hipStream_t s;
  int solo_grid;  // its grid as a launch of its own
};
thread_local int g_pair_open = 0;  // 0: no pair, 1: open, 2: holding the first GEMM
thread_local HeldGemm g_held;

int pair_grid() {
  const int half = cu_count() / 2 / kLaneGridStep * kLaneGridStep;
  return std::max(kLaneGridStep, std::min(half, kMaxDwGrid));
}

template <int V>
int launch_solo(Args p, hipStream_t s) {
  VMOE_LAUNCH(grouped_gemm_kernel<V>, dim3((unsigned)p.grid), dim3(kThreads), 0, s, p);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

int launch_variant(int v, const Args& p, hipStream_t s) {
  switch (v) {
    case UP_FWD: return launch_solo<UP_FWD>(p, s);
    case DOWN_FWD: return launch_solo<DOWN_FWD>(p, s);
    case UP_DX: return launch_solo<UP_DX>(p, s);
    case UP_DW: return launch_solo<UP_DW>(p, s);
    case DOWN_DH: return launch_solo<DOWN_DH>(p, s);
    case DOWN_DW: return launch_solo<DOWN_DW>(p, s);
    case UP_GLU: return launch_solo<UP_GLU>(p, s);
  }
  return VMOE_ERR_INVALID_ARG;
}

template <int V1, int V2>
int launch_pair_kernel(const Args& p1, const Args& p2, hipStream_t s) {
  VMOE_LAUNCH((grouped_gemm_pair_kernel<V1, V2>), dim3((unsigned)(2 * p1.grid)), dim3(kThreads),
              0, s, p1, p2);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
}

// Launches GEMM V with arguments p (p.grid: its grid as a launch of its own),
// or holds it / pairs it with the held one while a pair is open.
template <int V>
int submit(Args p, hipStream_t s) {
  if (g_pair_open == 0) return launch_solo<V>(p, s);
  const int solo = p.grid;
  p.grid = pair_grid();
  p.paired = 1;
  if (g_pair_open == 1 || g_held.s != s) {
    if (g_pair_open == 2) {  // another stream: the held GEMM goes alone
      HeldGemm h = g_held;
      h.p.grid = h.solo_grid;
      h.p.paired = 0;
      const int st = launch_variant(h.variant, h.p, h.s);
      if (st) return st;
    }
    g_held = HeldGemm{V, p, s, solo};
    g_pair_open = 2;
    return VMOE_OK;
  }
  const HeldGemm h = g_held;
  g_pair_open = 1;
  if (h.variant == DOWN_DH && V == DOWN_DW) return launch_pair_kernel<DOWN_DH, DOWN_DW>(h.p, p, s);
  if (h.variant == DOWN_DW && V == DOWN_DH) return launch_pair_kernel<DOWN_DW, DOWN_DH>(h.p, p, s);
  if (h.variant == UP_DW && V == UP_DX) return launch_pair_kernel<UP_DW, UP_DX>(h.p, p, s);
  if (h.variant == UP_DX && V == UP_DW) return launch_pair_kernel<UP_DX, UP_DW>(h.p, p, s);
  // no paired instance: each alone
  Args a = h.p;
  a.grid = h.solo_grid;
  a.paired = 0;
  int st = launch_variant(h.variant, a, s);
  if (st) return st;
  p.grid = solo;
  p.paired = 0;
  return launch_solo<V>(p, s);
}

template <int V>
int launch(Args p, int64_t items_bound, hipStream_t s) {
  if (items_bound <= 0) return VMOE_OK;
  p.grid = Cfg<V>::contig ? lane_grid() : gemm_grid(items_bound);
  return submit<V>(p, s);
}

// Workspace of a split dW launch: the arrival words (kConsumers per
// workgroup, 256-byte aligned region), then two partial tiles per workgroup.
inline size_t dw_arrive_bytes(int grid) {
  return ((size_t)grid * kConsumers * sizeof(uint32_t) + 255) / 256 * 256;
}

template <int V>
size_t dw_workspace(int grid) {
  return dw_arrive_bytes(grid) + (size_t)2 * grid * Cfg<V>::BM * Cfg<V>::BN * sizeof(float);
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
         ((nmax + out_cols<V>() - 1) / out_cols<V>());
}

// dW GEMM with split-K (one launch; split tiles are summed in the kernel).
template <int V>
int launch_dw(Args p, int64_t tmax, int64_t max_width, void* ws, size_t ws_bytes,
              hipStream_t s) {
  const int64_t E = p.E;
  p.lsh = lane_shift(p.hidden, max_width);
  if (!ws) {
    p.kc = 0;
    p.partial = nullptr;
    p.arrive = nullptr;
    return launch<V>(p, E * tmax, s);
  }
  // sum_e tiles_e * ceil(K_e / kc) <= tmax * (rows_bound / kc + E)
  const int64_t items = tmax * (E + p.rows_bound / kDwChunk + 1);
  if (items <= 0) return VMOE_OK;
  if (items > INT32_MAX || E * tmax > INT32_MAX) return VMOE_ERR_UNSUPPORTED;
  p.kc = kDwChunk;
  p.grid = lane_grid();
  if (ws_bytes < dw_workspace<V>(p.grid)) return VMOE_ERR_WORKSPACE;
  // (a paired launch runs on pair_grid() <= lane_grid() workgroups, whose
  // arrival words and partial slots are a prefix of these)
  p.arrive = reinterpret_cast<uint32_t*>(ws);
  p.partial = reinterpret_cast<float*>(static_cast<char*>(ws) + dw_arrive_bytes(p.grid));
  return submit<V>(p, s);
}

// Shared argument checks. Every dimension the kernels vectorise over must be a
// multiple of 8 elements and every base 16-byte aligned.
inline int check_common(const int32_t* eto, const int32_t* ewo, const int32_t* widths,
                        const int32_t* tpe, int32_t E, int64_t hidden, int64_t max_width,
                        int64_t rows_bound) {
  if (!eto || !ewo || !widths || !tpe || E <= 0 || hidden <= 0 || max_width < 0 ||
      rows_bound < 0)
    return VMOE_ERR_INVALID_ARG;
  if (E > kMaxExperts) return VMOE_ERR_UNSUPPORTED;
  if (hidden % 8 != 0 || max_width % 8 != 0 || hidden > INT32_MAX / 2 ||
      rows_bound > INT32_MAX)
    return VMOE_ERR_UNSUPPORTED;
  return VMOE_OK;
}

inline bool ld_ok(int64_t ld) { return ld > 0 && ld % 8 == 0; }

// Leading dimension of a source of `cols` columns; a source read through a
// row map may also be one row broadcast to all (ld = 0).
inline bool src_ld_ok(int64_t ld, int64_t cols, const int32_t* map) {
  return (map && ld == 0) || (ld_ok(ld) && ld >= cols);
}

// DMA offsets are 31-bit byte offsets from an operand base (rebased to the
// tile where rows are not gathered): every source the kernels address by a
// row index must span less than 2 GiB.
inline bool span_ok(int64_t rows, int64_t ld) { return rows * ld * 2 < ((int64_t)1 << 31); }

}  // namespace

void gemm_pair_begin() { g_pair_open = 1; }

int gemm_pair_end() {
  int st = VMOE_OK;
  if (g_pair_open == 2) {
    HeldGemm h = g_held;
    h.p.grid = h.solo_grid;
    h.p.paired = 0;
    st = launch_variant(h.variant, h.p, h.s);
  }
  g_pair_open = 0;
  return st;
}

}  // namespace vmoe

using namespace vmoe;

extern "C" int vmoe_gemm_up_fwd(const uint16_t* x, int64_t ldx, int64_t x_rows,
                                const int32_t* gather_map, const uint16_t* w1, int64_t ldw1,
                                uint16_t* out, uint16_t* pre_act, int64_t ldo, int32_t activation,
                                const float* row_scale, const int32_t* eto, const int32_t* ewo,
                                const int32_t* widths, const int32_t* tpe, int32_t E,
                                int64_t hidden, int64_t max_width, int64_t rows_bound,
                                vmoe_stream_t stream) {
  int st = check_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (activation != VMOE_ACT_NONE && activation != VMOE_ACT_RELU_SQUARED)
    return VMOE_ERR_INVALID_ARG;
  if (!x || !w1 || !out || x_rows < 0) return VMOE_ERR_INVALID_ARG;
  if (!src_ld_ok(ldx, hidden, gather_map) || !ld_ok(ldw1) || !ld_ok(ldo) || ldo < max_width)
    return VMOE_ERR_UNSUPPORTED;
  if (!a16(x) || !a16(w1) || !a16(out) || (pre_act && !a16(pre_act)))
    return VMOE_ERR_UNSUPPORTED;
  if ((gather_map && !span_ok(x_rows, ldx)) || !span_ok(hidden, ldw1))
    return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = x; p.lda = ldx; p.a_map = gather_map; p.a_rows = gather_map ? x_rows : 0;
  p.b = w1; p.ldb = ldw1;
  p.c = out; p.c2 = activation == VMOE_ACT_RELU_SQUARED ? pre_act : nullptr; p.ldc = ldo;
  p.row_scale = row_scale;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = activation; p.rows_bound = rows_bound;
  return launch<UP_FWD>(p, row_items<UP_FWD>(rows_bound, E, max_width),
                        reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vmoe_gemm_up_glu(const uint16_t* x, int64_t ldx, int64_t x_rows,
                                const int32_t* gather_map, const uint16_t* w1, int64_t ldw1,
                                uint16_t* out, uint16_t* gate, uint16_t* up, int64_t ldo,
                                const float* row_scale, const int32_t* eto, const int32_t* ewo,
                                const int32_t* widths, const int32_t* tpe, int32_t E,
                                int64_t hidden, int64_t max_width, int64_t rows_bound,
                                vmoe_stream_t stream) {
  int st = check_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (!x || !w1 || (!out && !gate && !up) || x_rows < 0) return VMOE_ERR_INVALID_ARG;
  if (!src_ld_ok(ldx, hidden, gather_map) || !ld_ok(ldw1) || !ld_ok(ldo) || ldo < max_width)
    return VMOE_ERR_UNSUPPORTED;
  if (!a16(x) || !a16(w1) || (out && !a16(out)) || (gate && !a16(gate)) || (up && !a16(up)))
    return VMOE_ERR_UNSUPPORTED;
  if ((gather_map && !span_ok(x_rows, ldx)) || !span_ok(hidden, ldw1))
    return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = x; p.lda = ldx; p.a_map = gather_map; p.a_rows = gather_map ? x_rows : 0;
  p.b = w1; p.ldb = ldw1;
  p.c = out; p.c2 = gate; p.c3 = up; p.ldc = ldo;
  p.row_scale = row_scale;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = VMOE_ACT_NONE; p.rows_bound = rows_bound;
  return launch<UP_GLU>(p, row_items<UP_GLU>(rows_bound, E, max_width),
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

extern "C" int vmoe_glu_grad(const uint16_t* grad_h, int64_t ldgh, const uint16_t* gate,
                             const uint16_t* up, int64_t ld, uint16_t* grad_gu, int64_t ldo,
                             const int32_t* eto, const int32_t* widths, const int32_t* tpe,
                             int32_t E, int64_t rows, int64_t max_width, vmoe_stream_t stream) {
  if (rows < 0 || E <= 0 || max_width < 0 || ld < max_width || ldgh < max_width ||
      ldo < 2 * max_width)
    return VMOE_ERR_INVALID_ARG;
  if (rows == 0 || max_width == 0) return VMOE_OK;
  if (!grad_h || !gate || !up || !grad_gu || !eto || !widths || !tpe)
    return VMOE_ERR_INVALID_ARG;
  if (E > kMaxExperts || max_width % 8 || ld % 8 || ldo % 8 || ldgh % 8 || !a16(grad_h) ||
      !a16(gate) || !a16(up) || !a16(grad_gu) || max_width > INT32_MAX / 2)
    return VMOE_ERR_UNSUPPORTED;
  VMOE_LAUNCH(glu_grad_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), grad_h, ldgh, gate, up, ld, grad_gu,
                     ldo, eto, widths, tpe, E, rows, (int)max_width);
  VMOE_CHECK_LAUNCH();
  return VMOE_OK;
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
  VMOE_LAUNCH(relu2_grad_kernel, dim3((unsigned)grid), dim3(256), 0,
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
  const int grid = lane_grid();
  return std::max(dw_workspace<UP_DW>(grid), dw_workspace<DOWN_DW>(grid));
}

extern "C" size_t vmoe_gemm_dw_workspace_zero_bytes(void) {
  // launch_dw's arrival words for the largest grid a dW launch takes
  return dw_arrive_bytes(kMaxDwGrid);
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
  if (!src_ld_ok(ldx, hidden, gather_map) || !ld_ok(ldg) || !ld_ok(ldgw))
    return VMOE_ERR_UNSUPPORTED;
  if (!a16(x) || !a16(grad_act) || !a16(grad_w1)) return VMOE_ERR_UNSUPPORTED;
  if (!span_ok(gather_map ? x_rows : rows_bound, ldx) || !span_ok(rows_bound, ldg))
    return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = x; p.lda = ldx; p.a_map = gather_map; p.a_rows = gather_map ? x_rows : 0;
  p.b = grad_act; p.ldb = ldg;
  p.c = grad_w1; p.ldc = ldgw;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = VMOE_ACT_NONE; p.rows_bound = rows_bound;
  return launch_dw<UP_DW>(p, tiles_max<UP_DW>(hidden, max_width), max_width, workspace,
                          workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vmoe_gemm_down_bwd_dh(const uint16_t* grad_y, int64_t ldgy, int64_t gy_rows,
                                     const int32_t* gather_map, const uint16_t* grad_scale,
                                     const uint16_t* w2,
                                     int64_t ldw2, const uint16_t* pre_act,
                                     const float* row_scale, uint16_t* grad_h, int64_t ldgh,
                                     const int32_t* eto, const int32_t* ewo,
                                     const int32_t* widths, const int32_t* tpe, int32_t E,
                                     int64_t hidden, int64_t max_width, int64_t rows_bound,
                                     float* row_dot, int64_t ld_row_dot, vmoe_stream_t stream) {
  int st = check_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (!grad_y || !w2 || !grad_h || gy_rows < 0) return VMOE_ERR_INVALID_ARG;
  if (row_dot && (!pre_act || ld_row_dot < (max_width + 63) / 64)) return VMOE_ERR_INVALID_ARG;
  if (!src_ld_ok(ldgy, hidden, gather_map) || !ld_ok(ldw2) || !ld_ok(ldgh) || ldw2 < hidden ||
      ldgh < max_width)
    return VMOE_ERR_UNSUPPORTED;
  if (!a16(grad_y) || !a16(w2) || !a16(grad_h) || (pre_act && !a16(pre_act)))
    return VMOE_ERR_UNSUPPORTED;
  if (gather_map && !span_ok(gy_rows, ldgy)) return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = grad_y; p.lda = ldgy; p.a_map = gather_map; p.a_rows = gather_map ? gy_rows : 0;
  p.b = w2; p.ldb = ldw2;
  p.c = grad_h; p.ldc = ldgh;
  p.pre = pre_act;
  p.row_scale = row_scale;
  p.gscale = grad_scale;
  p.row_dot = row_dot; p.ld_rd = ld_row_dot;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = VMOE_ACT_NONE; p.rows_bound = rows_bound;
  return launch<DOWN_DH>(p, row_items<DOWN_DH>(rows_bound, E, max_width),
                         reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vmoe_gemm_down_bwd_dw(const uint16_t* h, int64_t ldh, const uint16_t* grad_y,
                                     int64_t ldgy, int64_t gy_rows, const int32_t* gather_map,
                                     const uint16_t* grad_scale, uint16_t* grad_w2, int64_t ldgw, const int32_t* eto,
                                     const int32_t* ewo, const int32_t* widths,
                                     const int32_t* tpe, int32_t E, int64_t hidden,
                                     int64_t max_width, int64_t rows_bound, void* workspace,
                                     size_t workspace_bytes, vmoe_stream_t stream) {
  int st = check_common(eto, ewo, widths, tpe, E, hidden, max_width, rows_bound);
  if (st) return st;
  if (!h || !grad_y || !grad_w2 || gy_rows < 0) return VMOE_ERR_INVALID_ARG;
  if (!ld_ok(ldh) || !src_ld_ok(ldgy, hidden, gather_map) || !ld_ok(ldgw) || ldgw < hidden)
    return VMOE_ERR_UNSUPPORTED;
  if (!a16(h) || !a16(grad_y) || !a16(grad_w2)) return VMOE_ERR_UNSUPPORTED;
  if (!span_ok(rows_bound, ldh) || !span_ok(gather_map ? gy_rows : rows_bound, ldgy))
    return VMOE_ERR_UNSUPPORTED;
  Args p{};
  p.a = grad_y; p.lda = ldgy; p.a_map = gather_map; p.a_rows = gather_map ? gy_rows : 0;
  p.b = h; p.ldb = ldh;
  p.gscale = grad_scale;
  p.c = grad_w2; p.ldc = ldgw;
  p.eto = eto; p.ewo = ewo; p.widths = widths; p.tpe = tpe;
  p.E = E; p.hidden = (int)hidden; p.act = VMOE_ACT_NONE; p.rows_bound = rows_bound;
  return launch_dw<DOWN_DW>(p, tiles_max<DOWN_DW>(hidden, max_width), max_width, workspace,
                            workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}
