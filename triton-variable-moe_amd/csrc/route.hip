// Routing on gfx950: stable counting sort of expert ids, histogram, rounded
// inclusive scans and the padded-row maps, in two launches (one after the
// module's top-k, which writes the histograms; three above 1024 experts).
//
// Semantics follow fused_route (triton_moe/kernels/fused_cumsum.py:85-171):
//   sorted order = torch.sort(selected, stable=True), i.e. by expert id, ties
//   by ascending assignment index; tokens_per_expert = bincount; rounded =
//   round_{up,down,nearest}(count, block) (fused_cumsum.py:61-66); kept =
//   min(count, rounded) (:71); bins / padded_bins = inclusive cumsums of kept /
//   rounded (:76-77); with dropping, the sorted arrays keep the first `kept`
//   entries of each expert (:154-169).
// and precompute_gather_map (triton_moe/kernels/grouped_gemm.py:104-149):
//   the q-th kept assignment of expert e lands on padded row
//   padded_bins[e-1] + q, and gather_map[row] = assignment / top_k.
//
// Stable counting sort, MI355X style: the assignments are cut into tiles of
// kTile; launch 1 counts experts per tile in LDS; the placement launch then
// derives, in every workgroup, the first sorted position of each (expert,
// tile) from those counts (expert-major order of the prefix is exactly the
// sort key order), re-reads its tile and ranks equal ids within a wave with
// ballots, so the order inside an expert is the original order (stable),
// without any comparison sort (route_small_kernel for E <= 64,
// route_fused_kernel up to 1024 experts; beyond that a single-workgroup scan
// launch, route_scan_kernel, and route_place_kernel).

#include <algorithm>
#include <mutex>

#include "router_aux.h"
#include "vmoe_common.h"

namespace vmoe {
namespace {

// One assignment per thread of a 1024-assignment tile: the placement
// ranks each wave's 64 assignments with one round of ballots, and the
// per-expert totals of the two-launch path take one round of loads (16
// lanes per expert at E = 64); 256 threads measured 14.0 + 4.6 us at cfg3
// against 10.9 + 2.7 us.
constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / kWave;
constexpr int kTile = kRouteTile;               // assignments per tile
constexpr int kWaveSpan = kTile / kRouteWaves;  // contiguous assignments per wave
constexpr int kMaxExperts = 2048;  // the placement's per-wave tables, 17 E ints, fit the LDS
constexpr int kScanThreads = 1024;

__device__ __forceinline__ int64_t load_sel(const void* sel, int is64, int64_t p) {
  return is64 ? reinterpret_cast<const int64_t*>(sel)[p]
              : (int64_t)reinterpret_cast<const int32_t*>(sel)[p];
}

// Workspace layout (int32): counts [E * ntiles * S], bad-id flag per count
// column [ntiles * S], then per expert: start (first unkept sorted
// position), kept, bs (bins[e-1]), ps (padded_bins[e-1]). S = 1 (one count
// column per tile) except after vmoe_router_topk_hist (route_hist_split).
struct RouteWs {
  int32_t* counts;
  int32_t* bad;
  int32_t* start;
  int32_t* kept;
  int32_t* bs;
  int32_t* ps;
};

__host__ __device__ inline int64_t route_ntiles(int64_t A) { return route_tiles(A); }

__host__ __device__ inline RouteWs route_ws(void* base, int64_t A, int E, int S = 1) {
  RouteWs w;
  int32_t* p = reinterpret_cast<int32_t*>(base);
  w.counts = p;
  p += (int64_t)E * route_ntiles(A) * S;
  w.bad = p;
  p += route_ntiles(A) * S;
  w.start = p; p += E;
  w.kept = p; p += E;
  w.bs = p; p += E;
  w.ps = p;
  return w;
}

// Launch 1: per-tile expert histogram.
__global__ __launch_bounds__(kRouteThreads) void route_hist_kernel(
    const void* __restrict__ sel, int is64, int64_t A, int E, int ntiles,
    int32_t* __restrict__ counts, int32_t* __restrict__ bad_flags) {
  extern __shared__ int32_t hist[];
  __shared__ int32_t any_bad;
  if (threadIdx.x == 0) any_bad = 0;
  for (int e = threadIdx.x; e < E; e += kRouteThreads) hist[e] = 0;
  __syncthreads();
  const int64_t t0 = (int64_t)blockIdx.x * kTile;
  const int64_t t1 = min(A, t0 + kTile);
  bool bad = false;
  for (int64_t p = t0 + threadIdx.x; p < t1; p += kRouteThreads) {
    int64_t e = load_sel(sel, is64, p);
    if (e >= 0 && e < E)
      atomicAdd(&hist[(int)e], 1);
    else
      bad = true;
  }
  if (bad) any_bad = 1;
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kRouteThreads)
    counts[(int64_t)e * ntiles + blockIdx.x] = hist[e];
  if (threadIdx.x == 0) bad_flags[blockIdx.x] = any_bad;
}

__device__ __forceinline__ int32_t round_count(int32_t c, int32_t b, int mode) {
  if (mode == VMOE_ROUND_UP) return ((c + b - 1) / b) * b;
  if (mode == VMOE_ROUND_DOWN) return (c / b) * b;
  return ((c + b / 2) / b) * b;
}

// Launch 2: one workgroup. Flat exclusive scan of counts[E][ntiles] in place,
// then per-expert rounding and the bins / padded_bins scans, then the pad
// rows of row_src / gather_map, then info[].
__global__ __launch_bounds__(kScanThreads) void route_scan_kernel(
    RouteWs ws, int E, int ntiles, int block, int mode, int32_t* __restrict__ tpe,
    int32_t* __restrict__ bins, int32_t* __restrict__ padded_bins,
    int32_t* __restrict__ row_src, int32_t* __restrict__ gather_map, int32_t map_pad,
    float* __restrict__ row_weight, int64_t row_capacity, int32_t* __restrict__ info,
    int32_t* __restrict__ expert_offsets, int32_t* __restrict__ padded_counts) {
  __shared__ int32_t scan_smem[kScanThreads / kWave + 1];
  __shared__ int32_t carry_kept, carry_rounded, any_bad;
  extern __shared__ int32_t lds[];
  int32_t* expert_start = lds;        // [E + 1]
  int32_t* ps_lds = lds + E + 1;      // [E]
  int32_t* kept_lds = ps_lds + E;     // [E]
  int32_t* rounded_lds = kept_lds + E;  // [E]

  const int tid = threadIdx.x;
  if (tid == 0) {
    carry_kept = 0;
    carry_rounded = 0;
    any_bad = 0;
  }
  const int64_t n = (int64_t)E * ntiles;
  const int64_t per = (n + kScanThreads - 1) / kScanThreads;
  const int64_t i0 = min(n, per * tid), i1 = min(n, i0 + per);
  int32_t s = 0;
  for (int64_t i = i0; i < i1; ++i) s += ws.counts[i];
  int32_t total;
  int32_t run = block_exclusive_scan<int32_t, kScanThreads>(s, scan_smem, &total);
  // any_bad was zeroed before the scan's barriers.
  bool bad = false;
  for (int t = tid; t < ntiles; t += kScanThreads) bad |= ws.bad[t] != 0;
  if (bad) any_bad = 1;
  for (int64_t i = i0; i < i1; ++i) {
    int32_t c = ws.counts[i];
    ws.counts[i] = run;
    if (i % ntiles == 0) expert_start[i / ntiles] = run;
    run += c;
  }
  // With no tiles every expert starts at 0.
  if (ntiles == 0)
    for (int e = tid; e < E; e += kScanThreads) expert_start[e] = 0;
  if (tid == 0) expert_start[E] = total;
  __syncthreads();

  // Per-expert counts, rounding and the two inclusive scans, 1024 experts per pass.
  for (int e0 = 0; e0 < E; e0 += kScanThreads) {
    const int e = e0 + tid;
    int32_t c = 0, r = 0, k = 0;
    if (e < E) {
      c = expert_start[e + 1] - expert_start[e];
      r = round_count(c, block, mode);
      k = min(c, r);
    }
    int32_t tot_k, tot_r;
    const int32_t ek = block_exclusive_scan<int32_t, kScanThreads>(k, scan_smem, &tot_k);
    __syncthreads();
    const int32_t er = block_exclusive_scan<int32_t, kScanThreads>(r, scan_smem, &tot_r);
    const int32_t bk = carry_kept, br = carry_rounded;
    if (e < E) {
      tpe[e] = c;
      bins[e] = bk + ek + k;
      padded_bins[e] = br + er + r;
      ws.start[e] = expert_start[e];
      ws.kept[e] = k;
      ws.bs[e] = bk + ek;
      ws.ps[e] = br + er;
      ps_lds[e] = br + er;
      kept_lds[e] = k;
      rounded_lds[e] = r;
      // The module's expert_token_offsets = [0, padded_bins] and padded
      // tokens_per_expert = diff(padded_bins) (moe.py:193-202).
      if (expert_offsets) {
        expert_offsets[e + 1] = br + er + r;
        if (e == 0) expert_offsets[0] = 0;
      }
      if (padded_counts) padded_counts[e] = r;
    }
    __syncthreads();
    if (tid == 0) {
      carry_kept = bk + tot_k;
      carry_rounded = br + tot_r;
    }
    __syncthreads();
  }

  // Pad rows [ps + kept, ps + rounded) of every expert: one wave per expert.
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  for (int e = wave; e < E; e += kScanThreads / kWave) {
    const int64_t ps = ps_lds[e];
    for (int32_t q = kept_lds[e] + lane; q < rounded_lds[e]; q += kWave) {
      const int64_t row = ps + q;
      if (row < row_capacity) {
        row_src[row] = -1;
        gather_map[row] = map_pad;
        if (row_weight) row_weight[row] = 0.0f;
      }
    }
  }
  if (tid == 0) {
    int32_t err = any_bad ? (int32_t)VMOE_ROUTE_BAD_EXPERT_ID : 0;
    if ((int64_t)carry_rounded > row_capacity) err |= (int32_t)VMOE_ROUTE_ROW_OVERFLOW;
    info[VMOE_INFO_ROWS] = carry_rounded;
    info[VMOE_INFO_KEPT] = carry_kept;
    info[VMOE_INFO_ERRORS] = err;
    info[3] = 0;
  }
}

constexpr int kSpanSteps = kWaveSpan / kWave;

// One wave's span of a tile, held in registers from the start of the
// placement kernels so the loads overlap the prefix work: expert id per
// assignment (-1 past A or out of range) and its bf16 routing weight.
struct TileSel {
  int32_t e[kSpanSteps];
  uint16_t w[kSpanSteps];
};

__device__ __forceinline__ TileSel load_tile(const void* __restrict__ sel, int is64, int64_t A,
                                             int E, int tile,
                                             const uint16_t* __restrict__ weights) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int64_t w0 = (int64_t)tile * kTile + (int64_t)wave * kWaveSpan;
  TileSel t;
#pragma unroll
  for (int i = 0; i < kSpanSteps; ++i) {
    const int64_t p = w0 + i * kWave + lane;
    int64_t ev = -1;
    uint16_t wv = 0;
    if (p < A) {
      ev = load_sel(sel, is64, p);
      if (weights) wv = weights[p];
    }
    t.e[i] = ev >= 0 && ev < E ? (int32_t)ev : -1;
    t.w[i] = wv;
  }
  return t;
}

// Stable placement of tile `tile` (kTile assignments). Each wave walks its
// kWaveSpan assignments in order, 64 at a time; lanes holding the same
// expert id find each other with ballots over the id bits, and rank = number
// of equal lanes below. tile_start[e] is the sorted position of the tile's
// first assignment of expert e; start/kept/bs/ps are per expert (the sorted
// position of the expert's first assignment, its kept count, bins[e-1] and
// padded_bins[e-1]). wbase is kRouteWaves * E ints of LDS.
__device__ void place_tile(const TileSel& ts, int E, int nbits, int tile, int top_k,
                           const int32_t* tile_start, const int32_t* start,
                           const int32_t* kept, const int32_t* bs, const int32_t* ps,
                           int32_t* wbase, int32_t* __restrict__ bin_ids,
                           int32_t* __restrict__ indices, int32_t* __restrict__ row_src,
                           int32_t* __restrict__ gather_map, int64_t row_capacity,
                           int32_t* __restrict__ assignment_row,
                           float* __restrict__ row_weight) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  for (int i = tid; i < kRouteWaves * E; i += kRouteThreads) wbase[i] = 0;
  __syncthreads();

  const int64_t w0 = (int64_t)tile * kTile + (int64_t)wave * kWaveSpan;
  // Per-wave histogram of this wave's span.
#pragma unroll
  for (int i = 0; i < kSpanSteps; ++i)
    if (ts.e[i] >= 0) atomicAdd(&wbase[wave * E + ts.e[i]], 1);
  __syncthreads();
  // Turn the per-wave counts into per-wave first sorted positions.
  for (int e = tid; e < E; e += kRouteThreads) {
    int32_t run = tile_start[e];
#pragma unroll
    for (int w = 0; w < kRouteWaves; ++w) {
      int32_t c = wbase[w * E + e];
      wbase[w * E + e] = run;
      run += c;
    }
  }
  __syncthreads();

  int32_t* base = wbase + wave * E;
#pragma unroll
  for (int st = 0; st < kSpanSteps; ++st) {
    const int64_t p = w0 + st * kWave + lane;
    const bool valid = ts.e[st] >= 0;
    const int e = valid ? ts.e[st] : 0;
    uint64_t same = ballot64(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t ones = ballot64(valid && bit);
      same &= bit ? ones : ~ones;
    }
    const int rank = lanes_below(same);
    int32_t first = 0;
    if (valid) first = base[e];
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      const int32_t q = first + rank - start[e];  // rank inside expert e
      if (q < kept[e]) {
        const int32_t i = bs[e] + q;
        const int64_t row = (int64_t)ps[e] + q;
        bin_ids[i] = e;
        indices[i] = (int32_t)p;
        assignment_row[p] = (int32_t)row;
        if (row < row_capacity) {
          row_src[row] = (int32_t)p;
          gather_map[row] = (int32_t)(p / top_k);
          if (row_weight) row_weight[row] = __uint_as_float((uint32_t)ts.w[st] << 16);
        }
      } else {
        assignment_row[p] = -1;
      }
      if (rank == 0) base[e] = first + __popcll(same);
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// Launch 3 (three-launch path): placement from the scan's in-place prefix.
__global__ __launch_bounds__(kRouteThreads) void route_place_kernel(
    const void* __restrict__ sel, int is64, int64_t A, int E, int nbits, int ntiles,
    int top_k, RouteWs ws, int32_t* __restrict__ bin_ids, int32_t* __restrict__ indices,
    int32_t* __restrict__ row_src, int32_t* __restrict__ gather_map, int64_t row_capacity,
    int32_t* __restrict__ assignment_row, const uint16_t* __restrict__ weights,
    float* __restrict__ row_weight) {
  extern __shared__ int32_t lds[];
  int32_t* wbase = lds;                        // [kRouteWaves][E]
  int32_t* tile_start = wbase + kRouteWaves * E;  // [E]
  const TileSel ts = load_tile(sel, is64, A, E, blockIdx.x, row_weight ? weights : nullptr);
  for (int e = threadIdx.x; e < E; e += kRouteThreads)
    tile_start[e] = ws.counts[(int64_t)e * ntiles + blockIdx.x];
  place_tile(ts, E, nbits, blockIdx.x, top_k, tile_start, ws.start, ws.kept, ws.bs, ws.ps,
             wbase, bin_ids, indices, row_src, gather_map, row_capacity, assignment_row,
             row_weight);
}

// Launch 2 of the two-launch path (E <= kFusedMaxExperts and E * tiles <=
// kFusedMaxCounts): every workgroup derives what the scan would give it from
// the per-tile histograms (E * tiles counts, from L2): per-expert totals and
// the prefix of its own tile (one wave per expert), then the rounded counts
// and the scans over experts; workgroup 0 writes the per-expert outputs and
// info[], workgroup b the pad rows of experts e = b (mod grid), and workgroup
// b < tiles places tile b. This saves the single-workgroup scan launch.
constexpr int kFusedMaxExperts = 1024;
constexpr int64_t kFusedMaxCounts = 65536;

__global__ __launch_bounds__(kRouteThreads) void route_fused_kernel(
    const void* __restrict__ sel, int is64, int64_t A, int E, int nbits, int ntiles, int S,
    int block, int mode, int top_k, RouteWs ws, int32_t* __restrict__ tpe,
    int32_t* __restrict__ bins, int32_t* __restrict__ padded_bins,
    int32_t* __restrict__ bin_ids, int32_t* __restrict__ indices,
    int32_t* __restrict__ row_src, int32_t* __restrict__ gather_map, int32_t map_pad,
    int64_t row_capacity, int32_t* __restrict__ assignment_row,
    const uint16_t* __restrict__ weights, float* __restrict__ row_weight,
    int32_t* __restrict__ info, int32_t* __restrict__ expert_offsets,
    int32_t* __restrict__ padded_counts) {
  __shared__ int32_t scan_smem[kRouteWaves + 1];
  __shared__ int32_t tot_k, tot_r, any_bad;
  extern __shared__ int32_t lds[];
  int32_t* wbase = lds;                       // [kRouteWaves][E]
  int32_t* cnt = wbase + kRouteWaves * E;     // [E] tokens per expert
  int32_t* tstart = cnt + E;                  // [E] count in tiles before this one, then start
  int32_t* start = tstart + E;                // [E]
  int32_t* kept = start + E;                  // [E]
  int32_t* rnd = kept + E;                    // [E]
  int32_t* bs = rnd + E;                      // [E]
  int32_t* ps = bs + E;                       // [E]
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int b = blockIdx.x;
  if (tid == 0) any_bad = 0;
  const TileSel ts = load_tile(sel, is64, A, E, b, row_weight ? weights : nullptr);

  // Totals and this tile's prefix: G lanes per expert (a power of two that
  // divides the wave), each summing every G-th count column (S per tile), so
  // a thread has all of its counts loads in flight at once; then a
  // butterfly over the G lanes.
  int G = kWave;
  while (G > 1 && G * E > kRouteThreads) G >>= 1;
  const int j = tid & (G - 1);
  const int ncols = ntiles * S, bcol = b * S;
  for (int e = tid / G; e < E; e += kRouteThreads / G) {
    const int32_t* c = ws.counts + (int64_t)e * ncols;
    int32_t tot = 0, pre = 0;
    int t = j;
    // 16 loads in flight per round (one round at cfg3's 256 columns)
    for (; t + 15 * G < ncols; t += 16 * G) {
      int32_t v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = c[t + u * G];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        tot += v[u];
        pre += t + u * G < bcol ? v[u] : 0;
      }
    }
#pragma unroll 8
    for (; t < ncols; t += G) {
      const int32_t v = c[t];
      tot += v;
      pre += t < bcol ? v : 0;
    }
    for (int off = G / 2; off > 0; off >>= 1) {
      tot += __shfl_xor(tot, off, kWave);
      pre += __shfl_xor(pre, off, kWave);
    }
    if (j == 0) {
      cnt[e] = tot;
      tstart[e] = pre;
    }
  }
  __syncthreads();
  // Scans over experts (E <= 1024: up to 4 consecutive experts per thread).
  const int per = (E + kRouteThreads - 1) / kRouteThreads;
  const int e0 = min(E, tid * per), e1 = min(E, e0 + per);
  int32_t sc = 0, sk = 0, sr = 0;
  for (int e = e0; e < e1; ++e) {
    const int32_t c = cnt[e], r = round_count(c, block, mode);
    rnd[e] = r;
    kept[e] = min(c, r);
    sc += c;
    sk += min(c, r);
    sr += r;
  }
  int32_t t_c, t_k, t_r;
  int32_t xc = block_exclusive_scan<int32_t, kRouteThreads>(sc, scan_smem, &t_c);
  __syncthreads();
  int32_t xk = block_exclusive_scan<int32_t, kRouteThreads>(sk, scan_smem, &t_k);
  __syncthreads();
  int32_t xr = block_exclusive_scan<int32_t, kRouteThreads>(sr, scan_smem, &t_r);
  for (int e = e0; e < e1; ++e) {
    start[e] = xc;
    tstart[e] += xc;
    bs[e] = xk;
    ps[e] = xr;
    xc += cnt[e];
    xk += kept[e];
    xr += rnd[e];
  }
  if (tid == 0) {
    tot_k = t_k;
    tot_r = t_r;
  }
  if (b == 0) {
    bool bad = false;
    for (int t = tid; t < ntiles * S; t += kRouteThreads) bad |= ws.bad[t] != 0;
    if (bad) any_bad = 1;
  }
  __syncthreads();

  if (b == 0) {
    for (int e = tid; e < E; e += kRouteThreads) {
      tpe[e] = cnt[e];
      bins[e] = bs[e] + kept[e];
      padded_bins[e] = ps[e] + rnd[e];
      // The module's expert_token_offsets = [0, padded_bins] and padded
      // tokens_per_expert = diff(padded_bins) (moe.py:193-202).
      if (expert_offsets) {
        expert_offsets[e + 1] = ps[e] + rnd[e];
        if (e == 0) expert_offsets[0] = 0;
      }
      if (padded_counts) padded_counts[e] = rnd[e];
    }
    if (tid == 0) {
      int32_t err = any_bad ? (int32_t)VMOE_ROUTE_BAD_EXPERT_ID : 0;
      if ((int64_t)tot_r > row_capacity) err |= (int32_t)VMOE_ROUTE_ROW_OVERFLOW;
      info[VMOE_INFO_ROWS] = tot_r;
      info[VMOE_INFO_KEPT] = tot_k;
      info[VMOE_INFO_ERRORS] = err;
      info[3] = 0;
    }
  }
  // Pad rows [ps + kept, ps + rounded) of the experts this workgroup owns.
  for (int e = b + (int)gridDim.x * wave; e < E; e += (int)gridDim.x * kRouteWaves) {
    for (int32_t q = kept[e] + lane; q < rnd[e]; q += kWave) {
      const int64_t row = (int64_t)ps[e] + q;
      if (row < row_capacity) {
        row_src[row] = -1;
        gather_map[row] = map_pad;
        if (row_weight) row_weight[row] = 0.0f;
      }
    }
  }
  if (b < ntiles)
    place_tile(ts, E, nbits, b, top_k, tstart, start, kept, bs, ps, wbase, bin_ids, indices,
               row_src, gather_map, row_capacity, assignment_row, row_weight);
}

// The same launch for E <= 64 experts, with two workgroup barriers instead
// of the nine of route_fused_kernel: lane e of every wave holds expert e, so
// each wave runs the scans over experts itself (shuffles, no LDS) and reads
// the values of its assignments' experts with shuffles. Thread t of
// workgroup b places assignment b * kTile + t; its rank among equal ids in
// its wave comes from ballots over the id bits, the counts of the waves
// before it from an LDS table [wave][expert].
constexpr int kSmallExperts = kWave;
static_assert(kTile == kRouteThreads, "one assignment per thread");

__global__ __launch_bounds__(kRouteThreads) void route_small_kernel(
    const void* __restrict__ sel, int is64, int64_t A, int E, int nbits, int ntiles, int S,
    int block, int mode, int top_k, RouteWs ws, int32_t* __restrict__ tpe,
    int32_t* __restrict__ bins, int32_t* __restrict__ padded_bins,
    int32_t* __restrict__ bin_ids, int32_t* __restrict__ indices,
    int32_t* __restrict__ row_src, int32_t* __restrict__ gather_map, int32_t map_pad,
    int64_t row_capacity, int32_t* __restrict__ assignment_row,
    const uint16_t* __restrict__ weights, float* __restrict__ row_weight,
    int32_t* __restrict__ info, int32_t* __restrict__ expert_offsets,
    int32_t* __restrict__ padded_counts, RouteAux aux) {
  __shared__ int32_t wcnt[kRouteWaves][kSmallExperts];  // ids of expert e in wave w
  __shared__ int32_t cnt_s[kSmallExperts], pre_s[kSmallExperts];
  __shared__ int32_t any_bad;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int b = blockIdx.x;
  wcnt[wave][lane] = 0;
  if (tid == 0) any_bad = 0;
  const int64_t p = (int64_t)b * kTile + tid;
  int32_t e = -1;
  uint16_t wv = 0;
  if (p < A) {
    const int64_t ev = load_sel(sel, is64, p);
    if (row_weight) wv = weights[p];
    e = ev >= 0 && ev < E ? (int32_t)ev : -1;
  }
  // Totals and this tile's prefix per expert, G lanes per expert (as in
  // route_fused_kernel); workgroup 0 also collects the bad-id flags.
  int G = kWave;
  while (G > 1 && G * E > kRouteThreads) G >>= 1;
  const int j = tid & (G - 1), ex = tid / G;
  const int ncols = ntiles * S, bcol = b * S;
  int32_t tot = 0, pre = 0;
  if (ex < E) {
    const int32_t* c = ws.counts + (int64_t)ex * ncols;
    int t = j;
    for (; t + 15 * G < ncols; t += 16 * G) {
      int32_t v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = c[t + u * G];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        tot += v[u];
        pre += t + u * G < bcol ? v[u] : 0;
      }
    }
#pragma unroll 8
    for (; t < ncols; t += G) {
      const int32_t v = c[t];
      tot += v;
      pre += t < bcol ? v : 0;
    }
  }
  bool bad = false;
  if (b == 0)
    for (int t = tid; t < ncols; t += kRouteThreads) bad |= ws.bad[t] != 0;
  __syncthreads();  // wcnt zeroed
  for (int off = G / 2; off > 0; off >>= 1) {
    tot += __shfl_xor(tot, off, kWave);
    pre += __shfl_xor(pre, off, kWave);
  }
  if (ex < E && j == 0) {
    cnt_s[ex] = tot;
    pre_s[ex] = pre;
  }
  if (bad) any_bad = 1;
  // Rank among the equal ids of this wave; the lowest lane of each id
  // records the id's count in this wave.
  const bool valid = e >= 0;
  const int ee = valid ? e : 0;
  uint64_t same = ballot64(valid);
  for (int bit = 0; bit < nbits; ++bit) {
    const bool on = (ee >> bit) & 1;
    const uint64_t ones = ballot64(valid && on);
    same &= on ? ones : ~ones;
  }
  const int rank = lanes_below(same);
  if (valid && rank == 0) wcnt[wave][ee] = __popcll(same);
  __syncthreads();
  // The workgroup after the placement ones (launched only with aux.partial)
  // owns no assignments; it forms the auxiliary losses from the expert
  // totals it has just summed.
  const int nplace = max(ntiles, 1);
  if (b == nplace) {
    router_aux_block<false>(aux.partial, aux.nblk, aux.T, E, cnt_s, aux.coef, aux.wn, aux.f_i,
                            aux.f_i32, aux.p_i, aux.z, aux.losses);
    return;
  }

  // Per expert (lane x = expert x): count, rounded count, kept, and the
  // exclusive scans over experts of all three.
  const int32_t cx = lane < E ? cnt_s[lane] : 0;
  const int32_t px = lane < E ? pre_s[lane] : 0;
  const int32_t rx = lane < E ? round_count(cx, block, mode) : 0;
  const int32_t kx = min(cx, rx);
  const int32_t ic = wave_inclusive_scan(cx), ik = wave_inclusive_scan(kx),
                ir = wave_inclusive_scan(rx);
  const int32_t bsx = ik - kx, psx = ir - rx;
  (void)ic;
  // Counts of expert e in the waves before this one.
  int32_t before = 0;
  for (int w = 0; w < wave; ++w) before += wcnt[w][ee];
  const int32_t pre_e = __shfl(px, ee, kWave), kept_e = __shfl(kx, ee, kWave);
  const int32_t bs_e = __shfl(bsx, ee, kWave), ps_e = __shfl(psx, ee, kWave);
  if (valid) {
    const int32_t q = pre_e + before + rank;  // rank inside expert e
    if (q < kept_e) {
      const int32_t i = bs_e + q;
      const int64_t row = (int64_t)ps_e + q;
      bin_ids[i] = e;
      indices[i] = (int32_t)p;
      assignment_row[p] = (int32_t)row;
      if (row < row_capacity) {
        row_src[row] = (int32_t)p;
        gather_map[row] = (int32_t)(p / top_k);
        if (row_weight) row_weight[row] = __uint_as_float((uint32_t)wv << 16);
      }
    } else {
      assignment_row[p] = -1;
    }
  }
  if (b == 0 && wave == 0) {
    if (lane < E) {
      tpe[lane] = cx;
      bins[lane] = ik;
      padded_bins[lane] = ir;
      // The module's expert_token_offsets = [0, padded_bins] and padded
      // tokens_per_expert = diff(padded_bins) (moe.py:193-202).
      if (expert_offsets) {
        expert_offsets[lane + 1] = ir;
        if (lane == 0) expert_offsets[0] = 0;
      }
      if (padded_counts) padded_counts[lane] = rx;
    }
    const int32_t tot_k = __shfl(ik, kWave - 1, kWave), tot_r = __shfl(ir, kWave - 1, kWave);
    if (lane == 0) {
      int32_t err = any_bad ? (int32_t)VMOE_ROUTE_BAD_EXPERT_ID : 0;
      if ((int64_t)tot_r > row_capacity) err |= (int32_t)VMOE_ROUTE_ROW_OVERFLOW;
      info[VMOE_INFO_ROWS] = tot_r;
      info[VMOE_INFO_KEPT] = tot_k;
      info[VMOE_INFO_ERRORS] = err;
      info[3] = 0;
    }
  }
  // Pad rows [ps + kept, ps + rounded) of the experts this workgroup owns.
  for (int x = b + nplace * wave; x < E; x += nplace * kRouteWaves) {
    const int32_t kept_x = __shfl(kx, x, kWave), rnd_x = __shfl(rx, x, kWave);
    const int32_t ps_x = __shfl(psx, x, kWave);
    for (int32_t q = kept_x + lane; q < rnd_x; q += kWave) {
      const int64_t row = (int64_t)ps_x + q;
      if (row < row_capacity) {
        row_src[row] = -1;
        gather_map[row] = map_pad;
        if (row_weight) row_weight[row] = 0.0f;
      }
    }
  }
}

// Row maps from caller arrays (vmoe_row_maps): init, then place.
__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

__global__ void row_maps_place_kernel(const int32_t* __restrict__ indices,
                                      const int32_t* __restrict__ bin_ids,
                                      const int32_t* __restrict__ bins,
                                      const int32_t* __restrict__ padded_bins,
                                      int64_t num_sorted, int E, int top_k, int64_t num_rows,
                                      int64_t num_assignments, int32_t* __restrict__ row_src,
                                      int32_t* __restrict__ gather_map,
                                      int32_t* __restrict__ assignment_row) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < num_sorted;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int e = bin_ids[i];
    if (e < 0 || e >= E) continue;
    const int64_t bs = e > 0 ? bins[e - 1] : 0;
    const int64_t ps = e > 0 ? padded_bins[e - 1] : 0;
    const int64_t row = ps + i - bs;
    const int32_t a = indices[i];
    if (row < 0 || row >= num_rows) continue;
    if (row_src) row_src[row] = a;
    if (gather_map) gather_map[row] = a / top_k;
    if (assignment_row && a >= 0 && a < num_assignments) assignment_row[a] = (int32_t)row;
  }
}

inline int grid_for(int64_t n, int threads, int cap = 65536) {
  int64_t g = (n + threads - 1) / threads;
  return (int)std::max<int64_t>(1, std::min<int64_t>(g, cap));
}

}  // namespace
}  // namespace vmoe

using namespace vmoe;

extern "C" int vmoe_route_max_experts(void) { return kMaxExperts; }

namespace {
size_t route_ws_size(int64_t A, int E, int S) {
  const size_t nt = (size_t)route_ntiles(A) * (size_t)S;
  return sizeof(int32_t) * ((size_t)E * nt + nt + 4 * (size_t)E) + 256;
}
}  // namespace

extern "C" size_t vmoe_route_workspace_bytes(int64_t A, int32_t E) {
  if (A < 0 || E <= 0) return 0;
  return route_ws_size(A, E, 1);
}

extern "C" size_t vmoe_route_counted_workspace_bytes(int64_t T, int32_t E, int32_t top_k) {
  const int S = T > 0 && E > 0 ? route_hist_split(T, E, top_k) : 0;
  return S ? route_ws_size(T * top_k, E, S) : 0;
}

namespace {
// vmoe_route; `counted`: the workspace already holds the per-tile counts and
// bad-id flags (vmoe_router_topk_hist), so launch 1 is skipped.
int route_impl(const void* sel, int32_t is64, int64_t A, int32_t E, int32_t top_k,
               int32_t block, int32_t rounding, int32_t* bin_ids, int32_t* indices,
               int32_t* tpe, int32_t* bins, int32_t* padded_bins, int32_t* row_src,
               int32_t* gather_map, int32_t gather_map_pad, int64_t row_capacity,
               int32_t* assignment_row, int32_t* info, int32_t* expert_offsets,
               int32_t* padded_counts, const uint16_t* weights, float* row_weight,
               void* workspace, size_t ws_bytes, vmoe_stream_t stream, bool counted,
               const RouteAux* aux = nullptr, bool* aux_done = nullptr) {
  if (A < 0 || E <= 0 || top_k <= 0 || block <= 0 || row_capacity < 0)
    return VMOE_ERR_INVALID_ARG;
  if (rounding < VMOE_ROUND_UP || rounding > VMOE_ROUND_NEAREST) return VMOE_ERR_INVALID_ARG;
  if (E > kMaxExperts || A > INT32_MAX) return VMOE_ERR_UNSUPPORTED;
  if (!tpe || !bins || !padded_bins || !info || !workspace) return VMOE_ERR_INVALID_ARG;
  if (A > 0 && (!sel || !bin_ids || !indices || !assignment_row)) return VMOE_ERR_INVALID_ARG;
  if (row_capacity > 0 && (!row_src || !gather_map)) return VMOE_ERR_INVALID_ARG;
  if (A > 0 && row_weight && !weights) return VMOE_ERR_INVALID_ARG;
  // counted: the S count columns per tile of vmoe_router_topk_hist for the
  // same tokens, experts and k
  const int S = counted ? (A % top_k == 0 ? route_hist_split(A / top_k, E, top_k) : 0) : 1;
  if (S == 0) return VMOE_ERR_UNSUPPORTED;
  if (ws_bytes < route_ws_size(A, E, S)) return VMOE_ERR_WORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);

  const int ntiles = (int)route_ntiles(A);
  RouteWs ws = route_ws(workspace, A, E, S);
  if (ntiles > 0 && !counted) {
    VMOE_LAUNCH(route_hist_kernel, dim3(ntiles), dim3(kRouteThreads),
                       sizeof(int32_t) * E, s, sel, is64, A, E, ntiles, ws.counts, ws.bad);
    VMOE_CHECK_LAUNCH();
  }
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  // (route_hist_split keeps the counted case inside these limits)
  if (E <= kSmallExperts && (int64_t)E * ntiles * S <= kFusedMaxCounts) {
    static_assert(kAuxThreads == kRouteThreads, "the loss workgroup runs in the routing launch");
    const bool with_aux = aux && aux->partial;
    const RouteAux none = {};
    VMOE_LAUNCH(route_small_kernel, dim3(std::max(ntiles, 1) + (with_aux ? 1 : 0)),
                       dim3(kRouteThreads), 0, s, sel, is64, A, E, nbits, ntiles, S, block,
                       rounding, top_k, ws, tpe, bins, padded_bins, bin_ids, indices, row_src,
                       gather_map, gather_map_pad, row_capacity, assignment_row, weights,
                       row_weight, info, expert_offsets, padded_counts, with_aux ? *aux : none);
    VMOE_CHECK_LAUNCH();
    if (with_aux && aux_done) *aux_done = true;
    return VMOE_OK;
  }
  if (E <= kFusedMaxExperts && (int64_t)E * ntiles * S <= kFusedMaxCounts) {
    VMOE_LAUNCH(route_fused_kernel, dim3(std::max(ntiles, 1)), dim3(kRouteThreads),
                       sizeof(int32_t) * (kRouteWaves + 7) * E, s, sel, is64, A, E, nbits,
                       ntiles, S, block, rounding, top_k, ws, tpe, bins, padded_bins, bin_ids,
                       indices, row_src, gather_map, gather_map_pad, row_capacity,
                       assignment_row, weights, row_weight, info, expert_offsets,
                       padded_counts);
    VMOE_CHECK_LAUNCH();
    return VMOE_OK;
  }
  VMOE_LAUNCH(route_scan_kernel, dim3(1), dim3(kScanThreads), sizeof(int32_t) * (4 * E + 1),
                     s, ws, E, ntiles, block, rounding, tpe, bins, padded_bins, row_src,
                     gather_map, gather_map_pad, row_weight, row_capacity, info,
                     expert_offsets, padded_counts);
  VMOE_CHECK_LAUNCH();
  if (ntiles > 0) {
    VMOE_LAUNCH(route_place_kernel, dim3(ntiles), dim3(kRouteThreads),
                       sizeof(int32_t) * (kRouteWaves + 1) * E, s, sel, is64, A, E, nbits,
                       ntiles,
                       top_k, ws, bin_ids, indices, row_src, gather_map, row_capacity,
                       assignment_row, weights, row_weight);
    VMOE_CHECK_LAUNCH();
  }
  return VMOE_OK;
}
}  // namespace

extern "C" int vmoe_route(const void* sel, int32_t is64, int64_t A, int32_t E, int32_t top_k,
                          int32_t block, int32_t rounding, int32_t* bin_ids, int32_t* indices,
                          int32_t* tpe, int32_t* bins, int32_t* padded_bins, int32_t* row_src,
                          int32_t* gather_map, int32_t gather_map_pad, int64_t row_capacity,
                          int32_t* assignment_row, int32_t* info, int32_t* expert_offsets,
                          int32_t* padded_counts, const uint16_t* weights, float* row_weight,
                          void* workspace, size_t ws_bytes, vmoe_stream_t stream) {
  return route_impl(sel, is64, A, E, top_k, block, rounding, bin_ids, indices, tpe, bins,
                    padded_bins, row_src, gather_map, gather_map_pad, row_capacity,
                    assignment_row, info, expert_offsets, padded_counts, weights, row_weight,
                    workspace, ws_bytes, stream, false);
}

extern "C" int vmoe_route_counted(const void* sel, int32_t is64, int64_t A, int32_t E,
                                  int32_t top_k, int32_t block, int32_t rounding,
                                  int32_t* bin_ids, int32_t* indices, int32_t* tpe,
                                  int32_t* bins, int32_t* padded_bins, int32_t* row_src,
                                  int32_t* gather_map, int32_t gather_map_pad,
                                  int64_t row_capacity, int32_t* assignment_row, int32_t* info,
                                  int32_t* expert_offsets, int32_t* padded_counts,
                                  const uint16_t* weights, float* row_weight, void* workspace,
                                  size_t ws_bytes, vmoe_stream_t stream) {
  return route_impl(sel, is64, A, E, top_k, block, rounding, bin_ids, indices, tpe, bins,
                    padded_bins, row_src, gather_map, gather_map_pad, row_capacity,
                    assignment_row, info, expert_offsets, padded_counts, weights, row_weight,
                    workspace, ws_bytes, stream, true);
}

namespace vmoe {
int route_counted_aux(const void* sel, int32_t is64, int64_t A, int32_t E, int32_t top_k,
                      int32_t block, int32_t rounding, int32_t* bin_ids, int32_t* indices,
                      int32_t* tpe, int32_t* bins, int32_t* padded_bins, int32_t* row_src,
                      int32_t* gather_map, int32_t gather_map_pad, int64_t row_capacity,
                      int32_t* assignment_row, int32_t* info, int32_t* expert_offsets,
                      int32_t* padded_counts, const uint16_t* weights, float* row_weight,
                      void* workspace, size_t ws_bytes, vmoe_stream_t stream,
                      const RouteAux* aux, bool* aux_done) {
  if (aux && aux->partial &&
      (aux->nblk <= 0 || aux->T < 0 || !aux->coef || !aux->wn || !aux->f_i || !aux->f_i32 ||
       !aux->p_i || !aux->z || !aux->losses))
    return VMOE_ERR_INVALID_ARG;
  return route_impl(sel, is64, A, E, top_k, block, rounding, bin_ids, indices, tpe, bins,
                    padded_bins, row_src, gather_map, gather_map_pad, row_capacity,
                    assignment_row, info, expert_offsets, padded_counts, weights, row_weight,
                    workspace, ws_bytes, stream, true, aux, aux_done);
}
}  // namespace vmoe

// vmoe_route_static: vmoe_route with its workspace in a file-scope device
// array, for callers that cannot allocate. Each GPU the library runs on holds
// its own copy of `scratch` (kRouteStaticBytes) until the process ends. In
// host code the array's name is only a stand-in for the symbol: its device
// address is looked up once per device, with that device current, by
// hipGetSymbolAddress, and only that address is passed to the kernels.
// vmoe_route rewrites every word of the workspace it reads (the per-tile
// counts and error flags, then the per-expert starts), so nothing has to be
// cleared between calls. Calls that overlap on one GPU share the array and
// race.
constexpr size_t kRouteStaticBytes = 1u << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kRouteStaticBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on first use).
int static_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return VMOE_ERR_LAUNCH;
  if (dev < 0 || dev >= kMaxDevices) return VMOE_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr)
      return VMOE_ERR_LAUNCH;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return VMOE_OK;
}
}  // namespace

extern "C" int vmoe_route_static(const void* sel, int32_t is64, int64_t A, int32_t E,
                                 int32_t top_k, int32_t block, int32_t rounding,
                                 int32_t* bin_ids, int32_t* indices, int32_t* tpe, int32_t* bins,
                                 int32_t* padded_bins, int32_t* row_src, int32_t* gather_map,
                                 int32_t gather_map_pad, int64_t row_capacity,
                                 int32_t* assignment_row, int32_t* info, int32_t* expert_offsets,
                                 int32_t* padded_counts, const uint16_t* weights,
                                 float* row_weight, vmoe_stream_t stream) {
  if (A < 0 || E <= 0) return VMOE_ERR_INVALID_ARG;
  if (vmoe_route_workspace_bytes(A, E) > kRouteStaticBytes) return VMOE_ERR_WORKSPACE;
  void* ws = nullptr;
  const int st = static_scratch(&ws);
  if (st) return st;
  return vmoe_route(sel, is64, A, E, top_k, block, rounding, bin_ids, indices, tpe, bins,
                    padded_bins, row_src, gather_map, gather_map_pad, row_capacity,
                    assignment_row, info, expert_offsets, padded_counts, weights, row_weight, ws,
                    kRouteStaticBytes, stream);
}

extern "C" int vmoe_row_maps(const int32_t* indices, const int32_t* bin_ids,
                             const int32_t* bins, const int32_t* padded_bins, int64_t num_sorted,
                             int32_t E, int32_t top_k, int64_t num_rows, int64_t num_assignments,
                             int32_t* row_src, int32_t* gather_map, int32_t* assignment_row,
                             vmoe_stream_t stream) {
  if (num_sorted < 0 || E <= 0 || top_k <= 0 || num_rows < 0 || num_assignments < 0)
    return VMOE_ERR_INVALID_ARG;
  if (num_sorted > 0 && (!indices || !bin_ids || !bins || !padded_bins))
    return VMOE_ERR_INVALID_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (row_src && num_rows > 0) {
    VMOE_LAUNCH(fill_i32_kernel, dim3(grid_for(num_rows, 256)), dim3(256), 0, s, row_src,
                       num_rows, -1);
    VMOE_CHECK_LAUNCH();
  }
  if (gather_map && num_rows > 0) {
    VMOE_LAUNCH(fill_i32_kernel, dim3(grid_for(num_rows, 256)), dim3(256), 0, s,
                       gather_map, num_rows, 0);
    VMOE_CHECK_LAUNCH();
  }
  if (assignment_row && num_assignments > 0) {
    VMOE_LAUNCH(fill_i32_kernel, dim3(grid_for(num_assignments, 256)), dim3(256), 0, s,
                       assignment_row, num_assignments, -1);
    VMOE_CHECK_LAUNCH();
  }
  if (num_sorted > 0) {
    VMOE_LAUNCH(row_maps_place_kernel, dim3(grid_for(num_sorted, 256)), dim3(256), 0, s,
                       indices, bin_ids, bins, padded_bins, num_sorted, E, top_k, num_rows,
                       num_assignments, row_src, gather_map, assignment_row);
    VMOE_CHECK_LAUNCH();
  }
  return VMOE_OK;
}
