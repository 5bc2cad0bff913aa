/*
 * route_oracle.c -- CPU restatement of the reference's routing, used ONLY as
 * test infrastructure (the checker of the HIP path, and nothing the product
 * ships or calls). Plain scalar C, one pass per step, no cleverness.
 *
 * Restates:
 *   fused_route            triton_moe/kernels/fused_cumsum.py:85-171
 *     - stable sort of ids (torch.sort(stable=True), :130)   -> counting sort
 *     - histogram (torch.bincount, :134)
 *     - rounding up/down/nearest (:61-66), kept = min (:71)
 *     - bins / padded_bins inclusive cumsums (:76-77)
 *     - keep mask for down/nearest (:154-169)
 *   precompute_gather_map  triton_moe/kernels/grouped_gemm.py:104-149
 *   padded row of a sorted position, as used by _padded_gather_kernel
 *     (triton_moe/kernels/gather.py:34-60) and _padded_scatter_kernel
 *     (triton_moe/kernels/scatter.py:35-69)
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static int32_t round_count(int32_t c, int32_t b, int32_t mode) {
  if (mode == 0) return ((c + b - 1) / b) * b; /* up (fused_cumsum.py:62) */
  if (mode == 1) return (c / b) * b;           /* down (:64) */
  return ((c + b / 2) / b) * b;                /* nearest (:66) */
}

/* Returns 0 on success, 1 on an id outside [0, E), 2 on bad arguments,
 * 3 on allocation failure. n_kept receives the length of bin_ids/indices. */
int oracle_route(const int64_t* sel, int64_t A, int32_t E, int32_t block, int32_t rounding,
                 int32_t* bin_ids, int32_t* indices, int32_t* tpe, int32_t* bins,
                 int32_t* padded_bins, int64_t* n_kept) {
  if (A < 0 || E <= 0 || block <= 0 || rounding < 0 || rounding > 2) return 2;
  for (int64_t p = 0; p < A; ++p)
    if (sel[p] < 0 || sel[p] >= E) return 1;

  int64_t* start = (int64_t*)calloc((size_t)E + 1, sizeof(int64_t));
  int64_t* cursor = (int64_t*)calloc((size_t)E, sizeof(int64_t));
  int32_t* s_ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)(A > 0 ? A : 1));
  int32_t* s_idx = (int32_t*)malloc(sizeof(int32_t) * (size_t)(A > 0 ? A : 1));
  if (!start || !cursor || !s_ids || !s_idx) {
    free(start); free(cursor); free(s_ids); free(s_idx);
    return 3;
  }
  /* histogram */
  memset(tpe, 0, sizeof(int32_t) * (size_t)E);
  for (int64_t p = 0; p < A; ++p) tpe[sel[p]] += 1;
  /* stable counting sort: expert-major, original order inside an expert */
  for (int32_t e = 0; e < E; ++e) start[e + 1] = start[e] + tpe[e];
  for (int64_t p = 0; p < A; ++p) {
    const int64_t e = sel[p];
    const int64_t pos = start[e] + cursor[e]++;
    s_ids[pos] = (int32_t)e;
    s_idx[pos] = (int32_t)p;
  }
  /* rounding, kept, cumsums, and the keep mask */
  int64_t kb = 0, rb = 0, out = 0;
  for (int32_t e = 0; e < E; ++e) {
    const int32_t c = tpe[e];
    const int32_t r = round_count(c, block, rounding);
    const int32_t k = c < r ? c : r;
    kb += k;
    rb += r;
    bins[e] = (int32_t)kb;
    padded_bins[e] = (int32_t)rb;
    for (int32_t q = 0; q < k; ++q) {
      bin_ids[out] = s_ids[start[e] + q];
      indices[out] = s_idx[start[e] + q];
      ++out;
    }
  }
  *n_kept = out;
  free(start); free(cursor); free(s_ids); free(s_idx);
  return 0;
}

/* precompute_gather_map (grouped_gemm.py:124-149): zeros, then for every
 * sorted position i of expert e = bin_ids[i]:
 *   gm[padded_start[e] + i - bin_start[e]] = indices[i] / top_k.
 * Also the two maps the HIP path uses: row_src[row] = indices[i] (-1 where no
 * position lands) and assignment_row[indices[i]] = row (-1 where unplaced).
 * Any output may be NULL. Rows outside [0, P) are skipped. */
void oracle_row_maps(const int32_t* indices, const int32_t* bin_ids, const int32_t* bins,
                     const int32_t* padded_bins, int64_t n_sorted, int32_t E, int32_t top_k,
                     int64_t P, int64_t A, int32_t* gather_map, int32_t* row_src,
                     int32_t* assignment_row) {
  for (int64_t r = 0; r < P; ++r) {
    if (gather_map) gather_map[r] = 0;
    if (row_src) row_src[r] = -1;
  }
  if (assignment_row)
    for (int64_t a = 0; a < A; ++a) assignment_row[a] = -1;
  for (int64_t i = 0; i < n_sorted; ++i) {
    const int32_t e = bin_ids[i];
    if (e < 0 || e >= E) continue;
    const int64_t bin_start = e > 0 ? bins[e - 1] : 0;
    const int64_t padded_start = e > 0 ? padded_bins[e - 1] : 0;
    const int64_t row = padded_start + (i - bin_start);
    if (row < 0 || row >= P) continue;
    if (gather_map) gather_map[row] = indices[i] / top_k;
    if (row_src) row_src[row] = indices[i];
    if (assignment_row && indices[i] >= 0 && indices[i] < A) assignment_row[indices[i]] = (int32_t)row;
  }
}
