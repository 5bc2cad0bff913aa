/*
 * vmoe.h -- C ABI of the MI355X (gfx950) variable-width MoE MLP hot path.
 *
 * Every entry point is asynchronous on the given HIP stream: nothing here
 * synchronises, allocates device memory or reads device memory from the host.
 * Buffers are raw device pointers; bf16 tensors are passed as uint16_t*
 * (bit patterns), metadata as int32_t*. Leading dimensions are in elements.
 * Return value: VMOE_OK (0) or a vmoe_status code; vmoe_status_string()
 * turns it into text. A launch failure is reported as VMOE_ERR_LAUNCH.
 *
 * Reference interface each entry point replaces is cited as
 * <reference file>:<line>, relative to hbfreed/triton-variable-moe.
 */
#ifndef VMOE_H
#define VMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* vmoe_stream_t; /* == hipStream_t */

enum vmoe_status {
  VMOE_OK = 0,
  VMOE_ERR_INVALID_ARG = 1, /* null pointer, negative size, bad enum */
  VMOE_ERR_UNSUPPORTED = 2, /* size/alignment outside what the kernels take */
  VMOE_ERR_LAUNCH = 3,      /* hipLaunchKernel / hipGetLastError failure */
  VMOE_ERR_WORKSPACE = 4    /* workspace smaller than *_workspace_bytes() */
};

/* Rounding modes of fused_route (triton_moe/kernels/fused_cumsum.py:126-128). */
enum vmoe_rounding { VMOE_ROUND_UP = 0, VMOE_ROUND_DOWN = 1, VMOE_ROUND_NEAREST = 2 };

/* Activations of grouped_gemm_up (triton_moe/kernels/grouped_gemm.py:435).
 * VMOE_ACT_SWIGLU is taken by the fp32 GEMMs only; the bf16 SwiGLU forward is
 * vmoe_gemm_up_glu. */
enum vmoe_activation { VMOE_ACT_NONE = 0, VMOE_ACT_RELU_SQUARED = 1, VMOE_ACT_SWIGLU = 2 };

/* Bits of info[VMOE_INFO_ERRORS] written by vmoe_route. */
enum vmoe_route_error { VMOE_ROUTE_BAD_EXPERT_ID = 1, VMOE_ROUTE_ROW_OVERFLOW = 2 };
enum vmoe_info_slot { VMOE_INFO_ROWS = 0, VMOE_INFO_KEPT = 1, VMOE_INFO_ERRORS = 2, VMOE_INFO_LEN = 4 };

const char* vmoe_status_string(int status);
int vmoe_version(void);
/* Measurement hook (no counterpart in the reference; for benchmarks that time
 * each entry point): while stop_event is non-NULL, every kernel the calling
 * host thread launches carries the two hipEvent_t handles on its own dispatch
 * (hipExtLaunchKernelGGL): the first launch records start_event at its start,
 * each launch records stop_event at its end, so the pair spans the kernels of
 * the next entry point without the gaps of separate event records. Pass NULL,
 * NULL to switch it off. VMOE_ERR_INVALID_ARG for a start without a stop. */
int vmoe_set_launch_timing(void* start_event, void* stop_event);
/* Largest num_experts vmoe_route accepts. */
int vmoe_route_max_experts(void);

/* ------------------------------------------------------------------------
 * Routing.
 * Replaces fused_route (triton_moe/kernels/fused_cumsum.py:85-171: torch.sort
 * stable + torch.bincount + _cumsum_kernel + the rounding keep-mask) and, in
 * the same pass, precompute_gather_map (triton_moe/kernels/grouped_gemm.py:104-149).
 *
 *   selected_experts  [A] int32 or int64 (selected_is_int64), flat t*k+j order
 *   bin_ids, indices  [A] int32: expert-sorted (stable) ids and positions;
 *                     the first info[VMOE_INFO_KEPT] entries are valid
 *   tokens_per_expert, bins, padded_bins  [E] int32
 *   row_src     [row_capacity] int32: padded row -> assignment index, -1 = pad
 *   gather_map  [row_capacity] int32: padded row -> token (assignment / top_k); pad rows
 *               hold gather_map_pad (0 in the reference's precompute_gather_map; -1
 *               makes the GEMMs' row gather read zeros for them)
 *   assignment_row [A] int32: assignment -> padded row, -1 = dropped
 *   info        [VMOE_INFO_LEN] int32: rows P, kept count, error bits
 *   expert_offsets [E+1] int32 (nullable): [0, padded_bins], the module's
 *               expert_token_offsets (triton_moe/moe.py:193-197)
 *   padded_counts  [E] int32 (nullable): rounded counts, diff(padded_bins),
 *               the module's padded tokens_per_expert (moe.py:198-202)
 *   weights     [A] bf16 (nullable): routing weights in the order of
 *               selected_experts; with row_weight [row_capacity] fp32 (nullable)
 *               row_weight[row] = weights[row_src[row]], 0 for pad rows: the
 *               per-row factor the module's up GEMM and dH GEMM apply
 * Only the first P = padded_bins[E-1] rows of row_src/gather_map are written;
 * row_capacity >= A + E*(block_size-1) always suffices.
 * ---------------------------------------------------------------------- */
size_t vmoe_route_workspace_bytes(int64_t num_assignments, int32_t num_experts);
int vmoe_route(const void* selected_experts, int32_t selected_is_int64,
               int64_t num_assignments, int32_t num_experts, int32_t top_k,
               int32_t block_size, int32_t rounding, int32_t* bin_ids, int32_t* indices,
               int32_t* tokens_per_expert, int32_t* bins, int32_t* padded_bins,
               int32_t* row_src, int32_t* gather_map, int32_t gather_map_pad,
               int64_t row_capacity, int32_t* assignment_row, int32_t* info,
               int32_t* expert_offsets, int32_t* padded_counts, const uint16_t* weights,
               float* row_weight, void* workspace, size_t workspace_bytes,
               vmoe_stream_t stream);

/* vmoe_route for selections whose per-block histograms vmoe_router_topk_hist
 * already wrote into `workspace` (vmoe_route_counted_workspace_bytes(
 * num_assignments / top_k, num_experts, top_k) bytes; same tokens, experts,
 * k and the selected ids that call wrote): the counting launch is skipped,
 * everything else, outputs and status codes included, is vmoe_route's
 * (VMOE_ERR_UNSUPPORTED where vmoe_router_topk_hist does not apply): after
 * the top-k kernel, routing is one launch instead of two. Same replacement
 * as vmoe_route (fused_cumsum.py:85-171 with grouped_gemm.py:104-149); the
 * reference counts inside torch.bincount. */
int vmoe_route_counted(const void* selected_experts, int32_t selected_is_int64,
                       int64_t num_assignments, int32_t num_experts, int32_t top_k,
                       int32_t block_size, int32_t rounding, int32_t* bin_ids, int32_t* indices,
                       int32_t* tokens_per_expert, int32_t* bins, int32_t* padded_bins,
                       int32_t* row_src, int32_t* gather_map, int32_t gather_map_pad,
                       int64_t row_capacity, int32_t* assignment_row, int32_t* info,
                       int32_t* expert_offsets, int32_t* padded_counts,
                       const uint16_t* weights, float* row_weight, void* workspace,
                       size_t workspace_bytes, vmoe_stream_t stream);

/* vmoe_route without a workspace argument and without any allocation: the
 * workspace is a file-scope device array of 1 MiB per GPU (each GPU the
 * library runs on holds it until the process ends). No counterpart in the
 * reference; it is for callers that cannot allocate device memory (code
 * under graph capture, serving loops, harnesses that forbid hipMalloc).
 * Arguments, outputs and status codes are those of vmoe_route; a call whose
 * vmoe_route_workspace_bytes(num_assignments, num_experts) exceeds 1 MiB
 * returns VMOE_ERR_WORKSPACE without launching anything (1 MiB holds, e.g.,
 * 262144 assignments over 512 experts). Calls that overlap on one GPU share
 * the array and race: run them in one stream. */
int vmoe_route_static(const void* selected_experts, int32_t selected_is_int64,
                      int64_t num_assignments, int32_t num_experts, int32_t top_k,
                      int32_t block_size, int32_t rounding, int32_t* bin_ids, int32_t* indices,
                      int32_t* tokens_per_expert, int32_t* bins, int32_t* padded_bins,
                      int32_t* row_src, int32_t* gather_map, int32_t gather_map_pad,
                      int64_t row_capacity, int32_t* assignment_row, int32_t* info,
                      int32_t* expert_offsets, int32_t* padded_counts, const uint16_t* weights,
                      float* row_weight, vmoe_stream_t stream);

/* Row maps from caller-supplied routing arrays, for the stand-alone
 * gather/scatter/gather-map entry points. Follows the per-sorted-position
 * placement of _padded_gather_kernel (triton_moe/kernels/gather.py:34-60) and
 * precompute_gather_map (triton_moe/kernels/grouped_gemm.py:124-149): sorted
 * position i of expert e = bin_ids[i] lands on row
 * padded_bins[e-1] + i - bins[e-1]. Rows nobody lands on get row_src = -1,
 * gather_map = 0; assignments nobody places get assignment_row = -1.
 * Any output pointer may be NULL. */
int vmoe_row_maps(const int32_t* indices, const int32_t* bin_ids, const int32_t* bins,
                  const int32_t* padded_bins, int64_t num_sorted, int32_t num_experts,
                  int32_t top_k, int64_t num_rows, int64_t num_assignments,
                  int32_t* row_src, int32_t* gather_map, int32_t* assignment_row,
                  vmoe_stream_t stream);

/* ------------------------------------------------------------------------
 * Router front end (TritonMoEMLP.forward, triton_moe/moe.py:166-182 and the
 * auxiliary losses at moe.py:253-303).
 * vmoe_router_topk: from bf16 router logits L [T, E] (row stride ld_logits)
 *   p = sigmoid(float(L)); top_k of p per token in torch.topk's output order
 *   on ROCm (equal values included); weights[t*k+j] = bf16(v_j / (sum v +
 *   1e-20)) (normalize != 0) or bf16(v_j); selected_i32 / selected_i64 (either
 *   may be NULL, not both) the expert ids; probs (nullable) p as fp32 [T, E];
 *   lse [T] fp32 = bf16-rounded logsumexp_e L[t, e]; partial = per-workgroup
 *   sums for vmoe_router_aux (vmoe_router_partial_floats(T, E) floats; the
 *   row count is returned in *num_partial_rows). Limits: E <= 2048, k <= 64.
 * vmoe_router_aux: after routing, z_loss (bf16), [load_balance, compute] (fp32
 *   in losses[0..1]), f_i = bf16(tpe / sum tpe) (bf16 and fp32 copies; 0 when
 *   nothing was routed) and
 *   p_i = mean_t p [E] fp32. coef[e] is the load-balance weight of expert e:
 *   E for uniform widths, 1 without expert groups, else
 *   group_size / num_groups for experts in a group and 0 otherwise
 *   (moe.py:276-303); widths_normalized is the module's buffer as fp32.
 * vmoe_router_aux_bwd: grad_logits[t, e] = bf16(g_z 2 lse_t softmax(L[t])_e / T
 *   + (g_lb coef_e f_e + g_cl wn_e) / T p (1 - p)); g_* are device fp32
 *   scalars (nullable = 0). The top-k weights get no gradient (scatter.py:176).
 * ---------------------------------------------------------------------- */
/* Router logits: logits[T, E] = bf16(x[T, hidden] @ weight[E, hidden]^T), fp32
 * accumulation (nn.Linear(n_embd, num_experts, bias=False), triton_moe/moe.py:78
 * and its call at moe.py:166). Supports E % 8 == 0, E <= 128, hidden % 256 == 0,
 * 16-byte aligned x / weight rows and 8-byte aligned logits rows; other shapes
 * return VMOE_ERR_UNSUPPORTED (the caller's own linear layer covers them). */
int vmoe_router_logits(const uint16_t* x, int64_t ldx, int64_t num_tokens, int64_t hidden,
                       const uint16_t* weight, int64_t ldw, int32_t num_experts,
                       uint16_t* logits, int64_t ld_logits, vmoe_stream_t stream);

size_t vmoe_router_partial_floats(int64_t num_tokens, int32_t num_experts);
int vmoe_router_topk(const uint16_t* logits, int64_t ld_logits, int64_t num_tokens,
                     int32_t num_experts, int32_t top_k, int32_t normalize, uint16_t* weights,
                     int32_t* selected_i32, int64_t* selected_i64, float* probs, float* lse,
                     float* partial, size_t partial_floats, int32_t* num_partial_rows,
                     vmoe_stream_t stream);
/* vmoe_router_topk that also counts how many of its selections went to each
 * expert in every block of consecutive assignments (1 to 8 blocks per
 * routing tile of 1024 assignments, one top-k workgroup each, so the launch
 * stays near 256 workgroups), into route_workspace
 * (vmoe_route_counted_workspace_bytes(T, E, k) bytes) in the layout
 * vmoe_route_counted reads. weights, selected, probs and lse are
 * vmoe_router_topk's, bit for bit; partial has
 * vmoe_router_topk_hist_blocks(T, E, k) rows of E + 1 floats (returned in
 * *num_partial_rows), so vmoe_router_aux adds the per-token terms in another
 * fixed order. Applies when vmoe_router_topk_hist_blocks > 0 (E % 8 == 0,
 * E <= 128, k <= 8 dividing 1024, T > 0, E * blocks <= 65536),
 * ld_logits % 8 == 0 and logits / probs are 16-byte aligned; otherwise
 * VMOE_ERR_UNSUPPORTED and nothing is launched (use vmoe_router_topk +
 * vmoe_route). Replaces the same reference lines as vmoe_router_topk
 * (moe.py:168-176) and the torch.bincount of fused_route
 * (fused_cumsum.py:134). */
int vmoe_router_topk_hist_blocks(int64_t num_tokens, int32_t num_experts, int32_t top_k);
size_t vmoe_route_counted_workspace_bytes(int64_t num_tokens, int32_t num_experts,
                                          int32_t top_k);
int vmoe_router_topk_hist(const uint16_t* logits, int64_t ld_logits, int64_t num_tokens,
                          int32_t num_experts, int32_t top_k, int32_t normalize,
                          uint16_t* weights, int32_t* selected_i32, int64_t* selected_i64,
                          float* probs, float* lse, float* partial, size_t partial_floats,
                          int32_t* num_partial_rows, void* route_workspace,
                          size_t route_workspace_bytes, vmoe_stream_t stream);
int vmoe_router_aux(const float* partial, int32_t num_partial_rows, int64_t num_tokens,
                    int32_t num_experts, const int32_t* tokens_per_expert, const float* coef,
                    const float* widths_normalized, uint16_t* f_i, float* f_i_f32, float* p_i,
                    uint16_t* z_loss, float* losses, vmoe_stream_t stream);
int vmoe_router_aux_bwd(const uint16_t* logits, int64_t ld_logits, int64_t num_tokens,
                        int32_t num_experts, const float* lse, const float* f_i_f32,
                        const float* coef, const float* widths_normalized, const float* grad_z,
                        const float* grad_lb, const float* grad_cl, uint16_t* grad_logits,
                        int64_t ld_grad, vmoe_stream_t stream);

/* vmoe_router_weight_bwd: opt-in gradient of the routing weights with respect
 * to the logits, which the reference does not compute (its padded_scatter
 * returns None for the weights, triton_moe/kernels/scatter.py:176; the chain
 * is moe.py:168-176). For token t, slot j with expert s_j, p_j =
 * sigmoid(float(L[t, s_j])) and g_j = grad_weights[t * ld_grad_weights + j]
 * (bf16): dp_j = (g_j - sum_i g_i p_i / S) / S with S = sum_j p_j + 1e-20
 * when normalize != 0, else dp_j = g_j; grad_logits[t, s_j] =
 * bf16(dp_j p_j (1 - p_j)) and 0 for every other expert (the whole row is
 * written). selected_i32 / selected_i64 as for vmoe_router_topk. */
int vmoe_router_weight_bwd(const uint16_t* logits, int64_t ld_logits, int64_t num_tokens,
                           int32_t num_experts, int32_t top_k, int32_t normalize,
                           const int32_t* selected_i32, const int64_t* selected_i64,
                           const uint16_t* grad_weights, int64_t ld_grad_weights,
                           uint16_t* grad_logits, int64_t ld_grad, vmoe_stream_t stream);

/* fp32 forms of the router entry points for a float32 module (the
 * reference's TritonMoEMLP runs in whatever dtype its parameters have; a
 * float32 one has float32 logits, weights and logit gradients, moe.py:166-176,
 * 253-257): the same kernels, arguments and limits, with logits, weights,
 * f_i, z_loss, grad_weights and grad_logits as fp32. logsumexp and its square
 * are not rounded (torch evaluates them in fp32 for fp32 logits) and
 * f_i = tpe / sum tpe unrounded (moe.py:257 casts to x.dtype). */
int vmoe_router_topk_f32(const float* logits, int64_t ld_logits, int64_t num_tokens,
                         int32_t num_experts, int32_t top_k, int32_t normalize, float* weights,
                         int32_t* selected_i32, int64_t* selected_i64, float* probs, float* lse,
                         float* partial, size_t partial_floats, int32_t* num_partial_rows,
                         vmoe_stream_t stream);
int vmoe_router_topk_hist_f32(const float* logits, int64_t ld_logits, int64_t num_tokens,
                              int32_t num_experts, int32_t top_k, int32_t normalize,
                              float* weights, int32_t* selected_i32, int64_t* selected_i64,
                              float* probs, float* lse, float* partial, size_t partial_floats,
                              int32_t* num_partial_rows, void* route_workspace,
                              size_t route_workspace_bytes, vmoe_stream_t stream);
int vmoe_router_aux_f32(const float* partial, int32_t num_partial_rows, int64_t num_tokens,
                        int32_t num_experts, const int32_t* tokens_per_expert, const float* coef,
                        const float* widths_normalized, float* f_i, float* f_i_f32, float* p_i,
                        float* z_loss, float* losses, vmoe_stream_t stream);
int vmoe_router_aux_bwd_f32(const float* logits, int64_t ld_logits, int64_t num_tokens,
                            int32_t num_experts, const float* lse, const float* f_i_f32,
                            const float* coef, const float* widths_normalized,
                            const float* grad_z, const float* grad_lb, const float* grad_cl,
                            float* grad_logits, int64_t ld_grad, vmoe_stream_t stream);
int vmoe_router_weight_bwd_f32(const float* logits, int64_t ld_logits, int64_t num_tokens,
                               int32_t num_experts, int32_t top_k, int32_t normalize,
                               const int32_t* selected_i32, const int64_t* selected_i64,
                               const float* grad_weights, int64_t ld_grad_weights,
                               float* grad_logits, int64_t ld_grad, vmoe_stream_t stream);

/* ------------------------------------------------------------------------
 * Token permutation (bf16).
 * vmoe_gather: out[r] = x[row_src[r] / top_k] (times weights[row_src[r]] when
 * weights != NULL, product rounded to bf16), zero where row_src[r] < 0.
 *   - unweighted: padded_gather (triton_moe/kernels/gather.py:63-115)
 *   - weighted:   _weighted_padded_gather, the scatter backward
 *                 (triton_moe/kernels/gather.py:177-218, scatter.py:161-176)
 * num_rows_dev (nullable) caps num_rows with a device-side row count.
 * ---------------------------------------------------------------------- */
int vmoe_gather(const uint16_t* x, int64_t x_rows, int64_t ldx, const int32_t* row_src,
                int32_t top_k, const uint16_t* weights, int64_t num_weights, uint16_t* out,
                int64_t ldo, int64_t num_rows, const int32_t* num_rows_dev, int64_t hidden,
                vmoe_stream_t stream);

/* vmoe_gather_tokens: the same output as vmoe_gather for maps produced
 * together by vmoe_route, computed token by token: for t < num_tokens and
 * j < top_k, out[assignment_row[t*k+j]] = x[t] (times weights[t*k+j] when
 * weights != NULL, rounded to bf16); rows r < num_rows with row_src[r] < 0
 * are zeroed. x is read once per token instead of once per row, and ldx may
 * be 0 (one row broadcast to every token, e.g. the gradient of out.sum()).
 * Replaces the same reference functions as vmoe_gather
 * (triton_moe/kernels/gather.py:63-115, 177-218). Requires hidden, ldx and
 * ldo multiples of 8, 16-byte aligned x and out, and top_k <= 64. */
int vmoe_gather_tokens(const uint16_t* x, int64_t ldx, const int32_t* assignment_row,
                       int64_t num_tokens, int32_t top_k, const uint16_t* weights,
                       const int32_t* row_src, uint16_t* out, int64_t ldo, int64_t num_rows,
                       const int32_t* num_rows_dev, int64_t hidden, vmoe_stream_t stream);

/* vmoe_combine: out[t] = bf16( sum_j f32( bf16( y[assignment_row[t*k+j]] * w[t*k+j] ) ) ),
 * j = 0..top_k-1 in order, slots with assignment_row < 0 contribute 0.
 *   - weighted:   padded_scatter + intermediate.sum(1)
 *                 (triton_moe/kernels/scatter.py:72-133)
 *   - weights == NULL: the gather backward, padded_scatter with all-ones
 *                 weights (triton_moe/kernels/gather.py:245-265) */
int vmoe_combine(const uint16_t* y, int64_t y_rows, int64_t ldy, const int32_t* assignment_row,
                 const uint16_t* weights, int32_t top_k, uint16_t* out, int64_t ldo,
                 int64_t num_tokens, int64_t hidden, vmoe_stream_t stream);

/* vmoe_combine_weight_grad: gradient of vmoe_combine's routing weights,
 *   grad_weights[t*k+j] = sum_c f32(grad[t, c]) * f32(y[assignment_row[t*k+j], c])
 * in fp32, 0 for slots with assignment_row < 0 (the per-slot bf16 rounding is
 * taken as identity). Opt-in: the reference's PaddedScatterOp.backward returns
 * None for the weights (triton_moe/kernels/scatter.py:176); this is the
 * routing-weight gradient its padded_scatter lacks. grad may be a broadcast
 * row (ldg = 0). */
int vmoe_combine_weight_grad(const uint16_t* grad, int64_t ldg, const uint16_t* y, int64_t y_rows,
                             int64_t ldy, const int32_t* assignment_row, int32_t top_k,
                             float* grad_weights, int64_t num_tokens, int64_t hidden,
                             vmoe_stream_t stream);

/* vmoe_routing_weight_grad: the routing-weight gradient of the module path
 * (opt-in; the reference has none, scatter.py:176), which scales H by the
 * weight in the up GEMM (H' = bf16(w * relu(z)^2)), so that
 * dL/dw = sum_c dL/dH'[c] relu(z)[c]^2:
 *   grad_weights[a] = bf16( sum_{b < num_blocks} row_dot[row][b] / row_weight[row] ),
 *   row = assignment_row[a], with row_dot from vmoe_gemm_down_bwd_dh; 0 when
 *   row < 0, row >= rows or |row_weight[row]| < 2^-64 (zero and bf16
 *   denormals: the division loses those, vmoe_routing_weight_grad_direct
 *   fills them). */
int vmoe_routing_weight_grad(const float* row_dot, int64_t ld_row_dot, int32_t num_blocks,
                             int64_t rows, const float* row_weight,
                             const int32_t* assignment_row, int64_t num_assignments,
                             uint16_t* grad_weights, vmoe_stream_t stream);

/* vmoe_routing_weight_grad_direct: the entries of the same gradient whose
 * row weight is below 2^-64 in magnitude, from the definition
 *   grad_weights[a] = bf16( sum_{c < w_e} (grad_y[a / top_k] . w2[ewo[e] + c])
 *                           * pre_act[row][c]^2 ),
 * row = assignment_row[a], e the expert with eto[e] <= row < eto[e+1], the
 * dots in fp32 (grad_y rows past gy_rows count as zero; ldgy = 0 reads one
 * row for all), times the bf16 scalar *grad_scale when it is not NULL (as
 * vmoe_gemm_down_bwd_dh's). Other entries are left as they are, so it runs after
 * vmoe_routing_weight_grad; with no tiny weight it reads assignment_row and
 * row_weight once. pre_act [rows, ld_pre >= max width] as for
 * vmoe_gemm_down_bwd_dh; eto/ewo/widths as for the GEMMs below. */
int vmoe_routing_weight_grad_direct(const uint16_t* grad_y, int64_t ldgy, int64_t gy_rows,
                                    const uint16_t* grad_scale, const uint16_t* w2, int64_t ldw2, const uint16_t* pre_act,
                                    int64_t ld_pre, const float* row_weight,
                                    const int32_t* assignment_row, int64_t num_assignments,
                                    int32_t top_k, const int32_t* eto, const int32_t* ewo,
                                    const int32_t* widths, int32_t num_experts, int64_t hidden,
                                    int64_t rows, uint16_t* grad_weights, vmoe_stream_t stream);

/* ------------------------------------------------------------------------
 * Token permutation in fp32, for a float32 module (the reference's gather and
 * scatter kernels are dtype-generic; gather.py:63-115, 177-218,
 * scatter.py:61-69, 133, 141-189): arguments as in the bf16 forms, all rows
 * fp32, every product and sum in fp32 (slots summed in ascending j).
 * vmoe_combine_f32: out[t] = sum_j y[row(t, j)] * weights[t*k+j] (weights
 *   NULL: 1), the reference's padded_scatter in fp32.
 * vmoe_gather_f32: out[r] = x[row_src[r] / top_k] * weights[row_src[r]]
 *   (weights NULL: 1), zeros where row_src[r] < 0; ldx = 0 reads one row
 *   for every token (a broadcast output gradient).
 * vmoe_combine_weight_grad_f32: grad_weights[t*k+j] = sum_c grad[t, c] *
 *   y[row(t, j), c], 0 for slots with no row (opt-in; the reference returns
 *   None, scatter.py:176).
 * 4-float vectors where row starts are 16-byte aligned, single floats
 * otherwise; no alignment rule.
 * ---------------------------------------------------------------------- */
int vmoe_combine_f32(const float* y, int64_t y_rows, int64_t ldy, const int32_t* assignment_row,
                     const float* weights, int32_t top_k, float* out, int64_t ldo,
                     int64_t num_tokens, int64_t hidden, vmoe_stream_t stream);
int vmoe_gather_f32(const float* x, int64_t x_rows, int64_t ldx, const int32_t* row_src,
                    int32_t top_k, const float* weights, int64_t num_weights, float* out,
                    int64_t ldo, int64_t num_rows, const int32_t* num_rows_dev, int64_t hidden,
                    vmoe_stream_t stream);
int vmoe_combine_weight_grad_f32(const float* grad, int64_t ldg, const float* y, int64_t y_rows,
                                 int64_t ldy, const int32_t* assignment_row, int32_t top_k,
                                 float* grad_weights, int64_t num_tokens, int64_t hidden,
                                 vmoe_stream_t stream);

/* ------------------------------------------------------------------------
 * Variable-width grouped GEMMs (bf16 in, fp32 MFMA accumulate, bf16 out).
 * Per-expert metadata as in the reference kernels:
 *   eto    [E+1] expert_token_offsets (row ranges in the padded layout)
 *   ewo    [E+1] expert_weight_offsets (column/row offset of expert e in W1/W2)
 *   widths [E]   expert_widths
 *   tpe    [E]   tokens_per_expert (rows tiled per expert; the module passes
 *                the padded counts)
 * rows_bound: upper bound of sum(tpe) and of eto[E]; sizes the grid and
 * bounds every row index (outputs have at least rows_bound rows).
 * Tiles are found on the device from the metadata, so no host sync is needed.
 * hidden, every width and ewo entry, and all leading dimensions must be
 * multiples of 8 and buffers 16-byte aligned (VMOE_ERR_UNSUPPORTED otherwise).
 * ---------------------------------------------------------------------- */

/* out = act(x_e @ W1[:, ewo[e]:ewo[e]+w_e]); pre_act = relu(z) (nullable).
 * Rows of x_e are x[gather_map[row]] when gather_map != NULL (the reference's
 * USE_GATHER_MAP path; x then has x_rows rows, ldx = 0 reads one row for all;
 * map entries outside [0, x_rows), such as -1 for pad rows, read zeros), else
 * x[row]. row_scale [rows_bound] fp32 (nullable): out[row] =
 * bf16(row_scale[row] * act(z)) (pre_act is not scaled); the module passes
 * each row's routing weight (vmoe_route's row_weight), which moves the
 * weight of the combine onto H.
 * Replaces grouped_gemm_up / _grouped_gemm_up_kernel
 * (triton_moe/kernels/grouped_gemm.py:212-368, 379-477). */
int vmoe_gemm_up_fwd(const uint16_t* x, int64_t ldx, int64_t x_rows, const int32_t* gather_map,
                     const uint16_t* w1, int64_t ldw1,
                     uint16_t* out, uint16_t* pre_act, int64_t ldo, int32_t activation,
                     const float* row_scale, const int32_t* eto, const int32_t* ewo,
                     const int32_t* widths, const int32_t* tpe, int32_t num_experts,
                     int64_t hidden, int64_t max_width, int64_t rows_bound,
                     vmoe_stream_t stream);

/* y = h_e[:, :w_e] @ W2[ewo[e]:ewo[e+1], :].
 * Replaces grouped_gemm_down / _grouped_gemm_down_kernel
 * (triton_moe/kernels/grouped_gemm.py:480-651). */
int vmoe_gemm_down_fwd(const uint16_t* h, int64_t ldh, const uint16_t* w2, int64_t ldw2,
                       uint16_t* y, int64_t ldy, const int32_t* eto, const int32_t* ewo,
                       const int32_t* widths, const int32_t* tpe, int32_t num_experts,
                       int64_t hidden, int64_t max_width, int64_t rows_bound,
                       vmoe_stream_t stream);

/* GA = bf16(pre_act > 0 ? 2 * grad_h * pre_act : 0) elementwise over
 * [rows, cols]: the relu^2 derivative of the reference's backward kernels
 * (triton_moe/kernels/grouped_gemm.py:751-766, 914-928), for callers holding
 * grad_h and pre_act separately. cols, ld, ldo multiples of 8. */
int vmoe_relu2_grad(const uint16_t* grad_h, const uint16_t* pre_act, int64_t ld,
                    uint16_t* grad_act, int64_t ldo, int64_t rows, int64_t cols,
                    vmoe_stream_t stream);

/* SwiGLU up projection (activation="swiglu"; the reference's
 * _grouped_gemm_up_kernel with ACTIVATION == 2, triton_moe/kernels/
 * grouped_gemm.py:293-349): expert e's gate columns are W1[:, ewo_e + c] and
 * its up columns W1[:, ewo_e + w_e + c], c < w_e (ewo need not be contiguous
 * in steps of 2 w_e; widths <= max_width, multiples of 8). One GEMM stages
 * both halves of 128 output columns per tile and, from the fp32
 * accumulators g and u,
 *   out  = bf16(row_scale * (g * sigmoid(g)) * u)   (row_scale nullable: 1)
 *   gate = bf16(g), up = bf16(u)
 * each output nullable (not all three), [rows, max_width] with row stride
 * ldo; rows, gather_map and the other arguments as vmoe_gemm_up_fwd. The
 * reference saves the gate as pre_act. */
int vmoe_gemm_up_glu(const uint16_t* x, int64_t ldx, int64_t x_rows, const int32_t* gather_map,
                     const uint16_t* w1, int64_t ldw1, uint16_t* out, uint16_t* gate,
                     uint16_t* up, int64_t ldo, const float* row_scale, const int32_t* eto,
                     const int32_t* ewo, const int32_t* widths, const int32_t* tpe,
                     int32_t num_experts, int64_t hidden, int64_t max_width,
                     int64_t rows_bound, vmoe_stream_t stream);

/* SwiGLU backward (the reference's is an unfinished placeholder,
 * grouped_gemm.py:768-790; this is the derivative of the forward above):
 * for each row r of expert e (eto[e] <= r < eto[e+1], r < rows) and c < w_e,
 *   grad_gu[r, c]       = dG = bf16(gh * u * s * (1 + g * (1 - s)))
 *   grad_gu[r, w_e + c] = dU = bf16(gh * g * s),   s = sigmoid(g)
 * from grad_h (gh), gate (g) and up (u) at [r, c]; rows past the expert's
 * min(tpe[e], eto[e+1] - eto[e]) get zeros. grad_gu [rows, >= 2 max_width]
 * is then the gradient of the expert's 2 w_e contiguous W1 columns: one
 * vmoe_gemm_up_bwd_dx and one vmoe_gemm_up_bwd_dw with widths 2 w_e give
 * grad_x and grad_w1. Strides and max_width multiples of 8. */
int vmoe_glu_grad(const uint16_t* grad_h, int64_t ldgh, const uint16_t* gate,
                  const uint16_t* up, int64_t ld, uint16_t* grad_gu, int64_t ldo,
                  const int32_t* eto, const int32_t* widths, const int32_t* tpe,
                  int32_t num_experts, int64_t rows, int64_t max_width, vmoe_stream_t stream);

/* grad_x = GA_e @ W1_e^T, GA = gradient w.r.t. the pre-activation (the output
 * of vmoe_relu2_grad, or grad_h itself for activation "none").
 * Replaces _grouped_gemm_up_backward_dx_kernel
 * (triton_moe/kernels/grouped_gemm.py:654-802, launched at 1214-1250). */
int vmoe_gemm_up_bwd_dx(const uint16_t* grad_act, int64_t ldg, const uint16_t* w1,
                        int64_t ldw1, uint16_t* grad_x, int64_t ldgx, const int32_t* eto,
                        const int32_t* ewo, const int32_t* widths, const int32_t* tpe,
                        int32_t num_experts, int64_t hidden, int64_t max_width,
                        int64_t rows_bound, vmoe_stream_t stream);

/* Workspace of the two dW GEMMs' split-K on the current device: arrival
 * words, then fp32 partial tiles. The arrival words (the first
 * vmoe_gemm_dw_workspace_zero_bytes() bytes) must be zero when a call starts,
 * and every call leaves them zero: zero-fill them once when the workspace is
 * allocated and reuse it for calls in stream order; calls that may overlap
 * need workspaces of their own. The partial tiles need no initial value. A
 * dW call with workspace == NULL runs without split-K (same result to
 * summation order, one work item per output tile, slow when one expert holds
 * most tokens). */
size_t vmoe_gemm_dw_workspace_bytes(int32_t num_experts, int64_t hidden, int64_t max_width,
                                    int64_t rows_bound);
/* Bytes at the start of a dW workspace that must be zero when a call starts
 * (the arrival words; a multiple of 256, at most 8 KiB). No counterpart in
 * the reference, whose Triton dW kernels need no workspace. */
size_t vmoe_gemm_dw_workspace_zero_bytes(void);

/* grad_w1[:, ewo[e]:+w_e] = X_e^T @ GA_e, X_e rows read as x[gather_map[row]]
 * when gather_map != NULL (fused gather), else x[row]. K (the expert's rows) is
 * split into chunks summed in a fixed order, so results are deterministic.
 * Replaces _grouped_gemm_up_backward_dw_kernel
 * (triton_moe/kernels/grouped_gemm.py:805-967, launched at 1252-1290). */
int vmoe_gemm_up_bwd_dw(const uint16_t* x, int64_t ldx, int64_t x_rows,
                        const int32_t* gather_map, const uint16_t* grad_act, int64_t ldg,
                        uint16_t* grad_w1, int64_t ldgw, const int32_t* eto,
                        const int32_t* ewo, const int32_t* widths, const int32_t* tpe,
                        int32_t num_experts, int64_t hidden, int64_t max_width,
                        int64_t rows_bound, void* workspace, size_t workspace_bytes,
                        vmoe_stream_t stream);

/* grad_h = grad_y @ W2_e^T (columns >= w_e untouched). With pre_act != NULL
 * (same leading dimension as grad_h) the output is instead the relu^2
 * gradient GA = bf16(pre_act > 0 ? 2 * bf16(grad_h) * pre_act : 0), computed in
 * the epilogue, which is what the up-projection backward consumes.
 * gather_map (nullable): rows of grad_y are grad_y[gather_map[row]] (grad_y
 * has gy_rows rows; ldgy = 0 reads one row for all; entries outside
 * [0, gy_rows) read zeros), e.g. the token gradient of the combine, read
 * without materialising its per-row copy. row_scale (nullable, fp32
 * [rows_bound]): grad_h[row] = bf16(row_scale[row] * (grad_y @ W2_e^T)[row])
 * before the relu^2 rule. grad_scale (nullable, one bf16 on the device): the
 * output is scaled by it, so a broadcast gradient c * ones (out.sum(),
 * out.mean()) is passed as a row of ones (ldgy = 0) and grad_scale = &c.
 * row_dot (nullable; needs pre_act; fp32 [rows_bound, ld_row_dot] with
 * ld_row_dot >= ceil(max_width / 64)): row_dot[row][b] = sum over the
 * columns c of 64-column block b of GH[row][c] * pre_act[row][c]^2, GH the
 * bf16 (scaled) gradient before the relu^2 rule; blocks at or past an
 * expert's width are not written. It is the module's routing-weight
 * gradient before division by the weight (vmoe_routing_weight_grad).
 * Replaces _grouped_gemm_down_backward_dintermediate_kernel
 * (triton_moe/kernels/grouped_gemm.py:970-1063, launched at 1336-1362). */
int vmoe_gemm_down_bwd_dh(const uint16_t* grad_y, int64_t ldgy, int64_t gy_rows,
                          const int32_t* gather_map, const uint16_t* grad_scale,
                          const uint16_t* w2, int64_t ldw2,
                          const uint16_t* pre_act, const float* row_scale, uint16_t* grad_h,
                          int64_t ldgh, const int32_t* eto, const int32_t* ewo,
                          const int32_t* widths, const int32_t* tpe, int32_t num_experts,
                          int64_t hidden, int64_t max_width, int64_t rows_bound,
                          float* row_dot, int64_t ld_row_dot, vmoe_stream_t stream);

/* grad_w2[ewo[e]:+w_e, :] = H_e^T @ grad_y_e; rows of grad_y_e are
 * grad_y[gather_map[row]] when gather_map != NULL (gy_rows, ldgy = 0 and
 * out-of-range entries as for vmoe_gemm_down_bwd_dh), else grad_y[row];
 * grad_scale as for vmoe_gemm_down_bwd_dh.
 * Replaces _grouped_gemm_down_backward_dw_kernel
 * (triton_moe/kernels/grouped_gemm.py:1066-1162, launched at 1364-1390). */
int vmoe_gemm_down_bwd_dw(const uint16_t* h, int64_t ldh, const uint16_t* grad_y,
                          int64_t ldgy, int64_t gy_rows, const int32_t* gather_map,
                          const uint16_t* grad_scale, uint16_t* grad_w2, int64_t ldgw, const int32_t* eto,
                          const int32_t* ewo, const int32_t* widths, const int32_t* tpe,
                          int32_t num_experts, int64_t hidden, int64_t max_width,
                          int64_t rows_bound, void* workspace, size_t workspace_bytes,
                          vmoe_stream_t stream);

/* Zero columns [widths[e], max_width) of every row of expert e in a padded
 * [rows, max_width] buffer: the zero-initialised tails the reference's
 * torch.zeros outputs carry (triton_moe/kernels/grouped_gemm.py:422,426,1328). */
int vmoe_zero_tail_cols(uint16_t* buf, int64_t ld, const int32_t* eto, const int32_t* widths,
                        int32_t num_experts, int64_t max_width, int64_t rows_bound,
                        vmoe_stream_t stream);

/* ------------------------------------------------------------------------
 * fp32 grouped GEMMs: the float32 inputs of grouped_gemm_up / _down and their
 * backward and autograd functions (the reference's kernels are dtype-generic:
 * triton_moe/kernels/grouped_gemm.py:217-1162; its fp32 autograd tests:
 * tests/test_grouped_gemm_backward.py:151-208). fp32 in, fp32 fma
 * accumulation in k order, fp32 out. Metadata, rows_bound and the rows each
 * expert covers are as for the bf16 GEMMs above; no alignment or multiple-of-8
 * requirement. Only the rows and columns the experts cover are written: the
 * caller zero-fills the rest (as the reference's torch.zeros outputs are).
 * activation: VMOE_ACT_NONE, VMOE_ACT_RELU_SQUARED or VMOE_ACT_SWIGLU, whose
 * gate columns of expert e are ewo[e] + [0, w_e) and its up columns
 * ewo[e] + w_e + [0, w_e) (grouped_gemm.py:295-297).
 * ---------------------------------------------------------------------- */

/* out = act(x_e @ W1_e) [rows, ldo >= max_width] (grouped_gemm.py:217-368).
 * relu^2: pre_act = relu(z) (optional), out = pre_act^2. SwiGLU: pre_act =
 * the gate g, up = u, out = g * sigmoid(g) * u (each optional, out or one of
 * the others required). x rows through gather_map when it is non-null (a map
 * entry outside [0, x_rows) reads zeros). */
int vmoe_gemm_f32_up_fwd(const float* x, int64_t ldx, int64_t x_rows, const int32_t* gather_map,
                         const float* w1, int64_t ldw1, float* out, float* pre_act, float* up,
                         int64_t ldo, int32_t activation, const int32_t* eto,
                         const int32_t* ewo, const int32_t* widths, const int32_t* tpe,
                         int32_t num_experts, int64_t hidden, int64_t max_width,
                         int64_t rows_bound, vmoe_stream_t stream);

/* y = h_e @ W2_e [rows, hidden] (grouped_gemm.py:485-584). */
int vmoe_gemm_f32_down_fwd(const float* h, int64_t ldh, const float* w2, int64_t ldw2, float* y,
                           int64_t ldy, const int32_t* eto, const int32_t* ewo,
                           const int32_t* widths, const int32_t* tpe, int32_t num_experts,
                           int64_t hidden, int64_t max_width, int64_t rows_bound,
                           vmoe_stream_t stream);

/* grad_x [rows, hidden] = GA_e @ W1_e^T (grouped_gemm.py:659-807), GA the
 * gradient w.r.t. the pre-activation formed from grad_h (the gradient of the
 * activated output) as it is loaded: relu^2 GA = pre > 0 ? grad_h * 2 * pre :
 * 0 (pre_act = relu(z)); SwiGLU [dG | dU] over the expert's 2 w_e columns
 * from the gate (pre_act) and up; none GA = grad_h. grad_h, pre_act and up
 * share the leading dimension ldg >= max_width. */
int vmoe_gemm_f32_up_bwd_dx(const float* grad_h, const float* pre_act, const float* up,
                            int64_t ldg, int32_t activation, const float* w1, int64_t ldw1,
                            float* grad_x, int64_t ldgx, const int32_t* eto, const int32_t* ewo,
                            const int32_t* widths, const int32_t* tpe, int32_t num_experts,
                            int64_t hidden, int64_t max_width, int64_t rows_bound,
                            vmoe_stream_t stream);

/* grad_act = pre_act > 0 ? grad_h * 2 * pre_act : 0, elementwise over
 * [rows, cols] in fp32 (the relu^2 rule of grouped_gemm.py:751-764): GA formed
 * once for the fp32 dX and dW GEMMs, which then take it with
 * VMOE_ACT_NONE. grad_h and pre_act share ld. */
int vmoe_f32_relu2_grad(const float* grad_h, const float* pre_act, int64_t ld, float* grad_act,
                        int64_t ldo, int64_t rows, int64_t cols, vmoe_stream_t stream);

/* grad_w1 = X_e^T @ GA_e into W1's layout (grouped_gemm.py:810-972), GA as
 * for vmoe_gemm_f32_up_bwd_dx, X through gather_map when it is non-null. */
int vmoe_gemm_f32_up_bwd_dw(const float* x, int64_t ldx, int64_t x_rows,
                            const int32_t* gather_map, const float* grad_h, const float* pre_act,
                            const float* up, int64_t ldg, int32_t activation, float* grad_w1,
                            int64_t ldgw, const int32_t* eto, const int32_t* ewo,
                            const int32_t* widths, const int32_t* tpe, int32_t num_experts,
                            int64_t hidden, int64_t max_width, int64_t rows_bound,
                            vmoe_stream_t stream);

/* grad_h [rows, max_width] = grad_y_e @ W2_e^T (grouped_gemm.py:975-1068). */
int vmoe_gemm_f32_down_bwd_dh(const float* grad_y, int64_t ldgy, const float* w2, int64_t ldw2,
                              float* grad_h, int64_t ldgh, const int32_t* eto,
                              const int32_t* ewo, const int32_t* widths, const int32_t* tpe,
                              int32_t num_experts, int64_t hidden, int64_t max_width,
                              int64_t rows_bound, vmoe_stream_t stream);

/* grad_w2 = H_e^T @ grad_y_e into W2's layout (grouped_gemm.py:1071-1162). */
int vmoe_gemm_f32_down_bwd_dw(const float* h, int64_t ldh, const float* grad_y, int64_t ldgy,
                              float* grad_w2, int64_t ldgw, const int32_t* eto,
                              const int32_t* ewo, const int32_t* widths, const int32_t* tpe,
                              int32_t num_experts, int64_t hidden, int64_t max_width,
                              int64_t rows_bound, vmoe_stream_t stream);

/* ------------------------------------------------------------------------
 * The module's expert path, one call per direction: the routing placement,
 * the up GEMM reading x through the row map (H' = bf16(w relu(z)^2), PRE =
 * relu(z)), the down GEMM and the unweighted combine of TritonMoEMLP.forward
 * (triton_moe/moe.py:186-250: fused_route's placement, padded_gather,
 * grouped_gemm_up, grouped_gemm_down, padded_scatter), and their backward,
 * as sequences of the entry points above. No counterpart in the reference
 * (its module makes these calls one by one from Python); for bindings whose
 * per-call cost matters (small batches).
 *
 * Buffers are the caller's: `saved` (kept from the forward to the backward),
 * one scratch buffer per direction (used only during the call), sized by
 * vmoe_expert_layout: out[0] saved bytes, out[1] forward scratch bytes,
 * out[2] backward scratch bytes, out[3] the padded-row bound rows_bound =
 * T k + E (block_size - 1), out[4 + s] the byte offset in `saved` of slot s
 * below (each 256-byte aligned; the routing arrays are vmoe_route's, with
 * gather_map_pad -1, row_weight from the weights, dropless rounding; H and
 * PRE bf16 [rows_bound, max_width]). counted != 0: the forward will get the
 * routing workspace of vmoe_router_topk_hist (its scratch then holds no
 * routing workspace). Rows past the routed count are left unwritten.
 * ---------------------------------------------------------------------- */
enum vmoe_expert_slot {
  VMOE_X_BIN_IDS = 0, VMOE_X_INDICES, VMOE_X_TPE, VMOE_X_BINS, VMOE_X_PADDED_BINS,
  VMOE_X_ROW_SRC, VMOE_X_GATHER_MAP, VMOE_X_ASSIGNMENT_ROW, VMOE_X_INFO,
  VMOE_X_EXPERT_OFFSETS, VMOE_X_PADDED_COUNTS, VMOE_X_ROW_WEIGHT, VMOE_X_H, VMOE_X_PRE,
  VMOE_X_NSLOTS
};
int vmoe_expert_layout(int64_t num_tokens, int32_t num_experts, int32_t top_k,
                       int32_t block_size, int64_t hidden, int64_t max_width, int32_t counted,
                       int64_t* out /* [4 + VMOE_X_NSLOTS] */);
/* out[t] = bf16(sum_j Y'[row(t, j)]), Y' = H' W2_e, H' = bf16(w relu(x[t] W1_e)^2)
 * for the routing of selected / weights (bf16 [T k]); route_workspace: the
 * counted routing workspace (vmoe_route_counted) or NULL (vmoe_route, its
 * workspace in the scratch). ewo / widths [E(+1)] device int32 as for the
 * GEMMs; the GEMMs' alignment rules apply. */
int vmoe_expert_forward(const void* selected, int32_t selected_is_int64, const uint16_t* weights,
                        int64_t num_tokens, int32_t num_experts, int32_t top_k,
                        int32_t block_size, void* route_workspace, size_t route_workspace_bytes,
                        const uint16_t* x, int64_t ldx, const uint16_t* w1, int64_t ldw1,
                        const uint16_t* w2, int64_t ldw2, const int32_t* ewo,
                        const int32_t* widths, int64_t hidden, int64_t max_width, void* saved,
                        void* scratch, uint16_t* out, int64_t ldo, vmoe_stream_t stream);
/* Gradients of vmoe_expert_forward for the output gradient grad_out [T, hidden]
 * (ldg = 0 reads one row for every token; grad_scale nullable, as for
 * vmoe_gemm_down_bwd_dh): grad_x [T, hidden], grad_w1 / grad_w2 (every column /
 * row an expert covers), and with grad_weights != NULL the routing weights'
 * (vmoe_routing_weight_grad, then its direct form). dW2 and dW1 run on
 * side_stream when it is not NULL (ordered by events; the call returns with
 * `stream` waiting for it), with dw_workspace (vmoe_gemm_dw_workspace_bytes
 * at E, hidden, max_width, rows_bound) used by both in turn. */
int vmoe_expert_backward(const void* saved, int64_t num_tokens, int32_t num_experts,
                         int32_t top_k, int32_t block_size, const uint16_t* x, int64_t ldx,
                         const uint16_t* w1, int64_t ldw1, const uint16_t* w2, int64_t ldw2,
                         const int32_t* ewo, const int32_t* widths, int64_t hidden,
                         int64_t max_width, const uint16_t* grad_out, int64_t ldg,
                         const uint16_t* grad_scale, uint16_t* grad_x, int64_t ldgx,
                         uint16_t* grad_w1, int64_t ldgw1, uint16_t* grad_w2, int64_t ldgw2,
                         uint16_t* grad_weights, void* scratch, void* dw_workspace,
                         size_t dw_workspace_bytes, vmoe_stream_t stream,
                         vmoe_stream_t side_stream);

/* ------------------------------------------------------------------------
 * The whole layer after the router Linear, one call per direction: from
 * bf16 router logits [T, E] (contiguous, 16-byte aligned) the top-k
 * (vmoe_router_topk_hist where it applies, else vmoe_router_topk + the
 * routing's own count), the expert path of vmoe_expert_forward, and the
 * auxiliary losses (vmoe_router_aux): TritonMoEMLP.forward after
 * self.router (triton_moe/moe.py:167-303). No counterpart in the reference
 * (for bindings whose per-call cost matters). vmoe_moe_layout: out[0..3] as
 * vmoe_expert_layout's, out[4 + s] the expert slots, out[4 + VMOE_X_NSLOTS + s]
 * the slots below (selected int32 [T k], weights bf16 [T k], lse fp32 [T],
 * f_i fp32 [E]), out[4 + VMOE_X_NSLOTS + VMOE_M_NSLOTS] 1 when the counted
 * top-k applies. Outputs: out [T, hidden], z_loss (bf16 scalar),
 * losses[0..1] (load balance, compute; fp32), f_i bf16 [E].
 * vmoe_moe_backward: grad_out nullable (then no x / w1 / w2 gradients);
 * grad_logits [T, E] bf16 nullable, else the auxiliary losses' logit
 * gradient for the device fp32 scalars grad_z / grad_lb / grad_cl
 * (nullable = 0; not all NULL unless weight_grad), plus with weight_grad the
 * routing weights' chain (vmoe_routing_weight_grad, its direct form and
 * vmoe_router_weight_bwd), the two added as bf16(a + b).
 * ---------------------------------------------------------------------- */
enum vmoe_moe_slot { VMOE_M_SELECTED = 0, VMOE_M_WEIGHTS, VMOE_M_LSE, VMOE_M_F_I32, VMOE_M_NSLOTS };
int vmoe_moe_layout(int64_t num_tokens, int32_t num_experts, int32_t top_k, int32_t block_size,
                    int64_t hidden, int64_t max_width,
                    int64_t* out /* [5 + VMOE_X_NSLOTS + VMOE_M_NSLOTS] */);
int vmoe_moe_forward(const uint16_t* logits, int64_t num_tokens, int32_t num_experts,
                     int32_t top_k, int32_t normalize, int32_t block_size, const uint16_t* x,
                     int64_t ldx, const uint16_t* w1, int64_t ldw1, const uint16_t* w2,
                     int64_t ldw2, const int32_t* ewo, const int32_t* widths, int64_t hidden,
                     int64_t max_width, const float* coef, const float* widths_normalized,
                     void* saved, void* scratch, uint16_t* out, int64_t ldo, uint16_t* z_loss,
                     float* losses, uint16_t* f_i, vmoe_stream_t stream);
int vmoe_moe_backward(const void* saved, const uint16_t* logits, int64_t num_tokens,
                      int32_t num_experts, int32_t top_k, int32_t normalize, int32_t block_size,
                      const uint16_t* x, int64_t ldx, const uint16_t* w1, int64_t ldw1,
                      const uint16_t* w2, int64_t ldw2, const int32_t* ewo,
                      const int32_t* widths, int64_t hidden, int64_t max_width,
                      const float* coef, const float* widths_normalized,
                      const uint16_t* grad_out, int64_t ldg, const uint16_t* grad_scale,
                      const float* grad_z, const float* grad_lb, const float* grad_cl,
                      int32_t weight_grad, uint16_t* grad_x, int64_t ldgx, uint16_t* grad_w1,
                      int64_t ldgw1, uint16_t* grad_w2, int64_t ldgw2, uint16_t* grad_logits,
                      void* scratch, void* dw_workspace, size_t dw_workspace_bytes,
                      vmoe_stream_t stream, vmoe_stream_t side_stream);

#ifdef __cplusplus
}
#endif

#endif /* VMOE_H */
