// The module's expert path, one call per direction: TritonMoEMLP.forward's
// routing placement, fused token gather, grouped GEMMs and combine
// (triton_moe/moe.py:186-250 of the reference), and their backward, as a
// sequence of the per-op entry points of this library. A framework binding
// then makes one call per direction instead of one per kernel with its
// buffer bookkeeping in between (the host-side cost that dominates small
// configurations). Host code only: no kernel of its own except a zero fill.
//
// Buffers are the caller's: `saved` holds what the forward leaves for the
// backward (routing arrays, the fp32 row weights, H' and PRE), the two
// scratch buffers what each direction needs only while it runs (the
// routing workspace and Y'; GA, the gathered dX rows and the routing-weight
// row sums). vmoe_expert_layout gives their sizes and the slot offsets;
// every slot starts on a 256-byte boundary.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>

#include "router_aux.h"
#include "vmoe_common.h"

namespace vmoe {
namespace {

constexpr int64_t kAlign = 256;

inline int64_t up256(int64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct Layout {
  int64_t A = 0, cap = 0, nblk = 0;
  int64_t slot[VMOE_X_NSLOTS] = {};
  int64_t saved = 0;
  int64_t f_route_ws = 0, f_y = 0, f_scratch = 0;  // forward scratch
  int64_t b_ga = 0, b_gxg = 0, b_rowdot = 0, b_scratch = 0;  // backward scratch
  size_t route_ws_bytes = 0;
};

bool make_layout(int64_t T, int E, int k, int b, int64_t hidden, int64_t max_w, bool counted,
                 Layout& L) {
  if (T < 0 || E <= 0 || k <= 0 || b <= 0 || hidden <= 0 || max_w <= 0) return false;
  L.A = T * k;
  L.cap = L.A + (int64_t)E * (b - 1);  // rows of a dropless ("up") routing, at most
  L.nblk = (max_w + 63) / 64;
  const int64_t A = L.A, cap = L.cap;
  const int64_t bytes[VMOE_X_NSLOTS] = {
      4 * A, 4 * A, 4 * (int64_t)E, 4 * (int64_t)E, 4 * (int64_t)E,     // bin_ids .. padded_bins
      4 * cap, 4 * cap, 4 * A, 4 * VMOE_INFO_LEN,                       // row_src .. info
      4 * ((int64_t)E + 1), 4 * (int64_t)E, 4 * cap,                   // offsets, counts, weight
      2 * cap * max_w, 2 * cap * max_w};                                // H', PRE
  int64_t off = 0;
  for (int s = 0; s < VMOE_X_NSLOTS; ++s) {
    L.slot[s] = off;
    off += up256(std::max<int64_t>(bytes[s], 4));
  }
  L.saved = off;
  L.route_ws_bytes = counted ? 0 : vmoe_route_workspace_bytes(A, E);
  L.f_route_ws = 0;
  L.f_y = up256((int64_t)L.route_ws_bytes);
  L.f_scratch = L.f_y + up256(2 * cap * hidden);
  L.b_ga = 0;
  L.b_gxg = up256(2 * cap * max_w);
  L.b_rowdot = L.b_gxg + up256(2 * cap * hidden);
  L.b_scratch = L.b_rowdot + up256(4 * cap * L.nblk);
  return true;
}

template <typename T>
T* at(void* base, int64_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(base) + off);
}
template <typename T>
const T* at(const void* base, int64_t off) {
  return reinterpret_cast<const T*>(static_cast<const char*>(base) + off);
}

__global__ void zero_f32_kernel(float* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0.0f;
}

// Events that order the backward's two streams, three per device (one per
// hand-over), created on first use and kept for the process. An event is
// recorded again only after the wait on its previous record was queued, so
// reusing it loses no dependency.
constexpr int kMaxDevices = 64;
std::mutex g_ev_mu;
hipEvent_t g_ev[kMaxDevices][3];
bool g_ev_ok[kMaxDevices];

int events_for(hipEvent_t** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return VMOE_ERR_LAUNCH;
  std::lock_guard<std::mutex> g(g_ev_mu);
  if (!g_ev_ok[dev]) {
    for (int i = 0; i < 3; ++i)
      if (hipEventCreateWithFlags(&g_ev[dev][i], hipEventDisableTiming) != hipSuccess)
        return VMOE_ERR_LAUNCH;
    g_ev_ok[dev] = true;
  }
  *out = g_ev[dev];
  return VMOE_OK;
}

int order(hipStream_t waiter, hipStream_t signaler, hipEvent_t ev) {
  if (hipEventRecord(ev, signaler) != hipSuccess ||
      hipStreamWaitEvent(waiter, ev, 0) != hipSuccess)
    return VMOE_ERR_LAUNCH;
  return VMOE_OK;
}

}  // namespace
}  // namespace vmoe

using namespace vmoe;

#define VMOE_TRY(expr)              \
  do {                              \
    const int st_ = (expr);         \
    if (st_ != VMOE_OK) return st_; \
  } while (0)

extern "C" int vmoe_expert_layout(int64_t num_tokens, int32_t num_experts, int32_t top_k,
                                  int32_t block_size, int64_t hidden, int64_t max_width,
                                  int32_t counted, int64_t* out) {
  Layout L;
  if (!out || !make_layout(num_tokens, num_experts, top_k, block_size, hidden, max_width,
                           counted != 0, L))
    return VMOE_ERR_INVALID_ARG;
  out[0] = L.saved;
  out[1] = L.f_scratch;
  out[2] = L.b_scratch;
  out[3] = L.cap;
  for (int s = 0; s < VMOE_X_NSLOTS; ++s) out[4 + s] = L.slot[s];
  return VMOE_OK;
}

namespace vmoe {
namespace {
// vmoe_expert_forward; `aux` (with a routing workspace of counts): the
// auxiliary losses go into the routing launch where it can take them
// (route_counted_aux sets *aux_done).
int expert_forward(const void* selected, int32_t selected_is_int64, const uint16_t* weights,
                   int64_t num_tokens, int32_t num_experts, int32_t top_k, int32_t block_size,
                   void* route_workspace, size_t route_workspace_bytes, const uint16_t* x,
                   int64_t ldx, const uint16_t* w1, int64_t ldw1, const uint16_t* w2,
                   int64_t ldw2, const int32_t* ewo, const int32_t* widths, int64_t hidden,
                   int64_t max_width, void* saved, void* scratch, uint16_t* out, int64_t ldo,
                   vmoe_stream_t stream, const RouteAux* aux, bool* aux_done) {
  Layout L;
  if (!make_layout(num_tokens, num_experts, top_k, block_size, hidden, max_width,
                   route_workspace != nullptr, L))
    return VMOE_ERR_INVALID_ARG;
  if (num_tokens == 0) return VMOE_OK;
  if (!selected || !weights || !x || !w1 || !w2 || !ewo || !widths || !saved || !scratch ||
      !out || ldo < hidden)
    return VMOE_ERR_INVALID_ARG;
  const int E = num_experts, k = top_k;
  int32_t* row_src = at<int32_t>(saved, L.slot[VMOE_X_ROW_SRC]);
  int32_t* gmap = at<int32_t>(saved, L.slot[VMOE_X_GATHER_MAP]);
  int32_t* arow = at<int32_t>(saved, L.slot[VMOE_X_ASSIGNMENT_ROW]);
  int32_t* eto = at<int32_t>(saved, L.slot[VMOE_X_EXPERT_OFFSETS]);
  int32_t* ptpe = at<int32_t>(saved, L.slot[VMOE_X_PADDED_COUNTS]);
  float* rw = at<float>(saved, L.slot[VMOE_X_ROW_WEIGHT]);
  uint16_t* h = at<uint16_t>(saved, L.slot[VMOE_X_H]);
  uint16_t* pre = at<uint16_t>(saved, L.slot[VMOE_X_PRE]);
  uint16_t* y = at<uint16_t>(scratch, L.f_y);
  // routing placement, pad rows of the map -1 (the GEMMs' gather reads zeros)
  if (route_workspace) {
    VMOE_TRY(route_counted_aux(
        selected, selected_is_int64, L.A, E, k, block_size, VMOE_ROUND_UP,
        at<int32_t>(saved, L.slot[VMOE_X_BIN_IDS]), at<int32_t>(saved, L.slot[VMOE_X_INDICES]),
        at<int32_t>(saved, L.slot[VMOE_X_TPE]), at<int32_t>(saved, L.slot[VMOE_X_BINS]),
        at<int32_t>(saved, L.slot[VMOE_X_PADDED_BINS]), row_src, gmap, -1, L.cap, arow,
        at<int32_t>(saved, L.slot[VMOE_X_INFO]), eto, ptpe, weights, rw, route_workspace,
        route_workspace_bytes, stream, aux, aux_done));
  } else {
    VMOE_TRY(vmoe_route(
        selected, selected_is_int64, L.A, E, k, block_size, VMOE_ROUND_UP,
        at<int32_t>(saved, L.slot[VMOE_X_BIN_IDS]), at<int32_t>(saved, L.slot[VMOE_X_INDICES]),
        at<int32_t>(saved, L.slot[VMOE_X_TPE]), at<int32_t>(saved, L.slot[VMOE_X_BINS]),
        at<int32_t>(saved, L.slot[VMOE_X_PADDED_BINS]), row_src, gmap, -1, L.cap, arow,
        at<int32_t>(saved, L.slot[VMOE_X_INFO]), eto, ptpe, weights, rw,
        at<void>(scratch, L.f_route_ws), L.route_ws_bytes, stream));
  }
  // H' = bf16(w * relu(x[map] W1_e)^2), PRE = relu(z); Y' = H' W2_e; combine
  VMOE_TRY(vmoe_gemm_up_fwd(x, ldx, num_tokens, gmap, w1, ldw1, h, pre, max_width,
                            VMOE_ACT_RELU_SQUARED, rw, eto, ewo, widths, ptpe, E, hidden,
                            max_width, L.cap, stream));
  VMOE_TRY(vmoe_gemm_down_fwd(h, max_width, w2, ldw2, y, hidden, eto, ewo, widths, ptpe, E,
                              hidden, max_width, L.cap, stream));
  return vmoe_combine(y, L.cap, hidden, arow, nullptr, k, out, ldo, num_tokens, hidden, stream);
}
}  // namespace
}  // namespace vmoe

extern "C" int vmoe_expert_forward(const void* selected, int32_t selected_is_int64,
                                   const uint16_t* weights, int64_t num_tokens,
                                   int32_t num_experts, int32_t top_k, int32_t block_size,
                                   void* route_workspace, size_t route_workspace_bytes,
                                   const uint16_t* x, int64_t ldx, const uint16_t* w1,
                                   int64_t ldw1, const uint16_t* w2, int64_t ldw2,
                                   const int32_t* ewo, const int32_t* widths, int64_t hidden,
                                   int64_t max_width, void* saved, void* scratch, uint16_t* out,
                                   int64_t ldo, vmoe_stream_t stream) {
  return expert_forward(selected, selected_is_int64, weights, num_tokens, num_experts, top_k,
                        block_size, route_workspace, route_workspace_bytes, x, ldx, w1, ldw1, w2,
                        ldw2, ewo, widths, hidden, max_width, saved, scratch, out, ldo, stream,
                        nullptr, nullptr);
}

extern "C" int vmoe_expert_backward(
    const void* saved, int64_t num_tokens, int32_t num_experts, int32_t top_k,
    int32_t block_size, const uint16_t* x, int64_t ldx, const uint16_t* w1, int64_t ldw1,
    const uint16_t* w2, int64_t ldw2, const int32_t* ewo, const int32_t* widths, int64_t hidden,
    int64_t max_width, const uint16_t* grad_out, int64_t ldg, const uint16_t* grad_scale,
    uint16_t* grad_x, int64_t ldgx, uint16_t* grad_w1, int64_t ldgw1, uint16_t* grad_w2,
    int64_t ldgw2, uint16_t* grad_weights, void* scratch, void* dw_workspace,
    size_t dw_workspace_bytes, vmoe_stream_t stream, vmoe_stream_t side_stream) {
  Layout L;
  if (!make_layout(num_tokens, num_experts, top_k, block_size, hidden, max_width, true, L))
    return VMOE_ERR_INVALID_ARG;
  if (num_tokens == 0) return VMOE_OK;
  if (!saved || !x || !w1 || !w2 || !ewo || !widths || !grad_out || !grad_x || !grad_w1 ||
      !grad_w2 || !scratch || !dw_workspace || ldg < 0 || ldgx < hidden)
    return VMOE_ERR_INVALID_ARG;
  const int E = num_experts, k = top_k;
  const int32_t* gmap = at<int32_t>(saved, L.slot[VMOE_X_GATHER_MAP]);
  const int32_t* arow = at<int32_t>(saved, L.slot[VMOE_X_ASSIGNMENT_ROW]);
  const int32_t* eto = at<int32_t>(saved, L.slot[VMOE_X_EXPERT_OFFSETS]);
  const int32_t* ptpe = at<int32_t>(saved, L.slot[VMOE_X_PADDED_COUNTS]);
  const float* rw = at<float>(saved, L.slot[VMOE_X_ROW_WEIGHT]);
  const uint16_t* h = at<uint16_t>(saved, L.slot[VMOE_X_H]);
  const uint16_t* pre = at<uint16_t>(saved, L.slot[VMOE_X_PRE]);
  uint16_t* ga = at<uint16_t>(scratch, L.b_ga);
  uint16_t* gxg = at<uint16_t>(scratch, L.b_gxg);
  float* row_dot = grad_weights ? at<float>(scratch, L.b_rowdot) : nullptr;
  hipStream_t main_s = reinterpret_cast<hipStream_t>(stream);
  hipStream_t side_s = side_stream ? reinterpret_cast<hipStream_t>(side_stream) : main_s;
  const bool two = side_s != main_s;
  hipEvent_t* ev = nullptr;
  if (two) VMOE_TRY(events_for(&ev));
  if (row_dot) {
    // blocks at or past an expert's width are not written by the dH GEMM
    const int64_t n = L.cap * L.nblk;
    VMOE_LAUNCH(zero_f32_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 4096)),
                       dim3(256), 0, main_s, row_dot, n);
    VMOE_CHECK_LAUNCH();
  }
  // dW2 (needs only G and H') runs on the side stream beside dH; dW1 beside
  // dX and the combine once GA exists. With one stream the two GEMMs of each
  // pair share one launch, on half of the CUs each (gemm_pair_begin).
  if (two) VMOE_TRY(order(side_s, main_s, ev[0]));
  if (!two) gemm_pair_begin();
  int st = vmoe_gemm_down_bwd_dh(grad_out, ldg, num_tokens, gmap, grad_scale, w2, ldw2, pre, rw,
                                 ga, max_width, eto, ewo, widths, ptpe, E, hidden, max_width,
                                 L.cap, row_dot, L.nblk, stream);
  if (st == VMOE_OK)
    st = vmoe_gemm_down_bwd_dw(h, max_width, grad_out, ldg, num_tokens, gmap, grad_scale, grad_w2,
                               ldgw2, eto, ewo, widths, ptpe, E, hidden, max_width, L.cap,
                               dw_workspace, dw_workspace_bytes,
                               reinterpret_cast<vmoe_stream_t>(side_s));
  if (!two) {
    const int st2 = gemm_pair_end();
    if (st == VMOE_OK) st = st2;
  }
  VMOE_TRY(st);
  if (two) VMOE_TRY(order(side_s, main_s, ev[1]));
  if (!two) gemm_pair_begin();
  st = vmoe_gemm_up_bwd_dw(x, ldx, num_tokens, gmap, ga, max_width, grad_w1, ldgw1, eto, ewo,
                           widths, ptpe, E, hidden, max_width, L.cap, dw_workspace,
                           dw_workspace_bytes, reinterpret_cast<vmoe_stream_t>(side_s));
  if (st == VMOE_OK)
    st = vmoe_gemm_up_bwd_dx(ga, max_width, w1, ldw1, gxg, hidden, eto, ewo, widths, ptpe, E,
                             hidden, max_width, L.cap, stream);
  if (!two) {
    const int st2 = gemm_pair_end();
    if (st == VMOE_OK) st = st2;
  }
  VMOE_TRY(st);
  VMOE_TRY(vmoe_combine(gxg, L.cap, hidden, arow, nullptr, k, grad_x, ldgx, num_tokens, hidden,
                        stream));
  if (two) VMOE_TRY(order(main_s, side_s, ev[2]));
  if (grad_weights) {
    VMOE_TRY(vmoe_routing_weight_grad(row_dot, L.nblk, (int32_t)L.nblk, L.cap, rw, arow, L.A,
                                      grad_weights, stream));
    VMOE_TRY(vmoe_routing_weight_grad_direct(grad_out, ldg, num_tokens, grad_scale, w2, ldw2,
                                             pre, max_width, rw, arow, L.A, k, eto, ewo, widths,
                                             E, hidden, L.cap, grad_weights, stream));
  }
  return VMOE_OK;
}

// ---------------------------------------------------------------------------
// The whole layer after the router Linear: top-k (with the routing counts
// where vmoe_router_topk_hist applies), the expert path above and the
// auxiliary losses; backward: the expert path's, the auxiliary losses'
// logit gradient and, opt-in, the routing weights' chain into the logits.
// saved = [expert saved block][selected int32 A][weights bf16 A][lse fp32 T]
// [f_i fp32 E]; forward scratch = [expert forward scratch][partial rows]
// [counted routing workspace][p_i fp32 E]; backward scratch = [expert
// backward scratch][routing-weight gradient bf16 A][logit gradient bf16 T E].
// ---------------------------------------------------------------------------

namespace vmoe {
namespace {

struct MoeLayout {
  Layout x;
  bool counted = false;
  int64_t partial_rows = 0;
  int64_t slot[VMOE_M_NSLOTS] = {};
  int64_t saved = 0;
  int64_t f_partial = 0, f_route_ws = 0, f_p_i = 0, f_scratch = 0;
  size_t route_ws_bytes = 0;
  int64_t b_gw = 0, b_gl = 0, b_scratch = 0;
};

bool make_moe_layout(int64_t T, int E, int k, int b, int64_t hidden, int64_t max_w,
                     MoeLayout& M) {
  const int hist = (T > 0 && E <= 2048) ? vmoe_router_topk_hist_blocks(T, E, k) : 0;
  M.counted = hist > 0;
  if (!make_layout(T, E, k, b, hidden, max_w, M.counted, M.x)) return false;
  if (E > 2048 || k > kWave) return false;
  M.partial_rows = M.counted ? hist
                             : (int64_t)(vmoe_router_partial_floats(std::max<int64_t>(T, 1), E) /
                                         (size_t)(E + 1));
  const int64_t A = M.x.A;
  const int64_t bytes[VMOE_M_NSLOTS] = {4 * A, 2 * A, 4 * T, 4 * (int64_t)E};
  int64_t off = M.x.saved;
  for (int s = 0; s < VMOE_M_NSLOTS; ++s) {
    M.slot[s] = off;
    off += up256(std::max<int64_t>(bytes[s], 4));
  }
  M.saved = off;
  M.route_ws_bytes = M.counted ? vmoe_route_counted_workspace_bytes(T, E, k) : 0;
  M.f_partial = M.x.f_scratch;
  M.f_route_ws = M.f_partial + up256(4 * M.partial_rows * ((int64_t)E + 1));
  M.f_p_i = M.f_route_ws + up256((int64_t)M.route_ws_bytes);
  M.f_scratch = M.f_p_i + up256(4 * (int64_t)E);
  M.b_gw = M.x.b_scratch;
  M.b_gl = M.b_gw + up256(2 * A);
  M.b_scratch = M.b_gl + up256(2 * T * (int64_t)E);
  return true;
}

// a[i] = bf16(a[i] + b[i]) (fp32 sum, one rounding): two bf16 gradients of
// one tensor added as autograd's accumulation adds them.
__global__ void add_bf16_kernel(uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    a[i] = (uint16_t)f32_to_bf16(bf16_to_f32(a[i]) + bf16_to_f32(b[i]));
}

}  // namespace
}  // namespace vmoe

extern "C" int vmoe_moe_layout(int64_t num_tokens, int32_t num_experts, int32_t top_k,
                               int32_t block_size, int64_t hidden, int64_t max_width,
                               int64_t* out) {
  MoeLayout M;
  if (!out || !make_moe_layout(num_tokens, num_experts, top_k, block_size, hidden, max_width,
                               M))
    return VMOE_ERR_INVALID_ARG;
  out[0] = M.saved;
  out[1] = M.f_scratch;
  out[2] = M.b_scratch;
  out[3] = M.x.cap;
  for (int s = 0; s < VMOE_X_NSLOTS; ++s) out[4 + s] = M.x.slot[s];
  for (int s = 0; s < VMOE_M_NSLOTS; ++s) out[4 + VMOE_X_NSLOTS + s] = M.slot[s];
  out[4 + VMOE_X_NSLOTS + VMOE_M_NSLOTS] = M.counted;
  return VMOE_OK;
}

extern "C" int vmoe_moe_forward(const uint16_t* logits, int64_t num_tokens, int32_t num_experts,
                                int32_t top_k, int32_t normalize, int32_t block_size,
                                const uint16_t* x, int64_t ldx, const uint16_t* w1, int64_t ldw1,
                                const uint16_t* w2, int64_t ldw2, const int32_t* ewo,
                                const int32_t* widths, int64_t hidden, int64_t max_width,
                                const float* coef, const float* widths_normalized, void* saved,
                                void* scratch, uint16_t* out, int64_t ldo, uint16_t* z_loss,
                                float* losses, uint16_t* f_i, vmoe_stream_t stream) {
  MoeLayout M;
  if (!make_moe_layout(num_tokens, num_experts, top_k, block_size, hidden, max_width, M))
    return VMOE_ERR_INVALID_ARG;
  if (num_tokens == 0) return VMOE_OK;
  if (!logits || !saved || !scratch || !coef || !widths_normalized || !z_loss || !losses || !f_i)
    return VMOE_ERR_INVALID_ARG;
  const int E = num_experts;
  int32_t* sel = at<int32_t>(saved, M.slot[VMOE_M_SELECTED]);
  uint16_t* wts = at<uint16_t>(saved, M.slot[VMOE_M_WEIGHTS]);
  float* lse = at<float>(saved, M.slot[VMOE_M_LSE]);
  float* partial = at<float>(scratch, M.f_partial);
  const size_t nfl = (size_t)M.partial_rows * (size_t)(E + 1);
  void* route_ws = nullptr;
  if (M.counted) {
    route_ws = at<void>(scratch, M.f_route_ws);
    VMOE_TRY(vmoe_router_topk_hist(logits, E, num_tokens, E, top_k, normalize, wts, sel, nullptr,
                                   nullptr, lse, partial, nfl, nullptr, route_ws,
                                   M.route_ws_bytes, stream));
  } else {
    VMOE_TRY(vmoe_router_topk(logits, E, num_tokens, E, top_k, normalize, wts, sel, nullptr,
                              nullptr, lse, partial, nfl, nullptr, stream));
  }
  // The losses ride in the routing launch where it takes them (E <= 64),
  // else they get their own launch after the expert path.
  const RouteAux aux = {partial, (int)M.partial_rows, num_tokens, coef, widths_normalized,
                        f_i, at<float>(saved, M.slot[VMOE_M_F_I32]),
                        at<float>(scratch, M.f_p_i), z_loss, losses};
  bool aux_done = false;
  VMOE_TRY(expert_forward(sel, 0, wts, num_tokens, E, top_k, block_size, route_ws,
                          M.route_ws_bytes, x, ldx, w1, ldw1, w2, ldw2, ewo, widths, hidden,
                          max_width, saved, scratch, out, ldo, stream,
                          M.counted ? &aux : nullptr, &aux_done));
  if (aux_done) return VMOE_OK;
  return vmoe_router_aux(partial, (int32_t)M.partial_rows, num_tokens, E,
                         at<int32_t>(saved, M.x.slot[VMOE_X_TPE]), coef, widths_normalized, f_i,
                         at<float>(saved, M.slot[VMOE_M_F_I32]), at<float>(scratch, M.f_p_i),
                         z_loss, losses, stream);
}

extern "C" int vmoe_moe_backward(
    const void* saved, const uint16_t* logits, int64_t num_tokens, int32_t num_experts,
    int32_t top_k, int32_t normalize, int32_t block_size, const uint16_t* x, int64_t ldx,
    const uint16_t* w1, int64_t ldw1, const uint16_t* w2, int64_t ldw2, const int32_t* ewo,
    const int32_t* widths, int64_t hidden, int64_t max_width, const float* coef,
    const float* widths_normalized, const uint16_t* grad_out, int64_t ldg,
    const uint16_t* grad_scale, const float* grad_z, const float* grad_lb, const float* grad_cl,
    int32_t weight_grad, uint16_t* grad_x, int64_t ldgx, uint16_t* grad_w1, int64_t ldgw1,
    uint16_t* grad_w2, int64_t ldgw2, uint16_t* grad_logits, void* scratch, void* dw_workspace,
    size_t dw_workspace_bytes, vmoe_stream_t stream, vmoe_stream_t side_stream) {
  MoeLayout M;
  if (!make_moe_layout(num_tokens, num_experts, top_k, block_size, hidden, max_width, M))
    return VMOE_ERR_INVALID_ARG;
  if (num_tokens == 0) return VMOE_OK;
  if (!saved || !scratch) return VMOE_ERR_INVALID_ARG;
  const int E = num_experts;
  const int64_t T = num_tokens;
  uint16_t* gw = weight_grad && grad_out && grad_logits ? at<uint16_t>(scratch, M.b_gw) : nullptr;
  if (grad_out) {
    VMOE_TRY(vmoe_expert_backward(saved, T, E, top_k, block_size, x, ldx, w1, ldw1, w2, ldw2, ewo,
                                  widths, hidden, max_width, grad_out, ldg, grad_scale, grad_x,
                                  ldgx, grad_w1, ldgw1, grad_w2, ldgw2, gw, scratch, dw_workspace,
                                  dw_workspace_bytes, stream, side_stream));
  }
  if (!grad_logits) return VMOE_OK;
  const bool aux = grad_z || grad_lb || grad_cl;
  if (!aux && !gw) return VMOE_ERR_INVALID_ARG;  // the caller returns no logit gradient then
  if (!logits || !coef || !widths_normalized) return VMOE_ERR_INVALID_ARG;
  const float* lse = at<float>(saved, M.slot[VMOE_M_LSE]);
  const float* f_i32 = at<float>(saved, M.slot[VMOE_M_F_I32]);
  if (aux)
    VMOE_TRY(vmoe_router_aux_bwd(logits, E, T, E, lse, f_i32, coef, widths_normalized, grad_z,
                                 grad_lb, grad_cl, grad_logits, E, stream));
  if (gw) {
    uint16_t* dst = aux ? at<uint16_t>(scratch, M.b_gl) : grad_logits;
    VMOE_TRY(vmoe_router_weight_bwd(logits, E, T, E, top_k, normalize,
                                    at<int32_t>(saved, M.slot[VMOE_M_SELECTED]), nullptr, gw,
                                    top_k, dst, E, stream));
    if (aux) {
      const int64_t n = T * E;
      VMOE_LAUNCH(add_bf16_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 4096)),
                         dim3(256), 0, reinterpret_cast<hipStream_t>(stream), grad_logits, dst, n);
      VMOE_CHECK_LAUNCH();
    }
  }
  return VMOE_OK;
}
