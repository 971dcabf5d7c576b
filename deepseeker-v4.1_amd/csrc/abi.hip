// C ABI of libdsk_moe: host-side validation, workspace layout and launch
// sequencing.  No entry point allocates device memory or synchronises; every
// check happens on the host before the first launch, so a failed call leaves
// the stream untouched.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "dsk_internal.h"
#include "resnorm.h"

namespace dsk {

static thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return DSK_OK;
  return fail(DSK_EHIP, "%s: %s", what, hipGetErrorString(e));
}

thread_local StageClock g_stage_clock;

void stage_close() { g_stage_clock.open = -1; }

hipError_t stage_open(int stage) {
  StageClock& c = g_stage_clock;
  if (!c.ev) return hipSuccess;
  c.open = stage;
  c.launched = false;
  return hipSuccess;
}

namespace {
// Arms the stage clock for one timed forward (this thread) and disarms it on exit.
struct StageTiming {
  explicit StageTiming(const hipEvent_t* ev) {
    g_stage_clock = StageClock{};
    g_stage_clock.ev = ev;
  }
  ~StageTiming() { g_stage_clock = StageClock{}; }
};
}  // namespace

static size_t align_up(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

Workspace workspace_layout(const dsk_moe_desc& d) {
  Workspace L{};
  const size_t T = static_cast<size_t>(d.tokens), H = d.hidden, E = d.n_experts, k = d.top_k;
  const size_t I = d.inter, Is = d.inter_shared, N = T * k;
  size_t o = 0;
  auto take = [&](size_t bytes) { size_t at = o; o = align_up(o + bytes); return at; };
  // Arrival counters first, at a fixed offset for every shape, so one
  // zero-filled workspace can serve calls of different shapes.
  L.ctr = take(kCounterBytes);
  L.scores = take(T * E * 4);
  L.idx = take(N * 4);
  L.wts = take(N * 4);
  L.counts = take(E * 4);
  L.offsets = take((E + 1) * 4);
  L.perm = take(N * 4);
  L.rank = take(N * 4);
  L.active = take((E + 1) * 4);
  L.desc = take(E * sizeof(SlotDesc));
  L.rowmap = take(static_cast<size_t>(64) * T * 4);
  L.xrow = take(N * 4);
  L.wrow = take(N * 4);
  const size_t xplane = (d.x_dtype == DSK_DTYPE_F32) ? T * H * 2 : 0;
  L.xb_hi = take(xplane);
  L.xb_lo = take(xplane);
  L.h_hi = take(N * I * 2);
  L.h_lo = take(N * I * 2);
  L.hs_hi = take(T * Is * 2);
  L.hs_lo = take(T * Is * 2);
  const bool mx = mx_decode(d);
  L.hq = take(mx ? N * 3 * T * I : 0);
  L.hqs = take(mx ? N * 3 * T * (I / 32) : 0);
  L.y = take(N * H * 4);
  L.ys = take(T * H * 4);
  L.shared_x = take(mx && Is > 0 ? T * H * 2 : 0);
  // the grouped FP4 gate/up's x planes: every batch the grouped path may take (below the
  // prefill GEMM), bf16 x
  if (prefill_mx(d)) {
    L.xp = take(T * (2 * H + H / 32));
    L.hp = take(N * (2 * I + I / 32));
  } else {
    // q3: x scaled for the factored gate/up [T][H] bf16, then its 64-group sums [T][H/64][2] f32
    const bool bf16x = d.x_dtype == DSK_DTYPE_BF16 && !prefill_gemm(d);
    L.xp = take(bf16x && d.quant == DSK_QUANT_FP4 ? T * 2 * (H + H / 32)
                : bf16x && grouped_x_q3(d)     ? T * (2 * H + H / 8)
                                               : 0);
    L.hp = take(!prefill_gemm(d) && grouped_h_planes(d) ? N * 3 * (I + I / 32) : 0);
  }
  L.pf_tiles = take(prefill_gemm(d) ? (3 + 2 * static_cast<size_t>(prefill_max_tiles(d))) * 4 : 0);
  L.disp_hist = take(dispatch_hist_ints(static_cast<int>(N), static_cast<int>(E)) * 4);
  L.total = o;
  return L;
}

}  // namespace dsk

using namespace dsk;

static int check_desc(const dsk_moe_desc* d) {
  if (!d) return fail(DSK_EINVAL, "desc is NULL");
  if (d->tokens < 1) return fail(DSK_EINVAL, "tokens=%d must be >= 1", d->tokens);
  if (d->n_experts < 1 || d->n_experts > 1024)
    return fail(DSK_EINVAL, "n_experts=%d must be in [1, 1024]", d->n_experts);
  if (d->top_k < 1 || d->top_k > 16 || d->top_k > d->n_experts)
    return fail(DSK_EINVAL, "top_k=%d must be in [1, min(16, n_experts)]", d->top_k);
  if (d->score_func != DSK_SCORE_SIGMOID && d->score_func != DSK_SCORE_SQRTSOFTPLUS)
    return fail(DSK_EINVAL, "unknown score_func %d", d->score_func);
  if (d->x_dtype != DSK_DTYPE_BF16 && d->x_dtype != DSK_DTYPE_F32)
    return fail(DSK_EINVAL, "x_dtype %d must be BF16 or F32", d->x_dtype);
  if (d->gate_dtype != DSK_DTYPE_BF16 && d->gate_dtype != DSK_DTYPE_F32)
    return fail(DSK_EINVAL, "gate_dtype %d must be BF16 or F32", d->gate_dtype);
  if (d->hidden < 32 || d->hidden % 32)
    return fail(DSK_EINVAL, "hidden=%d must be a positive multiple of 32", d->hidden);
  if (static_cast<int64_t>(d->tokens) * d->top_k > (1 << 24))
    return fail(DSK_EINVAL, "tokens*top_k=%lld exceeds 2^24",
                static_cast<long long>(d->tokens) * d->top_k);
  return DSK_OK;
}

static int check_expert_desc(const dsk_moe_desc* d) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (d->quant == DSK_QUANT_FP4) {
    if (d->inter < 32 || d->inter % 32)
      return fail(DSK_EINVAL, "inter=%d must be a positive multiple of 32 for FP4", d->inter);
  } else if (d->quant == DSK_QUANT_Q3) {
    if (d->inter < 128 || d->inter % 128 || d->hidden % 128)
      return fail(DSK_EINVAL, "Q3 needs hidden=%d and inter=%d to be multiples of 128", d->hidden, d->inter);
  } else {
    return fail(DSK_EINVAL, "unknown quant %d", d->quant);
  }
  if (d->inter_shared < 0 || d->inter_shared % 32)
    return fail(DSK_EINVAL, "inter_shared=%d must be 0 or a positive multiple of 32", d->inter_shared);
  if (!(d->limit > 0.0f)) return fail(DSK_EINVAL, "limit must be > 0");
  return DSK_OK;
}

static bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

extern "C" {

int dsk_abi_version(void) { return DSK_ABI_VERSION; }

const char* dsk_last_error(void) { return g_err; }

int dsk_workspace_size(const dsk_moe_desc* d, size_t* bytes) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (!bytes) return fail(DSK_EINVAL, "bytes is NULL");
  *bytes = workspace_layout(*d).total;
  return DSK_OK;
}

int dsk_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
  if (!workspace) return fail(DSK_EINVAL, "dsk_workspace_init: workspace is NULL");
  if (!aligned(workspace, 256)) return fail(DSK_EALIGN, "dsk_workspace_init: workspace must be 256-byte aligned");
  return hip_check(launch_zero_fill(workspace, workspace_bytes, static_cast<hipStream_t>(stream)),
                   "dsk_workspace_init launch");
}

int dsk_route(const dsk_moe_desc* d, const void* x, const void* gate_w, const float* gate_b,
              float* scores, int32_t* idx, float* weights, void* stream) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (!x || !gate_w || !gate_b || !scores || !idx || !weights)
    return fail(DSK_EINVAL, "dsk_route: NULL pointer argument");
  if (!aligned(x, 16) || !aligned(gate_w, 16))
    return fail(DSK_EALIGN, "dsk_route: x and gate_w must be 16-byte aligned");
  return hip_check(launch_route(*d, x, gate_w, gate_b, scores, idx, weights,
                                static_cast<hipStream_t>(stream)),
                   "dsk_route launch");
}

int dsk_cap_union(int32_t tokens, int32_t n_experts, int32_t top_k, int32_t budget, int32_t strict,
                  const float* scores, int32_t* idx, float* weights, void* stream) {
  if (tokens < 1 || n_experts < 1 || n_experts > 1024 || top_k < 1 || top_k > 16 || top_k > n_experts)
    return fail(DSK_EINVAL, "dsk_cap_union: tokens=%d, n_experts=%d, top_k=%d out of range", tokens, n_experts,
                top_k);
  if (budget < 1) return fail(DSK_EINVAL, "dsk_cap_union: budget=%d must be >= 1", budget);
  if (!scores || !idx || !weights) return fail(DSK_EINVAL, "dsk_cap_union: NULL pointer argument");
  if (cap_union_lds(tokens, n_experts, top_k) > kMaxLds)
    return fail(DSK_EUNSUPPORTED, "dsk_cap_union: tokens*top_k=%lld is beyond the one-block cap (%zu bytes of LDS)",
                static_cast<long long>(tokens) * top_k, cap_union_lds(tokens, n_experts, top_k));
  return hip_check(launch_cap_union(scores, idx, weights, tokens, n_experts, top_k, budget, strict ? 1 : 0,
                                    static_cast<hipStream_t>(stream)),
                   "dsk_cap_union launch");
}

int dsk_dispatch(const dsk_moe_desc* d, const int32_t* idx, int32_t* counts, int32_t* offsets,
                 int32_t* perm, int32_t* rank, int32_t* active, void* stream) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (!idx || !counts || !offsets || !perm || !rank || !active)
    return fail(DSK_EINVAL, "dsk_dispatch: NULL pointer argument");
  DispatchOut o{counts, offsets, perm, rank, active, nullptr, nullptr, nullptr};
  return hip_check(launch_dispatch(*d, idx, nullptr, nullptr, o, static_cast<hipStream_t>(stream)),
                   "dsk_dispatch launch");
}

int dsk_dispatch_workspace_size(const dsk_moe_desc* d, size_t* bytes) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (!bytes) return fail(DSK_EINVAL, "dsk_dispatch_workspace_size: bytes is NULL");
  *bytes = dispatch_hist_ints(d->tokens * d->top_k, d->n_experts) * sizeof(int32_t);
  return 0;
}

int dsk_dispatch_ws(const dsk_moe_desc* d, const int32_t* idx, int32_t* counts, int32_t* offsets,
                    int32_t* perm, int32_t* rank, int32_t* active, void* workspace, size_t workspace_bytes,
                    void* stream) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (!idx || !counts || !offsets || !perm || !rank || !active)
    return fail(DSK_EINVAL, "dsk_dispatch_ws: NULL pointer argument");
  const size_t need = dispatch_hist_ints(d->tokens * d->top_k, d->n_experts) * sizeof(int32_t);
  if (need > 0 && !workspace) return fail(DSK_EINVAL, "dsk_dispatch_ws: workspace is NULL");
  if (workspace_bytes < need)
    return fail(DSK_ESPACE, "dsk_dispatch_ws: workspace %zu bytes < required %zu", workspace_bytes, need);
  if (need > 0 && !aligned(workspace, 256)) return fail(DSK_EALIGN, "dsk_dispatch_ws: workspace must be 256-byte aligned");
  DispatchOut o{counts, offsets, perm, rank, active, nullptr, nullptr, nullptr,
                need > 0 ? static_cast<int32_t*>(workspace) : nullptr};
  return hip_check(launch_dispatch(*d, idx, nullptr, nullptr, o, static_cast<hipStream_t>(stream)),
                   "dsk_dispatch_ws launch");
}

int dsk_experts(const dsk_moe_desc* d, const dsk_expert_ptrs* table, const void* ws1,
                const void* ws3, const void* ws2, const void* shared_out, const void* x,
                const float* weights,
                const int32_t* counts, const int32_t* offsets, const int32_t* perm,
                const int32_t* rank, const int32_t* active, void* out, void* workspace,
                size_t workspace_bytes, void* stream) {
  int rc = check_expert_desc(d);
  if (rc) return rc;
  if (!table || !x || !weights || !counts || !offsets || !perm || !rank || !active || !out ||
      !workspace)
    return fail(DSK_EINVAL, "dsk_experts: NULL pointer argument");
  if (d->inter_shared > 0 && (!ws1 || !ws3 || !ws2))
    return fail(DSK_EINVAL, "dsk_experts: shared expert weights are NULL but inter_shared=%d",
                d->inter_shared);
  if (shared_out && !aligned(shared_out, 16))
    return fail(DSK_EALIGN, "dsk_experts: shared_out must be 16-byte aligned");
  if (!aligned(x, 16) || !aligned(out, 16) || !aligned(workspace, 256) ||
      (d->inter_shared > 0 && (!aligned(ws1, 16) || !aligned(ws3, 16) || !aligned(ws2, 16))))
    return fail(DSK_EALIGN, "dsk_experts: x/out/shared weights need 16-byte, workspace 256-byte alignment");
  const Workspace L = workspace_layout(*d);
  if (workspace_bytes < L.total)
    return fail(DSK_ESPACE, "workspace %zu bytes < required %zu", workspace_bytes, L.total);
  ExpertsArgs a{};
  a.table = table; a.ws1 = ws1; a.ws3 = ws3; a.ws2 = ws2; a.shared_out = shared_out; a.x = x; a.weights = weights;
  a.counts = counts; a.offsets = offsets; a.perm = perm; a.rank = rank; a.active = active;
  a.out = out; a.ws = static_cast<char*>(workspace);
  return hip_check(launch_experts(*d, L, a, static_cast<hipStream_t>(stream), 1),
                   "dsk_experts launch");
}

int dsk_expert_rows(const dsk_moe_desc* d, const dsk_expert_ptrs* table, const void* x,
                    const float* weights, const int32_t* counts, const int32_t* offsets,
                    const int32_t* perm, const int32_t* rank, const int32_t* active, float* rows,
                    void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_expert_desc(d);
  if (rc) return rc;
  if (d->inter_shared != 0)
    return fail(DSK_EINVAL, "dsk_expert_rows: inter_shared must be 0 (routed experts only), got %d",
                d->inter_shared);
  if (!table || !x || !weights || !counts || !offsets || !perm || !rank || !active || !rows || !workspace)
    return fail(DSK_EINVAL, "dsk_expert_rows: NULL pointer argument");
  if (!aligned(x, 16) || !aligned(rows, 16) || !aligned(workspace, 256))
    return fail(DSK_EALIGN, "dsk_expert_rows: x/rows need 16-byte, workspace 256-byte alignment");
  const Workspace L = workspace_layout(*d);
  if (workspace_bytes < L.total)
    return fail(DSK_ESPACE, "workspace %zu bytes < required %zu", workspace_bytes, L.total);
  ExpertsArgs a{};
  a.table = table; a.x = x; a.weights = weights;
  a.counts = counts; a.offsets = offsets; a.perm = perm; a.rank = rank; a.active = active;
  a.ws = static_cast<char*>(workspace);
  a.rows_out = rows;
  return hip_check(launch_experts(*d, L, a, static_cast<hipStream_t>(stream), 1),
                   "dsk_expert_rows launch");
}

}  // extern "C"

int dsk::check_forward(const dsk_moe_desc* d, const void* x, const void* gate_w,
                       const float* gate_b, const dsk_expert_ptrs* table, const void* ws1,
                       const void* ws3, const void* ws2, const void* shared_out, void* out,
                       const void* workspace, bool own_scratch, void* const* events, int repeat) {
  int rc = check_expert_desc(d);
  if (rc) return rc;
  if (!x || !gate_w || !gate_b || !table || !out || (!workspace && !own_scratch))
    return fail(DSK_EINVAL, "dsk_moe_forward: NULL pointer argument");
  if (d->inter_shared > 0 && (!ws1 || !ws3 || !ws2))
    return fail(DSK_EINVAL, "dsk_moe_forward: shared expert weights are NULL but inter_shared=%d",
                d->inter_shared);
  if (shared_out && !aligned(shared_out, 16))
    return fail(DSK_EALIGN, "dsk_moe_forward: shared_out must be 16-byte aligned");
  if (!aligned(x, 16) || !aligned(gate_w, 16) || !aligned(out, 16) || (!own_scratch && !aligned(workspace, 256)) ||
      (d->inter_shared > 0 && (!aligned(ws1, 16) || !aligned(ws3, 16) || !aligned(ws2, 16))))
    return fail(DSK_EALIGN, "dsk_moe_forward: x/gate_w/out/shared need 16-byte, workspace 256-byte alignment");
  if (events)
    for (int i = 0; i < DSK_STAGE_EVENTS; ++i)
      if (!events[i]) return fail(DSK_EINVAL, "dsk_moe_forward_timed: event %d is NULL", i);
  if (repeat < 1 || repeat > 1000) return fail(DSK_EINVAL, "repeat=%d must be in [1, 1000]", repeat);
  return DSK_OK;
}

bool dsk::resnorm_fusable(const dsk_moe_desc& d) {
  // the first kernel of the decode pipeline is k_gate_shared (MX) or the
  // one-token-tile gate k_gate<1, 1>; both hold the rows in LDS
  return decode_pipeline(d) && (mx_decode(d) || d.tokens < 16) && d.x_dtype == DSK_DTYPE_BF16 &&
         d.hidden % 4 == 0 && d.hidden <= kResNormMaxHidden && d.tokens <= kResNormRows;
}

int dsk::forward_layer(const dsk_moe_desc* d, const void* x, const void* gate_w,
                       const float* gate_b, const dsk_expert_ptrs* table, const void* ws1,
                       const void* ws3, const void* ws2, const void* shared_out, void* out,
                       int32_t* idx, float* weights, void* workspace, size_t workspace_bytes,
                       void* stream, void* const* events, int repeat, const ResNorm* rn) {
  int rc = check_forward(d, x, gate_w, gate_b, table, ws1, ws3, ws2, shared_out, out, workspace, false, events,
                         repeat);
  if (rc) return rc;
  const Workspace L = workspace_layout(*d);
  if (workspace_bytes < L.total)
    return fail(DSK_ESPACE, "workspace %zu bytes < required %zu", workspace_bytes, L.total);
  char* ws = static_cast<char*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const hipEvent_t* ev = reinterpret_cast<const hipEvent_t*>(events);
  float* scores = reinterpret_cast<float*>(ws + L.scores);
  int32_t* idx_buf = idx ? idx : reinterpret_cast<int32_t*>(ws + L.idx);
  float* w_buf = weights ? weights : reinterpret_cast<float*>(ws + L.wts);
  int32_t* counts = reinterpret_cast<int32_t*>(ws + L.counts);
  int32_t* offsets = reinterpret_cast<int32_t*>(ws + L.offsets);
  int32_t* perm = reinterpret_cast<int32_t*>(ws + L.perm);
  int32_t* rank = reinterpret_cast<int32_t*>(ws + L.rank);
  int32_t* active = reinterpret_cast<int32_t*>(ws + L.active);
  RouteArgs ra{};
  ra.x = x; ra.gate_w = gate_w; ra.gate_b = gate_b;
  ra.scores = scores; ra.idx = idx_buf; ra.weights = w_buf; ra.table = table;
  ra.out = DispatchOut{counts, offsets, perm, rank, active,
                       reinterpret_cast<SlotDesc*>(ws + L.desc),
                       reinterpret_cast<int32_t*>(ws + L.xrow),
                       reinterpret_cast<float*>(ws + L.wrow),
                       dispatch_hist_ints(d->tokens * d->top_k, d->n_experts) > 0
                           ? reinterpret_cast<int32_t*>(ws + L.disp_hist)
                           : nullptr};
  ra.ctr = reinterpret_cast<unsigned int*>(ws + L.ctr);
  ra.rowmap = reinterpret_cast<int32_t*>(ws + L.rowmap);
  ExpertsArgs a{};
  a.table = table; a.desc = ra.out.desc; a.xrow = ra.out.xrow; a.wrow = ra.out.wrow;
  a.ws1 = ws1; a.ws3 = ws3; a.ws2 = ws2; a.shared_out = shared_out; a.x = x; a.gate_w = gate_w;
  a.weights = w_buf; a.counts = counts; a.offsets = offsets; a.perm = perm; a.rank = rank;
  a.active = active; a.out = out; a.ws = ws;
  a.rowmap = ra.rowmap;
  a.scores = scores; a.bias = gate_b;
  a.route = DecodeRoute{idx_buf, w_buf, ra.out.desc, active, ra.rowmap, ra.out.xrow, ra.out.wrow, rank};
  const bool decode = decode_pipeline(*d);
  // the unfused top-k kernel writes x in the form the gate/up that follows reads (FP8
  // planes for FP4 experts, the factored q3 form for q3 experts; prefill: its MX planes)
  if (!decode && d->tokens > kFusedMaxTokens && !rn && d->x_dtype == DSK_DTYPE_BF16) {
    const bool pf = prefill_mx(*d);
    if (pf || (!prefill_gemm(*d) && grouped_path(*d) && (grouped_up_mx(*d) || grouped_x_q3(*d)))) {
      ra.xp = reinterpret_cast<uint8_t*>(ws + L.xp);
      ra.xform = pf ? kXPrefillPlanes : d->quant == DSK_QUANT_Q3 ? kXGroupedQ3 : kXGroupedPlanes;
      a.x_planes_ready = 1;
    }
  }
  StageTiming timing(ev);
  stage_open(kStageGate);
  if (rn && !resnorm_fusable(*d)) {
    // the residual update and RMSNorm as their own kernel, then the layer on its rows
    for (int r = 0; r < repeat && !rc; ++r)
      rc = hip_check(launch_rmsnorm(rn->h, rn->d, rn->gamma, d->tokens, d->hidden, rn->eps, d->x_dtype,
                                    rn->h_out, rn->x_out, s),
                     "residual rmsnorm launch");
    if (rc) return rc;
    rn = nullptr;
  }
  ra.rn = rn;
  a.rn = rn;
  if (decode && mx_decode(*d)) {
    // gate scores beside the shared expert's gate/up; the top-k and the slot map beside
    // the shared expert's down; then the routed experts, which add the shared output
    rc = hip_check(launch_gate_shared(*d, L, a, s, repeat), "gate / shared gate-up launch");
    if (rc) return rc;
    stage_open(kStageRoute);
    rc = hip_check(launch_route_sdown(*d, L, a, s, repeat), "route / shared down launch");
    if (rc) return rc;
    dsk_moe_desc dr = *d;
    ExpertsArgs ar = a;
    if (d->inter_shared > 0) {
      dr.inter_shared = 0;
      ar.ws1 = ar.ws3 = ar.ws2 = nullptr;
      ar.shared_out = ws + L.shared_x;
    }
    rc = hip_check(launch_experts_decode(dr, L, ar, s, repeat), "decode experts launch");
  } else if (decode) {
    // gate scores; then the top-k and the slot map beside the shared expert's gate/up
    for (int r = 0; r < repeat && !rc; ++r) rc = hip_check(launch_gate_scores(*d, ra, s), "gate launch");
    if (rc) return rc;
    stage_open(kStageRoute);
    rc = hip_check(launch_route_shared(*d, L, a, s, repeat), "route / shared gate-up launch");
    if (rc) return rc;
    rc = hip_check(launch_experts_decode(*d, L, a, s, repeat), "decode experts launch");
  } else {
    // gate (the fused router of a few tokens also selects and dispatches), then top-k + dispatch
    for (int r = 0; r < repeat && !rc; ++r)
      rc = hip_check(launch_route_dispatch(*d, ra, s), "route launch");
    if (rc) return rc;
    rc = hip_check(launch_experts(*d, L, a, s, repeat), "experts launch");
  }
  stage_close();
  return rc;
}

extern "C" {

int dsk_moe_forward(const dsk_moe_desc* d, const void* x, const void* gate_w, const float* gate_b,
                    const dsk_expert_ptrs* table, const void* ws1, const void* ws3,
                    const void* ws2, const void* shared_out, void* out, int32_t* idx,
                    float* weights, void* workspace, size_t workspace_bytes, void* stream) {
  return forward_layer(d, x, gate_w, gate_b, table, ws1, ws3, ws2, shared_out, out, idx, weights,
                       workspace, workspace_bytes, stream, nullptr, 1);
}

int dsk_moe_forward_residual(const dsk_moe_desc* d, const dsk_residual* r, const void* gate_w,
                             const float* gate_b, const dsk_expert_ptrs* table, const void* ws1,
                             const void* ws3, const void* ws2, void* out, int32_t* idx, float* weights,
                             void* workspace, size_t workspace_bytes, void* stream) {
  if (!d || !r) return fail(DSK_EINVAL, "dsk_moe_forward_residual: NULL desc or residual");
  if (!r->h || !r->d || !r->h_out || !r->x_out)
    return fail(DSK_EINVAL, "dsk_moe_forward_residual: h, d, h_out and x_out are required");
  if (!(r->eps >= 0.0f)) return fail(DSK_EINVAL, "dsk_moe_forward_residual: eps must be >= 0");
  if (!aligned(r->h, 16) || !aligned(r->d, 16) || !aligned(r->h_out, 16) || !aligned(r->x_out, 16) ||
      (r->gamma && !aligned(r->gamma, 16)))
    return fail(DSK_EALIGN, "dsk_moe_forward_residual: stream pointers must be 16-byte aligned");
  int rc = check_forward(d, r->x_out, gate_w, gate_b, table, ws1, ws3, ws2, nullptr, out, workspace, false,
                         nullptr, 1);
  if (rc) return rc;
  const size_t bytes = static_cast<size_t>(d->tokens) * d->hidden * (d->x_dtype == DSK_DTYPE_BF16 ? 2 : 4);
  auto overlap = [bytes](const void* a, const void* b) {
    const char* x = static_cast<const char*>(a);
    const char* y = static_cast<const char*>(b);
    return x < y + bytes && y < x + bytes;
  };
  if (overlap(r->x_out, r->h) || overlap(r->x_out, r->d) || overlap(r->x_out, r->h_out) ||
      overlap(r->x_out, out) || overlap(r->h_out, r->d) ||
      (r->h_out != r->h && overlap(r->h_out, r->h)))
    return fail(DSK_EINVAL, "dsk_moe_forward_residual: x_out and h_out must not overlap the other buffers "
                "(h_out may be h itself)");
  ResNorm rn{static_cast<const uint16_t*>(r->h), static_cast<const uint16_t*>(r->d), r->gamma, r->eps,
             static_cast<uint16_t*>(r->h_out), static_cast<uint16_t*>(r->x_out)};
  if (r->h_out == r->h) {
    // in place: every block of a fused first kernel reads h, so the update runs as its own kernel
    rc = hip_check(launch_rmsnorm(r->h, r->d, r->gamma, d->tokens, d->hidden, r->eps, d->x_dtype, r->h_out,
                                  r->x_out, static_cast<hipStream_t>(stream)),
                   "residual rmsnorm launch");
    if (rc) return rc;
    return forward_layer(d, r->x_out, gate_w, gate_b, table, ws1, ws3, ws2, nullptr, out, idx, weights,
                         workspace, workspace_bytes, stream, nullptr, 1);
  }
  return forward_layer(d, r->x_out, gate_w, gate_b, table, ws1, ws3, ws2, nullptr, out, idx, weights,
                       workspace, workspace_bytes, stream, nullptr, 1, &rn);
}

int dsk_moe_forward_timed(const dsk_moe_desc* d, const void* x, const void* gate_w,
                          const float* gate_b, const dsk_expert_ptrs* table, const void* ws1,
                          const void* ws3, const void* ws2, const void* shared_out, void* out,
                          int32_t* idx, float* weights, void* workspace,
                          size_t workspace_bytes, void* stream, void* const* events,
                          int32_t repeat) {
  if (!events) return fail(DSK_EINVAL, "dsk_moe_forward_timed: events is NULL");
  return forward_layer(d, x, gate_w, gate_b, table, ws1, ws3, ws2, shared_out, out, idx, weights,
                       workspace, workspace_bytes, stream, events, repeat);
}

int dsk_fp4_dequant(const uint8_t* packed, const uint8_t* scales, int64_t rows, int64_t cols,
                    void* out, int32_t out_dtype, void* stream) {
  if (!packed || !scales || !out) return fail(DSK_EINVAL, "dsk_fp4_dequant: NULL pointer argument");
  if (rows < 0 || cols < 0 || cols % 32) return fail(DSK_EINVAL, "cols=%lld must be a multiple of 32", (long long)cols);
  if (out_dtype != DSK_DTYPE_F32 && out_dtype != DSK_DTYPE_BF16)
    return fail(DSK_EINVAL, "out_dtype %d must be F32 or BF16", out_dtype);
  if (!aligned(packed, 16) || !aligned(out, 16))
    return fail(DSK_EALIGN, "dsk_fp4_dequant: packed and out must be 16-byte aligned");
  return hip_check(launch_fp4_dequant(packed, scales, rows, cols, out, out_dtype,
                                      static_cast<hipStream_t>(stream)),
                   "dsk_fp4_dequant launch");
}

int dsk_fp8_block_dequant(const uint8_t* codes, const uint8_t* scales, int64_t rows, int64_t cols, void* out,
                          int32_t out_dtype, void* stream) {
  if (!codes || !scales || !out) return fail(DSK_EINVAL, "dsk_fp8_block_dequant: NULL pointer argument");
  if (rows < 0 || cols < 0 || rows % 32 || cols % 32)
    return fail(DSK_EINVAL, "rows=%lld and cols=%lld must be multiples of 32", (long long)rows, (long long)cols);
  if (out_dtype != DSK_DTYPE_F32 && out_dtype != DSK_DTYPE_BF16)
    return fail(DSK_EINVAL, "out_dtype %d must be F32 or BF16", out_dtype);
  if (!aligned(codes, 16) || !aligned(out, 16))
    return fail(DSK_EALIGN, "dsk_fp8_block_dequant: codes and out must be 16-byte aligned");
  return hip_check(launch_fp8_block_dequant(codes, scales, rows, cols, out, out_dtype,
                                            static_cast<hipStream_t>(stream)),
                   "dsk_fp8_block_dequant launch");
}

int dsk_fp4_quantize(const float* w, int64_t rows, int64_t cols, uint8_t* packed, uint8_t* scales,
                     void* stream) {
  if (!w || !packed || !scales) return fail(DSK_EINVAL, "dsk_fp4_quantize: NULL pointer argument");
  if (rows < 0 || cols < 0 || cols % 32) return fail(DSK_EINVAL, "cols=%lld must be a multiple of 32", (long long)cols);
  if (!aligned(w, 16) || !aligned(packed, 16))
    return fail(DSK_EALIGN, "dsk_fp4_quantize: w and packed must be 16-byte aligned");
  return hip_check(launch_fp4_quantize(w, rows, cols, packed, scales, static_cast<hipStream_t>(stream)),
                   "dsk_fp4_quantize launch");
}

int dsk_q3_quantize(const float* w, int64_t rows, int64_t cols, uint8_t* packed, uint16_t* scales,
                    uint16_t* biases, void* stream) {
  if (!w || !packed || !scales || !biases) return fail(DSK_EINVAL, "dsk_q3_quantize: NULL pointer argument");
  if (rows < 0 || cols < 0 || cols % 128 || cols > INT32_MAX)
    return fail(DSK_EINVAL, "cols=%lld must be a multiple of 128 below 2^31", (long long)cols);
  if (!aligned(w, 4) || !aligned(packed, 4) || !aligned(scales, 2) || !aligned(biases, 2))
    return fail(DSK_EALIGN, "dsk_q3_quantize: misaligned pointer");
  return hip_check(launch_q3_quantize(w, rows, cols, packed, scales, biases,
                                      static_cast<hipStream_t>(stream)),
                   "dsk_q3_quantize launch");
}

int dsk_q3_repack(const uint8_t* src, int64_t rows, int64_t cols, uint8_t* packed, void* stream) {
  if (!src || !packed) return fail(DSK_EINVAL, "dsk_q3_repack: NULL pointer argument");
  if (rows < 0 || cols < 0 || cols % 128 || cols > INT32_MAX)
    return fail(DSK_EINVAL, "cols=%lld must be a multiple of 128 below 2^31", (long long)cols);
  if (!aligned(src, 4) || !aligned(packed, 4))
    return fail(DSK_EALIGN, "dsk_q3_repack: src and packed must be 4-byte aligned");
  const uintptr_t a = reinterpret_cast<uintptr_t>(src), b = reinterpret_cast<uintptr_t>(packed);
  const uintptr_t n = static_cast<uintptr_t>(rows) * static_cast<uintptr_t>(cols / 8 * 3);
  if (n && a < b + n && b < a + n) return fail(DSK_EINVAL, "dsk_q3_repack: src and packed overlap");
  return hip_check(launch_q3_repack(src, rows, cols, packed, static_cast<hipStream_t>(stream)),
                   "dsk_q3_repack launch");
}

int dsk_q3_dequant(const uint8_t* packed, const uint16_t* scales, const uint16_t* biases,
                   int64_t rows, int64_t cols, void* out, int32_t out_dtype, void* stream) {
  if (!packed || !scales || !biases || !out) return fail(DSK_EINVAL, "dsk_q3_dequant: NULL pointer argument");
  if (rows < 0 || cols < 0 || cols % 128 || cols > INT32_MAX)
    return fail(DSK_EINVAL, "cols=%lld must be a multiple of 128 below 2^31", (long long)cols);
  if (out_dtype != DSK_DTYPE_F32 && out_dtype != DSK_DTYPE_BF16)
    return fail(DSK_EINVAL, "out_dtype %d must be F32 or BF16", out_dtype);
  if (!aligned(packed, 4) || !aligned(out, 4))
    return fail(DSK_EALIGN, "dsk_q3_dequant: misaligned pointer");
  return hip_check(launch_q3_dequant(packed, scales, biases, rows, cols, out, out_dtype,
                                     static_cast<hipStream_t>(stream)),
                   "dsk_q3_dequant launch");
}

int dsk_rmsnorm(const void* x, const void* residual, const float* gamma, int64_t rows, int32_t hidden,
                float eps, int32_t dtype, void* h_out, void* out, void* stream) {
  if (!x) return fail(DSK_EINVAL, "dsk_rmsnorm: x is NULL");
  if (!out && !(residual && h_out))
    return fail(DSK_EINVAL, "dsk_rmsnorm: nothing to write (out is NULL and no residual update)");
  if (rows < 0 || hidden < 4 || hidden % 4)
    return fail(DSK_EINVAL, "dsk_rmsnorm: rows=%lld, hidden=%d must be >= 0 and a positive multiple of 4",
                (long long)rows, hidden);
  if (dtype != DSK_DTYPE_F32 && dtype != DSK_DTYPE_BF16)
    return fail(DSK_EINVAL, "dsk_rmsnorm: dtype %d must be F32 or BF16", dtype);
  if (!(eps >= 0.0f)) return fail(DSK_EINVAL, "dsk_rmsnorm: eps must be >= 0");
  if (!aligned(x, 16) || (residual && !aligned(residual, 16)) || (gamma && !aligned(gamma, 16)) ||
      (h_out && !aligned(h_out, 16)) || (out && !aligned(out, 16)))
    return fail(DSK_EALIGN, "dsk_rmsnorm: pointers must be 16-byte aligned");
  return hip_check(launch_rmsnorm(x, residual, gamma, rows, hidden, eps, dtype, h_out, out,
                                  static_cast<hipStream_t>(stream)),
                   "dsk_rmsnorm launch");
}

}  // extern "C"
