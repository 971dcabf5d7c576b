// Router: gate logits, scores, biased top-k with normalised weights, and
// (small batches) the dispatch, in one kernel.
//
// Replaces the reference's sqrtsoftplus_scores and route_topk
// (src/deepseeker/mlx_forward.py:62-81) and the host-side grouping of
// moe_layer (:294-312).  Indices must be bit-identical to the CPU oracle, so
// every floating-point step follows one defined order (this file is compiled
// without contraction, and the pragma below makes that explicit):
//   logit  H is cut into 256-element steps and the steps into 4 segments of
//          ceil(steps/4); wave w of a block owns segment w.  Lane l keeps a
//          float32 partial that adds, over the segment's steps m and then
//          v = 0..3, the rounded product x[256m+4l+v] * W[e][256m+4l+v]; an XOR
//          butterfly (s = 32..1: p[l] = p[l] + p[l^s]) gives the segment sum
//          s_w, and z = ((s_0 + s_1) + s_2) + s_3.
//   score  in double with this file's own exp (Cody-Waite ln2 split, degree-14
//          Taylor in Horner form) and log1p (2*atanh(u/(2+u)), odd series),
//          rounded once to float; sqrt-softplus takes the correctly rounded
//          float sqrt found by exact midpoint tests.
//   top-k  key = (s + bias) + 0; k largest keys, descending, ties to the
//          lower expert id (64-bit composite of order-preserving key bits and
//          the inverted id, reduced across the wave).
//   weight w_j = (s_j / (((s_0 + s_1) + ...) + 1e-20f)) * route_scale.
//
// Fused path (few tokens): block (expert tile, token tile) computes its
// logits; the last block to finish a token tile (one atomic add per block on
// an arrival counter) does that tile's top-k, and the last token tile to
// finish runs the dispatch.  The last arrival resets its counter, so the
// counter region, zero-filled once before first use, stays zero between
// calls (and across graph replays).
#include <algorithm>

#include "dispatch_block.h"
#include "gate.h"
#include "tile.h"

#pragma clang fp contract(off)

namespace dsk {
namespace {

struct GateArgs {
  const void* x; const void* gw; const float* bias;
  int T, H, E, k, score_func, nbits;
  float route_scale;
  float* scores; int32_t* idx; float* weights;
  const dsk_expert_ptrs* table;
  DispatchOut out;
  unsigned int* ctr;
};

// Block = 4 waves (one segment each) x a TW-token x EW-expert tile.
template <int TW, int EW, bool kXBF16, bool kWBF16, bool kFused>
__global__ __launch_bounds__(256) void k_gate(GateArgs g) {
  extern __shared__ float smem[];
  float* segsum = smem;                       // [4][TW*EW]
  int* flag = reinterpret_cast<int*>(smem + kSegments * TW * EW);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_et = (g.E + EW - 1) / EW;
  const int et = blockIdx.x % n_et, tt = blockIdx.x / n_et;
  const int t0 = tt * TW, e0 = et * EW;
  const int T = g.T, E = g.E;
  gate_tile<TW, EW, kXBF16, kWBF16>(g.x, g.gw, T, g.H, E, g.score_func, g.scores, t0, e0, wave, lane,
                                    threadIdx.x, segsum);
  if constexpr (kFused) {
    const int n_tt = (T + TW - 1) / TW;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) *flag = arrive_last(&g.ctr[tt], static_cast<unsigned int>(n_et));
    __syncthreads();
    if (!*flag) return;
    __threadfence();
    if (wave < TW && t0 + wave < T) {
      const int t = t0 + wave;
      topk_token(g.scores + static_cast<int64_t>(t) * E, g.bias, E, g.k, g.route_scale,
                 g.idx + static_cast<int64_t>(t) * g.k, g.weights + static_cast<int64_t>(t) * g.k);
    }
    __threadfence();
    __syncthreads();
    if (n_tt > 1) {
      if (threadIdx.x == 0) *flag = arrive_last(&g.ctr[n_tt], static_cast<unsigned int>(n_tt));
      __syncthreads();
      if (!*flag) return;
      __threadfence();
    }
    dispatch_block(g.idx, T * g.k, E, g.k, g.nbits, g.weights, g.table, g.out, flag + 4);
  }
}

// One wave per token: biased top-k + normalised weights (unfused path).
__global__ __launch_bounds__(256) void k_topk(const float* __restrict__ scores,
                                              const float* __restrict__ bias, int T, int E,
                                              int k, float route_scale,
                                              int32_t* __restrict__ idx,
                                              float* __restrict__ weights) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  topk_token(scores + static_cast<int64_t>(t) * E, bias, E, k, route_scale,
             idx + static_cast<int64_t>(t) * k, weights + static_cast<int64_t>(t) * k);
}

template <int TW, int EW, bool kFused>
hipError_t launch_gate(const dsk_moe_desc& d, const GateArgs& g, hipStream_t s) {
  const int n_et = (d.n_experts + EW - 1) / EW;
  const int n_tt = (d.tokens + TW - 1) / TW;
  const unsigned blocks = static_cast<unsigned>(n_et * n_tt);
  size_t lds = (kSegments * TW * EW + 4) * sizeof(float);
  if (kFused) lds += static_cast<size_t>(4 * d.n_experts + d.n_experts + 32) * sizeof(int32_t);
  const bool xb = d.x_dtype == DSK_DTYPE_BF16, wb = d.gate_dtype == DSK_DTYPE_BF16;
  if (xb && wb) k_gate<TW, EW, true, true, kFused><<<blocks, 256, lds, s>>>(g);
  else if (xb) k_gate<TW, EW, true, false, kFused><<<blocks, 256, lds, s>>>(g);
  else if (wb) k_gate<TW, EW, false, true, kFused><<<blocks, 256, lds, s>>>(g);
  else k_gate<TW, EW, false, false, kFused><<<blocks, 256, lds, s>>>(g);
  return hipGetLastError();
}

// Top-k of T <= 16 tokens (wave t: token t) and the one-wave dispatch of the
// decode pipeline, in one block after the gate kernel.  The other waves (and
// the top-k waves once done) copy the expert table into LDS meanwhile, so the
// dispatch's descriptor writes do not wait on global loads.
__global__ __launch_bounds__(1024) void k_route_tail(GateArgs g, int32_t* rowmap) {
  extern __shared__ __align__(16) int32_t tail_lds[];
  const int wave = threadIdx.x >> 6;
  const int N = g.T * g.k;
  int32_t* lidx = tail_lds;                                  // [64]
  float* lw = reinterpret_cast<float*>(tail_lds + 64);       // [64]
  uint64_t* ltab = reinterpret_cast<uint64_t*>(tail_lds + 128);   // [E * 9]
  int32_t* ldisp = tail_lds + 128 + 2 * 9 * g.E;
  if (wave < g.T)
    topk_token(g.scores + static_cast<int64_t>(wave) * g.E, g.bias, g.E, g.k, g.route_scale,
               g.idx + static_cast<int64_t>(wave) * g.k, g.weights + static_cast<int64_t>(wave) * g.k,
               lidx + wave * g.k, lw + wave * g.k);
  {
    constexpr int kWords = sizeof(dsk_expert_ptrs) / 8;
    const uint64_t* src = reinterpret_cast<const uint64_t*>(g.table);
    const int n = g.E * kWords;
    constexpr int kU = 8;
    for (int i0 = threadIdx.x; i0 < n; i0 += kU * blockDim.x) {
      uint64_t v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int i = i0 + u * blockDim.x;
        v[u] = i < n ? src[i] : 0ull;
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int i = i0 + u * blockDim.x;
        if (i < n) ltab[i] = v[u];
      }
    }
  }
  __syncthreads();
  if (wave == 0)
    dispatch_wave(lidx, N, g.E, g.k, g.T, lw, reinterpret_cast<const dsk_expert_ptrs*>(ltab), g.out,
                  rowmap, ldisp);
}

GateArgs make_gate_args(const dsk_moe_desc& d, const void* x, const void* gate_w,
                        const float* gate_b, float* scores, int32_t* idx, float* weights) {
  GateArgs g{};
  g.x = x; g.gw = gate_w; g.bias = gate_b;
  g.T = d.tokens; g.H = d.hidden; g.E = d.n_experts; g.k = d.top_k;
  g.score_func = d.score_func; g.nbits = bits_for(d.n_experts);
  g.route_scale = d.route_scale;
  g.scores = scores; g.idx = idx; g.weights = weights;
  return g;
}

hipError_t launch_route_unfused(const dsk_moe_desc& d, const GateArgs& g, hipStream_t s) {
  hipError_t e = (d.tokens >= 16) ? launch_gate<4, 4, false>(d, g, s) : launch_gate<1, 1, false>(d, g, s);
  if (e != hipSuccess) return e;
  const unsigned blocks = static_cast<unsigned>((d.tokens + 3) / 4);
  k_topk<<<blocks, 256, 0, s>>>(g.scores, g.bias, d.tokens, d.n_experts, d.top_k, d.route_scale,
                                g.idx, g.weights);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_route(const dsk_moe_desc& d, const void* x, const void* gate_w,
                        const float* gate_b, float* scores, int32_t* idx, float* weights,
                        hipStream_t s) {
  return launch_route_unfused(d, make_gate_args(d, x, gate_w, gate_b, scores, idx, weights), s);
}

GateArgs route_gate_args(const dsk_moe_desc& d, const RouteArgs& a) {
  GateArgs g = make_gate_args(d, a.x, a.gate_w, a.gate_b, a.scores, a.idx, a.weights);
  g.table = a.table;
  g.out = a.out;
  g.ctr = a.ctr;
  return g;
}

hipError_t launch_route_dispatch(const dsk_moe_desc& d, const RouteArgs& a, hipStream_t s) {
  const GateArgs g = route_gate_args(d, a);
  if (d.tokens <= kFusedMaxTokens) {
    return d.tokens == 1 ? launch_gate<1, 4, true>(d, g, s) : launch_gate<4, 1, true>(d, g, s);
  }
  hipError_t e = launch_route_unfused(d, g, s);
  if (e != hipSuccess) return e;
  return launch_dispatch(d, a.idx, a.weights, a.table, a.out, s);
}

hipError_t launch_gate_scores(const dsk_moe_desc& d, const RouteArgs& a, hipStream_t s) {
  const GateArgs g = route_gate_args(d, a);
  return d.tokens >= 16 ? launch_gate<4, 4, false>(d, g, s) : launch_gate<1, 1, false>(d, g, s);
}

hipError_t launch_route_tail(const dsk_moe_desc& d, const RouteArgs& a, hipStream_t s) {
  const GateArgs g = route_gate_args(d, a);
  const int per = (d.n_experts + 63) / 64;
  const size_t lds = static_cast<size_t>(128 + 2 * 9 * d.n_experts + 64 + 64 * per + 64 * d.tokens) *
                     sizeof(int32_t);
  // top-k waves plus at least three copy waves
  const int waves = d.tokens + 3 < 16 ? d.tokens + 3 : 16;
  const unsigned threads = static_cast<unsigned>(64 * waves);
  k_route_tail<<<1, threads, lds, s>>>(g, a.rowmap);
  return hipGetLastError();
}

}  // namespace dsk
