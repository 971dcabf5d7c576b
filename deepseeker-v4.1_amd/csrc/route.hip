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
//          float32 partial that starts at +0 and takes, over the segment's
//          steps m and then v = 0..3, p = fma(x[256m+4l+v], W[e][256m+4l+v], p)
//          (one rounding per step); an XOR butterfly (s = 32..1:
//          p[l] = p[l] + p[l^s]) gives the segment sum s_w, and
//          z = ((s_0 + s_1) + s_2) + s_3.
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
#include "mx.h"
#include "resnorm.h"
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
  ResNorm rn; int norm;     // norm: x is h + d normalised here (resnorm.h); block 0 writes it out
  uint8_t* xp;              // k_topk: also write x for the grouped gate/up here, or null:
  int xform;                // XForm
};

// Byte offset of the normalised rows in k_gate's LDS (after the segment sums and flags).
constexpr size_t kGateNormOffset = 512;

// Block = 4 waves (one segment each) x a TW-token x EW-expert tile.
// kNorm: x is the residual stream's update normalised here (resnorm.h).
template <int TW, int EW, bool kXBF16, bool kWBF16, bool kFused, bool kNorm = false>
__global__ __launch_bounds__(256) void k_gate(GateArgs g) {
  extern __shared__ float smem[];
  float* segsum = smem;                       // [4][TW*EW]
  int* flag = reinterpret_cast<int*>(smem + kSegments * TW * EW);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_et = (g.E + EW - 1) / EW;
  const int et = blockIdx.x % n_et, tt = blockIdx.x / n_et;
  const int t0 = tt * TW, e0 = et * EW;
  const int T = g.T, E = g.E;
  if constexpr (kNorm) {
    // every block normalises the rows itself (LDS, row stride H) while its
    // first gate weights load; block 0 also writes the new residual stream and
    // the rows for the layer's later kernels
    static_assert(!kFused && kXBF16, "the stream is bf16 and the scores go to the top-k kernel");
    __shared__ float rn_wsum[kResNormWsum];
    uint16_t* y = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(smem) + kGateNormOffset);
    ResNormIn<256> in;
    resnorm_issue<256>(g.rn, T, g.H, in);
    asm volatile("" ::: "memory");   // the rows' loads first: waiting for them leaves the weights in flight
    GateWFirst<TW, EW, kWBF16> pre;
    gate_w_issue<TW, EW, kWBF16>(g.gw, g.H, E, e0, wave, lane, true, pre);
    resnorm_rows<256>(g.rn, T, g.H, y, g.H, blockIdx.x == 0, rn_wsum, in);
    gate_tile<TW, EW, kXBF16, kWBF16, true>(y, g.gw, T, g.H, E, g.score_func, g.scores, t0, e0, wave, lane,
                                            threadIdx.x, segsum, true, &pre);
  } else {
    gate_tile<TW, EW, kXBF16, kWBF16>(g.x, g.gw, T, g.H, E, g.score_func, g.scores, t0, e0, wave, lane,
                                      threadIdx.x, segsum);
  }
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
// With xp, the blocks after the top-k's ((T + 3) / 4) write x in the form
// of the gate/up that follows, one 8-value chunk per thread (XForm: the work
// of k_x_planes, k_x_q3 or k_pf_planes, without a launch of its own).
__global__ __launch_bounds__(256) void k_topk(const float* __restrict__ scores,
                                              const float* __restrict__ bias, int T, int E,
                                              int k, float route_scale,
                                              int32_t* __restrict__ idx,
                                              float* __restrict__ weights, const uint16_t* __restrict__ x,
                                              int H, uint8_t* __restrict__ xp, int form) {
  const int tb = (T + 3) / 4;
  if (static_cast<int>(blockIdx.x) >= tb) {
    const int n = T * (H / 8);
    const int c = (static_cast<int>(blockIdx.x) - tb) * 256 + static_cast<int>(threadIdx.x);
    // every lane takes part in the group exchange / sums
    const size_t plane_bytes = static_cast<size_t>(T) * H * 2;
    if (form == kXGroupedQ3)
      x_q3_chunk(x, H, min(c, n - 1), c < n, reinterpret_cast<uint16_t*>(xp),
                 reinterpret_cast<float*>(xp + plane_bytes));
    else if (form == kXPrefillPlanes)
      pf_planes_chunk(x, H, min(c, n - 1), c < n, xp, xp + plane_bytes);
    else
      x_planes_chunk(x, T, H, min(c, n - 1), c < n, xp);
    return;
  }
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  topk_token(scores + static_cast<int64_t>(t) * E, bias, E, k, route_scale,
             idx + static_cast<int64_t>(t) * k, weights + static_cast<int64_t>(t) * k);
}

// Wide gate for large batches.  Block = 8 waves and a 32-token x 16-expert
// tile; wave w owns tokens 8 (w & 3) + [0, 8) and experts 8 (w >> 2) +
// [0, 8), and lane l the partial l of each of its 64 (token, expert) pairs.
// Each 256-element step m is staged through LDS (double-buffered: x [32][256],
// W [16][256]) and every partial takes, for v = 0..3, the fused multiply-add
// at position 256m + 4l + v: the order of the definition above.  At the end of a
// segment the 64 partials of each pair are combined by the same XOR tree,
// computed as a reduce-scatter: at stride s a lane keeps the upper half of
// its pairs if bit s of its lane id is set and adds the partner's (lane ^ s)
// copy of them, so after strides 32..1 lane l holds the segment sum of pair l
// -- the sum lane 0 of the full butterfly holds, at a sixth of the additions
// and exchanges.  The kernel is held to 128 registers, so two blocks share a
// CU (four waves per SIMD): a step's products of one block run while the
// other waits at its barrier or for its LDS reads.
constexpr int kGwThreads = 512;
constexpr int kGwTok = 32, kGwExp = 16;
constexpr int kGateWideMinTokens = 128;

template <bool kBF16>
__device__ __forceinline__ f32x4 lds_f32x4(const char* row, int lane) {
  if constexpr (kBF16) {
    const uint2 raw = *reinterpret_cast<const uint2*>(row + 8 * lane);
    return f32x4{__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                 __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u)};
  } else {
    return *reinterpret_cast<const f32x4*>(row + 16 * lane);
  }
}

// Value of lane l ^ S (S = 8, 4, 2, 1): DPP within a row of 16 lanes (a
// rotation by 8 is the XOR with 8 there), the LDS crossbar's swizzle for 4.
template <int S>
__device__ __forceinline__ float lane_xor(float v) {
  const int u = __float_as_int(v);
  int r;
  if constexpr (S == 8) r = __builtin_amdgcn_update_dpp(0, u, 0x128, 0xF, 0xF, false);        // row_ror:8
  else if constexpr (S == 4) r = __builtin_amdgcn_ds_swizzle(u, 0x1F | (4 << 10));            // xor 4
  else if constexpr (S == 2) r = __builtin_amdgcn_update_dpp(0, u, 0x4E, 0xF, 0xF, false);    // [2,3,0,1]
  else r = __builtin_amdgcn_update_dpp(0, u, 0xB1, 0xF, 0xF, false);                          // [1,0,3,2]
  return __int_as_float(r);
}

// Reduce-scatter of N values per lane across the 64 lanes at stride S (then
// S/2 .. 1); on return lane l holds in vals[0 .. N/64) the tree sums of
// values l*N/64 .. of the full XOR butterfly.  At stride S a lane keeps the
// upper half of its values if bit S of its id is set, else the lower half,
// and adds the partner's (lane ^ S) copy of them.  Strides 32 and 16 are one
// v_permlane32_swap / v_permlane16_swap per pair of values: the swap leaves
// in each lane exactly the two addends of its kept value (vals[j] of lane l
// and of lane l ^ S in the lower lanes, vals[j + N/2] of both in the upper
// ones), and their sum is the same in either order.
template <int N, int S>
__device__ __forceinline__ void xor_reduce_scatter(float* vals, int lane) {
#pragma clang fp contract(off)
  if constexpr (S >= 16) {
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
      const uint32_t a = __float_as_uint(vals[j]), b = __float_as_uint(vals[j + N / 2]);
      const auto sw = S == 32 ? __builtin_amdgcn_permlane32_swap(a, b, false, false)
                              : __builtin_amdgcn_permlane16_swap(a, b, false, false);
      vals[j] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    xor_reduce_scatter<N / 2, S / 2>(vals, lane);
  } else if constexpr (S >= 1) {
    const bool upper = (lane & S) != 0;
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
      const float send = upper ? vals[j] : vals[j + N / 2];
      const float mine = upper ? vals[j + N / 2] : vals[j];
      vals[j] = mine + lane_xor<S>(send);
    }
    xor_reduce_scatter<N / 2, S / 2>(vals, lane);
  }
}

// kFull: the tile's 32 tokens and 16 experts all exist and H is a multiple
// of 256, so the staging loads need no clamps and the stores no masks.
template <bool kXBF16, bool kWBF16, bool kFull>
__device__ __forceinline__ void gate_wide_tile(const GateArgs& g, char* gw_lds, int t0, int e0) {
#pragma clang fp contract(off)
  constexpr int kSx = kXBF16 ? 2 : 4, kSw = kWBF16 ? 2 : 4;
  constexpr int kXBytes = kGwTok * 256 * kSx, kWBytes = kGwExp * 256 * kSw;
  constexpr int kBuf = kXBytes + kWBytes;
  constexpr int kXChunks = kXBytes / 16 / kGwThreads, kWChunks = kWBytes / 16 / kGwThreads;
  static_assert(kXChunks >= 1 && kWChunks >= 1, "staging chunks");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wt = wave & 3, we = wave >> 2;
  const int H = g.H, steps = (H + 255) / 256, seg = (steps + kSegments - 1) / kSegments;
  // staging: thread chunk c = tid + 512 q of the x tile ([32][256] elements,
  // 16-byte chunks), the same for W; addresses recomputed per step
  // The loads are issued without conditions (a load under a per-lane
  // condition compiles to a branch whose merge waits for it): a chunk past H
  // re-reads the row's last in-range chunk and is zeroed by a mask when it
  // is stored.
  u32x4 xr[kXChunks], wr[kWChunks];
  uint32_t xkeep[kXChunks], wkeep[kWChunks];
  // full tiles: each chunk's byte offset from the (uniform) array start,
  // the step adds 256 elements (the arrays are below 2 GB: kFull's test)
  uint32_t xo[kXChunks], wo[kWChunks];
  if constexpr (kFull) {
#pragma unroll
    for (int q = 0; q < kXChunks; ++q) {
      constexpr int per_row = 256 * kSx / 16;
      const int c = tid + kGwThreads * q;
      xo[q] = static_cast<uint32_t>(((t0 + c / per_row) * H + (c % per_row) * (16 / kSx)) * kSx);
    }
#pragma unroll
    for (int q = 0; q < kWChunks; ++q) {
      constexpr int per_row = 256 * kSw / 16;
      const int c = tid + kGwThreads * q;
      wo[q] = static_cast<uint32_t>(((e0 + c / per_row) * H + (c % per_row) * (16 / kSw)) * kSw);
    }
  }
  auto load = [&](int m) {
    if constexpr (kFull) {
      const char* xbase = static_cast<const char*>(g.x) + static_cast<int64_t>(256 * kSx) * m;
      const char* wbase = static_cast<const char*>(g.gw) + static_cast<int64_t>(256 * kSw) * m;
#pragma unroll
      for (int q = 0; q < kXChunks; ++q) xr[q] = ldg16(xbase + xo[q]);
#pragma unroll
      for (int q = 0; q < kWChunks; ++q) wr[q] = ldg16(wbase + wo[q]);
    } else {
#pragma unroll
      for (int q = 0; q < kXChunks; ++q) {
        constexpr int per_row = 256 * kSx / 16;
        const int c = tid + kGwThreads * q;
        const int col = 256 * m + (c % per_row) * (16 / kSx);
        const int64_t row = min(t0 + c / per_row, g.T - 1);
        xkeep[q] = col < H ? ~0u : 0u;
        xr[q] = ldg16(static_cast<const char*>(g.x) + (row * H + min(col, H - 16 / kSx)) * kSx);
      }
#pragma unroll
      for (int q = 0; q < kWChunks; ++q) {
        constexpr int per_row = 256 * kSw / 16;
        const int c = tid + kGwThreads * q;
        const int col = 256 * m + (c % per_row) * (16 / kSw);
        const int64_t row = min(e0 + c / per_row, g.E - 1);
        wkeep[q] = col < H ? ~0u : 0u;
        wr[q] = ldg16(static_cast<const char*>(g.gw) + (row * H + min(col, H - 16 / kSw)) * kSw);
      }
    }
  };
  auto store = [&](int buf) {
    char* b = gw_lds + buf * kBuf;
#pragma unroll
    for (int q = 0; q < kXChunks; ++q)
      *reinterpret_cast<u32x4*>(b + 16 * (tid + kGwThreads * q)) = kFull ? xr[q] : (xr[q] & xkeep[q]);
#pragma unroll
    for (int q = 0; q < kWChunks; ++q)
      *reinterpret_cast<u32x4*>(b + kXBytes + 16 * (tid + kGwThreads * q)) = kFull ? wr[q] : (wr[q] & wkeep[q]);
  };
  float p[64];
  float z = 0.0f;
#pragma unroll
  for (int i = 0; i < 64; ++i) p[i] = 0.0f;
  load(0);
  store(0);
  __syncthreads();
  int done_segments = 0;
  for (int m = 0; m < steps; ++m) {
    // step m + 1 (the last step reloads itself: the loop body stays one
    // block, so the loads, the products and the stores keep their order)
    load(min(m + 1, steps - 1));
    asm volatile("" ::: "memory");   // the loads go out before this step's LDS reads
    const char* b = gw_lds + (m & 1) * kBuf;
    f32x4 xv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xv[i] = lds_f32x4<kXBF16>(b + (8 * wt + i) * 256 * kSx, lane);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const f32x4 wv = lds_f32x4<kWBF16>(b + kXBytes + (8 * we + j) * 256 * kSw, lane);
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          p[8 * i + j] = __builtin_fmaf(xv[i][v], wv[v], p[8 * i + j]);
        }
    }
    // the staged chunks are stored after the products, so their loads have
    // the whole step to arrive (the compiler would otherwise place the
    // stores, and the wait for the loads, above the products: the empty asm
    // statements take every partial, and the stores cannot pass the memory
    // clobber); after the last step they go to the buffer nobody reads any more
#pragma unroll
    for (int i = 0; i < 64; ++i) asm volatile("" : "+v"(p[i]));
    asm volatile("" ::: "memory");
    store((m + 1) & 1);
    if (m + 1 == steps || (m + 1) % seg == 0) {
      xor_reduce_scatter<64, 32>(p, lane);
      z = done_segments == 0 ? p[0] : z + p[0];
      ++done_segments;
#pragma unroll
      for (int i = 0; i < 64; ++i) p[i] = 0.0f;
    }
    __syncthreads();
  }
  for (int w = done_segments; w < kSegments; ++w) z = z + 0.0f;   // empty segments add +0
  const int t = t0 + 8 * wt + lane / 8, e = e0 + 8 * we + lane % 8;
  if (t < g.T && e < g.E) g.scores[static_cast<int64_t>(t) * g.E + e] = score_of(z, g.score_func);
}

template <bool kXBF16, bool kWBF16>
__global__ __launch_bounds__(kGwThreads, 4) void k_gate_wide(GateArgs g) {
  extern __shared__ __align__(16) char gw_lds[];
  const int n_et = (g.E + kGwExp - 1) / kGwExp;
  const int t0 = (blockIdx.x / n_et) * kGwTok, e0 = (blockIdx.x % n_et) * kGwExp;
  const int64_t xbytes = static_cast<int64_t>(g.T) * g.H * (kXBF16 ? 2 : 4);
  const int64_t wbytes = static_cast<int64_t>(g.E) * g.H * (kWBF16 ? 2 : 4);
  if (t0 + kGwTok <= g.T && e0 + kGwExp <= g.E && g.H % 256 == 0 && xbytes < (1ll << 31) && wbytes < (1ll << 31))
    gate_wide_tile<kXBF16, kWBF16, true>(g, gw_lds, t0, e0);
  else
    gate_wide_tile<kXBF16, kWBF16, false>(g, gw_lds, t0, e0);
}

hipError_t launch_gate_wide(const dsk_moe_desc& d, const GateArgs& g, hipStream_t s) {
  const unsigned blocks = static_cast<unsigned>(((d.tokens + kGwTok - 1) / kGwTok) *
                                                ((d.n_experts + kGwExp - 1) / kGwExp));
  const bool xb = d.x_dtype == DSK_DTYPE_BF16, wb = d.gate_dtype == DSK_DTYPE_BF16;
  const size_t lds = 2 * static_cast<size_t>(kGwTok * 256 * (xb ? 2 : 4) + kGwExp * 256 * (wb ? 2 : 4));
  if (xb && wb) launch_kernel(k_gate_wide<true, true>, blocks, kGwThreads, lds, s, g);
  else if (xb) launch_kernel(k_gate_wide<true, false>, blocks, kGwThreads, lds, s, g);
  else if (wb) launch_kernel(k_gate_wide<false, true>, blocks, kGwThreads, lds, s, g);
  else launch_kernel(k_gate_wide<false, false>, blocks, kGwThreads, lds, s, g);
  return hipGetLastError();
}

template <int TW, int EW, bool kFused>
hipError_t launch_gate(const dsk_moe_desc& d, const GateArgs& g, hipStream_t s) {
  const int n_et = (d.n_experts + EW - 1) / EW;
  const int n_tt = (d.tokens + TW - 1) / TW;
  const unsigned blocks = static_cast<unsigned>(n_et * n_tt);
  size_t lds = (kSegments * TW * EW + 4) * sizeof(float);
  if (kFused) lds += static_cast<size_t>(4 * d.n_experts + d.n_experts + 32) * sizeof(int32_t);
  static_assert(kFused || TW * EW > 16 || (kSegments * TW * EW + 4) * sizeof(float) <= kGateNormOffset,
                "segment sums before the rows (the residual form's one-token tiles)");
  const bool xb = d.x_dtype == DSK_DTYPE_BF16, wb = d.gate_dtype == DSK_DTYPE_BF16;
  if (g.norm) {
    // the residual form: one-token tiles of a bf16 stream only (resnorm_fusable)
    if constexpr (TW == 1 && EW == 1 && !kFused) {
      if (!xb) return hipErrorInvalidValue;
      lds = kGateNormOffset + static_cast<size_t>(d.tokens) * d.hidden * 2;
      if (wb) launch_kernel(k_gate<1, 1, true, true, false, true>, blocks, 256, lds, s, g);
      else launch_kernel(k_gate<1, 1, true, false, false, true>, blocks, 256, lds, s, g);
      return hipGetLastError();
    } else {
      return hipErrorInvalidValue;
    }
  }
  if (xb && wb) launch_kernel(k_gate<TW, EW, true, true, kFused>, blocks, 256, lds, s, g);
  else if (xb) launch_kernel(k_gate<TW, EW, true, false, kFused>, blocks, 256, lds, s, g);
  else if (wb) launch_kernel(k_gate<TW, EW, false, true, kFused>, blocks, 256, lds, s, g);
  else launch_kernel(k_gate<TW, EW, false, false, kFused>, blocks, 256, lds, s, g);
  return hipGetLastError();
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

// 16-127 tokens: tiles of 8 tokens x 4 experts (each expert's gate row read by
// half as many tiles as with 4 x 4: 64 tokens 13.8 -> 10.4 us; 4 x 8, 8 x 8,
// 16 x 4, 8 x 2 and 16 x 2 measured 12.1-17.6 us).
hipError_t launch_route_unfused(const dsk_moe_desc& d, const GateArgs& g, hipStream_t s) {
  hipError_t e = (d.tokens >= kGateWideMinTokens) ? launch_gate_wide(d, g, s)
                 : (d.tokens >= 16)              ? launch_gate<8, 4, false>(d, g, s)
                                                 : launch_gate<1, 1, false>(d, g, s);
  if (e != hipSuccess) return e;
  if ((e = stage_open(kStageRoute)) != hipSuccess) return e;
  const int64_t chunks = static_cast<int64_t>(d.tokens) * (d.hidden / 8);
  const unsigned blocks = static_cast<unsigned>((d.tokens + 3) / 4 + (g.xp ? (chunks + 255) / 256 : 0));
  launch_kernel(k_topk, blocks, 256, 0, s, g.scores, g.bias, d.tokens, d.n_experts, d.top_k, d.route_scale,
                g.idx, g.weights, static_cast<const uint16_t*>(g.x), d.hidden, g.xp, g.xform);
  return hipGetLastError();
}

// ---------------------------------------------------------------- union cap
// cap_union of the reference (src/deepseeker/mlx_forward.py:213-254) on the
// device routing of a lock-step batch, in place, one block.  idx / w arrive in
// the build's order (descending key per row); the reference works on its
// ascending-key order, so every order-dependent step walks a row's slots from
// j = k-1 down to 0.  Steps (float32, no contraction):
//   score[e]  sum of scores[t][e] over the rows t routed to e, rows ascending;
//   keep      the `budget` largest scores, ties to the lower expert id (the
//             reference's argpartition leaves exact ties unspecified);
//   rescue    a row with nothing kept keeps its largest weight (the first
//             maximum in the reference's order) unless strict;
//   weights   scale = rowsum(w) / (rowsum(kept w) + 1e-20), w' = kept w * scale,
//             with numpy's float32 pairwise row sum (< 8 terms one by one from
//             0; else 8 running sums of terms i, i+8, ... combined as
//             ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), then the tail one by one);
//   dropped slots get index -1.
// Nothing changes when the batch's union already fits the budget.
constexpr int kCapThreads = 1024;

__device__ __forceinline__ float numpy_row_sum(const float* v, int n) {
  // v in the reference's order
  if (n < 8) {
    float r = 0.0f;
    for (int i = 0; i < n; ++i) r = r + v[i];
    return r;
  }
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = v[j];
  int i = 8;
  for (; i < n - (n % 8); i += 8)
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = r[j] + v[i + j];
  float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  for (; i < n; ++i) res = res + v[i];
  return res;
}

__global__ __launch_bounds__(kCapThreads) void k_cap_union(const float* __restrict__ scores, int32_t* __restrict__ idx,
                                                           float* __restrict__ w, int T, int E, int k, int budget,
                                                           int strict) {
  extern __shared__ __align__(16) unsigned char lds_cap[];
  int32_t* li = reinterpret_cast<int32_t*>(lds_cap);                 // [T*k]
  float* sum = reinterpret_cast<float*>(li + T * k);                // [E]
  int32_t* cnt = reinterpret_cast<int32_t*>(sum + E);               // [E]
  uint8_t* keep = reinterpret_cast<uint8_t*>(cnt + E);              // [E]
  __shared__ int union_size;
  const int tid = threadIdx.x, N = T * k;
  for (int i = tid; i < N; i += kCapThreads) li[i] = idx[i];
  if (tid == 0) union_size = 0;
  __syncthreads();
  // per-expert score sums, rows ascending (an expert appears at most once per row)
  for (int e = tid; e < E; e += kCapThreads) {
    float s = 0.0f;
    int c = 0;
    for (int t = 0; t < T; ++t)
      for (int j = 0; j < k; ++j)
        if (li[t * k + j] == e) {
          s = s + scores[static_cast<int64_t>(t) * E + e];
          ++c;
        }
    sum[e] = s;
    cnt[e] = c;
    if (c > 0) atomicAdd(&union_size, 1);
  }
  __syncthreads();
  if (union_size <= budget) return;                 // the union fits: unchanged
  // rank by score (descending), ties to the lower id; keep the first `budget`
  for (int e = tid; e < E; e += kCapThreads) {
    const float se = sum[e];
    int rank = 0;
    for (int f = 0; f < E; ++f) {
      const float sf = sum[f];
      rank += (sf > se || (sf == se && f < e)) ? 1 : 0;
    }
    keep[e] = rank < budget ? 1 : 0;
  }
  __syncthreads();
  // rows: kept mask, rescue, renormalised weights (slots in the reference's order)
  for (int t = tid; t < T; t += kCapThreads) {
    float wr[16], kw[16];
    bool kept[16];
    bool any = false;
    for (int r = 0; r < k; ++r) {                   // r: reference slot = build slot k-1-r
      const int j = k - 1 - r;
      const int e = li[t * k + j];
      wr[r] = w[static_cast<int64_t>(t) * k + j];
      kept[r] = e >= 0 && e < E && keep[e];
      any = any || kept[r];
    }
    if (!any && !strict) {
      int best = 0;
      for (int r = 1; r < k; ++r)
        if (wr[r] > wr[best]) best = r;             // first maximum in the reference's order
      kept[best] = true;
    }
    for (int r = 0; r < k; ++r) kw[r] = kept[r] ? wr[r] : 0.0f;
    const float scale = numpy_row_sum(wr, k) / (numpy_row_sum(kw, k) + 1e-20f);
    for (int r = 0; r < k; ++r) {
      const int j = k - 1 - r;
      const int64_t o = static_cast<int64_t>(t) * k + j;
      w[o] = kw[r] * scale;
      if (!kept[r]) idx[o] = -1;
    }
  }
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
  g.xp = a.xp;
  g.xform = a.xform;
  if (a.rn) {
    g.rn = *a.rn;
    g.norm = 1;
  }
  return g;
}

hipError_t launch_route_dispatch(const dsk_moe_desc& d, const RouteArgs& a, hipStream_t s) {
  const GateArgs g = route_gate_args(d, a);
  if (d.tokens <= kFusedMaxTokens) {
    return d.tokens == 1 ? launch_gate<1, 4, true>(d, g, s) : launch_gate<4, 1, true>(d, g, s);
  }
  hipError_t e = launch_route_unfused(d, g, s);   // opens the route stage after the gate
  if (e != hipSuccess) return e;
  return launch_dispatch(d, a.idx, a.weights, a.table, a.out, s);
}

// Below 16 tokens one-token tiles stay the faster ones (8 tokens: 5.1 us against
// 8.0-9.2 us for 2 x 4, 4 x 4 and 8 x 4 tiles).
hipError_t launch_gate_scores(const dsk_moe_desc& d, const RouteArgs& a, hipStream_t s) {
  const GateArgs g = route_gate_args(d, a);
  return d.tokens >= 16 ? launch_gate<8, 4, false>(d, g, s) : launch_gate<1, 1, false>(d, g, s);
}

size_t cap_union_lds(int T, int E, int k) {
  return static_cast<size_t>(T) * k * 4 + static_cast<size_t>(E) * 9;
}

hipError_t launch_cap_union(const float* scores, int32_t* idx, float* w, int T, int E, int k, int budget,
                            int strict, hipStream_t s) {
  launch_kernel(k_cap_union, 1, kCapThreads, cap_union_lds(T, E, k), s, scores, idx, w, T, E, k, budget, strict);
  return hipGetLastError();
}

}  // namespace dsk
