// Token -> expert dispatch run by one workgroup (device code shared by the
// standalone dispatch kernel and the last block of the fused router).
//
// Same grouping as the reference's np.unique / row discovery in moe_layer
// (src/deepseeker/mlx_forward.py:294-312, 388-396) and the moe_align_block_size
// contract (src/deepseeker/moe_align.py:21-46): flat (token, slot) positions
// sorted by (expert, position).  S = blockDim.x / 64 waves; wave w owns a
// contiguous segment of positions.  Pass 1: per-wave histograms with LDS
// integer atomics (order free, result exact).  Scan: per expert a prefix
// over waves, then an exclusive scan over experts.  Pass 2 walks each
// segment in 64-position chunks, in order: lanes holding the same expert
// are found with one ballot per expert-id bit, ranked by popcount of the
// lower lanes; the highest such lane advances the (wave, expert) cursor,
// which keeps the permutation stable.  Besides counts / offsets / perm /
// rank / active it writes, for the expert kernels, one descriptor per
// active expert and the token and route weight of every dispatch row.
#pragma once

#include "dsk_internal.h"

namespace dsk {

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) {
    int o = __shfl_up(v, s, 64);
    if (lane >= s) v += o;
  }
  return v;
}

// Wave-wide max / min of a uint32 without LDS: DPP exchanges inside each
// 16-lane row (quad swaps, half-row mirror, row mirror leave every lane with
// its row's extreme), then the four rows' values through readlane.
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), kCtrl, 0xF, 0xF, false));
}
constexpr int kDppQuadSwap1 = 0xB1;    // quad_perm [1, 0, 3, 2]
constexpr int kDppQuadSwap2 = 0x4E;    // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppRowMirror = 0x140;   // row_mirror

__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int l) {
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), l));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<kDppQuadSwap1>(v));
  v = max(v, dpp_u32<kDppQuadSwap2>(v));
  v = max(v, dpp_u32<kDppHalfMirror>(v));
  v = max(v, dpp_u32<kDppRowMirror>(v));
  return max(max(readlane_u32(v, 0), readlane_u32(v, 16)), max(readlane_u32(v, 32), readlane_u32(v, 48)));
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, dpp_u32<kDppQuadSwap1>(v));
  v = min(v, dpp_u32<kDppQuadSwap2>(v));
  v = min(v, dpp_u32<kDppHalfMirror>(v));
  v = min(v, dpp_u32<kDppRowMirror>(v));
  return min(min(readlane_u32(v, 0), readlane_u32(v, 16)), min(readlane_u32(v, 32), readlane_u32(v, 48)));
}

// Chunks of 64 positions whose loads a wave issues together.
constexpr int kDispBatch = 8;

// LDS needed: (S * E + E + 32) int32.
__device__ __forceinline__ void dispatch_block(const int32_t* __restrict__ idx, int N, int E, int k,
                                               int nbits, const float* __restrict__ wflat,
                                               const dsk_expert_ptrs* __restrict__ table,
                                               const DispatchOut& o, int32_t* lds) {
  const int nthr = blockDim.x;
  const int S = nthr >> 6;
  int32_t* hist = lds;                         // [S][E]
  int32_t* base = lds + S * E;                 // [E]
  int32_t* wsum = base + E;                    // [16]
  int32_t* wflag = wsum + 16;                  // [16]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  for (int i = tid; i < S * E; i += nthr) hist[i] = 0;
  __syncthreads();

  const int seg = ((N + S - 1) / S + 63) & ~63;
  const int beg = min(wave * seg, N), end = min(beg + seg, N);
  // the segment is read kDispBatch chunks of 64 positions at a time, the loads
  // of a batch issued together (clamped into the segment, no conditions)
  for (int c0 = beg; c0 < end; c0 += 64 * kDispBatch) {
    int ev[kDispBatch];
#pragma unroll
    for (int j = 0; j < kDispBatch; ++j) ev[j] = idx[min(c0 + 64 * j + lane, end - 1)];
#pragma unroll
    for (int j = 0; j < kDispBatch; ++j) {
      const int e = ev[j];
      if (c0 + 64 * j + lane < end && e >= 0 && e < E) atomicAdd(&hist[wave * E + e], 1);
    }
  }
  __syncthreads();

  const int per = (E + nthr - 1) / nthr;
  const int e_beg = min(tid * per, E), e_end = min(e_beg + per, E);
  int run_cnt = 0, run_act = 0;
  for (int e = e_beg; e < e_end; ++e) {
    int r = 0;
    for (int w = 0; w < S; ++w) {
      const int c = hist[w * E + e];
      hist[w * E + e] = r;
      r += c;
    }
    o.counts[e] = r;
    base[e] = r;            // the count, until the scan below
    run_cnt += r;
    run_act += (r > 0);
  }
  const int ic = wave_incl_scan(run_cnt, lane);
  const int ia = wave_incl_scan(run_act, lane);
  if (lane == 63) { wsum[wave] = ic; wflag[wave] = ia; }
  __syncthreads();
  int off_c = 0, off_a = 0;
  for (int w = 0; w < wave; ++w) { off_c += wsum[w]; off_a += wflag[w]; }
  int xc = off_c + ic - run_cnt, xa = off_a + ia - run_act;
  for (int e = e_beg; e < e_end; ++e) {
    const int c = base[e];
    o.offsets[e] = xc;
    base[e] = xc;
    if (c > 0) {
      o.active[1 + xa] = e;
      if (o.desc) {
        SlotDesc d;
        d.e = e; d.n_tok = c; d.tok_base = xc; d.pad = 0;
        const dsk_expert_ptrs t = table[e];
        d.p[0] = t.w1; d.p[1] = t.s1; d.p[2] = t.b1;
        d.p[3] = t.w3; d.p[4] = t.s3; d.p[5] = t.b3;
        d.p[6] = t.w2; d.p[7] = t.s2; d.p[8] = t.b2;
        d.pad2 = nullptr;
        o.desc[xa] = d;
      }
      ++xa;
    }
    xc += c;
  }
  if (tid == nthr - 1) {
    o.offsets[E] = xc;
    o.active[0] = xa;
  }
  __syncthreads();

  const uint64_t lt = (lane == 0) ? 0ull : ((~0ull) >> (64 - lane));
  for (int cb = beg; cb < end; cb += 64 * kDispBatch) {
    int ev[kDispBatch];
    float wv[kDispBatch];
#pragma unroll
    for (int j = 0; j < kDispBatch; ++j) {
      const int pc = min(cb + 64 * j + lane, end - 1);
      ev[j] = idx[pc];
      wv[j] = o.xrow ? wflat[pc] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kDispBatch; ++j) {
      const int c0 = cb + 64 * j;
      if (c0 >= end) break;
      const int p = c0 + lane;
      const bool in = p < end;
      const int e = in ? ev[j] : -1;
      const bool ok = in && e >= 0 && e < E;
      uint64_t mask = __ballot(ok);
      for (int b = 0; b < nbits; ++b) {
        const bool bit = ok && ((e >> b) & 1);
        const uint64_t bb = __ballot(bit);
        mask &= bit ? bb : ~bb;
      }
      if (ok) {
        const int rk = __popcll(mask & lt);
        const int pos = base[e] + hist[wave * E + e] + rk;
        o.perm[pos] = p;
        o.rank[p] = pos;
        if (o.xrow) {
          o.xrow[pos] = p / k;
          o.wrow[pos] = wv[j];
        }
      } else if (in) {
        o.rank[p] = -1;
      }
      // the highest lane of each group advances the cursor (after every lane read it)
      __builtin_amdgcn_wave_barrier();
      if (ok && lane == 63 - __clzll(mask)) hist[wave * E + e] += __popcll(mask);
      __builtin_amdgcn_wave_barrier();
    }
  }
}

__host__ __device__ inline int bits_for(int E) {
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  return nbits;
}

}  // namespace dsk
