// Standalone token -> expert dispatch: one workgroup (dispatch_block, the
// grouping the fused router also runs in its last block), or for many
// positions the same grouping over several workgroups in three kernels.
#include "dispatch_block.h"

namespace dsk {
namespace {

__global__ __launch_bounds__(1024) void k_dispatch(const int32_t* __restrict__ idx, int N, int E,
                                                   int k, int nbits, const float* __restrict__ wflat,
                                                   const dsk_expert_ptrs* __restrict__ table,
                                                   DispatchOut o) {
  extern __shared__ int32_t lds[];
  dispatch_block(idx, N, E, k, nbits, wflat, table, o, lds);
}

// Multi-block form.  Block b takes positions [b C, (b + 1) C) (C =
// kDispBlockPositions), its wave w the 128 positions b C + 128 w ..; the
// positions are ordered by (block, wave, position), so a per-(block, wave)
// cursor that starts at the expert's offset plus the counts of every earlier
// block and of the block's earlier waves, and advances in position order,
// gives the stable order of dispatch_block.
constexpr int kDispWaves = 16;
constexpr int kDispWavePositions = kDispBlockPositions / kDispWaves;   // 128
static_assert(kDispWavePositions == 128, "two 64-position chunks per wave");

// Per-wave expert counts of block b's positions into lh[16][E].
__device__ __forceinline__ void disp_wave_counts(const int32_t* __restrict__ idx, int N, int E, int32_t* lh) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < kDispWaves * E; i += kDispWaves * 64) lh[i] = 0;
  __syncthreads();
  const int p0 = blockIdx.x * kDispBlockPositions + wave * kDispWavePositions;
  int ev[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) ev[j] = idx[min(p0 + 64 * j + lane, N - 1)];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e = ev[j];
    if (p0 + 64 * j + lane < N && e >= 0 && e < E) atomicAdd(&lh[wave * E + e], 1);
  }
  __syncthreads();
}

// 1. per-block expert counts -> hist[b][e]
__global__ __launch_bounds__(kDispWaves * 64) void k_disp_count(const int32_t* __restrict__ idx, int N, int E,
                                                                int32_t* __restrict__ hist) {
  extern __shared__ int32_t lh[];   // [16][E]
  disp_wave_counts(idx, N, E, lh);
  int32_t* out = hist + static_cast<size_t>(blockIdx.x) * E;
  for (int e = threadIdx.x; e < E; e += kDispWaves * 64) {
    int c = 0;
    for (int w = 0; w < kDispWaves; ++w) c += lh[w * E + e];
    out[e] = c;
  }
}

// 2. one block, thread e = expert e (E <= 1024): hist[.][e] becomes the
// exclusive prefix over blocks; counts, offsets (exclusive scan over
// experts), the active list and one descriptor per active expert.
__global__ __launch_bounds__(1024) void k_disp_scan(int n_seg, int E, const dsk_expert_ptrs* __restrict__ table,
                                                    DispatchOut o) {
  __shared__ int32_t wsum[16], wflag[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int e = tid;
  int cnt = 0;
  if (e < E) {
    constexpr int kB = 16;   // loads issued together
    for (int q0 = 0; q0 < n_seg; q0 += kB) {
      int c[kB];
#pragma unroll
      for (int j = 0; j < kB; ++j) c[j] = o.hist[static_cast<size_t>(min(q0 + j, n_seg - 1)) * E + e];
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        if (q0 + j < n_seg) {
          o.hist[static_cast<size_t>(q0 + j) * E + e] = cnt;
          cnt += c[j];
        }
      }
    }
    o.counts[e] = cnt;
  }
  const int act = cnt > 0 ? 1 : 0;
  const int ic = wave_incl_scan(cnt, lane);
  const int ia = wave_incl_scan(act, lane);
  if (lane == 63) { wsum[wave] = ic; wflag[wave] = ia; }
  __syncthreads();
  int off_c = 0, off_a = 0, tot_c = 0, tot_a = 0;
  for (int w = 0; w < 16; ++w) {
    off_c += w < wave ? wsum[w] : 0;
    off_a += w < wave ? wflag[w] : 0;
    tot_c += wsum[w];
    tot_a += wflag[w];
  }
  const int xc = off_c + ic - cnt, xa = off_a + ia - act;
  if (e < E) {
    o.offsets[e] = xc;
    if (act) {
      o.active[1 + xa] = e;
      if (o.desc) {
        SlotDesc d;
        d.e = e; d.n_tok = cnt; d.tok_base = xc; d.pad = 0;
        const dsk_expert_ptrs t = table[e];
        d.p[0] = t.w1; d.p[1] = t.s1; d.p[2] = t.b1;
        d.p[3] = t.w3; d.p[4] = t.s3; d.p[5] = t.b3;
        d.p[6] = t.w2; d.p[7] = t.s2; d.p[8] = t.b2;
        d.pad2 = nullptr;
        o.desc[xa] = d;
      }
    }
  }
  if (tid == 0) {
    o.offsets[E] = tot_c;
    o.active[0] = tot_a;
  }
}

// 3. the block counts its waves again, and each wave walks its 128 positions
// in order (as dispatch_block's second pass) with cursors offsets[e] +
// hist[b][e] + the counts of the block's earlier waves.
__global__ __launch_bounds__(kDispWaves * 64) void k_disp_scatter(const int32_t* __restrict__ idx, int N, int E,
                                                                  int k, int nbits,
                                                                  const float* __restrict__ wflat,
                                                                  DispatchOut o) {
  extern __shared__ int32_t cur[];   // [16][E]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  disp_wave_counts(idx, N, E, cur);
  const int32_t* hb = o.hist + static_cast<size_t>(blockIdx.x) * E;
  for (int e = tid; e < E; e += kDispWaves * 64) {
    int r = o.offsets[e] + hb[e];
    for (int w = 0; w < kDispWaves; ++w) {
      const int c = cur[w * E + e];
      cur[w * E + e] = r;
      r += c;
    }
  }
  __syncthreads();
  const int p0 = blockIdx.x * kDispBlockPositions + wave * kDispWavePositions;
  int ev[2];
  float wv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int pc = min(p0 + 64 * j + lane, N - 1);
    ev[j] = idx[pc];
    wv[j] = o.xrow ? wflat[pc] : 0.0f;
  }
  const uint64_t lt = (lane == 0) ? 0ull : ((~0ull) >> (64 - lane));
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int p = p0 + 64 * j + lane;
    const bool in = p < N;
    const int e = in ? ev[j] : -1;
    const bool ok = in && e >= 0 && e < E;
    uint64_t mask = __ballot(ok);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = ok && ((e >> b) & 1);
      const uint64_t bb = __ballot(bit);
      mask &= bit ? bb : ~bb;
    }
    if (ok) {
      const int pos = cur[wave * E + e] + __popcll(mask & lt);
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
    if (ok && lane == 63 - __clzll(mask)) cur[wave * E + e] += __popcll(mask);
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace

hipError_t launch_dispatch(const dsk_moe_desc& d, const int32_t* idx, const float* wflat,
                           const dsk_expert_ptrs* table, const DispatchOut& o, hipStream_t s) {
  const int E = d.n_experts;
  const int N = d.tokens * d.top_k;
  if (o.hist && dispatch_hist_ints(N, E) > 0) {
    const int nblk = (N + kDispBlockPositions - 1) / kDispBlockPositions;
    const size_t lds = static_cast<size_t>(kDispWaves) * E * sizeof(int32_t);
    launch_kernel(k_disp_count, nblk, kDispWaves * 64, lds, s, idx, N, E, o.hist);
    launch_kernel(k_disp_scan, 1, 1024, 0, s, nblk, E, table, o);
    launch_kernel(k_disp_scatter, nblk, kDispWaves * 64, lds, s, idx, N, E, d.top_k, bits_for(E), wflat, o);
    return hipGetLastError();
  }
  const int S = (E <= 512) ? 16 : 8;
  const size_t lds = static_cast<size_t>(S * E + E + 32) * sizeof(int32_t);
  launch_kernel(k_dispatch, 1, S * 64, lds, s, idx, N, E, d.top_k, bits_for(E), wflat, table, o);
  return hipGetLastError();
}

}  // namespace dsk
