// Token -> expert dispatch: per-expert counts, exclusive offsets, the stable
// permutation of flat (token, slot) positions by expert, its inverse, and the
// ascending list of active experts.
//
// Replaces the host-side np.unique / row discovery of the reference's
// moe_layer (src/deepseeker/mlx_forward.py:294-312, 388-396) and states the
// same grouping as the moe_align_block_size contract
// (src/deepseeker/moe_align.py:21-46): positions sorted by (expert, position).
//
// One workgroup of S waves.  Wave w owns a contiguous segment of positions.
// Pass 1 builds per-wave histograms with LDS integer atomics (order free,
// result exact); the histograms are turned into per-(wave, expert) bases by
// a prefix over waves and an exclusive scan over experts.  Pass 2 walks each
// segment in 64-position chunks, in order: lanes holding the same expert are
// found with one ballot per expert-id bit, ranked by popcount of the lower
// lanes, and the highest such lane advances the (wave, expert) cursor, which
// keeps the permutation stable.
#include "dsk_internal.h"

namespace dsk {
namespace {

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) {
    int o = __shfl_up(v, s, 64);
    if (lane >= s) v += o;
  }
  return v;
}

__global__ __launch_bounds__(1024) void k_dispatch(const int32_t* __restrict__ idx, int N, int E,
                                                   int nbits, int32_t* __restrict__ counts,
                                                   int32_t* __restrict__ offsets,
                                                   int32_t* __restrict__ perm,
                                                   int32_t* __restrict__ rank,
                                                   int32_t* __restrict__ active) {
  extern __shared__ int32_t lds[];
  const int nthr = blockDim.x;
  const int S = nthr >> 6;                     // waves
  int32_t* hist = lds;                         // [S][E]
  int32_t* base = lds + S * E;                 // [E] exclusive offsets
  int32_t* wsum = base + E;                    // [S] wave totals for scans
  int32_t* wflag = wsum + 16;                  // [S]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  for (int i = tid; i < S * E; i += nthr) hist[i] = 0;
  __syncthreads();

  const int seg = ((N + S - 1) / S + 63) & ~63;
  const int beg = min(wave * seg, N), end = min(beg + seg, N);
  for (int p = beg + lane; p < end; p += 64) {
    const int e = idx[p];
    if (e >= 0 && e < E) atomicAdd(&hist[wave * E + e], 1);
  }
  __syncthreads();

  // Per expert: prefix over waves; per thread: a run of consecutive experts.
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
    counts[e] = r;
    base[e] = r;            // temporarily the count
    run_cnt += r;
    run_act += (r > 0);
  }
  // Block-wide exclusive scan of (run_cnt, run_act) over threads.
  int ic = wave_incl_scan(run_cnt, lane);
  int ia = wave_incl_scan(run_act, lane);
  if (lane == 63) { wsum[wave] = ic; wflag[wave] = ia; }
  __syncthreads();
  int off_c = 0, off_a = 0;
  for (int w = 0; w < wave; ++w) { off_c += wsum[w]; off_a += wflag[w]; }
  int xc = off_c + ic - run_cnt, xa = off_a + ia - run_act;
  for (int e = e_beg; e < e_end; ++e) {
    const int c = base[e];
    offsets[e] = xc;
    base[e] = xc;
    if (c > 0) active[1 + xa++] = e;
    xc += c;
  }
  if (tid == nthr - 1) {
    offsets[E] = xc;
    active[0] = xa;
  }
  __syncthreads();

  // Pass 2: stable scatter.
  const uint64_t lt = (lane == 0) ? 0ull : ((~0ull) >> (64 - lane));
  for (int c0 = beg; c0 < end; c0 += 64) {
    const int p = c0 + lane;
    const bool in = p < end;
    const int e = in ? idx[p] : -1;
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
      perm[pos] = p;
      rank[p] = pos;
    } else if (in) {
      rank[p] = -1;
    }
    // the highest lane of each group advances the cursor (after every lane read it)
    __builtin_amdgcn_wave_barrier();
    if (ok && lane == 63 - __clzll(mask)) hist[wave * E + e] += __popcll(mask);
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace

hipError_t launch_dispatch(const dsk_moe_desc& d, const int32_t* idx, int32_t* counts,
                           int32_t* offsets, int32_t* perm, int32_t* rank, int32_t* active,
                           hipStream_t s) {
  const int E = d.n_experts;
  const int N = d.tokens * d.top_k;
  const int S = (E <= 512) ? 16 : 8;
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  const size_t lds = static_cast<size_t>(S * E + E + 32) * sizeof(int32_t);
  k_dispatch<<<1, S * 64, lds, s>>>(idx, N, E, nbits, counts, offsets, perm, rank, active);
  return hipGetLastError();
}

}  // namespace dsk
