// Top-k and slot map of a decode batch in one workgroup.
//
// The decode kernels need, per active expert (slot), its weight pointers and
// the dispatch row of each token routed to it, and per dispatch row its route
// weight.  For at most kDecodeMaxTokens tokens and kDecodeMaxPositions
// positions one workgroup derives them from the gate scores: one wave per
// token for the biased top-k, then one wave for the slot map.  The numbering
// is the dispatch's (src/deepseeker/mlx_forward.py:294-312): slots are the
// selected experts in ascending id, and dispatch rows are the flat positions
// t*k + j sorted by (expert, position), as the dispatch kernel numbers them.
#pragma once

#include "gate.h"

namespace dsk {

struct BlockRoute {
  int32_t key[kDecodeMaxPositions];      // expert of flat position t*k + j
  float w[kDecodeMaxPositions];          // its route weight
  int32_t sorted[kDecodeMaxPositions];   // expert at each sorted position (E past the valid ones)
  int32_t slot_e[kDecodeMaxPositions];   // expert of slot s
  float row_w[kDecodeMaxPositions];      // route weight of dispatch row r
  int32_t n_act, pad[3];
  int32_t rmap[kDecodeMaxPositions * kDecodeMaxTokens];   // [slot][token] dispatch row, -1 if none
};

// 8-byte words of the expert pointer table each thread prefetches into LDS.
constexpr int kRouteTabWords = 5;
constexpr int kTabWordsPerExpert = static_cast<int>(sizeof(dsk_expert_ptrs) / 8);
static_assert(sizeof(dsk_expert_ptrs) % 8 == 0, "pointer table entries are whole 8-byte words");

// Wait for the wave's LDS operations only (s_waitcnt lgkmcnt(0); vmcnt and
// expcnt at their maxima), so LDS hand-offs inside wave 0 do not also wait
// for the acknowledgement of the global stores issued before them.
__device__ __forceinline__ void wait_lds_only() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Top-k of the T tokens (wave w: tokens w, w + waves, ...) from the gate
// scores, then the slot map in wave 0, into r.  With `publish` the block also
// writes the routing outputs of the layer (o): idx / weights, and for the
// expert kernels active, one descriptor per slot, rowmap, the row weights
// and rank.  ltab (ltab_words 8-byte words of LDS, or null) receives the
// whole pointer table, loaded together with the scores, when it fits there
// and in the block's registers; the descriptors then read it from LDS
// instead of making a dependent global load.  Contains two block barriers.
__device__ __forceinline__ void block_route(BlockRoute& r, const float* scores, const float* bias, int T,
                                            int E, int k, float route_scale, const dsk_expert_ptrs* table,
                                            bool publish, const DecodeRoute& o, uint64_t* ltab,
                                            int ltab_words) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int waves = blockDim.x >> 6;
  const int nthr = static_cast<int>(blockDim.x);
  const int nq = E * kTabWordsPerExpert;
  const bool tab = publish && ltab != nullptr && nq <= ltab_words && nq <= kRouteTabWords * nthr;
  uint64_t tq[kRouteTabWords];
  if (tab) {
    // no conditions on the loads: words past the table re-read its last word
    const uint64_t* tg = reinterpret_cast<const uint64_t*>(table);
#pragma unroll
    for (int i = 0; i < kRouteTabWords; ++i) tq[i] = tg[min(tid + i * nthr, nq - 1)];
  }
  for (int t = wave; t < T; t += waves)
    topk_token(scores + static_cast<int64_t>(t) * E, bias, E, k, route_scale,
               publish ? o.idx + static_cast<int64_t>(t) * k : nullptr,
               publish ? o.weights + static_cast<int64_t>(t) * k : nullptr, r.key + t * k, r.w + t * k);
  if (tab) {
#pragma unroll
    for (int i = 0; i < kRouteTabWords; ++i)
      if (tid + i * nthr < nq) ltab[tid + i * nthr] = tq[i];
  }
  __syncthreads();
  if (wave == 0) {
    const int N = T * k;
    const int e_in = lane < N ? r.key[lane] : -1;
    const bool ok = lane < N && e_in >= 0 && e_in < E;
    const int key = ok ? e_in : E;
    int pos = 0;
    for (int j = 0; j < N; ++j) {
      const int kj = __builtin_amdgcn_readlane(key, j);
      pos += (kj < key) || (kj == key && j < lane);
    }
    const int n_valid = __popcll(__ballot(ok));
    if (lane < N) r.sorted[pos] = key;
    else r.sorted[lane] = E;
    __builtin_amdgcn_wave_barrier();
    wait_lds_only();
    __builtin_amdgcn_wave_barrier();
    const int se = r.sorted[lane];
    const bool first = lane < n_valid && (lane == 0 || r.sorted[lane - 1] != se);
    const uint64_t firsts = __ballot(first);
    const uint64_t le = (lane == 63) ? ~0ull : ((1ull << (lane + 1)) - 1ull);
    const int n_act = __popcll(firsts);
    const int slot_here = __popcll(firsts & le) - 1;
    if (first) {
      r.slot_e[slot_here] = se;
      if (publish) {
        const uint64_t above = (lane == 63) ? 0ull : (firsts & ~le);
        const int next = above ? __builtin_ctzll(above) : n_valid;
        SlotDesc d;
        d.e = se; d.n_tok = next - lane; d.tok_base = lane; d.pad = 0;
        dsk_expert_ptrs t;
        if (tab) t = reinterpret_cast<const dsk_expert_ptrs*>(ltab)[se];
        else t = table[se];
        d.p[0] = t.w1; d.p[1] = t.s1; d.p[2] = t.b1;
        d.p[3] = t.w3; d.p[4] = t.s3; d.p[5] = t.b3;
        d.p[6] = t.w2; d.p[7] = t.s2; d.p[8] = t.b2;
        d.pad2 = nullptr;
        o.desc[slot_here] = d;
        o.active[1 + slot_here] = se;
      }
    }
    if (lane == 0) {
      r.n_act = n_act;
      if (publish) o.active[0] = n_act;
    }
    for (int i = lane; i < n_act * T; i += 64) r.rmap[i] = -1;
    __builtin_amdgcn_wave_barrier();
    wait_lds_only();
    __builtin_amdgcn_wave_barrier();
    const int my_slot = __shfl(slot_here, pos & 63, 64);
    if (ok) {
      r.rmap[my_slot * T + lane / k] = pos;
      r.row_w[pos] = r.w[lane];
      if (publish) {
        o.wrow[pos] = r.w[lane];
        o.xrow[pos] = lane / k;
      }
    }
    if (publish && lane < N) o.rank[lane] = ok ? pos : -1;
    if (publish) {
      __builtin_amdgcn_wave_barrier();
      wait_lds_only();
      __builtin_amdgcn_wave_barrier();
      for (int i = lane; i < n_act * T; i += 64) o.rowmap[i] = r.rmap[i];
    }
  }
  __syncthreads();
}

}  // namespace dsk
