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

// Serial form: top-k of the T tokens (wave w: tokens w, w + waves, ...) from
// the gate scores, then the slot map in wave 0, into r.  With `publish` the block also
// writes the routing outputs of the layer (o): idx / weights, and for the
// expert kernels active, one descriptor per slot, rowmap, the row weights
// and rank.  ltab (ltab_words 8-byte words of LDS, or null) receives the
// whole pointer table, loaded together with the scores, when it fits there
// and in the block's registers; the descriptors then read it from LDS
// instead of making a dependent global load.  Contains two block barriers.
__device__ __forceinline__ void block_route_serial(BlockRoute& r, const float* scores, const float* bias,
                                                   int T, int E, int k, float route_scale,
                                                   const dsk_expert_ptrs* table, bool publish,
                                                   const DecodeRoute& o, uint64_t* ltab, int ltab_words) {
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

// Rank form, for batches whose (token, expert) pairs fit kRouteRankPairs and
// E <= the block's threads.  The serial form's selection is k rounds of two
// wave reductions each, one wave per token, and its slot map another chain of
// dependent LDS round trips in one wave: several microseconds of
// latency-bound code.  Here the same outcome follows from ranks:
//   1. each (token, expert) pair's ordered key (the serial form's: bits of
//      (score + bias) + 0, sign-folded, 0 reserved for none) and score into
//      LDS; thread e also loads table entry e (all of the block's loads go
//      out together);
//   2. rank of a pair = the number of keys of its token ahead of it in the
//      serial form's order (larger key first, lower id first among equal
//      keys).  A lane owns four consecutive pairs of a token and compares
//      them with a range of that token's keys (the waves of a token split
//      its keys; 16-byte broadcast reads, so each key read serves four
//      comparisons): keys of lower ids count when >= (compared > key - 1),
//      others when >, and equal keys inside the lane's own four come from
//      registers.  Partial counts meet in LDS (atomic adds);
//   3. thread e: the tokens whose rank of e is below k (a bit mask), the
//      j-th selection of each such token (j = the rank), and from wave
//      ballots its slot (experts below it with a token) and first dispatch
//      row (positions with a smaller expert), plus the waves' totals;
//   4. thread e writes slot e's descriptor (from its table entry), the rows
//      of its tokens in token order, their route weights (the serial form's
//      arithmetic and summation order) and the routing outputs of those
//      positions; a position without a selection (fewer than k nonzero keys)
//      gets idx -1 and rank -1 from the position's own thread.
// Outputs equal the serial form's bit for bit.  Three block barriers.
constexpr int kRouteRankPairs = 1024;
struct BlockRouteRank {
  uint32_t key[kRouteRankPairs];          // [t][Es] ordered key, 0: none (Es = E rounded up to 16)
  float score[kRouteRankPairs];           // [t][Es]
  int32_t rank[kRouteRankPairs];          // [t][Es]
  int32_t sel_e[kDecodeMaxPositions];     // expert of position t*k + j, -1 if none
  float sel_s[kDecodeMaxPositions];       // its score
  int32_t wtot[16][2];                    // per wave: experts with a token, dispatch rows
};

__device__ __forceinline__ uint32_t route_key_bits(float s, float b) {
#pragma clang fp contract(off)
  const float key = (s + b) + 0.0f;
  const uint32_t u = __float_as_uint(key);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ bool block_route_rank_fits(int T, int E, int nthr) {
  return E <= nthr && T <= 16 && T * ((E + 15) & ~15) <= kRouteRankPairs && T * ((E + 15) & ~15) <= 2 * nthr;
}

__device__ __forceinline__ void block_route_rank(BlockRouteRank& r, const float* scores, const float* bias,
                                                 int T, int E, int k, float route_scale,
                                                 const dsk_expert_ptrs* table, const DecodeRoute& o) {
#pragma clang fp contract(off)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nthr = static_cast<int>(blockDim.x);
  const int waves = nthr >> 6;
  const int Es = (E + 15) & ~15;   // row stride of the pair arrays
  const int NP = T * Es, N = T * k;
  // 1. keys and scores of this thread's pairs, the table entry of expert tid
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = tid + i * nthr;
    const int t = q / Es, e = q - t * Es;
    const bool v = q < NP && e < E;
    const float sc = v ? scores[static_cast<int64_t>(t) * E + e] : 0.0f;
    const uint32_t kb = v ? route_key_bits(sc, bias[e]) : 0u;
    if (q < NP) {
      r.key[q] = kb;
      r.score[q] = sc;
      r.rank[q] = 0;
    }
  }
  dsk_expert_ptrs te = {};
  if (tid < E) te = table[tid];
  for (int p = tid; p < N; p += nthr) {
    r.sel_e[p] = -1;
    r.sel_s[p] = 0.0f;
  }
  // (the table entry lands with the scores; waiting for it here keeps a wait
  // for every outstanding load out of the rank loop)
  asm volatile("" ::"v"(te.w1), "v"(te.s1), "v"(te.b1), "v"(te.w3), "v"(te.s3), "v"(te.b3), "v"(te.w2),
               "v"(te.s2), "v"(te.b2));
  __syncthreads();
  // 2. ranks: unit u = (token u / nb, pairs 256 (u % nb) .. + 255), `ways`
  // waves per unit splitting the token's key chunks (4 keys each)
  {
    const int nb = (Es + 255) >> 8, U = T * nb;
    const int ways = U <= waves ? waves / U : 1;
    const int nc = Es >> 2;
    for (int u = wave / ways; u < U && wave < (U <= waves ? U * ways : waves); u += (U <= waves ? U : waves)) {
      const int way = wave % ways;
      const int t = u / nb;
      const int own = ((u - t * nb) << 6) + lane;   // own chunk: pairs 4 own .. 4 own + 3
      if (4 * own >= Es) continue;
      const uint32_t* row = r.key + t * Es;
      const uint4 ok = *reinterpret_cast<const uint4*>(row + 4 * own);
      const uint32_t ov[4] = {ok.x, ok.y, ok.z, ok.w};
      const uint32_t om[4] = {ok.x - 1u, ok.y - 1u, ok.z - 1u, ok.w - 1u};
      int cnt[4] = {0, 0, 0, 0};
      if (way == 0) {
        // equal keys of lower ids inside the own chunk
#pragma unroll
        for (int i = 1; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < i; ++j) cnt[i] += ov[j] == ov[i];
      }
      const int c0 = way * nc / ways, c1 = (way + 1) * nc / ways;
#pragma unroll 4
      for (int c = c0; c < c1; ++c) {
        const uint4 sv = *reinterpret_cast<const uint4*>(row + 4 * c);
        const bool before = c < own;   // every key of the chunk has a lower id than the own four
        uint32_t th[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) th[i] = before ? om[i] : ov[i];
#pragma unroll
        for (int i = 0; i < 4; ++i) cnt[i] += (sv.x > th[i]) + (sv.y > th[i]) + (sv.z > th[i]) + (sv.w > th[i]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) atomicAdd(&r.rank[t * Es + 4 * own + i], cnt[i]);
    }
  }
  __syncthreads();
  // 3. per expert: its tokens (their j-th selection: j = rank), slot and
  // first row within the wave
  uint32_t mask = 0u;
  if (tid < E) {
    for (int t = 0; t < T; ++t) {
      const int q = t * Es + tid;
      const int j = r.rank[q];
      if (r.key[q] != 0u && j < k) {
        mask |= 1u << t;
        r.sel_e[t * k + j] = tid;
        r.sel_s[t * k + j] = r.score[q];
      }
    }
  }
  const int cnt = __popc(mask);
  const uint64_t lt = (1ull << lane) - 1ull;
  const uint64_t has = __ballot(cnt > 0);
  const int slot_in = __popcll(has & lt);
  int row_in = 0, row_tot = 0;
#pragma unroll
  for (int b = 0; b < 5; ++b) {   // cnt <= 16
    const uint64_t bb = __ballot((cnt >> b) & 1);
    row_in += __popcll(bb & lt) << b;
    row_tot += __popcll(bb) << b;
  }
  if (lane == 0) {
    r.wtot[wave][0] = __popcll(has);
    r.wtot[wave][1] = row_tot;
  }
  __syncthreads();
  // 4. slot and rows of expert tid, the routing outputs
  int slot_base = 0, row_base = 0, n_act = 0;
  for (int w = 0; w < waves; ++w) {
    const int a = r.wtot[w][0], b = r.wtot[w][1];
    if (w < wave) { slot_base += a; row_base += b; }
    n_act += a;
  }
  if (tid == 0) o.active[0] = n_act;
  auto weight = [&](int t, float s) {
    float acc = 0.0f;   // the selection's scores in order, as the serial form
    for (int j = 0; j < k; ++j) acc = acc + r.sel_s[t * k + j];
    return (s / (acc + 1e-20f)) * route_scale;
  };
  if (cnt > 0) {
    const int s = slot_base + slot_in, rb = row_base + row_in;
    SlotDesc d;
    d.e = tid; d.n_tok = cnt; d.tok_base = rb; d.pad = 0;
    d.p[0] = te.w1; d.p[1] = te.s1; d.p[2] = te.b1;
    d.p[3] = te.w3; d.p[4] = te.s3; d.p[5] = te.b3;
    d.p[6] = te.w2; d.p[7] = te.s2; d.p[8] = te.b2;
    d.pad2 = nullptr;
    o.desc[s] = d;
    o.active[1 + s] = tid;
    int row = rb;
    for (int t = 0; t < T; ++t) {
      if (!((mask >> t) & 1u)) {
        o.rowmap[s * T + t] = -1;
        continue;
      }
      const int j = r.rank[t * Es + tid];
      const float w = weight(t, r.sel_s[t * k + j]);
      o.rowmap[s * T + t] = row;
      o.xrow[row] = t;
      o.wrow[row] = w;
      o.rank[t * k + j] = row;
      o.idx[t * k + j] = tid;
      o.weights[t * k + j] = w;
      ++row;
    }
  }
  for (int p = tid; p < N; p += nthr) {
    if (r.sel_e[p] < 0) {
      const int t = p / k;
      o.idx[p] = -1;
      o.weights[p] = weight(t, 0.0f);
      o.rank[p] = -1;
    }
  }
  __syncthreads();
}

// Top-k and slot map of the decode batch: the rank form where it fits, else
// the serial form.  lds holds either form's state (block_route_lds_bytes).
__device__ __forceinline__ void block_route(void* lds, const float* scores, const float* bias, int T, int E,
                                            int k, float route_scale, const dsk_expert_ptrs* table,
                                            const DecodeRoute& o, uint64_t* ltab, int ltab_words) {
  if (block_route_rank_fits(T, E, static_cast<int>(blockDim.x)))
    block_route_rank(*static_cast<BlockRouteRank*>(lds), scores, bias, T, E, k, route_scale, table, o);
  else
    block_route_serial(*static_cast<BlockRoute*>(lds), scores, bias, T, E, k, route_scale, table, true, o, ltab,
                       ltab_words);
}

constexpr size_t kBlockRouteLds = sizeof(BlockRoute) > sizeof(BlockRouteRank) ? sizeof(BlockRoute)
                                                                               : sizeof(BlockRouteRank);

}  // namespace dsk
