// Grouped expert products for medium batches (a few to a few dozen tokens).
//
// Replaces the per-expert gate/up and w2 products of the reference's
// moe_layer (src/deepseeker/mlx_forward.py:388-406) and its shared expert
// (src/deepseeker/mlx_runner.py:765-783) when each active expert sees only a
// handful of tokens: every expert's weights must be streamed from HBM once,
// and the MFMA B operand (16 columns) is mostly empty.  A block takes one
// slot (an active expert, or the shared expert as a pseudo-slot over all T
// tokens) and a group of row tiles; it walks the slot's dispatch rows in
// column tiles of kGNC.  For each column tile the block gathers only that
// tile's activation rows into LDS (x for gate/up, the h planes for down), the
// waves issue their first weight batches behind those loads (not in front of
// them, where the LDS stores would wait for the weights too), and each wave
// then multiplies its K range; K ranges are added in a fixed
// order through LDS.  Gate/up writes h = SwiGLU(gate, up) * route weight by
// dispatch row (hs by token for the shared expert); down writes one float32
// output row per dispatch row (ys per token for the shared expert), which
// the combine kernel adds in ascending expert id.
#include "mx.h"

namespace dsk {
namespace {

constexpr int kGI = 2;              // gate/up: row tiles of a block
constexpr int kGKS = 4;             // gate/up: K ranges of a row tile (one wave each)
constexpr int kGW = kGI * kGKS;     // waves of a gate/up block
constexpr int kDI = 8;              // down: row tiles of a block
constexpr int kDKS = 1;             // down: K ranges of a row tile
constexpr int kDW = kDI * kDKS;     // waves of a down block
constexpr int kGNC = 8;             // dispatch rows (B columns) of a column tile
constexpr int kDnRingFP4 = 4;       // down: FP4 weight batches in flight per wave

static_assert(kGW == kDW, "both kernels use the same block size");

struct GroupedArgs {
  int T, H, I, Is, k;
  float limit;
  const SlotDesc* desc; const int32_t* active;   // active[0] = number of descriptors
  const int32_t* xrow; const float* wrow;        // per dispatch row: token, route weight
  const uint16_t* x;                             // [T][H] bf16
  const uint16_t* ws1; const uint16_t* ws3;      // shared [Is][H] bf16
  const uint16_t* ws2;                           // shared [H][Is] bf16
  uint16_t* h_hi; uint16_t* h_lo;                // [T*k][I] by dispatch row
  uint16_t* hs_hi; uint16_t* hs_lo;              // [T][Is]
  float* y;                                      // [T*k][H]
  float* ys;                                     // [T][H]
  int up_groups, up_shared;                      // gate/up: row-tile groups per slot, shared blocks
  int dn_groups, dn_shared;                      // down: the same
  int q3f;                                       // q3 gate/up in the factored form (up_block_q3f)
  int q3fd;                                      // q3 down in the factored form (down_block_q3f)
  int mx;                                        // FP4 gate/up on scaled MFMAs: blocks per wave, or 0
  uint8_t* xp;                                   // mx: x as FP8 planes [T][2][H], then E8M0 [T][2][H/32]
  int hplanes;                                   // FP4 slots' h as FP8 planes, the down on scaled MFMAs
  uint8_t* hp;                                   // hplanes: [T*k][3][I], then E8M0 [T*k][3][I/32]
};

// K blocks per weight batch, two batches in flight per wave, within the
// register budget of four waves per SIMD: one for bf16 rows (64 bytes per
// lane and K block) and for q3 (20 bytes, but its dequantisation needs many
// temporaries), two for FP4 (20 bytes).
template <typename Raw>
constexpr int batch_blocks() { return std::is_same_v<Raw, RawFP4> ? 2 : 1; }
// Weight batches in flight per wave in the down kernel.
template <typename Raw>
constexpr int down_ring() { return std::is_same_v<Raw, RawFP4> ? kDnRingFP4 : 2; }

// Rows [c0, c0 + cols) of the slot's activations (row r comes from source row
// src(r) of `base`, row stride `ld` elements, K elements) into LDS rows of
// stride K + 8, Q chunks per thread in flight per pass.
template <int Q, typename Src>
__device__ __forceinline__ void stage_rows_q(uint16_t* dst, const uint16_t* base, int ld, int K, int cols,
                                             Src src) {
  const int cpr = K / 8, chunks = cols * cpr, nt = blockDim.x;
  for (int c = threadIdx.x; c < chunks; c += Q * nt) {
    u32x4 v[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int cc = min(c + q * nt, chunks - 1);   // no condition on the load (see load_raw_nc)
      v[q] = ldg16(base + static_cast<int64_t>(src(cc / cpr)) * ld + (cc % cpr) * 8);
    }
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int cc = c + q * nt;
      if (cc < chunks) *reinterpret_cast<u32x4*>(dst + (cc / cpr) * (K + 8) + (cc % cpr) * 8) = v[q];
    }
  }
}

// Up to two chunks per thread: one pass of two; more: passes of four (a pass
// is a round trip; four chunks where two would do cost their issue slots).
template <typename Src>
__device__ __forceinline__ void stage_rows(uint16_t* dst, const uint16_t* base, int ld, int K, int cols,
                                           Src src) {
  if (cols * (K / 8) <= 2 * static_cast<int>(blockDim.x)) stage_rows_q<2>(dst, base, ld, K, cols, src);
  else stage_rows_q<4>(dst, base, ld, K, cols, src);
}

// Gate/up of one block: row tile rt (rows 16 rt ..) of w1 and w3 for the n
// dispatch rows base .. base + n - 1 (shared: tokens 0 .. n - 1).
template <typename Raw, typename LoadW, typename WPtr>
__device__ __forceinline__ void up_block(const GroupedArgs& p, LoadW load_w, WPtr wptr, int rt, bool rok, int n,
                                         int base, bool shared, uint16_t* lds) {
  constexpr int G = batch_blocks<Raw>();
  const int lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int item = wave / kGKS, ks = wave % kGKS;
  const int K = p.H, nblk = K / 128;
  const int per = (nblk + kGKS - 1) / kGKS;
  const int k0 = min(ks * per, nblk), k1 = min(k0 + per, nblk);
  const int xs = K + 8;
  const uint32_t row = static_cast<uint32_t>(rt * 16 + r16);
  float (*red)[kGKS][2][64][4] = reinterpret_cast<float (*)[kGKS][2][64][4]>(lds);   // over the x tile
  for (int c0 = 0; c0 < n; c0 += kGNC) {
    const int cols = min(kGNC, n - c0);
    Raw a1[G], a3[G], b1[G], b3[G];
    // FP4: each role's scales of a batch's 2 blocks (all lane groups) as one
    // 8-byte window instead of one byte per lane and block (picked at use)
    u32x2 wa1{}, wa3{}, wb1{}, wb3{};
    // no condition on the loads (see load_raw_nc): rows past the tile read
    // row 0, blocks past the range the range's last block (not computed)
    auto ld = [&](Raw (&r1)[G], Raw (&r3)[G], u32x2& w1, u32x2& w3, int kb) {
      const uint32_t rw = rok ? row : 0u;
      if constexpr (std::is_same_v<Raw, RawFP4> && G == 2) {
        const int kbc = min(kb, k1 - 2);   // every range has an even number of blocks
        const uint32_t co = rw * static_cast<uint32_t>(K / 2) + g4 * 16, so = rw * static_cast<uint32_t>(K / 32) + kbc * 4;
#pragma unroll
        for (int i = 0; i < G; ++i) {
          r1[i].c = ldg16(static_cast<const uint8_t*>(wptr(0)) + co + (kbc + i) * 64);
          r3[i].c = ldg16(static_cast<const uint8_t*>(wptr(3)) + co + (kbc + i) * 64);
        }
        w1 = ldg<u32x2>(static_cast<const uint8_t*>(wptr(1)) + so);
        w3 = ldg<u32x2>(static_cast<const uint8_t*>(wptr(4)) + so);
      } else {
#pragma unroll
        for (int i = 0; i < G; ++i) {
          const int kc = min(kb + i, k1 - 1) * 128 + g4 * 32;
          load_w(r1[i], 0, rw, kc);
          load_w(r3[i], 1, rw, kc);
        }
      }
    };
    // the tile's activation rows first: their loads are then not queued behind the
    // weights', so the LDS stores and the barrier do not wait for the weights
    if (shared) stage_rows(lds, p.x, K, K, cols, [&](int r) { return c0 + r; });
    else stage_rows(lds, p.x, K, K, cols, [&](int r) { return p.xrow[base + c0 + r]; });
    ld(a1, a3, wa1, wa3, k0);
    ld(b1, b3, wb1, wb3, k0 + G);
    __syncthreads();
    const bool tv = r16 < cols;
    const uint16_t* brow = lds + (tv ? r16 : 0) * xs;
    f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = ag;
    auto mm = [&](Raw (&r1)[G], Raw (&r3)[G], const u32x2& w1, const u32x2& w3, int kb) {
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int kc = (kb + i) * 128 + g4 * 32;
        if constexpr (std::is_same_v<Raw, RawFP4> && G == 2) {
          r1[i].s = ((i == 0 ? w1.x : w1.y) >> (8 * g4)) & 0xffu;
          r3[i].s = ((i == 0 ? w3.x : w3.y) >> (8 * g4)) & 0xffu;
        }
        mma_block2(r1[i], r3[i], brow, kc, tv && kb + i < k1, ag, au);
      }
    };
    // batches a, b alternate; pairs whose reloads both lie in the range run
    // without conditions (exact waits, see down_block), the last pair reloads
    // only what remains
    const int nb = (k1 - k0 + G - 1) / G;
    int j0 = 0;
    for (; j0 + 4 <= nb; j0 += 2) {
      mm(a1, a3, wa1, wa3, k0 + j0 * G);
      ld(a1, a3, wa1, wa3, k0 + (j0 + 2) * G);
      mm(b1, b3, wb1, wb3, k0 + (j0 + 1) * G);
      ld(b1, b3, wb1, wb3, k0 + (j0 + 3) * G);
    }
    for (; j0 < nb; j0 += 2) {
      mm(a1, a3, wa1, wa3, k0 + j0 * G);
      if (j0 + 2 < nb) ld(a1, a3, wa1, wa3, k0 + (j0 + 2) * G);
      if (j0 + 1 < nb) mm(b1, b3, wb1, wb3, k0 + (j0 + 1) * G);
      if (j0 + 3 < nb) ld(b1, b3, wb1, wb3, k0 + (j0 + 3) * G);
    }
    if constexpr (kGKS > 1) {
      __syncthreads();   // every wave is done with the x tile
      *reinterpret_cast<f32x4*>(&red[item][ks][0][lane][0]) = ag;
      *reinterpret_cast<f32x4*>(&red[item][ks][1][lane][0]) = au;
      __syncthreads();
    }
    if (ks == 0 && rok && tv) {
#pragma unroll
      for (int w = 1; w < kGKS; ++w) {
        ag += *reinterpret_cast<const f32x4*>(&red[item][w][0][lane][0]);
        au += *reinterpret_cast<const f32x4*>(&red[item][w][1][lane][0]);
      }
      const int r = base + c0 + r16;              // dispatch row (shared: token)
      const float wr = shared ? 1.0f : p.wrow[r];
      uint16_t hh[4], hl[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) split_bf16(silu_clamped(ag[q], au[q], p.limit) * wr, hh[q], hl[q]);
      const int ldh = shared ? p.Is : p.I;
      const int64_t off = static_cast<int64_t>(r) * ldh + rt * 16 + 4 * g4;
      uint16_t* dh = shared ? p.hs_hi : p.h_hi;
      uint16_t* dl = shared ? p.hs_lo : p.h_lo;
      *reinterpret_cast<uint2*>(dh + off) = uint2{hh[0] | (uint32_t(hh[1]) << 16), hh[2] | (uint32_t(hh[3]) << 16)};
      *reinterpret_cast<uint2*>(dl + off) = uint2{hl[0] | (uint32_t(hl[1]) << 16), hl[2] | (uint32_t(hl[3]) << 16)};
    }
    __syncthreads();   // the next column tile reuses the LDS
  }
}

// Gate/up of one q3 block in the factored form (x . W = s * sum(q x) + b *
// sum(x) per 64-group, see q3m_pair): row tile rt of w1 / w3 for the n
// dispatch rows base .. in column tiles of kGNC; the A operand is the
// activations (row 2t + h: dispatch row c0 + t of the tile on the K block's
// h-th 64-group), the B operand the raw codes.  Block = one row tile x kQ3gKS
// K ranges (one wave each); every wave's range is whole 512-code superblocks
// (hidden % (kQ3gKS * 512) == 0), one batch (superblock) in flight.  The
// tile's x rows (divided by 8 at the 8q positions, k_x_q3) and their group
// sums are copied into LDS first; then the weights are issued.
constexpr int kQ3gKS = kGW;
constexpr int kQ3gMaxGroups = 128;   // 64-groups of a row: hidden up to 8192
__device__ __forceinline__ void up_block_q3f(const GroupedArgs& p, const void* const* wp, int rt, bool rok, int n,
                                             int base, uint16_t* lds) {
  constexpr int G = 4;                       // K blocks per batch: one superblock
  constexpr int NT = kGW * 64;
  constexpr int kSumRegs = kQ3gMaxGroups * kGNC / NT;   // group sums per thread
  static_assert(kSumRegs * NT == kQ3gMaxGroups * kGNC, "whole passes of group sums");
  const int tid = threadIdx.x, lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int ks = wave;
  const int K = p.H, nblk = K / 128, ng = K / 64;
  const uint16_t* xq = reinterpret_cast<const uint16_t*>(p.xp);
  const float* xg = reinterpret_cast<const float*>(p.xp + static_cast<size_t>(p.T) * K * 2);
  const int per = nblk / kQ3gKS;
  const int k0 = ks * per, k1 = k0 + per;
  const int xs = K + 8;
  uint16_t* xh = lds;                                                        // [kGNC][K + 8]
  float* xsum = reinterpret_cast<float*>(lds + kGNC * xs);                   // [nblk][8][2][2]
  u32x4* zero4 = reinterpret_cast<u32x4*>(xsum + nblk * kQ3fMaxTokens * 4);  // 64 zero bytes
  const uint16_t* zero = reinterpret_cast<const uint16_t*>(zero4);
  float (*red)[2][64][2] = reinterpret_cast<float (*)[2][64][2]>(lds);       // [wave][role], over the x tile
  if (tid < 4) zero4[tid] = u32x4{0u, 0u, 0u, 0u};
  const uint32_t rowc = rok ? static_cast<uint32_t>(rt * 16 + r16) : 0u;   // rows past the tile: row 0, not stored
  const uint32_t code_row = rowc * static_cast<uint32_t>(K / 8 * 3);
  const uint32_t sb_row = rowc * static_cast<uint32_t>(K / 64) * 2;        // bytes
  const uint8_t* W1 = static_cast<const uint8_t*>(wp[0]);
  const uint8_t* W3 = static_cast<const uint8_t*>(wp[3]);
  const uint8_t* SB[4] = {static_cast<const uint8_t*>(wp[1]), static_cast<const uint8_t*>(wp[2]),
                          static_cast<const uint8_t*>(wp[4]), static_cast<const uint8_t*>(wp[5])};
  // loads without conditions (see load_raw_nc): a batch past the range re-reads its last superblock
  auto ld = [&](Q3Batch<G>& b, int kb0) {
    const int kbc = min(kb0, k1 - G);
    const uint32_t off = code_row + (kbc >> 2) * 192 + 48 * g4;
    const auto c1 = gptr<u32x4>(W1 + off);
    const auto c3 = gptr<u32x4>(W3 + off);
#pragma unroll
    for (int v = 0; v < 3; ++v) {
      const u32x4 a = c1[v];
      const u32x4 e = c3[v];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        b.c1[(4 * v + j) / 3][(4 * v + j) % 3] = a[j];
        b.c3[(4 * v + j) / 3][(4 * v + j) % 3] = e[j];
      }
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const u32x4 w = ldg16(SB[a] + sb_row + kbc * 4);
#pragma unroll
      for (int i = 0; i < G; ++i) b.sb[a][i] = w[i];
    }
  };
  const int ta = r16 >> 1;
  const Q3Masks km = q3_masks();
  for (int c0 = 0; c0 < n; c0 += kGNC) {
    const int cols = min(kGNC, n - c0);
    // the tile's x rows and group sums first (written once per call by
    // k_x_q3; their registers are free again before the weights land): the
    // sums' loads go out ahead of the rows', both stored once the rows land
    {
      const int nsum = cols * ng;
      u32x2 sv[kSumRegs];   // {sum x, sum x / m} as loaded
#pragma unroll
      for (int j = 0; j < kSumRegs; ++j) {
        const int i = min(tid + j * NT, nsum - 1);
        const int r = i / ng, gi = i - r * ng;
        sv[j] = ldg<u32x2>(xg + (static_cast<int64_t>(p.xrow[base + c0 + r]) * ng + gi) * 2);
      }
      stage_rows(xh, xq, K, K, cols, [&](int r) { return p.xrow[base + c0 + r]; });
#pragma unroll
      for (int j = 0; j < kSumRegs; ++j) {
        const int i = tid + j * NT;
        if (i < nsum) {
          const int r = i / ng, gi = i - r * ng;
          *reinterpret_cast<u32x2*>(xsum + (((gi >> 1) * kQ3fMaxTokens + r) * 2 + (gi & 1)) * 2) = sv[j];
        }
      }
    }
    Q3Batch<G> A;
    ld(A, k0);
    __syncthreads();
    const bool av = ta < cols && (r16 & 1) == (g4 >> 1);
    const int t0 = 2 * g4;
    float acc1[2] = {0.0f, 0.0f}, acc3[2] = {0.0f, 0.0f};
    auto mm = [&](const Q3Batch<G>& b, int kb0) {
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int kb = kb0 + i;
        const uint16_t* ah = av ? xh + ta * xs + kb * 128 + 32 * g4 : zero;
        f32x4 d1 = {0.0f, 0.0f, 0.0f, 0.0f}, d3 = d1;
#define DSK_Q3G_STEP(M)                                                              \
        {                                                                            \
          const bf16x8 xa = as_bf16x8(*reinterpret_cast<const u32x4*>(ah + 8 * M)); \
          d1 = mfma16(xa, q3m_operand<M>(b.c1[i], km), d1);                          \
          d3 = mfma16(xa, q3m_operand<M>(b.c3[i], km), d3);                          \
        }
        DSK_Q3G_STEP(0) DSK_Q3G_STEP(1) DSK_Q3G_STEP(2) DSK_Q3G_STEP(3)
#undef DSK_Q3G_STEP
        const float* xg = xsum + (kb * kQ3fMaxTokens + t0) * 4;
        const f32x4 xa = *reinterpret_cast<const f32x4*>(xg);
        const f32x4 xb = *reinterpret_cast<const f32x4*>(xg + 4);
        q3_factor(d1, b.sb[0][i], b.sb[1][i], xa, xb, acc1);
        q3_factor(d3, b.sb[2][i], b.sb[3][i], xa, xb, acc3);
      }
    };
    for (int kb = k0; kb < k1; kb += G) {   // one batch at hidden 4096
      if (kb > k0) ld(A, kb);
      mm(A, kb);
    }
    // K ranges added in order, through LDS over the x tile
    __syncthreads();
    *reinterpret_cast<float2*>(&red[ks][0][lane][0]) = float2{acc1[0], acc1[1]};
    *reinterpret_cast<float2*>(&red[ks][1][lane][0]) = float2{acc3[0], acc3[1]};
    __syncthreads();
    if (ks == 0 && rok && t0 < cols) {
#pragma unroll
      for (int w = 1; w < kQ3gKS; ++w) {
        const float2 g = *reinterpret_cast<const float2*>(&red[w][0][lane][0]);
        const float2 u = *reinterpret_cast<const float2*>(&red[w][1][lane][0]);
        acc1[0] += g.x; acc1[1] += g.y;
        acc3[0] += u.x; acc3[1] += u.y;
      }
      const int n16 = rt * 16 + r16;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        if (t0 + q < cols) {
          const int r = base + c0 + t0 + q;   // dispatch row
          uint16_t hh, hl;
          split_bf16(silu_clamped(acc1[q], acc3[q], p.limit) * p.wrow[r], hh, hl);
          p.h_hi[static_cast<int64_t>(r) * p.I + n16] = hh;
          p.h_lo[static_cast<int64_t>(r) * p.I + n16] = hl;
        }
      }
    }
    __syncthreads();   // the next column tile reuses the LDS
  }
}

// ---------------------------------------------------------------- MX gate/up (FP4 slots)
// The FP4 slots' gate/up on v_mfma_scale_f32_16x16x128_f8f6f4 (mx.h): the
// codes and E8M0 bytes go into the product as loaded, so a wave holds its
// whole K range of both roles in flight (kGxMaxBlocks 128-code blocks: 16
// bytes of codes and a 4-byte scale word per block, role and lane) for each
// column tile.  The activations are two FP8 planes per token,
// written once per call by k_x_planes in the B-operand layout; a column tile
// copies its rows' planes into LDS (column 2r + p: plane p of the tile's row
// r).  K ranges are added in wave order, then a row's two plane columns; h
// leaves as the bf16 hi / lo pair of the other gate/up paths.
constexpr int kGxMaxBlocks = 8;     // K blocks per wave held (H <= kGKS * 8 * 128)

// x's two FP8 planes (v ~ q0 2^e + q1 2^(e-4) per 32-value group, e =
// ilogb(group max) - 7, mx.h) into xp (x_planes_chunk's layout), one thread
// per 8 values.
__global__ __launch_bounds__(256) void k_x_planes(const uint16_t* __restrict__ x, int T, int H,
                                                  uint8_t* __restrict__ xp) {
  const int n = T * (H / 8);
  const int c0 = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  x_planes_chunk(x, T, H, min(c0, n - 1), c0 < n, xp);   // every lane takes part in the group exchange
}

// x for the factored q3 gate/up (up_block_q3f), once per call instead of once
// per block (x_q3_chunk); the blocks copy the rows and sums of their column tile.
__global__ __launch_bounds__(256) void k_x_q3(const uint16_t* __restrict__ x, int T, int H,
                                              uint16_t* __restrict__ xq, float* __restrict__ xg) {
  const int n = T * (H / 8);
  const int c = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  x_q3_chunk(x, H, min(c, n - 1), c < n, xq, xg);   // every lane takes part in the group's sums
}

// LDS of up_block_mx: the column tile's planes [H/128][16][128] bytes, then
// their E8M0 words [H/128][16] (4 bytes: the block's four groups); the K-range
// partial sums [kGI][kGKS][2][64][4] f32 reuse the planes after the products.
__host__ __device__ inline size_t gx_lds_bytes(int H) { return static_cast<size_t>(H / 128) * 16 * (128 + 4); }

// Gate/up of one FP4 slot block: row tile rt of w1 / w3 for the n dispatch
// rows base .. base + n - 1.  Every wave's range is PER = H / 128 / kGKS
// blocks (the launcher's condition), so the weight loads are uniform role
// pointers + one 32-bit lane offset + an immediate per block.
template <int PER>
__device__ __forceinline__ void up_block_mx(const GroupedArgs& p, const void* const* wp, int rt, bool rok, int n,
                                            int base, uint8_t* lds) {
  static_assert(PER <= kGxMaxBlocks, "blocks held per wave");
  const int tid = threadIdx.x, lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int item = wave / kGKS, ks = wave % kGKS;
  const int K = p.H, nblk = K / 128;
  const int k0 = ks * PER;
  uint8_t* xq = lds;
  uint32_t* xe = reinterpret_cast<uint32_t*>(lds + static_cast<size_t>(nblk) * 16 * 128);
  float (*red)[kGKS][2][64][4] = reinterpret_cast<float (*)[kGKS][2][64][4]>(lds);
  // the wave's range within each role (uniform), this lane's row within it (32 bits: one role < 4 GB)
  const uint8_t* W1 = static_cast<const uint8_t*>(wp[0]) + k0 * 64;
  const uint8_t* S1 = static_cast<const uint8_t*>(wp[1]) + k0 * 4;
  const uint8_t* W3 = static_cast<const uint8_t*>(wp[3]) + k0 * 64;
  const uint8_t* S3 = static_cast<const uint8_t*>(wp[4]) + k0 * 4;
  const uint32_t row = rok ? static_cast<uint32_t>(rt * 16 + r16) : 0u;
  const uint32_t cb = row * static_cast<uint32_t>(K / 2) + static_cast<uint32_t>(g4 * 16);
  const uint32_t sb = row * static_cast<uint32_t>(K / 32);
  const uint8_t* xs = p.xp + static_cast<size_t>(p.T) * 2 * K;   // the planes' E8M0 bytes
  // the h planes' 16-row maxima [kGI][16] f32, past the partial sums
  float* gmx = reinterpret_cast<float*>(lds + static_cast<size_t>(kGI) * kGKS * 2 * 64 * 4 * sizeof(float));
  // the wave's whole K range of both roles first (every product waits for it
  // anyway), held across the slot's column tiles; then per tile its plane rows
  // (16-byte chunks) and their exponents
  u32x4 c1[PER], c3[PER];
  uint32_t s1[PER], s3[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    c1[i] = ldg16(W1 + cb + i * 64);
    c3[i] = ldg16(W3 + cb + i * 64);
    s1[i] = ldg<uint32_t>(S1 + sb + i * 4);
    s3[i] = ldg<uint32_t>(S3 + sb + i * 4);
  }
  for (int c0 = 0; c0 < n; c0 += kGNC) {
    const int cols = min(kGNC, n - c0);
    asm volatile("" ::: "memory");
    {
      const int cpr = K / 16, chunks = 2 * cols * cpr;
      for (int ch = tid; ch < chunks; ch += 2 * kGW * 64) {   // two chunks per thread in flight
        u32x4 v[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int cc = min(ch + q * kGW * 64, chunks - 1);   // no condition on the load
          const int col = cc / cpr, j = cc % cpr;
          const int tok = p.xrow[base + c0 + (col >> 1)];
          v[q] = ldg16(p.xp + static_cast<size_t>(2 * tok + (col & 1)) * K + 16 * j);
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int cc = ch + q * kGW * 64;
          if (cc < chunks) {
            const int col = cc / cpr, j = cc % cpr;   // j: 16-byte chunk of the row, block j / 8
            *reinterpret_cast<u32x4*>(xq + ((j >> 3) * 16 + col) * 128 + 16 * (j & 7)) = v[q];
          }
        }
      }
      const int words = 2 * cols * nblk;
      for (int wi = tid; wi < words; wi += kGW * 64) {
        const int col = wi / nblk, kb = wi % nblk;
        const int tok = p.xrow[base + c0 + (col >> 1)];
        xe[kb * 16 + col] = ldg<uint32_t>(xs + static_cast<size_t>(2 * tok + (col & 1)) * (K / 32) + 4 * kb);
      }
    }
    __syncthreads();
    // B column of this lane: plane r16 & 1 of tile row r16 >> 1 (columns past
    // the tile's rows repeat its last one; their results are not stored)
    const int bc = min(r16, 2 * cols - 1);
    f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = ag;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int col = (k0 + i) * 16 + bc;
      const u32x4* src = reinterpret_cast<const u32x4*>(xq + col * 128 + g4 * 32);
      const u32x4 blo = src[0], bhi = src[1];
      const uint32_t bs = (xe[col] >> (8 * g4)) & 0xffu;
      ag = mx_mfma(c1[i], (s1[i] >> (8 * g4)) & 0xffu, blo, bhi, bs, ag);
      au = mx_mfma(c3[i], (s3[i] >> (8 * g4)) & 0xffu, blo, bhi, bs, au);
    }
    __syncthreads();   // every wave is done with the planes
    *reinterpret_cast<f32x4*>(&red[item][ks][0][lane][0]) = ag;
    *reinterpret_cast<f32x4*>(&red[item][ks][1][lane][0]) = au;
    __syncthreads();
    float hv[4] = {0.f, 0.f, 0.f, 0.f};   // h of this lane's column and rows (ks == 0 waves)
    if (ks == 0) {
#pragma unroll
      for (int w = 1; w < kGKS; ++w) {
        ag += *reinterpret_cast<const f32x4*>(&red[item][w][0][lane][0]);
        au += *reinterpret_cast<const f32x4*>(&red[item][w][1][lane][0]);
      }
      float g[4], u[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {   // the row's two plane columns (lanes 2r, 2r + 1)
        g[q] = ag[q] + lane_xor1(ag[q]);
        u[q] = au[q] + lane_xor1(au[q]);
      }
      const int rr = r16 >> 1;
      const int r = base + c0 + min(rr, cols - 1);   // dispatch row (columns past the tile: its last)
      const float wr = p.wrow[r];
#pragma unroll
      for (int q = 0; q < 4; ++q) hv[q] = silu_clamped(g[q], u[q], p.limit) * wr;
      if (!p.hplanes && rok && (r16 & 1) == 0 && rr < cols) {
        uint16_t hh[4], hl[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) split_bf16(hv[q], hh[q], hl[q]);
        const int64_t off = static_cast<int64_t>(r) * p.I + rt * 16 + 4 * g4;
        *reinterpret_cast<uint2*>(p.h_hi + off) = uint2{hh[0] | (uint32_t(hh[1]) << 16), hh[2] | (uint32_t(hh[3]) << 16)};
        *reinterpret_cast<uint2*>(p.h_lo + off) = uint2{hl[0] | (uint32_t(hl[1]) << 16), hl[2] | (uint32_t(hl[3]) << 16)};
      }
      if (p.hplanes) {
        // one exponent per (row, 32-row group): the largest |h| of this tile's 16 rows
        float m = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) m = fmaxf(m, fabsf(hv[q]));
        m = max_over_rows(m);
        // (addresses from a copy of the lane id made here: forms hoisted out of the
        // column loop stayed live across the weight stream and spilled)
        int ln = lane;
        asm volatile("" : "+v"(ln));
        if (ln < 16) gmx[item * 16 + ln] = m;
      }
    }
    if (p.hplanes) {
      // h as three FP8 planes per dispatch row (the MX down's B operand): the
      // block's two row tiles are one 32-row exponent group
      __syncthreads();
      int ln = lane;   // (as above)
      asm volatile("" : "+v"(ln));
      const int c16 = ln & 15, q4 = ln >> 4, rr = c16 >> 1;
      if (ks == 0 && rok && (c16 & 1) == 0 && rr < cols) {
        const int r = base + c0 + rr;
        const int e = fp8_plane_exp(fmaxf(gmx[c16], gmx[16 + c16]));
        uint32_t w[3];
        fp8_planes4<3>(hv, e, w);
        const int I = p.I, i0 = rt * 16 + 4 * q4;
        uint8_t* dst = p.hp + static_cast<size_t>(3 * r) * I + (i0 >> 7) * 128 + b_perm(i0 & 127);
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) *reinterpret_cast<uint32_t*>(dst + static_cast<size_t>(pl) * I) = w[pl];
        if (item == 0 && q4 == 0) {
          uint8_t* sc = p.hp + static_cast<size_t>(p.T) * p.k * 3 * I;
#pragma unroll
          for (int pl = 0; pl < 3; ++pl)
            sc[static_cast<size_t>(3 * r + pl) * (I / 32) + (i0 >> 5)] = static_cast<uint8_t>(e8m0_byte(e - 4 * pl));
        }
      }
    }
    __syncthreads();   // the next column tile reuses the LDS
  }
}

// The shared expert over more than kGNC tokens.  Its weights are 50 MB of
// bf16 at hidden 4096 / inter 2048, which the column-tile walk above would
// stream once per kGNC tokens (8x at 64 tokens).  Here a block's waves each
// take one row tile (16 rows of one weight matrix) over the whole of K and
// step through K together: at step s every wave multiplies K block s of its
// rows against the same activation block (up to kGsCols tokens x 128 of K,
// four 16-column MFMA tiles) staged in LDS.  The activations are
// L2-resident and small next to the weights; they go through registers into
// two LDS buffers, one barrier per step (gs_walk).  Weights stream once per
// kGsCols tokens.
constexpr int kGsCols = 64;              // tokens of a wide shared column group
constexpr int kGsCT = kGsCols / 16;      // its 16-column MFMA tiles
constexpr int kGsStride = 128 + 8;       // LDS row stride (elements) of a staged K block
constexpr int kGsPlane = kGsCols * kGsStride;

__host__ __device__ constexpr size_t gs_up_lds_bytes() { return 2 * size_t{kGsPlane} * 2; }
__host__ __device__ constexpr size_t gs_down_lds_bytes() { return 2 * 2 * size_t{kGsPlane} * 2; }

// K block kb of the group's rows g0 .. g0 + ncol - 1 of a [rows][ld] bf16
// matrix: thread t's 16-byte chunks t and t + 512 (row c / 16, 8 elements
// c % 16); rows past the group read its last row (never stored).
__device__ __forceinline__ void gs_load(u32x4 (&v)[2], const uint16_t* m, int ld, int g0, int ncol, int kb) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int c = static_cast<int>(threadIdx.x) + q * kGW * 64;
    const int r = min(c >> 4, ncol - 1);
    v[q] = ldg16(m + static_cast<int64_t>(g0 + r) * ld + kb * 128 + (c & 15) * 8);
  }
}

__device__ __forceinline__ void gs_store(const u32x4 (&v)[2], uint16_t* buf) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int c = static_cast<int>(threadIdx.x) + q * kGW * 64;
    *reinterpret_cast<u32x4*>(buf + (c >> 4) * kGsStride + (c & 15) * 8) = v[q];
  }
}

static_assert(kGW * 64 * 2 * 8 == kGsCols * 128, "two chunks per thread stage one K block of the group");

// Steps 0 .. nb - 1 of a wide shared walk with rings of NB weight batches
// and NB activation register slots, and two LDS buffers: mm(i, buf)
// multiplies batch i against buffer buf, ldw(i, kb) reloads batch i with K
// block kb, ldx(i, kb) loads K block kb's activations into slot i, stx(i,
// buf) copies slot i into buffer buf.  Block t's activations are loaded NB
// steps ahead, before the weights of block t, so copying them into LDS at
// step t - 1 waits only for weights already used.  Loads past the end
// re-read block nb - 1 (unused), so no load in the main loop sits under a
// condition; the last steps load only what remains.
template <int NB, typename MM, typename LW, typename LX, typename SX>
__device__ __forceinline__ void gs_walk(int nb, MM mm, LW ldw, LX ldx, SX stx) {
  constexpr int U = NB % 2 == 0 ? NB : 2 * NB;   // steps per pass: slots and buffers back in phase
#pragma unroll
  for (int i = 0; i < NB; ++i) ldx(i, min(i, nb - 1));
#pragma unroll
  for (int i = 0; i < NB; ++i) ldw(i, min(i, nb - 1));
  stx(0, 0);
  __syncthreads();
  int s = 0;
  for (; s + U <= nb; s += U) {
#pragma unroll
    for (int i = 0; i < U; ++i) {
      mm(i % NB, i & 1);
      ldx(i % NB, min(s + i + NB, nb - 1));
      ldw(i % NB, min(s + i + NB, nb - 1));
      stx((i + 1) % NB, (i + 1) & 1);
      __syncthreads();
    }
  }
  // the last nb - s < U steps
#pragma unroll
  for (int i = 0; i < U - 1; ++i) {
    if (s + i < nb) {
      mm(i % NB, i & 1);
      if (s + i + NB < nb) {
        ldx(i % NB, s + i + NB);
        ldw(i % NB, s + i + NB);
      }
      if (s + i + 1 < nb) stx((i + 1) % NB, (i + 1) & 1);
      __syncthreads();
    }
  }
}

// Gate/up of the shared expert over more than kGNC tokens: waves 2i and
// 2i + 1 take row tile 4b + i of w1 (gate) and of w3 (up), so that a wave
// holds one role's accumulators and a ring of four weight batches; the up
// wave hands its sums to the gate wave through LDS for SwiGLU.
__device__ __forceinline__ void up_shared_wide(const GroupedArgs& p, int b, uint16_t* lds) {
  constexpr int NB = 3;
  const int lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int role = wave & 1, pair = wave >> 1;
  const int rt = b * (kGW / 2) + pair;
  const bool rok = rt < p.Is / 16;
  const uint32_t row = rok ? static_cast<uint32_t>(rt * 16 + r16) : 0u;
  const uint16_t* W = role ? p.ws3 : p.ws1;
  const int K = p.H, nb = K / 128;
  f32x4 (*xch)[kGsCT][64] = reinterpret_cast<f32x4 (*)[kGsCT][64]>(lds);   // [pair][tile][lane], after the walk
  for (int g0 = 0; g0 < p.T; g0 += kGsCols) {
    const int ncol = min(kGsCols, p.T - g0);
    const int nct = (ncol + 15) / 16;
    RawBF16 w[NB];
    u32x4 xv[NB][2];
    f32x4 acc[kGsCT];
#pragma unroll
    for (int c = 0; c < kGsCT; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto mm = [&](int i, int buf) {
#pragma unroll
      for (int c = 0; c < kGsCT; ++c)
        if (c < nct) mma_block(w[i], lds + buf * kGsPlane + (c * 16 + r16) * kGsStride, g4 * 32, true, acc[c]);
    };
    auto ldw = [&](int i, int kb) { load_raw_nc(w[i], W, row, K, kb * 128 + g4 * 32); };
    auto ldx = [&](int slot, int kb) { gs_load(xv[slot], p.x, K, g0, ncol, kb); };
    auto stx = [&](int slot, int buf) { gs_store(xv[slot], lds + buf * kGsPlane); };
    gs_walk<NB>(nb, mm, ldw, ldx, stx);   // ends with a barrier: the buffers are free
    if (role) {
#pragma unroll
      for (int c = 0; c < kGsCT; ++c) xch[pair][c][lane] = acc[c];
    }
    __syncthreads();
    if (!role && rok) {
#pragma unroll
      for (int c = 0; c < kGsCT; ++c) {
        const int t = c * 16 + r16;
        if (t < ncol) {
          const f32x4 au = xch[pair][c][lane];
          uint16_t hh[4], hl[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) split_bf16(silu_clamped(acc[c][q], au[q], p.limit), hh[q], hl[q]);
          const int64_t off = static_cast<int64_t>(g0 + t) * p.Is + rt * 16 + 4 * g4;
          *reinterpret_cast<uint2*>(p.hs_hi + off) =
              uint2{hh[0] | (uint32_t(hh[1]) << 16), hh[2] | (uint32_t(hh[3]) << 16)};
          *reinterpret_cast<uint2*>(p.hs_lo + off) =
              uint2{hl[0] | (uint32_t(hl[1]) << 16), hl[2] | (uint32_t(hl[3]) << 16)};
        }
      }
    }
    __syncthreads();   // the exchange is read before the next group restages the buffers
  }
}

static_assert(size_t{kGW / 2} * kGsCT * 64 * 16 <= gs_up_lds_bytes(), "the SwiGLU exchange fits the buffers");

// Down of the shared expert over more than kGNC tokens, as up_shared_wide:
// block b's eight waves each take one row tile of w2 (16 output rows) over
// K = Is, the h planes (hi, lo) of up to kGsCols tokens staged per K block.
__device__ __forceinline__ void down_shared_wide(const GroupedArgs& p, int b, uint16_t* lds) {
  constexpr int NB = 2;
  const int lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int rt = b * kDW + wave;
  const uint32_t row = static_cast<uint32_t>(rt * 16 + r16);
  const int K = p.Is, nb = K / 128;
  for (int g0 = 0; g0 < p.T; g0 += kGsCols) {
    const int ncol = min(kGsCols, p.T - g0);
    const int nct = (ncol + 15) / 16;
    RawBF16 w[NB];
    u32x4 xh[NB][2], xl[NB][2];
    f32x4 acc[kGsCT];
#pragma unroll
    for (int c = 0; c < kGsCT; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto mm = [&](int i, int buf) {
      const uint16_t* hi = lds + buf * 2 * kGsPlane;
#pragma unroll
      for (int c = 0; c < kGsCT; ++c) {
        if (c < nct) {
          const int o = (c * 16 + r16) * kGsStride;
          mma_block(w[i], hi + o, g4 * 32, true, acc[c]);
          mma_block(w[i], hi + kGsPlane + o, g4 * 32, true, acc[c]);
        }
      }
    };
    auto ldw = [&](int i, int kb) { load_raw_nc(w[i], p.ws2, row, K, kb * 128 + g4 * 32); };
    auto ldx = [&](int slot, int kb) {
      gs_load(xh[slot], p.hs_hi, K, g0, ncol, kb);
      gs_load(xl[slot], p.hs_lo, K, g0, ncol, kb);
    };
    auto stx = [&](int slot, int buf) {
      gs_store(xh[slot], lds + buf * 2 * kGsPlane);
      gs_store(xl[slot], lds + buf * 2 * kGsPlane + kGsPlane);
    };
    gs_walk<NB>(nb, mm, ldw, ldx, stx);
#pragma unroll
    for (int c = 0; c < kGsCT; ++c) {
      const int t = c * 16 + r16;
      if (t < ncol) *reinterpret_cast<f32x4*>(p.ys + static_cast<int64_t>(g0 + t) * p.H + rt * 16 + 4 * g4) = acc[c];
    }
    __syncthreads();   // the next group restages buffer 0
  }
}

// Blocks [0, up_shared): the shared expert (bf16 w1/w3, all T tokens); the
// others: up_groups blocks per slot.
template <typename Raw>
__global__ __launch_bounds__(kGW * 64) __attribute__((amdgpu_waves_per_eu(4))) void k_up_grouped(GroupedArgs p) {
  extern __shared__ __align__(16) uint16_t lds_g[];
  const int b = static_cast<int>(blockIdx.x);
  const int item = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) / kGKS;
  if (b < p.up_shared) {
    if (p.T > kGNC) {
      up_shared_wide(p, b, lds_g);
      return;
    }
    const int rt = b * kGI + item;
    auto load_w = [&](RawBF16& r, int role, uint32_t row, int kc) { load_raw_nc(r, role ? p.ws3 : p.ws1, row, p.H, kc); };
    up_block<RawBF16>(p, load_w, [&](int) -> const void* { return p.ws1; }, rt, rt < p.Is / 16, p.T, 0, true, lds_g);
    return;
  }
  const int rb = b - p.up_shared;
  const int slot = rb / p.up_groups;
  if (slot >= p.active[0]) return;
  const SlotDesc* d = p.desc + slot;
  const int rt = (rb % p.up_groups) * kGI + item;
  const void* const wp[6] = {desc_ptr(p.desc, slot, 0), desc_ptr(p.desc, slot, 1), desc_ptr(p.desc, slot, 2),
                             desc_ptr(p.desc, slot, 3), desc_ptr(p.desc, slot, 4), desc_ptr(p.desc, slot, 5)};
  if constexpr (std::is_same_v<Raw, RawQ3>) {
    if (p.q3f) {   // one row tile per block (up_groups = I / 16)
      const int rt1 = rb % p.up_groups;
      up_block_q3f(p, wp, rt1, rt1 < p.I / 16, d->n_tok, d->tok_base, lds_g);
      return;
    }
  }
  if constexpr (std::is_same_v<Raw, RawFP4>) {
    if (p.mx) {
      uint8_t* lds = reinterpret_cast<uint8_t*>(lds_g);
      const bool rok = rt < p.I / 16;
      switch (p.mx) {   // blocks per wave: H / 128 / kGKS
        case 2: up_block_mx<2>(p, wp, rt, rok, d->n_tok, d->tok_base, lds); break;
        case 4: up_block_mx<4>(p, wp, rt, rok, d->n_tok, d->tok_base, lds); break;
        case 6: up_block_mx<6>(p, wp, rt, rok, d->n_tok, d->tok_base, lds); break;
        default: up_block_mx<8>(p, wp, rt, rok, d->n_tok, d->tok_base, lds); break;
      }
      return;
    }
  }
  auto load_w = [&](Raw& r, int role, uint32_t row, int kc) { load_role_nc(r, wp, role, row, p.H, kc); };
  up_block<Raw>(p, load_w, [&](int i) { return wp[i]; }, rt, rt < p.I / 16, d->n_tok, d->tok_base, false, lds_g);
}

// Down of one block: row tile rt (output rows 16 rt ..) of w2 for the n
// dispatch rows base .. base + n - 1 (shared: tokens 0 .. n - 1), K = I (Is).
template <typename Raw, typename LoadW, typename WPtr>
__device__ __forceinline__ void down_block(const GroupedArgs& p, LoadW load_w, WPtr wptr, int rt, int n, int base,
                                           bool shared, uint16_t* lds) {
  constexpr int G = batch_blocks<Raw>();
  const int lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int item = wave / kDKS, ks = wave % kDKS;
  const int K = shared ? p.Is : p.I, nblk = K / 128;
  const int per = (nblk + kDKS - 1) / kDKS;
  const int k0 = min(ks * per, nblk), k1 = min(k0 + per, nblk);
  const int hs = K + 8;
  const uint32_t row = static_cast<uint32_t>(rt * 16 + r16);
  const uint16_t* src_hi = shared ? p.hs_hi : p.h_hi;
  const uint16_t* src_lo = shared ? p.hs_lo : p.h_lo;
  uint16_t* thi = lds;                      // [kGNC][K + 8] hi plane
  uint16_t* tlo = lds + kGNC * hs;          // [kGNC][K + 8] lo plane
  float (*red)[kDKS][64][4] = reinterpret_cast<float (*)[kDKS][64][4]>(lds);   // over the h tile
  constexpr int NB = down_ring<Raw>();
  for (int c0 = 0; c0 < n; c0 += kGNC) {
    const int cols = min(kGNC, n - c0);
    Raw a[NB][G];
    // FP4: the scales of a batch's 2 blocks (all lane groups) as one 8-byte
    // window instead of one byte per lane and block; the byte is picked at use
    u32x2 wa[NB] = {};
    // no condition on the loads (see load_raw_nc): blocks past the range
    // re-read its last block (not computed)
    auto ld = [&](Raw (&r)[G], u32x2& w, int kb) {
      if constexpr (std::is_same_v<Raw, RawFP4> && G == 2) {
        const int kbc = min(kb, k1 - 2);   // the range has an even number of blocks
#pragma unroll
        for (int i = 0; i < G; ++i) r[i].c = ldg16(static_cast<const uint8_t*>(wptr(0)) + row * static_cast<uint32_t>(K / 2) + (kbc + i) * 64 + g4 * 16);
        w = ldg<u32x2>(static_cast<const uint8_t*>(wptr(1)) + row * static_cast<uint32_t>(K / 32) + kbc * 4);
      } else {
#pragma unroll
        for (int i = 0; i < G; ++i) load_w(r[i], row, min(kb + i, k1 - 1) * 128 + g4 * 32);
      }
    };
    // the h rows first (see up_block)
    stage_rows(thi, src_hi, K, K, cols, [&](int r) { return base + c0 + r; });
    stage_rows(tlo, src_lo, K, K, cols, [&](int r) { return base + c0 + r; });
#pragma unroll
    for (int i = 0; i < NB; ++i) ld(a[i], wa[i], k0 + i * G);
    __syncthreads();
    const bool tv = r16 < cols;
    const uint16_t* bh = thi + (tv ? r16 : 0) * hs;
    const uint16_t* bl = tlo + (tv ? r16 : 0) * hs;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    auto mm = [&](Raw (&r)[G], const u32x2& w, int kb) {
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int kc = (kb + i) * 128 + g4 * 32;
        const bool ok = tv && kb + i < k1;
        if constexpr (std::is_same_v<Raw, RawFP4> && G == 2) r[i].s = ((i == 0 ? w.x : w.y) >> (8 * g4)) & 0xffu;
        mma_block(r[i], bh, kc, ok, acc);
        mma_block(r[i], bl, kc, ok, acc);
      }
    };
    // NB batches in a ring: each is multiplied, then reloaded NB batches ahead.
    // Groups whose reloads all lie in the range run without conditions (a load
    // under a condition makes the next use of an older batch wait for every
    // load, as at a branch merge the wait counter cannot tell which were
    // issued); the last groups reload only what remains.
    const int nb = (k1 - k0 + G - 1) / G;
    int j0 = 0;
    for (; j0 + 2 * NB <= nb; j0 += NB) {
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        mm(a[i], wa[i], k0 + (j0 + i) * G);
        ld(a[i], wa[i], k0 + (j0 + i + NB) * G);
      }
    }
    for (; j0 < nb; j0 += NB) {
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        if (j0 + i < nb) {
          mm(a[i], wa[i], k0 + (j0 + i) * G);
          if (j0 + i + NB < nb) ld(a[i], wa[i], k0 + (j0 + i + NB) * G);
        }
      }
    }
    if constexpr (kDKS > 1) {
      __syncthreads();   // every wave is done with the h tile
      *reinterpret_cast<f32x4*>(&red[item][ks][lane][0]) = acc;
      __syncthreads();
    }
    if (ks == 0 && tv) {
#pragma unroll
      for (int w = 1; w < kDKS; ++w) acc += *reinterpret_cast<const f32x4*>(&red[item][w][lane][0]);
      float* out = shared ? p.ys : p.y;
      *reinterpret_cast<f32x4*>(out + static_cast<int64_t>(base + c0 + r16) * p.H + rt * 16 + 4 * g4) = acc;
    }
    __syncthreads();   // the next column tile reuses the LDS
  }
}

// Down of one FP4 slot block on scaled MFMAs: row tile rt (output rows
// 16 rt ..) of w2 over K = I = 128 NKB, for the n dispatch rows base ..
// base + n - 1, h as the gate/up's three FP8 planes per row (B column 3r + p:
// five rows per column tile).  The wave's whole range of w2 codes and E8M0
// words is issued first, then the tile's plane rows are copied into LDS;
// one MFMA per block, a row's three plane columns added in order.  Writes
// one float32 output row per dispatch row, as down_block.
constexpr int kGdRows = 5;   // dispatch rows of an MX down column tile (15 B columns)

__host__ __device__ inline size_t gd_lds_bytes(int I) { return static_cast<size_t>(I / 128) * 16 * (128 + 4); }

template <int NKB>
__device__ __forceinline__ void down_block_mx(const GroupedArgs& p, int slot, int rt, int n, int base,
                                              uint8_t* lds) {
  const int tid = threadIdx.x, lane = __lane_id();
  const int r16 = lane & 15, g4 = lane >> 4;
  const int I = p.I;
  uint8_t* hq = lds;
  uint32_t* he = reinterpret_cast<uint32_t*>(lds + static_cast<size_t>(NKB) * 16 * 128);
  const uint8_t* W = static_cast<const uint8_t*>(desc_ptr(p.desc, slot, 6));
  const uint8_t* S = static_cast<const uint8_t*>(desc_ptr(p.desc, slot, 7));
  const uint32_t row = static_cast<uint32_t>(rt * 16 + r16);
  const uint32_t cb = row * static_cast<uint32_t>(I / 2) + static_cast<uint32_t>(g4 * 16);
  const uint32_t sb = row * static_cast<uint32_t>(I / 32);
  const uint8_t* hs = p.hp + static_cast<size_t>(p.T) * p.k * 3 * I;   // the planes' E8M0 bytes
  for (int c0 = 0; c0 < n; c0 += kGdRows) {
    const int cols = min(kGdRows, n - c0);
    u32x4 c[NKB];
    uint32_t sc[NKB];
#pragma unroll
    for (int i = 0; i < NKB; ++i) {
      c[i] = ldg16(W + cb + i * 64);
      sc[i] = ldg<uint32_t>(S + sb + i * 4);
    }
    asm volatile("" ::: "memory");
    {
      const int cpr = I / 16, chunks = 3 * cols * cpr;
      for (int ch = tid; ch < chunks; ch += 4 * kDW * 64) {
        u32x4 v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int cc = min(ch + q * kDW * 64, chunks - 1);   // no condition on the load
          const int col = cc / cpr, j = cc % cpr;
          v[q] = ldg16(p.hp + static_cast<size_t>(3 * (base + c0) + col) * I + 16 * j);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int cc = ch + q * kDW * 64;
          if (cc < chunks) {
            const int col = cc / cpr, j = cc % cpr;
            *reinterpret_cast<u32x4*>(hq + ((j >> 3) * 16 + col) * 128 + 16 * (j & 7)) = v[q];
          }
        }
      }
      const int words = 3 * cols * NKB;
      for (int wi = tid; wi < words; wi += kDW * 64) {
        const int col = wi / NKB, kb = wi % NKB;
        he[kb * 16 + col] = ldg<uint32_t>(hs + static_cast<size_t>(3 * (base + c0) + col) * (I / 32) + 4 * kb);
      }
    }
    __syncthreads();
    // B column of this lane: plane r16 % 3 of tile row r16 / 3 (columns past
    // the tile's rows repeat its last one; their results are not stored)
    const int bc = min(r16, 3 * cols - 1);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NKB; ++i) {
      const int col = i * 16 + bc;
      const u32x4* src = reinterpret_cast<const u32x4*>(hq + col * 128 + g4 * 32);
      const u32x4 blo = src[0], bhi = src[1];
      const uint32_t bs = (he[col] >> (8 * g4)) & 0xffu;
      acc = mx_mfma(c[i], (sc[i] >> (8 * g4)) & 0xffu, blo, bhi, bs, acc);
    }
    // row t = r16 of this lane group: columns 3t .. 3t + 2, added in order
    const int t = min(r16, cols - 1), gb = lane & 48;
    f32x4 ra;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      ra[q] = (__shfl(acc[q], gb + 3 * t, 64) + __shfl(acc[q], gb + 3 * t + 1, 64)) + __shfl(acc[q], gb + 3 * t + 2, 64);
    if (r16 < cols)
      *reinterpret_cast<f32x4*>(p.y + static_cast<int64_t>(base + c0 + r16) * p.H + rt * 16 + 4 * g4) = ra;
    __syncthreads();   // the next column tile reuses the LDS
  }
}

// Down of one q3 block in the factored form (as up_block_q3f): output row
// tile rt (one wave) over all of K = I in 512-code superblocks (I % 512 ==
// 0), two in flight; A operand row 2t + h on the hi plane and then the lo
// plane of dispatch row c0 + t's h (both into one accumulator), B operand the
// raw w2 codes; the tile's h rows are staged divided by 8 at the 8q positions
// with the group sums of hi + lo.  Writes one float32 row per dispatch row.
struct Q3Sb { uint32_t c[4][3]; u32x4 s, b; };   // one superblock of a lane's w2 row: codes, windows

__device__ __forceinline__ void down_block_q3f(const GroupedArgs& p, int slot, int rt, int n, int base,
                                               uint16_t* lds) {
  constexpr int kStg = 2;                    // h chunks per thread in flight while staging
  constexpr int NT = kDW * 64;
  const int tid = threadIdx.x, lane = __lane_id();
  const int r16 = lane & 15, g4 = lane >> 4;
  const int K = p.I, nblk = K / 128, nsb = K / 512, cpr = K / 8;
  const int hs = K + 8;
  uint16_t* thi = lds;                                                       // [kGNC][K + 8]
  uint16_t* tlo = lds + kGNC * hs;                                           // [kGNC][K + 8]
  float* hsum = reinterpret_cast<float*>(lds + 2 * kGNC * hs);               // [nblk][8][2][2]
  u32x4* zero4 = reinterpret_cast<u32x4*>(hsum + nblk * kQ3fMaxTokens * 4);  // 64 zero bytes
  const uint16_t* zero = reinterpret_cast<const uint16_t*>(zero4);
  if (tid < 4) zero4[tid] = u32x4{0u, 0u, 0u, 0u};
  const uint32_t row = static_cast<uint32_t>(rt * 16 + r16);
  const uint8_t* W = static_cast<const uint8_t*>(desc_ptr(p.desc, slot, 6));
  const uint8_t* S = static_cast<const uint8_t*>(desc_ptr(p.desc, slot, 7));
  const uint8_t* B = static_cast<const uint8_t*>(desc_ptr(p.desc, slot, 8));
  const uint32_t code_row = row * static_cast<uint32_t>(K / 8 * 3), sb_row = row * static_cast<uint32_t>(K / 64) * 2;
  // no condition on the loads (see load_raw_nc): past the last superblock, the last again (not computed)
  auto ld = [&](Q3Sb& r, int sb) {
    const int sbc = min(sb, nsb - 1);
    const auto c = gptr<u32x4>(W + code_row + sbc * 192 + 48 * g4);
#pragma unroll
    for (int v = 0; v < 3; ++v) {
      const u32x4 a = c[v];
#pragma unroll
      for (int j = 0; j < 4; ++j) r.c[(4 * v + j) / 3][(4 * v + j) % 3] = a[j];
    }
    r.s = ldg16(S + sb_row + sbc * 16);
    r.b = ldg16(B + sb_row + sbc * 16);
  };
  const int ta = r16 >> 1;
  const Q3Masks km = q3_masks();
  for (int c0 = 0; c0 < n; c0 += kGNC) {
    const int cols = min(kGNC, n - c0);
    // the tile's h rows (hi + lo), kStg chunks per thread in flight (whole lane groups)
    const int xch = cols * cpr;
    for (int cb = 0; cb < xch; cb += kStg * NT) {
      u32x4 vh[kStg], vl[kStg];
#pragma unroll
      for (int j = 0; j < kStg; ++j) {
        const int c = min(cb + j * NT + tid, xch - 1);
        const int64_t e = static_cast<int64_t>(base + c0 + c / cpr) * K + (c % cpr) * 8;
        vh[j] = ldg16(p.h_hi + e);
        vl[j] = ldg16(p.h_lo + e);
      }
#pragma unroll
      for (int j = 0; j < kStg; ++j) {
        const int c = cb + j * NT + tid;
        if (c < xch) {
          // hi + lo is exact in float32; staged again as a (hi, lo) pair of the scaled value
          const uint32_t wh[4] = {vh[j].x, vh[j].y, vh[j].z, vh[j].w}, wl[4] = {vl[j].x, vl[j].y, vl[j].z, vl[j].w};
          uint32_t f[8];
#pragma unroll
          for (int e2 = 0; e2 < 8; ++e2) {
            const uint32_t sh = (e2 & 1) ? 0u : 16u;
            const float v = __uint_as_float(((wh[e2 >> 1] << sh) & 0xffff0000u)) +
                            __uint_as_float(((wl[e2 >> 1] << sh) & 0xffff0000u));
            f[e2] = __float_as_uint(v);
          }
          stage_chunk_q3<true>(thi, tlo, hsum, hs, cpr, c, u32x4{f[0], f[1], f[2], f[3]}, u32x4{f[4], f[5], f[6], f[7]});
        }
      }
    }
    // keep the weight loads below the staging (their registers would overlap)
    __builtin_amdgcn_sched_barrier(0);
    Q3Sb ra, rb;
    ld(ra, 0);
    ld(rb, 1);
    __syncthreads();
    const bool av = ta < cols && (r16 & 1) == (g4 >> 1);
    const int t0 = 2 * g4;
    float acc[2] = {0.0f, 0.0f};
    auto mm = [&](const Q3Sb& r, int sb) {
      const uint32_t sw[4] = {r.s.x, r.s.y, r.s.z, r.s.w}, bw[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kb = 4 * sb + i;
        const int ao = ta * hs + kb * 128 + 32 * g4;
        const uint16_t* ah = av ? thi + ao : zero;
        const uint16_t* al = av ? tlo + ao : zero;
        f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#define DSK_Q3D_STEP(M)                                                                                \
        d = mfma16(as_bf16x8(*reinterpret_cast<const u32x4*>(ah + 8 * M)), q3m_operand<M>(r.c[i], km), d); \
        d = mfma16(as_bf16x8(*reinterpret_cast<const u32x4*>(al + 8 * M)), q3m_operand<M>(r.c[i], km), d);
        DSK_Q3D_STEP(0) DSK_Q3D_STEP(1) DSK_Q3D_STEP(2) DSK_Q3D_STEP(3)
#undef DSK_Q3D_STEP
        const float* xg = hsum + (kb * kQ3fMaxTokens + t0) * 4;
        q3_factor(d, sw[i], bw[i], *reinterpret_cast<const f32x4*>(xg), *reinterpret_cast<const f32x4*>(xg + 4), acc);
      }
    };
    for (int sb = 0; sb < nsb; sb += 2) {
      mm(ra, sb);
      if (sb + 2 < nsb) ld(ra, sb + 2);
      if (sb + 1 < nsb) mm(rb, sb + 1);
      if (sb + 3 < nsb) ld(rb, sb + 3);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (t0 + q < cols) p.y[static_cast<int64_t>(base + c0 + t0 + q) * p.H + rt * 16 + r16] = acc[q];
    __syncthreads();   // the next column tile reuses the LDS
  }
}

// Blocks [0, dn_shared): the shared expert's w2 (bf16, all T tokens); the
// others: dn_groups blocks per slot.
// q3: three waves per SIMD (the factored product keeps two superblocks of w2
// in flight per wave)
template <typename Raw>
__global__ __launch_bounds__(kDW * 64) __attribute__((amdgpu_waves_per_eu(std::is_same_v<Raw, RawQ3> ? 3 : 4))) void
k_down_grouped(GroupedArgs p) {
  extern __shared__ __align__(16) uint16_t lds_g[];
  const int b = static_cast<int>(blockIdx.x);
  const int item = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) / kDKS;
  if (b < p.dn_shared) {
    if (p.T > kGNC) {
      down_shared_wide(p, b, lds_g);
      return;
    }
    const int rt = b * kDI + item;
    auto load_w = [&](RawBF16& r, uint32_t row, int kc) { load_raw_nc(r, p.ws2, row, p.Is, kc); };
    down_block<RawBF16>(p, load_w, [&](int) -> const void* { return p.ws2; }, rt, p.T, 0, true, lds_g);
    return;
  }
  const int rb = b - p.dn_shared;
  const int slot = rb / p.dn_groups;
  if (slot >= p.active[0]) return;
  const SlotDesc* d = p.desc + slot;
  const int rt = (rb % p.dn_groups) * kDI + item;
  if constexpr (std::is_same_v<Raw, RawQ3>) {
    if (p.q3fd) {
      down_block_q3f(p, slot, rt, d->n_tok, d->tok_base, lds_g);
      return;
    }
  }
  if constexpr (std::is_same_v<Raw, RawFP4>) {
    if (p.hplanes) {
      uint8_t* lds = reinterpret_cast<uint8_t*>(lds_g);
      switch (p.I / 128) {   // blocks of K per wave (grouped_h_planes)
        case 4: down_block_mx<4>(p, slot, rt, d->n_tok, d->tok_base, lds); break;
        case 8: down_block_mx<8>(p, slot, rt, d->n_tok, d->tok_base, lds); break;
        default: down_block_mx<16>(p, slot, rt, d->n_tok, d->tok_base, lds); break;
      }
      return;
    }
  }
  auto load_w = [&](Raw& r, uint32_t row, int kc) { load_w2_nc(r, p.desc, slot, row, p.I, kc); };
  auto wptr = [&](int i) { return desc_ptr(p.desc, slot, 6 + i); };   // 0: w2 codes, 1: w2 scales
  down_block<Raw>(p, load_w, wptr, rt, d->n_tok, d->tok_base, false, lds_g);
}

// The factored q3 gate/up: every wave's K range whole superblocks.
bool up_q3f(const dsk_moe_desc& d) {
  return d.quant == DSK_QUANT_Q3 && d.hidden % (kQ3gKS * 512) == 0 && d.hidden <= kQ3gMaxGroups * 64;
}

// The FP4 gate/up on scaled MFMAs: bf16 x (planes made from it), every wave's
// K range 2, 4, 6 or 8 whole blocks (up_block_mx's instances).
bool up_mx(const dsk_moe_desc& d) {
  const int per = d.hidden / 128 / kGKS;
  return d.quant == DSK_QUANT_FP4 && d.x_dtype == DSK_DTYPE_BF16 && d.hidden % (kGKS * 256) == 0 &&
         per >= 2 && per <= kGxMaxBlocks;
}

}  // namespace

// h as FP8 planes and the FP4 down on scaled MFMAs: the gate/up on scaled MFMAs
// (up_mx), I a whole 4, 8 or 16 blocks (down_block_mx's instances), and at most
// 512 dispatch rows (measured up to there): at 8 and 20 tokens (top-8) the down
// went 57.9 -> 50.5 and 102.8 -> 88.6 us; at 64 (once the shared expert's weights
// streamed once per call) 173.3 -> 157.7 us while the planes epilogue added
// 11.5 us to the gate/up.
bool grouped_up_mx(const dsk_moe_desc& d) { return up_mx(d); }

bool grouped_x_q3(const dsk_moe_desc& d) { return up_q3f(d); }

bool grouped_h_planes(const dsk_moe_desc& d) {
  return up_mx(d) && (d.inter == 512 || d.inter == 1024 || d.inter == 2048) &&
         static_cast<int64_t>(d.tokens) * d.top_k <= 512;
}

namespace {

size_t up_lds(const dsk_moe_desc& d) {
  const size_t x_tile = static_cast<size_t>(kGNC) * (d.hidden + 8) * 2;
  const size_t red = static_cast<size_t>(kGI) * kGKS * 2 * 64 * 4 * sizeof(float);
  // factored q3: the x tile, its group sums [H/128][8][2][2] f32, 64 zero bytes
  const size_t q3f = x_tile + static_cast<size_t>(d.hidden / 128) * kQ3fMaxTokens * 16 + 64;
  size_t base = x_tile > red ? x_tile : red;
  if (up_mx(d) && gx_lds_bytes(d.hidden) > base) base = gx_lds_bytes(d.hidden);
  if (d.tokens > kGNC && d.inter_shared > 0 && gs_up_lds_bytes() > base) base = gs_up_lds_bytes();
  return up_q3f(d) && q3f > base ? q3f : base;
}

hipError_t launch_x_q3(const dsk_moe_desc& d, const GroupedArgs& p, hipStream_t s) {
  const int64_t n = static_cast<int64_t>(d.tokens) * (d.hidden / 8);
  uint16_t* xq = reinterpret_cast<uint16_t*>(p.xp);
  float* xg = reinterpret_cast<float*>(p.xp + static_cast<size_t>(d.tokens) * d.hidden * 2);
  launch_kernel(k_x_q3, static_cast<unsigned>((n + 255) / 256), 256, 0, s, p.x, d.tokens, d.hidden, xq, xg);
  return hipGetLastError();
}

hipError_t launch_x_planes(const dsk_moe_desc& d, const GroupedArgs& p, hipStream_t s) {
  const int64_t n = static_cast<int64_t>(d.tokens) * (d.hidden / 8);
  launch_kernel(k_x_planes, static_cast<unsigned>((n + 255) / 256), 256, 0, s, p.x, d.tokens, d.hidden, p.xp);
  return hipGetLastError();
}

// The factored q3 down: K = I whole superblocks.
bool down_q3f(const dsk_moe_desc& d) { return d.quant == DSK_QUANT_Q3 && d.inter % 512 == 0; }

size_t down_lds(const dsk_moe_desc& d) {
  const int K = d.inter > d.inter_shared ? d.inter : d.inter_shared;
  const size_t h_tile = 2 * static_cast<size_t>(kGNC) * (K + 8) * 2;
  const size_t red = static_cast<size_t>(kDI) * kDKS * 64 * 4 * sizeof(float);
  const size_t base = h_tile > red ? h_tile : red;
  // factored q3: the h tile of I, its group sums [I/128][8][2][2] f32, 64 zero bytes
  const size_t q3f = 2 * static_cast<size_t>(kGNC) * (d.inter + 8) * 2 +
                     static_cast<size_t>(d.inter / 128) * kQ3fMaxTokens * 16 + 64;
  const size_t mx = grouped_h_planes(d) ? gd_lds_bytes(d.inter) : 0;
  size_t b2 = mx > base ? mx : base;
  if (d.tokens > kGNC && d.inter_shared > 0 && gs_down_lds_bytes() > b2) b2 = gs_down_lds_bytes();
  return down_q3f(d) && q3f > b2 ? q3f : b2;
}

}  // namespace

bool grouped_path(const dsk_moe_desc& d) {
  // FP4 reads 2-block scale windows: an even number of K blocks in every
  // wave's range (down: I % 256 == 0; gate/up, 4 ranges: H % 1024 == 0)
  return d.x_dtype == DSK_DTYPE_BF16 && d.hidden % (kGI * 16) == 0 && d.hidden % (kDI * 16) == 0 &&
         (d.quant != DSK_QUANT_FP4 || (d.inter % 256 == 0 && d.hidden % (kGKS * 256) == 0)) &&
         d.hidden % 128 == 0 && d.inter % 128 == 0 && d.inter % (kGI * 16) == 0 &&
         d.inter_shared % 128 == 0 && d.inter_shared % (kGI * 16) == 0 &&
         up_lds(d) <= kMaxLds && down_lds(d) <= kMaxLds;
}

namespace {

GroupedArgs grouped_args(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a, const SlotDesc* desc,
                         const int32_t* xrow, const float* wrow) {
  GroupedArgs p{};
  p.T = d.tokens; p.H = d.hidden; p.I = d.inter; p.Is = d.inter_shared; p.k = d.top_k; p.limit = d.limit;
  p.desc = desc; p.active = a.active; p.xrow = xrow; p.wrow = wrow;
  p.x = static_cast<const uint16_t*>(a.x);
  p.ws1 = static_cast<const uint16_t*>(a.ws1);
  p.ws3 = static_cast<const uint16_t*>(a.ws3);
  p.ws2 = static_cast<const uint16_t*>(a.ws2);
  p.h_hi = reinterpret_cast<uint16_t*>(a.ws + L.h_hi);
  p.h_lo = reinterpret_cast<uint16_t*>(a.ws + L.h_lo);
  p.hs_hi = reinterpret_cast<uint16_t*>(a.ws + L.hs_hi);
  p.hs_lo = reinterpret_cast<uint16_t*>(a.ws + L.hs_lo);
  p.y = rows_buffer(a.rows_out, a.ws, L);
  p.ys = reinterpret_cast<float*>(a.ws + L.ys);
  p.q3f = up_q3f(d) ? 1 : 0;
  p.q3fd = down_q3f(d) ? 1 : 0;
  p.mx = up_mx(d) ? d.hidden / 128 / kGKS : 0;
  p.xp = reinterpret_cast<uint8_t*>(a.ws + L.xp);
  p.hplanes = 0;   // set by the launchers where the grouped gate/up writes h
  p.hp = reinterpret_cast<uint8_t*>(a.ws + L.hp);
  p.up_groups = p.q3f ? d.inter / 16 : d.inter / 16 / kGI;   // factored q3: one row tile per block
  // shared gate/up: past kGNC tokens, four row tiles per block (up_shared_wide)
  p.up_shared = d.tokens > kGNC ? (d.inter_shared / 16 + kGW / 2 - 1) / (kGW / 2) : d.inter_shared / 16 / kGI;
  p.dn_groups = d.hidden / 16 / kDI;
  p.dn_shared = d.inter_shared > 0 ? p.dn_groups : 0;
  return p;
}

int max_slots(const dsk_moe_desc& d) { return d.n_experts < d.tokens * d.top_k ? d.n_experts : d.tokens * d.top_k; }

hipError_t grouped_down(const dsk_moe_desc& d, const GroupedArgs& p, hipStream_t s, int repeat) {
  const unsigned blocks = static_cast<unsigned>(p.dn_shared + max_slots(d) * p.dn_groups);
  const size_t lds = down_lds(d);
  for (int r = 0; r < repeat; ++r) {
    if (d.quant == DSK_QUANT_Q3) launch_kernel(k_down_grouped<RawQ3>, blocks, kDW * 64, lds, s, p);
    else launch_kernel(k_down_grouped<RawFP4>, blocks, kDW * 64, lds, s, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_experts_grouped(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a,
                                  const SlotDesc* desc, const int32_t* xrow, const float* wrow, hipStream_t s,
                                  int repeat) {
  GroupedArgs p = grouped_args(d, L, a, desc, xrow, wrow);
  p.hplanes = grouped_h_planes(d) ? 1 : 0;
  const unsigned up_blocks = static_cast<unsigned>(p.up_shared + max_slots(d) * p.up_groups);
  const size_t ul = up_lds(d);
  hipError_t e;
  if ((e = stage_open(kStageUp)) != hipSuccess) return e;
  for (int r = 0; r < repeat; ++r) {
    if (p.mx && !a.x_planes_ready && (e = launch_x_planes(d, p, s)) != hipSuccess) return e;
    if (p.q3f && !a.x_planes_ready && (e = launch_x_q3(d, p, s)) != hipSuccess) return e;
    if (d.quant == DSK_QUANT_Q3) launch_kernel(k_up_grouped<RawQ3>, up_blocks, kGW * 64, ul, s, p);
    else launch_kernel(k_up_grouped<RawFP4>, up_blocks, kGW * 64, ul, s, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if ((e = stage_open(kStageDown)) != hipSuccess) return e;
  return grouped_down(d, p, s, repeat);
}

hipError_t launch_grouped_up_routed(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a,
                                    const SlotDesc* desc, const int32_t* xrow, const float* wrow, hipStream_t s,
                                    int repeat, bool x_planes_ready) {
  GroupedArgs p = grouped_args(d, L, a, desc, xrow, wrow);
  p.up_shared = 0;
  p.hplanes = grouped_h_planes(d) ? 1 : 0;
  const unsigned blocks = static_cast<unsigned>(max_slots(d) * p.up_groups);
  const size_t lds = up_lds(d);
  for (int r = 0; r < repeat; ++r) {
    if (p.mx && !x_planes_ready) {
      const hipError_t e = launch_x_planes(d, p, s);
      if (e != hipSuccess) return e;
    }
    if (p.q3f) {
      const hipError_t e = launch_x_q3(d, p, s);
      if (e != hipSuccess) return e;
    }
    if (d.quant == DSK_QUANT_Q3) launch_kernel(k_up_grouped<RawQ3>, blocks, kGW * 64, lds, s, p);
    else launch_kernel(k_up_grouped<RawFP4>, blocks, kGW * 64, lds, s, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_grouped_down(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a,
                               const SlotDesc* desc, hipStream_t s, int repeat, bool h_planes) {
  GroupedArgs p = grouped_args(d, L, a, desc, nullptr, nullptr);
  p.hplanes = h_planes ? 1 : 0;
  return grouped_down(d, p, s, repeat);
}

}  // namespace dsk
