// Decode pipeline of the expert products (up to 16 tokens and 64 routed
// positions), after the gate kernel has written the scores:
//   k_route_shared  block 0: top-k and slot map (descriptors, token ->
//                   dispatch-row map, row weights); the other blocks: the
//                   shared expert's gate/up -> hs;
//   k_up_stream     routed gate/up tiles of the active experts (FP4 or q3) -> h;
//   k_down_decode[_staged]  per 16 output rows: every active expert's w2 rows in
//                   ascending expert id, then the shared expert's w2 rows
//                   (bf16), and the final add and cast -- no separate combine.
// Token slot of the MFMA tiles = token index (T <= 16), so the products of
// all experts accumulate into one tile; tokens not routed to an expert get a
// zero B operand.  Replaces the per-expert loop, the shared expert and the
// combine of the reference's moe_layer (src/deepseeker/mlx_forward.py:388-419,
// src/deepseeker/mlx_runner.py:765-783).
#include "block_route.h"
#include "mx.h"
#include "resnorm.h"
#include "tile.h"

namespace dsk {
namespace {

constexpr int kUpItems = 2;            // row tiles of a gate/up block
constexpr int kUpKS = 4;               // K splits of a row tile (one wave each)
constexpr int kUpW = kUpItems * kUpKS; // waves of a gate/up block
constexpr int kUpXRegChunks = 1;       // x chunks per thread staged through registers
constexpr int kUpBatch = 4;            // K blocks per weight batch (two batches in flight)
constexpr int kDownW = 16;             // waves of a down block (split K = I and Is)
constexpr int kDownGroup = 8;          // experts whose w2 blocks a wave holds at once
// staged down kernel (all h rows in LDS)
constexpr int kStW = 8;                // waves
constexpr int kStKB = 2;               // K blocks of each expert per wave (I = kStW * kStKB * 128)
constexpr int kStSlots = 2;            // experts per routed batch
constexpr int kStMaxSlots = 16;        // active experts the staged kernel handles
// routed batches in flight per wave: one (the next is loaded once the current one
// has landed).  Every CU asking for all of its weights at once was slower at one
// token (down 17.2 us) than one batch at a time (15.3 us): the products of a batch
// then overlap the later batches' loads instead of waiting for the last byte.
constexpr int kStRing = 1;
constexpr int kStRedBytes = 2 * kStW * 64 * 4 * 4;   // wave partial sums, routed and shared

struct DecodeArgs {
  int T, H, I, Is, k;
  float limit;
  const SlotDesc* desc; const int32_t* active; const int32_t* rowmap; const float* wrow;
  // routing block of k_route_shared: gate scores and selection bias in, routing out
  float* scores; const float* bias; const dsk_expert_ptrs* table;
  int E; float route_scale;
  DecodeRoute route;
  // gate scores of k_gate_shared
  const void* gate_w; int score_func;
  // shared output of k_route_sdown [T][H] (x dtype)
  void* shared_x;
  int route_lds;                       // LDS bytes of the routing kernels' launch
  const void* x; int x_f32;
  const uint16_t* ws1; const uint16_t* ws3;   // shared w1, w3 [Is][H] bf16
  uint16_t* hs_hi; uint16_t* hs_lo;    // [T][Is]
  uint16_t* h_hi; uint16_t* h_lo;      // [T*k][I] by dispatch row
  uint8_t* hq; uint8_t* hqs;           // MX: [slot][3T][I] FP8 planes, [slot][3T][I/32] E8M0
  const uint16_t* ws2;                 // shared w2 [H][Is] bf16
  const void* shared_out;              // precomputed shared output [T][H] (x dtype) or null
  void* out;                           // [T][H] x dtype
  int up_tiles;                        // I / 16
  ResNorm rn; int norm;                // norm: k_gate_shared computes x from the residual stream
  uint8_t* xp;                         // k_route_shared: also write x's FP8 planes here (or null)
};

// One x chunk (8 values at column `col` of token row t) into the LDS planes.
__device__ __forceinline__ void put_x_chunk(uint16_t* xh, uint16_t* xl, int off, const u32x4& v0,
                                            const u32x4& v1, bool f32) {
  if (!f32) {
    *reinterpret_cast<u32x4*>(xh + off) = v0;
    return;
  }
  const float f[8] = {__uint_as_float(v0.x), __uint_as_float(v0.y), __uint_as_float(v0.z),
                      __uint_as_float(v0.w), __uint_as_float(v1.x), __uint_as_float(v1.y),
                      __uint_as_float(v1.z), __uint_as_float(v1.w)};
  uint16_t h[8], l[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) split_bf16(f[q], h[q], l[q]);
  *reinterpret_cast<u32x4*>(xh + off) = pack_bf16x8(h);
  *reinterpret_cast<u32x4*>(xl + off) = pack_bf16x8(l);
}

// One batch of G K blocks of a wave's gate and up rows: FP4 codes, and either
// one 4-byte scale window per lane (kWin: lane group g holds the four scale
// bytes of K block kb + g, one per lane group) or one scale byte per K block.
template <int G>
struct UpBatch {
  u32x4 c1[G], c3[G];
  uint32_t s1[G], s3[G];
  uint32_t w1[G / 4], w3[G / 4];
};

// Loads without conditions (see load_raw_nc): blocks past the wave's range
// re-read its last block and rows past the tile read row 0; mma_batch gives
// them a zero B operand and their rows are not stored.  k1 >= 1.
template <int G, bool kWin>
__device__ __forceinline__ void load_batch(UpBatch<G>& b, const uint8_t* W1, const uint8_t* S1,
                                           const uint8_t* W3, const uint8_t* S3, uint32_t row, int K,
                                           int kb, int k1, int g4, bool rok) {
  // 32-bit offsets from the (uniform) role base pointers: one expert role is < 4 GB
  const uint32_t rowc = rok ? row : 0u;
  const uint32_t cb = rowc * static_cast<uint32_t>(K / 2), sb = rowc * static_cast<uint32_t>(K / 32);
  if constexpr (kWin) {
#pragma unroll
    for (int v = 0; v < G / 4; ++v) {
      const int kw = min(kb + 4 * v + g4, k1 - 1);    // K block whose scales this lane fetches
      b.w1[v] = ldg<uint32_t>(S1 + sb + 4 * kw);
      b.w3[v] = ldg<uint32_t>(S3 + sb + 4 * kw);
    }
  }
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int kc = min(min(kb + i, k1 - 1) * 128 + g4 * 32, K - 32);
    b.c1[i] = ldg16(W1 + cb + kc / 2);
    b.c3[i] = ldg16(W3 + cb + kc / 2);
    if constexpr (!kWin) {
      b.s1[i] = ldg<uint8_t>(S1 + sb + kc / 32);
      b.s3[i] = ldg<uint8_t>(S3 + sb + kc / 32);
    }
  }
}

// Scale windows -> per-lane scale bytes through a wave-private LDS tile
// xch[2][16][20] (role, row, 16 bytes + pad).
template <int G, bool kWin>
__device__ __forceinline__ void batch_scales(UpBatch<G>& b, uint8_t* xch, int r16, int g4) {
  if constexpr (kWin) {
#pragma unroll
    for (int v = 0; v < G / 4; ++v) {
      uint8_t* r1 = xch + r16 * 20;
      uint8_t* r3 = xch + 320 + r16 * 20;
      *reinterpret_cast<uint32_t*>(r1 + 4 * g4) = b.w1[v];
      *reinterpret_cast<uint32_t*>(r3 + 4 * g4) = b.w3[v];
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        b.s1[4 * v + i] = r1[4 * i + g4];
        b.s3[4 * v + i] = r3[4 * i + g4];
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
}

template <int G>
__device__ __forceinline__ void mma_batch(const UpBatch<G>& b, const uint16_t* xh, const uint16_t* xl,
                                          int K, int kb, int k1, int g4, bool tv, bool two_planes,
                                          f32x4& ag, f32x4& au) {
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int kc = (kb + i) * 128 + g4 * 32;
    const bool ok = tv && kb + i < k1 && kc < K;
    const RawFP4 r1{b.c1[i], b.s1[i]}, r3{b.c3[i], b.s3[i]};
    mma_block2(r1, r3, xh, kc, ok, ag, au);
    if (two_planes) mma_block2(r1, r3, xl, kc, ok, ag, au);
  }
}

// The tokens' activations x [T][H] of a gate/up block: into registers xv when
// they fit (returns true; put_staged_x writes them to the LDS planes later,
// once the block's weight loads are in flight), else straight into the LDS
// planes xh / xl (row stride xs).
template <bool kF32, int NT>
__device__ __forceinline__ bool load_x(const DecodeArgs& p, uint16_t* xh, uint16_t* xl, int xs, int tid,
                                       u32x4 (&xv)[kUpXRegChunks][2]) {
  const int K = p.H, cpr = K / 8, xchunks = p.T * cpr;
  if (xchunks <= kUpXRegChunks * NT) {
#pragma unroll
    for (int j = 0; j < kUpXRegChunks; ++j) {
      const int c = min(tid + j * NT, xchunks - 1);   // no condition on the load (see load_raw_nc)
      const int64_t e = static_cast<int64_t>(c / cpr) * K + (c % cpr) * 8;
      if (!kF32) {
        xv[j][0] = ldg16(static_cast<const uint16_t*>(p.x) + e);
      } else {
        xv[j][0] = ldg16(static_cast<const float*>(p.x) + e);
        xv[j][1] = ldg16(static_cast<const float*>(p.x) + e + 4);
      }
    }
    return true;
  }
  for (int c = tid; c < xchunks; c += NT) {
    const int64_t e = static_cast<int64_t>(c / cpr) * K + (c % cpr) * 8;
    const int off = (c / cpr) * xs + (c % cpr) * 8;
    if (!kF32) put_x_chunk(xh, xl, off, ldg16(static_cast<const uint16_t*>(p.x) + e), u32x4{}, false);
    else put_x_chunk(xh, xl, off, ldg16(static_cast<const float*>(p.x) + e),
                     ldg16(static_cast<const float*>(p.x) + e + 4), true);
  }
  return false;
}

template <bool kF32, int NT>
__device__ __forceinline__ void put_staged_x(const DecodeArgs& p, uint16_t* xh, uint16_t* xl, int xs, int tid,
                                             const u32x4 (&xv)[kUpXRegChunks][2]) {
  const int cpr = p.H / 8, xchunks = p.T * cpr;
#pragma unroll
  for (int j = 0; j < kUpXRegChunks; ++j) {
    const int c = tid + j * NT;
    if (c < xchunks) put_x_chunk(xh, xl, (c / cpr) * xs + (c % cpr) * 8, xv[j][0], xv[j][1], kF32);
  }
}

// Shared-expert gate/up tile rt (block = NW waves, ROWS (8 or 16) rows of w1
// and w3, all K; wave w takes the w-th K range).  16 rows: two K blocks in
// flight.  8 rows (T <= 8): the MFMA's A rows 8..15 hold the same 8 weight
// rows at the next K block and its B columns 8..15 the tokens' activations
// there, so one MFMA covers a pair of K blocks (D rows 0..7 x columns 0..7
// and rows 8..15 x columns 8..15 are added once at the end); the wave's four
// K blocks are then all in flight in the registers of two, and twice the
// tiles spread the shared stream over twice the CUs.  Called after the
// block's x chunks have been loaded into registers; writes them to LDS once
// its own weight loads are in flight.  kNorm: called after the loads of the
// residual rows instead (resnorm_issue into rin), and normalises them
// into the planes once its weight loads are in flight.
template <bool kF32, int NW, int ROWS, bool kNorm = false>
__device__ __forceinline__ void shared_up_tile(const DecodeArgs& p, int rt, uint16_t* xh, uint16_t* xl, int xs,
                                               bool xreg, const u32x4 (&xv)[kUpXRegChunks][2], uint16_t* lds,
                                               int tid, int lane, int wave, int r16, int g4,
                                               ResNormIn<NW * 64>* rin = nullptr, float* rn_wsum = nullptr) {
  const int T = p.T, K = p.H;
  const uint32_t row = static_cast<uint32_t>(rt * ROWS + (r16 & (ROWS - 1)));
  const int nblk = (K + 127) / 128;
  const int per = (nblk + NW - 1) / NW;
  const int k0 = min(wave * per, nblk), k1 = min(k0 + per, nblk);
  // 8 rows: this lane's half of a K-block pair (A row r16 and B column r16 agree)
  constexpr int kStep = ROWS == 8 ? 2 : 1;            // K blocks per MFMA group
  const int half = ROWS == 8 ? (r16 >> 3) : 0;
  const int tok = ROWS == 8 ? (r16 & 7) : r16;        // this lane's B column token
  const bool tv = tok < T;
  RawBF16 a1, a3, b1, b3;
  auto ld = [&](RawBF16& r1, RawBF16& r3, int kb) {
    // no condition (see load_raw_nc): past the range, the last block again
    const int kc = min(min(kb + half, k1 - 1) * 128 + g4 * 32, K - 32);
    load_raw_nc(r1, p.ws1, row, K, kc);
    load_raw_nc(r3, p.ws3, row, K, kc);
  };
  ld(a1, a3, k0);
  ld(b1, b3, k0 + kStep);
  if constexpr (kNorm) {
    // the rows (their loads issued before these) normalised into the planes; ends on a barrier
    resnorm_rows<NW * 64>(p.rn, T, K, xh, xs, rt == 0, rn_wsum, *rin);
  } else {
    if (xreg) put_staged_x<kF32, NW * 64>(p, xh, xl, xs, tid, xv);
    __syncthreads();
  }
  const uint16_t* bh = xh + (tv ? tok : 0) * xs;
  const uint16_t* bl = xl + (tv ? tok : 0) * xs;
  f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = ag;
  auto mm = [&](const RawBF16& r1, const RawBF16& r3, int kb) {
    const int kbl = kb + half;
    const int kc = kbl * 128 + g4 * 32;
    const bool ok = tv && kbl < k1 && kc < K;
    mma_block2(r1, r3, bh, kc, ok, ag, au);
    if (kF32) mma_block2(r1, r3, bl, kc, ok, ag, au);
  };
  for (int kb = k0; kb < k1; kb += 2 * kStep) {
    mm(a1, a3, kb);
    if (kb + 2 * kStep < k1) ld(a1, a3, kb + 2 * kStep);
    if (kb + kStep < k1) mm(b1, b3, kb + kStep);
    if (kb + 3 * kStep < k1) ld(b1, b3, kb + 3 * kStep);
  }
  if constexpr (ROWS == 8) {
    // D[r][t] (K blocks of the first halves) + D[8 + r][8 + t] (second halves):
    // lane l (rows 4 g4 .., column r16) and lane l + 40
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ag[q] += __shfl_down(ag[q], 40, 64);
      au[q] += __shfl_down(au[q], 40, 64);
    }
  }
  // K ranges added in wave order; the partial sums reuse the activation area
  // once every wave is done with it
  float (*red)[2][64][4] = reinterpret_cast<float (*)[2][64][4]>(lds);
  __syncthreads();
  *reinterpret_cast<f32x4*>(&red[wave][0][lane][0]) = ag;
  *reinterpret_cast<f32x4*>(&red[wave][1][lane][0]) = au;
  __syncthreads();
  if (wave == 0 && tv && g4 < ROWS / 4 && (ROWS == 16 || r16 < 8)) {
#pragma unroll
    for (int w = 1; w < NW; ++w) {
      ag += *reinterpret_cast<const f32x4*>(&red[w][0][lane][0]);
      au += *reinterpret_cast<const f32x4*>(&red[w][1][lane][0]);
    }
    uint16_t hh[4], hl[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) split_bf16(silu_clamped(ag[q], au[q], p.limit), hh[q], hl[q]);
    const int64_t off = static_cast<int64_t>(tok) * p.Is + rt * ROWS + 4 * g4;
    *reinterpret_cast<uint2*>(p.hs_hi + off) = uint2{hh[0] | (uint32_t(hh[1]) << 16), hh[2] | (uint32_t(hh[3]) << 16)};
    *reinterpret_cast<uint2*>(p.hs_lo + off) = uint2{hl[0] | (uint32_t(hl[1]) << 16), hl[2] | (uint32_t(hl[3]) << 16)};
  }
}

// The decode pipeline's first two kernels carry the shared expert beside the
// routing: k_gate_shared computes the gate scores and the shared expert's
// gate/up (both need only x), k_route_sdown runs the top-k and slot map in
// one block beside the shared expert's down product, which it writes to
// shared_x in x's dtype (the routed down kernels then add it as a
// precomputed shared output).
// Shared gate/up tiles of 8 rows up to 8 tokens (a 2048-row shared expert:
// 256 tiles; K-block pairs per MFMA, see shared_up_tile), else 16.
constexpr int kRsW = 8;
// LDS of both kernels: the routing block's state and after it the expert
// pointer table, a shared gate/up tile's activation planes and then (over
// them) its wave partial sums [kRsW][2][64][4] f32, a shared down tile's
// wave partial sums [kRsW][64][4] f32, or two gate tiles' segment sums.
constexpr size_t kRsRedBytes = kRsW * 2 * 64 * 4 * 4;
constexpr size_t kRsTabOffset = (kBlockRouteLds + 15) / 16 * 16;
static_assert(kRsTabOffset < kRsRedBytes, "routing block state must fit the route/shared LDS");
constexpr int kRsTileDelay = 15;   // x 64 clocks (~0.4 us)
// k_gate_shared's gate blocks: the normalised rows after the two tiles' segment sums
constexpr size_t kGsNormOffset = 64;

__host__ __device__ inline int shared_up_tiles(int T, int Is) { return Is / (T <= 8 ? 8 : 16); }

// Blocks [0, shared_up_tiles): one shared gate/up tile each; the rest: two
// gate tiles each (waves 0-3 and 4-7: one token x one expert of the score
// grid, tile = token * E + expert, as the router's own gate kernel).
// kNorm: with the residual stream given, every block normalises the rows
// itself (into its activation planes, or after the gate tiles' segment sums)
// while its first weights load, and block 0 also writes the new stream and
// the rows for the later kernels (resnorm.h).
template <bool kF32, bool kWBF16, bool kNorm = false>
__global__ __launch_bounds__(kRsW * 64) __attribute__((amdgpu_waves_per_eu(4))) void k_gate_shared(
    DecodeArgs p) {
  static_assert(!(kNorm && kF32), "the residual stream is bf16");
  extern __shared__ __align__(16) uint16_t lds_up[];
  __shared__ float rn_wsum[kResNormWsum];
  const int tid = threadIdx.x, lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_sh = shared_up_tiles(p.T, p.Is);
  const int b = static_cast<int>(blockIdx.x);
  if (b < n_sh) {
    const int r16 = lane & 15, g4 = lane >> 4;
    const int xs = p.H + 8;
    uint16_t* xh = lds_up;
    uint16_t* xl = lds_up + p.T * xs;
    u32x4 xv[kUpXRegChunks][2];
    if constexpr (kNorm) {
      ResNormIn<kRsW * 64> in;
      resnorm_issue<kRsW * 64>(p.rn, p.T, p.H, in);
      asm volatile("" ::: "memory");   // the rows' loads first: waiting for them leaves the weights in flight
      // T <= kResNormRows: 8-row tiles
      shared_up_tile<kF32, kRsW, 8, true>(p, b, xh, xl, xs, false, xv, lds_up, tid, lane, wave, r16, g4, &in,
                                          rn_wsum);
      return;
    }
    const bool xreg = load_x<kF32, kRsW * 64>(p, xh, xl, xs, tid, xv);
    if (p.T <= 8) shared_up_tile<kF32, kRsW, 8>(p, b, xh, xl, xs, xreg, xv, lds_up, tid, lane, wave, r16, g4);
    else shared_up_tile<kF32, kRsW, 16>(p, b, xh, xl, xs, xreg, xv, lds_up, tid, lane, wave, r16, g4);
    return;
  }
  const int tile = 2 * (b - n_sh) + (wave >> 2);
  const bool active = tile < p.T * p.E;
  const int t = active ? tile / p.E : 0, e = active ? tile - t * p.E : 0;
  float* segsum = reinterpret_cast<float*>(lds_up) + (wave >> 2) * kSegments;
  if constexpr (kNorm) {
    uint16_t* y = lds_up + kGsNormOffset / 2;
    ResNormIn<kRsW * 64> in;
    resnorm_issue<kRsW * 64>(p.rn, p.T, p.H, in);
    asm volatile("" ::: "memory");
    GateWFirst<1, 1, kWBF16> pre;
    gate_w_issue<1, 1, kWBF16>(p.gate_w, p.H, p.E, e, wave & 3, lane, active, pre);
    resnorm_rows<kRsW * 64>(p.rn, p.T, p.H, y, p.H, b == 0, rn_wsum, in);
    gate_tile<1, 1, true, kWBF16, true>(y, p.gate_w, p.T, p.H, p.E, p.score_func, p.scores, t, e, wave & 3,
                                        lane, tid & 255, segsum, active, &pre);
  } else {
    gate_tile<1, 1, !kF32, kWBF16>(p.x, p.gate_w, p.T, p.H, p.E, p.score_func, p.scores, t, e, wave & 3, lane,
                                   tid & 255, segsum, active);
  }
}

// Shared down tile rb of k_route_sdown: output rows 16 rb .. 16 rb + 15 of
// the shared expert, K (its intermediate) split over the block's waves in
// 128-wide blocks (wave w: blocks w, w + kRsW, ...), bf16 MFMAs on the rows
// of w2 and the hs planes read straight from global memory (B column c:
// plane c & 1 of token t0 + c / 2, eight tokens per pass).  Wave sums added
// in order, then hi + lo, rounded to x's dtype into shared_x.
template <bool kF32>
__device__ __forceinline__ void shared_down_tile(const DecodeArgs& p, int rb, float (*red)[64][4], int lane,
                                                 int wave) {
  const int r16 = lane & 15, g4 = lane >> 4;
  const int T = p.T, Is = p.Is, H = p.H;
  const int row0 = rb * 16;
  const uint32_t row = static_cast<uint32_t>(row0 + r16);
  const int nkb = (Is + 127) / 128;
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  for (int t0 = 0; t0 < T; t0 += 8) {
    const int t = min(t0 + (r16 >> 1), T - 1);   // columns past the last token repeat it (not used)
    const uint16_t* hrow = ((r16 & 1) ? p.hs_lo : p.hs_hi) + static_cast<int64_t>(t) * Is;
    f32x4 acc[4] = {z, z, z, z};
    for (int kb = wave; kb < nkb; kb += 2 * kRsW) {
      // two K blocks in flight, loads without conditions (past the end: the last block again)
      RawBF16 w[2], h[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int kc = min(min(kb + j * kRsW, nkb - 1) * 128 + g4 * 32, Is - 32);
        load_raw_nc(w[j], p.ws2, row, Is, kc);
        load_raw_nc(h[j], hrow, 0, 0, kc);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int kbj = kb + j * kRsW;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const bool ok = kbj < nkb && kbj * 128 + g4 * 32 + 8 * jj < Is;
          acc[jj] = mfma16(a_operand(w[j], jj), ok ? as_bf16x8(h[j].v[jj]) : bf16x8{}, acc[jj]);
        }
      }
    }
    *reinterpret_cast<f32x4*>(&red[wave][lane][0]) = ((acc[0] + acc[1]) + acc[2]) + acc[3];
    __syncthreads();
    if (wave == 0) {
      f32x4 a = z;
      for (int w = 0; w < kRsW; ++w) a += *reinterpret_cast<const f32x4*>(&red[w][lane][0]);
#pragma unroll
      for (int q = 0; q < 4; ++q) a[q] += lane_xor1(a[q]);
      const int tok = t0 + (r16 >> 1);
      if ((r16 & 1) == 0 && tok < T) {
        const int64_t o = static_cast<int64_t>(tok) * H + row0 + 4 * g4;
        if constexpr (kF32) {
          *reinterpret_cast<f32x4*>(static_cast<float*>(p.shared_x) + o) = a;
        } else {
          *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.shared_x) + o) =
              uint2{f32_to_bf16_bits(a[0]) | (uint32_t(f32_to_bf16_bits(a[1])) << 16),
                    f32_to_bf16_bits(a[2]) | (uint32_t(f32_to_bf16_bits(a[3])) << 16)};
        }
      }
    }
    __syncthreads();
  }
}

// Block 0: top-k of every token and the slot map of the routed kernels
// (block_route); blocks 1 .. H/16: shared down tiles.  The routing block's
// dependent loads and wave reductions overlap the shared expert's stream.
template <bool kF32>
__global__ __launch_bounds__(kRsW * 64) __attribute__((amdgpu_waves_per_eu(4))) void k_route_sdown(
    DecodeArgs p) {
  extern __shared__ __align__(16) uint16_t lds_up[];
  if (blockIdx.x == 0) {
    block_route(lds_up, p.scores, p.bias, p.T, p.E, p.k, p.route_scale, p.table, p.route,
                reinterpret_cast<uint64_t*>(lds_up + kRsTabOffset / 2),
                static_cast<int>((p.route_lds - static_cast<int>(kRsTabOffset)) / 8));
    return;
  }
  const int tid = threadIdx.x, lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // The routing block's loads (scores, bias, pointer table) are the kernel's
  // critical path: behind the tiles' weight stream their latency grows
  // several-fold, so the tiles hold their first loads back until those have
  // had time to return.
  if (p.T <= 2) __builtin_amdgcn_s_sleep(kRsTileDelay);
  shared_down_tile<kF32>(p, static_cast<int>(blockIdx.x) - 1, reinterpret_cast<float (*)[64][4]>(lds_up), lane,
                         wave);
}

// Outside the MX kernels the decode pipeline keeps the shared expert's gate/up
// beside the routing and its down in the routed down kernels (the gate kernel
// alone before): block 0 runs the top-k and slot map, blocks 1 ..
// shared_up_tiles the shared gate/up tiles -> hs.
template <bool kF32>
__global__ __launch_bounds__(kRsW * 64) __attribute__((amdgpu_waves_per_eu(4))) void k_route_shared(
    DecodeArgs p) {
  extern __shared__ __align__(16) uint16_t lds_up[];
  if (blockIdx.x == 0) {
    block_route(lds_up, p.scores, p.bias, p.T, p.E, p.k, p.route_scale, p.table, p.route,
                reinterpret_cast<uint64_t*>(lds_up + kRsTabOffset / 2),
                static_cast<int>((p.route_lds - static_cast<int>(kRsTabOffset)) / 8));
    return;
  }
  const int tid = threadIdx.x, lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // At one or two tokens the routing block ends the kernel: its score loads
  // wait for whatever the tile block beside it on the same CU requested
  // first.  The tile blocks wait ~0.5 us (19 x 64 clocks) before their first
  // loads, so the routing block's go out ahead of them.
  if (p.T <= 2) __builtin_amdgcn_s_sleep(19);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int xs = p.H + 8;
  uint16_t* xh = lds_up;
  uint16_t* xl = lds_up + p.T * xs;
  u32x4 xv[kUpXRegChunks][2];
  const bool xreg = load_x<kF32, kRsW * 64>(p, xh, xl, xs, tid, xv);
  const int rt = static_cast<int>(blockIdx.x) - 1;
  if (p.T <= 8) shared_up_tile<kF32, kRsW, 8>(p, rt, xh, xl, xs, xreg, xv, lds_up, tid, lane, wave, r16, g4);
  else shared_up_tile<kF32, kRsW, 16>(p, rt, xh, xl, xs, xreg, xv, lds_up, tid, lane, wave, r16, g4);
  if constexpr (!kF32) {
    if (p.xp && tid < 16) {
      // x's FP8 planes for the grouped FP4 gate/up, 16 chunks per tile block (the
      // 16 lanes iterate together: every group of four chunks is exchanged whole)
      const int n = p.T * (p.H / 8), stride = (static_cast<int>(gridDim.x) - 1) * 16;
      for (int c = rt * 16 + tid; c - tid < n; c += stride)
        x_planes_chunk(static_cast<const uint16_t*>(p.x), p.T, p.H, min(c, n - 1), c < n, p.xp);
    }
  }
}

// Routed gate/up of the decode pipeline.  Each block takes kUpItems row
// tiles of one active expert, kUpKS waves per tile, each streaming one K
// range of its FP4 (or q3) w1/w3 rows in batches of G K blocks;
// h[drow] = SwiGLU(gate, up) * route weight.  The first batch is issued with
// the tokens' activations, which are written to LDS once the batch is in
// flight; the next batch goes out when the first is about to be used, so two
// are in flight from then on (FP4); K ranges are added in wave order.
template <int G, bool kWin, bool kF32, bool kQ3>
__global__ __launch_bounds__(kUpW * 64) __attribute__((amdgpu_waves_per_eu(kF32 ? 3 : 4))) void k_up_stream(DecodeArgs p) {
  extern __shared__ __align__(16) uint16_t lds_up[];
  // wave-uniform indices in scalar registers
  const int tid = threadIdx.x, lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int groups = (p.up_tiles + kUpItems - 1) / kUpItems;
  const int rb = static_cast<int>(blockIdx.x);
  const int slot = rb / groups;
  if (slot >= p.active[0]) return;
  const int T = p.T, K = p.H;
  const int item = wave / kUpKS, ks = wave % kUpKS;
  const int rt = (rb % groups) * kUpItems + item;
  const bool rok = rt < p.up_tiles;
  const int drow = r16 < T ? p.rowmap[slot * T + r16] : -1;
  const bool tv = drow >= 0;
  const int xs = K + 8;                       // padded LDS row stride (elements)
  constexpr bool f32 = kF32;
  uint16_t* xh = lds_up;
  uint16_t* xl = lds_up + T * xs;
  u32x4 xv[kUpXRegChunks][2];
  const bool xreg = load_x<kF32, kUpW * 64>(p, xh, xl, xs, tid, xv);
  const SlotDesc* d = p.desc + slot;
  const uint32_t row = static_cast<uint32_t>(rt * 16 + r16);
  const int nblk = (K + 127) / 128;
  const int per = (nblk + kUpKS - 1) / kUpKS;
  const int k0 = min(ks * per, nblk), k1 = min(k0 + per, nblk);
  float (*red)[kUpKS][2][64][4] =
      reinterpret_cast<float (*)[kUpKS][2][64][4]>(lds_up + (f32 ? 2 : 1) * T * xs);
  f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = ag;
  float wr = 0.0f;
  if constexpr (kQ3) {
    // weights: two batches of G K blocks in flight (q3 codes, scale and bias
    // per lane).  kWin: each batch's 2G (scale, bias) groups of a row come as
    // one 16-byte window per role, and every lane picks its group's pair from
    // it (the batch lies inside the row, see the launcher).
    RawQ3 a1[G], a3[G], b1[G], b3[G];
    u32x4 aw[4], bw[4];   // windows: scales w1, biases w1, scales w3, biases w3
    auto ld = [&](RawQ3 (&r1)[G], RawQ3 (&r3)[G], u32x4 (&win)[4], int kb) {
      if constexpr (kWin) {
        const uint8_t* W1 = static_cast<const uint8_t*>(d->p[0]);
        const uint8_t* W3 = static_cast<const uint8_t*>(d->p[3]);
        const int64_t code_row = static_cast<int64_t>(row) * (K / 8 * 3);
#pragma unroll
        for (int i = 0; i < G; ++i) {
          const bool ok = rok && kb + i < k1;
          const int64_t off = code_row + q3_chunk_offset(K, kb + i, g4);
          const auto c1 = gptr<uint32_t>(W1 + off);
          const auto c3 = gptr<uint32_t>(W3 + off);
#pragma unroll
          for (int q = 0; q < 3; ++q) {
            r1[i].w[q] = ok ? c1[q] : 0u;
            r3[i].w[q] = ok ? c3[q] : 0u;
          }
        }
        const bool ok = rok && kb < k1;
        const int64_t wo = (static_cast<int64_t>(row) * (K / 64) + 2 * kb) * 2;   // bytes
#pragma unroll
        for (int q = 0; q < 4; ++q)
          win[q] = ok ? ldg16(static_cast<const uint8_t*>(d->p[(q >> 1) * 3 + 1 + (q & 1)]) + wo)
                      : u32x4{0u, 0u, 0u, 0u};
      } else {
#pragma unroll
        for (int i = 0; i < G; ++i) {
          const int kc = (kb + i) * 128 + g4 * 32;
          const bool ok = rok && kb + i < k1 && kc < K;
          load_role(r1[i], d->p, 0, row, K, kc, ok);
          load_role(r3[i], d->p, 1, row, K, kc, ok);
        }
      }
    };
    // (scale, bias) of K block i of a windowed batch: group 2i + (g4 >> 1)
    auto win_sb = [&](RawQ3 (&r1)[G], RawQ3 (&r3)[G], const u32x4 (&win)[4]) {
      if constexpr (kWin) {
        const int sh = 16 * (g4 >> 1);
#pragma unroll
        for (int i = 0; i < G; ++i) {
          r1[i].s = (win[0][i] >> sh) & 0xffffu;
          r1[i].b = (win[1][i] >> sh) & 0xffffu;
          r3[i].s = (win[2][i] >> sh) & 0xffffu;
          r3[i].b = (win[3][i] >> sh) & 0xffffu;
        }
      }
    };
    ld(a1, a3, aw, k0);
    ld(b1, b3, bw, k0 + G);
    if (xreg) put_staged_x<kF32, kUpW * 64>(p, xh, xl, xs, tid, xv);
    wr = tv ? p.wrow[drow] : 0.0f;
    __syncthreads();
    const uint16_t* bh = xh + (tv ? r16 : 0) * xs;
    const uint16_t* bl = xl + (tv ? r16 : 0) * xs;
    auto mm = [&](RawQ3 (&r1)[G], RawQ3 (&r3)[G], const u32x4 (&win)[4], int kb) {
      win_sb(r1, r3, win);
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int kc = (kb + i) * 128 + g4 * 32;
        const bool ok = tv && kb + i < k1 && kc < K;
        mma_block2(r1[i], r3[i], bh, kc, ok, ag, au);
        if (f32) mma_block2(r1[i], r3[i], bl, kc, ok, ag, au);
      }
    };
    for (int kb = k0; kb < k1; kb += 2 * G) {
      mm(a1, a3, aw, kb);
      if (kb + 2 * G < k1) ld(a1, a3, aw, kb + 2 * G);
      if (kb + G < k1) mm(b1, b3, bw, kb + G);
      if (kb + 3 * G < k1) ld(b1, b3, bw, kb + 3 * G);
    }
  } else {
    // weights: up to two batches in flight
    const uint8_t* W1 = static_cast<const uint8_t*>(d->p[0]);
    const uint8_t* S1 = static_cast<const uint8_t*>(d->p[1]);
    const uint8_t* W3 = static_cast<const uint8_t*>(d->p[3]);
    const uint8_t* S3 = static_cast<const uint8_t*>(d->p[4]);
    // the second batch is issued after the barrier, when the first is about to be
    // used (both issued up front: 17.9 us at one token; this way 17.3 us)
    UpBatch<G> A, B;
    load_batch<G, kWin>(A, W1, S1, W3, S3, row, K, k0, k1, g4, rok);
    if (xreg) put_staged_x<kF32, kUpW * 64>(p, xh, xl, xs, tid, xv);
    wr = tv ? p.wrow[drow] : 0.0f;
    uint8_t* xch = reinterpret_cast<uint8_t*>(red + kUpItems) + wave * 640;
    __syncthreads();
    const uint16_t* bh = xh + (tv ? r16 : 0) * xs;
    const uint16_t* bl = xl + (tv ? r16 : 0) * xs;
    for (int kb = k0; kb < k1; kb += 2 * G) {
      if (kb == k0) load_batch<G, kWin>(B, W1, S1, W3, S3, row, K, k0 + G, k1, g4, rok);
      batch_scales<G, kWin>(A, xch, r16, g4);
      mma_batch<G>(A, bh, bl, K, kb, k1, g4, tv, f32, ag, au);
      if (kb + 2 * G < k1) load_batch<G, kWin>(A, W1, S1, W3, S3, row, K, kb + 2 * G, k1, g4, rok);
      if (kb + G < k1) {
        batch_scales<G, kWin>(B, xch, r16, g4);
        mma_batch<G>(B, bh, bl, K, kb + G, k1, g4, tv, f32, ag, au);
      }
      if (kb + 3 * G < k1) load_batch<G, kWin>(B, W1, S1, W3, S3, row, K, kb + 3 * G, k1, g4, rok);
    }
  }
  // K ranges added in order: ((r0 + r1) + r2) + r3
  *reinterpret_cast<f32x4*>(&red[item][ks][0][lane][0]) = ag;
  *reinterpret_cast<f32x4*>(&red[item][ks][1][lane][0]) = au;
  __syncthreads();
  if (ks == 0 && rok && tv) {
#pragma unroll
    for (int w = 1; w < kUpKS; ++w) {
      ag += *reinterpret_cast<const f32x4*>(&red[item][w][0][lane][0]);
      au += *reinterpret_cast<const f32x4*>(&red[item][w][1][lane][0]);
    }
    uint16_t hh[4], hl[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) split_bf16(silu_clamped(ag[q], au[q], p.limit) * wr, hh[q], hl[q]);
    const int64_t off = static_cast<int64_t>(drow) * p.I + rt * 16 + 4 * g4;
    *reinterpret_cast<uint2*>(p.h_hi + off) = uint2{hh[0] | (uint32_t(hh[1]) << 16), hh[2] | (uint32_t(hh[3]) << 16)};
    *reinterpret_cast<uint2*>(p.h_lo + off) = uint2{hl[0] | (uint32_t(hl[1]) << 16), hl[2] | (uint32_t(hl[3]) << 16)};
  }
}

// ---------------------------------------------------------------- MX gate/up (FP4, bf16 x, T <= 2)
// LDS of k_up_mx: K-range partial sums [kUpItems][kUpKS][2][64][4] f32, the
// waves' scale-exchange tiles [kUpW][640] bytes, the 32-row maxima
// [kUpItems][kMxMaxTokens] f32, then the activation planes xq [H/128][2T][128]
// and their E8M0 bytes xe [H/128][2T][4].
static_assert(kUpItems * 16 == 32, "a gate/up block's row tiles are one 32-row exponent group of h");
static_assert(kStW * kStKB * 128 == kMxInter, "the MX down kernel's waves cover the intermediate");
constexpr size_t kMxUpRedBytes = kUpItems * kUpKS * 2 * 64 * 4 * 4;
constexpr size_t kMxUpXchOffset = kMxUpRedBytes;
constexpr size_t kMxUpMaxOffset = kMxUpXchOffset + kUpW * 640;
constexpr size_t kMxUpXqOffset = kMxUpMaxOffset + kUpItems * kMxMaxTokens * 4;

// One activation chunk (8 bf16 values at K offset k8 of token t) into the
// B-operand planes of the MX gate/up: column 2t + p holds plane p, and each
// 32-value group's first plane has exponent ilogb(max) - 7.  The group's four
// chunks are in consecutive lanes, and every lane of the wave takes part in
// the max exchange (ok: this lane's chunk exists and is stored).
__device__ __forceinline__ void put_x_mx(uint8_t* xq, uint8_t* xe, int T, int t, int k8, const u32x4& v,
                                         bool ok) {
  const float f0[4] = {__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                       __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u)};
  const float f1[4] = {__uint_as_float(v.z << 16), __uint_as_float(v.z & 0xffff0000u),
                       __uint_as_float(v.w << 16), __uint_as_float(v.w & 0xffff0000u)};
  float m = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q) m = fmaxf(m, fmaxf(fabsf(f0[q]), fabsf(f1[q])));
  m = fmaxf(m, __shfl_xor(m, 1, 64));
  m = fmaxf(m, __shfl_xor(m, 2, 64));
  const int e = fp8_plane_exp(m);
  uint32_t w0[2], w1[2];
  fp8_planes4<2>(f0, e, w0);
  fp8_planes4<2>(f1, e, w1);
  if (ok) {
    const int kb = k8 >> 7, kk = k8 & 127;
#pragma unroll
    for (int pl = 0; pl < 2; ++pl) {
      const int col = kb * 2 * T + 2 * t + pl;
      *reinterpret_cast<uint2*>(xq + col * 128 + b_perm(kk)) = uint2{w0[pl], w1[pl]};
      if ((kk & 31) == 0) xe[col * 4 + (kk >> 5)] = static_cast<uint8_t>(e8m0_byte(e - 4 * pl));
    }
  }
}

// Routed gate/up of the decode pipeline for FP4 experts and one or two bf16
// tokens, on scaled FP4 x FP8 MFMAs (mx.h).  Blocks, waves, K ranges and the
// weight stream are those of k_up_stream (two batches of G K blocks, scale
// windows); the activations are staged in LDS as two FP8 planes per token
// (B column 2t + p), so one v_mfma_scale_f32_16x16x128_f8f6f4 per K block
// and role takes the FP4 codes and their E8M0 bytes as loaded.  The K ranges
// are added in wave order, then a token's two plane columns; h = SwiGLU(gate,
// up) * route weight (0 for a token not routed to the slot) leaves as three
// FP8 planes per (slot, token) with one exponent per 32-row group -- the two
// row tiles of a block -- in the B-operand layout of k_down_mx.
template <int G>
__global__ __launch_bounds__(kUpW * 64) __attribute__((amdgpu_waves_per_eu(4))) void k_up_mx(DecodeArgs p) {
  extern __shared__ __align__(16) uint16_t lds_up[];
  const int tid = threadIdx.x, lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  // the intermediate is kMxInter (the launcher's condition), so the block ->
  // slot map needs no argument
  constexpr int kTiles = kMxInter / 16;
  constexpr int groups = (kTiles + kUpItems - 1) / kUpItems;
  const int rb = static_cast<int>(blockIdx.x);
  const int slot = rb / groups;
  // the argument words the first loads address, read in one go
  asm volatile("" ::"s"(p.active), "s"(p.desc), "s"(p.rowmap), "s"(p.wrow), "s"(p.x));
  // the active count, the slot's weight pointers and (below) the dispatch row
  // and x go out together: the descriptor array has an entry for every slot
  // index (its pointers are used only for a live slot), so nothing waits for
  // the count before the block's first weight batch
  const int U = p.active[0];
  const uint8_t* W1 = static_cast<const uint8_t*>(desc_ptr(p.desc, slot, 0));
  const uint8_t* S1 = static_cast<const uint8_t*>(desc_ptr(p.desc, slot, 1));
  const uint8_t* W3 = static_cast<const uint8_t*>(desc_ptr(p.desc, slot, 3));
  const uint8_t* S3 = static_cast<const uint8_t*>(desc_ptr(p.desc, slot, 4));
  const int T = p.T, K = p.H;
  const int item = wave / kUpKS, ks = wave % kUpKS;
  const int rt = (rb % groups) * kUpItems + item;
  const bool rok = rt < kTiles;
  char* base = reinterpret_cast<char*>(lds_up);
  float (*red)[kUpKS][2][64][4] = reinterpret_cast<float (*)[kUpKS][2][64][4]>(base);
  uint8_t* xch = reinterpret_cast<uint8_t*>(base + kMxUpXchOffset) + wave * 640;
  float* gmax = reinterpret_cast<float*>(base + kMxUpMaxOffset);
  uint8_t* xq = reinterpret_cast<uint8_t*>(base + kMxUpXqOffset);
  const int nblk = K / 128;
  uint8_t* xe = xq + nblk * 2 * T * 128;
  // 1. this lane's dispatch row (output column 2t + p: token t) and the first two
  // activation chunks of this thread, ahead of the weights
  const int t = r16 >> 1;
  const int drow = t < T ? p.rowmap[slot * T + t] : -1;
  const int cpr = K / 8, xchunks = T * cpr;
  constexpr int NT = kUpW * 64;
  u32x4 xv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = min(tid + j * NT, xchunks - 1);   // no condition on the load (see load_raw_nc)
    xv[j] = ldg16(static_cast<const uint16_t*>(p.x) + static_cast<int64_t>(c / cpr) * K + (c % cpr) * 8);
  }
  // (the pointers are read before the count is tested)
  asm volatile("" ::"s"(W1), "s"(S1), "s"(W3), "s"(S3));
  if (slot >= U) return;
  // 2. the first weight batch
  const uint32_t row = static_cast<uint32_t>(rt * 16 + r16);
  const int per = (nblk + kUpKS - 1) / kUpKS;
  const int k0 = min(ks * per, nblk), k1 = min(k0 + per, nblk);
  UpBatch<G> A, B;
  load_batch<G, true>(A, W1, S1, W3, S3, row, K, k0, k1, g4, rok);
  const bool tv = drow >= 0 && rok;
  const float wr = tv ? p.wrow[drow] : 0.0f;
  // 3. the activations as FP8 planes (chunk rounds of the whole block, so that
  // the lanes of a 32-group are all present in each round)
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = tid + j * NT;
    put_x_mx(xq, xe, T, min(c, xchunks - 1) / cpr, (min(c, xchunks - 1) % cpr) * 8, xv[j], c < xchunks);
  }
  for (int c0 = 2 * NT; c0 < xchunks; c0 += NT) {
    const int c = min(c0 + tid, xchunks - 1);
    const u32x4 v = ldg16(static_cast<const uint16_t*>(p.x) + static_cast<int64_t>(c / cpr) * K + (c % cpr) * 8);
    put_x_mx(xq, xe, T, c / cpr, (c % cpr) * 8, v, c0 + tid < xchunks);
  }
  __syncthreads();
  // B column of this lane: plane r16 & 1 of token r16 >> 1 (columns past 2T
  // repeat the last one; their results are not used)
  const int bc = min(r16, 2 * T - 1);
  f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = ag;
  auto mm = [&](UpBatch<G>& b, int kb) {
    batch_scales<G, true>(b, xch, r16, g4);
#pragma unroll
    for (int i = 0; i < G; ++i) {
      if (kb + i < k1) {
        const int col = (kb + i) * 2 * T + bc;
        const u32x4* src = reinterpret_cast<const u32x4*>(xq + col * 128 + g4 * 32);
        const u32x4 blo = src[0], bhi = src[1];
        const uint32_t bs = xe[col * 4 + g4];
        ag = mx_mfma(b.c1[i], b.s1[i], blo, bhi, bs, ag);
        au = mx_mfma(b.c3[i], b.s3[i], blo, bhi, bs, au);
      }
    }
  };
  for (int kb = k0; kb < k1; kb += 2 * G) {
    if (kb == k0) load_batch<G, true>(B, W1, S1, W3, S3, row, K, k0 + G, k1, g4, rok);
    mm(A, kb);
    if (kb + 2 * G < k1) load_batch<G, true>(A, W1, S1, W3, S3, row, K, kb + 2 * G, k1, g4, rok);
    if (kb + G < k1) mm(B, kb + G);
    if (kb + 3 * G < k1) load_batch<G, true>(B, W1, S1, W3, S3, row, K, kb + 3 * G, k1, g4, rok);
  }
  // 4. K ranges added in order ((r0 + r1) + r2) + r3, then the two plane columns
  *reinterpret_cast<f32x4*>(&red[item][ks][0][lane][0]) = ag;
  *reinterpret_cast<f32x4*>(&red[item][ks][1][lane][0]) = au;
  __syncthreads();
  float hv[4] = {0.f, 0.f, 0.f, 0.f};
  if (ks == 0) {
#pragma unroll
    for (int w = 1; w < kUpKS; ++w) {
      ag += *reinterpret_cast<const f32x4*>(&red[item][w][0][lane][0]);
      au += *reinterpret_cast<const f32x4*>(&red[item][w][1][lane][0]);
    }
    float m = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float h = silu_clamped_fast(ag[q] + lane_xor1(ag[q]), au[q] + lane_xor1(au[q]), p.limit) * wr;
      hv[q] = tv ? h : 0.0f;
      m = fmaxf(m, fabsf(hv[q]));
    }
    // one exponent per (token, 32-row group): the largest |h| of the lane's
    // column over this tile, then over the block's two tiles
    m = max_over_rows(m);
    if (lane < 2 * T && (lane & 1) == 0) gmax[item * kMxMaxTokens + t] = m;
  }
  __syncthreads();
  if (ks == 0 && rok && (r16 & 1) == 0 && t < T) {
    float mg = gmax[t];
#pragma unroll
    for (int it = 1; it < kUpItems; ++it) mg = fmaxf(mg, gmax[it * kMxMaxTokens + t]);
    const int e = fp8_plane_exp(mg);
    uint32_t w[3];
    fp8_planes4<3>(hv, e, w);
    const int I = p.I, r = rt * 16 + 4 * g4;
    const int64_t col = static_cast<int64_t>(slot) * 3 * T + 3 * t;
    uint8_t* dst = p.hq + (r >> 7) * 128 + b_perm(r & 127);
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) *reinterpret_cast<uint32_t*>(dst + (col + pl) * I) = w[pl];
    if (item == 0 && g4 == 0) {
#pragma unroll
      for (int pl = 0; pl < 3; ++pl) p.hqs[(col + pl) * (I / 32) + rt / kUpItems] = static_cast<uint8_t>(e8m0_byte(e - 4 * pl));
    }
  }
}

// ---------------------------------------------------------------- q3 gate/up, factored
constexpr int kQ3fItems = 1;                      // row tiles of a block
constexpr int kQ3fKS = 8;                         // K ranges of a row tile (one wave each)
constexpr int kQ3fW = kQ3fItems * kQ3fKS;

// Routed gate/up of the decode pipeline for q3 experts (T <= 8), factored
// (see q3m_pair): the codes go into the MFMA as exact bf16 integers and each
// 64-group's scale and bias are applied once per K block to the MFMA output,
// about a fifth of the vector instructions of dequantising every weight.  The
// activations are the A operand (row 2t + h: token t restricted to the K
// block's h-th 64-group, zero elsewhere -- lane groups 0, 1 of a block hold
// group 0, lane groups 2, 3 group 1), the weights the B operand (column =
// weight row), so a 16x16x32 MFMA covers both groups of a block for up to 8
// tokens and a lane's outputs are one weight row of tokens 2g, 2g + 1.
// Block = kQ3fItems row tiles x kQ3fKS K ranges (one wave each; at hidden
// 4096 a wave's range is one 512-code superblock, so one batch per wave),
// kTwo: two batches in flight where a range is longer (a separate variant,
// so that the one-batch kernel keeps its registers); kR = 2 (one batch per
// range): each wave takes its K range of two row tiles, both batches issued
// at once, so that every block of the launch is resident in one round; K
// ranges added in order.
template <bool kWin, bool kF32, bool kTwo, int kR = 1>
__global__ __launch_bounds__(kQ3fW * 64) __attribute__((amdgpu_waves_per_eu(kF32 || !kWin || kTwo ? 3 : 4))) void k_up_q3(DecodeArgs p) {
  static_assert(kR == 1 || (kR == 2 && !kTwo), "two row tiles per wave take one batch each");
  constexpr int G = kUpBatch;
  extern __shared__ __align__(16) uint16_t lds_up[];
  const int tid = threadIdx.x, lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int groups = (p.up_tiles + kQ3fItems * kR - 1) / (kQ3fItems * kR);
  const int rb = static_cast<int>(blockIdx.x);
  const int slot = rb / groups;
  if (slot >= p.active[0]) return;
  const int T = p.T, K = p.H;
  const int item = wave / kQ3fKS, ks = wave % kQ3fKS;
  const int rt = ((rb % groups) * kQ3fItems + item) * kR;   // row tiles rt .. rt + kR - 1
  // this lane's A operand row: token ta, group half ha
  const int ta = r16 >> 1;
  const int drow_a = ta < T ? p.rowmap[slot * T + ta] : -1;
  const bool av = drow_a >= 0 && (r16 & 1) == (g4 >> 1);
  // this lane's output tokens
  const int t0 = 2 * g4;
  const int drow0 = t0 < T ? p.rowmap[slot * T + t0] : -1;
  const int drow1 = t0 + 1 < T ? p.rowmap[slot * T + t0 + 1] : -1;
  const int xs = K + 8, nblk = K / 128, cpr = K / 8, xchunks = T * cpr;
  constexpr int NT = kQ3fW * 64;
  uint16_t* xh = lds_up;
  uint16_t* xl = lds_up + T * xs;
  float* xsum = reinterpret_cast<float*>(lds_up + (kF32 ? 2 : 1) * T * xs);   // [nblk][8][2][2]
  float (*red)[kQ3fKS][2][64][2] = reinterpret_cast<float (*)[kQ3fKS][2][64][2]>(xsum + nblk * kQ3fMaxTokens * 4);
  const uint16_t* zero = reinterpret_cast<const uint16_t*>(red + kQ3fItems * kR);   // 64 zero bytes
  if (tid < 4) reinterpret_cast<u32x4*>(red + kQ3fItems * kR)[tid] = u32x4{0u, 0u, 0u, 0u};
  // activations: into registers when they fit (staged after the weight loads are issued)
  const bool xreg = xchunks <= NT;
  u32x4 xv0{}, xv1{};
  if (xreg) {
    const int c = min(tid, xchunks - 1);   // no condition on the load (see load_raw_nc)
    const int64_t e = static_cast<int64_t>(c) * 8;   // the rows are contiguous: chunk c at 8c
    if constexpr (!kF32) {
      xv0 = ldg16(static_cast<const uint16_t*>(p.x) + e);
    } else {
      xv0 = ldg16(static_cast<const float*>(p.x) + e);
      xv1 = ldg16(static_cast<const float*>(p.x) + e + 4);
    }
  } else {
    for (int c0 = 0; c0 < xchunks; c0 += NT) {   // xchunks is a multiple of 8: whole lane groups
      const int c = c0 + tid;
      if (c < xchunks) {
        const int64_t e = static_cast<int64_t>(c / cpr) * K + (c % cpr) * 8;
        u32x4 v0, v1{};
        if constexpr (!kF32) {
          v0 = ldg16(static_cast<const uint16_t*>(p.x) + e);
        } else {
          v0 = ldg16(static_cast<const float*>(p.x) + e);
          v1 = ldg16(static_cast<const float*>(p.x) + e + 4);
        }
        stage_chunk_q3<kF32>(xh, xl, xsum, xs, cpr, c, v0, v1);
      }
    }
  }
  const SlotDesc* d = p.desc + slot;
  const int per = (nblk + kQ3fKS - 1) / kQ3fKS;
  const int k0 = min(ks * per, nblk), k1 = min(k0 + per, nblk);
  const uint8_t* W1 = static_cast<const uint8_t*>(d->p[0]);
  const uint8_t* W3 = static_cast<const uint8_t*>(d->p[3]);
  const uint8_t* SB[4] = {static_cast<const uint8_t*>(d->p[1]), static_cast<const uint8_t*>(d->p[2]),
                          static_cast<const uint8_t*>(d->p[4]), static_cast<const uint8_t*>(d->p[5])};
  // loads without conditions (see load_raw_nc): rows past the tile read row
  // 0 (not stored), blocks past the wave's range re-read its last ones (not
  // computed: mm stops at k1); every wave has k1 > k0 here except the ones
  // past a short row, which clamp to the row's last block
  uint32_t code_rows[kR], sb_rows[kR];
#pragma unroll
  for (int i = 0; i < kR; ++i) {
    const uint32_t rowc = rt + i < p.up_tiles ? static_cast<uint32_t>((rt + i) * 16 + r16) : 0u;
    code_rows[i] = rowc * static_cast<uint32_t>(K / 8 * 3);
    sb_rows[i] = rowc * static_cast<uint32_t>(K / 64) * 2;   // bytes
  }
  auto ld = [&](Q3Batch<G>& b, int kb0, int ri) {
    const uint32_t code_row = code_rows[ri], sb_row = sb_rows[ri];
    if constexpr (kWin) {
      // a batch is one 512-code superblock: this lane group's chunks of its
      // 4 blocks are 48 contiguous bytes (windowed: k1 - k0 is a multiple of 4, >= 4)
      const int kbc = kb0 < k1 ? kb0 : k1 - G;
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
      // one 16-byte window per array: the 8 groups of the batch's 4 blocks
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const u32x4 w = ldg16(SB[a] + sb_row + kbc * 4);
#pragma unroll
        for (int i = 0; i < G; ++i) b.sb[a][i] = w[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int kb = min(kb0 + i, nblk - 1);
        const uint32_t off = code_row + q3_chunk_offset(K, kb, g4);
        const auto c1 = gptr<uint32_t>(W1 + off);
        const auto c3 = gptr<uint32_t>(W3 + off);
#pragma unroll
        for (int q = 0; q < 3; ++q) {
          b.c1[i][q] = c1[q];
          b.c3[i][q] = c3[q];
        }
#pragma unroll
        for (int a = 0; a < 4; ++a) b.sb[a][i] = ldg<uint32_t>(SB[a] + sb_row + kb * 4);
      }
    }
  };
  // batch A streams while the activations are staged, then batch B
  Q3Batch<G> A, B;
  ld(A, k0, 0);
  if (xreg && tid < xchunks) stage_chunk_q3<kF32>(xh, xl, xsum, xs, cpr, tid, xv0, xv1);   // whole lane groups
  if (kTwo) ld(B, k0 + G, 0);
  if (kR == 2) ld(B, k0, 1);
  const float wr0 = drow0 >= 0 ? p.wrow[drow0] : 0.0f;
  const float wr1 = drow1 >= 0 ? p.wrow[drow1] : 0.0f;
  __syncthreads();
  float acc1s[kR][2] = {}, acc3s[kR][2] = {};
  const Q3Masks km = q3_masks();
  auto mm = [&](const Q3Batch<G>& b, int kb0, int ri) {
    float (&acc1)[2] = acc1s[ri];
    float (&acc3)[2] = acc3s[ri];
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int kb = kb0 + i;
      if (kb >= k1) break;   // wave-uniform; blocks past the range must add nothing
      const int ao = ta * xs + kb * 128 + 32 * g4;
      const uint16_t* ah = av ? xh + ao : zero;
      f32x4 d1 = {0.0f, 0.0f, 0.0f, 0.0f}, d3 = d1;
#define DSK_Q3F_STEP(M)                                                             \
      {                                                                            \
        const bf16x8 xa = as_bf16x8(*reinterpret_cast<const u32x4*>(ah + 8 * M)); \
        d1 = mfma16(xa, q3m_operand<M>(b.c1[i], km), d1);                              \
        d3 = mfma16(xa, q3m_operand<M>(b.c3[i], km), d3);                              \
        if constexpr (kF32) {                                                      \
          const uint16_t* al = av ? xl + ao : zero;                                \
          const bf16x8 xb = as_bf16x8(*reinterpret_cast<const u32x4*>(al + 8 * M)); \
          d1 = mfma16(xb, q3m_operand<M>(b.c1[i], km), d1);                            \
          d3 = mfma16(xb, q3m_operand<M>(b.c3[i], km), d3);                            \
        }                                                                          \
      }
      DSK_Q3F_STEP(0) DSK_Q3F_STEP(1) DSK_Q3F_STEP(2) DSK_Q3F_STEP(3)
#undef DSK_Q3F_STEP
      const float* xg = xsum + (kb * kQ3fMaxTokens + t0) * 4;
      const f32x4 xa = *reinterpret_cast<const f32x4*>(xg);
      const f32x4 xb = *reinterpret_cast<const f32x4*>(xg + 4);
      q3_factor(d1, b.sb[0][i], b.sb[1][i], xa, xb, acc1);
      q3_factor(d3, b.sb[2][i], b.sb[3][i], xa, xb, acc3);
    }
  };
  if constexpr (kTwo) {
    for (int kb = k0; kb < k1; kb += 2 * G) {
      mm(A, kb, 0);
      if (kb + 2 * G < k1) ld(A, kb + 2 * G, 0);
      if (kb + G < k1) mm(B, kb + G, 0);
      if (kb + 3 * G < k1) ld(B, kb + 3 * G, 0);
    }
  } else {
    mm(A, k0, 0);   // the range is one batch
    if constexpr (kR == 2) mm(B, k0, 1);
  }
  // K ranges added in order: ((r0 + r1) + r2) + ...
#pragma unroll
  for (int i = 0; i < kR; ++i) {
    *reinterpret_cast<float2*>(&red[item * kR + i][ks][0][lane][0]) = float2{acc1s[i][0], acc1s[i][1]};
    *reinterpret_cast<float2*>(&red[item * kR + i][ks][1][lane][0]) = float2{acc3s[i][0], acc3s[i][1]};
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kR; ++i) {
  float (&acc1)[2] = acc1s[i];
  float (&acc3)[2] = acc3s[i];
  if (ks == 0 && rt + i < p.up_tiles && (drow0 >= 0 || drow1 >= 0)) {
#pragma unroll
    for (int w = 1; w < kQ3fKS; ++w) {
      const float2 g = *reinterpret_cast<const float2*>(&red[item * kR + i][w][0][lane][0]);
      const float2 u = *reinterpret_cast<const float2*>(&red[item * kR + i][w][1][lane][0]);
      acc1[0] += g.x; acc1[1] += g.y;
      acc3[0] += u.x; acc3[1] += u.y;
    }
    const int n = (rt + i) * 16 + r16;
    if (drow0 >= 0) {
      uint16_t hh, hl;
      split_bf16(silu_clamped(acc1[0], acc3[0], p.limit) * wr0, hh, hl);
      p.h_hi[static_cast<int64_t>(drow0) * p.I + n] = hh;
      p.h_lo[static_cast<int64_t>(drow0) * p.I + n] = hl;
    }
    if (drow1 >= 0) {
      uint16_t hh, hl;
      split_bf16(silu_clamped(acc1[1], acc3[1], p.limit) * wr1, hh, hl);
      p.h_hi[static_cast<int64_t>(drow1) * p.I + n] = hh;
      p.h_lo[static_cast<int64_t>(drow1) * p.I + n] = hl;
    }
  }
  }
}

// acc += W(16 rows, K block) x (hi + lo) of a 16-bit activation plane pair.
template <typename Raw>
__device__ __forceinline__ void mma_hilo(const Raw& a, const uint16_t* hi, const uint16_t* lo, int kc,
                                         bool ok, f32x4& acc) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16x8 av = a_operand(a, j);
    acc = mfma16(av, b_operand(hi, kc, j, ok), acc);
    acc = mfma16(av, b_operand(lo, kc, j, ok), acc);
  }
}

// Final add and cast of one 16-row output tile (wave 0 after the reduction).
__device__ __forceinline__ void down_epilogue(const DecodeArgs& p, f32x4 a, f32x4 sh, int row0,
                                              int r16, int g4) {
  const int64_t o = static_cast<int64_t>(r16) * p.H + row0 + 4 * g4;
  if (!p.x_f32) {
    // the shared output is rounded to x's dtype before it is added
    if (p.Is > 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) a[q] += bf16_bits_to_f32(f32_to_bf16_bits(sh[q]));
    } else if (p.shared_out) {
      const uint2 raw = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p.shared_out) + o);
      a += f32x4{__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                 __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u)};
    }
    uint16_t* ob = static_cast<uint16_t*>(p.out);
    *reinterpret_cast<uint2*>(ob + o) =
        uint2{f32_to_bf16_bits(a[0]) | (uint32_t(f32_to_bf16_bits(a[1])) << 16),
              f32_to_bf16_bits(a[2]) | (uint32_t(f32_to_bf16_bits(a[3])) << 16)};
  } else {
    if (p.Is > 0) a += sh;
    else if (p.shared_out) a += *reinterpret_cast<const f32x4*>(static_cast<const float*>(p.shared_out) + o);
    *reinterpret_cast<f32x4*>(static_cast<float*>(p.out) + o) = a;
  }
}

// Down + combine with every routed h row (N = T*k of them) and hs staged in
// LDS once per block.  Block = 16 output rows, kStW waves; wave w owns the K
// blocks [kStKB*w, kStKB*w + kStKB) of every expert's w2 rows and of the
// shared w2 rows.  The first NST activation chunks of every thread are loaded
// first (all of them up to two tokens), then the shared batch and kStRing
// routed batches of kStSlots experts are all issued, then the activations are
// written to LDS (each store waits only for its own load, which was issued
// ahead of the weights), and the batches are computed in order as they land.  The MFMA's B columns carry the hi and lo
// planes of each token (T <= 8), so one MFMA per K step covers both; four
// accumulator chains per wave for routed and for shared work, added in
// order, then the waves in order, then hi + lo.

template <typename Raw>
struct DownBatch {
  Raw r[kStSlots][kStKB];
};

// FP4: the codes of each slot's kStKB blocks and, instead of one scale byte
// per block and lane (a wave instruction touching 16 cache lines per block),
// one 8-byte window per slot holding the scales of both blocks for all four
// lane groups (byte 4j + g of block kb0 + j); the byte is picked at use.
template <>
struct DownBatch<RawFP4> {
  u32x4 c[kStSlots][kStKB];
  u32x2 sw[kStSlots];
};
static_assert(kStKB == 2, "the FP4 scale window holds two blocks");

template <typename Raw>
__device__ __forceinline__ void load_down_batch(DownBatch<Raw>& b, const DecodeArgs& p, int u0, int U,
                                                uint32_t row, int kb0, int g4) {
  const int I = p.I;
#pragma unroll
  for (int i = 0; i < kStSlots; ++i) {
    const int su = u0 + i < U ? u0 + i : 0;   // slots past U re-read slot 0 and are not computed
    if constexpr (std::is_same_v<Raw, RawFP4>) {
      // the staged kernel's K blocks cover I exactly (I = kStW * kStKB * 128)
      const uint8_t* W = static_cast<const uint8_t*>(desc_ptr(p.desc, su, 6));
      const uint8_t* S = static_cast<const uint8_t*>(desc_ptr(p.desc, su, 7));
#pragma unroll
      for (int j = 0; j < kStKB; ++j) b.c[i][j] = ldg16(W + row * static_cast<uint32_t>(I / 2) + (kb0 + j) * 64 + g4 * 16);
      b.sw[i] = ldg<u32x2>(S + row * static_cast<uint32_t>(I / 32) + kb0 * 4);
    } else {
#pragma unroll
      for (int j = 0; j < kStKB; ++j) load_w2_nc(b.r[i][j], p.desc, su, row, I, min((kb0 + j) * 128 + g4 * 32, I - 32));
    }
  }
}

// acc[j] += W(16 rows, K block) x B where B column c is plane (c & 1) (hi, lo)
// of token c >> 1: one MFMA per 32-wide K step, four independent chains.
template <typename Raw>
__device__ __forceinline__ void mma_cols(const Raw& a, const uint16_t* brow, int kc, bool ok, f32x4 (&acc)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = mfma16(a_operand(a, j), b_operand(brow, kc, j, ok), acc[j]);
}

template <typename Raw>
__device__ __forceinline__ void mma_down_batch(const DownBatch<Raw>& b, int u0, int U, const int* ldrow, int T,
                                               int t, const uint16_t* plane, int is, int kb0, int I,
                                               int g4, f32x4 (&acc)[4]) {
#pragma unroll
  for (int i = 0; i < kStSlots; ++i) {
    if (u0 + i >= U) break;
    const int dr = t < T ? ldrow[(u0 + i) * T + t] : -1;
    const bool tok = dr >= 0;
    const uint16_t* brow = plane + (tok ? dr : 0) * is;
#pragma unroll
    for (int j = 0; j < kStKB; ++j) {
      const int kc = (kb0 + j) * 128 + g4 * 32;
      if constexpr (std::is_same_v<Raw, RawFP4>) {
        const uint32_t w = j == 0 ? b.sw[i].x : b.sw[i].y;
        mma_cols(RawFP4{b.c[i][j], (w >> (8 * g4)) & 0xffu}, brow, kc, tok && kc < I, acc);
      } else {
        mma_cols(b.r[i][j], brow, kc, tok && kc < I, acc);
      }
    }
  }
}

template <typename Raw, int NST>
__global__ __launch_bounds__(kStW * 64) void k_down_decode_staged(DecodeArgs p) {
  extern __shared__ __align__(16) uint16_t lds_dn[];
  const int tid = threadIdx.x, lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int row0 = blockIdx.x * 16;
  const uint32_t row = static_cast<uint32_t>(row0 + r16);
  const int U = p.active[0];
  const int N = p.T * p.k;
  const int I = p.I, Is = p.Is;
  const int is = I + 8, iss = Is + 8;       // padded LDS row strides
  uint16_t* hh = lds_dn;
  uint16_t* hl = hh + N * is;
  uint16_t* sh_h = hl + N * is;
  uint16_t* sh_l = sh_h + p.T * iss;
  // the wave partial sums reuse the activation area once every wave is done with it
  float (*red)[kStW][64][4] = reinterpret_cast<float (*)[kStW][64][4]>(lds_dn);
  const int act_bytes = (N * is + p.T * iss) * 4;
  int* ldrow = reinterpret_cast<int*>(reinterpret_cast<char*>(lds_dn) +   // [U][T] dispatch rows (rowmap copy)
                                      (act_bytes > kStRedBytes ? act_bytes : kStRedBytes));
  const int kb0 = wave * kStKB;
  // 16 bytes past the dispatch rows take the stores of chunks past the end
  uint16_t* dump = reinterpret_cast<uint16_t*>(ldrow + kStMaxSlots * 8);
  // chunk c < hch: h row c / (I/8); c >= hch: hs row
  const int hch = N * (I / 8), sch = p.T * (Is / 8);
  // global element offset and LDS destinations of chunk c (no branches: selects)
  auto chunk_src = [&](int c, const uint16_t*& ph, const uint16_t*& pl) {
    c = min(c, hch + sch - 1);            // chunks past the end re-read the last one
    const bool shr = c >= hch;
    const int cs = shr ? c - hch : c, w = shr ? Is / 8 : I / 8, k = shr ? Is : I;
    ph = shr ? p.hs_hi : p.h_hi;
    pl = shr ? p.hs_lo : p.h_lo;
    return static_cast<int64_t>(cs / w) * k + (cs % w) * 8;
  };
  auto chunk_dst = [&](int c, uint16_t*& dh, uint16_t*& dl) {
    const bool shr = c >= hch, past = c >= hch + sch;
    const int cs = shr ? c - hch : c, w = shr ? Is / 8 : I / 8, stride = shr ? iss : is;
    const int off = (cs / w) * stride + (cs % w) * 8;
    dh = past ? dump : (shr ? sh_h : hh) + off;
    dl = past ? dump : (shr ? sh_l : hl) + off;
  };
  // 1. dispatch rows (one entry per thread: U * T <= kStMaxSlots * 8 <= kStW * 64) and the
  // first NST activation chunks of this thread, loaded ahead of the weights
  const int rm = p.rowmap[min(tid, U * p.T - 1)];
  u32x4 vh[NST], vl[NST];
#pragma unroll
  for (int j = 0; j < NST; ++j) {
    const uint16_t *ph, *pl;
    const int64_t e = chunk_src(tid + j * kStW * 64, ph, pl);
    vh[j] = ldg16(ph + e);
    vl[j] = ldg16(pl + e);
  }
  __builtin_amdgcn_sched_barrier(0);   // these loads go out before the weights
  // 2. every weight of the block in flight: the shared batch and kStRing routed batches,
  // all without conditions, so the compiler knows exactly how many loads follow the
  // activation loads and each activation store waits for its own load only (batches
  // past U re-read slot 0 and are not computed; without a shared expert its batch
  // re-reads the start of h)
  RawBF16 rs[kStKB];
  {
    const bool sh = Is > 0;
    const uint16_t* W = sh ? p.ws2 : p.h_hi;
#pragma unroll
    for (int j = 0; j < kStKB; ++j)
      load_raw_nc(rs[j], W, sh ? row : 0u, sh ? Is : 0, sh ? min((kb0 + j) * 128 + g4 * 32, Is - 32) : 0);
  }
  DownBatch<Raw> ring[kStRing];
#pragma unroll
  for (int q = 0; q < kStRing; ++q) load_down_batch(ring[q], p, q * kStSlots, U, row, kb0, g4);
  __builtin_amdgcn_sched_barrier(0);
  // 3. the activations into LDS: the first NST chunks from registers (each store
  // waits for its own load only), any further chunks (more than two tokens) after
#pragma unroll
  for (int j = 0; j < NST; ++j) {
    uint16_t *dh, *dl;
    chunk_dst(tid + j * kStW * 64, dh, dl);
    *reinterpret_cast<u32x4*>(dh) = vh[j];
    *reinterpret_cast<u32x4*>(dl) = vl[j];
  }
  if (tid < U * p.T) ldrow[tid] = rm;
  for (int c = tid + NST * kStW * 64; c < hch + sch; c += kStW * 64) {
    const uint16_t *ph, *pl;
    const int64_t e = chunk_src(c, ph, pl);
    uint16_t *dh, *dl;
    chunk_dst(c, dh, dl);
    *reinterpret_cast<u32x4*>(dh) = ldg16(ph + e);
    *reinterpret_cast<u32x4*>(dl) = ldg16(pl + e);
  }
  __syncthreads();
  // B column r16: plane r16 & 1 (hi, lo) of token r16 >> 1
  const int t = r16 >> 1;
  const bool tcol = t < p.T;
  const uint16_t* hplane = (r16 & 1) ? hl : hh;
  const uint16_t* splane = (r16 & 1) ? sh_l : sh_h;
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[4] = {z, z, z, z}, accs[4] = {z, z, z, z};
  if (Is > 0) {
    const uint16_t* brow = splane + (tcol ? t : 0) * iss;
#pragma unroll
    for (int j = 0; j < kStKB; ++j) {
      const int kc = (kb0 + j) * 128 + g4 * 32;
      mma_cols(rs[j], brow, kc, tcol && kc < Is, accs);
    }
  }
  // 3. routed batches in order; batch q + kStRing reuses batch q's registers
  for (int u0 = 0; u0 < U; u0 += kStRing * kStSlots) {
#pragma unroll
    for (int q = 0; q < kStRing; ++q) {
      const int ub = u0 + q * kStSlots;
      if (ub < U) {
        mma_down_batch(ring[q], ub, U, ldrow, p.T, t, hplane, is, kb0, I, g4, acc);
        if (ub + kStRing * kStSlots < U) load_down_batch(ring[q], p, ub + kStRing * kStSlots, U, row, kb0, g4);
      }
    }
  }
  __syncthreads();
  *reinterpret_cast<f32x4*>(&red[0][wave][lane][0]) = ((acc[0] + acc[1]) + acc[2]) + acc[3];
  *reinterpret_cast<f32x4*>(&red[1][wave][lane][0]) = ((accs[0] + accs[1]) + accs[2]) + accs[3];
  __syncthreads();
  if (wave == 0) {
    f32x4 a = z, sh = z;
    for (int w = 0; w < kStW; ++w) {
      a += *reinterpret_cast<const f32x4*>(&red[0][w][lane][0]);
      sh += *reinterpret_cast<const f32x4*>(&red[1][w][lane][0]);
    }
    // hi column + lo column of each token (lanes 2t and 2t + 1)
    f32x4 alo, slo;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      alo[q] = __shfl_xor(a[q], 1, 64);
      slo[q] = __shfl_xor(sh[q], 1, 64);
    }
    if ((r16 & 1) == 0 && tcol) down_epilogue(p, a + alo, sh + slo, row0, t, g4);
  }
}

// ---------------------------------------------------------------- MX down (FP4, T <= 2)
constexpr int kMxSlots = 8;   // routed experts per round of k_down_mx (all of them at one token)

// Wave-private LDS of k_down_mx, after the wave partial sums: the round's h
// planes of the wave's two K blocks [kMxSlots][3T][256 B] (B-operand order)
// and their E8M0 windows [kMxSlots][3T][8 B] (rounded up to 256 B).
constexpr int kMxDnRedBytes = kStW * 64 * 4 * 4;   // wave partial sums
constexpr int mx_dn_h_bytes(int T) { return kMxSlots * 3 * T * 256; }
constexpr int mx_dn_s_bytes(int T) { return (kMxSlots * 3 * T * 8 + 255) / 256 * 256; }
constexpr int mx_dn_wave_bytes(int T) { return mx_dn_h_bytes(T) + mx_dn_s_bytes(T); }
static_assert((kMxSlots * 3) % 4 == 0, "h DMA instructions cover whole (slot, column) pairs");

// Down + combine of the decode pipeline for FP4 experts and T (one or two)
// tokens on scaled FP4 x FP8 MFMAs.  Block = 16 output rows, kStW waves;
// wave w owns the K blocks [kStKB*w, kStKB*w + kStKB) of every active
// expert's w2 rows.  Everything of a round of kMxSlots experts is in flight
// at once: first the wave's slices of the FP8 h planes k_up_mx wrote (B
// column 3t + p: plane p of token t; zero planes for a token not routed to
// the slot) and of their E8M0 windows, 16 contiguous bytes per lane, then
// every expert's w2 codes and scale windows.  The h loads do not wait for
// the active count (it arrives with the slots' descriptors), so they are
// ahead of the weights of every block.  The slices go to wave-private LDS as
// they land (each store waits for its own load), and each expert is computed
// as its weights land, one v_mfma_scale_f32_16x16x128_f8f6f4 per K block with
// the B operand read back from LDS.  Slots past the active count re-read slot
// 0's weights and are computed with a zero B operand (straight-line code, so
// that every wait is for the loads it needs only).  One accumulator chain
// per K block of the wave, each over the slots in order -- a token's sum does
// not depend on the other token's experts (a slot the token is not routed to
// adds exact zeros), so two tokens give the rows of two single-token calls --
// the chains added in order, the waves in order, then a token's plane columns
// ((p0 + p1) + p2) and the final add of the precomputed shared output and
// cast.
template <int T>
__global__ __launch_bounds__(kStW * 64) void k_down_mx(DecodeArgs p) {
  extern __shared__ __align__(16) uint8_t lds_mx[];
  constexpr int C = 3 * T;
  float (*red)[64][4] = reinterpret_cast<float (*)[64][4]>(lds_mx);
  const int tid = threadIdx.x, lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int row0 = blockIdx.x * 16;
  const uint32_t row = static_cast<uint32_t>(row0 + r16);
  const int U = p.active[0];   // at least 1 (every token has top_k >= 1 experts)
  const int ms = min(p.E, T * p.k);   // slots of the h planes the gate/up grid covers
  const int I = p.I;
  const int kb0 = wave * kStKB;
  uint8_t* hl = lds_mx + kMxDnRedBytes + wave * mx_dn_wave_bytes(T);   // [kMxSlots][C][256]
  uint8_t* sl = hl + mx_dn_h_bytes(T);                                  // [kMxSlots][C][8]
  // B column of this lane (past the last one, repeats of it; their results are not used)
  const int bc = min(r16, C - 1);
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[kStKB] = {z, z};
  // the shared output of this lane's output elements (wave 0, token min(r16, T - 1))
  // before anything else, so that the epilogue does not wait for it
  uint2 shr = {0u, 0u};
  if (wave == 0 && p.shared_out)
    shr = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p.shared_out) +
                                          static_cast<int64_t>(min(r16, T - 1)) * p.H + row0 + 4 * g4);
  const uint8_t* W0 = static_cast<const uint8_t*>(desc_ptr(p.desc, 0, 6));
  const uint8_t* S0 = static_cast<const uint8_t*>(desc_ptr(p.desc, 0, 7));
  int u0 = 0;
  do {
    // (the round's start as an opaque value: nothing of a round is computed
    // ahead of the previous one)
    asm volatile("" : "+s"(u0));
    // the round's descriptors go out with the count (entries below E exist for
    // every index; a slot past the count takes slot 0's pointers), the h planes
    // with them (they do not wait for the count), and only the weights wait
    const uint8_t* Wr[kMxSlots];
    const uint8_t* Sr[kMxSlots];
#pragma unroll
    for (int i = 0; i < kMxSlots; ++i) {
      const int ui = min(u0 + i, p.E - 1);
      Wr[i] = static_cast<const uint8_t*>(desc_ptr(p.desc, ui, 6));
      Sr[i] = static_cast<const uint8_t*>(desc_ptr(p.desc, ui, 7));
    }
    // 1. the round's h planes and E8M0 windows (slot indices past the gate/up
    // grid re-read its last slot; a slot past the count is not used):
    // lane l takes 16 bytes of (slot, column) pair 4q + l / 16, 4 bytes of pair 32q + l / 2
    constexpr int NH = kMxSlots * C / 4, NS = mx_dn_s_bytes(T) / 256;
    u32x4 hv[NH];
    uint32_t sv[NS];
#pragma unroll
    for (int q = 0; q < NH; ++q) {
      const int pair = 4 * q + (lane >> 4), i = pair / C, c = pair - i * C;
      const int su = min(u0 + i, ms - 1);
      hv[q] = ldg16(p.hq + static_cast<uint32_t>(su * C + c) * static_cast<uint32_t>(I) + kb0 * 128 + (lane & 15) * 16);
    }
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      const int pair = min(32 * q + (lane >> 1), kMxSlots * C - 1), i = pair / C, c = pair - i * C;
      const int su = min(u0 + i, ms - 1);
      sv[q] = ldg<uint32_t>(p.hqs + static_cast<uint32_t>(su * C + c) * static_cast<uint32_t>(I / 32) + kb0 * 4 + 4 * (lane & 1));
    }
    __builtin_amdgcn_sched_barrier(0);
    // (the descriptors are all read before the first weight load)
    asm volatile("" ::"s"(Wr[0]), "s"(Wr[1]), "s"(Wr[2]), "s"(Wr[3]), "s"(Wr[4]), "s"(Wr[5]), "s"(Wr[6]),
                 "s"(Wr[7]), "s"(Sr[0]), "s"(Sr[1]), "s"(Sr[2]), "s"(Sr[3]), "s"(Sr[4]), "s"(Sr[5]), "s"(Sr[6]),
                 "s"(Sr[7]));
    static_assert(kMxSlots == 8, "one operand per slot above");
    // 2. every expert's w2 codes and scale windows
    u32x4 wc[kMxSlots][kStKB];
    u32x2 ws[kMxSlots];
#pragma unroll
    for (int i = 0; i < kMxSlots; ++i) {
      const bool live = u0 + i < U;
      const uint8_t* W = live ? Wr[i] : W0;
      const uint8_t* S = live ? Sr[i] : S0;
#pragma unroll
      for (int j = 0; j < kStKB; ++j) wc[i][j] = ldg16(W + row * static_cast<uint32_t>(I / 2) + (kb0 + j) * 64 + g4 * 16);
      ws[i] = ldg<u32x2>(S + row * static_cast<uint32_t>(I / 32) + kb0 * 4);
    }
    __builtin_amdgcn_sched_barrier(0);
    // 3. the slices into the wave's LDS (in the lane order they were loaded); a
    // slot past the count gets zero planes with scale bytes 1.0 (what it read
    // may be anything, its weights are slot 0's), so it adds exact zeros
#pragma unroll
    for (int q = 0; q < NH; ++q) {
      const bool live = u0 + (4 * q + (lane >> 4)) / C < U;
      *reinterpret_cast<u32x4*>(hl + q * 1024 + lane * 16) = live ? hv[q] : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      const bool live = u0 + min(32 * q + (lane >> 1), kMxSlots * C - 1) / C < U;
      *reinterpret_cast<uint32_t*>(sl + q * 256 + lane * 4) = live ? sv[q] : 0x7f7f7f7fu;
    }
    // 4. the experts in slot order as they land
#pragma unroll
    for (int i = 0; i < kMxSlots; ++i) {
#pragma unroll
      for (int j = 0; j < kStKB; ++j) {
        const uint8_t* src = hl + (i * C + bc) * 256 + j * 128 + g4 * 32;
        const u32x4 lo = *reinterpret_cast<const u32x4*>(src);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(src + 16);
        const uint32_t hs = sl[(i * C + bc) * 8 + 4 * j + g4];
        const uint32_t wsb = ((j == 0 ? ws[i].x : ws[i].y) >> (8 * g4)) & 0xffu;
        acc[j] = mx_mfma(wc[i][j], wsb, lo, hi, hs, acc[j]);
      }
    }
    u0 += kMxSlots;
  } while (u0 < U);
  static_assert(kStKB == 2, "two K-block chains");
  *reinterpret_cast<f32x4*>(&red[wave][lane][0]) = acc[0] + acc[1];
  __syncthreads();
  if (wave == 0) {
    f32x4 a = z;
    for (int w = 0; w < kStW; ++w) a += *reinterpret_cast<const f32x4*>(&red[w][lane][0]);
    // token t = r16 of this lane group: columns 3t .. 3t + 2
    const int t = min(r16, T - 1), gb = lane & 48;
    f32x4 ra;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      ra[q] = (__shfl(a[q], gb + 3 * t, 64) + __shfl(a[q], gb + 3 * t + 1, 64)) + __shfl(a[q], gb + 3 * t + 2, 64);
    if (r16 < T) {
      // bf16 x: the shared output is already in x's dtype
      if (p.shared_out)
        ra += f32x4{__uint_as_float(shr.x << 16), __uint_as_float(shr.x & 0xffff0000u),
                    __uint_as_float(shr.y << 16), __uint_as_float(shr.y & 0xffff0000u)};
      uint16_t* ob = static_cast<uint16_t*>(p.out) + static_cast<int64_t>(r16) * p.H + row0 + 4 * g4;
      *reinterpret_cast<uint2*>(ob) = uint2{f32_to_bf16_bits(ra[0]) | (uint32_t(f32_to_bf16_bits(ra[1])) << 16),
                                            f32_to_bf16_bits(ra[2]) | (uint32_t(f32_to_bf16_bits(ra[3])) << 16)};
    }
  }
}

// ---------------------------------------------------------------- q3 down, factored
constexpr int kDqRouted = 8;        // routed waves: half a 512-code superblock of I each (I = 2048)
constexpr int kDqShared = 4;        // shared waves: a K quarter of Is each
constexpr int kDqW = kDqRouted + kDqShared;   // waves: 0..7 routed, 8..11 shared
constexpr int kDqMaxTokens = 4;     // A operand row 4t + 2h + plane
constexpr int kDqRing = 8;          // routed experts in flight per wave
constexpr int kDqSharedKB = 4;      // shared K blocks per shared wave (Is <= 2048)

// One routed expert's w2 data of a routed wave: this lane's chunks of 2 blocks
// (half hf of a superblock, whose lane slice holds 12 bytes per block: 24
// bytes, as a 16-byte and an 8-byte load, both naturally aligned) and the
// (scale, bias) windows of their 4 groups (word j: groups 2j, 2j + 1 of block j).
struct DqSlot {
  uint32_t c[2][3];
  u32x2 s, b;
};

__device__ __forceinline__ void load_dq_slot(DqSlot& r, const DecodeArgs& p, int u, int U, uint32_t row,
                                             int sbk, int hf, int g4) {
  // no condition on the loads (see load_raw_nc): slots past U re-read slot 0
  // and are not computed; descriptors through the scalar cache (desc_ptr)
  const int su = u < U ? u : 0;
  const int I = p.I;
  const uint8_t* cb = static_cast<const uint8_t*>(desc_ptr(p.desc, su, 6)) +
                      row * static_cast<uint32_t>(I / 8 * 3) + sbk * 192 + 48 * g4 + 24 * hf;
  uint32_t w[6];
  if (hf == 0) {
    const u32x4 a = *gptr<u32x4>(cb);
    const u32x2 e = *gptr<u32x2>(cb + 16);
    w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3]; w[4] = e[0]; w[5] = e[1];
  } else {
    const u32x2 e = *gptr<u32x2>(cb);
    const u32x4 a = *gptr<u32x4>(cb + 8);
    w[0] = e[0]; w[1] = e[1]; w[2] = a[0]; w[3] = a[1]; w[4] = a[2]; w[5] = a[3];
  }
#pragma unroll
  for (int j = 0; j < 6; ++j) r.c[j / 3][j % 3] = w[j];
  const uint32_t wo = (row * static_cast<uint32_t>(I / 64) + 8 * sbk + 4 * hf) * 2;   // bytes
  r.s = ldg<u32x2>(static_cast<const uint8_t*>(desc_ptr(p.desc, su, 7)) + wo);
  r.b = ldg<u32x2>(static_cast<const uint8_t*>(desc_ptr(p.desc, su, 8)) + wo);
}

// Final add and cast of one output element (token t, column n).
__device__ __forceinline__ void down_epilogue1(const DecodeArgs& p, float a, float sh, int n, int t) {
  const int64_t o = static_cast<int64_t>(t) * p.H + n;
  if (!p.x_f32) {
    // the shared output is rounded to x's dtype before it is added
    if (p.Is > 0) a += bf16_bits_to_f32(f32_to_bf16_bits(sh));
    else if (p.shared_out) a += bf16_bits_to_f32(static_cast<const uint16_t*>(p.shared_out)[o]);
    static_cast<uint16_t*>(p.out)[o] = f32_to_bf16_bits(a);
  } else {
    if (p.Is > 0) a += sh;
    else if (p.shared_out) a += static_cast<const float*>(p.shared_out)[o];
    static_cast<float*>(p.out)[o] = a;
  }
}

// Down + combine of the decode pipeline for q3 experts (T <= 4, I = 2048),
// factored like k_up_q3: the h activations are the A operand (row 4t + 2h +
// plane: token t's hi or lo plane restricted to a K block's h-th 64-group),
// the raw w2 codes the B operand (column = output row), and each group's
// scale and bias are applied once per block: acc += s (D_hi + D_lo - 128 *
// sum(h / m)) + b * sum(h).  Block = 16 output rows, kDqW waves: routed wave
// w streams K blocks 2w, 2w + 1 (half w & 1 of superblock w >> 1, 24
// contiguous bytes per lane) of every active expert's w2 rows, kDqRing experts
// in flight (two routed waves per SIMD share the products that follow the
// loads); shared wave kDqRouted + s takes K quarter s of the shared expert's
// bf16 w2 rows.  Routed h rows are staged
// in LDS with the 8q positions divided by 8 and their group sums, the shared
// hs rows as they are.  A token's routed sum runs over its experts in slot
// (ascending id) order, then the routed waves and the shared waves are each
// added in order: no term depends on the other tokens of the batch.
__global__ __launch_bounds__(kDqW * 64) void k_down_q3(DecodeArgs p) {
  extern __shared__ __align__(16) uint16_t lds_dq[];
  const int tid = threadIdx.x, lane = __lane_id(), wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int row0 = blockIdx.x * 16;
  const uint32_t row = static_cast<uint32_t>(row0 + r16);
  const int U = p.active[0];
  const int T = p.T, N = T * p.k;
  const int I = p.I, Is = p.Is;
  const int is = I + 8, iss = Is + 8;       // padded LDS row strides
  const int ng = I / 64;                    // 64-groups per h row
  uint16_t* hh = lds_dq;
  uint16_t* hl = hh + N * is;
  uint16_t* sh_h = hl + N * is;
  uint16_t* sh_l = sh_h + T * iss;
  float* hsum = reinterpret_cast<float*>(sh_l + T * iss);            // [N][ng][2]: sum h, sum h / m
  float (*red)[kDqRouted][kDqMaxTokens][16] =
      reinterpret_cast<float (*)[kDqRouted][kDqMaxTokens][16]>(hsum + N * ng * 2);   // [routed, shared]
  const uint16_t* zero = reinterpret_cast<const uint16_t*>(red + 2);                // 64 zero bytes
  int* ldrow = reinterpret_cast<int*>(red + 2) + 16;                                // [U][T]
  if (tid < 4) reinterpret_cast<u32x4*>(red + 2)[tid] = u32x4{0u, 0u, 0u, 0u};
  // 1. activations (routed rows scaled and summed per group) and dispatch rows
  // into LDS; one dispatch-row entry per thread (U * T <= 16 * 4 * 4 <= kDqW * 64)
  const int rm = p.rowmap[min(tid, U * T - 1)];
  {
    constexpr int NT = kDqW * 64;
    constexpr int kStg = 3;                     // chunks per thread in flight (T = 1, k = 8: 3)
    const int cpr = I / 8, hch = N * cpr, sch = T * (Is / 8);
    for (int c1 = 0; c1 < hch + sch; c1 += kStg * NT) {
      u32x4 lh[kStg], ll[kStg];
#pragma unroll
      for (int j = 0; j < kStg; ++j) {
        // no condition on the loads (see load_raw_nc): chunks past the end re-read the last one
        const int c = min(c1 + j * NT + tid, hch + sch - 1);
        const uint16_t* ph = p.h_hi;
        const uint16_t* pl = p.h_lo;
        int64_t e = static_cast<int64_t>(c / cpr) * I + (c % cpr) * 8;
        if (c >= hch) {
          const int cs = c - hch;
          ph = p.hs_hi;
          pl = p.hs_lo;
          e = static_cast<int64_t>(cs / (Is / 8)) * Is + (cs % (Is / 8)) * 8;
        }
        lh[j] = ldg16(ph + e);
        ll[j] = ldg16(pl + e);
      }
#pragma unroll
    for (int j = 0; j < kStg; ++j) {   // hch, sch: multiples of 8 (whole lane groups)
      const int c = c1 + j * NT + tid;
      if (c < hch) {
        const int r = c / cpr, cc = c % cpr;
        const u32x4 vh = lh[j], vl = ll[j];
        const uint32_t div8 = q3m_div8_pairs(cc & 3);
        const uint32_t wh[4] = {vh.x, vh.y, vh.z, vh.w}, wl[4] = {vl.x, vl.y, vl.z, vl.w};
        uint16_t oh[8], ol[8];
        float sx = 0.0f, sxm = 0.0f;
#pragma unroll
        for (int e2 = 0; e2 < 8; ++e2) {
          const float fh = __uint_as_float((e2 & 1) ? (wh[e2 >> 1] & 0xffff0000u) : (wh[e2 >> 1] << 16));
          const float fl = __uint_as_float((e2 & 1) ? (wl[e2 >> 1] & 0xffff0000u) : (wl[e2 >> 1] << 16));
          const float sc = ((div8 >> (e2 >> 1)) & 1u) ? 0.125f : 1.0f;
          oh[e2] = f32_to_bf16_bits(fh * sc);
          ol[e2] = f32_to_bf16_bits(fl * sc);
          const float v = fh + fl;
          sx += v;
          sxm += v * sc;
        }
        *reinterpret_cast<u32x4*>(hh + r * is + cc * 8) = pack_bf16x8(oh);
        *reinterpret_cast<u32x4*>(hl + r * is + cc * 8) = pack_bf16x8(ol);
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) {
          sx += __shfl_xor(sx, o, 8);
          sxm += __shfl_xor(sxm, o, 8);
        }
        if ((cc & 7) == 0) *reinterpret_cast<float2*>(hsum + (r * ng + (cc >> 3)) * 2) = float2{sx, sxm};
      } else if (c < hch + sch) {
        const int cs = c - hch;
        const int off = (cs / (Is / 8)) * iss + (cs % (Is / 8)) * 8;
        *reinterpret_cast<u32x4*>(sh_h + off) = lh[j];
        *reinterpret_cast<u32x4*>(sh_l + off) = ll[j];
      }
    }
    }
  }
  wait_vm_all();   // only staging loads outstanding (see wait_vm_all)
  if (tid < U * T) ldrow[tid] = rm;
  const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
  if (wave < kDqRouted) {
    // 2. routed: K blocks 2 wave, 2 wave + 1 of every active expert's w2 rows
    const int sbk = wave >> 1, hf = wave & 1;
    DqSlot ring[kDqRing];
#pragma unroll
    for (int q = 0; q < kDqRing; ++q)
      if (q < U) load_dq_slot(ring[q], p, q, U, row, sbk, hf, g4);
    __syncthreads();
    // A operand row of this lane: token ta, group half ha, plane pa
    const int ta = r16 >> 2, ha = (r16 >> 1) & 1;
    const uint16_t* aplane = (r16 & 1) ? hl : hh;
    const bool arow = ta < T && ha == (g4 >> 1);
    const int to = g4;                         // this lane's output token
    const Q3Masks km = q3_masks();
    float acc = 0.0f;
    auto mm = [&](const DqSlot& r, int u) {
      const int dra = arow ? ldrow[u * T + ta] : -1;
      const int dro = to < T ? ldrow[u * T + to] : -1;
      const uint32_t sw[2] = {r.s.x, r.s.y}, bw[2] = {r.b.x, r.b.y};
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int kb = 2 * wave + j;
        const uint16_t* ah = dra >= 0 ? aplane + dra * is + kb * 128 + 32 * g4 : zero;
        f32x4 d = z;
        d = mfma16(as_bf16x8(*reinterpret_cast<const u32x4*>(ah)), q3m_operand<0>(r.c[j], km), d);
        d = mfma16(as_bf16x8(*reinterpret_cast<const u32x4*>(ah + 8)), q3m_operand<1>(r.c[j], km), d);
        d = mfma16(as_bf16x8(*reinterpret_cast<const u32x4*>(ah + 16)), q3m_operand<2>(r.c[j], km), d);
        d = mfma16(as_bf16x8(*reinterpret_cast<const u32x4*>(ah + 24)), q3m_operand<3>(r.c[j], km), d);
        if (dro >= 0) {
          const f32x4 xs = *reinterpret_cast<const f32x4*>(hsum + (dro * ng + 2 * kb) * 2);
          acc = fmaf(f16_half<0>(sw[j]), fmaf(-128.0f, xs.y, d[0] + d[1]), acc);
          acc = fmaf(f16_half<0>(bw[j]), xs.x, acc);
          acc = fmaf(f16_half<1>(sw[j]), fmaf(-128.0f, xs.w, d[2] + d[3]), acc);
          acc = fmaf(f16_half<1>(bw[j]), xs.z, acc);
        }
      }
    };
    for (int u0 = 0; u0 < U; u0 += kDqRing) {
#pragma unroll
      for (int q = 0; q < kDqRing; ++q) {
        const int u = u0 + q;
        if (u < U) {
          mm(ring[q], u);
          if (u + kDqRing < U) load_dq_slot(ring[q], p, u + kDqRing, U, row, sbk, hf, g4);
        }
      }
    }
    if (to < T) red[0][wave][to][r16] = acc;
  } else {
    // 2'. shared: K quarter `s` of the shared expert's bf16 w2 rows
    const int s = wave - kDqRouted;
    const int nbs = Is / 128, per = (nbs + 3) / 4;
    const int k0 = min(s * per, nbs), k1 = min(k0 + per, nbs);
    RawBF16 rs[kDqSharedKB];
    // the barrier first: issuing these loads before it held the barrier (and with
    // it the routed waves' products) until the loads had gone out behind the
    // routed ring's, while the shared products have time to spare
    __syncthreads();
    if (k0 < k1) {
      // no condition on the loads (see load_raw_nc): past k1, the last block again (not computed)
#pragma unroll
      for (int j = 0; j < kDqSharedKB; ++j) load_raw_nc(rs[j], p.ws2, row, Is, min(k0 + j, k1 - 1) * 128 + g4 * 32);
    }
    // A operand row 2t + plane
    const int ta = r16 >> 1;
    const uint16_t* sbase = ta < T ? ((r16 & 1) ? sh_l : sh_h) + ta * iss + 32 * g4 : zero;
    f32x4 d = z;
#pragma unroll
    for (int j = 0; j < kDqSharedKB; ++j) {
      if (k0 + j < k1) {
        const uint16_t* a = ta < T ? sbase + (k0 + j) * 128 : zero;
#pragma unroll
        for (int m = 0; m < 4; ++m)
          d = mfma16(as_bf16x8(*reinterpret_cast<const u32x4*>(a + 8 * m)), as_bf16x8(rs[j].v[m]), d);
      }
    }
    // rows 4 g4 + q: token 2 g4 + (q >> 1), plane q & 1
    const int t0 = 2 * g4;
    if (t0 < T) red[1][s][t0][r16] = d[0] + d[1];
    if (t0 + 1 < T) red[1][s][t0 + 1][r16] = d[2] + d[3];
  }
  __syncthreads();
  if (wave == 0 && g4 < T) {
    float a = 0.0f, sh = 0.0f;
#pragma unroll
    for (int w = 0; w < kDqRouted; ++w) a += red[0][w][g4][r16];
#pragma unroll
    for (int w = 0; w < kDqShared; ++w) sh += red[1][w][g4][r16];
    down_epilogue1(p, a, sh, row0 + r16, g4);
  }
}

template <typename Raw>
__global__ __launch_bounds__(kDownW * 64) void k_down_decode(DecodeArgs p) {
  __shared__ float red[2][kDownW][64][4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int row0 = blockIdx.x * 16;
  const int64_t row = row0 + r16;
  const int U = p.active[0];
  const bool tok = r16 < p.T;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f}, accs = acc;
  {
    const int K = p.I;
    const int nblk = (K + 127) / 128;
    const int per = (nblk + kDownW - 1) / kDownW;
    const int kb0 = min(wave * per, nblk), kb1 = min(kb0 + per, nblk);
    for (int kb = kb0; kb < kb1; ++kb) {
      const int kc = kb * 128 + g4 * 32;
      const bool kok = kc < K;
      for (int u0 = 0; u0 < U; u0 += kDownGroup) {
        Raw r[kDownGroup];
        int drow[kDownGroup];
#pragma unroll
        for (int i = 0; i < kDownGroup; ++i) {
          const bool in = u0 + i < U;
          const SlotDesc* d = p.desc + (in ? u0 + i : 0);
          load_role(r[i], d->p, 2, row, K, kc, in && kok);
          drow[i] = (in && tok) ? p.rowmap[(u0 + i) * p.T + r16] : -1;
        }
#pragma unroll
        for (int i = 0; i < kDownGroup; ++i) {
          if (u0 + i >= U) break;
          const bool ok = kok && drow[i] >= 0;
          const int64_t hb = static_cast<int64_t>(ok ? drow[i] : 0) * K;
          mma_hilo(r[i], p.h_hi + hb, p.h_lo + hb, kc, ok, acc);
        }
      }
    }
  }
  if (p.Is > 0) {
    const int K = p.Is;
    const int nblk = (K + 127) / 128;
    const int per = (nblk + kDownW - 1) / kDownW;
    const int kb0 = min(wave * per, nblk), kb1 = min(kb0 + per, nblk);
    for (int kb = kb0; kb < kb1; ++kb) {
      const int kc = kb * 128 + g4 * 32;
      RawBF16 r;
      load_raw(r, p.ws2, row, K, kc, kc < K);
      const int64_t hb = static_cast<int64_t>(tok ? r16 : 0) * K;
      mma_hilo(r, p.hs_hi + hb, p.hs_lo + hb, kc, tok && kc < K, accs);
    }
  }
  *reinterpret_cast<f32x4*>(&red[0][wave][lane][0]) = acc;
  *reinterpret_cast<f32x4*>(&red[1][wave][lane][0]) = accs;
  __syncthreads();
  if (wave == 0 && tok) {
    f32x4 a = {0.f, 0.f, 0.f, 0.f}, sh = a;
    for (int w = 0; w < kDownW; ++w) {
      a += *reinterpret_cast<const f32x4*>(&red[0][w][lane][0]);
      sh += *reinterpret_cast<const f32x4*>(&red[1][w][lane][0]);
    }
    down_epilogue(p, a, sh, row0, r16, g4);
  }
}

// The routing kernel of the decode pipeline's non-MX form (k_route_shared) also
// writes x's FP8 planes for the grouped FP4 gate/up that follows it (saves
// that kernel's own launch): from kDecodeGroupedUpMin tokens, with shared tile
// blocks to do it.
bool route_writes_x_planes(const dsk_moe_desc& d) {
  return d.tokens >= kDecodeGroupedUpMin && d.x_dtype == DSK_DTYPE_BF16 && d.inter_shared > 0 &&
         grouped_path(d) && grouped_up_mx(d);
}

DecodeArgs decode_args(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a) {
  DecodeArgs p{};
  p.T = d.tokens; p.H = d.hidden; p.I = d.inter; p.Is = d.inter_shared; p.k = d.top_k;
  p.limit = d.limit;
  p.desc = a.desc; p.active = a.active; p.rowmap = a.rowmap; p.wrow = a.wrow;
  p.x = a.x; p.x_f32 = d.x_dtype == DSK_DTYPE_F32;
  p.ws1 = static_cast<const uint16_t*>(a.ws1);
  p.ws3 = static_cast<const uint16_t*>(a.ws3);
  p.hs_hi = reinterpret_cast<uint16_t*>(a.ws + L.hs_hi);
  p.hs_lo = reinterpret_cast<uint16_t*>(a.ws + L.hs_lo);
  p.h_hi = reinterpret_cast<uint16_t*>(a.ws + L.h_hi);
  p.h_lo = reinterpret_cast<uint16_t*>(a.ws + L.h_lo);
  p.hq = reinterpret_cast<uint8_t*>(a.ws + L.hq);
  p.hqs = reinterpret_cast<uint8_t*>(a.ws + L.hqs);
  p.ws2 = static_cast<const uint16_t*>(a.ws2);
  p.shared_out = a.shared_out;
  p.out = a.out;
  p.up_tiles = d.inter / 16;
  p.scores = a.scores; p.bias = a.bias; p.table = a.table;
  p.E = d.n_experts; p.route_scale = d.route_scale;
  p.route = a.route;
  p.gate_w = a.gate_w; p.score_func = d.score_func;
  p.shared_x = a.ws + L.shared_x;
  if (a.rn) {
    p.rn = *a.rn;
    p.norm = 1;
  }
  return p;
}

size_t up_lds_bytes(const DecodeArgs& p) {
  return static_cast<size_t>(p.x_f32 ? 2 : 1) * p.T * (p.H + 8) * 2 + kUpLdsFixed;
}

// k_up_q3: activation plane(s), xsum [H/128][8][2][2] f32, K-range partial
// sums [kQ3fItems][kQ3fKS][2][64][2] f32, 64 zero bytes.
size_t up_q3_lds_bytes(const DecodeArgs& p) {
  return static_cast<size_t>(p.x_f32 ? 2 : 1) * p.T * (p.H + 8) * 2 +
         static_cast<size_t>(p.H / 128) * kQ3fMaxTokens * 16 + kQ3fItems * 2 * kQ3fKS * 2 * 64 * 2 * 4 + 64;
}

size_t up_mx_lds_bytes(const DecodeArgs& p) {
  return kMxUpXqOffset + static_cast<size_t>(p.H / 128) * 2 * p.T * (128 + 4);
}

size_t rs_lds_bytes(const DecodeArgs& p) {
  const size_t planes = static_cast<size_t>(p.x_f32 ? 2 : 1) * p.T * (p.H + 8) * 2;
  return planes > kRsRedBytes ? planes : kRsRedBytes;
}

}  // namespace

hipError_t launch_gate_shared(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a, hipStream_t s,
                              int repeat) {
  const DecodeArgs p = decode_args(d, L, a);
  const int gate_blocks = (p.T * p.E + 1) / 2;
  const unsigned blocks = static_cast<unsigned>(shared_up_tiles(p.T, p.Is) + gate_blocks);
  size_t lds = rs_lds_bytes(p);
  const size_t norm_lds = kGsNormOffset + static_cast<size_t>(p.T) * p.H * 2;
  if (p.norm && norm_lds > lds) lds = norm_lds;
  const bool wb = d.gate_dtype == DSK_DTYPE_BF16;
  if (p.norm && p.x_f32) return hipErrorInvalidValue;   // the residual stream is bf16 (resnorm_fusable)
  for (int r = 0; r < repeat; ++r) {
    if (p.norm && wb) launch_kernel(k_gate_shared<false, true, true>, blocks, kRsW * 64, lds, s, p);
    else if (p.norm) launch_kernel(k_gate_shared<false, false, true>, blocks, kRsW * 64, lds, s, p);
    else if (p.x_f32 && wb) launch_kernel(k_gate_shared<true, true>, blocks, kRsW * 64, lds, s, p);
    else if (p.x_f32) launch_kernel(k_gate_shared<true, false>, blocks, kRsW * 64, lds, s, p);
    else if (wb) launch_kernel(k_gate_shared<false, true>, blocks, kRsW * 64, lds, s, p);
    else launch_kernel(k_gate_shared<false, false>, blocks, kRsW * 64, lds, s, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_route_sdown(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a, hipStream_t s,
                              int repeat) {
  DecodeArgs p = decode_args(d, L, a);
  const unsigned blocks = static_cast<unsigned>(1 + (p.Is > 0 ? p.H / 16 : 0));
  // the pointer table does not fit beside the routing state (it is read per slot from
  // global memory; an LDS copy of all of it, prefetched with the scores, measured slower)
  const size_t lds = kRsRedBytes;
  p.route_lds = static_cast<int>(lds);
  for (int r = 0; r < repeat; ++r) {
    if (p.x_f32) launch_kernel(k_route_sdown<true>, blocks, kRsW * 64, lds, s, p);
    else launch_kernel(k_route_sdown<false>, blocks, kRsW * 64, lds, s, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_route_shared(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a, hipStream_t s,
                               int repeat) {
  DecodeArgs p = decode_args(d, L, a);
  const unsigned blocks = static_cast<unsigned>(1 + shared_up_tiles(p.T, p.Is));
  if (route_writes_x_planes(d)) p.xp = reinterpret_cast<uint8_t*>(a.ws + L.xp);
  // the pointer table goes to LDS only where the activation planes leave room: prefetching
  // all of it beside the shared tiles' stream was slower (q3 B=1 route stage 10.2 -> 11.1 us)
  // than the slot map's dependent table loads
  const size_t lds = rs_lds_bytes(p);
  p.route_lds = static_cast<int>(lds);
  for (int r = 0; r < repeat; ++r) {
    if (p.x_f32) launch_kernel(k_route_shared<true>, blocks, kRsW * 64, lds, s, p);
    else launch_kernel(k_route_shared<false>, blocks, kRsW * 64, lds, s, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_experts_decode(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a,
                                 hipStream_t s, int repeat) {
  const DecodeArgs p = decode_args(d, L, a);
  const int groups = (p.up_tiles + kUpItems - 1) / kUpItems;
  const int max_slots = d.n_experts < d.tokens * d.top_k ? d.n_experts : d.tokens * d.top_k;
  const unsigned up_blocks = static_cast<unsigned>(max_slots * groups);
  hipError_t e;
  const size_t up_lds = up_lds_bytes(p);
  // scale windows need 4-byte aligned scale rows (H a multiple of 128)
  const bool win = d.hidden % 128 == 0;
  const bool q3 = d.quant == DSK_QUANT_Q3;
  const bool mx = mx_decode(d);
  // q3 (scale, bias) windows: every wave's K range a whole number of G-block
  // batches inside the row (so also 16-byte aligned windows)
  const bool q3win = d.hidden % (kUpKS * kUpBatch * 128) == 0;
  const bool q3fwin = d.hidden % (kQ3fKS * kUpBatch * 128) == 0;
  const bool q3f2 = (d.hidden / 128 + kQ3fKS - 1) / kQ3fKS > kUpBatch;   // a wave's range is two or more batches
  const unsigned q3f_blocks = static_cast<unsigned>(max_slots * ((p.up_tiles + kQ3fItems - 1) / kQ3fItems));
  const unsigned q3f2_blocks = static_cast<unsigned>(max_slots * ((p.up_tiles + 2 * kQ3fItems - 1) / (2 * kQ3fItems)));
  if ((e = stage_open(kStageUp)) != hipSuccess) return e;
  if (d.tokens >= kDecodeGroupedUpMin && grouped_path(d)) {
    e = launch_grouped_up_routed(d, L, a, a.route.desc, a.route.xrow, a.route.wrow, s, repeat,
                                 route_writes_x_planes(d));
    if (e != hipSuccess) return e;
  } else {
    // q3 up to 8 tokens: the factored kernel
    const size_t q3f_lds = up_q3_lds_bytes(p);
    const bool q3f = q3 && d.tokens <= kQ3fMaxTokens && q3f_lds <= kMaxLds;
    for (int r = 0; r < repeat; ++r) {
      if (q3f && !q3f2) {
        // two row tiles per wave from 2 tokens (B=2: 38.9 -> 37.9 us; at one token, whose
        // 8 slots fit the chip in about two rounds of one-tile blocks, 17.3 -> 18.2 us)
        if (q3fwin && !p.x_f32 && d.tokens >= 2)
          launch_kernel(k_up_q3<true, false, false, 2>, q3f2_blocks, kQ3fW * 64, q3f_lds, s, p);
        else if (q3fwin && !p.x_f32) launch_kernel(k_up_q3<true, false, false>, q3f_blocks, kQ3fW * 64, q3f_lds, s, p);
        else if (q3fwin) launch_kernel(k_up_q3<true, true, false>, q3f_blocks, kQ3fW * 64, q3f_lds, s, p);
        else if (!p.x_f32) launch_kernel(k_up_q3<false, false, false>, q3f_blocks, kQ3fW * 64, q3f_lds, s, p);
        else launch_kernel(k_up_q3<false, true, false>, q3f_blocks, kQ3fW * 64, q3f_lds, s, p);
      } else if (q3f) {
        if (q3fwin && !p.x_f32) launch_kernel(k_up_q3<true, false, true>, q3f_blocks, kQ3fW * 64, q3f_lds, s, p);
        else if (q3fwin) launch_kernel(k_up_q3<true, true, true>, q3f_blocks, kQ3fW * 64, q3f_lds, s, p);
        else if (!p.x_f32) launch_kernel(k_up_q3<false, false, true>, q3f_blocks, kQ3fW * 64, q3f_lds, s, p);
        else launch_kernel(k_up_q3<false, true, true>, q3f_blocks, kQ3fW * 64, q3f_lds, s, p);
      }
      else if (mx) launch_kernel(k_up_mx<kUpBatch>, up_blocks, kUpW * 64, up_mx_lds_bytes(p), s, p);
      else if (q3 && q3win && !p.x_f32) launch_kernel(k_up_stream<kUpBatch, true, false, true>, up_blocks, kUpW * 64, up_lds, s, p);
      else if (q3 && q3win) launch_kernel(k_up_stream<kUpBatch, true, true, true>, up_blocks, kUpW * 64, up_lds, s, p);
      else if (q3 && !p.x_f32) launch_kernel(k_up_stream<kUpBatch, false, false, true>, up_blocks, kUpW * 64, up_lds, s, p);
      else if (q3) launch_kernel(k_up_stream<kUpBatch, false, true, true>, up_blocks, kUpW * 64, up_lds, s, p);
      else if (win && !p.x_f32) launch_kernel(k_up_stream<kUpBatch, true, false, false>, up_blocks, kUpW * 64, up_lds, s, p);
      else if (win) launch_kernel(k_up_stream<kUpBatch, true, true, false>, up_blocks, kUpW * 64, up_lds, s, p);
      else if (!p.x_f32) launch_kernel(k_up_stream<kUpBatch, false, false, false>, up_blocks, kUpW * 64, up_lds, s, p);
      else launch_kernel(k_up_stream<kUpBatch, false, true, false>, up_blocks, kUpW * 64, up_lds, s, p);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
  }
  if ((e = stage_open(kStageDown)) != hipSuccess) return e;
  if (d.tokens >= kDecodeGroupedDownMin && grouped_path(d)) {
    // routed and shared down per slot (one output row per dispatch row), then the combine
    // h in FP8 planes where the grouped gate/up wrote it (from kDecodeGroupedUpMin tokens)
    const bool hpl = d.tokens >= kDecodeGroupedUpMin && grouped_h_planes(d);
    if ((e = launch_grouped_down(d, L, a, a.route.desc, s, repeat, hpl)) != hipSuccess) return e;
    return launch_combine(d, L, a, s, repeat);
  }
  if (mx) {
    // the shared expert's down ran beside the routing (no shared intermediate here)
    if (d.inter_shared != 0) return hipErrorInvalidValue;
    for (int r = 0; r < repeat; ++r) {
      const size_t lds = kMxDnRedBytes + kStW * mx_dn_wave_bytes(d.tokens);
      if (d.tokens == 1) launch_kernel(k_down_mx<1>, static_cast<unsigned>(d.hidden / 16), kStW * 64, lds, s, p);
      else launch_kernel(k_down_mx<2>, static_cast<unsigned>(d.hidden / 16), kStW * 64, lds, s, p);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return hipSuccess;
  }
  const int n_rows = d.tokens * d.top_k;
  const int max_u = d.n_experts < n_rows ? d.n_experts : n_rows;
  if (q3 && d.tokens <= kDqMaxTokens && d.inter == kDqRouted * 256 && d.inter_shared <= 2048 &&
      d.inter_shared % 128 == 0) {
    // factored q3 down: h planes, hs planes, group sums, partial sums, zeros, dispatch rows
    const size_t dq_lds = static_cast<size_t>(n_rows) * (d.inter + 8) * 4 +
                          static_cast<size_t>(d.tokens) * (d.inter_shared + 8) * 4 +
                          static_cast<size_t>(n_rows) * (d.inter / 64) * 8 + 2 * kDqRouted * kDqMaxTokens * 16 * 4 +
                          64 + static_cast<size_t>(max_u) * d.tokens * 4;
    if (dq_lds <= kMaxLds) {
      for (int r = 0; r < repeat; ++r) {
        launch_kernel(k_down_q3, static_cast<unsigned>(d.hidden / 16), kDqW * 64, dq_lds, s, p);
        if ((e = hipGetLastError()) != hipSuccess) return e;
      }
      return hipSuccess;
    }
  }
  const size_t act = static_cast<size_t>(n_rows) * (d.inter + 8) * 4 +
                     static_cast<size_t>(d.tokens) * (d.inter_shared + 8) * 4;
  // activations (or the wave sums), dispatch rows [kStMaxSlots * 8], 16 bytes for chunks past the end
  const size_t dn_lds = (act > kStRedBytes ? act : kStRedBytes) + kStMaxSlots * 8 * 4 + 16;
  // staged: all activations fit in LDS, each wave's K blocks cover I (and
  // Is), few enough experts, and at most 8 tokens (two B columns each)
  const bool staged = dn_lds <= kMaxLds && max_u <= kStMaxSlots && d.tokens <= 8 &&
                      d.inter == kStW * kStKB * 128 && d.inter_shared <= kStW * kStKB * 128;
  for (int r = 0; r < repeat; ++r) {
    const unsigned blocks = static_cast<unsigned>(d.hidden / 16);
    // activation chunks per thread: all of them in the first round up to two tokens
    const int chunks = (n_rows * (d.inter / 8) + d.tokens * (d.inter_shared / 8) + kStW * 64 - 1) / (kStW * 64);
    if (staged && q3 && chunks <= 5) launch_kernel(k_down_decode_staged<RawQ3, 5>, blocks, kStW * 64, dn_lds, s, p);
    else if (staged && q3) launch_kernel(k_down_decode_staged<RawQ3, 9>, blocks, kStW * 64, dn_lds, s, p);
    else if (staged && chunks <= 5) launch_kernel(k_down_decode_staged<RawFP4, 5>, blocks, kStW * 64, dn_lds, s, p);
    else if (staged) launch_kernel(k_down_decode_staged<RawFP4, 9>, blocks, kStW * 64, dn_lds, s, p);
    else if (q3) launch_kernel(k_down_decode<RawQ3>, blocks, kDownW * 64, 0, s, p);
    else launch_kernel(k_down_decode<RawFP4>, blocks, kDownW * 64, 0, s, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  // down and combine are one kernel here (the combine stage launches nothing)
  return hipSuccess;
}

}  // namespace dsk
