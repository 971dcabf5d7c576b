// Expert products of large token batches: bf16 MFMA GEMM tiles over the
// dispatch rows.
//
// Replaces, when many tokens reach each expert, the per-expert gate/up qmm,
// the clamped SwiGLU with the route weight and the w2 qmm of the reference's
// moe_layer (src/deepseeker/mlx_forward.py:388-406), and the shared expert's
// three products (src/deepseeker/mlx_runner.py:765-783).  The combine that
// follows is the general path's.
//
// Work unit: a block tile of 256 weight rows x 256 dispatch rows, K walked in
// stages of 64.  Each stage every thread dequantises the 64 codes of one
// weight row (FP4 / q3; the shared expert's bf16 rows are copied) and gathers
// 8 x 16 bytes of the token rows into a double-buffered LDS tile whose rows
// are padded to 144 bytes, which keeps the 16-byte operand reads free of bank
// conflicts.  The four waves then run v_mfma_f32_32x32x16_bf16 over 128 x 128
// sub-tiles (16 accumulators of 32 x 32 each) while the next stage's global
// loads are in flight; 32-token sub-tiles past the end of an expert's rows
// are skipped.  Operand mapping of the 32x32x16 MFMA: lane l supplies row
// (l & 31) of A (weights) and column (l & 31) of B (tokens) at the 8 K
// positions 16*s + 8*(l >> 5) .. +8 of K step s; the result holds, in lane l
// and register r, weight row 8*(r >> 2) + 4*(l >> 5) + (r & 3) of token
// column (l & 31), so every lane owns runs of 4 consecutive output features.
//
// The gate/up tile interleaves w1 and w3 rows (64 of each per half tile), so
// the gate and up accumulators of one output sit in the same lane and
// register; its epilogue applies min(g, L), clip(u, -L, L), SiLU and the route
// weight and stores h rounded to bf16.  The down tile stores float32 rows.
//
// Numerics: products of bf16 operands are exact and accumulate in float32.
// x is bf16 (exact); h is rounded once to bf16 (relative 2^-9 per element),
// where the decode and general kernels carry it as a bf16 hi/lo pair.
//
// Tile list: one entry per 256 dispatch rows of every active expert, then the
// shared expert's token tiles.  Workgroup b runs on XCD b mod 8; blocks are
// mapped to (tile, weight-row tile) so that each XCD walks a contiguous range
// with the row tiles of one token tile adjacent, which keeps that tile's
// activations in the XCD's L2 while they are reused.
#include "tile.h"

namespace dsk {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPfThreads = 512;                // 8 waves, two per SIMD
constexpr int kPfK = 64;                       // K per stage
constexpr int kPfLd = kPfK + 8;                // bf16 LDS row stride (144 bytes)
constexpr int kPfBBytes = kPfToks * kPfLd * 2; // token tile of one stage
static_assert(kPfRows == 256 && kPfToks == 256, "two threads per weight row, four token chunks per thread");

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void sts16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ void sts16(void* p, const bf16x8& v) {
  *reinterpret_cast<u32x4*>(p) = __builtin_bit_cast(u32x4, v);
}
__device__ __forceinline__ bf16x8 lds16(const void* p) {
  return as_bf16x8(*reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// K mapping inside a stage: in K step ks (16 positions) lane half
// h = lane >> 5 supplies positions 32h + 8ks .. +8, so a lane's 4 steps
// cover the 32 contiguous positions [32h, 32h + 32).  Thread t stages half
// t & 1 (32 positions) of weight row t >> 1.

// The shared expert's bf16 weights: 64 bytes of a row per thread and stage.
struct StageBF16 {
  u32x4 v[4];
  __device__ __forceinline__ void load(const uint16_t* W, int64_t row, int K, int st, int hf) {
    const uint16_t* w = W + row * K + st * kPfK + 32 * hf;
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = ldg16(w + 8 * q);
  }
  __device__ __forceinline__ bf16x8 chunk(int q) const { return as_bf16x8(v[q]); }
};

// q3: a stage is half of a 128-code block and exactly one 64-group; half hf
// of it is lane group 2 (st & 1) + hf of the block (12 bytes).
struct StageQ3 {
  RawQ3 r;
  __device__ __forceinline__ void load(const uint8_t* W, const uint16_t* S, const uint16_t* B,
                                       int64_t row, int K, int st, int hf) {
    const auto src = gptr<uint32_t>(W + row * (K / 8 * 3) + q3_chunk_offset(K, st >> 1, 2 * (st & 1) + hf));
    r.w[0] = src[0]; r.w[1] = src[1]; r.w[2] = src[2];
    const int64_t gi = row * (K / 64) + st;
    r.s = ldg<uint16_t>(S + gi);
    r.b = ldg<uint16_t>(B + gi);
  }
  __device__ __forceinline__ bf16x8 chunk(int q) const {
    return q == 0 ? q3_operand<0>(r) : (q == 1 ? q3_operand<1>(r) : (q == 2 ? q3_operand<2>(r) : q3_operand<3>(r)));
  }
};

// Weight-tile policies.
// Bf16Tile: the stage's weights as bf16 in LDS ([256][72], padded rows);
// bf16 weights are copied, q3 codes dequantised as they are stored.
struct Bf16Tile {
  static constexpr int kBytes = kPfRows * kPfLd * 2;
  template <class Regs>
  __device__ __forceinline__ static void store_slice(const Regs& r, char* tile, int t, int ks) {
    sts16(reinterpret_cast<uint16_t*>(tile) + (t >> 1) * kPfLd + 32 * (t & 1) + 8 * ks, r.chunk(ks));
  }
  struct Frag { const uint16_t* p; };
  __device__ __forceinline__ static void frag_begin(Frag& f, const char* tile, int wm, int lane) {
    f.p = reinterpret_cast<const uint16_t*>(tile) + (128 * wm + (lane & 31)) * kPfLd + 32 * (lane >> 5);
  }
  __device__ __forceinline__ static bf16x8 operand(const Frag& f, int i, int ks) {
    return lds16(f.p + i * 32 * kPfLd + 8 * ks);
  }
};

// Fp4Tile: the stage's FP4 codes and E8M0 scales stay packed in LDS (rows of
// 48 bytes: 32 code bytes, 2 scale bytes, padding that keeps the 16-byte
// fragment reads conflict-free); every wave decodes its own fragments with
// v_cvt_scalef32_pk_bf16_fp4, which costs a quarter of the LDS traffic of a
// bf16 weight tile.
struct Fp4Tile {
  static constexpr int kRow = 48;
  static constexpr int kBytes = kPfRows * kRow;
  struct Regs {
    u32x4 c;      // 32 codes of this thread's half row
    uint32_t s;   // their E8M0 scale
    __device__ __forceinline__ void load(const uint8_t* W, const uint8_t* S, int64_t row, int K, int st, int hf) {
      c = ldg16(W + row * (K / 2) + st * (kPfK / 2) + 16 * hf);
      s = ldg<uint8_t>(S + row * (K / 32) + st * 2 + hf);
    }
  };
  __device__ __forceinline__ static void store_slice(const Regs& r, char* tile, int t, int ks) {
    char* row = tile + (t >> 1) * kRow;
    if (ks == 0) *reinterpret_cast<u32x4*>(row + 16 * (t & 1)) = r.c;
    else if (ks == 1) *reinterpret_cast<uint8_t*>(row + 32 + (t & 1)) = static_cast<uint8_t>(r.s);
  }
  struct Frag { u32x4 c[4]; float sc[4]; };
  __device__ __forceinline__ static void frag_begin(Frag& f, const char* tile, int wm, int lane) {
    const int h = lane >> 5;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const char* row = tile + (128 * wm + 32 * i + (lane & 31)) * kRow;
      f.c[i] = *reinterpret_cast<const u32x4*>(row + 16 * h);
      f.sc[i] = e8m0_to_f32(*reinterpret_cast<const uint8_t*>(row + 32 + h));
    }
  }
  __device__ __forceinline__ static bf16x8 operand(const Frag& f, int i, int ks) {
    const uint32_t w = ks == 0 ? f.c[i].x : (ks == 1 ? f.c[i].y : (ks == 2 ? f.c[i].z : f.c[i].w));
    return fp4_word_to_bf16x8(w, f.sc[i]);
  }
};

// Operands of one K step: 4 weight fragments, 2 token fragments.
struct KOps {
  bf16x8 a[4], b[2];
};

template <class P>
__device__ __forceinline__ void pf_operands(KOps& o, const typename P::Frag& fa, const uint16_t* B, int ks) {
#pragma unroll
  for (int c = 0; c < 2; ++c) o.b[c] = lds16(B + c * 32 * kPfLd + 8 * ks);
#pragma unroll
  for (int i = 0; i < 4; ++i) o.a[i] = P::operand(fa, i, ks);
}

// 8 MFMAs of one K step: acc[i][c] += A(row tile i) x B(token tile c);
// unless kFull, token tiles c >= n_ct are skipped (n_ct is wave-uniform).
template <bool kFull>
__device__ __forceinline__ void pf_mma(const KOps& o, int n_ct, f32x16 (&acc)[4][2]) {
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    if (kFull || c < n_ct) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i][c] = mfma32(o.a[i], o.b[c], acc[i][c]);
    }
  }
}

// Operands of one stage, held in registers between the global loads and the
// LDS store.
template <class Regs>
struct StageRegs {
  Regs a;
  u32x4 b[4];
};

// Main loop of one block tile.  load_a(regs, st) fills this thread's half
// weight row of stage st; brow[j] is the token row of LDS row (t >> 3) + 64 j.
// An LDS stage buffer holds the weight tile (P) then the token tile
// ([256][72] bf16); two buffers alternate.  Per stage st (buffer st & 1):
//   read the weight fragments of st; MFMAs of the previous stage's last K
//   step (its operands were kept in registers, so they run while the LDS
//   reads are in flight); K steps 0-2 of st; operands of K step 3, kept;
//   store stage st + 1 (loaded during stage st - 1) into the other buffer;
//   issue the global loads of stage st + 2; barrier.
// The matrix pipe thus has work across the barrier, and a global load has a
// whole stage to arrive.  Wave w multiplies weight rows 128 (w & 1) +
// [0, 128) by tokens 64 (w >> 1) + [0, 64).
template <bool kFull, class P, class Regs, class LoadA>
__device__ __forceinline__ void pf_loop(LoadA load_a, const uint16_t* const (&brow)[4], int nst, int n_ct,
                                        char* lds, f32x16 (&acc)[4][2]) {
  const int t = threadIdx.x, lane = t & 63, wave = wave_id();
  const int wm = wave & 1, wn = wave >> 1;
  const int ch = 8 * (t & 7);
  constexpr int kBufBytes = P::kBytes + kPfBBytes;
  const int b_st = (t >> 3) * kPfLd + ch;
  const int b_rd = (64 * wn + (lane & 31)) * kPfLd + 32 * (lane >> 5);
  auto btile = [&](int buf) { return reinterpret_cast<uint16_t*>(lds + buf * kBufBytes + P::kBytes); };
  StageRegs<Regs> r;
  auto load = [&](int st) {
    load_a(r.a, st);
#pragma unroll
    for (int j = 0; j < 4; ++j) r.b[j] = ldg16(brow[j] + st * kPfK + ch);
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < kPfK / 16; ++ks) {
      P::store_slice(r.a, lds + buf * kBufBytes, t, ks);
      sts16(btile(buf) + b_st + 64 * ks * kPfLd, r.b[ks]);
    }
  };
  load(0);
  store(0);
  if (nst > 1) load(1);
  __syncthreads();
  KOps o, last;
  for (int st = 0; st < nst; ++st) {
    const int cur = st & 1;
    typename P::Frag fa;
    P::frag_begin(fa, lds + cur * kBufBytes, wm, lane);
    const uint16_t* B = btile(cur) + b_rd;
    if (st > 0) pf_mma<kFull>(last, n_ct, acc);
    pf_operands<P>(o, fa, B, 0);
    pf_mma<kFull>(o, n_ct, acc);
    pf_operands<P>(o, fa, B, 1);
    pf_mma<kFull>(o, n_ct, acc);
    pf_operands<P>(o, fa, B, 2);
    pf_mma<kFull>(o, n_ct, acc);
    pf_operands<P>(last, fa, B, 3);
    if (st + 1 < nst) store(cur ^ 1);
    if (st + 2 < nst) load(st + 2);
    __syncthreads();
  }
  pf_mma<kFull>(last, n_ct, acc);
}

template <class P, class Regs, class LoadA>
__device__ __forceinline__ void pf_gemm(LoadA load_a, const uint16_t* const (&brow)[4], int nst, int n_ct,
                                        char* lds, f32x16 (&acc)[4][2]) {
  if (n_ct == 2) pf_loop<true, P, Regs>(load_a, brow, nst, n_ct, lds, acc);
  else pf_loop<false, P, Regs>(load_a, brow, nst, n_ct, lds, acc);
}

constexpr size_t kPfLdsBytes = 2 * static_cast<size_t>(Bf16Tile::kBytes + kPfBBytes);
static_assert(kPfLdsBytes <= kMaxLds, "LDS stage buffers do not fit");

struct PfArgs {
  int T, H, I, Is;
  float limit;
  const SlotDesc* desc;
  const int32_t* tiles;   // [0] tiles, [1] routed tiles, [2 ..] slot (-1 shared), [2 + max_tiles ..] first row
  int max_tiles;
  const int32_t* xrow; const float* wrow;   // per dispatch row: token, route weight
  const uint16_t* x;                        // [T][H] bf16
  const uint16_t* ws1; const uint16_t* ws3; const uint16_t* ws2;
  uint16_t* h; uint16_t* hs;                // [T*k][I], [T][Is] bf16
  float* y; float* ys;                      // [T*k][H], [T][H] float32
  int row_tiles;                            // weight-row tiles per token tile
};

// Logical work unit of this block: contiguous per XCD (b mod 8), row tiles
// of one token tile adjacent.
__device__ __forceinline__ bool pf_unit(const PfArgs& p, int& tile, int& rt) {
  const int R = p.tiles[0] * p.row_tiles;
  const int b = blockIdx.x;
  if (b >= R) return false;
  const int xcd = b & 7;
  int start = 0;
  for (int y = 0; y < xcd; ++y) start += (R - y + 7) >> 3;
  const int L = start + (b >> 3);
  tile = L / p.row_tiles;
  rt = L - tile * p.row_tiles;
  return true;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return static_cast<uint32_t>(f32_to_bf16_bits(a)) | (static_cast<uint32_t>(f32_to_bf16_bits(b)) << 16);
}

__device__ __forceinline__ void zero(f32x16 (&acc)[4][2]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int c = 0; c < 2; ++c) acc[i][c] = f32x16{};
}

// Gate/up: local weight row r = 0..255 of the tile is w1 (r & 64 == 0) or
// w3 row rt*128 + (r >> 7)*64 + (r & 63), so wave rows 0..63 are gate rows
// and 64..127 the matching up rows; h[row][i] = silu(min(g,L)) * clip(u) * w.
template <bool kQ3>
__global__ __launch_bounds__(kPfThreads, 1) void k_pf_up(PfArgs p) {
  extern __shared__ __align__(16) char pf_lds[];
  int tile, rt;
  if (!pf_unit(p, tile, rt)) return;
  const int slot = p.tiles[2 + tile], first = p.tiles[2 + p.max_tiles + tile];
  const bool shared = slot < 0;
  if (rt * 128 >= (shared ? p.Is : p.I)) return;
  const SlotDesc* d = shared ? nullptr : p.desc + slot;
  const int n_tok = shared ? p.T : d->n_tok;
  const int tok_base = shared ? 0 : d->tok_base;
  const int cnt = min(kPfToks, n_tok - first);
  const int t = threadIdx.x, lane = t & 63, wave = wave_id();
  const int wm = wave & 1, wn = wave >> 1;
  const uint16_t* brow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tn = min((t >> 3) + 64 * j, cnt - 1);
    const int64_t xr = shared ? first + tn : p.xrow[tok_base + first + tn];
    brow[j] = p.x + xr * p.H;
  }
  const int r = t >> 1, hf = t & 1;
  const int role = (r >> 6) & 1;
  const int64_t arow = rt * 128 + (r >> 7) * 64 + (r & 63);
  const int n_ct = max(0, min(2, (cnt - 64 * wn + 31) >> 5));
  const int K = p.H, nst = K / kPfK;
  f32x16 acc[4][2];
  zero(acc);
  if (shared) {
    const uint16_t* W = role ? p.ws3 : p.ws1;
    pf_gemm<Bf16Tile, StageBF16>([&](StageBF16& a, int st) { a.load(W, arow, K, st, hf); }, brow, nst, n_ct,
                                 pf_lds, acc);
  } else if constexpr (kQ3) {
    const uint8_t* W = static_cast<const uint8_t*>(d->p[3 * role]);
    const uint16_t* S = static_cast<const uint16_t*>(d->p[3 * role + 1]);
    const uint16_t* B = static_cast<const uint16_t*>(d->p[3 * role + 2]);
    pf_gemm<Bf16Tile, StageQ3>([&](StageQ3& a, int st) { a.load(W, S, B, arow, K, st, hf); }, brow, nst, n_ct,
                               pf_lds, acc);
  } else {
    const uint8_t* W = static_cast<const uint8_t*>(d->p[3 * role]);
    const uint8_t* S = static_cast<const uint8_t*>(d->p[3 * role + 1]);
    pf_gemm<Fp4Tile, Fp4Tile::Regs>([&](Fp4Tile::Regs& a, int st) { a.load(W, S, arow, K, st, hf); }, brow,
                                    nst, n_ct, pf_lds, acc);
  }
  const int ld = shared ? p.Is : p.I;
  uint16_t* out = shared ? p.hs : p.h;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int n = 64 * wn + 32 * c + (lane & 31);
    if (n >= cnt) continue;
    const int64_t drow = shared ? first + n : tok_base + first + n;
    const float wr = shared ? 1.0f : p.wrow[drow];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      uint16_t* dst = out + drow * ld + rt * 128 + wm * 64 + 32 * i + 4 * (lane >> 5);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float hv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          hv[e] = silu_clamped(acc[i][c][4 * q + e], acc[i + 2][c][4 * q + e], p.limit) * wr;
        *reinterpret_cast<uint2*>(dst + 8 * q) = uint2{pack_bf16x2(hv[0], hv[1]), pack_bf16x2(hv[2], hv[3])};
      }
    }
  }
}

// Down: weight rows rt*256 + [0, 256) of w2; y[row][n] in float32.
template <bool kQ3>
__global__ __launch_bounds__(kPfThreads, 1) void k_pf_down(PfArgs p) {
  extern __shared__ __align__(16) char pf_lds[];
  int tile, rt;
  if (!pf_unit(p, tile, rt)) return;
  const int slot = p.tiles[2 + tile], first = p.tiles[2 + p.max_tiles + tile];
  const bool shared = slot < 0;
  const SlotDesc* d = shared ? nullptr : p.desc + slot;
  const int n_tok = shared ? p.T : d->n_tok;
  const int tok_base = shared ? 0 : d->tok_base;
  const int cnt = min(kPfToks, n_tok - first);
  const int K = shared ? p.Is : p.I, nst = K / kPfK;
  const uint16_t* src = shared ? p.hs : p.h;
  const int t = threadIdx.x, lane = t & 63, wave = wave_id();
  const int wm = wave & 1, wn = wave >> 1;
  const uint16_t* brow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tn = min((t >> 3) + 64 * j, cnt - 1);
    brow[j] = src + static_cast<int64_t>(tok_base + first + tn) * K;
  }
  const int hf = t & 1;
  const int64_t arow = rt * 256 + (t >> 1);
  const int n_ct = max(0, min(2, (cnt - 64 * wn + 31) >> 5));
  f32x16 acc[4][2];
  zero(acc);
  if (shared) {
    pf_gemm<Bf16Tile, StageBF16>([&](StageBF16& a, int st) { a.load(p.ws2, arow, K, st, hf); }, brow, nst, n_ct,
                                 pf_lds, acc);
  } else if constexpr (kQ3) {
    const uint8_t* W = static_cast<const uint8_t*>(d->p[6]);
    const uint16_t* S = static_cast<const uint16_t*>(d->p[7]);
    const uint16_t* B = static_cast<const uint16_t*>(d->p[8]);
    pf_gemm<Bf16Tile, StageQ3>([&](StageQ3& a, int st) { a.load(W, S, B, arow, K, st, hf); }, brow, nst, n_ct,
                               pf_lds, acc);
  } else {
    const uint8_t* W = static_cast<const uint8_t*>(d->p[6]);
    const uint8_t* S = static_cast<const uint8_t*>(d->p[7]);
    pf_gemm<Fp4Tile, Fp4Tile::Regs>([&](Fp4Tile::Regs& a, int st) { a.load(W, S, arow, K, st, hf); }, brow,
                                    nst, n_ct, pf_lds, acc);
  }
  float* out = shared ? p.ys : p.y;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int n = 64 * wn + 32 * c + (lane & 31);
    if (n >= cnt) continue;
    const int64_t drow = tok_base + first + n;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float* dst = out + drow * p.H + rt * 256 + wm * 128 + 32 * i + 4 * (lane >> 5);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<f32x4*>(dst + 8 * q) =
            f32x4{acc[i][c][4 * q], acc[i][c][4 * q + 1], acc[i][c][4 * q + 2], acc[i][c][4 * q + 3]};
    }
  }
}

// Tile list from the dispatch descriptors (one block of 1024 threads; one
// thread per active expert slot, E <= 1024).
__global__ __launch_bounds__(1024) void k_pf_tiles(const SlotDesc* __restrict__ desc,
                                                   const int32_t* __restrict__ active, int E, int T,
                                                   int with_shared, int max_tiles, int32_t* __restrict__ tiles) {
  __shared__ int32_t wsum[16];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int n_act = min(active[0], E);
  const int cnt = t < n_act ? (desc[t].n_tok + kPfToks - 1) / kPfToks : 0;
  int incl = cnt;
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) {
    const int v = __shfl_up(incl, s, 64);
    if (lane >= s) incl += v;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int base = 0, total = 0;
  for (int w = 0; w < 16; ++w) {
    base += w < wave ? wsum[w] : 0;
    total += wsum[w];
  }
  const int off = base + incl - cnt;
  for (int j = 0; j < cnt; ++j) {
    tiles[2 + off + j] = t;
    tiles[2 + max_tiles + off + j] = j * kPfToks;
  }
  const int sh = with_shared ? (T + kPfToks - 1) / kPfToks : 0;
  for (int j = t; j < sh; j += 1024) {
    tiles[2 + total + j] = -1;
    tiles[2 + max_tiles + total + j] = j * kPfToks;
  }
  if (t == 0) {
    tiles[0] = total + sh;
    tiles[1] = total;
  }
}

}  // namespace

int prefill_max_tiles(const dsk_moe_desc& d) {
  const int n = d.tokens * d.top_k;
  const int slots = d.n_experts < n ? d.n_experts : n;
  const int shared = d.inter_shared > 0 ? (d.tokens + kPfToks - 1) / kPfToks : 0;
  return (n + kPfToks - 1) / kPfToks + slots + shared;
}

hipError_t launch_experts_prefill(const dsk_moe_desc& d, const Workspace& L, const PrefillArgs& a,
                                  hipStream_t s, int repeat) {
  const int T = d.tokens, H = d.hidden, I = d.inter, Is = d.inter_shared;
  const bool q3 = d.quant == DSK_QUANT_Q3;
  const int max_tiles = prefill_max_tiles(d);
  int32_t* tiles = reinterpret_cast<int32_t*>(a.ws + L.pf_tiles);
  launch_kernel(k_pf_tiles, 1, 1024, 0, s, a.desc, a.active, d.n_experts, T, Is > 0 ? 1 : 0, max_tiles, tiles);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;

  PfArgs p{};
  p.T = T; p.H = H; p.I = I; p.Is = Is; p.limit = d.limit;
  p.desc = a.desc; p.tiles = tiles; p.max_tiles = max_tiles;
  p.xrow = a.xrow; p.wrow = a.wrow;
  p.x = static_cast<const uint16_t*>(a.x);
  p.ws1 = static_cast<const uint16_t*>(a.ws1);
  p.ws3 = static_cast<const uint16_t*>(a.ws3);
  p.ws2 = static_cast<const uint16_t*>(a.ws2);
  p.h = reinterpret_cast<uint16_t*>(a.ws + L.h_hi);
  p.hs = reinterpret_cast<uint16_t*>(a.ws + L.hs_hi);
  p.y = reinterpret_cast<float*>(a.ws + L.y);
  p.ys = reinterpret_cast<float*>(a.ws + L.ys);

  if ((e = stage_open(kStageUp)) != hipSuccess) return e;
  p.row_tiles = (I > Is ? I : Is) / 128;
  const unsigned up_blocks = static_cast<unsigned>(max_tiles * p.row_tiles);
  for (int r = 0; r < repeat; ++r) {
    if (q3) launch_kernel(k_pf_up<true>, up_blocks, kPfThreads, kPfLdsBytes, s, p);
    else launch_kernel(k_pf_up<false>, up_blocks, kPfThreads, kPfLdsBytes, s, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if ((e = stage_open(kStageDown)) != hipSuccess) return e;
  p.row_tiles = H / kPfRows;
  const unsigned down_blocks = static_cast<unsigned>(max_tiles * p.row_tiles);
  for (int r = 0; r < repeat; ++r) {
    if (q3) launch_kernel(k_pf_down<true>, down_blocks, kPfThreads, kPfLdsBytes, s, p);
    else launch_kernel(k_pf_down<false>, down_blocks, kPfThreads, kPfLdsBytes, s, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace dsk
