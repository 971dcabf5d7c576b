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
// FP4 experts with H and I multiples of 512 (and 16-byte aligned arrays) run
// both products on the scaled FP4 x FP8 MFMA instead (the MX loop below):
// x and h as two FP8 planes each, which hold their bf16 values exactly (see
// the MX loop's note); on random data the part runs these at ~1.36x the
// bf16 products' rate for the same work.  k_pf_planes writes x's planes
// before the gate/up; the gate/up's epilogue writes h's.
//
// Tile list: one entry per 256 dispatch rows of every active expert, then the
// shared expert's token tiles.  Workgroup b runs on XCD b mod 8; blocks are
// mapped to (tile, weight-row tile) so that each XCD walks a contiguous range
// with the row tiles of one token tile adjacent, which keeps that tile's
// activations in the XCD's L2 while they are reused.
#include "mx.h"

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

// ---------------------------------------------------------------------------
// FP4 kernels' loop: the stage tiles go from global memory straight into LDS
// (global_load_lds_dwordx4: lane i of a wave writes the 16 bytes it loaded at
// the instruction's LDS base + 16 i), so no registers hold a stage between
// its load and its store and no wave waits for a load before it can store.
// Any 16-byte chunk can be sent to any LDS position: the gather of token rows
// stays per lane, and 128-byte tile rows (64 bf16) are swizzled, chunk c of
// row r at position c ^ ((r >> 1) & 7), so the fragment reads (lanes on 16
// consecutive rows at one chunk) touch 16 distinct 16-byte bank groups with
// no padding.  The wait for a stage and the barrier are one s_waitcnt vmcnt(N)
// + s_barrier: the compiler's own barrier would wait for every load in flight.

__device__ __forceinline__ void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                   (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// All but the newest N loads of this wave have landed (in LDS, for the DMA
// loads), its LDS reads are complete, then the workgroup barrier.
template <int N>
__device__ __forceinline__ void wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 7); }

// The DMA loads read 16-byte pieces at 16-byte steps from the given bases.
__device__ __forceinline__ bool aligned16(const void* a, const void* b) {
  return ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15u) == 0;
}

// Stage chunk (row, chunk) loaded by lane i of load j of wave w, for 128-byte
// rows spread over 4 loads per lane: LDS position p = (4 w + j) 64 + i.
__device__ __forceinline__ int dma_row(int w, int j, int i) { return (4 * w + j) * 8 + (i >> 3); }
__device__ __forceinline__ int dma_chunk(int w, int j, int i) { return swz(dma_row(w, j, i), i & 7); }

// All but the newest n (0..7, wave-uniform) loads of this wave have landed.
__device__ __forceinline__ void wait_barrier_n(int n) {
  switch (n) {
    case 0: wait_barrier<0>(); break;
    case 1: wait_barrier<1>(); break;
    case 2: wait_barrier<2>(); break;
    case 3: wait_barrier<3>(); break;
    case 4: wait_barrier<4>(); break;
    case 5: wait_barrier<5>(); break;
    case 6: wait_barrier<6>(); break;
    default: wait_barrier<7>(); break;
  }
}

// FP4 weights (K a multiple of 512).  Each load reads whole 64-byte pieces of
// a row, so that a wave's load touches few cache lines: the codes of two
// stages at once (64 bytes of a row), the E8M0 scales of eight stages at once
// (16 bytes of a row).  The weights stream from beyond L2, so they are loaded
// further ahead than the tokens: when stage st starts, the tokens of stage
// st + 2, the codes of stages st + 4 and st + 5 (st even) and the scales of
// stages st + 8 .. st + 15 (st a multiple of 8).  LDS: three token buffers
// [256][128 B] (stage st in buffer st % 3), three code buffers [256][64 B]
// (stage pair g in buffer g % 3; 16-byte chunk q of row r at position
// q ^ ((r >> 2) & 3)), two scale buffers [256][16 B] (stages 8G..8G+7 in
// buffer G & 1, loaded by waves 0-3).
struct DmaFp4 {
  static constexpr int kB = 0, kBBuf = 32768;
  static constexpr int kC = 3 * kBBuf, kCBuf = 16384;
  static constexpr int kS = kC + 3 * kCBuf, kSBuf = 4096;
  static constexpr int kEnd = kS + 2 * kSBuf;
  static constexpr bool kWaitNewest = true;   // the end of a stage waits for all but its own loads
  const uint8_t* gc[2];   // this lane's code chunk of stage pair 0, loads j = 0, 1
  const uint8_t* gs;      // its row's scales of stages 0..7 (waves 0-3)
  const uint8_t* gb[4];   // token chunks of stage 0
  // code load j of wave w, lane i: row and logical chunk (16 bytes of the row's 64)
  __device__ __forceinline__ static int code_row(int w, int j, int i) { return ((2 * w + j) * 64 + i) >> 2; }
  __device__ __forceinline__ static int code_chunk(int w, int j, int i) {
    return (i & 3) ^ ((code_row(w, j, i) >> 2) & 3);
  }
  __device__ __forceinline__ void tokens(char* lds, int st, int wave) const {
    char* b = lds + kB + (st % 3) * kBBuf;
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(gb[j] + st * (kPfK * 2), b + (4 * wave + j) * 1024);
  }
  __device__ __forceinline__ void codes(char* lds, int g, int wave) const {
    char* c = lds + kC + (g % 3) * kCBuf;
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(gc[j] + g * kPfK, c + (2 * wave + j) * 1024);
  }
  __device__ __forceinline__ int scales(char* lds, int G, int wave) const {
    if (wave >= 4) return 0;
    dma16(gs + G * 16, lds + kS + (G & 1) * kSBuf + wave * 1024);
    return 1;
  }
  // loads before stage 0; returns how many of them stage 0 need not wait for
  __device__ __forceinline__ int prologue(char* lds, int nst, int wave) const {
    scales(lds, 0, wave);
    codes(lds, 0, wave);
    if (nst > 2) codes(lds, 1, wave);
    tokens(lds, 0, wave);
    if (nst > 1) {
      tokens(lds, 1, wave);
      return 4;
    }
    return 0;
  }
  // loads issued when stage st starts; returns their count
  __device__ __forceinline__ int issue_at(char* lds, int st, int nst, int wave) const {
    int n = 0;
    if (st + 2 < nst) {
      tokens(lds, st + 2, wave);
      n += 4;
    }
    if ((st & 1) == 0 && st + 4 < nst) {
      codes(lds, (st + 4) >> 1, wave);
      n += 2;
    }
    if ((st & 7) == 0 && st + 8 < nst) n += scales(lds, (st + 8) >> 3, wave);
    return n;
  }
  __device__ __forceinline__ static const char* bbase(const char* lds, int st) { return lds + kB + (st % 3) * kBBuf; }
  __device__ __forceinline__ static const char* abase(const char*, int) { return nullptr; }
  struct Frag { u32x4 c[4]; float sc[4]; };
  __device__ __forceinline__ static void frag_begin(Frag& f, const char* lds, int st, int wm, int lane) {
    const int h = lane >> 5, l = lane & 31;
    // rows 128 wm + 32 i + l share the chunk swizzle of l
    const char* c = lds + kC + ((st >> 1) % 3) * kCBuf + (128 * wm + l) * 64 +
                    ((((st & 1) * 2 + h) ^ ((l >> 2) & 3)) * 16);
    const char* sp = lds + kS + ((st >> 3) & 1) * kSBuf + (128 * wm + l) * 16 + (st & 7) * 2 + h;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f.c[i] = *reinterpret_cast<const u32x4*>(c + i * 32 * 64);
      f.sc[i] = e8m0_to_f32(*reinterpret_cast<const uint8_t*>(sp + i * 32 * 16));
    }
  }
  __device__ __forceinline__ static bf16x8 operand(const Frag& f, const char*, int i, int ks, int) {
    const uint32_t w = ks == 0 ? f.c[i].x : (ks == 1 ? f.c[i].y : (ks == 2 ? f.c[i].z : f.c[i].w));
    return fp4_word_to_bf16x8(w, f.sc[i]);
  }
};

// bf16 weights (the shared expert): per stage, weights and tokens [256][128 B]
// each, both swizzled; two buffers (three would not fit); the loads of stage
// st + 1 are issued when stage st starts and waited for at its end.
struct DmaBf16 {
  static constexpr int kA = 0, kB = 32768, kBuf = kB + 32768;
  static constexpr int kEnd = 2 * kBuf;
  static constexpr bool kWaitNewest = false;
  const uint8_t* ga[4];
  const uint8_t* gb[4];
  __device__ __forceinline__ void stage(char* lds, int st, int wave) const {
    char* buf = lds + (st & 1) * kBuf;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      dma16(ga[j] + st * (kPfK * 2), buf + kA + (4 * wave + j) * 1024);
      dma16(gb[j] + st * (kPfK * 2), buf + kB + (4 * wave + j) * 1024);
    }
  }
  __device__ __forceinline__ int prologue(char* lds, int, int wave) const {
    stage(lds, 0, wave);
    return 0;
  }
  __device__ __forceinline__ int issue_at(char* lds, int st, int nst, int wave) const {
    if (st + 1 < nst) stage(lds, st + 1, wave);
    return 0;
  }
  __device__ __forceinline__ static const char* bbase(const char* lds, int st) { return lds + (st & 1) * kBuf + kB; }
  __device__ __forceinline__ static const char* abase(const char* lds, int st) { return lds + (st & 1) * kBuf + kA; }
  struct Frag {};
  __device__ __forceinline__ static void frag_begin(Frag&, const char*, int, int, int) {}
  // arow: this lane's first weight row in the stage's tile; koff: its K step's chunk
  __device__ __forceinline__ static bf16x8 operand(const Frag&, const char* arow, int i, int, int koff) {
    return lds16(arow + i * 32 * 128 + koff);
  }
};

// Main loop of one block tile with LDS DMA stages.  Per stage st: issue the
// policy's loads; the previous stage's last K step's MFMAs; K steps 0-2;
// operands of K step 3, kept; wait until stage st + 1 has landed, barrier.
// Wave w multiplies weight rows 128 (w & 1) + [0, 128) by tokens
// 64 (w >> 1) + [0, 64).
template <bool kFull, class P>
__device__ __forceinline__ void pf_loop_dma(const P& src, int nst, int n_ct, char* lds, f32x16 (&acc)[4][2]) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int wm = wave & 1, wn = wave >> 1, h = lane >> 5;
  // rows 32 i + (lane & 31) of a 128-byte-row tile share the swizzle of lane & 31
  int koff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) koff[ks] = swz(lane & 31, 4 * h + ks) * 16;
  const int brow = (64 * wn + (lane & 31)) * 128;
  const int arow = (128 * wm + (lane & 31)) * 128;
  auto ops = [&](KOps& o, const typename P::Frag& fa, const char* B, const char* A, int ks) {
#pragma unroll
    for (int c = 0; c < 2; ++c) o.b[c] = lds16(B + brow + c * 32 * 128 + koff[ks]);
#pragma unroll
    for (int i = 0; i < 4; ++i) o.a[i] = P::operand(fa, A + arow, i, ks, koff[ks]);
  };
  wait_barrier_n(src.prologue(lds, nst, wave));
  KOps o, last;
  for (int st = 0; st < nst; ++st) {
    const int n = src.issue_at(lds, st, nst, wave);
    typename P::Frag fa;
    P::frag_begin(fa, lds, st, wm, lane);
    const char* B = P::bbase(lds, st);
    const char* A = P::abase(lds, st);
    if (st > 0) pf_mma<kFull>(last, n_ct, acc);
    ops(o, fa, B, A, 0);
    pf_mma<kFull>(o, n_ct, acc);
    ops(o, fa, B, A, 1);
    pf_mma<kFull>(o, n_ct, acc);
    ops(o, fa, B, A, 2);
    pf_mma<kFull>(o, n_ct, acc);
    ops(last, fa, B, A, 3);
    if (P::kWaitNewest) wait_barrier_n(n);
    else wait_barrier<0>();
  }
  pf_mma<kFull>(last, n_ct, acc);
}

template <class P>
__device__ __forceinline__ void pf_gemm_dma(const P& src, int nst, int n_ct, char* lds, f32x16 (&acc)[4][2]) {
  if (n_ct == 2) pf_loop_dma<true>(src, nst, n_ct, lds, acc);
  else pf_loop_dma<false>(src, nst, n_ct, lds, acc);
}

// ---------------------------------------------------------------------------
// MX loop: FP4 weights times activations held as two FP8 planes, on
// v_mfma_scale_f32_32x32x64_f8f6f4 (one product per 64-code stage, weight row
// tile and plane).  Operand layout (measured on the part): A lane l holds row
// l & 31, codes [32g, 32g + 32) of the stage (g = l >> 5), low nibble first,
// and the row's E8M0 byte of that 32-group; B lane l holds column l & 31 at
// K [16g, 16g + 16) in bytes 0..15 and [32 + 16g, 32 + 16g + 16) in bytes
// 16..31 and the column's E8M0 byte of 32-group g; C as the 32x32x16 bf16
// product.  A stage's token tile row is 128 bytes: plane 0's 64 then plane
// 1's, swizzled as the bf16 tiles.  Plane 1's scale is plane 0's / 16.
//
// Activation planes in global memory ("stage rows"): row r of K values takes
// 2K bytes, 128 per 64-value stage (plane 0, then plane 1, plain K order),
// and its E8M0 bytes [rows][K / 32] (plane 0's).  Two planes of a bf16 value
// within 2^13 of its 32-group's largest magnitude are exact, so the products
// are those of the bf16 operands; the part sums each stage's 64 products to
// about 2^-14 of the sum of their magnitudes.

__device__ __forceinline__ f32x16 mx32(const u32x4& a, uint32_t sa, const u32x4& blo, const u32x4& bhi,
                                       uint32_t sb, const f32x16& c) {
  const i32x8 av = {static_cast<int32_t>(a.x), static_cast<int32_t>(a.y), static_cast<int32_t>(a.z),
                    static_cast<int32_t>(a.w), 0, 0, 0, 0};
  const i32x8 bv = {static_cast<int32_t>(blo.x), static_cast<int32_t>(blo.y), static_cast<int32_t>(blo.z),
                    static_cast<int32_t>(blo.w), static_cast<int32_t>(bhi.x), static_cast<int32_t>(bhi.y),
                    static_cast<int32_t>(bhi.z), static_cast<int32_t>(bhi.w)};
  // cbsz 4: A is FP4 (e2m1); blgp 0: B is FP8 (e4m3); scale bytes from bits 0..7
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 4, 0, 0, static_cast<int>(sa), 0,
                                                         static_cast<int>(sb));
}

// One stage's operands of a wave: 4 weight fragments with their scale bytes,
// 2 token fragments per plane with their scale bytes (plane 0's).
struct MxOps {
  u32x4 a[4];
  uint32_t sa[4];
  u32x4 b[2][2][2];   // [token fragment][plane][low / high 16 bytes]
  uint32_t sb[2];
};

// 8 products of one plane: acc[i][c] += A(i) x B(c, plane); unless kFull,
// token fragments c >= n_ct (wave-uniform) are skipped.
template <bool kFull>
__device__ __forceinline__ void mx_mma(const MxOps& o, int pl, int n_ct, f32x16 (&acc)[4][2]) {
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    if (kFull || c < n_ct) {
      const uint32_t sb = o.sb[c] - 4u * static_cast<uint32_t>(pl);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i][c] = mx32(o.a[i], o.sa[i], o.b[c][pl][0], o.b[c][pl][1], sb, acc[i][c]);
    }
  }
}

// MX tiles run in workgroups of 4 waves (one per SIMD), two workgroups per
// CU: a tile of 256 weight rows x 128 dispatch rows, K in stages of 64.
// With one 8-wave workgroup per CU every stage's barrier held both waves of
// a SIMD in the same phase (both loading, then both multiplying); two
// independent workgroups drift apart, so one's products run while the
// other waits.  LDS per workgroup (77 824 bytes): tokens 2 x [128][128 B]
// (stage st in buffer st & 1, the plane rows' 128 bytes, chunk c of row r
// at c ^ ((r >> 1) & 7)), codes 2 x [256][64 B] (stage pair g in buffer
// g & 1, chunk q of row r at q ^ ((r >> 2) & 3)), weight scales 2 x
// [256][16 B] and activation exponents 2 x [128][16 B] (stages 8G..8G+7 in
// buffer G & 1).  Stage st + 1's tokens are loaded when stage st starts and
// waited for at its end; code pair g + 1 when stage 2g starts (two stages
// ahead); the scales of group G + 1 when stage 8G starts.
constexpr int kMxThreads = 256;
constexpr int kPfToksMx = 128;   // dispatch rows of an MX tile

struct DmaMx {
  static constexpr int kB = 0, kBBuf = 16384;
  static constexpr int kC = 2 * kBBuf, kCBuf = 16384;
  static constexpr int kS = kC + 2 * kCBuf, kSBuf = 4096;
  static constexpr int kE = kS + 2 * kSBuf, kEBuf = 2048;
  static constexpr int kEnd = kE + 2 * kEBuf;
  const uint8_t* gb[4];   // this lane's token chunk of stage 0, loads j = 0..3
  const uint8_t* gc[4];   // its code chunk of stage pair 0
  const uint8_t* gs;      // the scales of weight row 64 w + lane, stages 0..7
  const uint8_t* ge;      // waves 0, 1: the exponents of token row 64 w + lane, stages 0..7
  // load j of wave w, lane i writes LDS position (4 w + j) 64 + i (16 bytes each)
  __device__ __forceinline__ static int brow(int w, int j, int i) { return ((4 * w + j) * 64 + i) >> 3; }
  __device__ __forceinline__ static int bchunk(int w, int j, int i) { return swz(brow(w, j, i), i & 7); }
  __device__ __forceinline__ static int crow(int w, int j, int i) { return ((4 * w + j) * 64 + i) >> 2; }
  __device__ __forceinline__ static int cchunk(int w, int j, int i) { return (i & 3) ^ ((crow(w, j, i) >> 2) & 3); }
  __device__ __forceinline__ static int tbuf(int st) { return st & 1; }
  __device__ __forceinline__ static int cbuf(int st) { return (st >> 1) & 1; }
  __device__ __forceinline__ void tokens(char* lds, int st, int wave) const {
    char* b = lds + kB + (st & 1) * kBBuf;
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(gb[j] + st * (kPfK * 2), b + (4 * wave + j) * 1024);
  }
  __device__ __forceinline__ void codes(char* lds, int g, int wave) const {
    char* c = lds + kC + (g & 1) * kCBuf;
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(gc[j] + g * kPfK, c + (4 * wave + j) * 1024);
  }
  __device__ __forceinline__ int scales(char* lds, int G, int wave) const {
    dma16(gs + G * 16, lds + kS + (G & 1) * kSBuf + wave * 1024);
    if (wave >= 2) return 1;
    dma16(ge + G * 16, lds + kE + (G & 1) * kEBuf + wave * 1024);
    return 2;
  }
  // loads before stage 0 (all waited for)
  __device__ __forceinline__ void prologue(char* lds, int nst, int wave) const {
    scales(lds, 0, wave);
    codes(lds, 0, wave);
    tokens(lds, 0, wave);
  }
  // loads issued when stage st starts, stage st + 1's tokens first; returns
  // how many were issued after them (the end of the stage need not wait)
  __device__ __forceinline__ int issue_at(char* lds, int st, int nst, int wave) const {
    if (st + 1 < nst) tokens(lds, st + 1, wave);
    int n = 0;
    if ((st & 1) == 0 && st + 2 < nst) {
      codes(lds, (st >> 1) + 1, wave);
      n += 4;
    }
    if ((st & 7) == 0 && st + 8 < nst) n += scales(lds, (st >> 3) + 1, wave);
    return n;
  }
};

// Main loop of one block tile on the MX products.  Per stage st: issue the
// policy's loads; read the stage's operands (both planes); the previous
// stage's plane-1 products (operands kept in registers); this stage's plane-0
// products; wait until stage st + 1 has landed, barrier.  Wave w (0..3)
// multiplies weight rows 128 (w & 1) + [0, 128) by tokens 64 (w >> 1) +
// [0, 64).
template <bool kFull>
__device__ __forceinline__ void pf_loop_mx(const DmaMx& src, int nst, int n_ct, char* lds, f32x16 (&acc)[4][2]) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int wm = wave & 1, wn = wave >> 1, g = lane >> 5, l = lane & 31;
  // token rows 64 wn + 32 c + l share the swizzle of l
  int koff[2][2];
#pragma unroll
  for (int pl = 0; pl < 2; ++pl)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) koff[pl][hf] = swz(l, 4 * pl + 2 * hf + g) * 16;
  const int brow = (64 * wn + l) * 128;
  const int erow = (64 * wn + l) * 16 + g;
  auto read = [&](MxOps& o, int st) {
    const char* c = lds + DmaMx::kC + DmaMx::cbuf(st) * DmaMx::kCBuf + (128 * wm + l) * 64 +
                    ((((st & 1) * 2 + g) ^ ((l >> 2) & 3)) * 16);
    const char* sp = lds + DmaMx::kS + ((st >> 3) & 1) * DmaMx::kSBuf + (128 * wm + l) * 16 + (st & 7) * 2 + g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o.a[i] = *reinterpret_cast<const u32x4*>(c + i * 32 * 64);
      o.sa[i] = *reinterpret_cast<const uint8_t*>(sp + i * 32 * 16);
    }
    const char* B = lds + DmaMx::kB + DmaMx::tbuf(st) * DmaMx::kBBuf + brow;
    const char* E = lds + DmaMx::kE + ((st >> 3) & 1) * DmaMx::kEBuf + erow + (st & 7) * 2;
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
      for (int pl = 0; pl < 2; ++pl)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
          o.b[cc][pl][hf] = *reinterpret_cast<const u32x4*>(B + cc * 32 * 128 + koff[pl][hf]);
      o.sb[cc] = *reinterpret_cast<const uint8_t*>(E + cc * 32 * 16);
    }
  };
  src.prologue(lds, nst, wave);
  wait_barrier<0>();
  MxOps cur, prev;
  for (int st = 0; st < nst; ++st) {
    const int n = src.issue_at(lds, st, nst, wave);
    read(cur, st);
    if (st > 0) mx_mma<kFull>(prev, 1, n_ct, acc);
    mx_mma<kFull>(cur, 0, n_ct, acc);
    prev = cur;
    wait_barrier_n(n);
  }
  mx_mma<kFull>(prev, 1, n_ct, acc);
}

__device__ __forceinline__ void pf_gemm_mx(const DmaMx& src, int nst, int n_ct, char* lds, f32x16 (&acc)[4][2]) {
  if (n_ct == 2) pf_loop_mx<true>(src, nst, n_ct, lds, acc);
  else pf_loop_mx<false>(src, nst, n_ct, lds, acc);
}

static_assert(DmaBf16::kEnd <= DmaFp4::kEnd && 2 * (Bf16Tile::kBytes + kPfBBytes) <= DmaFp4::kEnd,
              "every loop's stages fit the FP4 DMA loop's LDS");

constexpr size_t kPfLdsBytes = DmaFp4::kEnd;
constexpr size_t kMxLdsBytes = DmaMx::kEnd;
static_assert(2 * kMxLdsBytes <= kMaxLds, "two MX workgroups share a CU's LDS");
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
  float* y;                                 // [T*k][H] float32 (or bf16 when y_bf16)
  uint16_t* ys;                             // [T][H] the shared output, rounded to bf16
  int y_bf16;                               // routed rows rounded to bf16 (FP4 layer, combined here)
  int row_tiles;                            // weight-row tiles per token tile
  const int32_t* mx_on;                     // [0]: routed tiles on the MX kernels (k_pf_tiles)
  const uint8_t* xq; const uint8_t* xe;     // x as FP8 planes in stage rows [T][2H], E8M0 [T][H/32]
  uint8_t* hq; uint8_t* he;                 // h of the MX slots, the same form [T*k][2I], [T*k][I/32]
};

// Logical work unit of this block among tiles [t0, t0 + n): contiguous per
// XCD (b mod 8), row tiles of one token tile adjacent.
__device__ __forceinline__ bool pf_unit_in(const PfArgs& p, int t0, int n, int& tile, int& rt) {
  const int R = n * p.row_tiles;
  const int b = blockIdx.x;
  if (b >= R) return false;
  const int xcd = b & 7;
  int start = 0;
  for (int y = 0; y < xcd; ++y) start += (R - y + 7) >> 3;
  const int L = start + (b >> 3);
  tile = L / p.row_tiles;
  rt = L - tile * p.row_tiles;
  tile += t0;
  return true;
}

// The 8-wave kernels' units: every tile, or only the shared expert's when
// the routed tiles run on the MX kernels.
// Units of tiles t0 .. t0 + n - 1 in 2-D blocks per XCD: XCD x takes a
// quarter of the tiles (token tiles) times half the row tiles, so that its
// workgroups, which run together, share each token tile's activations over
// RT/2 row tiles and each row tile's weights over n/4 token tiles in its L2
// (n % 4 == 0, RT % 2 == 0); the 1-D ranges of pf_unit_in share the weights
// only over the XCD's n/8 token tiles.
__device__ __forceinline__ bool pf_unit_2d(const PfArgs& p, int t0, int n, int& tile, int& rt) {
  const int RT = p.row_tiles, R = n * RT;
  const int b = blockIdx.x;
  if (b >= R) return false;
  const int xcd = b & 7, i = b >> 3;
  const int tn = n >> 2, rn = RT >> 1;   // token tiles and row tiles of an XCD
  tile = t0 + (xcd & 3) * tn + i / rn;
  rt = (xcd >> 2) * rn + i % rn;
  return true;
}

// The shared expert's units when the MX kernels take every routed tile
// (2-D per XCD where the shapes allow), else every unit (1-D per XCD).
__device__ __forceinline__ bool pf_unit(const PfArgs& p, int& tile, int& rt) {
  if (*p.mx_on) {
    const int n = p.tiles[0] - p.tiles[1];
    return n % 4 == 0 && p.row_tiles % 2 == 0 ? pf_unit_2d(p, p.tiles[1], n, tile, rt)
                                               : pf_unit_in(p, p.tiles[1], n, tile, rt);
  }
  return pf_unit_in(p, 0, p.tiles[0], tile, rt);
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
  const int n_ct = max(0, min(2, (cnt - 64 * wn + 31) >> 5));
  const int K = p.H, nst = K / kPfK;
  // local weight row r of the tile: w1 (r & 64 == 0) or w3 row rt*128 + (r >> 7)*64 + (r & 63)
  auto role_of = [](int r) { return (r >> 6) & 1; };
  auto arow_of = [&](int r) { return static_cast<int64_t>(rt * 128 + (r >> 7) * 64 + (r & 63)); };
  auto xrow_of = [&](int r) {
    const int tn = min(r, cnt - 1);
    return static_cast<int64_t>(shared ? first + tn : p.xrow[tok_base + first + tn]);
  };
  f32x16 acc[4][2];
  zero(acc);
  if constexpr (!kQ3) {
    const uint8_t* gb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      gb[j] = reinterpret_cast<const uint8_t*>(p.x + xrow_of(dma_row(wave, j, lane)) * p.H) +
              dma_chunk(wave, j, lane) * 16;
    if (shared) {
      DmaBf16 src;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = dma_row(wave, j, lane);
        src.ga[j] = reinterpret_cast<const uint8_t*>((role_of(r) ? p.ws3 : p.ws1) + arow_of(r) * K) +
                    dma_chunk(wave, j, lane) * 16;
        src.gb[j] = gb[j];
      }
      pf_gemm_dma(src, nst, n_ct, pf_lds, acc);
    } else if (K % 512 == 0 && aligned16(d->p[0], d->p[1]) && aligned16(d->p[3], d->p[4])) {
      DmaFp4 src;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = DmaFp4::code_row(wave, j, lane);
        src.gc[j] = static_cast<const uint8_t*>(d->p[3 * role_of(r)]) + arow_of(r) * (K / 2) +
                    DmaFp4::code_chunk(wave, j, lane) * 16;
      }
      const int rs = (64 * wave + lane) & 255;
      src.gs = static_cast<const uint8_t*>(d->p[3 * role_of(rs) + 1]) + arow_of(rs) * (K / 32);
#pragma unroll
      for (int j = 0; j < 4; ++j) src.gb[j] = gb[j];
      pf_gemm_dma(src, nst, n_ct, pf_lds, acc);
    } else {
      const uint16_t* brow[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) brow[j] = p.x + xrow_of((t >> 3) + 64 * j) * p.H;
      const int r = t >> 1, hf = t & 1;
      const uint8_t* W = static_cast<const uint8_t*>(d->p[3 * role_of(r)]);
      const uint8_t* S = static_cast<const uint8_t*>(d->p[3 * role_of(r) + 1]);
      const int64_t arow = arow_of(r);
      pf_gemm<Fp4Tile, Fp4Tile::Regs>([&](Fp4Tile::Regs& a, int st) { a.load(W, S, arow, K, st, hf); }, brow,
                                      nst, n_ct, pf_lds, acc);
    }
  } else {
    const uint16_t* brow[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) brow[j] = p.x + xrow_of((t >> 3) + 64 * j) * p.H;
    const int r = t >> 1, hf = t & 1;
    const int role = role_of(r);
    const int64_t arow = arow_of(r);
    if (shared) {
      const uint16_t* W = role ? p.ws3 : p.ws1;
      pf_gemm<Bf16Tile, StageBF16>([&](StageBF16& a, int st) { a.load(W, arow, K, st, hf); }, brow, nst, n_ct,
                                   pf_lds, acc);
    } else {
      const uint8_t* W = static_cast<const uint8_t*>(d->p[3 * role]);
      const uint16_t* S = static_cast<const uint16_t*>(d->p[3 * role + 1]);
      const uint16_t* B = static_cast<const uint16_t*>(d->p[3 * role + 2]);
      pf_gemm<Bf16Tile, StageQ3>([&](StageQ3& a, int st) { a.load(W, S, B, arow, K, st, hf); }, brow, nst, n_ct,
                                 pf_lds, acc);
    }
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
  auto hrow_of = [&](int r) { return static_cast<int64_t>(tok_base + first + min(r, cnt - 1)); };
  const int n_ct = max(0, min(2, (cnt - 64 * wn + 31) >> 5));
  const int64_t row0 = static_cast<int64_t>(rt) * 256;   // first w2 row of the tile
  f32x16 acc[4][2];
  zero(acc);
  if constexpr (!kQ3) {
    const uint8_t* gb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      gb[j] = reinterpret_cast<const uint8_t*>(src + hrow_of(dma_row(wave, j, lane)) * K) +
              dma_chunk(wave, j, lane) * 16;
    if (shared) {
      DmaBf16 s;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s.ga[j] = reinterpret_cast<const uint8_t*>(p.ws2 + (row0 + dma_row(wave, j, lane)) * K) +
                  dma_chunk(wave, j, lane) * 16;
        s.gb[j] = gb[j];
      }
      pf_gemm_dma(s, nst, n_ct, pf_lds, acc);
    } else if (K % 512 == 0 && aligned16(d->p[6], d->p[7])) {
      DmaFp4 s;
#pragma unroll
      for (int j = 0; j < 2; ++j)
        s.gc[j] = static_cast<const uint8_t*>(d->p[6]) + (row0 + DmaFp4::code_row(wave, j, lane)) * (K / 2) +
                  DmaFp4::code_chunk(wave, j, lane) * 16;
      s.gs = static_cast<const uint8_t*>(d->p[7]) + (row0 + ((64 * wave + lane) & 255)) * (K / 32);
#pragma unroll
      for (int j = 0; j < 4; ++j) s.gb[j] = gb[j];
      pf_gemm_dma(s, nst, n_ct, pf_lds, acc);
    } else {
      const uint16_t* brow[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) brow[j] = src + hrow_of((t >> 3) + 64 * j) * K;
      const uint8_t* W = static_cast<const uint8_t*>(d->p[6]);
      const uint8_t* S = static_cast<const uint8_t*>(d->p[7]);
      const int64_t arow = row0 + (t >> 1);
      const int hf = t & 1;
      pf_gemm<Fp4Tile, Fp4Tile::Regs>([&](Fp4Tile::Regs& a, int st) { a.load(W, S, arow, K, st, hf); }, brow,
                                      nst, n_ct, pf_lds, acc);
    }
  } else {
    const uint16_t* brow[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) brow[j] = src + hrow_of((t >> 3) + 64 * j) * K;
    const int hf = t & 1;
    const int64_t arow = row0 + (t >> 1);
    if (shared) {
      pf_gemm<Bf16Tile, StageBF16>([&](StageBF16& a, int st) { a.load(p.ws2, arow, K, st, hf); }, brow, nst,
                                   n_ct, pf_lds, acc);
    } else {
      const uint8_t* W = static_cast<const uint8_t*>(d->p[6]);
      const uint16_t* S = static_cast<const uint16_t*>(d->p[7]);
      const uint16_t* B = static_cast<const uint16_t*>(d->p[8]);
      pf_gemm<Bf16Tile, StageQ3>([&](StageQ3& a, int st) { a.load(W, S, B, arow, K, st, hf); }, brow, nst,
                                 n_ct, pf_lds, acc);
    }
  }
  // The shared output is rounded to bf16 here (the combine adds it rounded to
  // x's dtype, bf16 on this path); routed rows stay float32 unless y_bf16.
  const bool narrow = shared || p.y_bf16;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int n = 64 * wn + 32 * c + (lane & 31);
    if (n >= cnt) continue;
    const int64_t drow = tok_base + first + n;
    const int64_t col0 = drow * p.H + rt * 256 + wm * 128 + 4 * (lane >> 5);
    if (narrow) {
      uint16_t* out = shared ? p.ys : reinterpret_cast<uint16_t*>(p.y);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<uint2*>(out + col0 + 32 * i + 8 * q) =
              uint2{pack_bf16x2(acc[i][c][4 * q], acc[i][c][4 * q + 1]),
                    pack_bf16x2(acc[i][c][4 * q + 2], acc[i][c][4 * q + 3])};
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<f32x4*>(p.y + col0 + 32 * i + 8 * q) =
              f32x4{acc[i][c][4 * q], acc[i][c][4 * q + 1], acc[i][c][4 * q + 2], acc[i][c][4 * q + 3]};
    }
  }
}

// MX gate/up: a routed tile of 128 dispatch rows; local weight row r =
// 0..255 of the unit is w1 (r & 64 == 0) or w3 row rt*128 + (r >> 7)*64 +
// (r & 63), so wave rows 0..63 are gate rows and 64..127 the matching up
// rows.  h is rounded to bf16, then written as two FP8 planes in stage rows:
// features f0 + [0, 32) of fragment i (f0 = rt 128 + wm 64 + 32 i) are one
// 32-group; this lane holds 16 of them, at 8 (r >> 2) + 4 g + (r & 3), lane
// l ^ 32 (same token) the other 16.
__global__ __launch_bounds__(kMxThreads, 2) void k_pf_mx_up(PfArgs p) {
  extern __shared__ __align__(16) char mx_lds[];
  int tile, rt;
  if (!*p.mx_on || !pf_unit_in(p, 0, p.tiles[1], tile, rt)) return;
  const int slot = p.tiles[2 + tile], first = p.tiles[2 + p.max_tiles + tile];
  const SlotDesc* d = p.desc + slot;
  const int tok_base = d->tok_base;
  const int cnt = min(kPfToksMx, d->n_tok - first);
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int wm = wave & 1, wn = wave >> 1;
  const int n_ct = max(0, min(2, (cnt - 64 * wn + 31) >> 5));
  const int K = p.H;
  auto role_of = [](int r) { return (r >> 6) & 1; };
  auto arow_of = [&](int r) { return static_cast<int64_t>(rt * 128 + (r >> 7) * 64 + (r & 63)); };
  auto xrow_of = [&](int r) { return static_cast<int64_t>(p.xrow[tok_base + first + min(r, cnt - 1)]); };
  DmaMx src;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    src.gb[j] = p.xq + xrow_of(DmaMx::brow(wave, j, lane)) * (2 * K) + DmaMx::bchunk(wave, j, lane) * 16;
    const int r = DmaMx::crow(wave, j, lane);
    src.gc[j] = static_cast<const uint8_t*>(d->p[3 * role_of(r)]) + arow_of(r) * (K / 2) +
                DmaMx::cchunk(wave, j, lane) * 16;
  }
  const int rs = 64 * wave + lane;
  src.gs = static_cast<const uint8_t*>(d->p[3 * role_of(rs) + 1]) + arow_of(rs) * (K / 32);
  src.ge = p.xe + xrow_of(rs & 127) * (K / 32);
  f32x16 acc[4][2];
  zero(acc);
  pf_gemm_mx(src, K / kPfK, n_ct, mx_lds, acc);
  const int g = lane >> 5;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int n = 64 * wn + 32 * c + (lane & 31);
    if (n >= cnt) continue;
    const int64_t drow = tok_base + first + n;
    const float wr = p.wrow[drow];
    uint8_t* hrow = p.hq + drow * (2 * p.I) + (2 * rt + wm) * 128;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      float hv[16];
      float m = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float v = silu_clamped(acc[i][c][r], acc[i + 2][c][r], p.limit) * wr;
        hv[r] = __uint_as_float(static_cast<uint32_t>(f32_to_bf16_bits(v)) << 16);
        m = fmaxf(m, fabsf(hv[r]));
      }
      m = fmaxf(m, __shfl_xor(m, 32, 64));
      const int e = fp8_plane_exp(m);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float v4[4] = {hv[4 * q], hv[4 * q + 1], hv[4 * q + 2], hv[4 * q + 3]};
        uint32_t w[2];
        fp8_planes4<2>(v4, e, w);
#pragma unroll
        for (int pl = 0; pl < 2; ++pl)
          *reinterpret_cast<uint32_t*>(hrow + 64 * pl + 32 * i + 8 * q + 4 * g) = w[pl];
      }
      if (g == 0) p.he[drow * (p.I / 32) + 4 * rt + 2 * wm + i] = static_cast<uint8_t>(e8m0_byte(e));
    }
  }
}

// MX down: w2 rows rt*256 + [0, 256) by a routed tile of 128 dispatch rows,
// from h's planes; routed rows in float32 or bf16 (y_bf16).
__global__ __launch_bounds__(kMxThreads, 2) void k_pf_mx_down(PfArgs p) {
  extern __shared__ __align__(16) char mx_lds[];
  int tile, rt;
  if (!*p.mx_on || !pf_unit_in(p, 0, p.tiles[1], tile, rt)) return;
  const int slot = p.tiles[2 + tile], first = p.tiles[2 + p.max_tiles + tile];
  const SlotDesc* d = p.desc + slot;
  const int tok_base = d->tok_base;
  const int cnt = min(kPfToksMx, d->n_tok - first);
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int wm = wave & 1, wn = wave >> 1;
  const int n_ct = max(0, min(2, (cnt - 64 * wn + 31) >> 5));
  const int K = p.I;
  const int64_t row0 = static_cast<int64_t>(rt) * 256;
  auto hrow_of = [&](int r) { return static_cast<int64_t>(tok_base + first + min(r, cnt - 1)); };
  DmaMx src;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    src.gb[j] = p.hq + hrow_of(DmaMx::brow(wave, j, lane)) * (2 * K) + DmaMx::bchunk(wave, j, lane) * 16;
    src.gc[j] = static_cast<const uint8_t*>(d->p[6]) + (row0 + DmaMx::crow(wave, j, lane)) * (K / 2) +
                DmaMx::cchunk(wave, j, lane) * 16;
  }
  const int rs = 64 * wave + lane;
  src.gs = static_cast<const uint8_t*>(d->p[7]) + (row0 + rs) * (K / 32);
  src.ge = p.he + hrow_of(rs & 127) * (K / 32);
  f32x16 acc[4][2];
  zero(acc);
  pf_gemm_mx(src, K / kPfK, n_ct, mx_lds, acc);
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int n = 64 * wn + 32 * c + (lane & 31);
    if (n >= cnt) continue;
    const int64_t drow = tok_base + first + n;
    const int64_t col0 = drow * p.H + row0 + wm * 128 + 4 * (lane >> 5);
    if (p.y_bf16) {
      uint16_t* out = reinterpret_cast<uint16_t*>(p.y);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<uint2*>(out + col0 + 32 * i + 8 * q) =
              uint2{pack_bf16x2(acc[i][c][4 * q], acc[i][c][4 * q + 1]),
                    pack_bf16x2(acc[i][c][4 * q + 2], acc[i][c][4 * q + 3])};
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<f32x4*>(p.y + col0 + 32 * i + 8 * q) =
              f32x4{acc[i][c][4 * q], acc[i][c][4 * q + 1], acc[i][c][4 * q + 2], acc[i][c][4 * q + 3]};
    }
  }
}

// x [T][H] bf16 as two FP8 planes in stage rows (the MX gate/up's B tiles),
// one chunk per thread (pf_planes_chunk; H / 8 chunks per row, a multiple of
// 64, so whole waves leave).
__global__ __launch_bounds__(256) void k_pf_planes(const uint16_t* __restrict__ x, int64_t chunks, int H,
                                                  uint8_t* __restrict__ q, uint8_t* __restrict__ ex) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (c >= chunks) return;
  pf_planes_chunk(x, H, c, true, q, ex);
}

// Tile list from the dispatch descriptors (one block of 1024 threads; one
// thread per active expert slot, E <= 1024): routed tiles, then the shared
// expert's tiles of kPfToks tokens.  The routed tiles run on the MX kernels
// (kPfToksMx rows each) when the layer allows it (mx) and every active
// slot's six FP4 arrays are 16-byte aligned (the LDS DMA's pieces), else on
// the 8-wave kernels (kPfToks rows each); tiles[2 + 2 max_tiles] says which.
__global__ __launch_bounds__(1024) void k_pf_tiles(const SlotDesc* __restrict__ desc,
                                                   const int32_t* __restrict__ active, int E, int T,
                                                   int with_shared, int max_tiles, int mx,
                                                   int32_t* __restrict__ tiles) {
  __shared__ int32_t wsum[16];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int n_act = min(active[0], E);
  bool ok = true;
  if (mx && t < n_act) {
    const SlotDesc& d = desc[t];
    ok = aligned16(d.p[0], d.p[1]) && aligned16(d.p[3], d.p[4]) && aligned16(d.p[6], d.p[7]);
  }
  const bool on = mx && __syncthreads_and(ok ? 1 : 0);
  const int rtoks = on ? kPfToksMx : kPfToks;
  const int cnt = t < n_act ? (desc[t].n_tok + rtoks - 1) / rtoks : 0;
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
    tiles[2 + max_tiles + off + j] = j * rtoks;
  }
  const int sh = with_shared ? (T + kPfToks - 1) / kPfToks : 0;
  for (int j = t; j < sh; j += 1024) {
    tiles[2 + total + j] = -1;
    tiles[2 + max_tiles + total + j] = j * kPfToks;
  }
  if (t == 0) {
    tiles[0] = total + sh;
    tiles[1] = total;
    tiles[2 + 2 * max_tiles] = on ? 1 : 0;
  }
}

}  // namespace

int prefill_max_tiles(const dsk_moe_desc& d) {
  const int n = d.tokens * d.top_k;
  const int slots = d.n_experts < n ? d.n_experts : n;
  const int shared = d.inter_shared > 0 ? (d.tokens + kPfToks - 1) / kPfToks : 0;
  const int rtoks = prefill_mx(d) ? kPfToksMx : kPfToks;   // the smaller tile when the layer may use it
  return (n + rtoks - 1) / rtoks + slots + shared;
}

hipError_t launch_experts_prefill(const dsk_moe_desc& d, const Workspace& L, const PrefillArgs& a,
                                  hipStream_t s, int repeat) {
  const int T = d.tokens, H = d.hidden, I = d.inter, Is = d.inter_shared;
  const bool q3 = d.quant == DSK_QUANT_Q3;
  const int max_tiles = prefill_max_tiles(d);
  int32_t* tiles = reinterpret_cast<int32_t*>(a.ws + L.pf_tiles);
  const bool mx = prefill_mx(d);
  launch_kernel(k_pf_tiles, 1, 1024, 0, s, a.desc, a.active, d.n_experts, T, Is > 0 ? 1 : 0, max_tiles,
                mx ? 1 : 0, tiles);
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
  p.y = rows_buffer(a.rows_out, a.ws, L);
  p.ys = reinterpret_cast<uint16_t*>(a.ws + L.ys);
  p.y_bf16 = prefill_rows_bf16(d, a.rows_out) ? 1 : 0;
  p.mx_on = tiles + 2 + 2 * max_tiles;
  if (mx) {
    uint8_t* xp = reinterpret_cast<uint8_t*>(a.ws + L.xp);
    p.xq = xp;
    p.xe = xp + static_cast<size_t>(T) * 2 * H;
    uint8_t* hp = reinterpret_cast<uint8_t*>(a.ws + L.hp);
    p.hq = hp;
    p.he = hp + static_cast<size_t>(T) * d.top_k * 2 * I;
  }

  // MX layers: the routed tiles on the 4-wave MX kernels (two workgroups per
  // CU), then the shared expert's on the 8-wave kernels; each kernel's grid
  // covers its units for either tile size (k_pf_tiles decides on the device)
  if ((e = stage_open(kStageUp)) != hipSuccess) return e;
  const int up_rows = (I > Is ? I : Is) / 128;
  const int64_t x_chunks = static_cast<int64_t>(T) * (H / 8);
  for (int r = 0; r < repeat; ++r) {
    if (mx && !a.x_planes_ready) {
      launch_kernel(k_pf_planes, static_cast<unsigned>((x_chunks + 255) / 256), 256, 0, s,
                    static_cast<const uint16_t*>(a.x), x_chunks, H, const_cast<uint8_t*>(p.xq),
                    const_cast<uint8_t*>(p.xe));
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (mx) {
      p.row_tiles = I / 128;
      launch_kernel(k_pf_mx_up, static_cast<unsigned>(max_tiles * p.row_tiles), kMxThreads, kMxLdsBytes, s, p);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    p.row_tiles = up_rows;
    const unsigned up_blocks = static_cast<unsigned>(max_tiles * p.row_tiles);
    if (q3) launch_kernel(k_pf_up<true>, up_blocks, kPfThreads, kPfLdsBytes, s, p);
    else launch_kernel(k_pf_up<false>, up_blocks, kPfThreads, kPfLdsBytes, s, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if ((e = stage_open(kStageDown)) != hipSuccess) return e;
  p.row_tiles = H / kPfRows;
  const unsigned down_blocks = static_cast<unsigned>(max_tiles * p.row_tiles);
  for (int r = 0; r < repeat; ++r) {
    if (mx) {
      launch_kernel(k_pf_mx_down, down_blocks, kMxThreads, kMxLdsBytes, s, p);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (q3) launch_kernel(k_pf_down<true>, down_blocks, kPfThreads, kPfLdsBytes, s, p);
    else launch_kernel(k_pf_down<false>, down_blocks, kPfThreads, kPfLdsBytes, s, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace dsk
