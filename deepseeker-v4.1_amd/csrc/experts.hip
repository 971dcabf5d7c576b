// Routed experts, shared expert and combine of the MoE layer.
//
// Replaces the per-expert loop of the reference's moe_layer
// (src/deepseeker/mlx_forward.py:388-406: gate/up qmm, clamp, SiLU, route
// weight, w2 qmm, scatter-add), the shared expert
// (src/deepseeker/mlx_runner.py:765-783) and the final add and cast
// (mlx_forward.py:409-419).
//
// Decode-shaped products run on MFMA tiles of 16 weight rows x 16 token
// slots (v_mfma_f32_16x16x32_bf16).  Lane l of a wave owns weight row
// (l & 15) and token slot (l & 15); its lane group g = l >> 4 owns the
// 32-code K chunk [128*b + 32*g, +32) of K block b, loaded as one 128-bit word
// of FP4 codes plus one E8M0 byte (or 64 bytes of bf16 weights), so a wave
// reads 16 rows x 64 contiguous bytes per FP4 block.  Word j of that chunk
// (codes 32g+8j .. +8) is MFMA j's A operand; the B operand of the same lane
// is the activation at exactly those K positions, so A and B agree on the
// K-slot mapping.  FP4 is decoded with v_cvt_scalef32_pk_bf16_fp4 (two codes
// per instruction, E8M0 scale applied; e2m1 x 2^k is exact in bf16).
// Split-K: the waves of a block take K blocks round-robin and reduce their
// 16x16 partials through LDS in a fixed order.
//
// Numerics: products are exact (bf16 x bf16) and accumulate in float32.
// Activations that are not bf16 already (float32 x, the float32 intermediate
// h) are fed as a bf16 hi/lo pair (x = hi + lo, two MFMAs), which keeps them
// to about 2^-17 relative error.  h = silu(min(g,L)) * clip(u,-L,L) * w_route
// is applied in float32 before the split, as in the reference (route weight
// before w2).  The combine sums each token's expert outputs in ascending
// expert id, then adds the shared output rounded to x's dtype, in float32.
#include "tile.h"

namespace dsk {
namespace {

constexpr int kUpWaves = 8;     // split-K ways of the gate/up kernel (K = H)
constexpr int kDownWaves = 4;   // split-K ways of the down kernel (K = I)

__device__ __forceinline__ f32x4 mfma(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ RawFP4 load_fp4(const uint8_t* W, const uint8_t* S, int64_t row,
                                           int K, int kc, bool ok) {
  RawFP4 r;
  if (ok) {
    r.c = ldg16(W + row * (K / 2) + kc / 2);
    r.s = ldg<uint8_t>(S + row * (K / 32) + kc / 32);
  } else {
    r.c = u32x4{0u, 0u, 0u, 0u};
    r.s = 127u;
  }
  return r;
}

__device__ __forceinline__ RawBF16 load_bf16w(const uint16_t* W, int64_t row, int K, int kc, bool ok) {
  RawBF16 r;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    r.v[j] = ok ? ldg16(W + row * K + kc + 8 * j) : u32x4{0u, 0u, 0u, 0u};
  return r;
}

__device__ __forceinline__ void deq(const RawFP4& r, bf16x8 a[4]) {
  const float sc = e8m0_to_f32(r.s);
  a[0] = fp4_word_to_bf16x8(r.c.x, sc);
  a[1] = fp4_word_to_bf16x8(r.c.y, sc);
  a[2] = fp4_word_to_bf16x8(r.c.z, sc);
  a[3] = fp4_word_to_bf16x8(r.c.w, sc);
}

__device__ __forceinline__ void deq(const RawQ3& r, bf16x8 a[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) a[j] = a_operand(r, j);
}

__device__ __forceinline__ void deq(const RawBF16& r, bf16x8 a[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) a[j] = as_bf16x8(r.v[j]);
}

// B operand (16-bit activations) of one lane for one K block.
__device__ __forceinline__ void load_b(const uint16_t* plane, int64_t row, int K, int kc, bool ok,
                                       bf16x8 b[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    b[j] = as_bf16x8(ok ? ldg16(plane + row * K + kc + 8 * j) : u32x4{0u, 0u, 0u, 0u});
}

__device__ __forceinline__ void split_store(uint16_t* hi, uint16_t* lo, int64_t off, const float v[4]) {
  uint16_t h[4], l[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    h[q] = f32_to_bf16_bits(v[q]);
    l[q] = f32_to_bf16_bits(v[q] - bf16_bits_to_f32(h[q]));
  }
  *reinterpret_cast<uint2*>(hi + off) = uint2{h[0] | (uint32_t(h[1]) << 16), h[2] | (uint32_t(h[3]) << 16)};
  *reinterpret_cast<uint2*>(lo + off) = uint2{l[0] | (uint32_t(l[1]) << 16), l[2] | (uint32_t(l[3]) << 16)};
}


struct UpArgs {
  int T, H, I, Is, k;
  float limit;
  const SlotDesc* desc; const int32_t* active;   // active[0] = number of descriptors
  const int32_t* xrow; const float* wrow;        // per dispatch row: token, route weight
  const uint16_t* xb_hi; const uint16_t* xb_lo;  // [T][H] B planes of x
  const uint16_t* ws1; const uint16_t* ws3;      // shared [Is][H] bf16
  uint16_t* h_hi; uint16_t* h_lo;                // [T*k][I]   (dispatch row order)
  uint16_t* hs_hi; uint16_t* hs_lo;              // [T][Is]
  int tiles;                                     // I / 16
  int shared_blocks;                             // Is / 16 (blocks 0 .. shared_blocks-1)
};

// Per-wave partial products of one 16-row tile for NT token tiles, reduced
// across the block's waves, then the clamped SwiGLU epilogue.  Wave w owns
// the contiguous K blocks [w*per, (w+1)*per), walked in groups of G; the
// weight loads of a group are issued before anything that depends on the
// routing (token rows, activations), so they are in flight first.
template <int NT, bool XLO, int G, typename Raw, typename LoadA>
__device__ __forceinline__ void up_tile(const UpArgs& p, LoadA load_a, int K, int row0,
                                        int n_tok, int tok_base, bool shared, float (*red)[64][4]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int nblk = (K + 127) / 128;
  const int per = (nblk + kUpWaves - 1) / kUpWaves;
  const int kb0 = min(wave * per, nblk), kb1 = min(kb0 + per, nblk);
  const bool one_group = per <= G;
  Raw r1[G], r3[G];
  if (one_group) {
#pragma unroll
    for (int i = 0; i < G; ++i) load_a(kb0 + i, kb0 + i < kb1, r1[i], r3[i]);
  }
  for (int c0 = 0; c0 < n_tok; c0 += 16 * NT) {
    int xrow[NT];
    bool tv[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int n = c0 + 16 * nt + r16;
      tv[nt] = n < n_tok;
      xrow[nt] = !tv[nt] ? 0 : (shared ? n : p.xrow[tok_base + n]);
    }
    f32x4 ag[NT], au[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) { ag[nt] = f32x4{0.f, 0.f, 0.f, 0.f}; au[nt] = ag[nt]; }
    for (int gb = kb0; gb < kb1; gb += G) {
      if (!one_group) {
#pragma unroll
        for (int i = 0; i < G; ++i) load_a(gb + i, gb + i < kb1, r1[i], r3[i]);
      }
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int kc = (gb + i) * 128 + g4 * 32;
        const bool kok = gb + i < kb1 && kc < K;
        bf16x8 a1[4], a3[4];
        deq(r1[i], a1);
        deq(r3[i], a3);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          bf16x8 b[4];
          load_b(p.xb_hi, xrow[nt], K, kc, kok && tv[nt], b);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            ag[nt] = mfma(a1[j], b[j], ag[nt]);
            au[nt] = mfma(a3[j], b[j], au[nt]);
          }
          if constexpr (XLO) {
            load_b(p.xb_lo, xrow[nt], K, kc, kok && tv[nt], b);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              ag[nt] = mfma(a1[j], b[j], ag[nt]);
              au[nt] = mfma(a3[j], b[j], au[nt]);
            }
          }
        }
      }
    }
    // Cross-wave reduction (fixed order: wave 0, 1, ...) and epilogue, one token tile at a time.
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (c0 + 16 * nt >= n_tok) break;
      *reinterpret_cast<f32x4*>(&red[wave][lane][0]) = ag[nt];
      *reinterpret_cast<f32x4*>(&red[kUpWaves + wave][lane][0]) = au[nt];
      __syncthreads();
      if (wave == 0 && tv[nt]) {
        float g[4] = {0.f, 0.f, 0.f, 0.f}, u[4] = {0.f, 0.f, 0.f, 0.f};
        for (int w = 0; w < kUpWaves; ++w)
#pragma unroll
          for (int q = 0; q < 4; ++q) { g[q] += red[w][lane][q]; u[q] += red[kUpWaves + w][lane][q]; }
        const int n = c0 + 16 * nt + r16;
        float wr = 1.0f;
        int64_t dst;
        if (shared) {
          dst = static_cast<int64_t>(n) * p.Is;
        } else {
          const int dr = tok_base + n;
          wr = p.wrow[dr];
          dst = static_cast<int64_t>(dr) * p.I;
        }
        float h[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float gg = fminf(g[q], p.limit);
          const float uu = fminf(fmaxf(u[q], -p.limit), p.limit);
          h[q] = gg / (1.0f + expf(-gg)) * uu * wr;
        }
        const int64_t off = dst + row0 + 4 * g4;
        if (shared) split_store(p.hs_hi, p.hs_lo, off, h);
        else split_store(p.h_hi, p.h_lo, off, h);
      }
      __syncthreads();
    }
  }
}

// Load-group sizes (K blocks whose weights one wave holds at once): FP4 is
// 20 bytes per lane, role and block; bf16 is 64.
constexpr int kGroupFP4 = 4;
constexpr int kGroupBF16 = 2;

template <int NT, bool XLO, bool kQ3>
__global__ __launch_bounds__(kUpWaves * 64) void k_up_fp4(UpArgs p) {
  __shared__ float red[2 * kUpWaves][64][4];
  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int b = blockIdx.x;
  if (b >= p.shared_blocks) {
    const int rb = b - p.shared_blocks;
    const int slot = rb / p.tiles, rt = rb % p.tiles;
    if (slot >= p.active[0]) return;
    const SlotDesc* d = p.desc + slot;
    const int row0 = rt * 16;
    const int64_t row = row0 + r16;
    const int K = p.H;
    const uint8_t* W1 = static_cast<const uint8_t*>(d->p[0]);
    const uint8_t* S1 = static_cast<const uint8_t*>(d->p[1]);
    const uint8_t* W3 = static_cast<const uint8_t*>(d->p[3]);
    const uint8_t* S3 = static_cast<const uint8_t*>(d->p[4]);
    if constexpr (kQ3) {
      auto load_a = [&](int blk, bool in, RawQ3& r1, RawQ3& r3) {
        const int kc = blk * 128 + g4 * 32;
        const bool ok = in && kc < K;
        load_role(r1, d->p, 0, row, K, kc, ok);
        load_role(r3, d->p, 1, row, K, kc, ok);
      };
      up_tile<NT, XLO, kGroupFP4, RawQ3>(p, load_a, K, row0, d->n_tok, d->tok_base, false, red);
    } else {
      auto load_a = [&](int blk, bool in, RawFP4& r1, RawFP4& r3) {
        const int kc = blk * 128 + g4 * 32;
        const bool ok = in && kc < K;
        r1 = load_fp4(W1, S1, row, K, kc, ok);
        r3 = load_fp4(W3, S3, row, K, kc, ok);
      };
      up_tile<NT, XLO, kGroupFP4, RawFP4>(p, load_a, K, row0, d->n_tok, d->tok_base, false, red);
    }
  } else {
    const int row0 = b * 16;
    const int64_t row = row0 + r16;
    const int K = p.H;
    auto load_a = [&](int blk, bool in, RawBF16& r1, RawBF16& r3) {
      const int kc = blk * 128 + g4 * 32;
      const bool ok = in && kc < K;
      r1 = load_bf16w(p.ws1, row, K, kc, ok);
      r3 = load_bf16w(p.ws3, row, K, kc, ok);
    };
    up_tile<NT, XLO, kGroupBF16, RawBF16>(p, load_a, K, row0, p.T, 0, true, red);
  }
}

struct DownArgs {
  int T, H, I, Is;
  const SlotDesc* desc; const int32_t* active;
  const uint16_t* ws2;                   // shared [H][Is] bf16
  const uint16_t* h_hi; const uint16_t* h_lo;
  const uint16_t* hs_hi; const uint16_t* hs_lo;
  float* y;                              // [T*k][H]
  float* ys;                             // [T][H]
  int tiles;                             // H / 16
  int shared_blocks;                     // H / 16 when a shared expert is fused, else 0
};

template <int NT, int G, typename Raw, typename LoadA>
__device__ __forceinline__ void down_tile(const DownArgs& p, LoadA load_a, int K, int row0,
                                          int n_tok, int brow_base, const uint16_t* bhi,
                                          const uint16_t* blo, float* out, float (*red)[64][4]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int nblk = (K + 127) / 128;
  const int per = (nblk + kDownWaves - 1) / kDownWaves;
  const int kb0 = min(wave * per, nblk), kb1 = min(kb0 + per, nblk);
  const bool one_group = per <= G;
  Raw r[G];
  if (one_group) {
#pragma unroll
    for (int i = 0; i < G; ++i) load_a(kb0 + i, kb0 + i < kb1, r[i]);
  }
  for (int c0 = 0; c0 < n_tok; c0 += 16 * NT) {
    f32x4 acc[NT];
    bool tv[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
      tv[nt] = c0 + 16 * nt + r16 < n_tok;
    }
    for (int gb = kb0; gb < kb1; gb += G) {
      if (!one_group) {
#pragma unroll
        for (int i = 0; i < G; ++i) load_a(gb + i, gb + i < kb1, r[i]);
      }
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int kc = (gb + i) * 128 + g4 * 32;
        const bool kok = gb + i < kb1 && kc < K;
        bf16x8 a[4];
        deq(r[i], a);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int64_t brow = brow_base + c0 + 16 * nt + r16;
          bf16x8 b[4];
          load_b(bhi, brow, K, kc, kok && tv[nt], b);
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[nt] = mfma(a[j], b[j], acc[nt]);
          load_b(blo, brow, K, kc, kok && tv[nt], b);
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[nt] = mfma(a[j], b[j], acc[nt]);
        }
      }
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (c0 + 16 * nt >= n_tok) break;
      *reinterpret_cast<f32x4*>(&red[wave][lane][0]) = acc[nt];
      __syncthreads();
      if (wave == 0 && tv[nt]) {
        f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int w = 0; w < kDownWaves; ++w) s += *reinterpret_cast<const f32x4*>(&red[w][lane][0]);
        const int64_t brow = brow_base + c0 + 16 * nt + r16;
        *reinterpret_cast<f32x4*>(out + brow * p.H + row0 + 4 * g4) = s;
      }
      __syncthreads();
    }
  }
}

template <int NT, bool kQ3>
__global__ __launch_bounds__(kDownWaves * 64) void k_down_fp4(DownArgs p) {
  __shared__ float red[kDownWaves][64][4];
  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int b = blockIdx.x;
  if (b >= p.shared_blocks) {
    const int rb = b - p.shared_blocks;
    const int slot = rb / p.tiles, rt = rb % p.tiles;
    if (slot >= p.active[0]) return;
    const SlotDesc* d = p.desc + slot;
    const int row0 = rt * 16;
    const int64_t row = row0 + r16;
    const int K = p.I;
    const uint8_t* W2 = static_cast<const uint8_t*>(d->p[6]);
    const uint8_t* S2 = static_cast<const uint8_t*>(d->p[7]);
    if constexpr (kQ3) {
      auto load_a = [&](int blk, bool in, RawQ3& r) {
        const int kc = blk * 128 + g4 * 32;
        load_role(r, d->p, 2, row, K, kc, in && kc < K);
      };
      down_tile<NT, kGroupFP4, RawQ3>(p, load_a, K, row0, d->n_tok, d->tok_base, p.h_hi, p.h_lo, p.y, red);
    } else {
      auto load_a = [&](int blk, bool in, RawFP4& r) {
        const int kc = blk * 128 + g4 * 32;
        r = load_fp4(W2, S2, row, K, kc, in && kc < K);
      };
      down_tile<NT, kGroupFP4, RawFP4>(p, load_a, K, row0, d->n_tok, d->tok_base, p.h_hi, p.h_lo, p.y, red);
    }
  } else {
    const int row0 = b * 16;
    const int64_t row = row0 + r16;
    const int K = p.Is;
    auto load_a = [&](int blk, bool in, RawBF16& r) {
      const int kc = blk * 128 + g4 * 32;
      r = load_bf16w(p.ws2, row, K, kc, in && kc < K);
    };
    down_tile<NT, kGroupBF16, RawBF16>(p, load_a, K, row0, p.T, 0, p.hs_hi, p.hs_lo, p.ys, red);
  }
}

// float32 x -> bf16 hi/lo planes.
__global__ __launch_bounds__(256) void k_split_x(const float* __restrict__ x, int64_t n,
                                                 uint16_t* __restrict__ hi, uint16_t* __restrict__ lo) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  const uint16_t h = f32_to_bf16_bits(v);
  hi[i] = h;
  lo[i] = f32_to_bf16_bits(v - bf16_bits_to_f32(h));
}

// Descriptors and row tables from a caller-supplied dispatch (dsk_experts).
__global__ __launch_bounds__(256) void k_prepare(const int32_t* __restrict__ counts,
                                                 const int32_t* __restrict__ offsets,
                                                 const int32_t* __restrict__ perm,
                                                 const int32_t* __restrict__ active,
                                                 const float* __restrict__ wflat,
                                                 const dsk_expert_ptrs* __restrict__ table, int N,
                                                 int E, int k, SlotDesc* __restrict__ desc,
                                                 int32_t* __restrict__ xrow, float* __restrict__ wrow) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int n_valid = min(offsets[E], N);
  if (i < n_valid) {
    const int p = perm[i];
    xrow[i] = p / k;
    wrow[i] = wflat[p];
  }
  const int n_act = min(active[0], E);
  if (i < n_act) {
    const int e = active[1 + i];
    SlotDesc d;
    d.e = e; d.n_tok = counts[e]; d.tok_base = offsets[e]; d.pad = 0;
    const dsk_expert_ptrs t = table[e];
    d.p[0] = t.w1; d.p[1] = t.s1; d.p[2] = t.b1;
    d.p[3] = t.w3; d.p[4] = t.s3; d.p[5] = t.b3;
    d.p[6] = t.w2; d.p[7] = t.s2; d.p[8] = t.b2;
    d.pad2 = nullptr;
    desc[i] = d;
  }
}

// out[t] = cast( (sum over the token's expert rows in ascending expert id) + shared[t] ),
// shared[t] = ys[t] rounded to x's dtype (fused shared expert) or a
// precomputed x-dtype shared output.
enum SharedMode { kNoShared = 0, kSharedF32 = 1, kSharedExt = 2 };

constexpr int kCombineMaxK = 16;     // top-k the combine handles (validated on the host)
constexpr int kCombineBatch = 8;     // rows of a token whose loads are issued together

// V consecutive values (V = 4 or 8) at element offset f of a row of y
// (float32, or bf16 when YBF16) or of a bf16 / float32 row, as floats.
template <bool BF16, int V>
__device__ __forceinline__ void load_vals(const void* row, int f, float (&o)[V]) {
  if constexpr (BF16) {
    const uint16_t* p = static_cast<const uint16_t*>(row) + f;
    uint32_t w[V / 2];
    if constexpr (V == 8) {
      const u32x4 r = *reinterpret_cast<const u32x4*>(p);
      w[0] = r[0]; w[1] = r[1]; w[2] = r[2]; w[3] = r[3];
    } else {
      const uint2 r = *reinterpret_cast<const uint2*>(p);
      w[0] = r.x; w[1] = r.y;
    }
#pragma unroll
    for (int i = 0; i < V / 2; ++i) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
    const float* p = static_cast<const float*>(row) + f;
#pragma unroll
    for (int i = 0; i < V / 4; ++i) {
      const f32x4 r = *reinterpret_cast<const f32x4*>(p + 4 * i);
#pragma unroll
      for (int q = 0; q < 4; ++q) o[4 * i + q] = r[q];
    }
  }
}

// One block per (token, 256 V-value column group).  The token's ranks, their
// ascending order and the row addresses are the same for every lane: they
// are read into scalar registers and sorted by the scalar unit, so the
// vector work per value is its loads, its adds in order and the rounding.
template <bool XBF16, bool YBF16, int V>
__global__ __launch_bounds__(256) void k_combine(const void* __restrict__ y, const float* __restrict__ ys,
                                                 const void* __restrict__ shared_ext,
                                                 const int32_t* __restrict__ rank, int H, int k,
                                                 int shared_mode, void* __restrict__ out) {
#pragma clang fp contract(off)
  const int t = blockIdx.x;
  const int f = (blockIdx.y * 256 + threadIdx.x) * V;
  if (f >= H) return;
  // The token's k ranks (all loaded together; ranks past k re-read rank
  // k - 1), sorted ascending without the dropped ones (-1): rows[0 .. n).
  int rows[kCombineMaxK];
#pragma unroll
  for (int j = 0; j < kCombineMaxK; ++j)
    rows[j] = __builtin_amdgcn_readfirstlane(rank[static_cast<int64_t>(t) * k + min(j, k - 1)]);
  int n = 0;
#pragma unroll
  for (int j = 0; j < kCombineMaxK; ++j) {
    if (j >= k) break;
    const int r = rows[j];
    if (r < 0) continue;
    // insertion into rows[0 .. n) (rows[j] itself is past n: j >= n)
    int i = n++;
    while (i > 0 && rows[i - 1] > r) { rows[i] = rows[i - 1]; --i; }
    rows[i] = r;
  }
  const size_t ebytes = YBF16 ? 2 : 4;
  const char* yb = static_cast<const char*>(y);
  // the first kCombineBatch rows' loads together (rows past n read row 0, not added)
  float v[kCombineBatch][V];
#pragma unroll
  for (int q = 0; q < kCombineBatch; ++q) {
    const int r = q < n ? rows[q] : 0;
    load_vals<YBF16, V>(yb + static_cast<size_t>(r) * H * ebytes, f, v[q]);
  }
  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0f;
#pragma unroll
  for (int q = 0; q < kCombineBatch; ++q)
    if (q < n) {
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] = acc[i] + v[q][i];
    }
  for (int q = kCombineBatch; q < n; ++q) {
    float w[V];
    load_vals<YBF16, V>(yb + static_cast<size_t>(rows[q]) * H * ebytes, f, w);
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = acc[i] + w[i];
  }
  const size_t o = static_cast<size_t>(t) * H;
  if (shared_mode == kSharedF32) {
    float sv[V];
    load_vals<false, V>(ys + o, f, sv);
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = acc[i] + (XBF16 ? bf16_bits_to_f32(f32_to_bf16_bits(sv[i])) : sv[i]);
  } else if (shared_mode == kSharedExt) {
    float sv[V];
    if constexpr (XBF16) load_vals<true, V>(static_cast<const uint16_t*>(shared_ext) + o, f, sv);
    else load_vals<false, V>(static_cast<const float*>(shared_ext) + o, f, sv);
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = acc[i] + sv[i];
  }
  if constexpr (XBF16) {
    uint32_t w[V / 2];
#pragma unroll
    for (int i = 0; i < V / 2; ++i)
      w[i] = f32_to_bf16_bits(acc[2 * i]) | (uint32_t(f32_to_bf16_bits(acc[2 * i + 1])) << 16);
    uint16_t* ob = static_cast<uint16_t*>(out) + o + f;
    if constexpr (V == 8) *reinterpret_cast<u32x4*>(ob) = u32x4{w[0], w[1], w[2], w[3]};
    else *reinterpret_cast<uint2*>(ob) = uint2{w[0], w[1]};
  } else {
    float* of = static_cast<float*>(out) + o + f;
#pragma unroll
    for (int i = 0; i < V / 4; ++i) *reinterpret_cast<f32x4*>(of + 4 * i) = f32x4{acc[4 * i], acc[4 * i + 1], acc[4 * i + 2], acc[4 * i + 3]};
  }
}

template <int NT, bool XLO>
hipError_t launch_up(const UpArgs& a, unsigned blocks, bool q3, hipStream_t s) {
  if (q3) launch_kernel(k_up_fp4<NT, XLO, true>, blocks, kUpWaves * 64, 0, s, a);
  else launch_kernel(k_up_fp4<NT, XLO, false>, blocks, kUpWaves * 64, 0, s, a);
  return hipGetLastError();
}

template <int NT>
hipError_t launch_down(const DownArgs& a, unsigned blocks, bool q3, hipStream_t s) {
  if (q3) launch_kernel(k_down_fp4<NT, true>, blocks, kDownWaves * 64, 0, s, a);
  else launch_kernel(k_down_fp4<NT, false>, blocks, kDownWaves * 64, 0, s, a);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_zero_fill(u32x4* __restrict__ p, int64_t n16) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n16;
       i += static_cast<int64_t>(gridDim.x) * 256)
    p[i] = u32x4{0u, 0u, 0u, 0u};
}

}  // namespace

hipError_t launch_zero_fill(void* p, size_t bytes, hipStream_t s) {
  const int64_t n16 = static_cast<int64_t>(bytes / 16);
  if (n16 > 0) {
    const int64_t blocks = (n16 + 255) / 256;
    launch_kernel(k_zero_fill, static_cast<unsigned>(blocks < 4096 ? blocks : 4096), 256, 0, s,
        static_cast<u32x4*>(p), n16);
  }
  return hipGetLastError();
}

// out[t] from the routed rows y and the shared output (the combine stage).
hipError_t launch_combine(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a, hipStream_t s,
                          int repeat) {
  const int T = d.tokens, H = d.hidden, Is = d.inter_shared, k = d.top_k;
  const void* y = a.ws + L.y;
  const float* ys = reinterpret_cast<const float*>(a.ws + L.ys);
  // 8 values per lane for large batches (at T=4096 66 -> 62 us: the rank
  // bookkeeping per value halves and the kernel reaches the HBM rate); small
  // ones keep 4 and twice the blocks (B=64: 6.4 us against 7.0)
  const bool v8 = H % 8 == 0 && T >= 128;
  dim3 cg(static_cast<unsigned>(T), static_cast<unsigned>((H + (v8 ? 2047 : 1023)) / (v8 ? 2048 : 1024)));
  int mode = Is > 0 ? kSharedF32 : (a.shared_out ? kSharedExt : kNoShared);
  const void* shared_ext = a.shared_out;
  const bool pf = prefill_gemm(d);
  if (pf && Is > 0) {            // the prefill GEMM wrote the shared output already rounded to bf16
    mode = kSharedExt;
    shared_ext = ys;
  }
  const bool ybf = pf && prefill_rows_bf16(d, nullptr);
  hipError_t e = stage_open(kStageCombine);
  if (e != hipSuccess) return e;
  for (int r = 0; r < repeat; ++r) {
    if (d.x_dtype == DSK_DTYPE_F32 && v8)
      launch_kernel(k_combine<false, false, 8>, cg, 256, 0, s, y, ys, shared_ext, a.rank, H, k, mode, a.out);
    else if (d.x_dtype == DSK_DTYPE_F32)
      launch_kernel(k_combine<false, false, 4>, cg, 256, 0, s, y, ys, shared_ext, a.rank, H, k, mode, a.out);
    else if (ybf && v8)
      launch_kernel(k_combine<true, true, 8>, cg, 256, 0, s, y, ys, shared_ext, a.rank, H, k, mode, a.out);
    else if (ybf)
      launch_kernel(k_combine<true, true, 4>, cg, 256, 0, s, y, ys, shared_ext, a.rank, H, k, mode, a.out);
    else if (v8)
      launch_kernel(k_combine<true, false, 8>, cg, 256, 0, s, y, ys, shared_ext, a.rank, H, k, mode, a.out);
    else
      launch_kernel(k_combine<true, false, 4>, cg, 256, 0, s, y, ys, shared_ext, a.rank, H, k, mode, a.out);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return e;
}

hipError_t launch_experts(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a,
                          hipStream_t s, int repeat) {
  const int T = d.tokens, H = d.hidden, I = d.inter, Is = d.inter_shared, k = d.top_k;
  const int max_slots = (d.n_experts < T * k) ? d.n_experts : T * k;
  const bool x_f32 = d.x_dtype == DSK_DTYPE_F32;
  const bool q3 = d.quant == DSK_QUANT_Q3;
  hipError_t e;
  const SlotDesc* desc = a.desc;
  const int32_t* xrow = a.xrow;
  const float* wrow = a.wrow;
  if (!desc) {
    SlotDesc* dd = reinterpret_cast<SlotDesc*>(a.ws + L.desc);
    int32_t* xr = reinterpret_cast<int32_t*>(a.ws + L.xrow);
    float* wr = reinterpret_cast<float*>(a.ws + L.wrow);
    const int n = T * k > d.n_experts ? T * k : d.n_experts;
    launch_kernel(k_prepare, static_cast<unsigned>((n + 255) / 256), 256, 0, s,
        a.counts, a.offsets, a.perm, a.active, a.weights, a.table, T * k, d.n_experts, k, dd, xr, wr);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    desc = dd; xrow = xr; wrow = wr;
  }
  const uint16_t* xb_hi = static_cast<const uint16_t*>(a.x);
  const uint16_t* xb_lo = nullptr;
  if (prefill_gemm(d)) {
    PrefillArgs pa{desc, a.active, xrow, wrow, a.x, a.ws1, a.ws3, a.ws2, a.ws, a.rows_out, a.x_planes_ready};
    if ((e = launch_experts_prefill(d, L, pa, s, repeat)) != hipSuccess) return e;
    return a.rows_out ? hipSuccess : launch_combine(d, L, a, s, repeat);
  }
  if (grouped_path(d)) {
    if ((e = launch_experts_grouped(d, L, a, desc, xrow, wrow, s, repeat)) != hipSuccess) return e;
    return a.rows_out ? hipSuccess : launch_combine(d, L, a, s, repeat);
  }
  if ((e = stage_open(kStageUp)) != hipSuccess) return e;
  if (x_f32) {
    uint16_t* hi = reinterpret_cast<uint16_t*>(a.ws + L.xb_hi);
    uint16_t* lo = reinterpret_cast<uint16_t*>(a.ws + L.xb_lo);
    const int64_t n = static_cast<int64_t>(T) * H;
    launch_kernel(k_split_x, static_cast<unsigned>((n + 255) / 256), 256, 0, s, static_cast<const float*>(a.x), n, hi, lo);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    xb_hi = hi;
    xb_lo = lo;
  }
  const int nt = (T <= 16) ? 1 : (T <= 32 ? 2 : 4);

  UpArgs u{};
  u.T = T; u.H = H; u.I = I; u.Is = Is; u.k = k; u.limit = d.limit;
  u.desc = desc; u.active = a.active; u.xrow = xrow; u.wrow = wrow;
  u.xb_hi = xb_hi; u.xb_lo = xb_lo;
  u.ws1 = static_cast<const uint16_t*>(a.ws1); u.ws3 = static_cast<const uint16_t*>(a.ws3);
  u.h_hi = reinterpret_cast<uint16_t*>(a.ws + L.h_hi);
  u.h_lo = reinterpret_cast<uint16_t*>(a.ws + L.h_lo);
  u.hs_hi = reinterpret_cast<uint16_t*>(a.ws + L.hs_hi);
  u.hs_lo = reinterpret_cast<uint16_t*>(a.ws + L.hs_lo);
  u.tiles = I / 16;
  u.shared_blocks = Is > 0 ? Is / 16 : 0;
  const unsigned up_blocks = static_cast<unsigned>(u.shared_blocks + max_slots * u.tiles);
  for (int r = 0; r < repeat; ++r) {
    if (x_f32) e = nt == 1 ? launch_up<1, true>(u, up_blocks, q3, s) : nt == 2 ? launch_up<2, true>(u, up_blocks, q3, s) : launch_up<4, true>(u, up_blocks, q3, s);
    else e = nt == 1 ? launch_up<1, false>(u, up_blocks, q3, s) : nt == 2 ? launch_up<2, false>(u, up_blocks, q3, s) : launch_up<4, false>(u, up_blocks, q3, s);
    if (e != hipSuccess) return e;
  }
  if ((e = stage_open(kStageDown)) != hipSuccess) return e;

  DownArgs dn{};
  dn.T = T; dn.H = H; dn.I = I; dn.Is = Is;
  dn.desc = desc; dn.active = a.active;
  dn.ws2 = static_cast<const uint16_t*>(a.ws2);
  dn.h_hi = u.h_hi; dn.h_lo = u.h_lo; dn.hs_hi = u.hs_hi; dn.hs_lo = u.hs_lo;
  dn.y = rows_buffer(a.rows_out, a.ws, L);
  dn.ys = reinterpret_cast<float*>(a.ws + L.ys);
  dn.tiles = H / 16;
  dn.shared_blocks = Is > 0 ? H / 16 : 0;
  const unsigned down_blocks = static_cast<unsigned>(dn.shared_blocks + max_slots * dn.tiles);
  for (int r = 0; r < repeat; ++r) {
    e = nt == 1 ? launch_down<1>(dn, down_blocks, q3, s) : nt == 2 ? launch_down<2>(dn, down_blocks, q3, s) : launch_down<4>(dn, down_blocks, q3, s);
    if (e != hipSuccess) return e;
  }
  return a.rows_out ? hipSuccess : launch_combine(d, L, a, s, repeat);
}

}  // namespace dsk
