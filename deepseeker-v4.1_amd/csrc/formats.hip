// Weight-format kernels: FP4 (e2m1 + E8M0) and Q3 (3-bit affine, group 64)
// dequantisation and quantisation.
//
// FP4 decode follows the reference's e2m1 table and E8M0 scale
// (src/deepseeker/metal_fp4.py:21-26, 96-103): one thread per 32-code group,
// 16 packed bytes in one 128-bit load, decoded with gfx950's scaled FP4
// conversion (v_cvt_scalef32_pk_{f32,bf16}_fp4, two codes per instruction),
// the same instruction the expert GEMV uses in its load stage.
#include "dsk_internal.h"

// Dequantised values must match the oracle bit for bit: no fused multiply-add.
#pragma clang fp contract(off)

namespace dsk {
namespace {

constexpr int kThreads = 256;

// 8 codes of one 32-bit word -> 8 floats (scale applied).  The conversion
// decodes code 0x8 to -0; "+ 0.0f" turns that into the table's +0 (no other
// value changes).
__device__ __forceinline__ void fp4_word_to_f32(uint32_t word, float scale, float* o) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  f32x2 a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 0);
  f32x2 b = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 1);
  f32x2 c = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 2);
  f32x2 d = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 3);
  o[0] = a.x + 0.0f; o[1] = a.y + 0.0f; o[2] = b.x + 0.0f; o[3] = b.y + 0.0f;
  o[4] = c.x + 0.0f; o[5] = c.y + 0.0f; o[6] = d.x + 0.0f; o[7] = d.y + 0.0f;
}

// Two bf16 in one word: a negative zero half becomes +0.
__device__ __forceinline__ uint32_t bf16_pair_plus_zero(uint32_t w) {
  const uint32_t lo = (w & 0x7fffu) ? (w & 0xffffu) : 0u;
  const uint32_t hi = (w & 0x7fff0000u) ? (w & 0xffff0000u) : 0u;
  return lo | hi;
}

__global__ __launch_bounds__(kThreads) void k_fp4_dequant_f32(
    const uint8_t* __restrict__ packed, const uint8_t* __restrict__ scales,
    int64_t groups, float* __restrict__ out) {
  int64_t gidx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (gidx >= groups) return;
  u32x4 w = *reinterpret_cast<const u32x4*>(packed + gidx * 16);
  float sc = e8m0_to_f32(scales[gidx]);
  float v[32];
  fp4_word_to_f32(w.x, sc, v + 0);
  fp4_word_to_f32(w.y, sc, v + 8);
  fp4_word_to_f32(w.z, sc, v + 16);
  fp4_word_to_f32(w.w, sc, v + 24);
  f32x4* o = reinterpret_cast<f32x4*>(out + gidx * 32);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = f32x4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
}

__global__ __launch_bounds__(kThreads) void k_fp4_dequant_bf16(
    const uint8_t* __restrict__ packed, const uint8_t* __restrict__ scales,
    int64_t groups, uint16_t* __restrict__ out) {
  int64_t gidx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (gidx >= groups) return;
  u32x4 w = *reinterpret_cast<const u32x4*>(packed + gidx * 16);
  float sc = e8m0_to_f32(scales[gidx]);
  uint32_t words[4] = {w.x, w.y, w.z, w.w};
  u32x4 res[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(words[q], sc, 0);
    bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(words[q], sc, 1);
    bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(words[q], sc, 2);
    bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(words[q], sc, 3);
    res[q] = u32x4{bf16_pair_plus_zero(__builtin_bit_cast(uint32_t, p0)),
                   bf16_pair_plus_zero(__builtin_bit_cast(uint32_t, p1)),
                   bf16_pair_plus_zero(__builtin_bit_cast(uint32_t, p2)),
                   bf16_pair_plus_zero(__builtin_bit_cast(uint32_t, p3))};
  }
  u32x4* o = reinterpret_cast<u32x4*>(out + gidx * 32);
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = res[q];
}

// OCP FP8 E4M3 (e4m3fn): sign, 4 exponent bits (bias 7), 3 mantissa bits; no
// infinities, exponent 15 with mantissa 7 is NaN, exponent 0 is subnormal
// (m/8 * 2^-6).  Every value times a power of two stays exact in float32.
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  const uint32_t e = (b >> 3) & 0xFu, m = b & 7u;
  float v;
  if (e == 15u && m == 7u) v = __builtin_nanf("");
  else if (e == 0u) v = ldexpf(static_cast<float>(m), -9);
  else v = ldexpf(static_cast<float>(8u + m), static_cast<int>(e) - 10);
  return (b & 0x80u) ? -v : v;
}

// FP8 block dequant: codes [rows, cols] (one byte each) with one E8M0 scale
// per 32 x 32 block (scales [rows/32, cols/32]); thread = 16 consecutive codes.
template <bool kBF16>
__global__ __launch_bounds__(kThreads) void k_fp8_block_dequant(const uint8_t* __restrict__ codes,
                                                                const uint8_t* __restrict__ scales,
                                                                int64_t rows, int64_t cols, void* out) {
  const int64_t chunks = rows * (cols / 16);
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= chunks) return;
  const int64_t r = i / (cols / 16), c0 = (i % (cols / 16)) * 16;
  const u32x4 w = *reinterpret_cast<const u32x4*>(codes + r * cols + c0);
  const float sc = e8m0_to_f32(scales[(r / 32) * (cols / 32) + c0 / 32]);
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
  float v[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) v[q] = e4m3_to_f32((words[q / 4] >> (8 * (q % 4))) & 0xFFu) * sc;
  if constexpr (kBF16) {
    uint32_t packed[8];
#pragma unroll
    for (int q = 0; q < 8; ++q)
      packed[q] = f32_to_bf16_bits(v[2 * q]) | (uint32_t(f32_to_bf16_bits(v[2 * q + 1])) << 16);
    u32x4* o = reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + r * cols + c0);
    o[0] = u32x4{packed[0], packed[1], packed[2], packed[3]};
    o[1] = u32x4{packed[4], packed[5], packed[6], packed[7]};
  } else {
    f32x4* o = reinterpret_cast<f32x4*>(static_cast<float*>(out) + r * cols + c0);
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
  }
}

// Spec quantiser: per 32-group scale 2^ceil(log2(amax/6)), nearest-even e2m1
// code, saturating at 6, no negative zero.
__global__ __launch_bounds__(kThreads) void k_fp4_quantize(
    const float* __restrict__ w, int64_t groups, uint8_t* __restrict__ packed,
    uint8_t* __restrict__ scales) {
  int64_t gidx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (gidx >= groups) return;
  const f32x4* src = reinterpret_cast<const f32x4*>(w + gidx * 32);
  float v[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    f32x4 t = src[i];
    v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  int e = 0;
  if (amax != 0.f) {
    int x;
    float m = frexpf(amax, &x);
    e = (m <= 0.75f) ? x - 3 : x - 2;
  }
  int sb = min(max(e + 127, 0), 254);
  int eff = sb - 127;
  uint32_t outw[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    float q = ldexpf(fabsf(v[i]), -eff);
    uint32_t mag = (q > 0.25f) + (q >= 0.75f) + (q > 1.25f) + (q >= 1.75f) +
                   (q > 2.5f) + (q >= 3.5f) + (q > 5.0f);
    uint32_t code = (mag != 0u && v[i] < 0.f) ? (mag | 8u) : mag;
    outw[i >> 3] |= code << (4 * (i & 7));
  }
  *reinterpret_cast<u32x4*>(packed + gidx * 16) = u32x4{outw[0], outw[1], outw[2], outw[3]};
  scales[gidx] = static_cast<uint8_t>(sb);
}

// Canonical Q3 layout.  A 128-code block of a row is 48 bytes; lane group g
// (0..3) owns words d0..d2 at byte 12*g and holds the consecutive codes
// 32*g + 8*m + j (m, j < 4, 8); pair P = 4*m + j/2: P < 15 in word P/5 at
// bits 3*(P%5) (even j) and 16 + 3*(P%5) (odd j); pair 15 in bits 15 / 31 of
// the three words.
__device__ __forceinline__ void q3_block_codes(const uint32_t* wds /*[4][3]*/, uint8_t* q /*[128]*/) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t d0 = wds[3 * g], d1 = wds[3 * g + 1], d2 = wds[3 * g + 2];
    const uint32_t d[3] = {d0, d1, d2};
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      int m = p >> 2, i = p & 3;
      uint32_t lo, hi;
      if (p < 15) {
        uint32_t wv = d[p / 5];
        int s = 3 * (p % 5);
        lo = (wv >> s) & 7u;
        hi = (wv >> (16 + s)) & 7u;
      } else {
        lo = ((d0 >> 15) & 1u) | (((d1 >> 15) & 1u) << 1) | (((d2 >> 15) & 1u) << 2);
        hi = ((d0 >> 31) & 1u) | (((d1 >> 31) & 1u) << 1) | (((d2 >> 31) & 1u) << 2);
      }
      q[32 * g + 8 * m + 2 * i] = static_cast<uint8_t>(lo);
      q[32 * g + 8 * m + 2 * i + 1] = static_cast<uint8_t>(hi);
    }
  }
}

// Codes of one 128-code block -> its four lane-group chunks (words [g][3]).
__device__ __forceinline__ void q3_block_pack(const uint8_t* q /*[128]*/, uint32_t* wds /*[12]*/) {
#pragma unroll
  for (int i = 0; i < 12; ++i) wds[i] = 0u;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      int m = p >> 2, i = p & 3;
      uint32_t lo = q[32 * g + 8 * m + 2 * i], hi = q[32 * g + 8 * m + 2 * i + 1];
      if (p < 15) {
        int s = 3 * (p % 5);
        wds[3 * g + p / 5] |= (lo << s) | (hi << (16 + s));
      } else {
#pragma unroll
        for (int t = 0; t < 3; ++t)
          wds[3 * g + t] |= (((lo >> t) & 1u) << 15) | (((hi >> t) & 1u) << 31);
      }
    }
  }
}

// Stores the chunks of block b (row b / (cols/128), block b % (cols/128)) at their place.
__device__ __forceinline__ void q3_block_store(uint8_t* __restrict__ packed, int cols, int64_t b,
                                               const uint32_t* wds) {
  const int nbk = cols / 128;
  uint8_t* row = packed + (b / nbk) * (cols / 8 * 3);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    uint32_t* dst = reinterpret_cast<uint32_t*>(row + q3_chunk_offset(cols, static_cast<int>(b % nbk), g));
#pragma unroll
    for (int i = 0; i < 3; ++i) dst[i] = wds[3 * g + i];
  }
}

// One thread per 128-code block of one row.
__global__ __launch_bounds__(kThreads) void k_q3_quantize(
    const float* __restrict__ w, int64_t blocks, int cols, uint8_t* __restrict__ packed,
    uint16_t* __restrict__ scales, uint16_t* __restrict__ biases) {
  int64_t b = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (b >= blocks) return;
  const float* src = w + b * 128;
  uint8_t q[128];
#pragma unroll
  for (int grp = 0; grp < 2; ++grp) {
    float vmin = src[grp * 64], vmax = src[grp * 64];
    for (int i = 1; i < 64; ++i) {
      float t = src[grp * 64 + i];
      vmin = fminf(vmin, t);
      vmax = fmaxf(vmax, t);
    }
    float sc32 = (vmax - vmin) / 7.0f;
    _Float16 s16 = static_cast<_Float16>(sc32);
    _Float16 b16 = static_cast<_Float16>(vmin);
    float s = static_cast<float>(s16), bb = static_cast<float>(b16);
    for (int i = 0; i < 64; ++i) {
      float qq = 0.f;
      if (s != 0.f) qq = fminf(fmaxf(rintf((src[grp * 64 + i] - bb) / s), 0.f), 7.f);
      q[grp * 64 + i] = static_cast<uint8_t>(qq);
    }
    scales[2 * b + grp] = __builtin_bit_cast(uint16_t, s16);
    biases[2 * b + grp] = __builtin_bit_cast(uint16_t, b16);
  }
  uint32_t wds[12];
  q3_block_pack(q, wds);
  q3_block_store(packed, cols, b, wds);
}

// Checkpoint q3 (row-major 3-byte packs: a row is a little-endian bit stream
// with code c at bits 3c..3c+2, so a 128-code block is 48 contiguous bytes)
// -> the canonical layout.  One thread per 128-code block of one row.
__global__ __launch_bounds__(kThreads) void k_q3_repack(const uint8_t* __restrict__ src, int64_t blocks, int cols,
                                                        uint8_t* __restrict__ packed) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (b >= blocks) return;
  const uint32_t* w = reinterpret_cast<const uint32_t*>(src + b * 48);   // rows are 48 * cols/128 bytes
  uint32_t wv[13];
#pragma unroll
  for (int i = 0; i < 12; ++i) wv[i] = w[i];
  wv[12] = 0u;
  uint8_t q[128];
#pragma unroll
  for (int c = 0; c < 128; ++c) {
    const int bit = 3 * c, wi = bit >> 5, sh = bit & 31;
    uint32_t v = wv[wi] >> sh;
    if (sh > 29) v |= wv[wi + 1] << (32 - sh);
    q[c] = static_cast<uint8_t>(v & 7u);
  }
  uint32_t wds[12];
  q3_block_pack(q, wds);
  q3_block_store(packed, cols, b, wds);
}

__global__ __launch_bounds__(kThreads) void k_q3_dequant(
    const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, int64_t blocks, int cols, int out_bf16,
    void* __restrict__ out) {
  int64_t b = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (b >= blocks) return;
  uint32_t wds[12];
  const int nbk = cols / 128;
  const uint8_t* row = packed + (b / nbk) * (cols / 8 * 3);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(row + q3_chunk_offset(cols, static_cast<int>(b % nbk), g));
#pragma unroll
    for (int i = 0; i < 3; ++i) wds[3 * g + i] = src[i];
  }
  uint8_t q[128];
  q3_block_codes(wds, q);
  float s[2] = {f16_bits_to_f32(scales[2 * b]), f16_bits_to_f32(scales[2 * b + 1])};
  float bb[2] = {f16_bits_to_f32(biases[2 * b]), f16_bits_to_f32(biases[2 * b + 1])};
  for (int i = 0; i < 128; ++i) {
    float prod = s[i >> 6] * static_cast<float>(q[i]);
    float v = prod + bb[i >> 6];
    if (out_bf16)
      static_cast<uint16_t*>(out)[b * 128 + i] = f32_to_bf16_bits(v);
    else
      static_cast<float*>(out)[b * 128 + i] = v;
  }
}

inline unsigned grid_for(int64_t n) { return static_cast<unsigned>((n + kThreads - 1) / kThreads); }

}  // namespace

hipError_t launch_fp8_block_dequant(const uint8_t* codes, const uint8_t* scales, int64_t rows, int64_t cols,
                                    void* out, int out_dtype, hipStream_t s) {
  const int64_t chunks = rows * (cols / 16);
  if (chunks == 0) return hipSuccess;
  if (out_dtype == DSK_DTYPE_F32) launch_kernel(k_fp8_block_dequant<false>, grid_for(chunks), kThreads, 0, s, codes, scales, rows, cols, out);
  else launch_kernel(k_fp8_block_dequant<true>, grid_for(chunks), kThreads, 0, s, codes, scales, rows, cols, out);
  return hipGetLastError();
}

hipError_t launch_fp4_dequant(const uint8_t* packed, const uint8_t* scales, int64_t rows,
                              int64_t cols, void* out, int out_dtype, hipStream_t s) {
  int64_t groups = rows * (cols / 32);
  if (groups == 0) return hipSuccess;
  if (out_dtype == DSK_DTYPE_F32)
    launch_kernel(k_fp4_dequant_f32, grid_for(groups), kThreads, 0, s, packed, scales, groups,
                                                              static_cast<float*>(out));
  else
    launch_kernel(k_fp4_dequant_bf16, grid_for(groups), kThreads, 0, s, packed, scales, groups,
                                                               static_cast<uint16_t*>(out));
  return hipGetLastError();
}

hipError_t launch_fp4_quantize(const float* w, int64_t rows, int64_t cols, uint8_t* packed,
                               uint8_t* scales, hipStream_t s) {
  int64_t groups = rows * (cols / 32);
  if (groups == 0) return hipSuccess;
  launch_kernel(k_fp4_quantize, grid_for(groups), kThreads, 0, s, w, groups, packed, scales);
  return hipGetLastError();
}

hipError_t launch_q3_quantize(const float* w, int64_t rows, int64_t cols, uint8_t* packed,
                              uint16_t* scales, uint16_t* biases, hipStream_t s) {
  int64_t blocks = rows * (cols / 128);
  if (blocks == 0) return hipSuccess;
  launch_kernel(k_q3_quantize, grid_for(blocks), kThreads, 0, s, w, blocks, static_cast<int>(cols), packed, scales, biases);
  return hipGetLastError();
}

hipError_t launch_q3_repack(const uint8_t* src, int64_t rows, int64_t cols, uint8_t* packed, hipStream_t s) {
  const int64_t blocks = rows * (cols / 128);
  if (blocks == 0) return hipSuccess;
  launch_kernel(k_q3_repack, grid_for(blocks), kThreads, 0, s, src, blocks, static_cast<int>(cols), packed);
  return hipGetLastError();
}

hipError_t launch_q3_dequant(const uint8_t* packed, const uint16_t* scales,
                             const uint16_t* biases, int64_t rows, int64_t cols, void* out,
                             int out_dtype, hipStream_t s) {
  int64_t blocks = rows * (cols / 128);
  if (blocks == 0) return hipSuccess;
  launch_kernel(k_q3_dequant, grid_for(blocks), kThreads, 0, s, packed, scales, biases, blocks, static_cast<int>(cols),
                                                     out_dtype == DSK_DTYPE_BF16, out);
  return hipGetLastError();
}

}  // namespace dsk
