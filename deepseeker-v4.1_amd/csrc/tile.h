// Device building blocks of the expert products: 16-row weight tiles on
// v_mfma_f32_16x16x32_bf16.
//
// Lane l of a wave owns weight row (l & 15) -- the A operand row -- and token
// slot (l & 15) -- the B operand column; its lane group g = l >> 4 owns the
// 32-code K chunk [128*b + 32*g, +32) of K block b.  FP4: one 128-bit word of
// codes plus one E8M0 byte per lane and block, so a wave reads 16 rows x 64
// contiguous bytes per block; word j (codes 32g+8j .. +8) is MFMA j's A
// operand after v_cvt_scalef32_pk_bf16_fp4 (two codes per instruction, scale
// applied, exact in bf16).  bf16 weights: four 128-bit words per lane and
// block.  The B operand of the same lane is the activation at exactly the
// same K positions, so A and B agree on the K-slot mapping.  The output of
// one MFMA: lane l holds rows 4*(l>>4) .. +3 of token slot (l & 15).
#pragma once

#include "dsk_internal.h"

namespace dsk {

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4& v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ u32x4 ldg16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

__device__ __forceinline__ bf16x8 fp4_word_to_bf16x8(uint32_t word, float scale) {
  bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 0);
  bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 1);
  bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 2);
  bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 3);
  u32x4 r{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
          __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3)};
  return as_bf16x8(r);
}

// Raw A-operand data of one lane for one K block.
struct RawFP4 { u32x4 c; uint32_t s; };
struct RawBF16 { u32x4 v[4]; };

__device__ __forceinline__ void load_raw(RawFP4& r, const uint8_t* W, const uint8_t* S, int64_t row,
                                         int K, int kc, bool ok) {
  if (ok) {
    r.c = ldg16(W + row * (K / 2) + kc / 2);
    r.s = S[row * (K / 32) + kc / 32];
  } else {
    r.c = u32x4{0u, 0u, 0u, 0u};
    r.s = 127u;
  }
}

__device__ __forceinline__ void load_raw(RawBF16& r, const uint16_t* W, int64_t row, int K, int kc,
                                         bool ok) {
#pragma unroll
  for (int j = 0; j < 4; ++j) r.v[j] = ok ? ldg16(W + row * K + kc + 8 * j) : u32x4{0u, 0u, 0u, 0u};
}

__device__ __forceinline__ bf16x8 a_operand(const RawFP4& r, int j) {
  const float sc = e8m0_to_f32(r.s);
  const uint32_t w = j == 0 ? r.c.x : (j == 1 ? r.c.y : (j == 2 ? r.c.z : r.c.w));
  return fp4_word_to_bf16x8(w, sc);
}

__device__ __forceinline__ bf16x8 a_operand(const RawBF16& r, int j) { return as_bf16x8(r.v[j]); }

// B operand word j of one lane from a 16-bit activation row (global or LDS).
__device__ __forceinline__ bf16x8 b_operand(const uint16_t* row, int kc, int j, bool ok) {
  return ok ? as_bf16x8(*reinterpret_cast<const u32x4*>(row + kc + 8 * j)) : bf16x8{};
}

// acc += A(block) x B(block) for one K block.
template <typename Raw>
__device__ __forceinline__ void mma_block(const Raw& a, const uint16_t* brow, int kc, bool ok,
                                          f32x4& acc) {
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = mfma16(a_operand(a, j), b_operand(brow, kc, j, ok), acc);
}

// Two A tiles (gate and up rows) share the B operand.
template <typename Raw>
__device__ __forceinline__ void mma_block2(const Raw& a1, const Raw& a3, const uint16_t* brow, int kc,
                                           bool ok, f32x4& acc1, f32x4& acc3) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16x8 b = b_operand(brow, kc, j, ok);
    acc1 = mfma16(a_operand(a1, j), b, acc1);
    acc3 = mfma16(a_operand(a3, j), b, acc3);
  }
}

// float -> (hi, lo) bf16 pair with x = hi + lo to about 2^-17.
__device__ __forceinline__ void split_bf16(float v, uint16_t& hi, uint16_t& lo) {
  hi = f32_to_bf16_bits(v);
  lo = f32_to_bf16_bits(v - bf16_bits_to_f32(hi));
}

__device__ __forceinline__ float silu_clamped(float g, float u, float limit) {
  const float gg = fminf(g, limit);
  const float uu = fminf(fmaxf(u, -limit), limit);
  return gg / (1.0f + expf(-gg)) * uu;
}

}  // namespace dsk
