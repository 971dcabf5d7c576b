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

// Loads through the global address space.  Weight pointers come from
// descriptor tables, so the compiler cannot infer their address space; a
// generic (flat) load would also count against the LDS wait counter and make
// every LDS wait wait for it.
template <typename T>
__device__ __forceinline__ T ldg(const void* p) {
  return *(const __attribute__((address_space(1))) T*)(p);
}
__device__ __forceinline__ u32x4 ldg16(const void* p) { return ldg<u32x4>(p); }
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gptr(const void* p) {
  return (const __attribute__((address_space(1))) T*)(p);
}

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
    r.s = ldg<uint8_t>(S + row * (K / 32) + kc / 32);
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

// q3 affine (group 64, fp16 scale / bias) in the canonical layout: a
// 128-code block of a row is 48 bytes, lane group g's 12 bytes (three LE
// words) hold its 32 codes 32g + 8m + j as pairs P = 4m + j/2 -- P < 15 at
// bits 3(P%5) / 16 + 3(P%5) of word P/5, pair 15 in bits 15 / 31 of the
// three words.  A lane's 32 codes lie in one 64-group, so one scale and one
// bias per lane and block.
struct RawQ3 { uint32_t w[3]; uint32_t sb; };   // sb: fp16 scale (low), fp16 bias (high)

__device__ __forceinline__ void load_raw(RawQ3& r, const uint8_t* W, const uint16_t* S, const uint16_t* B,
                                         int64_t row, int K, int kc, bool ok) {
  if (ok) {
    const auto src = gptr<uint32_t>(W + row * (K / 8 * 3) + (kc >> 7) * 48 + ((kc >> 5) & 3) * 12);
    r.w[0] = src[0]; r.w[1] = src[1]; r.w[2] = src[2];
    const int64_t gi = row * (K / 64) + kc / 64;
    r.sb = static_cast<uint32_t>(ldg<uint16_t>(S + gi)) | (static_cast<uint32_t>(ldg<uint16_t>(B + gi)) << 16);
  } else {
    r.w[0] = r.w[1] = r.w[2] = 0u;
    r.sb = 0u;
  }
}

// Codes (lo, hi) of pair p of a lane's words.
template <int P>
__device__ __forceinline__ void q3_pair(const RawQ3& r, uint32_t& lo, uint32_t& hi) {
  if constexpr (P < 15) {
    const uint32_t t = r.w[P / 5] >> (3 * (P % 5));
    lo = t & 7u;
    hi = (t >> 16) & 7u;
  } else {
    lo = ((r.w[0] >> 15) & 1u) | ((r.w[1] >> 14) & 2u) | ((r.w[2] >> 13) & 4u);
    hi = ((r.w[0] >> 31) & 1u) | ((r.w[1] >> 30) & 2u) | ((r.w[2] >> 29) & 4u);
  }
}

// MFMA j's 8 dequantised weights: f32(s) * q + f32(b) (two roundings, as the
// format defines), rounded to bf16.
template <int J>
__device__ __forceinline__ bf16x8 q3_operand(const RawQ3& r) {
  const float s = f16_bits_to_f32(static_cast<uint16_t>(r.sb & 0xffffu));
  const float b = f16_bits_to_f32(static_cast<uint16_t>(r.sb >> 16));
  bf16x8 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t lo, hi;
    switch (4 * J + i) {
      case 0: q3_pair<0>(r, lo, hi); break;   case 1: q3_pair<1>(r, lo, hi); break;
      case 2: q3_pair<2>(r, lo, hi); break;   case 3: q3_pair<3>(r, lo, hi); break;
      case 4: q3_pair<4>(r, lo, hi); break;   case 5: q3_pair<5>(r, lo, hi); break;
      case 6: q3_pair<6>(r, lo, hi); break;   case 7: q3_pair<7>(r, lo, hi); break;
      case 8: q3_pair<8>(r, lo, hi); break;   case 9: q3_pair<9>(r, lo, hi); break;
      case 10: q3_pair<10>(r, lo, hi); break; case 11: q3_pair<11>(r, lo, hi); break;
      case 12: q3_pair<12>(r, lo, hi); break; case 13: q3_pair<13>(r, lo, hi); break;
      case 14: q3_pair<14>(r, lo, hi); break; default: q3_pair<15>(r, lo, hi); break;
    }
    v[2 * i] = static_cast<__bf16>(__fadd_rn(__fmul_rn(s, static_cast<float>(lo)), b));
    v[2 * i + 1] = static_cast<__bf16>(__fadd_rn(__fmul_rn(s, static_cast<float>(hi)), b));
  }
  return v;
}

__device__ __forceinline__ bf16x8 a_operand(const RawQ3& r, int j) {
  return j == 0 ? q3_operand<0>(r) : (j == 1 ? q3_operand<1>(r) : (j == 2 ? q3_operand<2>(r) : q3_operand<3>(r)));
}

// Load one role (0: w1, 1: w3, 2: w2) of an expert from its 9 descriptor
// pointers (codes, scales, biases per role).
__device__ __forceinline__ void load_role(RawFP4& r, const void* const* ptr, int role, int64_t row, int K,
                                          int kc, bool ok) {
  load_raw(r, static_cast<const uint8_t*>(ptr[3 * role]), static_cast<const uint8_t*>(ptr[3 * role + 1]),
           row, K, kc, ok);
}
__device__ __forceinline__ void load_role(RawQ3& r, const void* const* ptr, int role, int64_t row, int K,
                                          int kc, bool ok) {
  load_raw(r, static_cast<const uint8_t*>(ptr[3 * role]), static_cast<const uint16_t*>(ptr[3 * role + 1]),
           static_cast<const uint16_t*>(ptr[3 * role + 2]), row, K, kc, ok);
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
