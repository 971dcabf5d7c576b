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

// Wait for every outstanding vector memory load (s_waitcnt vmcnt(0); expcnt
// and lgkmcnt left alone).  After a staging loop whose stores are guarded,
// the loaded registers stay "pending" on the path that skipped the store, and
// the compiler's wait before their next use would also wait for every weight
// load issued in between; an explicit wait while only the staging loads are
// outstanding costs nothing and clears that state.
__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Loads without a condition: the caller passes an in-range row and K offset.
// The data of a block outside the wave's range is then loaded from a valid
// place and cancelled by a zero activation operand.  (A load under a per-lane
// condition compiles to a branch whose merge copies the loaded registers, and
// every copy waits for its load: a batch's loads then go out one memory
// latency at a time.)
__device__ __forceinline__ void load_raw_nc(RawFP4& r, const uint8_t* W, const uint8_t* S, int64_t row, int K,
                                            int kc) {
  r.c = ldg16(W + row * (K / 2) + kc / 2);
  r.s = ldg<uint8_t>(S + row * (K / 32) + kc / 32);
}

__device__ __forceinline__ void load_raw_nc(RawBF16& r, const uint16_t* W, int64_t row, int K, int kc) {
#pragma unroll
  for (int j = 0; j < 4; ++j) r.v[j] = ldg16(W + row * K + kc + 8 * j);
}

// q3 affine (group 64, fp16 scale / bias) in the canonical layout: lane group
// g's 12 bytes (three LE words, placed by q3_chunk_offset) of a 128-code block
// hold its 32 codes 32g + 8m + j as pairs P = 4m + j/2 -- P < 15 at bits
// 3(P%5) / 16 + 3(P%5) of word P/5, pair 15 in bits 15 / 31 of the three
// words.  A lane's 32 codes lie in one 64-group, so one scale and one bias per
// lane and block.
// s, b: fp16 scale and bias bits (low halves), loaded separately and combined at use
struct RawQ3 { uint32_t w[3]; uint32_t s, b; };

__device__ __forceinline__ void load_raw(RawQ3& r, const uint8_t* W, const uint16_t* S, const uint16_t* B,
                                         int64_t row, int K, int kc, bool ok) {
  if (ok) {
    const auto src = gptr<uint32_t>(W + row * (K / 8 * 3) + q3_chunk_offset(K, kc >> 7, (kc >> 5) & 3));
    r.w[0] = src[0]; r.w[1] = src[1]; r.w[2] = src[2];
    const int64_t gi = row * (K / 64) + kc / 64;
    r.s = ldg<uint16_t>(S + gi);
    r.b = ldg<uint16_t>(B + gi);
  } else {
    r.w[0] = r.w[1] = r.w[2] = 0u;
    r.s = r.b = 0u;
  }
}

// Dequantised values of the code pair at bits [sh, sh+3) / [16+sh, 16+sh+3)
// of word w: one mask, then each code is converted from the byte that holds
// it (v_cvt_f32_ubyteN), which yields q * 2^k for a position-dependent k; the
// matching s * 2^-k (exact: an fp16 scale has 11 significant bits) makes
// fma(s * 2^-k, q * 2^k, b) = round(s*q + b) -- s*q is exact in float32, so
// this is f32(s)*q + f32(b) with the format's rounding.
struct Q3Scales { float s, s2, s8, s16, b; };   // s, s/2, s/8, s/16, bias

__device__ __forceinline__ Q3Scales q3_scales(uint32_t sbits, uint32_t bbits) {
  const float s = f16_bits_to_f32(static_cast<uint16_t>(sbits));
  return Q3Scales{s, s * 0.5f, s * 0.125f, s * 0.0625f, f16_bits_to_f32(static_cast<uint16_t>(bbits))};
}

// Byte k of v as float (v_cvt_f32_ubyteK: no shift or mask needed).
template <int K>
__device__ __forceinline__ float ubyte_f32(uint32_t v) {
  float f;
  if constexpr (K == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(v));
  else if constexpr (K == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(v));
  else if constexpr (K == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(v));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(v));
  return f;
}

template <int SH>
__device__ __forceinline__ void q3_pair_f(uint32_t w, const Q3Scales& c, float& lo, float& hi) {
  const uint32_t m = w & ((7u << SH) | (7u << (16 + SH)));
  if constexpr (SH == 0) {          // bytes 0 / 2 hold q
    lo = __fmaf_rn(c.s, ubyte_f32<0>(m), c.b);
    hi = __fmaf_rn(c.s, ubyte_f32<2>(m), c.b);
  } else if constexpr (SH == 3) {   // bytes 0 / 2 hold 8q
    lo = __fmaf_rn(c.s8, ubyte_f32<0>(m), c.b);
    hi = __fmaf_rn(c.s8, ubyte_f32<2>(m), c.b);
  } else if constexpr (SH == 6) {   // straddles a byte boundary: shift first
    const uint32_t n = m >> 6;
    lo = __fmaf_rn(c.s, ubyte_f32<0>(n), c.b);
    hi = __fmaf_rn(c.s, ubyte_f32<2>(n), c.b);
  } else if constexpr (SH == 9) {   // bytes 1 / 3 hold 2q
    lo = __fmaf_rn(c.s2, ubyte_f32<1>(m), c.b);
    hi = __fmaf_rn(c.s2, ubyte_f32<3>(m), c.b);
  } else {                          // SH == 12: bytes 1 / 3 hold 16q
    lo = __fmaf_rn(c.s16, ubyte_f32<1>(m), c.b);
    hi = __fmaf_rn(c.s16, ubyte_f32<3>(m), c.b);
  }
}

// Pair P of a lane's 32 codes (P < 15: word P/5, shift 3(P%5); P = 15: bits
// 15 / 31 of the three words, gathered into bits 0-2 / 16-18).
template <int P>
__device__ __forceinline__ void q3_pair_val(const RawQ3& r, const Q3Scales& c, float& lo, float& hi) {
  if constexpr (P < 15) {
    q3_pair_f<3 * (P % 5)>(r.w[P / 5], c, lo, hi);
  } else {
    const uint32_t t = ((r.w[0] >> 15) & 0x00010001u) | ((r.w[1] >> 14) & 0x00020002u) |
                       ((r.w[2] >> 13) & 0x00040004u);
    q3_pair_f<0>(t, c, lo, hi);
  }
}

// MFMA j's 8 dequantised weights: f32(s) * q + f32(b) (the format's two
// roundings; s*q is exact), rounded to bf16.
template <int J>
__device__ __forceinline__ bf16x8 q3_operand(const RawQ3& r) {
  const Q3Scales c = q3_scales(r.s, r.b);
  float v[8];
  q3_pair_val<4 * J + 0>(r, c, v[0], v[1]);
  q3_pair_val<4 * J + 1>(r, c, v[2], v[3]);
  q3_pair_val<4 * J + 2>(r, c, v[4], v[5]);
  q3_pair_val<4 * J + 3>(r, c, v[6], v[7]);
  bf16x8 o;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = static_cast<__bf16>(v[i]);
  return o;
}

__device__ __forceinline__ bf16x8 a_operand(const RawQ3& r, int j) {
  return j == 0 ? q3_operand<0>(r) : (j == 1 ? q3_operand<1>(r) : (j == 2 ? q3_operand<2>(r) : q3_operand<3>(r)));
}

// Factored q3 product.  Per 64-group, x . W = s * sum(q x) + b * sum(x), so
// the MFMA can take the raw codes and the group's scale and bias are applied
// to its output.  A code pair masked into the low mantissa bits of 128.0
// (bf16 0x4300, ulp 1) is an exact bf16 integer: 128 + q for a code at bits
// 0..2 of its half, 128 + 8q for one at bits 3..5 (pairs with P % 5 == 1 or 3
// are used unshifted).  The activations at the 8q positions are staged
// divided by 8, so every product is (128 + m q) * (x / m), exact, and the
// MFMA sum over a group is sum(q x) + 128 * sum(x / m).

// Masks of the code pairs at bits 0..2 / 16..18 and 3..5 / 19..21 in VGPRs
// and the magic in an SGPR, as values the compiler cannot see through: with a
// literal mask and a literal magic it splits every (d & m) | magic into two
// instructions (a VOP3 encoding holds no literal here), with these it emits
// one v_and_or_b32.  (Writing v_and_or_b32 as inline assembly instead would
// hide a VALU write from the hazard checks, and an MFMA reading its result
// needs wait states the compiler then does not insert.)
struct Q3Masks { uint32_t m7, m38, magic; };

__device__ __forceinline__ Q3Masks q3_masks() {
  Q3Masks k;
  asm volatile("v_mov_b32 %0, 0x70007" : "=v"(k.m7));
  asm volatile("v_mov_b32 %0, 0x380038" : "=v"(k.m38));
  asm volatile("s_mov_b32 %0, 0x43004300" : "=s"(k.magic));
  return k;
}

template <int P>
__device__ __forceinline__ uint32_t q3m_pair(const uint32_t (&w)[3], const Q3Masks& k) {
  if constexpr (P < 15) {
    constexpr int s = P % 5;
    const uint32_t d = w[P / 5];
    if constexpr (s == 0) return (d & k.m7) | k.magic;
    else if constexpr (s == 1) return (d & k.m38) | k.magic;
    else if constexpr (s == 2) return ((d >> 6) & k.m7) | k.magic;
    else if constexpr (s == 3) return ((d >> 6) & k.m38) | k.magic;
    else return ((d >> 12) & k.m7) | k.magic;
  } else {
    // bit t of pair 15's codes is bit 15 / 31 of word t
    const uint32_t a = w[0] >> 15, b = w[1] >> 14, c = w[2] >> 13;
    const uint32_t ab = (a & 0x00010001u) | (b & ~0x00010001u);
    const uint32_t abc = (ab & 0x00030003u) | (c & ~0x00030003u);
    return (abc & k.m7) | k.magic;
  }
}

// MFMA step m's operand (pairs 4m .. 4m+3) of a lane's 32 codes.
template <int M>
__device__ __forceinline__ bf16x8 q3m_operand(const uint32_t (&w)[3], const Q3Masks& k) {
  return as_bf16x8(u32x4{q3m_pair<4 * M>(w, k), q3m_pair<4 * M + 1>(w, k), q3m_pair<4 * M + 2>(w, k),
                         q3m_pair<4 * M + 3>(w, k)});
}

// Bit i set: pair 4m + i of MFMA step m comes out as 128 + 8q (its two
// activations are staged divided by 8).  Steps 0..3: pairs {1,3}, {6}, {8,11}, {13}.
__device__ __forceinline__ uint32_t q3m_div8_pairs(int m) { return (0x294Au >> (4 * m)) & 0xFu; }

// Half h of a packed fp16 pair as float (folds into v_fma_mix_f32).
template <int H>
__device__ __forceinline__ float f16_half(uint32_t v) {
  return static_cast<float>(__builtin_bit_cast(f16x2, v)[H]);
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

__device__ __forceinline__ void load_raw_nc(RawQ3& r, const uint8_t* W, const uint16_t* S, const uint16_t* B,
                                            int64_t row, int K, int kc) {
  const auto src = gptr<uint32_t>(W + row * (K / 8 * 3) + q3_chunk_offset(K, kc >> 7, (kc >> 5) & 3));
  r.w[0] = src[0]; r.w[1] = src[1]; r.w[2] = src[2];
  const int64_t gi = row * (K / 64) + kc / 64;
  r.s = ldg<uint16_t>(S + gi);
  r.b = ldg<uint16_t>(B + gi);
}

__device__ __forceinline__ void load_role_nc(RawFP4& r, const void* const* ptr, int role, int64_t row, int K,
                                             int kc) {
  load_raw_nc(r, static_cast<const uint8_t*>(ptr[3 * role]), static_cast<const uint8_t*>(ptr[3 * role + 1]),
              row, K, kc);
}
__device__ __forceinline__ void load_role_nc(RawQ3& r, const void* const* ptr, int role, int64_t row, int K,
                                             int kc) {
  load_raw_nc(r, static_cast<const uint8_t*>(ptr[3 * role]), static_cast<const uint16_t*>(ptr[3 * role + 1]),
              static_cast<const uint16_t*>(ptr[3 * role + 2]), row, K, kc);
}

// Pointer i of slot u's descriptor (u wave-uniform) through the constant
// address space, i.e. a scalar load: the descriptors are written by an earlier
// kernel and only read here (the scalar cache starts empty at every launch).
// A vector load of a pointer would wait behind the weight loads already in
// flight before the next batch could be addressed.
__device__ __forceinline__ const void* desc_ptr(const SlotDesc* desc, int u, int i) {
  return ((const __attribute__((address_space(4))) SlotDesc*)desc)[u].p[i];
}

// Role 2 (w2) of slot u without conditions (see load_raw_nc).
__device__ __forceinline__ void load_w2_nc(RawFP4& r, const SlotDesc* desc, int u, int64_t row, int K, int kc) {
  load_raw_nc(r, static_cast<const uint8_t*>(desc_ptr(desc, u, 6)), static_cast<const uint8_t*>(desc_ptr(desc, u, 7)),
              row, K, kc);
}
__device__ __forceinline__ void load_w2_nc(RawQ3& r, const SlotDesc* desc, int u, int64_t row, int K, int kc) {
  load_raw_nc(r, static_cast<const uint8_t*>(desc_ptr(desc, u, 6)), static_cast<const uint16_t*>(desc_ptr(desc, u, 7)),
              static_cast<const uint16_t*>(desc_ptr(desc, u, 8)), row, K, kc);
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

// Eight 16-bit values as one 128-bit word.
__device__ __forceinline__ u32x4 pack_bf16x8(const uint16_t* v) {
  return u32x4{v[0] | (uint32_t(v[1]) << 16), v[2] | (uint32_t(v[3]) << 16),
               v[4] | (uint32_t(v[5]) << 16), v[6] | (uint32_t(v[7]) << 16)};
}

// Tokens of the factored q3 gate/up (A operand row 2t + h for t < 8).
constexpr int kQ3fMaxTokens = 8;

// One activation chunk (8 values, chunk cc of its row) for the factored q3
// product: the values at 8q code positions divided by 8 (exact), as bf16
// plane(s) hp (and lp), and the chunk's sum(x) and sum(x / m) reduced over the
// 8 lanes of its 64-group in a fixed order.  All lanes of an aligned 8-lane
// group call it together.
template <bool kF32>
__device__ __forceinline__ void q3_chunk(int cc, const u32x4& v0, const u32x4& v1, u32x4& hp, u32x4& lp,
                                         float& sx, float& sxm) {
  const uint32_t div8 = q3m_div8_pairs(cc & 3);
  float f[8];
  if constexpr (!kF32) {
    const uint32_t w[4] = {v0.x, v0.y, v0.z, v0.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
    const uint32_t w[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = __uint_as_float(w[i]);
  }
  uint16_t h[8], l[8];
  sx = 0.0f;
  sxm = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const bool d8 = (div8 >> (e >> 1)) & 1u;
    const float sc = d8 ? 0.125f : 1.0f, m = d8 ? 8.0f : 1.0f;
    if constexpr (!kF32) {
      h[e] = f32_to_bf16_bits(f[e] * sc);
      sx += f[e];
      sxm += f[e] * sc;
    } else {
      split_bf16(f[e] * sc, h[e], l[e]);
      const float v = bf16_bits_to_f32(h[e]) + bf16_bits_to_f32(l[e]);   // what the MFMA sees
      sx += v * m;
      sxm += v;
    }
  }
  hp = pack_bf16x8(h);
  if constexpr (kF32) lp = pack_bf16x8(l);
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) {
    sx += __shfl_xor(sx, o, 8);
    sxm += __shfl_xor(sxm, o, 8);
  }
}

// x for the factored q3 gate/up, chunk c of the T x H bf16 rows (every lane of
// an aligned 8-lane group takes part; `store` false: the lane only adds to the
// group's sums): the values at 8q code positions divided by 8 as bf16 [T][H]
// (xq) and every 64-group's {sum x, sum x / m} [T][H/64] (xg), as q3_chunk
// makes them.
__device__ __forceinline__ void x_q3_chunk(const uint16_t* x, int H, int c, bool store, uint16_t* xq, float* xg) {
  const int cpr = H / 8;
  const int t = c / cpr, cc = c - t * cpr;
  const int64_t o = static_cast<int64_t>(t) * H + cc * 8;
  u32x4 hp, lp;
  float sx, sxm;
  q3_chunk<false>(cc, ldg16(x + o), u32x4{}, hp, lp, sx, sxm);
  if (store) {
    *reinterpret_cast<u32x4*>(xq + o) = hp;
    if ((cc & 7) == 0) *reinterpret_cast<float2*>(xg + (static_cast<int64_t>(t) * (H / 64) + (cc >> 3)) * 2) = float2{sx, sxm};
  }
}

// q3_chunk of chunk cc of token t's row, staged: the plane(s) at row t of xh
// (xl), stride xs, and the group sums at xsum[kb][t][h] = {sum x, sum x / m}.
template <bool kF32>
__device__ __forceinline__ void stage_chunk_q3(uint16_t* xh, uint16_t* xl, float* xsum, int xs, int cpr, int c,
                                               const u32x4& v0, const u32x4& v1) {
  const int t = c / cpr, cc = c % cpr;
  u32x4 hp, lp;
  float sx, sxm;
  q3_chunk<kF32>(cc, v0, v1, hp, lp, sx, sxm);
  const int off = t * xs + cc * 8;
  *reinterpret_cast<u32x4*>(xh + off) = hp;
  if constexpr (kF32) *reinterpret_cast<u32x4*>(xl + off) = lp;
  if ((cc & 7) == 0) {
    const int gi = cc >> 3;
    *reinterpret_cast<float2*>(xsum + (((gi >> 1) * kQ3fMaxTokens + t) * 2 + (gi & 1)) * 2) = float2{sx, sxm};
  }
}

// One batch of G K blocks of a wave's q3 gate and up rows: three code words
// per lane, block and role, and the (scale, bias) pairs of the block's two
// 64-groups per role (sb: S1, B1, S3, B3; low half = first group).
template <int G>
struct Q3Batch {
  uint32_t c1[G][3], c3[G][3];
  uint32_t sb[4][G];
};

// acc[t] += s * (d - 128 * sum(x / m)) + b * sum(x) over the block's two
// groups h = 0, 1: d[2t' + h] is the MFMA output of token row 2t' + h of this
// lane, xa / xb = xsum of its two tokens {sum x, sum x / m} x {h = 0, 1}.
__device__ __forceinline__ void q3_factor(const f32x4& d, uint32_t s, uint32_t b, const f32x4& xa,
                                          const f32x4& xb, float (&acc)[2]) {
  acc[0] = fmaf(f16_half<0>(s), fmaf(-128.0f, xa.y, d[0]), acc[0]);
  acc[0] = fmaf(f16_half<0>(b), xa.x, acc[0]);
  acc[0] = fmaf(f16_half<1>(s), fmaf(-128.0f, xa.w, d[1]), acc[0]);
  acc[0] = fmaf(f16_half<1>(b), xa.z, acc[0]);
  acc[1] = fmaf(f16_half<0>(s), fmaf(-128.0f, xb.y, d[2]), acc[1]);
  acc[1] = fmaf(f16_half<0>(b), xb.x, acc[1]);
  acc[1] = fmaf(f16_half<1>(s), fmaf(-128.0f, xb.w, d[3]), acc[1]);
  acc[1] = fmaf(f16_half<1>(b), xb.z, acc[1]);
}


}  // namespace dsk
