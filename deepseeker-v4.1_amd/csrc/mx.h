// MX products on gfx950: v_mfma_scale_f32_16x16x128_f8f6f4 with the FP4 (e2m1)
// weights as the A operand exactly as the expert kernels load them, and the
// activations as the B operand in FP8 (OCP e4m3) planes with E8M0 scales.
//
// Operand layout of one 16 x 16 x 128 product (measured on the part):
//   A (FP4): lane l holds row l & 15, codes [32g, 32g + 32) of the 128-code K
//            block (g = l >> 4), low nibble first -- one 16-byte word of a
//            weight row -- and the row's E8M0 byte for those 32 codes.
//   B (FP8): lane l holds column l & 15 at K [16g, 16g + 16) in bytes 0..15 and
//            [64 + 16g, 64 + 16g + 16) in bytes 16..31, and the E8M0 byte of
//            (column l & 15, K group [32g, 32g + 32)).
//   C:       as v_mfma_f32_16x16x32_bf16 -- lane l holds rows 4g .. 4g + 3 of
//            column l & 15.
// One product covers a whole 128-code block (the bf16 path needs four
// v_mfma_f32_16x16x32_bf16 and sixteen FP4 -> bf16 conversions per lane).  The
// part sums the block's products with less than float32 precision (about
// 2^-14 of the sum of the terms' magnitudes), which the layer tolerance
// absorbs.
//
// FP8 planes: a float32 value v of a 32-element group is written as
// v ~ q0 * 2^e + q1 * 2^(e-4) + q2 * 2^(e-8) (q FP8, round to nearest even),
// e = ilogb(max |v| of the group) - 7, so max |v| / 2^e < 256 stays inside
// e4m3's range (448; larger values become NaN, not saturated) and each plane
// takes the rounding error of the previous one (at most 2^-4 of the value, so
// at most 128 in the next plane's units).  Two planes hold a bf16 value exactly
// when it lies within 2^13 of the group's largest (its 8 significant bits);
// three planes leave an error below 2^-14 of the group's largest magnitude.
#pragma once

#include "tile.h"

namespace dsk {

typedef int32_t i32x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mx_mfma(const u32x4& a_codes, uint32_t a_scale, const u32x4& b_lo,
                                         const u32x4& b_hi, uint32_t b_scale, const f32x4& c) {
  const i32x8 a = {static_cast<int32_t>(a_codes.x), static_cast<int32_t>(a_codes.y),
                   static_cast<int32_t>(a_codes.z), static_cast<int32_t>(a_codes.w), 0, 0, 0, 0};
  const i32x8 b = {static_cast<int32_t>(b_lo.x), static_cast<int32_t>(b_lo.y), static_cast<int32_t>(b_lo.z),
                   static_cast<int32_t>(b_lo.w), static_cast<int32_t>(b_hi.x), static_cast<int32_t>(b_hi.y),
                   static_cast<int32_t>(b_hi.z), static_cast<int32_t>(b_hi.w)};
  // cbsz 4: A is FP4 (e2m1); blgp 0: B is FP8 (e4m3); scale bytes from bits 0..7
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 4, 0, 0, static_cast<int>(a_scale), 0,
                                                          static_cast<int>(b_scale));
}

// Exponent e of the first plane of a group whose largest magnitude is m:
// ilogb(m) - 7, at least -118 so that the third plane's scale 2^(e-8) is a
// normal float and an E8M0 byte (groups below 2^-111 lose their low bits).
__device__ __forceinline__ int fp8_plane_exp(float m) {
  const int be = static_cast<int>((__float_as_uint(m) >> 23) & 0xffu);
  return max(be - 127 - 7, -118);
}

// Byte of K index k (0..127 of a K block) in a lane group's 32 B-operand bytes
// laid out lane group by lane group: group (k % 64) / 16, byte 16 (k / 64) + k % 16.
__device__ __forceinline__ int b_perm(int k) { return ((k & 63) >> 4) * 32 + ((k >> 6) << 4) + (k & 15); }

// E8M0 byte of 2^e (e clamped to the byte's range).
__device__ __forceinline__ uint32_t e8m0_byte(int e) {
  const int b = e + 127;
  return static_cast<uint32_t>(b < 0 ? 0 : (b > 254 ? 254 : b));
}

// 2^e as float for e in [-126, 127] (the planes' scales and their inverses
// stay inside it).
__device__ __forceinline__ float pow2f(int e) {
  const int b = e + 127;
  return __uint_as_float(static_cast<uint32_t>(b < 1 ? 1 : (b > 254 ? 254 : b)) << 23);
}

// Value of lane l ^ 1 (DPP quad permutation [1, 0, 3, 2]).
__device__ __forceinline__ float lane_xor1(float v) {
  return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0xB1, 0xF, 0xF, false));
}

// Maximum over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four 16-lane rows; the
// swaps exchange a lane's value with its partner row's, so the larger of the
// two results is the pair's maximum whichever way round they come back).
__device__ __forceinline__ float max_over_rows(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(v, fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1])));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(v, fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1])));
}

// SiLU(min(g, limit)) * clamp(u, -limit, limit) with e^-x = 2^(-x log2 e) on
// the exponential unit and the hardware reciprocal (a few ulp; the FP8 planes
// the result goes into keep 2^-14 of their group's largest value).
__device__ __forceinline__ float silu_clamped_fast(float g, float u, float limit) {
  const float gg = fminf(g, limit);
  const float uu = fminf(fmaxf(u, -limit), limit);
  return gg * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * gg)) * uu;
}

// NP planes of 4 values (one 4-byte word per plane, value q in byte q).
template <int NP>
__device__ __forceinline__ void fp8_planes4(const float (&v)[4], int e, uint32_t (&w)[NP]) {
  float r[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const float inv = pow2f(-(e - 4 * p)), sc = pow2f(e - 4 * p);
    int lo = __builtin_amdgcn_cvt_pk_fp8_f32(r[0] * inv, r[1] * inv, 0, false);
    int both = __builtin_amdgcn_cvt_pk_fp8_f32(r[2] * inv, r[3] * inv, lo, true);
    w[p] = static_cast<uint32_t>(both);
    if (p + 1 < NP) {
      r[0] = r[0] - __builtin_amdgcn_cvt_f32_fp8(both, 0) * sc;
      r[1] = r[1] - __builtin_amdgcn_cvt_f32_fp8(both, 1) * sc;
      r[2] = r[2] - __builtin_amdgcn_cvt_f32_fp8(both, 2) * sc;
      r[3] = r[3] - __builtin_amdgcn_cvt_f32_fp8(both, 3) * sc;
    }
  }
}

// Chunk c (8 values) of x [T][H] bf16 into the two-plane layout of the
// grouped FP4 gate/up: plane row (t, p) holds H bytes, each 128-value block in
// the B-operand byte order (b_perm), then the E8M0 bytes of every (t, p,
// 32-group) after all plane rows.  The four chunks of a 32-group must be in
// four consecutive lanes that all take part (the group maximum is exchanged);
// `store` false: the lane takes part and writes nothing.
__device__ __forceinline__ void x_planes_chunk(const uint16_t* x, int T, int H, int c, bool store, uint8_t* xp) {
  const int cpr = H / 8;
  const int t = c / cpr, k8 = (c % cpr) * 8;
  const u32x4 v = *reinterpret_cast<const u32x4*>(x + static_cast<int64_t>(t) * H + k8);
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
  if (store) {
    const int kb = k8 >> 7, kk = k8 & 127;
    uint8_t* scales = xp + static_cast<size_t>(T) * 2 * H;
#pragma unroll
    for (int pl = 0; pl < 2; ++pl) {
      const size_t prow = static_cast<size_t>(2 * t + pl);
      *reinterpret_cast<uint2*>(xp + prow * H + kb * 128 + b_perm(kk)) = uint2{w0[pl], w1[pl]};
      if ((k8 & 31) == 0) scales[prow * (H / 32) + (k8 >> 5)] = static_cast<uint8_t>(e8m0_byte(e - 4 * pl));
    }
  }
}

// Chunk c (8 values) of x [T][H] bf16 into the prefill MX gate/up's two FP8
// planes in stage rows: row t holds 2H bytes, each 64-value piece as its 64
// plane-0 bytes then its 64 plane-1 bytes (q), and one E8M0 byte per (t,
// 32-group) in ex.  The four chunks of a 32-group must be in four consecutive
// lanes that all take part; `store` false: the lane takes part and writes
// nothing.
__device__ __forceinline__ void pf_planes_chunk(const uint16_t* x, int H, int64_t c, bool store, uint8_t* q,
                                                uint8_t* ex) {
  const int cpr = H / 8;
  const int64_t t = c / cpr;
  const int k8 = static_cast<int>(c - t * cpr) * 8;
  const u32x4 v = *reinterpret_cast<const u32x4*>(x + t * H + k8);
  const float f0[4] = {__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                       __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u)};
  const float f1[4] = {__uint_as_float(v.z << 16), __uint_as_float(v.z & 0xffff0000u),
                       __uint_as_float(v.w << 16), __uint_as_float(v.w & 0xffff0000u)};
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) m = fmaxf(m, fmaxf(fabsf(f0[i]), fabsf(f1[i])));
  m = fmaxf(m, __shfl_xor(m, 1, 64));
  m = fmaxf(m, __shfl_xor(m, 2, 64));
  const int e = fp8_plane_exp(m);
  uint32_t w0[2], w1[2];
  fp8_planes4<2>(f0, e, w0);
  fp8_planes4<2>(f1, e, w1);
  if (!store) return;
  uint8_t* row = q + t * (2 * H) + (k8 >> 6) * 128 + (k8 & 63);
  *reinterpret_cast<uint2*>(row) = uint2{w0[0], w1[0]};
  *reinterpret_cast<uint2*>(row + 64) = uint2{w0[1], w1[1]};
  if ((k8 & 31) == 0) ex[t * (H / 32) + (k8 >> 5)] = static_cast<uint8_t>(e8m0_byte(e));
}

}  // namespace dsk
