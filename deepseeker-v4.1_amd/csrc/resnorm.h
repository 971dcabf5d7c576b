// The residual update and RMSNorm of a layer stack, evaluated inside the
// first kernel of the next layer: every block normalises the token rows it
// needs into LDS, and block 0 also writes the new residual stream and the
// normalised rows for the layer's later kernels.
//
// Replaces, between two MoE layers of the runner's loop
// (src/deepseeker/mlx_runner.py:2138-2145), the residual add and rmsnorm
// (src/deepseeker/mlx_forward.py:45-59) for bf16 streams, bit for bit as
// norm.hip's k_rmsnorm computes them: h = bf16(h_prev + d_prev); lane v of
// 256 adds the squares of the row's 4-element chunks v, v + 256, ... in order
// (product and sum each rounded, no fused multiply-add); an XOR tree per
// 64 lanes; the four wave sums in order; rstd = 1 / sqrt(sum / H + eps);
// y = bf16((h * rstd) * gamma).
//
// The loads are split from the arithmetic (resnorm_issue, then
// resnorm_rows), so that a kernel can issue the rows' loads, then its own
// first weight loads, and only then wait for the rows: the normalisation's
// latency hides under the weight stream's.  Every thread of the block loads
// a share of the rows (chunks tid, tid + B, ... of each of up to two rows),
// writes h to the output rows in LDS, and the sums read them back there in
// the order above; each thread then scales its own chunks in place.
#pragma once

#include "dsk_internal.h"

namespace dsk {

struct ResNorm {
  const uint16_t* h;     // [T][H] bf16 residual stream before the layer
  const uint16_t* d;     // [T][H] bf16 output of the previous layer
  const float* gamma;    // [H] or null (ones)
  float eps;
  uint16_t* h_out;       // [T][H] h + d (not h itself: every block reads h)
  uint16_t* x_out;       // [T][H] the normalised rows, the layer's input
};

__device__ __forceinline__ f32x4 bf16x4_to_f32(uint2 r) {
  return f32x4{__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u), __uint_as_float(r.y << 16),
               __uint_as_float(r.y & 0xffff0000u)};
}
__device__ __forceinline__ uint2 f32x4_to_bf16x4(const f32x4& v) {
  return uint2{f32_to_bf16_bits(v[0]) | (uint32_t(f32_to_bf16_bits(v[1])) << 16),
               f32_to_bf16_bits(v[2]) | (uint32_t(f32_to_bf16_bits(v[3])) << 16)};
}

constexpr int kResNormMaxHidden = 4096;  // row width limit (registers per thread)
constexpr int kResNormLanes = 256;       // lanes of the defined sum order
constexpr int kResNormRows = 2;          // rows (tokens) at most
constexpr int kResNormWsum = 4 * kResNormRows;   // floats of LDS for the wave sums

// One thread's share of the rows (B threads per block), as loaded.
template <int B>
struct ResNormIn {
  static constexpr int NC = kResNormMaxHidden / 4 / B;   // chunks per thread and row
  uint2 h[kResNormRows][NC], d[kResNormRows][NC];
  f32x4 g[NC];
};

// Issues the loads of rows 0 .. T-1, T <= kResNormRows (every load is in
// bounds).
template <int B>
__device__ __forceinline__ void resnorm_issue(const ResNorm r, int T, int H, ResNormIn<B>& in) {
  constexpr int NC = ResNormIn<B>::NC;
  const int tid = threadIdx.x, nch = H / 4;
  // uniform row bases + unsigned lane offsets (one address register per load)
#pragma unroll
  for (int j = 0; j < kResNormRows; ++j) {
    if (j < T) {   // uniform
      const size_t base = static_cast<size_t>(j) * H;
      const uint16_t* hr = r.h + base;
      const uint16_t* dr = r.d + base;
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const unsigned c = static_cast<unsigned>(min(tid + i * B, nch - 1));   // no per-lane condition
        in.h[j][i] = *reinterpret_cast<const uint2*>(hr + 4u * c);
        in.d[j][i] = *reinterpret_cast<const uint2*>(dr + 4u * c);
      }
    }
  }
  if (r.gamma) {
#pragma unroll
    for (int i = 0; i < NC; ++i)
      in.g[i] = *reinterpret_cast<const f32x4*>(r.gamma + 4u * static_cast<unsigned>(min(tid + i * B, nch - 1)));
  } else {
#pragma unroll
    for (int i = 0; i < NC; ++i) in.g[i] = f32x4{1.f, 1.f, 1.f, 1.f};
  }
}

// Rows 0 .. T-1 (T <= kResNormRows: one pass, the loads of which `in` holds
// from resnorm_issue) normalised into y (bf16, row stride ys elements,
// 8-byte aligned); with `write`, h + d and y also go to r.h_out and r.x_out.
// H % 4 == 0, H <= kResNormMaxHidden, B = blockDim.x a multiple of 256.
// Every thread of the block calls it (it holds barriers, the last one after y
// is complete).  wsum: kResNormWsum floats of LDS.
template <int B>
__device__ __forceinline__ void resnorm_rows(const ResNorm r, int T, int H, uint16_t* y, int ys, bool write,
                                             float* wsum, const ResNormIn<B>& in) {
#pragma clang fp contract(off)
  constexpr int NC = ResNormIn<B>::NC, G = B / kResNormLanes;
  constexpr int kLaneChunks = kResNormMaxHidden / 4 / kResNormLanes;
  static_assert(B % kResNormLanes == 0, "whole groups of 256 lanes");
  const int tid = threadIdx.x, lane = tid & 63;
  const int v = tid % kResNormLanes, grp = tid / kResNormLanes;
  const int nch = H / 4;
  // h = bf16(h + d), staged in the output rows
  uint2 hb[kResNormRows][NC];
#pragma unroll
  for (int j = 0; j < kResNormRows; ++j) {
    if (j < T) {
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const f32x4 hv = bf16x4_to_f32(in.h[j][i]), dv = bf16x4_to_f32(in.d[j][i]);
        f32x4 s;
#pragma unroll
        for (int q = 0; q < 4; ++q) s[q] = hv[q] + dv[q];
        hb[j][i] = f32x4_to_bf16x4(s);
        const int c = tid + i * B;
        if (c < nch) *reinterpret_cast<uint2*>(y + j * ys + 4 * c) = hb[j][i];
      }
    }
  }
  __syncthreads();
  // the sums: lane v of row j, for the rows j of this lane group
#pragma unroll
  for (int jj = 0; jj < kResNormRows; jj += G) {
    const int j = jj + grp;
    if (j < T) {
      const uint16_t* yr = y + j * ys;
      float ss = 0.0f;
#pragma unroll
      for (int k = 0; k < kLaneChunks; ++k) {
        const int c = v + k * kResNormLanes;
        if (c < nch) {
          const f32x4 hv = bf16x4_to_f32(*reinterpret_cast<const uint2*>(yr + 4 * c));
#pragma unroll
          for (int q = 0; q < 4; ++q) ss = ss + hv[q] * hv[q];
        }
      }
#pragma unroll
      for (int s = 32; s >= 1; s >>= 1) ss = ss + __shfl_xor(ss, s, 64);
      if (lane == 0) wsum[4 * j + (v >> 6)] = ss;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kResNormRows; ++j) {
    if (j < T) {
      float tot = 0.0f;
#pragma unroll
      for (int w = 0; w < 4; ++w) tot = tot + wsum[4 * j + w];
      const float rstd = 1.0f / sqrtf(tot / static_cast<float>(H) + r.eps);
      const size_t base = static_cast<size_t>(j) * H;
      uint16_t* xr = r.x_out + base;
      uint16_t* hr = r.h_out + base;
      uint16_t* yr = y + j * ys;
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const unsigned c = static_cast<unsigned>(tid + i * B);
        if (c < static_cast<unsigned>(nch)) {
          const f32x4 hv = bf16x4_to_f32(hb[j][i]);
          f32x4 o;
#pragma unroll
          for (int q = 0; q < 4; ++q) o[q] = (hv[q] * rstd) * in.g[i][q];
          const uint2 yb = f32x4_to_bf16x4(o);
          *reinterpret_cast<uint2*>(yr + 4u * c) = yb;
          if (write) {
            *reinterpret_cast<uint2*>(xr + 4u * c) = yb;
            *reinterpret_cast<uint2*>(hr + 4u * c) = hb[j][i];
          }
        }
      }
    }
  }
  __syncthreads();   // y complete
}

}  // namespace dsk
