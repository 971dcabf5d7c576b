// RMSNorm with the residual add of a layer stack.
//
// Replaces rmsnorm (src/deepseeker/mlx_forward.py:45-59) on the residual
// stream of a stack of MoE layers: h = x (+ residual, rounded to the stream's
// dtype), y = h / sqrt(mean(h^2) + eps) * gamma.  For bf16 streams the
// reference's explicit form is followed: everything in float32, one rounding
// of y to bf16 (and one of h when a residual is added).  One block per row;
// the sum of squares is accumulated per thread over a strided slice, then
// across the block in a fixed order, so results are deterministic.
#include "dsk_internal.h"

namespace dsk {
namespace {

constexpr int kNormThreads = 256;

template <bool kBF16>
__device__ __forceinline__ f32x4 ld4(const void* p, int64_t i) {
  if constexpr (kBF16) {
    const uint2 r = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
    return f32x4{__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u), __uint_as_float(r.y << 16),
                  __uint_as_float(r.y & 0xffff0000u)};
  } else {
    return *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i);
  }
}

template <bool kBF16>
__device__ __forceinline__ void st4(void* p, int64_t i, const f32x4& v) {
  if constexpr (kBF16) {
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + i) =
        uint2{f32_to_bf16_bits(v[0]) | (uint32_t(f32_to_bf16_bits(v[1])) << 16),
              f32_to_bf16_bits(v[2]) | (uint32_t(f32_to_bf16_bits(v[3])) << 16)};
  } else {
    *reinterpret_cast<f32x4*>(static_cast<float*>(p) + i) = v;
  }
}

// Round a float32 value to the stream's dtype and back.
template <bool kBF16>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (kBF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  return v;
}

// Row r: h = x[r] (+ res[r]); h_out[r] = h (if given; may be x itself);
// y[r] = rmsnorm(h) (if given).  H % 4 == 0; thread t handles the 4-element
// chunks t, t + 256, ... in both passes, so an in-place h_out is re-read by
// the thread that wrote it.
template <bool kBF16>
__global__ __launch_bounds__(kNormThreads) void k_rmsnorm(const void* x, const void* res,
                                                          const float* __restrict__ gamma, int H, float eps,
                                                          void* h_out, void* __restrict__ y) {
#pragma clang fp contract(off)
  __shared__ float wsum[kNormThreads / 64];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nch = H / 4;
  float ss = 0.0f;
  for (int c = tid; c < nch; c += kNormThreads) {
    f32x4 h = ld4<kBF16>(x, base + 4 * c);
    if (res) {
      const f32x4 r = ld4<kBF16>(res, base + 4 * c);
#pragma unroll
      for (int q = 0; q < 4; ++q) h[q] = round_to<kBF16>(h[q] + r[q]);
      if (h_out) st4<kBF16>(h_out, base + 4 * c, h);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) ss = ss + h[q] * h[q];
  }
  if (!y) return;
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) ss = ss + __shfl_xor(ss, s, 64);
  if (lane == 0) wsum[wave] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < kNormThreads / 64; ++w) tot = tot + wsum[w];
  const float rstd = 1.0f / sqrtf(tot / static_cast<float>(H) + eps);
  for (int c = tid; c < nch; c += kNormThreads) {
    f32x4 h;
    if (res && h_out) {
      h = ld4<kBF16>(h_out, base + 4 * c);
    } else {
      h = ld4<kBF16>(x, base + 4 * c);
      if (res) {
        const f32x4 r = ld4<kBF16>(res, base + 4 * c);
#pragma unroll
        for (int q = 0; q < 4; ++q) h[q] = round_to<kBF16>(h[q] + r[q]);
      }
    }
    const f32x4 g = gamma ? *reinterpret_cast<const f32x4*>(gamma + 4 * c) : f32x4{1.f, 1.f, 1.f, 1.f};
    f32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = (h[q] * rstd) * g[q];
    st4<kBF16>(y, base + 4 * c, o);
  }
}

}  // namespace

hipError_t launch_rmsnorm(const void* x, const void* res, const float* gamma, int64_t rows, int H, float eps,
                          int dtype, void* h_out, void* y, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (dtype == DSK_DTYPE_BF16)
    launch_kernel(k_rmsnorm<true>, static_cast<unsigned>(rows), kNormThreads, 0, s, x, res, gamma, H, eps, h_out, y);
  else
    launch_kernel(k_rmsnorm<false>, static_cast<unsigned>(rows), kNormThreads, 0, s, x, res, gamma, H, eps, h_out, y);
  return hipGetLastError();
}

}  // namespace dsk
