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
// rows up to 4096 / 8192 wide are held in registers (4 / 8 chunks per thread)

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
// the thread that wrote it.  With NC > 0 (rows up to NC * 1024 wide) the row
// stays in registers: one round of loads instead of one per chunk (the loop
// form's loads cannot pass the store to h_out, which may be x); chunks past
// the row re-read the last one and add exact zeros to the (non-negative) sum.
template <bool kBF16, bool kRes, bool kGamma, int NC>
__global__ __launch_bounds__(kNormThreads) void k_rmsnorm(const void* x, const void* res,
                                                          const float* __restrict__ gamma, int H, float eps,
                                                          void* h_out, void* __restrict__ y) {
#pragma clang fp contract(off)
  __shared__ float wsum[kNormThreads / 64];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nch = H / 4;
  if constexpr (NC > 0) {
    // the row in registers: every load (x, residual, gamma) issued before the
    // first use, then the same sums in the same order as the loop form below
    f32x4 h[NC], r[NC], g[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = min(tid + i * kNormThreads, nch - 1);   // no condition on the loads
      h[i] = ld4<kBF16>(x, base + 4 * c);
      if constexpr (kRes) r[i] = ld4<kBF16>(res, base + 4 * c);
      if constexpr (kGamma) g[i] = *reinterpret_cast<const f32x4*>(gamma + 4 * c);
      else g[i] = f32x4{1.f, 1.f, 1.f, 1.f};
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = tid + i * kNormThreads;
      const bool v = c < nch;
      if constexpr (kRes) {
#pragma unroll
        for (int q = 0; q < 4; ++q) h[i][q] = round_to<kBF16>(h[i][q] + r[i][q]);
        if (h_out && v) st4<kBF16>(h_out, base + 4 * c, h[i]);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) ss = ss + (v ? h[i][q] * h[i][q] : 0.0f);
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
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = tid + i * kNormThreads;
      if (c < nch) {
        f32x4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = (h[i][q] * rstd) * g[i][q];
        st4<kBF16>(y, base + 4 * c, o);
      }
    }
    return;
  } else {
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
}

template <bool kBF16, int NC>
void launch_rmsnorm_nc(const void* x, const void* res, const float* gamma, int64_t rows, int H, float eps,
                       void* h_out, void* y, hipStream_t s) {
  const unsigned b = static_cast<unsigned>(rows);
  if (res && gamma) launch_kernel(k_rmsnorm<kBF16, true, true, NC>, b, kNormThreads, 0, s, x, res, gamma, H, eps, h_out, y);
  else if (res) launch_kernel(k_rmsnorm<kBF16, true, false, NC>, b, kNormThreads, 0, s, x, res, gamma, H, eps, h_out, y);
  else if (gamma) launch_kernel(k_rmsnorm<kBF16, false, true, NC>, b, kNormThreads, 0, s, x, res, gamma, H, eps, h_out, y);
  else launch_kernel(k_rmsnorm<kBF16, false, false, NC>, b, kNormThreads, 0, s, x, res, gamma, H, eps, h_out, y);
}

template <bool kBF16>
void launch_rmsnorm_t(const void* x, const void* res, const float* gamma, int64_t rows, int H, float eps,
                      void* h_out, void* y, hipStream_t s) {
  const int nch = H / 4;
  if (nch <= 4 * kNormThreads) launch_rmsnorm_nc<kBF16, 4>(x, res, gamma, rows, H, eps, h_out, y, s);
  else if (nch <= 8 * kNormThreads) launch_rmsnorm_nc<kBF16, 8>(x, res, gamma, rows, H, eps, h_out, y, s);
  else launch_rmsnorm_nc<kBF16, 0>(x, res, gamma, rows, H, eps, h_out, y, s);
}

}  // namespace

hipError_t launch_rmsnorm(const void* x, const void* res, const float* gamma, int64_t rows, int H, float eps,
                          int dtype, void* h_out, void* y, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (dtype == DSK_DTYPE_BF16) launch_rmsnorm_t<true>(x, res, gamma, rows, H, eps, h_out, y, s);
  else launch_rmsnorm_t<false>(x, res, gamma, rows, H, eps, h_out, y, s);
  return hipGetLastError();
}

}  // namespace dsk
