// Router: gate logits, scores and biased top-k with normalised weights.
//
// Replaces the reference's sqrtsoftplus_scores and route_topk
// (src/deepseeker/mlx_forward.py:62-81).  Indices must be bit-identical to
// the CPU oracle, so every floating-point step follows one defined order
// (this file is compiled without contraction, and the pragma below makes that
// explicit):
//   logit  z[t,e]: lane l of a wave keeps a float32 partial that adds, for
//          m = 0, 1, ... and v = 0..3, the rounded product
//          x[256m+4l+v] * W[e][256m+4l+v]; the 64 partials are combined by an
//          XOR butterfly (s = 32, 16, ..., 1: p[l] = p[l] + p[l^s]).
//   score  in double with this file's own exp (Cody-Waite ln2 split, degree-14
//          Taylor in Horner form) and log1p (2*atanh(u/(2+u)), odd series),
//          rounded once to float; sqrt-softplus takes the correctly rounded
//          float sqrt found by exact midpoint tests.
//   top-k  key = (s + bias) + 0; k largest keys, descending, ties to the
//          lower expert id (64-bit composite of order-preserving key bits and
//          the inverted id, reduced across the wave).
//   weight w_j = (s_j / (((s_0 + s_1) + ...) + 1e-20f)) * route_scale.
#include "dsk_internal.h"

#pragma clang fp contract(off)

namespace dsk {
namespace {

// ln2 split: LN2_HI keeps 32 significant bits, so k*LN2_HI is exact for |k| < 2^21.
constexpr double kLn2Hi = 0x1.62e42fee00000p-1;
constexpr double kLn2Lo = 0x1.a39ef35793c76p-33;
constexpr double kLog2e = 0x1.71547652b82fep+0;
// 1/n!, n = 0..14
constexpr double kExpCoef[15] = {
    0x1.0000000000000p+0, 0x1.0000000000000p+0, 0x1.0000000000000p-1, 0x1.5555555555555p-3,
    0x1.5555555555555p-5, 0x1.1111111111111p-7, 0x1.6c16c16c16c17p-10, 0x1.a01a01a01a01ap-13,
    0x1.a01a01a01a01ap-16, 0x1.71de3a556c734p-19, 0x1.27e4fb7789f5cp-22, 0x1.ae64567f544e4p-26,
    0x1.1eed8eff8d898p-29, 0x1.6124613a86d09p-33, 0x1.93974a8c07c9dp-37};
// 1/(2n+1), n = 0..18
constexpr double kAtanhCoef[19] = {
    0x1.0000000000000p+0, 0x1.5555555555555p-2, 0x1.999999999999ap-3, 0x1.2492492492492p-3,
    0x1.c71c71c71c71cp-4, 0x1.745d1745d1746p-4, 0x1.3b13b13b13b14p-4, 0x1.1111111111111p-4,
    0x1.e1e1e1e1e1e1ep-5, 0x1.af286bca1af28p-5, 0x1.8618618618618p-5, 0x1.642c8590b2164p-5,
    0x1.47ae147ae147bp-5, 0x1.2f684bda12f68p-5, 0x1.1a7b9611a7b96p-5, 0x1.0842108421084p-5,
    0x1.f07c1f07c1f08p-6, 0x1.d41d41d41d41dp-6, 0x1.bacf914c1bad0p-6};
constexpr double kSigmoidClamp = 200.0;
constexpr double kSoftplusTail = 1000.0;

__device__ __forceinline__ double exp_d(double x) {
  double k = rint(x * kLog2e);
  double r = (x - k * kLn2Hi) - k * kLn2Lo;
  double p = kExpCoef[14];
#pragma unroll
  for (int n = 13; n >= 0; --n) p = p * r + kExpCoef[n];
  return ldexp(p, static_cast<int>(k));
}

__device__ __forceinline__ double log1p_d(double u) {
  double s = u / (2.0 + u);
  double s2 = s * s;
  double p = kAtanhCoef[18];
#pragma unroll
  for (int n = 17; n >= 0; --n) p = p * s2 + kAtanhCoef[n];
  return 2.0 * (s * p);
}

// Correctly rounded float sqrt of v >= 0 (round half to even).
__device__ __forceinline__ float sqrt_round_f32(double v) {
  float r = static_cast<float>(sqrt(v));
  double rd = r;
  float dn = nextafterf(r, 0.0f);
  float up = nextafterf(r, __builtin_inff());
  double lo = (rd + static_cast<double>(dn)) * 0.5;
  double hi = (rd + static_cast<double>(up)) * 0.5;
  double lo2 = lo * lo, hi2 = hi * hi;
  bool even = (__float_as_uint(r) & 1u) == 0u;
  if (r > 0.0f && (v < lo2 || (v == lo2 && !even))) return dn;
  if (v > hi2 || (v == hi2 && !even)) return up;
  return r;
}

__device__ __forceinline__ float score_of(float z, int score_func) {
  double zd = z;
  if (score_func == DSK_SCORE_SIGMOID) {
    double zc = fmin(fmax(zd, -kSigmoidClamp), kSigmoidClamp);
    return static_cast<float>(1.0 / (1.0 + exp_d(-zc)));
  }
  double a = fabs(zd);
  double u = (a > kSoftplusTail) ? 0.0 : exp_d(-fmin(a, kSoftplusTail));
  double sp = fmax(zd, 0.0) + log1p_d(u);
  return sqrt_round_f32(sp);
}

template <bool kBF16>
__device__ __forceinline__ f32x4 load4(const void* base, int64_t elem) {
  if constexpr (kBF16) {
    uint2 raw = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + elem);
    return f32x4{__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                 __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u)};
  } else {
    return *reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + elem);
  }
}

// One wave computes a TW x EW tile of logits (tokens x experts) and their
// scores.  Block = 4 waves.
template <int TW, int EW, bool kXBF16, bool kWBF16>
__global__ __launch_bounds__(256) void k_gate(const void* __restrict__ x,
                                              const void* __restrict__ gw, int T, int H,
                                              int E, int score_func, float* __restrict__ scores) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int n_et = (E + EW - 1) / EW;
  const int et = wave % n_et, tt = wave / n_et;
  const int t0 = tt * TW, e0 = et * EW;
  if (t0 >= T) return;
  float p[TW][EW];
#pragma unroll
  for (int i = 0; i < TW; ++i)
#pragma unroll
    for (int j = 0; j < EW; ++j) p[i][j] = 0.0f;
  const int steps = (H + 255) / 256;
#pragma unroll 4
  for (int m = 0; m < steps; ++m) {
    const int c = 256 * m + 4 * lane;
    const bool ok = c < H;
    f32x4 xv[TW], wv[EW];
#pragma unroll
    for (int i = 0; i < TW; ++i) {
      const int t = min(t0 + i, T - 1);
      xv[i] = ok ? load4<kXBF16>(x, static_cast<int64_t>(t) * H + c) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < EW; ++j) {
      const int e = min(e0 + j, E - 1);
      wv[j] = ok ? load4<kWBF16>(gw, static_cast<int64_t>(e) * H + c) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
      for (int i = 0; i < TW; ++i)
#pragma unroll
        for (int j = 0; j < EW; ++j) {
          float prod = xv[i][v] * wv[j][v];
          p[i][j] = p[i][j] + prod;
        }
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1)
#pragma unroll
    for (int i = 0; i < TW; ++i)
#pragma unroll
      for (int j = 0; j < EW; ++j) p[i][j] = p[i][j] + __shfl_xor(p[i][j], s, 64);
  // Lane i*EW + j scores pair (i, j): all lanes hold the same sums.
#pragma unroll
  for (int i = 0; i < TW; ++i)
#pragma unroll
    for (int j = 0; j < EW; ++j) {
      if (lane == i * EW + j) {
        const int t = t0 + i, e = e0 + j;
        if (t < T && e < E) scores[static_cast<int64_t>(t) * E + e] = score_of(p[i][j], score_func);
      }
    }
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
    uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), s, 64);
    uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), s, 64);
    uint64_t o = (static_cast<uint64_t>(hi) << 32) | lo;
    v = o > v ? o : v;
  }
  return v;
}

constexpr int kMaxSlots = 16;  // E <= 1024

// One wave per token: biased top-k + normalised weights.
__global__ __launch_bounds__(256) void k_topk(const float* __restrict__ scores,
                                              const float* __restrict__ bias, int T, int E,
                                              int k, float route_scale,
                                              int32_t* __restrict__ idx,
                                              float* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* srow = scores + static_cast<int64_t>(t) * E;
  // ord[i]: order-preserving bits of the key of expert lane + 64*i; 0 = taken or absent.
  uint32_t ord[kMaxSlots];
#pragma unroll
  for (int i = 0; i < kMaxSlots; ++i) {
    const int e = lane + 64 * i;
    uint32_t o = 0u;
    if (e < E) {
      const float key = (srow[e] + bias[e]) + 0.0f;
      const uint32_t u = __float_as_uint(key);
      o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    }
    ord[i] = o;
  }
  // Lane j keeps the j-th selected expert.
  int my_e = 0;
  for (int j = 0; j < k; ++j) {
    uint32_t bk = 0u;
    int bi = 0;
#pragma unroll
    for (int i = 0; i < kMaxSlots; ++i)
      if (ord[i] > bk) { bk = ord[i]; bi = i; }      // first maximum = lowest id
    const uint64_t mine = bk ? ((static_cast<uint64_t>(bk) << 32) |
                                static_cast<uint32_t>(~static_cast<uint32_t>(lane + 64 * bi)))
                             : 0ull;
    const uint64_t best = wave_max_u64(mine);
    const int e = static_cast<int>(~static_cast<uint32_t>(best));
    if (lane == j) my_e = e;
    if ((e & 63) == lane) {
#pragma unroll
      for (int i = 0; i < kMaxSlots; ++i)
        if (i == (e >> 6)) ord[i] = 0u;
    }
  }
  // my_e < 0 only if a key has the bit pattern of -NaN with all payload bits set.
  const float my_s = (lane < k && my_e >= 0) ? srow[my_e] : 0.0f;
  // Every lane forms the same sum, in selection order.
  float acc = 0.0f;
  for (int j = 0; j < k; ++j) acc = acc + __shfl(my_s, j, 64);
  const float denom = acc + 1e-20f;
  if (lane < k) {
    idx[static_cast<int64_t>(t) * k + lane] = my_e;
    weights[static_cast<int64_t>(t) * k + lane] = (my_s / denom) * route_scale;
  }
}

template <int TW, int EW>
hipError_t launch_gate_tile(const dsk_moe_desc& d, const void* x, const void* gw, float* scores,
                            hipStream_t s) {
  const int n_et = (d.n_experts + EW - 1) / EW;
  const int n_tt = (d.tokens + TW - 1) / TW;
  const int64_t waves = static_cast<int64_t>(n_et) * n_tt;
  const unsigned blocks = static_cast<unsigned>((waves + 3) / 4);
  const bool xb = d.x_dtype == DSK_DTYPE_BF16, wb = d.gate_dtype == DSK_DTYPE_BF16;
#define DSK_GATE(XB, WB)                                                                      \
  k_gate<TW, EW, XB, WB><<<blocks, 256, 0, s>>>(x, gw, d.tokens, d.hidden, d.n_experts, \
                                                   d.score_func, scores)
  if (xb && wb) DSK_GATE(true, true);
  else if (xb) DSK_GATE(true, false);
  else if (wb) DSK_GATE(false, true);
  else DSK_GATE(false, false);
#undef DSK_GATE
  return hipGetLastError();
}

}  // namespace

hipError_t launch_route(const dsk_moe_desc& d, const void* x, const void* gate_w,
                        const float* gate_b, float* scores, int32_t* idx, float* weights,
                        hipStream_t s) {
  hipError_t e = (d.tokens >= 16) ? launch_gate_tile<4, 4>(d, x, gate_w, scores, s)
                                  : launch_gate_tile<1, 1>(d, x, gate_w, scores, s);
  if (e != hipSuccess) return e;
  const unsigned blocks = static_cast<unsigned>((d.tokens + 3) / 4);
  k_topk<<<blocks, 256, 0, s>>>(scores, gate_b, d.tokens, d.n_experts, d.top_k,
                                d.route_scale, idx, weights);
  return hipGetLastError();
}

}  // namespace dsk
