// Router math shared by the router kernels and the fused decode kernel:
// score functions, gate logits of a tile, biased top-k, arrival counters.
// Every function here evaluates floating point in one fixed order without
// contraction (the pragma opens each body; the gate's fused multiply-adds are
// explicit), because the expert indices must be bit-identical to the CPU
// oracle.  The order is described in route.hip.
#pragma once

#include "dispatch_block.h"

namespace dsk {

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
constexpr int kSegments = 4;         // waves per gate block
constexpr int kMaxSlots = 16;        // E <= 1024 keys per lane in top-k

__device__ __forceinline__ double exp_d(double x) {
#pragma clang fp contract(off)
  double k = rint(x * kLog2e);
  double r = (x - k * kLn2Hi) - k * kLn2Lo;
  double p = kExpCoef[14];
#pragma unroll
  for (int n = 13; n >= 0; --n) p = p * r + kExpCoef[n];
  return ldexp(p, static_cast<int>(k));
}

__device__ __forceinline__ double log1p_d(double u) {
#pragma clang fp contract(off)
  double s = u / (2.0 + u);
  double s2 = s * s;
  double p = kAtanhCoef[18];
#pragma unroll
  for (int n = 17; n >= 0; --n) p = p * s2 + kAtanhCoef[n];
  return 2.0 * (s * p);
}

// Correctly rounded float sqrt of v >= 0 (round half to even).
__device__ __forceinline__ float sqrt_round_f32(double v) {
#pragma clang fp contract(off)
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
#pragma clang fp contract(off)
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

// Four gate operands as loaded (bf16 bits or float) and as floats.
template <bool kBF16> struct GateRaw { using T = f32x4; };
template <> struct GateRaw<true> { using T = uint2; };

template <bool kBF16>
__device__ __forceinline__ typename GateRaw<kBF16>::T load_raw4(const void* base, int64_t elem) {
  if constexpr (kBF16) return *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + elem);
  else return *reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + elem);
}

template <bool kBF16>
__device__ __forceinline__ f32x4 raw4_f32(const typename GateRaw<kBF16>::T& raw) {
  if constexpr (kBF16) {
    return f32x4{__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                 __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u)};
  } else {
    return raw;
  }
}

template <bool kBF16>
__device__ __forceinline__ f32x4 load4(const void* base, int64_t elem) {
  return raw4_f32<kBF16>(load_raw4<kBF16>(base, elem));
}

// Steps (of 256 elements) per load batch of a gate tile.
template <int TW, int EW> constexpr int kGateBatch = TW * EW == 1 ? 4 : 2;

// The first load batch of a gate tile's weights, issued by gate_w_issue
// ahead of work that produces x (gate_tile then takes them from here).
template <int TW, int EW, bool kWBF16>
struct GateWFirst {
  typename GateRaw<kWBF16>::T w[kGateBatch<TW, EW>][EW];
};

// Segment [m0, m1) of wave w in steps of 256 elements.
__device__ __forceinline__ void gate_segment(int H, int wave, bool active, int& m0, int& m1) {
  const int steps = (H + 255) / 256;
  const int seg = (steps + kSegments - 1) / kSegments;
  m0 = wave * seg;
  m1 = active ? min(m0 + seg, steps) : m0;
}

// Element offset of lane's four values in step min(mb, m1 - 1) (clamped to
// the row, so that every load is in bounds; steps past the segment are
// zeroed before the product).
__device__ __forceinline__ int gate_col(int mb, int m1, int lane, int H) {
  return min(256 * max(min(mb, m1 - 1), 0) + 4 * lane, H - 4);
}

template <int TW, int EW, bool kWBF16>
__device__ __forceinline__ void gate_w_issue(const void* gw, int H, int E, int e0, int wave, int lane,
                                             bool active, GateWFirst<TW, EW, kWBF16>& f) {
  int m0, m1;
  gate_segment(H, wave, active, m0, m1);
#pragma unroll
  for (int q = 0; q < kGateBatch<TW, EW>; ++q) {
    const int c = gate_col(m0 + q, m1, lane, H);
#pragma unroll
    for (int j = 0; j < EW; ++j) f.w[q][j] = load_raw4<kWBF16>(gw, static_cast<int64_t>(min(e0 + j, E - 1)) * H + c);
  }
}

// Gate logits and scores of a TW-token x EW-expert tile by 4 waves (wave w
// owns segment w of H; see the order above).  `gtid` is the thread index
// within the 4-wave group; segsum is [4][TW*EW] floats of LDS.  Contains a
// __syncthreads() (reached also when !active: then nothing is loaded or
// written).
template <int TW, int EW, bool kXBF16, bool kWBF16, bool kPre = false>
__device__ __forceinline__ void gate_tile(const void* x, const void* gw, int T, int H, int E,
                                          int score_func, float* scores, int t0, int e0, int wave,
                                          int lane, int gtid, float* segsum, bool active = true,
                                          const GateWFirst<TW, EW, kWBF16>* pre = nullptr) {
#pragma clang fp contract(off)
  float p[TW][EW];
#pragma unroll
  for (int i = 0; i < TW; ++i)
#pragma unroll
    for (int j = 0; j < EW; ++j) p[i][j] = 0.0f;
  int m0, m1;
  gate_segment(H, wave, active, m0, m1);
  // The loads of kC steps are issued together and without conditions (a load
  // under a per-lane condition compiles to a branch whose merge waits for
  // it): out-of-range elements are read from an in-range place and zeroed
  // before the product, and steps past the segment add +0, which leaves a
  // partial that starts at +0 unchanged -- the sums are those of the plain
  // loop, in the same order.  With kPre the first batch's weights were
  // issued earlier (gate_w_issue, same places).
  constexpr int kC = kGateBatch<TW, EW>;
  // x loads and the products of the batch at step mb, weights given
  auto batch = [&](int mb, const f32x4 (&wv)[kC][EW]) {
    f32x4 xv[kC][TW];
#pragma unroll
    for (int q = 0; q < kC; ++q) {
      const int c = gate_col(mb + q, m1, lane, H);
#pragma unroll
      for (int i = 0; i < TW; ++i) xv[q][i] = load4<kXBF16>(x, static_cast<int64_t>(min(t0 + i, T - 1)) * H + c);
    }
#pragma unroll
    for (int q = 0; q < kC; ++q) {
      const bool ok = mb + q < m1 && 256 * (mb + q) + 4 * lane < H;
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int i = 0; i < TW; ++i)
#pragma unroll
          for (int j = 0; j < EW; ++j) {
            p[i][j] = __builtin_fmaf(ok ? xv[q][i][v] : 0.0f, ok ? wv[q][j][v] : 0.0f, p[i][j]);
          }
    }
  };
  int mb = m0;
  if constexpr (kPre) {
    if (mb < m1) {
      f32x4 wv[kC][EW];
#pragma unroll
      for (int q = 0; q < kC; ++q)
#pragma unroll
        for (int j = 0; j < EW; ++j) wv[q][j] = raw4_f32<kWBF16>(pre->w[q][j]);
      batch(mb, wv);
    }
    mb += kC;
  }
  for (; mb < m1; mb += kC) {
    f32x4 wv[kC][EW];
#pragma unroll
    for (int q = 0; q < kC; ++q) {
      const int c = gate_col(mb + q, m1, lane, H);
#pragma unroll
      for (int j = 0; j < EW; ++j) wv[q][j] = load4<kWBF16>(gw, static_cast<int64_t>(min(e0 + j, E - 1)) * H + c);
    }
    batch(mb, wv);
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1)
#pragma unroll
    for (int i = 0; i < TW; ++i)
#pragma unroll
      for (int j = 0; j < EW; ++j) p[i][j] = p[i][j] + __shfl_xor(p[i][j], s, 64);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < TW; ++i)
#pragma unroll
      for (int j = 0; j < EW; ++j) segsum[wave * TW * EW + i * EW + j] = p[i][j];
  }
  __syncthreads();
  if (active && gtid < TW * EW) {
    const int i = gtid / EW, j = gtid % EW;
    const int t = t0 + i, e = e0 + j;
    const float z = ((segsum[gtid] + segsum[TW * EW + gtid]) + segsum[2 * TW * EW + gtid]) +
                    segsum[3 * TW * EW + gtid];
    if (t < T && e < E) scores[static_cast<int64_t>(t) * E + e] = score_of(z, score_func);
  }
}

// One wave: biased top-k and normalised weights of one token.  Lane l holds
// the keys of experts l + 64*i, i < S.  Each round every lane takes its best
// remaining key (lowest id among equal keys), the wave maximum key is found
// with DPP, and among the lanes holding it the lowest expert id wins.
// Results go to idx_row / w_row and to the LDS copies lidx / lw, each pair
// when given (the LDS copies feed the dispatch that follows).
template <int S>
__device__ __forceinline__ void topk_token_s(const float* __restrict__ srow, const float* __restrict__ bias,
                                             int E, int k, float route_scale, int32_t* __restrict__ idx_row,
                                             float* __restrict__ w_row, int32_t* lidx, float* lw) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  // ord[i]: order-preserving bits of the key of expert lane + 64*i; 0 = taken or absent.
  // sv[i]: the score itself, kept for the weights (no second load).
  uint32_t ord[S];
  float sv[S];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    const int e = lane + 64 * i;
    uint32_t o = 0u;
    float s = 0.0f;
    if (e < E) {
      s = srow[e];
      const float key = (s + bias[e]) + 0.0f;
      const uint32_t u = __float_as_uint(key);
      o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    }
    ord[i] = o;
    sv[i] = s;
  }
  int my_e = 0;                         // lane j keeps the j-th selected expert
  float my_s = 0.0f;                    // and its score
  for (int j = 0; j < k; ++j) {
    uint32_t bk = ord[0];
    int bi = 0;
#pragma unroll
    for (int i = 1; i < S; ++i)
      if (ord[i] > bk) { bk = ord[i]; bi = i; }      // first maximum = lowest id
    const uint32_t m = wave_max_u32(bk);
    int e = -1;   // only if every remaining key has the bit pattern of -NaN with all payload bits set
    if (m != 0u) e = static_cast<int>(wave_min_u32(bk == m ? static_cast<uint32_t>(lane + 64 * bi) : ~0u));
    float se = 0.0f;                    // score of expert e (wave-uniform e: a lane read)
    if (e >= 0) {
      float v = sv[0];
#pragma unroll
      for (int i = 1; i < S; ++i)
        if (i == (e >> 6)) v = sv[i];
      se = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), e & 63));
    }
    if (lane == j) { my_e = e; my_s = se; }
    if (e >= 0 && (e & 63) == lane) {
#pragma unroll
      for (int i = 0; i < S; ++i)
        if (i == (e >> 6)) ord[i] = 0u;
    }
  }
  float acc = 0.0f;                     // every lane forms the same sum, in selection order
  for (int j = 0; j < k; ++j) acc = acc + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_s), j));
  const float denom = acc + 1e-20f;
  if (lane < k) {
    const float w = (my_s / denom) * route_scale;
    if (idx_row) { idx_row[lane] = my_e; w_row[lane] = w; }
    if (lidx) { lidx[lane] = my_e; lw[lane] = w; }
  }
}

__device__ __forceinline__ void topk_token(const float* __restrict__ srow, const float* __restrict__ bias,
                                           int E, int k, float route_scale, int32_t* __restrict__ idx_row,
                                           float* __restrict__ w_row, int32_t* lidx = nullptr,
                                           float* lw = nullptr) {
  if (E <= 256) topk_token_s<4>(srow, bias, E, k, route_scale, idx_row, w_row, lidx, lw);
  else topk_token_s<kMaxSlots>(srow, bias, E, k, route_scale, idx_row, w_row, lidx, lw);
}

// Arrival counter: returns true for the n-th arrival and resets the counter
// to zero for the next call (the counter region starts zero-filled).
__device__ __forceinline__ bool arrive_last(unsigned int* c, unsigned int n) {
  const unsigned int old = atomicAdd(c, 1u);
  if (old + 1u == n) {
    atomicExch(c, 0u);
    return true;
  }
  return false;
}

}  // namespace dsk
