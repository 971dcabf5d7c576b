// Internal declarations shared by the HIP translation units of libdsk_moe.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/dsk_moe.h"

namespace dsk {

// ---------------------------------------------------------------- errors
int fail(int code, const char* fmt, ...);   // records the message, returns code
int hip_check(hipError_t e, const char* what);

// ---------------------------------------------------------------- types
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// float -> bf16 bits, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

// E8M0 byte -> float32 scale 2^(b-127); 0 -> 2^-127 (subnormal), 0xFF -> NaN.
__device__ __forceinline__ float e8m0_to_f32(uint32_t b) {
  uint32_t bits = (b == 0u) ? 0x00400000u : (b == 255u ? 0x7fc00000u : (b << 23));
  return __uint_as_float(bits);
}

// ---------------------------------------------------------------- workspace
// Regions of the caller-owned workspace used by dsk_moe_forward / dsk_experts.
struct Workspace {
  size_t scores, idx, wts, counts, offsets, perm, rank, active;  // routing
  size_t xb_hi, xb_lo;      // B-operand planes of x   [T][H]  (16-bit)
  size_t h_hi, h_lo;        // routed intermediate      [T*k][I] (16-bit)
  size_t hs_hi, hs_lo;      // shared intermediate      [T][Is]  (16-bit)
  size_t y;                 // routed outputs          [T*k][H] f32
  size_t ys;                // shared output           [T][H]   f32
  size_t total;
};

Workspace workspace_layout(const dsk_moe_desc& d);

// ---------------------------------------------------------------- launchers
// All launchers assume validated arguments.
hipError_t launch_route(const dsk_moe_desc& d, const void* x, const void* gate_w,
                        const float* gate_b, float* scores, int32_t* idx,
                        float* weights, hipStream_t s);

hipError_t launch_dispatch(const dsk_moe_desc& d, const int32_t* idx, int32_t* counts,
                           int32_t* offsets, int32_t* perm, int32_t* rank,
                           int32_t* active, hipStream_t s);

struct ExpertsArgs {
  const dsk_expert_ptrs* table;
  const void* ws1; const void* ws3; const void* ws2;
  const void* shared_out;    // precomputed shared output [T][H] in x dtype (or null)
  const void* x;
  const float* weights;      // [T*k] by flat position
  const int32_t* counts; const int32_t* offsets; const int32_t* perm;
  const int32_t* rank; const int32_t* active;
  void* out;
  char* ws;                  // workspace base
};

// ev (nullable): 3 events recorded after the gate/up kernel, the down kernel
// and the combine kernel.
hipError_t launch_experts(const dsk_moe_desc& d, const Workspace& L,
                          const ExpertsArgs& a, hipStream_t s, const hipEvent_t* ev);

hipError_t launch_fp4_dequant(const uint8_t* packed, const uint8_t* scales,
                              int64_t rows, int64_t cols, void* out, int out_dtype,
                              hipStream_t s);
hipError_t launch_fp4_quantize(const float* w, int64_t rows, int64_t cols,
                               uint8_t* packed, uint8_t* scales, hipStream_t s);
hipError_t launch_q3_quantize(const float* w, int64_t rows, int64_t cols,
                              uint8_t* packed, uint16_t* scales, uint16_t* biases,
                              hipStream_t s);
hipError_t launch_q3_dequant(const uint8_t* packed, const uint16_t* scales,
                             const uint16_t* biases, int64_t rows, int64_t cols,
                             void* out, int out_dtype, hipStream_t s);

}  // namespace dsk
