// Internal declarations shared by the HIP translation units of libdsk_moe.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <type_traits>

#include "../../include/dsk_moe.h"

namespace dsk {

// ---------------------------------------------------------------- errors
int fail(int code, const char* fmt, ...);   // records the message, returns code
int hip_check(hipError_t e, const char* what);

// ---------------------------------------------------------------- stage timing
// The timed forward (dsk_moe_forward_timed) arms a thread-local table of two
// events per stage.  Every kernel launched through launch_kernel() while a
// stage is open carries the stage's start event (on its first launch) and
// its stop event (on every launch, so the last launch's end counts): the
// events then hold the kernels' own begin / end timestamps, the ones a
// profiler reports, with no marker packets between the kernels.
enum StageId { kStageGate = 0, kStageRoute, kStageUp, kStageDown, kStageCombine, kStageCount };
static_assert(2 * kStageCount == DSK_STAGE_EVENTS, "two events per stage");
struct StageClock {
  const hipEvent_t* ev = nullptr;  // 2 * kStageCount events, or null (not timing)
  int open = -1;                   // stage whose kernels are being launched
  bool launched = false;           // the open stage has launched a kernel
};
extern thread_local StageClock g_stage_clock;
// Opens `stage` (the next launches belong to it); no-op unless timing.  A
// stage that launches nothing leaves its events unrecorded.
hipError_t stage_open(int stage);
void stage_close();

template <class T> struct same_type { using type = T; };

// Kernel launch (all launches of the library go through here).  A failed
// launch is also the thread's last HIP error, which every launcher reads with
// hipGetLastError() after its launches.
template <typename... P>
inline void launch_kernel(void (*kernel)(P...), dim3 grid, dim3 block, size_t lds, hipStream_t s,
                          typename same_type<P>::type... args) {
  void* argv[] = {const_cast<void*>(static_cast<const void*>(&args))..., nullptr};
  hipEvent_t start = nullptr, stop = nullptr;
  StageClock& c = g_stage_clock;
  if (c.ev && c.open >= 0) {
    if (!c.launched) start = c.ev[2 * c.open];
    stop = c.ev[2 * c.open + 1];
    c.launched = true;
  }
  static_cast<void>(hipExtLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, argv, lds, s, start, stop, 0));
}

// ---------------------------------------------------------------- types
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// float -> bf16 bits, round to nearest even (NaN stays NaN, made quiet).
// Both results are formed and one is selected: no branch per element.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t nan = (u >> 16) | 0x40u;
  return static_cast<uint16_t>((u & 0x7fffffffu) > 0x7f800000u ? nan : rne);
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

// Byte offset, within a row of a q3 role, of lane group g's 12 bytes (its 32
// codes 128*kb + 32*g + [0, 32)) of 128-code block kb.  Every full 512-code
// superblock (4 blocks, 192 bytes) holds lane group g's chunks of its 4 blocks
// contiguously at byte 48*g, in block order, so one lane reads 4 blocks as
// three 16-byte words; blocks after the last full superblock are plain
// 48-byte blocks (chunk g at byte 12*g).
__host__ __device__ __forceinline__ uint32_t q3_chunk_offset(int K, int kb, int g) {
  return (kb >> 2) < (K >> 9) ? static_cast<uint32_t>((kb >> 2) * 192 + 48 * g + 12 * (kb & 3))
                              : static_cast<uint32_t>(kb * 48 + 12 * g);
}

// ---------------------------------------------------------------- dispatch
// One active expert, written by the dispatch for the expert kernels.
struct SlotDesc {
  int32_t e, n_tok, tok_base, pad;
  const void* p[9];          // w1 s1 b1 w3 s3 b3 w2 s2 b2 (copied from the table)
  const void* pad2;
};
static_assert(sizeof(SlotDesc) == 96, "SlotDesc layout");

struct DispatchOut {
  int32_t* counts; int32_t* offsets; int32_t* perm; int32_t* rank; int32_t* active;
  SlotDesc* desc;            // [E] or null
  int32_t* xrow;             // [T*k] token of each dispatch row, or null
  float* wrow;               // [T*k] route weight of each dispatch row
  int32_t* hist = nullptr;   // [blocks][E] per-block counts of the multi-block form, or null
};

// From this many (token, slot) positions, and with a histogram area, the
// dispatch runs as three kernels over blocks of kDispBlockPositions.
constexpr int kDispMultiMin = 8192;
constexpr int kDispBlockPositions = 2048;
inline size_t dispatch_hist_ints(int N, int E) {
  return N >= kDispMultiMin ? static_cast<size_t>((N + kDispBlockPositions - 1) / kDispBlockPositions) * E : 0;
}

// ---------------------------------------------------------------- workspace
// Regions of the caller-owned workspace used by dsk_moe_forward / dsk_experts.
struct Workspace {
  size_t scores, idx, wts, counts, offsets, perm, rank, active;  // routing
  size_t desc, xrow, wrow;  // dispatch descriptors
  size_t ctr;               // arrival counters of the fused router (zero between calls)
  size_t disp_hist;         // per-block counts of the multi-block dispatch
  size_t rowmap;            // decode pipeline: [min(E,64)][T] token -> dispatch row
  size_t xb_hi, xb_lo;      // B-operand planes of x   [T][H]  (16-bit)
  size_t h_hi, h_lo;        // routed intermediate      [T*k][I] (16-bit)
  size_t hs_hi, hs_lo;      // shared intermediate      [T][Is]  (16-bit)
  size_t hq, hqs;           // MX decode: routed intermediate as FP8 planes [T*k][3T][I]
                            // and their E8M0 bytes [T*k][3T][I/32] (mx_decode only)
  size_t y;                 // routed outputs          [T*k][H] f32
  size_t ys;                // shared output           [T][H]   f32
  size_t shared_x;          // decode pipeline: shared output [T][H] (x dtype)
  size_t xp;                // grouped FP4 gate/up: x as FP8 planes [T][2][H] + E8M0 [T][2][H/32];
                            // MX prefill: x as FP8 planes in stage rows [T][2H] + E8M0 [T][H/32]
                            // grouped q3: x scaled for the factored gate/up [T][H] bf16 + 64-group
                            // sums [T][H/64][2] f32
  size_t hp;                // grouped FP4: h as FP8 planes [T*k][3][I] + E8M0 [T*k][3][I/32];
                            // MX prefill: h in stage rows [T*k][2I] + E8M0 [T*k][I/32]
  size_t pf_tiles;          // prefill GEMM tile list  [2 + 2 * prefill_max_tiles] + the MX switch
  size_t total;
};

Workspace workspace_layout(const dsk_moe_desc& d);

// Bytes reserved at the start of every workspace for the fused router's
// arrival counters (one per token tile plus one, for the fused router of up
// to kFusedMaxTokens tokens).
constexpr size_t kCounterBytes = 1024;
constexpr int kFusedMaxTokens = 8;
// Decode pipeline limits and the shared expert's gate/up K split.
constexpr int kDecodeMaxTokens = 16;
// From this many tokens the decode pipeline runs the grouped down kernel and
// the combine instead of its fused down + combine kernel.
constexpr int kDecodeGroupedDownMin = 3;
// ... and from this many its routed gate/up in the grouped kernel.
constexpr int kDecodeGroupedUpMin = 8;
constexpr int kDecodeMaxPositions = 64;
constexpr size_t kMaxLds = 163840;          // LDS bytes one gfx950 workgroup may use
constexpr size_t kUpLdsFixed = 2 * 4 * 2 * 64 * 4 * 4 + 8 * 640;   // decode gate/up: reduction + scale tiles
// Prefill GEMM tiles: 256 weight rows x 256 dispatch rows per block.
constexpr int kPfRows = 256;
constexpr int kPfToks = 256;
constexpr int kPrefillMinTokens = 128;

// Large batches of bf16 tokens run the expert products as MFMA GEMM tiles
// (gate/up tiles of 128 intermediate rows, down tiles of 256 output rows).
inline bool prefill_gemm(const dsk_moe_desc& d) {
  return d.x_dtype == DSK_DTYPE_BF16 && d.tokens >= kPrefillMinTokens && d.hidden % kPfRows == 0 &&
         d.inter % 128 == 0 && d.inter_shared % 128 == 0;
}
int prefill_max_tiles(const dsk_moe_desc& d);
// FP4 prefill GEMMs on the scaled FP4 x FP8 MFMAs (x and h as two FP8 planes;
// K of both products a multiple of 512, the LDS DMA loop's).
inline bool prefill_mx(const dsk_moe_desc& d) {
  return prefill_gemm(d) && d.quant == DSK_QUANT_FP4 && d.hidden % 512 == 0 && d.inter % 512 == 0;
}
// The prefill GEMM's routed rows for the combine are rounded to bf16 when the
// experts are FP4 (relative 2^-9 per row, inside the layer tolerance); q3
// layers, whose dequantised weights are already rounded to bf16, and rows
// handed to the caller stay float32.  Its shared output is always bf16.
inline bool prefill_rows_bf16(const dsk_moe_desc& d, const float* rows_out) {
  return d.quant == DSK_QUANT_FP4 && rows_out == nullptr;
}

inline bool decode_pipeline(const dsk_moe_desc& d) {
  // the gate/up kernel stages the tokens' activations (bf16 hi, and lo for
  // float32 x) plus its reduction and scale-exchange buffers in LDS
  const size_t x_lds = static_cast<size_t>(d.x_dtype == DSK_DTYPE_F32 ? 2 : 1) * d.tokens *
                           (d.hidden + 8) * 2 + kUpLdsFixed;
  return d.tokens <= kDecodeMaxTokens && d.tokens * d.top_k <= kDecodeMaxPositions &&
         x_lds <= kMaxLds;
}

// FP4 experts, bf16 activations and one or two tokens: the decode gate/up and
// down kernels run the routed products as scaled FP4 x FP8 MFMAs, with the
// activations split into FP8 planes (two for x, three for h) on the B side.
// The down kernel's eight waves take two K blocks each of an intermediate of
// kMxInter (the shared expert runs in the decode pipeline's first two kernels).
constexpr int kMxMaxTokens = 2;
constexpr int kMxInter = 2048;
inline bool mx_decode(const dsk_moe_desc& d) {
  // gate/up LDS: 21.5 KB of partial sums and exchange tiles, 2.07 T H bytes of activation planes
  const size_t up_lds = 32768 + static_cast<size_t>(d.tokens) * d.hidden * 3;
  return d.quant == DSK_QUANT_FP4 && d.x_dtype == DSK_DTYPE_BF16 && d.tokens <= kMxMaxTokens &&
         decode_pipeline(d) && d.hidden % 128 == 0 && d.inter == kMxInter && up_lds <= kMaxLds;
}

// ---------------------------------------------------------------- launchers
// All launchers assume validated arguments.
hipError_t launch_route(const dsk_moe_desc& d, const void* x, const void* gate_w,
                        const float* gate_b, float* scores, int32_t* idx,
                        float* weights, hipStream_t s);

// Router + top-k + dispatch.  Small batches run as one kernel whose last
// blocks do the top-k and the dispatch; larger ones as three kernels.
struct ResNorm;   // resnorm.h: the stack's residual update + RMSNorm, fused into a layer's first kernel

// x as the gate/up after an unfused top-k reads it (written by the top-k's
// trailing blocks): the grouped FP4 gate/up's FP8 planes, the grouped q3
// gate/up's factored form, the prefill MX gate/up's FP8 planes.
enum XForm : int { kXGroupedPlanes = 0, kXGroupedQ3 = 1, kXPrefillPlanes = 2 };

struct RouteArgs {
  const void* x; const void* gate_w; const float* gate_b;
  const ResNorm* rn;        // non-null: the gate kernel computes x itself (resnorm.h)
  float* scores; int32_t* idx; float* weights;
  const dsk_expert_ptrs* table;
  DispatchOut out;
  unsigned int* ctr;        // [tokens + 1] arrival counters (fused path), zero between calls
  int32_t* rowmap;          // decode pipeline: [slot][tokens] token -> dispatch row map
  uint8_t* xp;              // unfused top-k: also write x here in the form of the gate/up
                            // that follows (Workspace::xp), or null:
  int xform;                // XForm
};
// Fused router + dispatch (general path).
hipError_t launch_route_dispatch(const dsk_moe_desc& d, const RouteArgs& a, hipStream_t s);

hipError_t launch_dispatch(const dsk_moe_desc& d, const int32_t* idx, const float* wflat,
                           const dsk_expert_ptrs* table, const DispatchOut& o, hipStream_t s);

// Routing of the decode pipeline: the layer's idx / weights [T][k], and for
// the decode kernels active (count, then the expert of each slot), one
// descriptor per slot, rowmap [slot][T] (-1: token not routed to the slot),
// the token and route weight of each dispatch row (xrow, wrow) and, for the
// combine, the dispatch row of each flat position (rank, -1 if dropped).
struct DecodeRoute {
  int32_t* idx; float* weights;
  SlotDesc* desc; int32_t* active; int32_t* rowmap; int32_t* xrow; float* wrow; int32_t* rank;
};

struct ExpertsArgs {
  const dsk_expert_ptrs* table;
  const SlotDesc* desc; const int32_t* xrow; const float* wrow;
  const void* ws1; const void* ws3; const void* ws2;
  const void* shared_out;    // precomputed shared output [T][H] in x dtype (or null)
  const void* gate_w;        // decode pipeline: gate weights [E][H] (gate dtype)
  const void* x;
  const float* weights;      // [T*k] by flat position
  const int32_t* counts; const int32_t* offsets; const int32_t* perm;
  const int32_t* rank; const int32_t* active;
  void* out;
  char* ws;                  // workspace base
  float* rows_out;           // dsk_expert_rows: the per-row outputs go here and nothing is combined
  const ResNorm* rn;         // non-null: the first kernel computes x itself (resnorm.h)
  const int32_t* rowmap;     // decode pipeline: [slot][T] dispatch row of token t, -1 if none
  // decode pipeline: gate scores and selection bias in, routing out
  float* scores; const float* bias;
  DecodeRoute route;
  int x_planes_ready;        // the routing kernels already wrote x's FP8 planes / q3 form (RouteArgs::xp)
};

// Opens the gate/up, down and combine stages as it launches them.
// repeat: each kernel is launched that many times in a row (timing only).
hipError_t launch_experts(const dsk_moe_desc& d, const Workspace& L,
                          const ExpertsArgs& a, hipStream_t s, int repeat);

hipError_t launch_zero_fill(void* p, size_t bytes, hipStream_t s);

// cap_union of a lock-step batch's routing, in place (one block): LDS bytes and launch.
size_t cap_union_lds(int T, int E, int k);
hipError_t launch_cap_union(const float* scores, int32_t* idx, float* w, int T, int E, int k, int budget,
                            int strict, hipStream_t s);

// The whole layer (dsk_moe_forward / _timed / _noalloc): check_forward validates
// every argument on the host (DSK_OK or a DSK_E* code with the message set;
// own_scratch: the library's scratch stands in for the caller's workspace);
// forward_layer validates, then launches on `stream` into `workspace`.
int check_forward(const dsk_moe_desc* d, const void* x, const void* gate_w, const float* gate_b,
                  const dsk_expert_ptrs* table, const void* ws1, const void* ws3, const void* ws2,
                  const void* shared_out, void* out, const void* workspace, bool own_scratch,
                  void* const* events, int repeat);
int forward_layer(const dsk_moe_desc* d, const void* x, const void* gate_w, const float* gate_b,
                  const dsk_expert_ptrs* table, const void* ws1, const void* ws3, const void* ws2,
                  const void* shared_out, void* out, int32_t* idx, float* weights, void* workspace,
                  size_t workspace_bytes, void* stream, void* const* events, int repeat,
                  const ResNorm* rn = nullptr);
// The decode pipeline's first kernel takes the residual update and RMSNorm
// itself (bf16 stream, one or two tokens, rows up to 4096 wide).
bool resnorm_fusable(const dsk_moe_desc& d);
hipError_t launch_rmsnorm(const void* x, const void* res, const float* gamma, int64_t rows, int H, float eps,
                          int dtype, void* h_out, void* y, hipStream_t s);

// Prefill GEMM path (prefill_gemm(d)): tile list, gate/up, down; the caller
// runs the combine.  Opens the gate/up and down stages.
// Where the expert kernels write their per-dispatch-row float32 outputs.
inline float* rows_buffer(float* rows_out, char* ws, const Workspace& L) {
  return rows_out ? rows_out : reinterpret_cast<float*>(ws + L.y);
}

struct PrefillArgs {
  const SlotDesc* desc; const int32_t* active; const int32_t* xrow; const float* wrow;
  const void* x; const void* ws1; const void* ws3; const void* ws2;
  char* ws;
  float* rows_out;           // per-row outputs instead of the workspace's (or null)
  int x_planes_ready;        // the routing kernels already wrote x's FP8 planes
};
hipError_t launch_experts_prefill(const dsk_moe_desc& d, const Workspace& L, const PrefillArgs& a,
                                  hipStream_t s, int repeat);

// Grouped path for batches below the prefill size (bf16 x, shapes that
// tile): per slot, column tiles of its dispatch rows with only their
// activation rows staged; the shared expert as a pseudo-slot.  Writes the
// routed rows y and the shared output ys for launch_combine.  Opens the
// gate/up and down stages.
bool grouped_path(const dsk_moe_desc& d);
hipError_t launch_experts_grouped(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a,
                                  const SlotDesc* desc, const int32_t* xrow, const float* wrow, hipStream_t s,
                                  int repeat);
// Its kernels one at a time, for the decode pipeline: the routed gate/up
// alone (from kDecodeGroupedUpMin tokens) and the down (routed rows from h,
// shared from hs; from kDecodeGroupedDownMin tokens).
// x_planes_ready: the routing kernel already wrote x's FP8 planes (grouped_up_mx).
hipError_t launch_grouped_up_routed(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a,
                                    const SlotDesc* desc, const int32_t* xrow, const float* wrow, hipStream_t s,
                                    int repeat, bool x_planes_ready);
// The grouped FP4 gate/up takes x as FP8 planes (Workspace::xp).
bool grouped_up_mx(const dsk_moe_desc& d);
// The grouped q3 gate/up takes x scaled for the factored product, with its
// 64-group sums (Workspace::xp).
bool grouped_x_q3(const dsk_moe_desc& d);
// h_planes: the routed h is in FP8 planes (the grouped gate/up ran and grouped_h_planes).
hipError_t launch_grouped_down(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a,
                               const SlotDesc* desc, hipStream_t s, int repeat, bool h_planes);
// The grouped FP4 gate/up writes h as FP8 planes and the down reads them on scaled MFMAs.
bool grouped_h_planes(const dsk_moe_desc& d);
// out[t] = cast(sum of the token's routed rows y in ascending expert id +
// shared); the combine stage.
hipError_t launch_combine(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a, hipStream_t s,
                          int repeat);

// Decode pipeline (decode_pipeline(d)), four kernels.  With the MX kernels
// (mx_decode(d)):
//   launch_gate_shared    gate scores (a.scores) beside the shared expert's gate/up (hs);
//   launch_route_sdown    top-k and slot map (a.route) in one block beside the shared
//                         expert's down, written to the workspace's shared_x (x dtype);
//   launch_experts_decode the routed gate/up and down, called with no shared
//                         intermediate and shared_x as the precomputed shared output.
// Otherwise:
//   launch_gate_scores    gate scores (a.scores);
//   launch_route_shared   top-k and slot map beside the shared expert's gate/up (hs);
//   launch_experts_decode the routed gate/up, then the routed and shared down and the
//                         combine in one kernel (stages as for launch_experts).
hipError_t launch_gate_shared(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a, hipStream_t s,
                              int repeat);
hipError_t launch_route_sdown(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a, hipStream_t s,
                              int repeat);
hipError_t launch_gate_scores(const dsk_moe_desc& d, const RouteArgs& a, hipStream_t s);
hipError_t launch_route_shared(const dsk_moe_desc& d, const Workspace& L, const ExpertsArgs& a, hipStream_t s,
                               int repeat);
hipError_t launch_experts_decode(const dsk_moe_desc& d, const Workspace& L,
                                 const ExpertsArgs& a, hipStream_t s, int repeat);

hipError_t launch_fp8_block_dequant(const uint8_t* codes, const uint8_t* scales, int64_t rows, int64_t cols,
                                    void* out, int out_dtype, hipStream_t s);
hipError_t launch_fp4_dequant(const uint8_t* packed, const uint8_t* scales,
                              int64_t rows, int64_t cols, void* out, int out_dtype,
                              hipStream_t s);
hipError_t launch_fp4_quantize(const float* w, int64_t rows, int64_t cols,
                               uint8_t* packed, uint8_t* scales, hipStream_t s);
hipError_t launch_q3_quantize(const float* w, int64_t rows, int64_t cols,
                              uint8_t* packed, uint16_t* scales, uint16_t* biases,
                              hipStream_t s);
hipError_t launch_q3_repack(const uint8_t* src, int64_t rows, int64_t cols, uint8_t* packed, hipStream_t s);
hipError_t launch_q3_dequant(const uint8_t* packed, const uint16_t* scales,
                             const uint16_t* biases, int64_t rows, int64_t cols,
                             void* out, int out_dtype, hipStream_t s);

}  // namespace dsk
