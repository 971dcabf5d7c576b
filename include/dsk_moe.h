/*
 * dsk_moe.h -- C ABI of the MI355X (gfx950) MoE-layer forward library.
 *
 * Every entry point is stream-ordered and asynchronous: it validates its
 * arguments on the host, launches HIP kernels on `stream` (a hipStream_t;
 * NULL is the default stream) and returns.  No entry point allocates device
 * memory or synchronises, except where stated.  All pointers are device
 * pointers unless stated otherwise; the caller owns every buffer, including
 * the workspace.  Return value: DSK_OK or a negative DSK_E* code; the
 * message of the last failure on the calling thread is in dsk_last_error().
 *
 * Layouts (row-major, the reference's expert weight layout):
 *   FP4 role [N, K]:  packed [N, K/2] u8 (two e2m1 codes per byte, low nibble
 *                     first) + scales [N, K/32] u8 (E8M0, 2^(b-127), 0xFF = NaN)
 *   Q3 role [N, K]:   packed [N, 3K/8] u8 (canonical packing: 128-code blocks
 *                     of four 12-byte lane-group chunks; in every full 512-code
 *                     superblock, chunk g of its 4 blocks sits at byte 48g,
 *                     block order; a tail block is plain 48 bytes) + scales
 *                     [N, K/64] f16 + biases [N, K/64] f16, W = s*q + b
 *   roles: w1, w3 [I, H]; w2 [H, I]; used as x @ W^T.
 *   shared expert: bf16 w1, w3 [Is, H]; w2 [H, Is].
 */
#ifndef DSK_MOE_H
#define DSK_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSK_ABI_VERSION 1

/* status codes */
#define DSK_OK 0
#define DSK_EINVAL (-1)        /* bad shape, null pointer or enum */
#define DSK_EALIGN (-2)        /* pointer not aligned as the kernel needs */
#define DSK_EUNSUPPORTED (-3)  /* valid request this build does not implement */
#define DSK_EHIP (-4)          /* a HIP runtime call failed */
#define DSK_ESPACE (-5)        /* workspace smaller than dsk_workspace_size() */

/* router score functions */
#define DSK_SCORE_SIGMOID 0       /* s = 1 / (1 + exp(-z)) */
#define DSK_SCORE_SQRTSOFTPLUS 1  /* s = sqrt(log(1 + exp(z))) */

/* routed expert formats */
#define DSK_QUANT_FP4 0  /* e2m1 + E8M0 per 32 along K */
#define DSK_QUANT_Q3 1   /* 3-bit affine, fp16 scale and bias per 64 along K */

/* element types */
#define DSK_DTYPE_BF16 0
#define DSK_DTYPE_F32 1

/* Layer description.  Mirrors the arguments of the reference's
 * moe_layer(x, gate_w, gate_b, expert_fn, shared_fn, top_k, limit)
 * (src/deepseeker/mlx_forward.py:257-263) plus the route scale of
 * route_topk (:68-69) and the expert format. */
typedef struct dsk_moe_desc {
  int32_t tokens;        /* T >= 1 rows of x */
  int32_t hidden;        /* H */
  int32_t n_experts;     /* E, 1..1024 */
  int32_t top_k;         /* k, 1..min(E, 16) */
  int32_t inter;         /* I, routed expert intermediate size */
  int32_t inter_shared;  /* Is, shared expert intermediate size; 0 = no shared expert */
  int32_t score_func;    /* DSK_SCORE_* */
  int32_t quant;         /* DSK_QUANT_* */
  int32_t x_dtype;       /* DSK_DTYPE_BF16 or _F32: x and out */
  int32_t gate_dtype;    /* DSK_DTYPE_F32 or _BF16: gate_w */
  float route_scale;     /* multiplies the normalised weights (reference default 1.5) */
  float limit;           /* SwiGLU clamp L (reference passes 10.0) */
} dsk_moe_desc;

/* Device pointers of one routed expert (an element of the device table
 * indexed by expert id).  b* are Q3 biases (NULL for FP4).  Code, scale and
 * bias pointers 16-byte aligned (the kernels read them in 16-byte pieces; the
 * prefill GEMM takes its register-staged loop for an FP4 expert that is not). */
typedef struct dsk_expert_ptrs {
  const void* w1; const void* s1; const void* b1;
  const void* w3; const void* s3; const void* b3;
  const void* w2; const void* s2; const void* b2;
} dsk_expert_ptrs;

int dsk_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* dsk_last_error(void);

/* Bytes of workspace dsk_moe_forward / dsk_experts need for this desc (host only). */
int dsk_workspace_size(const dsk_moe_desc* d, size_t* bytes);

/* Zero-fill a workspace (a fill kernel on `stream`, no memset node).  The
 * fused router keeps arrival counters in the workspace: it must be
 * zero-filled once before its first use; every completed call leaves the
 * counters at zero again.  No counterpart in the reference (it has no
 * device workspace). */
int dsk_workspace_init(void* workspace, size_t workspace_bytes, void* stream);

/* Router: replaces sqrtsoftplus_scores + route_topk
 * (src/deepseeker/mlx_forward.py:62-81).
 * x [T,H] (x_dtype), gate_w [E,H] (gate_dtype), gate_b [E] f32 ->
 * scores [T,E] f32, idx [T,k] i32 (descending key, ties to lower id),
 * weights [T,k] f32.  Bit-exact with the fixed-order definition of the oracle. */
int dsk_route(const dsk_moe_desc* d, const void* x, const void* gate_w,
              const float* gate_b, float* scores, int32_t* idx, float* weights,
              void* stream);

/* Dispatch: replaces the np.unique / row discovery of moe_layer
 * (src/deepseeker/mlx_forward.py:294-312, 388-396) and the
 * align_block_size contract (src/deepseeker/moe_align.py:21-46).
 * idx [T,k] i32 -> counts [E], offsets [E+1] (exclusive prefix sum),
 * perm [T*k] (flat positions t*k+j sorted by (expert, position)),
 * rank [T*k] (inverse of perm, -1 for dropped entries),
 * active [E+1] (active[0] = number of experts with a routed position,
 * then their ids ascending).  Entries < 0 or >= E are dropped. */
int dsk_dispatch(const dsk_moe_desc* d, const int32_t* idx, int32_t* counts,
                 int32_t* offsets, int32_t* perm, int32_t* rank, int32_t* active,
                 void* stream);

/* dsk_dispatch with the same outputs bit for bit, computed over several
 * workgroups when T*k >= 8192 (per-workgroup counts in the caller's
 * workspace, 256-byte aligned, of dsk_dispatch_workspace_size bytes; 0 bytes
 * below 8192 positions, where it is dsk_dispatch).  No counterpart in the
 * reference: the forward call's own dispatch, exposed so that callers with
 * large batches and tests reach it. */
int dsk_dispatch_workspace_size(const dsk_moe_desc* d, size_t* bytes);
int dsk_dispatch_ws(const dsk_moe_desc* d, const int32_t* idx, int32_t* counts,
                    int32_t* offsets, int32_t* perm, int32_t* rank, int32_t* active,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Union cap of a lock-step batch: replaces cap_union
 * (src/deepseeker/mlx_forward.py:213-254), which moe_layer applies when
 * union_budget > 0 and the batch has more than one row (:294-305).  In place on
 * the router's output: idx [T,k] i32 and weights [T,k] f32 in this library's
 * order (descending key per row), scores [T,E] f32 the un-biased gate scores
 * that rank the experts.  If the batch's expert union exceeds `budget`, the
 * `budget` experts with the largest summed score (rows ascending; exact ties
 * to the lower expert id) are kept, other slots get index -1 and weight 0, a
 * row left with nothing keeps its largest weight (first maximum in ascending
 * key order) unless `strict`, and each row is rescaled to its original weight
 * sum: scale = rowsum(w) / (rowsum(kept) + 1e-20) with numpy's float32 pairwise
 * row sum in ascending key order.  One block: T*top_k*4 + E*9 bytes must fit
 * the 160 KB of LDS (DSK_EUNSUPPORTED otherwise).  dsk_dispatch drops the -1
 * slots. */
int dsk_cap_union(int32_t tokens, int32_t n_experts, int32_t top_k, int32_t budget, int32_t strict,
                  const float* scores, int32_t* idx, float* weights, void* stream);

/* Experts + shared expert + combine, given routing and dispatch:
 * replaces the per-expert loop, the shared add and the final cast of
 * moe_layer (src/deepseeker/mlx_forward.py:388-419) and the shared expert
 * (src/deepseeker/mlx_runner.py:765-783).
 * table: device array [E] of dsk_expert_ptrs (all E entries readable; the
 * weights of experts that receive no token are never read, so their pointers
 * may be anything); ws1/ws3/ws2: shared expert bf16 weights
 * (used when inter_shared > 0); shared_out: an already computed shared
 * expert output [T,H] in x_dtype, added instead when inter_shared == 0
 * (NULL: no shared expert); out [T,H] in x_dtype. */
int dsk_experts(const dsk_moe_desc* d, const dsk_expert_ptrs* table,
                const void* ws1, const void* ws3, const void* ws2,
                const void* shared_out, const void* x, const float* weights, const int32_t* counts,
                const int32_t* offsets, const int32_t* perm, const int32_t* rank,
                const int32_t* active, void* out, void* workspace,
                size_t workspace_bytes, void* stream);

/* Weighted output rows of every routed (token, expert) pair, not combined:
 * replaces gather_pinned_contributions (src/deepseeker/mlx_forward.py:159-210),
 * the banked gate/up and w2 products of the runner's pinned experts
 * (src/deepseeker/mlx_runner.py:949-960).  rows [n, H] float32 receives, for
 * dispatch row r (pairs in dsk_dispatch's order: expert ascending, then flat
 * position t*k + j ascending, i.e. expert, token, slot), the row
 * w2 (silu(min(x w1, L)) * clip(x w3, -L, L) * weight) of that pair; n is the
 * number of pairs with an index in [0, E) and the buffer must hold T*k rows.
 * Routed experts only: d->inter_shared must be 0.  Arguments otherwise as for
 * dsk_experts (float32 x runs the products on bf16 hi/lo operands). */
int dsk_expert_rows(const dsk_moe_desc* d, const dsk_expert_ptrs* table, const void* x,
                    const float* weights, const int32_t* counts, const int32_t* offsets,
                    const int32_t* perm, const int32_t* rank, const int32_t* active, float* rows,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Whole layer: replaces moe_layer (src/deepseeker/mlx_forward.py:257-419):
 * dsk_route, dsk_dispatch and dsk_experts on one stream.  Shared-expert
 * arguments as for dsk_experts.  idx / weights are optional outputs
 * (NULL: kept in the workspace only). */
int dsk_moe_forward(const dsk_moe_desc* d, const void* x, const void* gate_w,
                    const float* gate_b, const dsk_expert_ptrs* table,
                    const void* ws1, const void* ws3, const void* ws2,
                    const void* shared_out, void* out,
                    int32_t* idx, float* weights, void* workspace,
                    size_t workspace_bytes, void* stream);

/* The residual stream between two layers of a stack, for
 * dsk_moe_forward_residual. */
typedef struct dsk_residual {
  const void* h;        /* [T,H] the stream before this layer, x_dtype */
  const void* d;        /* [T,H] the previous layer's output, x_dtype */
  const float* gamma;   /* [H] RMSNorm weight, or NULL (ones) */
  float eps;
  void* h_out;          /* [T,H] h + d rounded to x_dtype (may be h itself) */
  void* x_out;          /* [T,H] rmsnorm(h + d) * gamma: the layer's input */
} dsk_residual;

/* One step of the runner's layer loop (src/deepseeker/mlx_runner.py:2138-2145):
 * the residual add and rmsnorm (src/deepseeker/mlx_forward.py:45-59), then
 * moe_layer on the normalised rows -- the same results as dsk_rmsnorm(h, d,
 * gamma, ..., h_out, x_out) followed by dsk_moe_forward(x = x_out), bit for
 * bit.  In the decode pipeline at one or two bf16 tokens (rows up to 4096
 * wide) with h_out a buffer of its own, the layer's first kernel computes the
 * update itself (each block normalises the rows it needs, one block writes
 * h_out and x_out), which saves a launch per layer; otherwise the update runs
 * as its own kernel first.  x_out and h_out must not overlap the other
 * buffers.  Shared-expert arguments as for dsk_moe_forward (no precomputed
 * shared output). */
int dsk_moe_forward_residual(const dsk_moe_desc* d, const dsk_residual* r, const void* gate_w,
                             const float* gate_b, const dsk_expert_ptrs* table, const void* ws1,
                             const void* ws3, const void* ws2, void* out, int32_t* idx, float* weights,
                             void* workspace, size_t workspace_bytes, void* stream);

/* dsk_moe_forward that times its five stages with DSK_STAGE_EVENTS hipEvent_t
 * created by the caller: events[2i] and events[2i+1] receive the begin
 * timestamp of stage i's first kernel and the end timestamp of its last
 * kernel (the kernels are launched with hipExtLaunchKernel carrying the
 * events, so no marker packet runs between kernels and the interval is the
 * kernels' own execution time, as a profiler reports it).  Stages: 0 gate
 * scores (the fused router of up to 8 tokens also selects and dispatches
 * here), 1 top-k and dispatch (the decode pipeline: top-k and slot map beside
 * the shared expert's gate/up), 2 gate/up, 3 down, 4 combine.  A stage that
 * launches no kernel (the decode pipeline of 1-2 tokens combines inside its
 * down kernel) leaves its two events unrecorded.  Each
 * stage's kernels are launched `repeat` times in a row (every stage recomputes
 * its outputs from its inputs, so the result is that of one forward).
 * Create the events with hipEventDisableSystemFence where no system-scope
 * release is wanted at a stop timestamp.
 * No counterpart in the reference: it is for callers that time the stages
 * (the benchmark). */
#define DSK_STAGE_EVENTS 10
int dsk_moe_forward_timed(const dsk_moe_desc* d, const void* x, const void* gate_w,
                          const float* gate_b, const dsk_expert_ptrs* table,
                          const void* ws1, const void* ws3, const void* ws2,
                          const void* shared_out, void* out, int32_t* idx, float* weights,
                          void* workspace, size_t workspace_bytes, void* stream,
                          void* const* events, int32_t repeat);

/* Whole layer as dsk_moe_forward, on the library's own scratch memory instead
 * of a caller workspace: it allocates nothing (no hipMalloc, hipFree or
 * allocating library call).  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Each GPU the
 * library runs on holds one scratch array of DSK_SCRATCH_BYTES for the life
 * of the process (its device address is looked up on the first call on that
 * GPU); a call whose dsk_workspace_size exceeds it fails with DSK_ESPACE
 * before any launch (e.g. the full-size 256-expert layer up to ~128 tokens
 * fits).  All calls on one GPU share that array and it keeps the last call's
 * contents: calls that overlap in time on one GPU (several streams or host
 * threads) race, and the caller must order them. */
#define DSK_SCRATCH_BYTES (32u << 20)
int dsk_moe_forward_noalloc(const dsk_moe_desc* d, const void* x, const void* gate_w,
                            const float* gate_b, const dsk_expert_ptrs* table,
                            const void* ws1, const void* ws3, const void* ws2,
                            const void* shared_out, void* out, int32_t* idx, float* weights,
                            void* stream);

/* FP4 dequant: replaces metal_dequant / the Metal e2m1 kernels
 * (src/deepseeker/metal_fp4.py:28-66, 139-155) and dequant_fp4_rowmajor
 * (src/deepseeker/mlx_weights.py:148-166).  [rows, cols] FP4 role -> out
 * [rows, cols] in out_dtype (f32 or bf16; exact). cols % 32 == 0. */
int dsk_fp4_dequant(const uint8_t* packed, const uint8_t* scales, int64_t rows,
                    int64_t cols, void* out, int32_t out_dtype, void* stream);

/* FP8 block dequant of the checkpoint's dense weights (the shared expert):
 * replaces dequant_fp8_block and E4M3_TABLE (src/deepseeker/mlx_weights.py:29-41,
 * 82-89).  codes [rows, cols] OCP E4M3 bytes, scales [rows/32, cols/32] E8M0
 * (one per 32 x 32 block; 0xFF -> NaN) -> out [rows, cols] in out_dtype (f32 or
 * bf16; exact unless the scaled value leaves the bf16 range).  rows % 32 == 0,
 * cols % 32 == 0. */
int dsk_fp8_block_dequant(const uint8_t* codes, const uint8_t* scales, int64_t rows,
                          int64_t cols, void* out, int32_t out_dtype, void* stream);

/* FP4 quantise (spec rule: scale 2^ceil(log2(amax/6)) per 32, nearest-even
 * e2m1, saturate at 6): stands in for mx.quantize(mode="mxfp4") used by the
 * reference's tests and loaders.  w [rows, cols] f32. */
int dsk_fp4_quantize(const float* w, int64_t rows, int64_t cols, uint8_t* packed,
                     uint8_t* scales, void* stream);

/* Q3 affine quantise (group 64, fp16 scale/bias, canonical packing):
 * replaces convert_tensor (scripts/requant_experts_3bit.py:69-83).
 * cols % 128 == 0. */
int dsk_q3_quantize(const float* w, int64_t rows, int64_t cols, uint8_t* packed,
                    uint16_t* scales, uint16_t* biases, void* stream);

/* Q3 repack of checkpoint codes into the canonical layout: replaces the read
 * side of the reference's q3 checkpoints, unpack_int3_affine
 * (src/deepseeker/mlx_weights.py:119-141) over the U32_Q3_AFFINE tensors that
 * scripts/requant_experts_3bit.py:69-83, 135-148 writes.  src [rows, 3*cols/8]
 * bytes (= [rows, 3*cols/32] little-endian u32 words): row-major 3-byte packs,
 * bytes 3m..3m+2 of a row holding codes 8m..8m+7 as a 24-bit little-endian
 * integer with code i at bits 3i..3i+2 -> packed [rows, 3*cols/8] in the
 * canonical layout above (scales and biases are unchanged).  cols % 128 == 0;
 * src and packed must not overlap. */
int dsk_q3_repack(const uint8_t* src, int64_t rows, int64_t cols, uint8_t* packed, void* stream);

/* Q3 dequant: replaces mx.dequantize(bits=3, group_size=64)
 * (scripts/requant_experts_3bit.py:74-75); out = f32(s)*q + f32(b). */
int dsk_q3_dequant(const uint8_t* packed, const uint16_t* scales,
                   const uint16_t* biases, int64_t rows, int64_t cols, void* out,
                   int32_t out_dtype, void* stream);

/* RMSNorm on a residual stream: replaces rmsnorm (src/deepseeker/mlx_forward.py:45-59)
 * together with the residual add that precedes it in a stack of layers.
 * h = x (+ residual, rounded to dtype); h is written to h_out when given (h_out
 * may be x itself); out = h * (1 / sqrt(mean(h^2) + eps)) * gamma, in float32
 * with one rounding to dtype.  rows rows of `hidden` elements (dtype F32 or
 * BF16); gamma [hidden] f32 or NULL (all ones); out may be NULL when only the
 * residual update is wanted.  The sum of squares has one defined order (per
 * thread over chunks t, t+256, ... of 4 elements, an XOR tree over each wave,
 * the 4 waves in order), restated by the oracle.  16-byte aligned pointers. */
int dsk_rmsnorm(const void* x, const void* residual, const float* gamma, int64_t rows,
                int32_t hidden, float eps, int32_t dtype, void* h_out, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSK_MOE_H */
