// Standalone token -> expert dispatch kernel (one workgroup).  The grouping
// itself is dispatch_block (dispatch_block.h); the fused router runs the same
// code in its last block.
#include "dispatch_block.h"

namespace dsk {
namespace {

__global__ __launch_bounds__(1024) void k_dispatch(const int32_t* __restrict__ idx, int N, int E,
                                                   int k, int nbits, const float* __restrict__ wflat,
                                                   const dsk_expert_ptrs* __restrict__ table,
                                                   DispatchOut o) {
  extern __shared__ int32_t lds[];
  dispatch_block(idx, N, E, k, nbits, wflat, table, o, lds);
}

}  // namespace

hipError_t launch_dispatch(const dsk_moe_desc& d, const int32_t* idx, const float* wflat,
                           const dsk_expert_ptrs* table, const DispatchOut& o, hipStream_t s) {
  const int E = d.n_experts;
  const int N = d.tokens * d.top_k;
  const int S = (E <= 512) ? 16 : 8;
  const size_t lds = static_cast<size_t>(S * E + E + 32) * sizeof(int32_t);
  launch_kernel(k_dispatch, 1, S * 64, lds, s, idx, N, E, d.top_k, bits_for(E), wflat, table, o);
  return hipGetLastError();
}

}  // namespace dsk
