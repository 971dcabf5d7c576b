// dsk_moe_forward_noalloc: the whole layer on the library's own per-GPU
// scratch memory, for callers that cannot allocate device memory (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// The scratch is one file-scope device array per GPU.  In host code its name
// is only a host-side stand-in, never a device address: the device address is
// taken once per device with hipGetSymbolAddress (with that device current)
// and only that address is handed to kernels.  Every call on a GPU shares the
// GPU's array and it keeps the last call's contents; the only region a call
// needs at zero, the fused router's arrival counters, is zero-filled (by a
// kernel) when the array is first set up and left at zero by every completed
// call.  Calls that overlap in time on one GPU race on the array.
#include <mutex>

#include "dsk_internal.h"

namespace dsk {
namespace {

__device__ __align__(256) unsigned char scratch[DSK_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the device of stream `s` (set up once per device).
int scratch_address(hipStream_t s, void** out) {
  int dev = 0;
  hipError_t e = s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return hip_check(e, "dsk_moe_forward_noalloc: device of the stream");
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(DSK_EUNSUPPORTED, "dsk_moe_forward_noalloc: device %d (scratch is kept for %d devices)", dev,
                kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = 0;
    if ((e = hipGetDevice(&cur)) != hipSuccess) return hip_check(e, "dsk_moe_forward_noalloc: hipGetDevice");
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess)
      return hip_check(e, "dsk_moe_forward_noalloc: hipSetDevice");
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) {
      const hipError_t back = hipSetDevice(cur);
      if (e == hipSuccess) e = back;
    }
    if (e != hipSuccess) return hip_check(e, "dsk_moe_forward_noalloc: hipGetSymbolAddress(scratch)");
    if ((e = launch_zero_fill(p, kCounterBytes, s)) != hipSuccess)
      return hip_check(e, "dsk_moe_forward_noalloc: counter fill");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DSK_OK;
}

}  // namespace
}  // namespace dsk

using namespace dsk;

extern "C" int dsk_moe_forward_noalloc(const dsk_moe_desc* d, const void* x, const void* gate_w,
                                       const float* gate_b, const dsk_expert_ptrs* table,
                                       const void* ws1, const void* ws3, const void* ws2,
                                       const void* shared_out, void* out, int32_t* idx,
                                       float* weights, void* stream) {
  // every check on the host before anything reaches the stream (also the first call's set-up)
  int rc = check_forward(d, x, gate_w, gate_b, table, ws1, ws3, ws2, shared_out, out, nullptr, true, nullptr, 1);
  if (rc) return rc;
  const size_t need = workspace_layout(*d).total;
  if (need > DSK_SCRATCH_BYTES)
    return fail(DSK_ESPACE, "dsk_moe_forward_noalloc: this call needs %zu bytes of scratch; the library "
                "holds %zu per GPU (use dsk_moe_forward with a workspace)", need,
                static_cast<size_t>(DSK_SCRATCH_BYTES));
  void* ws = nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if ((rc = scratch_address(s, &ws))) return rc;
  return forward_layer(d, x, gate_w, gate_b, table, ws1, ws3, ws2, shared_out, out, idx, weights, ws,
                       DSK_SCRATCH_BYTES, s, nullptr, 1);
}
