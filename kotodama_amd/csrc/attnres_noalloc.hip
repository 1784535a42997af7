// attnres_route_bwd_noalloc: the routing backward without a caller workspace,
// for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc).
//
// attnres_route_bwd needs device memory beyond its inputs and outputs: one
// fp32 row of `hidden` per workgroup of its grid, holding that workgroup's
// partial sum of the query gradient, which the reduction kernels then sum (in
// place, in a fixed order).  This entry point takes that memory from
// `scratch`, a file-scope device array of ATTNRES_NOALLOC_SCRATCH_BYTES that
// every device the library runs on holds until the process ends.  Host code
// never passes the array's name to a kernel (on the host it names a
// stand-in, not a device address): set-up resolves its device address once
// per device with hipGetSymbolAddress, and every call passes that address on.
//
// Every workgroup of the backward writes its whole partial row before the
// reduction reads it, so nothing in `scratch` needs to start at zero.  All
// calls on one device share its array: calls that overlap on that device
// (different streams, or threads without ordering) race on it.
//
// Compiled by hipcc as HIP source (the array needs device code of its own);
// the kernels themselves live in the code-object parts of
// attnres_kernels.hip and receive the scratch address as an argument.

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <mutex>

#include "attnres.h"

// Error reporting of attnres_capi.cpp (sets attnres_last_error()).
extern "C" int attnres_internal_fail(int code, const char* msg);

static __device__ __align__(256) unsigned char scratch[ATTNRES_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;

std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device, resolved once per device.
// The first resolution may load the code object that holds the array (and so
// place the array in device memory); that must not happen inside a stream
// capture, so a call on a capturing `stream` before set-up is an error.
int scratch_for_current_device(void** out, hipStream_t stream = nullptr, bool check_capture = false) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return attnres_internal_fail(ATTNRES_ERR_HIP, "hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices) return attnres_internal_fail(ATTNRES_ERR_HIP, "device ordinal out of range");
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr && check_capture) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &status);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return attnres_internal_fail(ATTNRES_ERR_HIP, "hipStreamIsCapturing failed");
    }
    if (status != hipStreamCaptureStatusNone)
      return attnres_internal_fail(ATTNRES_ERR_ARG,
                                   "attnres_route_bwd_noalloc called under stream capture before set-up: call "
                                   "attnres_init() on this device before capturing");
  }
  if (p == nullptr) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr) {
        (void)hipGetLastError();
        return attnres_internal_fail(ATTNRES_ERR_HIP, "hipGetSymbolAddress(scratch) failed");
      }
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return ATTNRES_OK;
}

}  // namespace

// Set-up for the current device, called by attnres_init().
extern "C" __attribute__((visibility("hidden"))) int attnres_internal_scratch_setup(void) {
  void* p = nullptr;
  return scratch_for_current_device(&p);
}

extern "C" int attnres_route_bwd_noalloc(const void* const* sources, int num_sources, int64_t num_tokens, int hidden,
                                         int64_t src_ld, int src_dtype, const void* query, const void* gain,
                                         int param_dtype, float eps, const void* grad_out, int grad_out_dtype,
                                         int64_t grad_out_ld, const float* grad_lse, void* const* grad_sources,
                                         int64_t grad_ld, void* grad_query, void* grad_gain, void* stream) {
  if (num_tokens < 0 || hidden <= 0) return attnres_internal_fail(ATTNRES_ERR_ARG, "bad num_tokens/hidden");
  if (num_tokens == 0) {
    // attnres_route_bwd returns before any HIP call; so does this.
    return attnres_route_bwd(sources, num_sources, num_tokens, hidden, src_ld, src_dtype, query, gain, param_dtype,
                             eps, grad_out, grad_out_dtype, grad_out_ld, grad_lse, grad_sources, grad_ld, nullptr, 0,
                             grad_query, grad_gain, stream);
  }
  int64_t need = 0;
  int rc = attnres_route_bwd_workspace_size(num_tokens, hidden, &need);
  if (rc != ATTNRES_OK) return rc;
  if (need > (int64_t)ATTNRES_NOALLOC_SCRATCH_BYTES)
    return attnres_internal_fail(ATTNRES_ERR_UNSUPPORTED,
                                 "the backward needs more workspace than the fixed scratch array "
                                 "(ATTNRES_NOALLOC_SCRATCH_BYTES); use attnres_route_bwd");
  void* ws = nullptr;
  rc = scratch_for_current_device(&ws, static_cast<hipStream_t>(stream), true);
  if (rc != ATTNRES_OK) return rc;
  return attnres_route_bwd(sources, num_sources, num_tokens, hidden, src_ld, src_dtype, query, gain, param_dtype, eps,
                           grad_out, grad_out_dtype, grad_out_ld, grad_lse, grad_sources, grad_ld, ws,
                           (int64_t)ATTNRES_NOALLOC_SCRATCH_BYTES, grad_query, grad_gain, stream);
}
