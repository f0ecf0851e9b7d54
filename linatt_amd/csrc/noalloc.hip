// linatt_kata_bwd_noalloc: the KATA backward with its workspace taken from a
// fixed device array instead of a caller buffer, for callers that cannot
// allocate (code under HIP graph capture, serving loops, harnesses that
// forbid hipMalloc).  It has no counterpart in the reference.
//
// The array lives in this file's code object, one copy per device, from the
// first use on that device until the process ends.  Its device address comes
// from hipGetSymbolAddress once per device (the host-side name of a
// __device__ array is not a device address and must never reach a kernel).
// The dq kernel writes every byte of the workspace region the dk/dv kernel
// reads, so nothing is cleared between calls.  All calls on one device share
// the array: calls that overlap on one device (two streams, two threads)
// race and must be serialised by the caller.
#include <mutex>
#include <string>

#include "linatt_hip.h"
#include "misc_kernels.h"

namespace {

static __device__ __align__(256) unsigned char scratch[LINATT_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's copy of `scratch` (looked up once per
// device, with that device current); nullptr and a message on failure.
void* scratch_for_current_device(std::string* err) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *err = std::string("hipGetDevice failed: ") + hipGetErrorString(e);
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *err = "device index " + std::to_string(dev) + " out of range";
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      *err = std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e);
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" size_t linatt_noalloc_scratch_bytes(void) { return LINATT_NOALLOC_SCRATCH_BYTES; }

extern "C" int linatt_kata_bwd_noalloc(const void* q, const void* k, const void* v,
                                       const void* o, const float* den, const void* dout,
                                       void* dq, void* dk, void* dv, int B, int T, int HQ, int H,
                                       int dk_dim, int dv_dim, int num_groups, float scale,
                                       int variant, int dtype, void* stream) {
  // the size check comes first: an oversized call fails before any HIP call
  const size_t need = linatt_kata_bwd_workspace_bytes(B, T, HQ, dv_dim, dtype);
  if (need == 0)
    return linatt::set_last_error(LINATT_EINVAL, "linatt_kata_bwd_noalloc: non-positive dimension");
  if (need > (size_t)LINATT_NOALLOC_SCRATCH_BYTES) {
    const std::string msg = "linatt_kata_bwd_noalloc: workspace of " + std::to_string(need) +
                            " bytes exceeds the fixed scratch of " +
                            std::to_string((size_t)LINATT_NOALLOC_SCRATCH_BYTES) +
                            " bytes; use linatt_kata_bwd with a caller workspace";
    return linatt::set_last_error(LINATT_EINVAL, msg.c_str());
  }
  std::string err;
  void* ws = scratch_for_current_device(&err);
  if (!ws) return linatt::set_last_error(LINATT_ELAUNCH, ("linatt_kata_bwd_noalloc: " + err).c_str());
  return linatt_kata_bwd(q, k, v, o, den, dout, dq, dk, dv, ws, B, T, HQ, H, dk_dim, dv_dim,
                         num_groups, scale, variant, dtype, stream);
}
