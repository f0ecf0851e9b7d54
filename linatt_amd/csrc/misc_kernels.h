// Internal launch interface of the small helper kernels (row L2 norm).
#pragma once

#include <hip/hip_runtime.h>

namespace linatt {

template <typename T>
hipError_t launch_l2norm_fwd(const void* x, void* y, float* rstd, int n, int d, float eps,
                             hipStream_t s);
template <typename T>
hipError_t launch_l2norm_bwd(const void* y, const float* rstd, const void* dy, void* dx, int n,
                             int d, hipStream_t s);

// Sets the calling thread's linatt_last_error() message and returns code
// (defined with the C-ABI entry points in api.hip).
int set_last_error(int code, const char* msg);

}  // namespace linatt
