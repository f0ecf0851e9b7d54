// Row L2 normalisation y = x / sqrt(sum x^2 + eps) and its backward
// dx = rstd (dy - y <y, dy>), for the q/k normalisation fla applies inside
// its delta-rule kernels when use_qk_l2norm_in_kernel=True (third-party
// flash-linear-attention==0.5.0, scripts/setup.sh:27 of the reference;
// DeltaNet configs set qk_norm: l2, configs/model/200m/delta_net_200m.yaml:13).
// One wave per row, fp32 arithmetic.
#include "common.h"
#include "misc_kernels.h"

namespace linatt {

template <typename T>
__global__ __launch_bounds__(256) void l2norm_fwd_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                         float* __restrict__ rstd, int n, int d,
                                                         float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= n) return;
  const T* xr = x + (int64_t)row * d;
  float ss = 0.f;
  for (int e = lane; e < d; e += 64) {
    const float xv = (float)xr[e];
    ss += xv * xv;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  const float r = rsqrtf(ss + eps);
  T* yr = y + (int64_t)row * d;
  for (int e = lane; e < d; e += 64) yr[e] = (T)((float)xr[e] * r);
  if (lane == 0) rstd[row] = r;
}

template <typename T>
__global__ __launch_bounds__(256) void l2norm_bwd_kernel(const T* __restrict__ y,
                                                         const float* __restrict__ rstd,
                                                         const T* __restrict__ dy,
                                                         T* __restrict__ dx, int n, int d) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= n) return;
  const T* yr = y + (int64_t)row * d;
  const T* gr = dy + (int64_t)row * d;
  float dot = 0.f;
  for (int e = lane; e < d; e += 64) dot += (float)yr[e] * (float)gr[e];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) dot += __shfl_xor(dot, off);
  const float r = rstd[row];
  T* xr = dx + (int64_t)row * d;
  for (int e = lane; e < d; e += 64) xr[e] = (T)(r * ((float)gr[e] - (float)yr[e] * dot));
}

template <typename T>
hipError_t launch_l2norm_fwd(const void* x, void* y, float* rstd, int n, int d, float eps,
                             hipStream_t s) {
  l2norm_fwd_kernel<T><<<dim3((n + 3) / 4), dim3(256), 0, s>>>((const T*)x, (T*)y, rstd, n, d, eps);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_l2norm_bwd(const void* y, const float* rstd, const void* dy, void* dx, int n,
                             int d, hipStream_t s) {
  l2norm_bwd_kernel<T><<<dim3((n + 3) / 4), dim3(256), 0, s>>>((const T*)y, rstd, (const T*)dy,
                                                               (T*)dx, n, d);
  return hipGetLastError();
}

#define LINATT_L2_INST(T)                                                                       \
  template hipError_t launch_l2norm_fwd<T>(const void*, void*, float*, int, int, float, hipStream_t); \
  template hipError_t launch_l2norm_bwd<T>(const void*, const float*, const void*, void*, int, int, \
                                           hipStream_t);
LINATT_L2_INST(__bf16)
LINATT_L2_INST(_Float16)
LINATT_L2_INST(float)

}  // namespace linatt
