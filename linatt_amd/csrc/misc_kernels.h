// Internal launch interface of the small helper kernels: row L2 norm, the
// mixer's short convolution and RMSNorm.
#pragma once

#include <hip/hip_runtime.h>

namespace linatt {

template <typename T>
hipError_t launch_l2norm_fwd(const void* x, void* y, float* rstd, int n, int d, float eps,
                             hipStream_t s);
template <typename T>
hipError_t launch_l2norm_bwd(const void* y, const float* rstd, const void* dy, void* dx, int n,
                             int d, hipStream_t s);

// Causal depthwise short convolution (mixer.hip).  part / dw / db: backward
// only (partials workspace, weight and bias gradients).
struct ConvArgs {
  const void* x;         // (B, T, C)
  const float* w;        // (C, W)
  const float* bias;     // (C) or null
  const void* cache_in;  // (B, C, W) inputs before position 0 (newest last), or null
  void* y;               // (B, T, C)
  void* cache_out;       // (B, C, W) the W inputs before position T, or null
  const void* dy;
  void* dx;
  float* part;
  float* dw;
  float* db;
  int B, T, C, act;
};
template <typename T>
hipError_t launch_short_conv(const ConvArgs& a, int W, bool bwd, hipStream_t stream);
size_t short_conv_bwd_workspace(int B, int T, int C, int W);

// Fused q/k prologue (mixer.hip): short convolution + activation, per-head
// norm, rotary embedding, over (B, T, C = H D).
struct QKArgs {
  const void* x;         // (B, T, C) the projection output
  const float* w;        // (C, W) convolution weight
  const float* bias;     // (C) or null
  const void* cache_in;  // (B, C, W) or null
  const float* nw;       // (D) RMSNorm weight or null
  void* y;               // (B, T, H, D)
  void* cache_out;       // (B, C, W) or null
  const void* dy;
  void* dx;
  float* part;    // convolution weight / bias partials, then their sums
  float* npart;   // norm weight partials
  float* dw;
  float* db;
  float* dnw;
  int B, T, C, D, act, norm;  // norm: 0 none, 1 RMSNorm, 2 L2
  float eps, inv_n;           // r = (inv_n sum u^2 + eps)^-1/2
  int rw, rot, interleaved, offset;  // rotation rows of rw dims, first rot rotated; rot = 0: none
  float log2_base;
};
template <typename T>
hipError_t launch_qk_prologue(const QKArgs& a, int W, bool bwd, hipStream_t stream);
size_t qk_prologue_bwd_workspace(int B, int T, int C, int D, int W);

// RMSNorm over rows of d (mixer.hip): forward (out = y, rstd_out) or
// backward (out = dx, dw with the partials workspace).
template <typename T>
hipError_t launch_rmsnorm(const void* x, const float* w, const float* rstd_in, const void* dy,
                          void* out, float* rstd_out, float* dw, float* part, int n, int d,
                          float eps, bool bwd, hipStream_t stream);
int rmsnorm_bwd_blocks(int n, int d);

// Rotary position embedding over (B, T, H, D) rows (mixer.hip).
template <typename T>
hipError_t launch_rope(const void* x, void* y, int B, int T_, int H, int D, int rot_dim, float base,
                       int offset, int interleaved, int inverse, hipStream_t stream);

// Causal linear attention, chunked state form (linear_scan.hip); head-major,
// D = DV = 64, 16-bit types.
template <typename T>
hipError_t launch_linear_scan(const void* q, const void* k, const void* v, void* o, float* den, int B,
                              int H, int T_, float scale, float eps, hipStream_t stream);

// Column sums out[i] = sum_p part[p][i] of a (np, n) float32 array in a
// fixed order (mixer.hip).
hipError_t launch_colsum(const float* part, float* out, int np, int n, hipStream_t stream);

// Sets the calling thread's linatt_last_error() message and returns code
// (defined with the C-ABI entry points in api.hip).
int set_last_error(int code, const char* msg);

}  // namespace linatt
