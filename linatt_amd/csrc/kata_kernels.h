// Internal launch interface between the C-ABI layer (api.hip) and the KATA
// kernels.  Not part of the public header.
#pragma once

#include <hip/hip_runtime.h>

namespace linatt {

struct KataArgs {
  const void* q;     // (B, T, HQ, DK) time-major, contiguous
  const void* k;     // (B, T, H, DK)
  const void* v;     // (B, T, H, DV)
  const float* c;    // (B, T, HQ) cumulative log-decay, or null
  void* o;           // (B, T, HQ, DV)
  float* den;        // (B, T, HQ)
  const void* dout;  // (B, T, HQ, DV) upstream gradient (backward only)
  void* dq;          // (B, T, HQ, DK)
  void* dk;          // (B, T, H, DK)
  void* dv;          // (B, T, H, DV)
  float* delta;      // (B, T, HQ) workspace: <o, dO> per row
  int B, T, HQ, H, DK, DV, M;
  float scale;
};

template <typename T, int DK, int DV, int M, bool SUM, bool DECAY>
hipError_t launch_kata_fwd(const KataArgs& a, hipStream_t stream);

// parts: bit 0 = dq kernel (also writes delta), bit 1 = dk/dv kernel (reads delta)
enum { KATA_BWD_DQ = 1, KATA_BWD_DKDV = 2 };

template <typename T, int DK, int DV, int M, bool SUM>
hipError_t launch_kata_bwd(const KataArgs& a, int parts, hipStream_t stream);

// Compiled (dtype, DK, DV, M) combinations.  Each is built for the concat
// and sum scores; the forward also for the decayed concat score.
#define LINATT_KATA_SHAPES(X) \
  X(__bf16, 64, 64, 1)        \
  X(__bf16, 64, 64, 2)        \
  X(__bf16, 64, 64, 4)        \
  X(_Float16, 64, 64, 1)      \
  X(_Float16, 64, 64, 2)      \
  X(_Float16, 64, 64, 4)      \
  X(float, 64, 64, 1)         \
  X(float, 64, 64, 2)         \
  X(float, 64, 64, 4)

}  // namespace linatt
