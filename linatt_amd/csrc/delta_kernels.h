// Internal launch interface between the C-ABI layer (api.hip) and the
// chunked (gated) delta-rule kernels.  Not part of the public header.
//
// Shapes: B batch, T tokens, H heads, DK key dim, DV value dim, chunks of
// 64 tokens, NT = ceil(T / 64), Tp = 64 * NT.  q, k, v, o and their
// gradients are time-major (B, T, H, D); beta, g, dbeta, dg are (B, T, H)
// float32; states (B, H, DK, DV) float32.  Everything else lives in the
// context / workspace buffers carved by delta_layout().  "Operand order"
// (opord32 in common.h) permutes each 32-element block so that the MFMA
// operand a lane needs is one contiguous 16-byte load.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace linatt {

constexpr int kChunk = 64;

// Byte offsets of the forward context (kept from forward to backward) and of
// the backward scratch.  Sub-buffers are 256-byte aligned.
struct DeltaLayout {
  // context (written by the forward, read by the backward)
  size_t Gc;    // (B,H,Tp) f32  chunk-local inclusive cumsum of g (gated only)
  size_t Fk;    // (B,H,Tp) f32  e^(gamma - G_i), gamma = G at the chunk's last row (gated only)
  size_t Tm;    // (B,H,NT,64,64) T  (I + A)^-1, natural [i][j]
  size_t W;     // (B,H,Tp,DK) T  W = Tm diag(beta e^G) K
  size_t UT;    // (B,H,NT,DV,64) T  (Tm diag(beta) V)^T per chunk, rows i in operand order
  size_t KdT;   // (B,H,NT,DK,64) T  (e^(gamma - G_i) k_i)^T per chunk, rows i in operand order (gated only)
  size_t Qg;    // (B,H,Tp,DK) T  scale e^G_i q_i (zero past T; gated only)
  size_t Aqk;   // (B,H,NT,64,64) T  scale (q_i.k_j) e^(G_i-G_j) [j <= i]
  size_t hT;    // (B,H,NT,DV,DK) T  state entering each chunk, transposed [v][d]
  size_t VnT;   // (B,H,NT,DV,64) T  v_new^T per chunk, v_new = U - W h
  size_t ctx_bytes;
  // backward scratch
  size_t dVnT;  // (B,H,NT,DV,64) T  gradient of v_new, transposed
  size_t dhT;   // (B,H,NT,DV,DK) T  gradient of the state leaving each chunk, transposed
  size_t bwd_bytes;
};

DeltaLayout delta_layout(int B, int T, int H, int DK, int DV, int elt_bytes);

// Workgroups per head of the two state passes: the value columns of a head
// are split over this many workgroups (each on its own CU: one compute wave
// per 32 columns plus a copy wave), so the copy and store traffic of the
// serial chain spreads over that many CUs.  Measured at K = V = 128: one
// compute wave per workgroup beats two and four.
template <int DV>
constexpr int state_split() { return DV / 32; }
// Copy waves per workgroup of the state passes: one wave alone issues L2 ->
// LDS copies at about a third of what a CU takes in (44 against 125 GB/s
// per CU in a probe), so the copies of a chunk are split over two.
constexpr int kStateCopyWaves = 2;
// Threads of a forward state-pass workgroup: the compute wave, the copy
// waves and one output wave, which forms the output rows of each chunk from
// the states the compute wave staged for the copy waves' stores.
template <int DV>
constexpr int state_threads() { return 64 * (DV / 32 / state_split<DV>() + kStateCopyWaves + 1); }

struct DeltaArgs {
  // inputs
  const void* q;
  const void* k;
  const void* v;
  const float* beta;
  const float* g;     // null: ungated (DeltaNet)
  const float* h0;    // null: zero initial state
  const void* dout;   // backward
  const float* dht;   // backward, null: no gradient on the final state
  // outputs
  void* o;
  float* ht;          // null: final state not requested
  void* dq;
  void* dk;
  void* dv;
  float* dbeta;
  float* dg;
  float* dh0;         // null: no initial-state gradient
  // context / scratch base pointers (offsets from DeltaLayout)
  char* ctx;
  char* ws;
  int B, T, H, NT;
  float scale;
  // kernels to launch, in order: forward bit 0 prep, 1 state pass, 2 output;
  // backward bit 0 state pass, 1 chunk kernel
  int stages;
};

template <typename T, int DK, int DV, bool GATED>
hipError_t launch_delta_fwd(const DeltaArgs& a, hipStream_t stream);

template <typename T, int DK, int DV, bool GATED>
hipError_t launch_delta_bwd(const DeltaArgs& a, hipStream_t stream);

// Compiled (dtype, DK, DV) combinations; each for the plain and gated rule.
#define LINATT_DELTA_SHAPES(X) \
  X(__bf16, 128, 128)          \
  X(__bf16, 64, 64)            \
  X(_Float16, 128, 128)        \
  X(_Float16, 64, 64)

}  // namespace linatt
