// Internal launch interface between the C-ABI layer (api.hip) and the KATA
// kernels.  Not part of the public header.
#pragma once

#include <hip/hip_runtime.h>

namespace linatt {

// Byte offset of the prescaled dO (bf16) in the backward workspace, after the
// two per-row float arrays of nrows = B T HQ rows each.
__host__ __device__ inline size_t kata_dop_offset(int64_t nrows) {
  return ((size_t)nrows * 2 * sizeof(float) + 255) & ~(size_t)255;
}

struct KataArgs {
  const void* q;     // (B, T, HQ, DK) time-major, contiguous
  const void* k;     // (B, T, H, DK)
  const void* v;     // (B, T, H, DV)
  const float* c;    // (B, T, HQ) cumulative log-decay, or null
  void* o;           // (B, T, HQ, DV); backward: null reads as zero (delta = 0; internal callers)
  float* den;        // (B, T, HQ)
  const void* dout;  // (B, T, HQ, DV) upstream gradient (backward only)
  void* dq;          // (B, T, HQ, DK)
  void* dk;          // (B, T, H, DK)
  void* dv;          // (B, T, H, DV)
  float* delta;      // workspace: (2, B, T, HQ) per-row -<o, dO> (bf16: times scale^2 / den)
                     // and scale^2 / den; bf16: then dO scale^2 / den (B, T, HQ, DV)
  float* dc;         // (B, T, HQ) gradient of the cumulative log-decay c (decay backward)
  int B, T, HQ, H, DK, DV, M;
  float scale;
  // output RMSNorm over each (b, t, hq) row of o (16-bit 64 x 64 tile
  // kernels only): the forward writes y and rstd beside o and den when y is
  // set; the backward takes dy instead of dO when dy is set
  const float* nw;   // (DV) norm weight, or null (weight 1)
  void* y;           // (B, T, HQ, DV) normalised output, or null
  float* rstd;       // (B, T, HQ) (mean(o^2) + eps)^-1/2: forward writes, backward reads
  float eps;
  const void* dy;    // (B, T, HQ, DV) gradient of y, or null
  float* nw_part;    // (nqt B HQ, DV) per-workgroup weight-gradient partials (dq pass)
  // forward, 16-bit 64 x 64 tile kernels: when set, the unnormalised
  // numerator num = o den = sum_s A[t,s] v_s is written here in float32
  // instead of o (o may then be null)
  float* num32;
};

// The output-norm arguments of the tile kernels (a kernel argument struct).
struct OutNorm {
  const float* w;
  void* y;        // forward: normalised output; backward: dy
  float* rstd;
  float* part;    // backward: weight-gradient partials, or null
  float eps;
  float* num;     // forward: float32 numerator instead of o, or null
};

template <typename T, int DK, int DV, int M, bool SUM, bool DECAY>
hipError_t launch_kata_fwd(const KataArgs& a, hipStream_t stream);

// parts: bit 0 = dq kernel (also writes the per-row workspace), bit 1 = dk/dv kernel (reads it)
enum { KATA_BWD_DQ = 1, KATA_BWD_DKDV = 2 };

template <typename T, int DK, int DV, int M, bool SUM, bool DECAY>
hipError_t launch_kata_bwd(const KataArgs& a, int parts, hipStream_t stream);

// Compiled (dtype, DK, DV, M) combinations.  Each is built for the concat
// and sum scores and, forward and backward, for the decayed concat score.
// (128, 64, 2) is the shape of the offset-gated mixer (kata/layer.py:237-281:
// each group of E = 32 padded to 64, so dk = 128 for dv = 64 at M = 2), which
// is also the one decayed configuration (configs/model/
// kataconv_cat_l2_gdn_340m.yaml:12,18-19).
#define LINATT_KATA_SHAPES(X) \
  X(__bf16, 64, 64, 1)        \
  X(__bf16, 64, 64, 2)        \
  X(__bf16, 64, 64, 4)        \
  X(__bf16, 128, 64, 2)       \
  X(_Float16, 64, 64, 1)      \
  X(_Float16, 64, 64, 2)      \
  X(_Float16, 64, 64, 4)      \
  X(_Float16, 128, 64, 2)     \
  X(float, 64, 64, 1)         \
  X(float, 64, 64, 2)         \
  X(float, 64, 64, 4)         \
  X(float, 128, 64, 2)

}  // namespace linatt

namespace linatt {

// Long-context prefill in psi-state form and the recurrent decode step.
// Element strides (in elements) describe q/k (sb, st, sh), v (vsb, vst, vsh)
// and o (osb, ost, osh), so time-major and head-major inputs both work.
struct KataStateArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* den;          // (B, T, H) or strided like o without the feature dim
  int64_t sb, st, sh, vsb, vst, vsh, osb, ost, osh, dsb, dst, dsh;
  float* seg_S;        // (B*H, nseg, DV, 3P/4) f32 scratch, per-segment Psi(K)^T V transposed, packed rows
  float* seg_z;        // (B*H, nseg, P) f32 scratch
  void* HT;            // (B*H, nseg, DV, 3P/4) T scratch, weighted exclusive prefix (unscaled), packed rows
  float* Hz;           // (B*H, nseg, P) f32 scratch
  float* S_out;        // (B, H, P, DV) f32 final state psi(sqrt(scale) k) v^T, or null
  float* z_out;        // (B, H, P) f32, or null
  const float* S_in;   // (B, H, P, DV) f32 state before the first token (may alias S_out), or null
  const float* z_in;   // (B, H, P) f32 (may alias z_out), or null; set together with S_in
  int B, T, H, L, nseg;
  float scale, scale2, eps;
  // layout of S_in / z_in / S_out / z_out: 0 full (P rows), 1 packed
  // (the M E (E + 1) / 2 rows a <= b of each group; kata_state_tri_row)
  int tri;
};

// Packed state row of pair (a, b), a <= b, of group g (groups of width E):
// the upper triangle of each group, row by row.  The state rows p = g E^2 +
// a E + b and g E^2 + b E + a of the full layout both map here (psi(x) is
// symmetric in a and b).
__host__ __device__ inline int kata_state_tri_row(int E, int g, int a, int b) {
  return g * (E * (E + 1) / 2) + a * E - a * (a - 1) / 2 + (b - a);
}

template <typename T, int DK, int DV, int M>
hipError_t launch_kata_prefill(const KataStateArgs& a, hipStream_t stream);

// n floats from src to dst on the stream (a small copy kernel)
hipError_t launch_f32_copy(const float* src, float* dst, int64_t n, hipStream_t stream);

constexpr int kGenDecPart = 68;     // floats per decode partial: num[64], den, padding
constexpr int kGenDecMaxSplit = 16;  // workgroups per (b, h) of a split decode step
// workgroups per (b, h) for a decode step over P state rows: about 768 in all,
// at least 64 rows each; a state of fewer than 512 rows is not split (its
// step is short anyway, and the second launch would cost more than it saves)
inline int kata_gen_decode_splits(int BH, int P) {
  if (P < 512) return 1;
  int ns = (768 + BH - 1) / BH;
  if (ns > P / 64) ns = P / 64;
  if (ns > kGenDecMaxSplit) ns = kGenDecMaxSplit;
  return ns < 1 ? 1 : ns;
}

struct KataDecodeArgs {
  const void* q;   // (B, H, DK)
  const void* k;
  const void* v;   // (B, H, DV)
  void* o;         // (B, H, DV)
  float* S;        // (B, H, P, DV) f32, updated in place (tri: (B, H, M E (E + 1) / 2, DV))
  float* z;        // (B, H, P) f32, updated in place (tri: (B, H, M E (E + 1) / 2))
  int B, H;
  float scale, eps;
  int tri;         // packed state layout (kata_state_tri_row)
  int nsplit;      // workgroups per (b, h) (1: o written directly)
  float* part;     // nsplit > 1: (B*H, nsplit, kGenDecPart) partial num (64) and den
};

template <typename T, int DK, int DV, int M>
hipError_t launch_kata_decode(const KataDecodeArgs& a, hipStream_t stream);

// The state form of every flash score (kata_state_gen.hip): concat or sum
// features, optional decay, dk <= 128, dv = 64, fp32 state (B, H, P, 64).
struct KataGenStateArgs {
  const void* q;     // decode: (B, H, dk); readout: (B, T, H, dk)
  const void* k;     // decode: (B, H, dk); update: (B, T, H, dk)
  const void* v;     // decode: (B, H, 64); update: (B, T, H, 64)
  const float* c;    // decode: (B, H) the step's log-decay; else (B, T, H) cumulative in the call; or null
  float* S;          // (B, H, P, 64)
  float* z;          // (B, H, P)
  void* o;           // decode: (B, H, 64) out; readout: (B, T, H, 64) in (flash) and out
  float* den;        // readout: (B, T, H) in (flash) and out
  int B, T, H, dk, E, lgE, M, P, sum;
  int tri;           // 1: packed rows, one per unordered pair a <= b of each group
  int TE;            // packed rows per group, E (E + 1) / 2
  int nsplit;        // decode: workgroups per (b, h) (1: o written directly)
  float* part;       // decode, nsplit > 1: (B*H, nsplit, kGenDecPart) partial num (64) and den
  float scale, eps;
  int init;          // update: 1 = add to f_T S, 0 = start from zero
};
enum { KATA_GEN_DECODE = 0, KATA_GEN_READOUT = 1, KATA_GEN_UPDATE = 2 };

template <typename T>
hipError_t launch_kata_gen_state(const KataGenStateArgs& a, int which, hipStream_t stream);

// Compiled (dtype, DK, DV, M) combinations of the state form.
#define LINATT_KATA_STATE_SHAPES(X) \
  X(__bf16, 64, 64, 4)              \
  X(__bf16, 64, 64, 2)

}  // namespace linatt

namespace linatt {

// SPD delta rule (DeltaKata) forward: workspace layout (byte offsets) and
// launch arguments.
struct DKataLayout {
  size_t TmHi, TmLo;  // (B*H, NC, 64, 64) T: Tm = (I + N)^-1 per chunk, hi + lo
  size_t UT;          // (B*H, DV, 64 NC) T: U^T
  size_t Ub;          // (B, T, H, DV) T: U for the readout
  size_t Ein;         // (B, T, H, DV) f32: sum over earlier chunks of kappa(k_t, k_j) U_j
  size_t bytes;
};
DKataLayout dkata_layout(int B, int T, int H, int D, int DV, int eb);

// Backward scratch of the SPD delta rule, after the forward's workspace.
struct DKataBwdLayout {
  size_t dOp;   // (B, T, H, DV) T: do' = do / (den + eps) (or do)
  size_t O16;   // (B, T, H, DV) T: the normalised output (normalize only)
  size_t ones;  // (B, T, H) f32: 1, the KATA backward's den
  size_t kws;   // KATA backward workspace
  size_t dU;    // (B, T, H, DV) T: readout VJP, KATA backward's dv
  size_t dkr;   // (B, T, H, D) T: readout part of dk
  size_t Ksh;   // (B, T, H, D) T: k one token later (zero at T - 1), the erase pass's q
  size_t Xn;    // (B, T, H, DV) T: -beta dbV one token later (zero at T - 1), its dO
  size_t XT;    // (B*H, DV, 64 NC) T: (beta dbV)^T for the reverse solve
  size_t dbV;   // (B, T, H, DV) f32
  size_t dqe, dke, dve;  // erase pass outputs (T)
  size_t bytes;
};
DKataBwdLayout dkata_bwd_layout(int B, int T, int H, int D, int DV, int eb);

struct DKataArgs {
  const void* q;      // (B, T, H, D) time-major
  const void* k;
  const void* v;      // (B, T, H, DV)
  const float* beta;  // (B, T, H)
  float* U;           // (B, T, H, DV) f32 pseudo-values, or null
  float* o;           // (B, T, H, DV) f32
  float* den;         // (B, T, H) f32
  char* ws;
  DKataLayout L;
  int B, T, H;
  float scale, scale2, eps;
  int normalize;
  int keep_e;  // forward: also store Ein (for the backward)
};

struct DKataBwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* beta;
  const float* U;     // (B, T, H, DV) f32 from the forward
  const float* o;     // (B, T, H, DV) f32 forward output (normalize), else null
  const float* den;   // (B, T, H) f32 from the forward
  const float* dout;  // (B, T, H, DV) f32
  void* dq;           // (B, T, H, D) T
  void* dk;
  void* dv;           // (B, T, H, DV) T
  float* dbeta;       // (B, T, H) f32
  char* ws;           // the forward's workspace (kept) ...
  DKataLayout L;
  char* bws;          // ... and the backward's
  DKataBwdLayout BL;
  int B, T, H;
  float scale, scale2, eps;
  int normalize;
};

template <typename T, int D, int DV, int M>
hipError_t launch_dkata_bwd(const DKataBwdArgs& a, hipStream_t stream);

template <typename T, int D, int DV, int M>
hipError_t launch_dkata_fwd(const DKataArgs& a, hipStream_t stream);

// Compiled (dtype, D, DV, M) combinations of the SPD delta rule.
#define LINATT_DKATA_SHAPES(X) \
  X(__bf16, 64, 64, 1)         \
  X(__bf16, 64, 64, 2)         \
  X(__bf16, 64, 64, 4)         \
  X(_Float16, 64, 64, 1)       \
  X(_Float16, 64, 64, 2)       \
  X(_Float16, 64, 64, 4)

}  // namespace linatt
