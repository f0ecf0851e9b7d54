// C-ABI entry points: argument validation, dispatch to the compiled kernel
// instantiations, and per-thread error reporting.  See include/linatt_hip.h.
#include <cstdint>
#include <cstdio>
#include <string>

#include "linatt_hip.h"
#include "delta_kernels.h"
#include "kata_kernels.h"
#include "misc_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

template <typename T> constexpr int dtype_of();
template <> constexpr int dtype_of<float>() { return LINATT_FLOAT32; }
template <> constexpr int dtype_of<__bf16>() { return LINATT_BFLOAT16; }
template <> constexpr int dtype_of<_Float16>() { return LINATT_FLOAT16; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// the convolution kernels write cache_out from the block holding token T - 1
// while the block of tokens 0..15 reads cache_in: with more than one 16-token
// run the two must not share memory (one run reads its halo before it writes)
bool cache_races(const void* cache_in, const void* cache_out, int B, int C, int W, int T,
                 int dtype) {
  if (!cache_in || !cache_out || T <= 16) return false;
  const size_t n = (size_t)B * C * W * (dtype == LINATT_FLOAT32 ? 4 : 2);
  const uintptr_t i0 = reinterpret_cast<uintptr_t>(cache_in), o0 = reinterpret_cast<uintptr_t>(cache_out);
  return i0 < o0 + n && o0 < i0 + n;
}

std::string shape_str(int B, int T, int HQ, int H, int dk, int dv, int M) {
  char buf[160];
  snprintf(buf, sizeof buf, "B=%d T=%d HQ=%d H=%d dk=%d dv=%d num_groups=%d", B, T, HQ, H, dk,
           dv, M);
  return buf;
}

int check_common(int B, int T, int HQ, int H, int dk, int dv, int M, float scale, int variant,
                 int dtype) {
  const std::string s = shape_str(B, T, HQ, H, dk, dv, M);
  if (B <= 0 || T <= 0 || HQ <= 0 || H <= 0 || dk <= 0 || dv <= 0 || M <= 0)
    return fail(LINATT_EINVAL, "linatt: non-positive dimension (" + s + ")");
  if (HQ % H != 0) return fail(LINATT_EINVAL, "linatt: GQA requires HQ % H == 0 (" + s + ")");
  if (dk % M != 0) return fail(LINATT_EINVAL, "linatt: dk not divisible by num_groups (" + s + ")");
  if (!(scale > 0.f)) return fail(LINATT_EINVAL, "linatt: scale must be positive");
  if (variant != LINATT_KATA_CONCAT && variant != LINATT_KATA_SUM)
    return fail(LINATT_EINVAL, "linatt: unknown KATA variant");
  if (dtype != LINATT_FLOAT32 && dtype != LINATT_BFLOAT16 && dtype != LINATT_FLOAT16)
    return fail(LINATT_EINVAL, "linatt: unknown dtype");
  if ((int64_t)B * T * HQ > (int64_t)INT32_MAX / 2)
    return fail(LINATT_EINVAL, "linatt: B*T*HQ too large");
  return LINATT_OK;
}

}  // namespace

int linatt::set_last_error(int code, const char* msg) { return fail(code, msg); }

namespace {

using namespace linatt;

// Returns 1 and sets *err when a kernel exists for the combination (one
// group of the sum form runs the concat kernels: launch_kata_fwd / _bwd).
hipError_t dispatch_fwd(const KataArgs& a, int dtype, int variant, bool decay, hipStream_t s,
                        bool* found) {
  *found = false;
#define LINATT_TRY_FWD(T, DK_, DV_, M_)                                             \
  if (dtype == dtype_of<T>() && a.DK == DK_ && a.DV == DV_ && a.M == M_) {          \
    *found = true;                                                                  \
    if (decay) return launch_kata_fwd<T, DK_, DV_, M_, false, true>(a, s);           \
    if (variant == LINATT_KATA_SUM) return launch_kata_fwd<T, DK_, DV_, M_, true, false>(a, s); \
    return launch_kata_fwd<T, DK_, DV_, M_, false, false>(a, s);                    \
  }
  LINATT_KATA_SHAPES(LINATT_TRY_FWD)
#undef LINATT_TRY_FWD
  return hipSuccess;
}

hipError_t dispatch_bwd(const KataArgs& a, int parts, int dtype, int variant, bool decay,
                        hipStream_t s, bool* found) {
  *found = false;
#define LINATT_TRY_BWD(T, DK_, DV_, M_)                                             \
  if (dtype == dtype_of<T>() && a.DK == DK_ && a.DV == DV_ && a.M == M_) {          \
    *found = true;                                                                  \
    if (decay) return launch_kata_bwd<T, DK_, DV_, M_, false, true>(a, parts, s);    \
    if (variant == LINATT_KATA_SUM) return launch_kata_bwd<T, DK_, DV_, M_, true, false>(a, parts, s); \
    return launch_kata_bwd<T, DK_, DV_, M_, false, false>(a, parts, s);             \
  }
  LINATT_KATA_SHAPES(LINATT_TRY_BWD)
#undef LINATT_TRY_BWD
  return hipSuccess;
}

bool compiled(int dtype, int dk, int dv, int M) {
#define LINATT_HAS(T, DK_, DV_, M_) \
  if (dtype == dtype_of<T>() && dk == DK_ && dv == DV_ && M == M_) return true;
  LINATT_KATA_SHAPES(LINATT_HAS)
#undef LINATT_HAS
  return false;
}

bool delta_compiled(int dtype, int dk, int dv) {
#define LINATT_HAS_D(T, DK_, DV_) \
  if (dtype == dtype_of<T>() && dk == DK_ && dv == DV_) return true;
  LINATT_DELTA_SHAPES(LINATT_HAS_D)
#undef LINATT_HAS_D
  return false;
}

hipError_t dispatch_delta(const DeltaArgs& a, int dtype, int dk, int dv, bool gated, bool bwd,
                          hipStream_t s) {
#define LINATT_TRY_D(T, DK_, DV_)                                                         \
  if (dtype == dtype_of<T>() && dk == DK_ && dv == DV_) {                                 \
    if (bwd) return gated ? launch_delta_bwd<T, DK_, DV_, true>(a, s)                    \
                          : launch_delta_bwd<T, DK_, DV_, false>(a, s);                  \
    return gated ? launch_delta_fwd<T, DK_, DV_, true>(a, s) : launch_delta_fwd<T, DK_, DV_, false>(a, s); \
  }
  LINATT_DELTA_SHAPES(LINATT_TRY_D)
#undef LINATT_TRY_D
  return hipErrorInvalidValue;
}

int elt_bytes(int dtype) { return dtype == LINATT_FLOAT32 ? 4 : 2; }

bool state_compiled(int dtype, int dk, int dv, int M) {
#define LINATT_HAS_S(T, DK_, DV_, M_) \
  if (dtype == dtype_of<T>() && dk == DK_ && dv == DV_ && M == M_) return true;
  LINATT_KATA_STATE_SHAPES(LINATT_HAS_S)
#undef LINATT_HAS_S
  return false;
}

struct StateWs {
  size_t seg_S, seg_z, HT, Hz, zc, bytes;
};

StateWs state_ws(int B, int T, int H, int dk, int dv, int M, int L, int dtype) {
  StateWs w{};
  const size_t E = dk / M, P = M * E * E, BH = (size_t)B * H, nseg = (T + L - 1) / L;
  const size_t PP = 3 * P / 4;  // packed state rows (symmetric pairs; kata_state.hip)
  auto al = [](size_t x) { return (x + 255) & ~size_t(255); };
  size_t off = 0;
  w.seg_S = off; off = al(off + BH * nseg * dv * PP * 4);
  w.seg_z = off; off = al(off + BH * nseg * P * 4);
  w.HT = off; off = al(off + BH * nseg * dv * PP * elt_bytes(dtype));
  w.Hz = off; off = al(off + BH * nseg * P * 4);
  w.zc = off; off = al(off + BH * (M * E * (E + 1) / 2) * 4);  // packed z_in copy (in place)
  w.bytes = off;
  return w;
}

int check_state(const char* fn, int B, int T, int H, int dk, int dv, int M, float scale, float eps,
                int L, int dtype) {
  char buf[160];
  snprintf(buf, sizeof buf, "B=%d T=%d H=%d dk=%d dv=%d num_groups=%d seg_len=%d", B, T, H, dk,
           dv, M, L);
  if (B <= 0 || T <= 0 || H <= 0 || dk <= 0 || dv <= 0 || M <= 0)
    return fail(LINATT_EINVAL, std::string(fn) + ": non-positive dimension (" + buf + ")");
  if (dk % M) return fail(LINATT_EINVAL, std::string(fn) + ": dk not divisible by num_groups");
  if (!(scale > 0.f) || !(eps > 0.f))
    return fail(LINATT_EINVAL, std::string(fn) + ": scale and eps must be positive");
  if (L <= 0 || L % 128)
    return fail(LINATT_EINVAL, std::string(fn) + ": seg_len must be a positive multiple of 128");
  if (dtype != LINATT_FLOAT32 && dtype != LINATT_BFLOAT16 && dtype != LINATT_FLOAT16)
    return fail(LINATT_EINVAL, std::string(fn) + ": unknown dtype");
  if ((int64_t)B * T * H > (int64_t)INT32_MAX / 2)
    return fail(LINATT_EINVAL, std::string(fn) + ": B*T*H too large");
  if (!state_compiled(dtype, dk, dv, M))
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": no kernel compiled for dtype " +
                                         std::to_string(dtype) + " (" + buf + ")");
  return LINATT_OK;
}

int check_delta(const char* fn, int B, int T, int H, int dk, int dv, float scale, int dtype) {
  char buf[160];
  snprintf(buf, sizeof buf, "B=%d T=%d H=%d dk=%d dv=%d", B, T, H, dk, dv);
  if (B <= 0 || T <= 0 || H <= 0 || dk <= 0 || dv <= 0)
    return fail(LINATT_EINVAL, std::string(fn) + ": non-positive dimension (" + buf + ")");
  if (!(scale > 0.f)) return fail(LINATT_EINVAL, std::string(fn) + ": scale must be positive");
  if (dtype != LINATT_FLOAT32 && dtype != LINATT_BFLOAT16 && dtype != LINATT_FLOAT16)
    return fail(LINATT_EINVAL, std::string(fn) + ": unknown dtype");
  if ((int64_t)B * H * (T + 63) > (int64_t)INT32_MAX / 2)
    return fail(LINATT_EINVAL, std::string(fn) + ": B*H*T too large");
  if (!delta_compiled(dtype, dk, dv))
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": no kernel compiled for dtype " +
                                         std::to_string(dtype) + " (" + buf + ")");
  return LINATT_OK;
}

}  // namespace

extern "C" {

int linatt_abi_version(void) { return LINATT_ABI_VERSION; }

const char* linatt_last_error(void) { return g_last_error.c_str(); }

int linatt_kata_supported(int dtype, int dk, int dv, int num_groups, int variant, int decay) {
  if (decay && variant != LINATT_KATA_CONCAT) return 0;
  if (variant != LINATT_KATA_CONCAT && variant != LINATT_KATA_SUM) return 0;
  return compiled(dtype, dk, dv, num_groups) ? 1 : 0;
}

int linatt_kata_fwd(const void* q, const void* k, const void* v, const float* c, void* o,
                    float* den, int B, int T, int HQ, int H, int dk, int dv, int num_groups,
                    float scale, int variant, int dtype, void* stream) {
  g_last_error.clear();
  int st = check_common(B, T, HQ, H, dk, dv, num_groups, scale, variant, dtype);
  if (st) return st;
  if (!q || !k || !v || !o || !den) return fail(LINATT_EINVAL, "linatt_kata_fwd: null tensor pointer");
  if (c && variant != LINATT_KATA_CONCAT)
    return fail(LINATT_EUNSUPPORTED, "linatt_kata_fwd: decay is only defined for the concat score");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return fail(LINATT_EINVAL, "linatt_kata_fwd: q, k, v, o must be 16-byte aligned");
  KataArgs a{};
  a.q = q; a.k = k; a.v = v; a.c = c; a.o = o; a.den = den;
  a.B = B; a.T = T; a.HQ = HQ; a.H = H; a.DK = dk; a.DV = dv; a.M = num_groups; a.scale = scale;
  bool found = false;
  hipError_t e = dispatch_fwd(a, dtype, variant, c != nullptr, (hipStream_t)stream, &found);
  if (!found)
    return fail(LINATT_EUNSUPPORTED, "linatt_kata_fwd: no kernel compiled for " +
                                         shape_str(B, T, HQ, H, dk, dv, num_groups));
  if (e != hipSuccess)
    return fail(LINATT_ELAUNCH, std::string("linatt_kata_fwd: launch failed: ") + hipGetErrorString(e));
  return LINATT_OK;
}

size_t linatt_kata_bwd_workspace_bytes(int B, int T, int HQ, int dv_dim, int dtype) {
  if (B <= 0 || T <= 0 || HQ <= 0 || dv_dim <= 0) return 0;
  const int64_t rows = (int64_t)B * T * HQ;
  // bf16: the dk/dv pass reads dO prescaled by scale^2/den (written by dq)
  const size_t dop = dtype == LINATT_BFLOAT16 ? (size_t)rows * dv_dim * 2 : 0;
  return linatt::kata_dop_offset(rows) + dop;
}

// Shared body of the three backward entry points; `parts` selects the
// kernels (KATA_BWD_DQ and/or KATA_BWD_DKDV).  Pointers a part does not use
// may be null.
static int kata_bwd_entry(const char* fn, int parts, const void* q, const void* k, const void* v,
                          const void* o, const float* den, const void* dout, void* dq, void* dk,
                          void* dv, void* workspace, int B, int T, int HQ, int H, int dk_dim,
                          int dv_dim, int num_groups, float scale, int variant, int dtype,
                          void* stream, const float* c = nullptr, float* dc = nullptr) {
  g_last_error.clear();
  int st = check_common(B, T, HQ, H, dk_dim, dv_dim, num_groups, scale, variant, dtype);
  if (st) return st;
  const bool need_dq = parts & KATA_BWD_DQ, need_dkdv = parts & KATA_BWD_DKDV;
  if (!q || !k || !v || !den || !dout || !workspace || (need_dq && (!o || !dq)) ||
      (need_dkdv && (!dk || !dv)))
    return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  const void* ps[] = {q, k, v, o, dout, dq, dk, dv, workspace};
  for (const void* p : ps)
    if (p && !aligned16(p))
      return fail(LINATT_EINVAL, std::string(fn) + ": tensors and workspace must be 16-byte aligned");
  KataArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = const_cast<void*>(o); a.den = const_cast<float*>(den);
  a.dout = dout; a.dq = dq; a.dk = dk; a.dv = dv; a.delta = (float*)workspace;
  a.B = B; a.T = T; a.HQ = HQ; a.H = H; a.DK = dk_dim; a.DV = dv_dim; a.M = num_groups;
  a.scale = scale;
  a.c = c;
  a.dc = dc;
  bool found = false;
  hipError_t e = dispatch_bwd(a, parts, dtype, variant, c != nullptr, (hipStream_t)stream, &found);
  if (!found)
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": no kernel compiled for " +
                                         shape_str(B, T, HQ, H, dk_dim, dv_dim, num_groups));
  if (e != hipSuccess)
    return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

int linatt_kata_bwd(const void* q, const void* k, const void* v, const void* o,
                    const float* den, const void* dout, void* dq, void* dk, void* dv,
                    void* workspace, int B, int T, int HQ, int H, int dk_dim, int dv_dim,
                    int num_groups, float scale, int variant, int dtype, void* stream) {
  return kata_bwd_entry("linatt_kata_bwd", KATA_BWD_DQ | KATA_BWD_DKDV, q, k, v, o, den, dout,
                        dq, dk, dv, workspace, B, T, HQ, H, dk_dim, dv_dim, num_groups, scale,
                        variant, dtype, stream);
}

int linatt_kata_bwd_decay(const void* q, const void* k, const void* v, const float* c,
                          const void* o, const float* den, const void* dout, void* dq, void* dk,
                          void* dv, float* dc, void* workspace, int B, int T, int HQ, int H,
                          int dk_dim, int dv_dim, int num_groups, float scale, int dtype,
                          void* stream) {
  if (!c || !dc) {
    g_last_error = "linatt_kata_bwd_decay: null c or dc";
    return LINATT_EINVAL;
  }
  return kata_bwd_entry("linatt_kata_bwd_decay", KATA_BWD_DQ | KATA_BWD_DKDV, q, k, v, o, den,
                        dout, dq, dk, dv, workspace, B, T, HQ, H, dk_dim, dv_dim, num_groups,
                        scale, LINATT_KATA_CONCAT, dtype, stream, c, dc);
}

int linatt_kata_bwd_dq(const void* q, const void* k, const void* v, const void* o,
                       const float* den, const void* dout, void* dq, void* dk, void* dv,
                       void* workspace, int B, int T, int HQ, int H, int dk_dim, int dv_dim,
                       int num_groups, float scale, int variant, int dtype, void* stream) {
  return kata_bwd_entry("linatt_kata_bwd_dq", KATA_BWD_DQ, q, k, v, o, den, dout, dq, dk, dv,
                        workspace, B, T, HQ, H, dk_dim, dv_dim, num_groups, scale, variant,
                        dtype, stream);
}

int linatt_kata_bwd_dkdv(const void* q, const void* k, const void* v, const void* o,
                         const float* den, const void* dout, void* dq, void* dk, void* dv,
                         void* workspace, int B, int T, int HQ, int H, int dk_dim, int dv_dim,
                         int num_groups, float scale, int variant, int dtype, void* stream) {
  return kata_bwd_entry("linatt_kata_bwd_dkdv", KATA_BWD_DKDV, q, k, v, o, den, dout, dq, dk,
                        dv, workspace, B, T, HQ, H, dk_dim, dv_dim, num_groups, scale, variant,
                        dtype, stream);
}

// The output RMSNorm fused into the KATA tile kernels: 16-bit, dk = dv = 64
// (the backward: bf16, whose dk/dv pass reads the dO' the dq pass forms)
static int check_onorm(const char* fn, int dk, int dv, int dtype, float eps, bool bwd) {
  if (dk != 64 || dv != 64 || dtype == LINATT_FLOAT32 || (bwd && dtype != LINATT_BFLOAT16))
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": the fused output norm runs at dk = dv = 64 in " +
                                         (bwd ? "bfloat16" : "bfloat16 or float16"));
  if (!(eps >= 0.f)) return fail(LINATT_EINVAL, std::string(fn) + ": eps must be non-negative");
  return LINATT_OK;
}

static size_t onorm_part_offset(int B, int T, int HQ, int dv_dim, int dtype) {
  return (linatt_kata_bwd_workspace_bytes(B, T, HQ, dv_dim, dtype) + 255) & ~(size_t)255;
}

int linatt_kata_fwd_onorm(const void* q, const void* k, const void* v, const float* c, void* o,
                          float* den, const float* norm_weight, float eps, void* y, float* rstd,
                          int B, int T, int HQ, int H, int dk, int dv, int num_groups, float scale,
                          int variant, int dtype, void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_kata_fwd_onorm";
  int st = check_common(B, T, HQ, H, dk, dv, num_groups, scale, variant, dtype);
  if (st) return st;
  if ((st = check_onorm(fn, dk, dv, dtype, eps, false))) return st;
  if (!q || !k || !v || !o || !den || !y || !rstd) return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  if (c && variant != LINATT_KATA_CONCAT)
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": decay is only defined for the concat score");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || !aligned16(y) ||
      (norm_weight && !aligned16(norm_weight)))
    return fail(LINATT_EINVAL, std::string(fn) + ": q, k, v, o, y, norm_weight must be 16-byte aligned");
  KataArgs a{};
  a.q = q; a.k = k; a.v = v; a.c = c; a.o = o; a.den = den;
  a.B = B; a.T = T; a.HQ = HQ; a.H = H; a.DK = dk; a.DV = dv; a.M = num_groups; a.scale = scale;
  a.nw = norm_weight; a.y = y; a.rstd = rstd; a.eps = eps;
  bool found = false;
  hipError_t e = dispatch_fwd(a, dtype, variant, c != nullptr, (hipStream_t)stream, &found);
  if (!found)
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": no kernel compiled for " +
                                         shape_str(B, T, HQ, H, dk, dv, num_groups));
  if (e != hipSuccess)
    return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

int linatt_kata_fwd_num(const void* q, const void* k, const void* v, float* num, float* den,
                        int B, int T, int HQ, int H, int dk, int dv, int num_groups, float scale,
                        int variant, int dtype, void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_kata_fwd_num";
  int st = check_common(B, T, HQ, H, dk, dv, num_groups, scale, variant, dtype);
  if (st) return st;
  if (dk != 64 || dv != 64 || dtype == LINATT_FLOAT32)
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": runs at dk = dv = 64 in bfloat16 or float16");
  if (!q || !k || !v || !num || !den) return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(num))
    return fail(LINATT_EINVAL, std::string(fn) + ": q, k, v, num must be 16-byte aligned");
  KataArgs a{};
  a.q = q; a.k = k; a.v = v; a.num32 = num; a.den = den;
  a.B = B; a.T = T; a.HQ = HQ; a.H = H; a.DK = dk; a.DV = dv; a.M = num_groups; a.scale = scale;
  bool found = false;
  hipError_t e = dispatch_fwd(a, dtype, variant, false, (hipStream_t)stream, &found);
  if (!found)
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": no kernel compiled for " +
                                         shape_str(B, T, HQ, H, dk, dv, num_groups));
  if (e != hipSuccess)
    return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

size_t linatt_kata_bwd_onorm_workspace_bytes(int B, int T, int HQ, int dv_dim, int dtype) {
  if (B <= 0 || T <= 0 || HQ <= 0 || dv_dim <= 0) return 0;
  const size_t nblk = (size_t)B * HQ * ((T + 127) / 128);
  return onorm_part_offset(B, T, HQ, dv_dim, dtype) + nblk * dv_dim * sizeof(float);
}

int linatt_kata_bwd_onorm(const void* q, const void* k, const void* v, const float* c,
                          const void* o, const float* den, const float* rstd,
                          const float* norm_weight, const void* dy, void* dq, void* dk, void* dv,
                          float* dc, float* dnorm_weight, void* workspace, int B, int T, int HQ,
                          int H, int dk_dim, int dv_dim, int num_groups, float scale, int variant,
                          int dtype, void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_kata_bwd_onorm";
  int st = check_common(B, T, HQ, H, dk_dim, dv_dim, num_groups, scale, variant, dtype);
  if (st) return st;
  if ((st = check_onorm(fn, dk_dim, dv_dim, dtype, 0.f, true))) return st;
  if (!q || !k || !v || !o || !den || !rstd || !dy || !dq || !dk || !dv || !workspace)
    return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  if ((c == nullptr) != (dc == nullptr)) return fail(LINATT_EINVAL, std::string(fn) + ": c and dc go together");
  if (c && variant != LINATT_KATA_CONCAT)
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": decay is only defined for the concat score");
  if (dnorm_weight && !norm_weight)
    return fail(LINATT_EINVAL, std::string(fn) + ": dnorm_weight without norm_weight");
  const void* ps[] = {q, k, v, o, dy, dq, dk, dv, workspace, norm_weight};
  for (const void* p : ps)
    if (p && !aligned16(p))
      return fail(LINATT_EINVAL, std::string(fn) + ": tensors and workspace must be 16-byte aligned");
  KataArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = const_cast<void*>(o); a.den = const_cast<float*>(den);
  a.dout = nullptr; a.dq = dq; a.dk = dk; a.dv = dv; a.delta = (float*)workspace;
  a.B = B; a.T = T; a.HQ = HQ; a.H = H; a.DK = dk_dim; a.DV = dv_dim; a.M = num_groups;
  a.scale = scale; a.c = c; a.dc = dc;
  a.nw = norm_weight; a.rstd = const_cast<float*>(rstd); a.dy = dy;
  float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                         onorm_part_offset(B, T, HQ, dv_dim, dtype));
  a.nw_part = dnorm_weight ? part : nullptr;
  bool found = false;
  hipError_t e = dispatch_bwd(a, KATA_BWD_DQ | KATA_BWD_DKDV, dtype, variant, c != nullptr,
                              (hipStream_t)stream, &found);
  if (!found)
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": no kernel compiled for " +
                                         shape_str(B, T, HQ, H, dk_dim, dv_dim, num_groups));
  if (e == hipSuccess && dnorm_weight)
    e = launch_colsum(part, dnorm_weight, B * HQ * ((T + 127) / 128), dv_dim, (hipStream_t)stream);
  if (e != hipSuccess)
    return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

int linatt_delta_supported(int dtype, int dk, int dv) { return delta_compiled(dtype, dk, dv) ? 1 : 0; }

size_t linatt_delta_ctx_bytes(int B, int T, int H, int dk, int dv, int dtype) {
  if (B <= 0 || T <= 0 || H <= 0 || dk <= 0 || dv <= 0) return 0;
  return delta_layout(B, T, H, dk, dv, elt_bytes(dtype)).ctx_bytes;
}

size_t linatt_delta_bwd_workspace_bytes(int B, int T, int H, int dk, int dv, int dtype) {
  if (B <= 0 || T <= 0 || H <= 0 || dk <= 0 || dv <= 0) return 0;
  return delta_layout(B, T, H, dk, dv, elt_bytes(dtype)).bwd_bytes;
}

int linatt_delta_fwd(const void* q, const void* k, const void* v, const float* beta,
                     const float* g, const float* h0, void* o, float* ht, void* ctx, int B,
                     int T, int H, int dk, int dv, float scale, int dtype, void* stream) {
  return linatt_delta_fwd_stages(q, k, v, beta, g, h0, o, ht, ctx, B, T, H, dk, dv, scale, 3,
                                 dtype, stream);
}

int linatt_delta_fwd_stages(const void* q, const void* k, const void* v, const float* beta,
                            const float* g, const float* h0, void* o, float* ht, void* ctx, int B,
                            int T, int H, int dk, int dv, float scale, int stages, int dtype,
                            void* stream) {
  g_last_error.clear();
  if (stages < 0 || stages > 3)
    return fail(LINATT_EINVAL, "linatt_delta_fwd: stages must be a mask of bits 0-1");
  int st = check_delta("linatt_delta_fwd", B, T, H, dk, dv, scale, dtype);
  if (st) return st;
  if (!q || !k || !v || !beta || !o || !ctx)
    return fail(LINATT_EINVAL, "linatt_delta_fwd: null tensor pointer");
  const void* ps[] = {q, k, v, o, ctx, h0, ht};
  for (const void* p : ps)
    if (p && !aligned16(p))
      return fail(LINATT_EINVAL, "linatt_delta_fwd: tensors must be 16-byte aligned");
  DeltaArgs a{};
  a.q = q; a.k = k; a.v = v; a.beta = beta; a.g = g; a.h0 = h0; a.o = o; a.ht = ht;
  a.ctx = (char*)ctx;
  a.B = B; a.T = T; a.H = H; a.NT = (T + kChunk - 1) / kChunk; a.scale = scale;
  a.stages = stages;
  hipError_t e = dispatch_delta(a, dtype, dk, dv, g != nullptr, false, (hipStream_t)stream);
  if (e != hipSuccess)
    return fail(LINATT_ELAUNCH, std::string("linatt_delta_fwd: launch failed: ") + hipGetErrorString(e));
  return LINATT_OK;
}

int linatt_delta_bwd(const void* q, const void* k, const void* v, const float* beta,
                     const float* g, const float* h0, const void* dout, const float* dht,
                     const void* ctx, void* workspace, void* dq, void* dk, void* dv,
                     float* dbeta, float* dg, float* dh0, int B, int T, int H, int dk_dim,
                     int dv_dim, float scale, int dtype, void* stream) {
  return linatt_delta_bwd_stages(q, k, v, beta, g, h0, dout, dht, ctx, workspace, dq, dk, dv,
                                 dbeta, dg, dh0, B, T, H, dk_dim, dv_dim, scale, 3, dtype, stream);
}

int linatt_delta_bwd_stages(const void* q, const void* k, const void* v, const float* beta,
                            const float* g, const float* h0, const void* dout, const float* dht,
                            const void* ctx, void* workspace, void* dq, void* dk, void* dv,
                            float* dbeta, float* dg, float* dh0, int B, int T, int H, int dk_dim,
                            int dv_dim, float scale, int stages, int dtype, void* stream) {
  g_last_error.clear();
  if (stages < 0 || stages > 3)
    return fail(LINATT_EINVAL, "linatt_delta_bwd: stages must be a mask of bits 0-1");
  int st = check_delta("linatt_delta_bwd", B, T, H, dk_dim, dv_dim, scale, dtype);
  if (st) return st;
  if (!q || !k || !v || !beta || !dout || !ctx || !workspace || !dq || !dk || !dv || !dbeta ||
      (g && !dg))
    return fail(LINATT_EINVAL, "linatt_delta_bwd: null tensor pointer");
  const void* ps[] = {q, k, v, dout, ctx, workspace, dq, dk, dv, dht, dh0, h0};
  for (const void* p : ps)
    if (p && !aligned16(p))
      return fail(LINATT_EINVAL, "linatt_delta_bwd: tensors must be 16-byte aligned");
  DeltaArgs a{};
  a.q = q; a.k = k; a.v = v; a.beta = beta; a.g = g; a.h0 = h0; a.dout = dout; a.dht = dht;
  a.dq = dq; a.dk = dk; a.dv = dv; a.dbeta = dbeta; a.dg = dg; a.dh0 = dh0;
  a.ctx = (char*)const_cast<void*>(ctx);
  a.ws = (char*)workspace;
  a.B = B; a.T = T; a.H = H; a.NT = (T + kChunk - 1) / kChunk; a.scale = scale;
  a.stages = stages;
  hipError_t e = dispatch_delta(a, dtype, dk_dim, dv_dim, g != nullptr, true, (hipStream_t)stream);
  if (e != hipSuccess)
    return fail(LINATT_ELAUNCH, std::string("linatt_delta_bwd: launch failed: ") + hipGetErrorString(e));
  return LINATT_OK;
}

extern "C++" {
namespace {
template <typename F>
hipError_t by_dtype(int dtype, F&& f) {
  if (dtype == LINATT_BFLOAT16) return f(__bf16{});
  if (dtype == LINATT_FLOAT16) return f(_Float16{});
  if (dtype == LINATT_FLOAT32) return f(float{});
  return hipErrorInvalidValue;
}
bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }
bool known_dtype(int d) { return d == LINATT_BFLOAT16 || d == LINATT_FLOAT16 || d == LINATT_FLOAT32; }
}  // namespace
}  // extern "C++"

int linatt_short_conv_fwd(const void* x, const float* weight, const float* bias,
                          const void* cache_in, void* y, void* cache_out, int B, int T, int C,
                          int W, int activation, int dtype, void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_short_conv_fwd";
  if (B <= 0 || T <= 0 || C <= 0) return fail(LINATT_EINVAL, std::string(fn) + ": non-positive size");
  if (C % 8) return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": channels must be a multiple of 8");
  if (W < 2 || W > 4) return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": kernel size must be 2, 3 or 4");
  if (activation != 0 && activation != 1) return fail(LINATT_EINVAL, std::string(fn) + ": activation must be 0 (none) or 1 (silu)");
  if (!known_dtype(dtype)) return fail(LINATT_EINVAL, std::string(fn) + ": unknown dtype");
  if (!x || !weight || !y) return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  if (!aligned16(x) || !aligned16(y)) return fail(LINATT_EINVAL, std::string(fn) + ": x and y must be 16-byte aligned");
  if (cache_races(cache_in, cache_out, B, C, W, T, dtype))
    return fail(LINATT_EINVAL, std::string(fn) + ": cache_out overlaps cache_in with T > 16");
  ConvArgs a{};
  a.x = x; a.w = weight; a.bias = bias; a.cache_in = cache_in; a.y = y; a.cache_out = cache_out;
  a.B = B; a.T = T; a.C = C; a.act = activation;
  hipError_t e = by_dtype(dtype, [&](auto t) { return launch_short_conv<decltype(t)>(a, W, false, (hipStream_t)stream); });
  if (e != hipSuccess) return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

size_t linatt_short_conv_bwd_workspace_bytes(int B, int T, int C, int W) {
  if (B <= 0 || T <= 0 || C <= 0 || W < 2 || W > 4) return 0;
  return short_conv_bwd_workspace(B, T, C, W);
}

int linatt_short_conv_bwd(const void* x, const float* weight, const float* bias,
                          const void* cache_in, const void* dy, void* dx, float* dweight,
                          float* dbias, void* workspace, int B, int T, int C, int W,
                          int activation, int dtype, void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_short_conv_bwd";
  if (B <= 0 || T <= 0 || C <= 0) return fail(LINATT_EINVAL, std::string(fn) + ": non-positive size");
  if (C % 8) return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": channels must be a multiple of 8");
  if (W < 2 || W > 4) return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": kernel size must be 2, 3 or 4");
  if (activation != 0 && activation != 1) return fail(LINATT_EINVAL, std::string(fn) + ": activation must be 0 (none) or 1 (silu)");
  if (!known_dtype(dtype)) return fail(LINATT_EINVAL, std::string(fn) + ": unknown dtype");
  if (!x || !weight || !dy || !dx || !dweight || !workspace)
    return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  if (!aligned16(x) || !aligned16(dy) || !aligned16(dx))
    return fail(LINATT_EINVAL, std::string(fn) + ": x, dy and dx must be 16-byte aligned");
  ConvArgs a{};
  a.x = x; a.w = weight; a.bias = bias; a.cache_in = cache_in; a.dy = dy; a.dx = dx;
  a.part = (float*)workspace; a.dw = dweight; a.db = dbias;
  a.B = B; a.T = T; a.C = C; a.act = activation;
  hipError_t e = by_dtype(dtype, [&](auto t) { return launch_short_conv<decltype(t)>(a, W, true, (hipStream_t)stream); });
  if (e != hipSuccess) return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

int linatt_rope(const void* x, void* y, int B, int T, int H, int D, int rot_dim, float base,
                int offset, int interleaved, int inverse, int dtype, void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_rope";
  if (B <= 0 || T <= 0 || H <= 0 || D <= 0) return fail(LINATT_EINVAL, std::string(fn) + ": non-positive size");
  if (rot_dim <= 0 || rot_dim > D || rot_dim % 2 || (D - rot_dim) % 2)
    return fail(LINATT_EINVAL, std::string(fn) + ": rot_dim must be even, positive and at most D (D - rot_dim even)");
  if (!(base > 1.f)) return fail(LINATT_EINVAL, std::string(fn) + ": base must be > 1");
  if (offset < 0) return fail(LINATT_EINVAL, std::string(fn) + ": offset must be >= 0");
  if (!known_dtype(dtype)) return fail(LINATT_EINVAL, std::string(fn) + ": unknown dtype");
  if (!x || !y) return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  hipError_t e = by_dtype(dtype, [&](auto t) {
    return launch_rope<decltype(t)>(x, y, B, T, H, D, rot_dim, base, offset, interleaved ? 1 : 0,
                                    inverse ? 1 : 0, (hipStream_t)stream);
  });
  if (e != hipSuccess) return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

int linatt_linear_scan_fwd(const void* q, const void* k, const void* v, void* o, float* den, int B,
                           int H, int T, int d, int dv, float scale, float eps, int dtype,
                           void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_linear_scan_fwd";
  if (B <= 0 || T <= 0 || H <= 0 || d <= 0 || dv <= 0)
    return fail(LINATT_EINVAL, std::string(fn) + ": non-positive size");
  if ((int64_t)B * H * (T + 63) > (int64_t)INT32_MAX / 2)
    return fail(LINATT_EINVAL, std::string(fn) + ": B*H*T too large");
  if (!(scale > 0.f) || !(eps > 0.f)) return fail(LINATT_EINVAL, std::string(fn) + ": scale and eps must be positive");
  if (d != 64 || dv != 64 || (dtype != LINATT_BFLOAT16 && dtype != LINATT_FLOAT16))
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": compiled for d = dv = 64, bfloat16 / float16");
  if (!q || !k || !v || !o || !den) return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return fail(LINATT_EINVAL, std::string(fn) + ": tensors must be 16-byte aligned");
  const hipError_t e =
      dtype == LINATT_BFLOAT16
          ? launch_linear_scan<__bf16>(q, k, v, o, den, B, H, T, scale, eps, (hipStream_t)stream)
          : launch_linear_scan<_Float16>(q, k, v, o, den, B, H, T, scale, eps, (hipStream_t)stream);
  if (e != hipSuccess) return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

static int check_qk(const char* fn, int B, int T, int H, int D, int W, int activation, int norm,
                    const float* norm_weight, float eps, int rope_width, int rot_dim, float base,
                    int offset, int interleaved, int dtype) {
  if (B <= 0 || T <= 0 || H <= 0 || D <= 0) return fail(LINATT_EINVAL, std::string(fn) + ": non-positive size");
  if (B > 65535 || (T + 15) / 16 > 65535 || (int64_t)H * D > INT32_MAX / 8)
    return fail(LINATT_EINVAL, std::string(fn) + ": B, T or H*D too large");
  if (D != 32 && D != 64 && D != 128)
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": head dim must be 32, 64 or 128");
  if (W < 2 || W > 4) return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": kernel size must be 2, 3 or 4");
  if (activation != 0 && activation != 1) return fail(LINATT_EINVAL, std::string(fn) + ": activation must be 0 (none) or 1 (silu)");
  if (norm < 0 || norm > 2) return fail(LINATT_EINVAL, std::string(fn) + ": norm must be 0 (none), 1 (RMSNorm) or 2 (L2)");
  if (norm == 2 && norm_weight) return fail(LINATT_EINVAL, std::string(fn) + ": the L2 norm takes no weight");
  if (!(eps >= 0.f)) return fail(LINATT_EINVAL, std::string(fn) + ": eps must be >= 0");
  if (rot_dim != 0) {
    if (rope_width <= 0 || rope_width % 4 || D % rope_width)
      return fail(LINATT_EINVAL, std::string(fn) + ": rope_width must be a multiple of 4 dividing the head dim");
    if (rot_dim < 0 || rot_dim % 2 || rot_dim > rope_width)
      return fail(LINATT_EINVAL, std::string(fn) + ": rot_dim must be even, positive and at most rope_width");
    if (!interleaved && rot_dim % 8)
      return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": a non-interleaved rotation needs rot_dim a multiple of 8");
    if (!(base > 1.f)) return fail(LINATT_EINVAL, std::string(fn) + ": base must be > 1");
    if (offset < 0) return fail(LINATT_EINVAL, std::string(fn) + ": offset must be >= 0");
  }
  if (!known_dtype(dtype)) return fail(LINATT_EINVAL, std::string(fn) + ": unknown dtype");
  return LINATT_OK;
}

static QKArgs qk_args(const void* x, const float* w, const float* bias, const void* cache_in,
                      const float* nw, int B, int T, int H, int D, int activation, int norm,
                      float eps, int rope_width, int rot_dim, float base, int offset,
                      int interleaved) {
  QKArgs a{};
  a.x = x; a.w = w; a.bias = bias; a.cache_in = cache_in; a.nw = norm == 1 ? nw : nullptr;
  a.B = B; a.T = T; a.C = H * D; a.D = D; a.act = activation; a.norm = norm;
  a.eps = eps; a.inv_n = norm == 1 ? 1.f / D : 1.f;
  a.rot = rot_dim; a.rw = rot_dim ? rope_width : 0; a.interleaved = interleaved ? 1 : 0;
  a.offset = offset; a.log2_base = rot_dim ? log2f(base) : 0.f;
  return a;
}

int linatt_qk_prologue_fwd(const void* x, const float* conv_weight, const float* conv_bias,
                           const void* cache_in, const float* norm_weight, void* y,
                           void* cache_out, int B, int T, int H, int D, int W, int activation,
                           int norm, float eps, int rope_width, int rot_dim, float base,
                           int offset, int interleaved, int dtype, void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_qk_prologue_fwd";
  int st = check_qk(fn, B, T, H, D, W, activation, norm, norm_weight, eps, rope_width, rot_dim,
                    base, offset, interleaved, dtype);
  if (st) return st;
  if (!x || !conv_weight || !y) return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  if (!aligned16(x) || !aligned16(y)) return fail(LINATT_EINVAL, std::string(fn) + ": x and y must be 16-byte aligned");
  if (cache_races(cache_in, cache_out, B, H * D, W, T, dtype))
    return fail(LINATT_EINVAL, std::string(fn) + ": cache_out overlaps cache_in with T > 16");
  QKArgs a = qk_args(x, conv_weight, conv_bias, cache_in, norm_weight, B, T, H, D, activation,
                     norm, eps, rope_width, rot_dim, base, offset, interleaved);
  a.y = y; a.cache_out = cache_out;
  hipError_t e = by_dtype(dtype, [&](auto t) { return launch_qk_prologue<decltype(t)>(a, W, false, (hipStream_t)stream); });
  if (e != hipSuccess) return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

size_t linatt_qk_prologue_bwd_workspace_bytes(int B, int T, int H, int D, int W) {
  if (B <= 0 || T <= 0 || H <= 0 || D <= 0 || W < 2 || W > 4) return 0;
  return qk_prologue_bwd_workspace(B, T, H * D, D, W);
}

int linatt_qk_prologue_bwd(const void* x, const float* conv_weight, const float* conv_bias,
                           const void* cache_in, const float* norm_weight, const void* dy,
                           void* dx, float* dconv_weight, float* dconv_bias, float* dnorm_weight,
                           void* workspace, int B, int T, int H, int D, int W, int activation,
                           int norm, float eps, int rope_width, int rot_dim, float base,
                           int offset, int interleaved, int dtype, void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_qk_prologue_bwd";
  int st = check_qk(fn, B, T, H, D, W, activation, norm, norm_weight, eps, rope_width, rot_dim,
                    base, offset, interleaved, dtype);
  if (st) return st;
  if (!x || !conv_weight || !dy || !dx || !dconv_weight || !workspace || (dnorm_weight && !norm_weight))
    return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  if (!aligned16(x) || !aligned16(dy) || !aligned16(dx) || !aligned16(workspace))
    return fail(LINATT_EINVAL, std::string(fn) + ": x, dy, dx and the workspace must be 16-byte aligned");
  QKArgs a = qk_args(x, conv_weight, conv_bias, cache_in, norm_weight, B, T, H, D, activation,
                     norm, eps, rope_width, rot_dim, base, offset, interleaved);
  a.dy = dy; a.dx = dx; a.part = (float*)workspace;
  a.dw = dconv_weight; a.db = dconv_bias; a.dnw = dnorm_weight;
  hipError_t e = by_dtype(dtype, [&](auto t) { return launch_qk_prologue<decltype(t)>(a, W, true, (hipStream_t)stream); });
  if (e != hipSuccess) return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

static int check_rms(const char* fn, int n, int d, int dtype) {
  if (n <= 0 || d <= 0) return fail(LINATT_EINVAL, std::string(fn) + ": non-positive size");
  if (d % 8 || !pow2(d / 8) || d > 512)
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": row length must be 8 times a power of two, at most 512");
  if (!known_dtype(dtype)) return fail(LINATT_EINVAL, std::string(fn) + ": unknown dtype");
  return LINATT_OK;
}

int linatt_rmsnorm_fwd(const void* x, const float* weight, void* y, float* rstd, int n, int d,
                       float eps, int dtype, void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_rmsnorm_fwd";
  int st = check_rms(fn, n, d, dtype);
  if (st) return st;
  if (!(eps >= 0.f)) return fail(LINATT_EINVAL, std::string(fn) + ": eps must be >= 0");
  if (!x || !y || !rstd) return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  if (!aligned16(x) || !aligned16(y)) return fail(LINATT_EINVAL, std::string(fn) + ": x and y must be 16-byte aligned");
  hipError_t e = by_dtype(dtype, [&](auto t) {
    return launch_rmsnorm<decltype(t)>(x, weight, nullptr, nullptr, y, rstd, nullptr, nullptr, n, d,
                                       eps, false, (hipStream_t)stream);
  });
  if (e != hipSuccess) return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

size_t linatt_rmsnorm_bwd_workspace_bytes(int n, int d) {
  if (n <= 0 || d <= 0 || d % 8 || !pow2(d / 8) || d > 512) return 0;
  return (size_t)rmsnorm_bwd_blocks(n, d) * d * sizeof(float);
}

int linatt_rmsnorm_bwd(const void* x, const float* weight, const float* rstd, const void* dy,
                       void* dx, float* dweight, void* workspace, int n, int d, int dtype,
                       void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_rmsnorm_bwd";
  int st = check_rms(fn, n, d, dtype);
  if (st) return st;
  if (!x || !rstd || !dy || !dx || !workspace || (dweight && !weight))
    return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  if (!aligned16(x) || !aligned16(dy) || !aligned16(dx))
    return fail(LINATT_EINVAL, std::string(fn) + ": x, dy and dx must be 16-byte aligned");
  hipError_t e = by_dtype(dtype, [&](auto t) {
    return launch_rmsnorm<decltype(t)>(x, weight, rstd, dy, dx, nullptr, dweight, (float*)workspace,
                                       n, d, 0.f, true, (hipStream_t)stream);
  });
  if (e != hipSuccess) return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

int linatt_l2norm_fwd(const void* x, void* y, float* rstd, int n, int d, float eps, int dtype,
                      void* stream) {
  g_last_error.clear();
  if (n <= 0 || d <= 0) return fail(LINATT_EINVAL, "linatt_l2norm_fwd: non-positive size");
  if (!x || !y || !rstd) return fail(LINATT_EINVAL, "linatt_l2norm_fwd: null tensor pointer");
  if (!(eps >= 0.f)) return fail(LINATT_EINVAL, "linatt_l2norm_fwd: eps must be >= 0");
  hipError_t e;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == LINATT_BFLOAT16) e = launch_l2norm_fwd<__bf16>(x, y, rstd, n, d, eps, s);
  else if (dtype == LINATT_FLOAT16) e = launch_l2norm_fwd<_Float16>(x, y, rstd, n, d, eps, s);
  else if (dtype == LINATT_FLOAT32) e = launch_l2norm_fwd<float>(x, y, rstd, n, d, eps, s);
  else return fail(LINATT_EINVAL, "linatt_l2norm_fwd: unknown dtype");
  if (e != hipSuccess)
    return fail(LINATT_ELAUNCH, std::string("linatt_l2norm_fwd: launch failed: ") + hipGetErrorString(e));
  return LINATT_OK;
}

int linatt_l2norm_bwd(const void* y, const float* rstd, const void* dy, void* dx, int n, int d,
                      int dtype, void* stream) {
  g_last_error.clear();
  if (n <= 0 || d <= 0) return fail(LINATT_EINVAL, "linatt_l2norm_bwd: non-positive size");
  if (!y || !rstd || !dy || !dx) return fail(LINATT_EINVAL, "linatt_l2norm_bwd: null tensor pointer");
  hipError_t e;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == LINATT_BFLOAT16) e = launch_l2norm_bwd<__bf16>(y, rstd, dy, dx, n, d, s);
  else if (dtype == LINATT_FLOAT16) e = launch_l2norm_bwd<_Float16>(y, rstd, dy, dx, n, d, s);
  else if (dtype == LINATT_FLOAT32) e = launch_l2norm_bwd<float>(y, rstd, dy, dx, n, d, s);
  else return fail(LINATT_EINVAL, "linatt_l2norm_bwd: unknown dtype");
  if (e != hipSuccess)
    return fail(LINATT_ELAUNCH, std::string("linatt_l2norm_bwd: launch failed: ") + hipGetErrorString(e));
  return LINATT_OK;
}

int linatt_dkata_supported(int dtype, int d, int dv, int num_groups) {
#define LINATT_HAS_DK(T_, D_, DV_, M_) \
  if (dtype == dtype_of<T_>() && d == D_ && dv == DV_ && num_groups == M_) return 1;
  LINATT_DKATA_SHAPES(LINATT_HAS_DK)
#undef LINATT_HAS_DK
  return 0;
}

size_t linatt_dkata_workspace_bytes(int B, int T, int H, int d, int dv, int dtype) {
  if (B <= 0 || T <= 0 || H <= 0 || d <= 0 || dv <= 0) return 0;
  return dkata_layout(B, T, H, d, dv, elt_bytes(dtype)).bytes;
}

static int dkata_fwd_entry(const char* fn, int keep_e, const void* q, const void* k,
                           const void* v, const float* beta, float* U, float* o, float* den,
                           void* workspace, int B, int T, int H, int d, int dv, int num_groups,
                           float scale, int normalize, float eps, int dtype, void* stream);

int linatt_dkata_fwd(const void* q, const void* k, const void* v, const float* beta, float* U,
                     float* o, float* den, void* workspace, int B, int T, int H, int d, int dv,
                     int num_groups, float scale, int normalize, float eps, int dtype,
                     void* stream) {
  return dkata_fwd_entry("linatt_dkata_fwd", 0, q, k, v, beta, U, o, den, workspace, B, T, H, d,
                         dv, num_groups, scale, normalize, eps, dtype, stream);
}

int linatt_dkata_fwd_train(const void* q, const void* k, const void* v, const float* beta,
                           float* U, float* o, float* den, void* workspace, int B, int T, int H,
                           int d, int dv, int num_groups, float scale, int normalize, float eps,
                           int dtype, void* stream) {
  return dkata_fwd_entry("linatt_dkata_fwd_train", 1, q, k, v, beta, U, o, den, workspace, B, T,
                         H, d, dv, num_groups, scale, normalize, eps, dtype, stream);
}

size_t linatt_dkata_bwd_workspace_bytes(int B, int T, int H, int d, int dv, int dtype) {
  if (B <= 0 || T <= 0 || H <= 0 || d <= 0 || dv <= 0) return 0;
  return dkata_bwd_layout(B, T, H, d, dv, elt_bytes(dtype)).bytes;
}

int linatt_dkata_bwd(const void* q, const void* k, const void* v, const float* beta,
                     const float* U, const float* o, const float* den, const float* dout,
                     void* dq, void* dk, void* dv, float* dbeta, void* fwd_workspace,
                     void* workspace, int B, int T, int H, int d, int dv_dim, int num_groups,
                     float scale, int normalize, float eps, int dtype, void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_dkata_bwd";
  char buf[160];
  snprintf(buf, sizeof buf, "B=%d T=%d H=%d d=%d dv=%d num_groups=%d", B, T, H, d, dv_dim, num_groups);
  if (B <= 0 || T <= 0 || H <= 0 || d <= 0 || dv_dim <= 0 || num_groups <= 0)
    return fail(LINATT_EINVAL, std::string(fn) + ": non-positive dimension (" + buf + ")");
  if (!(scale > 0.f) || (normalize && !(eps >= 0.f)))
    return fail(LINATT_EINVAL, std::string(fn) + ": scale must be positive and eps non-negative");
  if ((int64_t)B * H * (T + 63) > (int64_t)INT32_MAX / 2)
    return fail(LINATT_EINVAL, std::string(fn) + ": B*H*T too large");
  if (!linatt_dkata_supported(dtype, d, dv_dim, num_groups))
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": no kernel compiled for dtype " +
                                         std::to_string(dtype) + " (" + buf + ")");
  // dU = lower(A_qk)^T do' is carried in the input dtype; fp16's range loses
  // it for small scales (kappa ~ scale^2), so the backward is bf16 only, the
  // dtype the mixer calls flash_delta with (kata/layer.py:409-412)
  if (dtype != LINATT_BFLOAT16)
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": the backward is compiled for bfloat16 only");
  if (!q || !k || !v || !beta || !den || !dout || !dq || !dk || !dv || !dbeta ||
      !fwd_workspace || !workspace || (normalize && !o))
    return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  const void* ps[] = {q, k, v, U, o, dout, dq, dk, dv, fwd_workspace, workspace};
  for (const void* p : ps)
    if (p && !aligned16(p))
      return fail(LINATT_EINVAL, std::string(fn) + ": tensors must be 16-byte aligned");
  DKataBwdArgs a{};
  a.q = q; a.k = k; a.v = v; a.beta = beta; a.U = U; a.o = o; a.den = den; a.dout = dout;
  a.dq = dq; a.dk = dk; a.dv = dv; a.dbeta = dbeta;
  a.ws = (char*)fwd_workspace;
  a.L = dkata_layout(B, T, H, d, dv_dim, elt_bytes(dtype));
  a.bws = (char*)workspace;
  a.BL = dkata_bwd_layout(B, T, H, d, dv_dim, elt_bytes(dtype));
  a.B = B; a.T = T; a.H = H;
  a.scale = scale; a.scale2 = scale * scale; a.eps = eps; a.normalize = normalize ? 1 : 0;
  hipError_t e = hipErrorInvalidValue;
#define LINATT_TRY_DKB(T_, D_, DV_, M_) \
  if (dtype == dtype_of<T_>() && d == D_ && dv_dim == DV_ && num_groups == M_) \
    e = launch_dkata_bwd<T_, D_, DV_, M_>(a, (hipStream_t)stream);
  LINATT_DKATA_SHAPES(LINATT_TRY_DKB)
#undef LINATT_TRY_DKB
  if (e != hipSuccess)
    return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

static int dkata_fwd_entry(const char* fn, int keep_e, const void* q, const void* k,
                           const void* v, const float* beta, float* U, float* o, float* den,
                           void* workspace, int B, int T, int H, int d, int dv, int num_groups,
                           float scale, int normalize, float eps, int dtype, void* stream) {
  g_last_error.clear();
  char buf[160];
  snprintf(buf, sizeof buf, "B=%d T=%d H=%d d=%d dv=%d num_groups=%d", B, T, H, d, dv, num_groups);
  if (B <= 0 || T <= 0 || H <= 0 || d <= 0 || dv <= 0 || num_groups <= 0)
    return fail(LINATT_EINVAL, std::string(fn) + ": non-positive dimension (" + buf + ")");
  if (!(scale > 0.f) || (normalize && !(eps >= 0.f)))
    return fail(LINATT_EINVAL, std::string(fn) + ": scale must be positive and eps non-negative");
  if ((int64_t)B * H * (T + 63) > (int64_t)INT32_MAX / 2)
    return fail(LINATT_EINVAL, std::string(fn) + ": B*H*T too large");
  if (!linatt_dkata_supported(dtype, d, dv, num_groups))
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": no kernel compiled for dtype " +
                                         std::to_string(dtype) + " (" + buf + ")");
  if (!q || !k || !v || !beta || !o || !den || !workspace)
    return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  const void* ps[] = {q, k, v, o, U, workspace};
  for (const void* p : ps)
    if (p && !aligned16(p))
      return fail(LINATT_EINVAL, std::string(fn) + ": tensors must be 16-byte aligned");
  DKataArgs a{};
  a.q = q; a.k = k; a.v = v; a.beta = beta; a.U = U; a.o = o; a.den = den;
  a.ws = (char*)workspace;
  a.L = dkata_layout(B, T, H, d, dv, elt_bytes(dtype));
  a.B = B; a.T = T; a.H = H;
  a.scale = scale; a.scale2 = scale * scale; a.eps = eps; a.normalize = normalize ? 1 : 0;
  a.keep_e = keep_e;
  hipError_t e = hipErrorInvalidValue;
#define LINATT_TRY_DK(T_, D_, DV_, M_) \
  if (dtype == dtype_of<T_>() && d == D_ && dv == DV_ && num_groups == M_) \
    e = launch_dkata_fwd<T_, D_, DV_, M_>(a, (hipStream_t)stream);
  LINATT_DKATA_SHAPES(LINATT_TRY_DK)
#undef LINATT_TRY_DK
  if (e != hipSuccess)
    return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

int linatt_kata_state_supported(int dtype, int dk, int dv, int num_groups) {
  return state_compiled(dtype, dk, dv, num_groups) ? 1 : 0;
}

size_t linatt_kata_prefill_workspace_bytes(int B, int T, int H, int dk, int dv, int num_groups,
                                           int seg_len, int dtype) {
  if (B <= 0 || T <= 0 || H <= 0 || dk <= 0 || dv <= 0 || num_groups <= 0 || dk % num_groups ||
      seg_len <= 0)
    return 0;
  return state_ws(B, T, H, dk, dv, num_groups, seg_len, dtype).bytes;
}

// the prefill with the state in the full (tri = 0) or packed (tri = 1) layout
static int kata_prefill_state_impl(const char* fn, int tri, const void* q, const void* k,
                                   const void* v, void* o, float* den, const float* S_in,
                                   const float* z_in, float* S_out, float* z_out, void* workspace,
                                   int B, int T, int H, int dk, int dv, int num_groups, float scale,
                                   float eps, int seg_len, int head_major, int dtype, void* stream) {
  g_last_error.clear();
  int st = check_state(fn, B, T, H, dk, dv, num_groups, scale, eps, seg_len, dtype);
  if (st) return st;
  if (!q || !k || !v || !o || !den || !workspace)
    return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  if ((S_in == nullptr) != (z_in == nullptr))
    return fail(LINATT_EINVAL, std::string(fn) + ": S_in and z_in must be given together");
  const void* ps[] = {q, k, v, o, workspace, S_out, z_out, S_in, z_in};
  for (const void* p : ps)
    if (p && !aligned16(p))
      return fail(LINATT_EINVAL, std::string(fn) + ": tensors must be 16-byte aligned");
  const StateWs w = state_ws(B, T, H, dk, dv, num_groups, seg_len, dtype);
  char* ws = (char*)workspace;
  KataStateArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = o; a.den = den;
  if (head_major) {  // (B, H, T, D)
    a.sb = (int64_t)H * T * dk; a.sh = (int64_t)T * dk; a.st = dk;
    a.vsb = (int64_t)H * T * dv; a.vsh = (int64_t)T * dv; a.vst = dv;
    a.osb = a.vsb; a.osh = a.vsh; a.ost = a.vst;
    a.dsb = (int64_t)H * T; a.dsh = T; a.dst = 1;
  } else {           // (B, T, H, D)
    a.sb = (int64_t)T * H * dk; a.st = (int64_t)H * dk; a.sh = dk;
    a.vsb = (int64_t)T * H * dv; a.vst = (int64_t)H * dv; a.vsh = dv;
    a.osb = a.vsb; a.ost = a.vst; a.osh = a.vsh;
    a.dsb = (int64_t)T * H; a.dst = H; a.dsh = 1;
  }
  a.seg_S = (float*)(ws + w.seg_S); a.seg_z = (float*)(ws + w.seg_z);
  a.HT = ws + w.HT; a.Hz = (float*)(ws + w.Hz);
  a.S_out = S_out; a.z_out = z_out; a.S_in = S_in; a.z_in = z_in;
  a.B = B; a.T = T; a.H = H; a.L = seg_len; a.nseg = (T + seg_len - 1) / seg_len;
  a.scale = scale; a.scale2 = scale * scale; a.eps = eps;
  a.tri = tri;
  hipError_t e = hipErrorInvalidValue;
  hipStream_t sm = (hipStream_t)stream;
  if (tri && z_in && z_in == z_out) {
    // packed layout in place: two scan threads read each off-diagonal pair's
    // z element and one of them writes it, so the scan reads a copy
    const int64_t n = (int64_t)B * H * (num_groups * (dk / num_groups) * (dk / num_groups + 1) / 2);
    e = launch_f32_copy(z_in, (float*)(ws + w.zc), n, sm);
    if (e != hipSuccess)
      return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
    a.z_in = (const float*)(ws + w.zc);
    e = hipErrorInvalidValue;
  }
#define LINATT_TRY_S(T_, DK_, DV_, M_) \
  if (dtype == dtype_of<T_>() && dk == DK_ && dv == DV_ && num_groups == M_) e = launch_kata_prefill<T_, DK_, DV_, M_>(a, sm);
  LINATT_KATA_STATE_SHAPES(LINATT_TRY_S)
#undef LINATT_TRY_S
  if (e != hipSuccess)
    return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

int linatt_kata_prefill_state(const void* q, const void* k, const void* v, void* o, float* den,
                              const float* S_in, const float* z_in, float* S_out, float* z_out,
                              void* workspace, int B, int T, int H, int dk, int dv, int num_groups,
                              float scale, float eps, int seg_len, int head_major, int dtype,
                              void* stream) {
  return kata_prefill_state_impl("linatt_kata_prefill_state", 0, q, k, v, o, den, S_in, z_in, S_out,
                                 z_out, workspace, B, T, H, dk, dv, num_groups, scale, eps, seg_len,
                                 head_major, dtype, stream);
}

int linatt_kata_prefill_state_packed(const void* q, const void* k, const void* v, void* o,
                                     float* den, const float* S_in, const float* z_in, float* S_out,
                                     float* z_out, void* workspace, int B, int T, int H, int dk,
                                     int dv, int num_groups, float scale, float eps, int seg_len,
                                     int head_major, int dtype, void* stream) {
  return kata_prefill_state_impl("linatt_kata_prefill_state_packed", 1, q, k, v, o, den, S_in, z_in,
                                 S_out, z_out, workspace, B, T, H, dk, dv, num_groups, scale, eps,
                                 seg_len, head_major, dtype, stream);
}

int linatt_kata_prefill(const void* q, const void* k, const void* v, void* o, float* den,
                        float* S_out, float* z_out, void* workspace, int B, int T, int H, int dk,
                        int dv, int num_groups, float scale, float eps, int seg_len,
                        int head_major, int dtype, void* stream) {
  return linatt_kata_prefill_state(q, k, v, o, den, nullptr, nullptr, S_out, z_out, workspace, B,
                                   T, H, dk, dv, num_groups, scale, eps, seg_len, head_major,
                                   dtype, stream);
}

// one decode step on the full (tri = 0) or packed (tri = 1) state
static int kata_decode_step_impl(const char* fn, int tri, const void* q, const void* k,
                                 const void* v, float* S, float* z, void* o, int B, int H, int dk,
                                 int dv, int num_groups, float scale, float eps, int dtype,
                                 void* stream, bool split = false, void* workspace = nullptr,
                                 size_t workspace_bytes = 0) {
  g_last_error.clear();
  int st = check_state(fn, B, 1, H, dk, dv, num_groups, scale, eps, 128, dtype);
  if (st) return st;
  if (!q || !k || !v || !S || !z || !o)
    return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  const void* ps[] = {S, z, o};
  for (const void* p : ps)
    if (!aligned16(p))
      return fail(LINATT_EINVAL, std::string(fn) + ": S, z, o must be 16-byte aligned");
  KataDecodeArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = o; a.S = S; a.z = z; a.B = B; a.H = H;
  a.scale = scale; a.eps = eps; a.tri = tri;
  a.nsplit = 1;
  if (split) {
    const int E = dk / num_groups;
    const int rows = num_groups * (tri ? E * (E + 1) / 2 : E * E);
    a.nsplit = kata_gen_decode_splits(B * H, rows);
    if (a.nsplit > 1) {
      const size_t need = (size_t)B * H * a.nsplit * kGenDecPart * sizeof(float);
      if (!workspace || workspace_bytes < need)
        return fail(LINATT_EINVAL, std::string(fn) + ": workspace smaller than linatt_kata_decode_workspace_bytes");
      if (!aligned16(workspace)) return fail(LINATT_EINVAL, std::string(fn) + ": workspace must be 16-byte aligned");
      a.part = reinterpret_cast<float*>(workspace);
    }
  }
  hipError_t e = hipErrorInvalidValue;
  hipStream_t sm = (hipStream_t)stream;
#define LINATT_TRY_DEC(T_, DK_, DV_, M_) \
  if (dtype == dtype_of<T_>() && dk == DK_ && dv == DV_ && num_groups == M_) e = launch_kata_decode<T_, DK_, DV_, M_>(a, sm);
  LINATT_KATA_STATE_SHAPES(LINATT_TRY_DEC)
#undef LINATT_TRY_DEC
  if (e != hipSuccess)
    return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

size_t linatt_kata_decode_workspace_bytes(int B, int H, int dk, int num_groups, int packed) {
  if (B <= 0 || H <= 0 || dk <= 0 || num_groups <= 0 || dk % num_groups) return 0;
  const int E = dk / num_groups;
  const int rows = num_groups * (packed ? E * (E + 1) / 2 : E * E);
  const int ns = kata_gen_decode_splits(B * H, rows);
  return ns > 1 ? (size_t)B * H * ns * kGenDecPart * sizeof(float) : 0;
}

int linatt_kata_decode_step_split(const void* q, const void* k, const void* v, float* S, float* z,
                                  void* o, void* workspace, size_t workspace_bytes, int B, int H,
                                  int dk, int dv, int num_groups, int packed, float scale, float eps,
                                  int dtype, void* stream) {
  return kata_decode_step_impl("linatt_kata_decode_step_split", packed ? 1 : 0, q, k, v, S, z, o,
                               B, H, dk, dv, num_groups, scale, eps, dtype, stream, true, workspace,
                               workspace_bytes);
}

int linatt_kata_decode_step(const void* q, const void* k, const void* v, float* S, float* z,
                            void* o, int B, int H, int dk, int dv, int num_groups, float scale,
                            float eps, int dtype, void* stream) {
  return kata_decode_step_impl("linatt_kata_decode_step", 0, q, k, v, S, z, o, B, H, dk, dv,
                               num_groups, scale, eps, dtype, stream);
}

int linatt_kata_decode_step_packed(const void* q, const void* k, const void* v, float* S, float* z,
                                   void* o, int B, int H, int dk, int dv, int num_groups,
                                   float scale, float eps, int dtype, void* stream) {
  return kata_decode_step_impl("linatt_kata_decode_step_packed", 1, q, k, v, S, z, o, B, H, dk, dv,
                               num_groups, scale, eps, dtype, stream);
}

// ---------------------------------------------------------------------------
// Generic state form (kata_state_gen.hip)
// ---------------------------------------------------------------------------
static int gen_state_args(const char* fn, KataGenStateArgs& a, int B, int T, int H, int dk, int dv,
                          int M, int variant, float scale, float eps, int dtype) {
  if (B <= 0 || T <= 0 || H <= 0 || dk <= 0 || dv <= 0 || M <= 0)
    return fail(LINATT_EINVAL, std::string(fn) + ": non-positive dimension");
  const int tri = (variant & LINATT_KATA_PACKED_STATE) ? 1 : 0;
  variant &= ~LINATT_KATA_PACKED_STATE;
  if (variant != LINATT_KATA_CONCAT && variant != LINATT_KATA_SUM)
    return fail(LINATT_EINVAL, std::string(fn) + ": unknown KATA variant");
  if (!known_dtype(dtype)) return fail(LINATT_EINVAL, std::string(fn) + ": unknown dtype");
  if (!(scale > 0.f) || !(eps > 0.f)) return fail(LINATT_EINVAL, std::string(fn) + ": scale and eps must be positive");
  if (dk % M) return fail(LINATT_EINVAL, std::string(fn) + ": dk not divisible by num_groups");
  const int E = dk / M;
  if (dv != 64 || dk > 128 || E < 16 || !pow2(E))
    return fail(LINATT_EUNSUPPORTED, std::string(fn) + ": needs dv = 64, dk <= 128 and a group width "
                                     "E = dk / num_groups that is a power of two >= 16");
  if ((int64_t)B * T * H > (int64_t)INT32_MAX / 64)
    return fail(LINATT_EINVAL, std::string(fn) + ": B*T*H too large");
  int lgE = 0;
  while ((1 << lgE) < E) ++lgE;
  a.B = B; a.T = T; a.H = H; a.dk = dk; a.E = E; a.lgE = lgE; a.M = M;
  a.sum = variant == LINATT_KATA_SUM ? 1 : 0;
  a.tri = tri;
  a.TE = E * (E + 1) / 2;
  a.P = (a.sum ? 1 : M) * (tri ? a.TE : E * E);
  a.nsplit = 1;
  a.scale = scale; a.eps = eps;
  return LINATT_OK;
}

static int gen_state_launch(const char* fn, const KataGenStateArgs& a, int which, int dtype, void* stream) {
  hipError_t e = by_dtype(dtype, [&](auto t) { return launch_kata_gen_state<decltype(t)>(a, which, (hipStream_t)stream); });
  if (e != hipSuccess) return fail(LINATT_ELAUNCH, std::string(fn) + ": launch failed: " + hipGetErrorString(e));
  return LINATT_OK;
}

int linatt_kata_gen_state_rows(int dk, int num_groups, int variant) {
  if (dk <= 0 || num_groups <= 0 || dk % num_groups) return 0;
  const int E = dk / num_groups;
  const bool tri = (variant & LINATT_KATA_PACKED_STATE) != 0;
  variant &= ~LINATT_KATA_PACKED_STATE;
  if (variant != LINATT_KATA_CONCAT && variant != LINATT_KATA_SUM) return 0;
  return (variant == LINATT_KATA_SUM ? 1 : num_groups) * (tri ? E * (E + 1) / 2 : E * E);
}

int linatt_kata_gen_decode(const void* q, const void* k, const void* v, const float* c, float* S,
                           float* z, void* o, int B, int H, int dk, int dv, int num_groups,
                           int variant, float scale, float eps, int dtype, void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_kata_gen_decode";
  KataGenStateArgs a{};
  int st = gen_state_args(fn, a, B, 1, H, dk, dv, num_groups, variant, scale, eps, dtype);
  if (st) return st;
  if (!q || !k || !v || !S || !z || !o) return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  if (!aligned16(S) || !aligned16(o)) return fail(LINATT_EINVAL, std::string(fn) + ": S and o must be 16-byte aligned");
  a.q = q; a.k = k; a.v = v; a.c = c; a.S = S; a.z = z; a.o = o;
  return gen_state_launch(fn, a, KATA_GEN_DECODE, dtype, stream);
}

size_t linatt_kata_gen_decode_workspace_bytes(int B, int H, int dk, int num_groups, int variant) {
  const int rows = linatt_kata_gen_state_rows(dk, num_groups, variant);
  if (B <= 0 || H <= 0 || rows <= 0) return 0;
  const int ns = kata_gen_decode_splits(B * H, rows);
  return ns > 1 ? (size_t)B * H * ns * kGenDecPart * sizeof(float) : 0;
}

int linatt_kata_gen_decode_split(const void* q, const void* k, const void* v, const float* c,
                                 float* S, float* z, void* o, void* workspace,
                                 size_t workspace_bytes, int B, int H, int dk, int dv,
                                 int num_groups, int variant, float scale, float eps, int dtype,
                                 void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_kata_gen_decode_split";
  KataGenStateArgs a{};
  int st = gen_state_args(fn, a, B, 1, H, dk, dv, num_groups, variant, scale, eps, dtype);
  if (st) return st;
  if (!q || !k || !v || !S || !z || !o) return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  if (!aligned16(S) || !aligned16(o)) return fail(LINATT_EINVAL, std::string(fn) + ": S and o must be 16-byte aligned");
  a.nsplit = kata_gen_decode_splits(B * H, a.P);
  if (a.nsplit > 1) {
    const size_t need = (size_t)B * H * a.nsplit * kGenDecPart * sizeof(float);
    if (!workspace || workspace_bytes < need)
      return fail(LINATT_EINVAL, std::string(fn) + ": workspace smaller than linatt_kata_gen_decode_workspace_bytes");
    if (!aligned16(workspace)) return fail(LINATT_EINVAL, std::string(fn) + ": workspace must be 16-byte aligned");
    a.part = reinterpret_cast<float*>(workspace);
  }
  a.q = q; a.k = k; a.v = v; a.c = c; a.S = S; a.z = z; a.o = o;
  return gen_state_launch(fn, a, KATA_GEN_DECODE, dtype, stream);
}

int linatt_kata_gen_readout(const void* q, const float* c, const float* S, const float* z,
                            void* o, float* den, int B, int T, int H, int dk, int dv,
                            int num_groups, int variant, float scale, float eps, int dtype,
                            void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_kata_gen_readout";
  KataGenStateArgs a{};
  int st = gen_state_args(fn, a, B, T, H, dk, dv, num_groups, variant, scale, eps, dtype);
  if (st) return st;
  if (!q || !S || !z || !o || !den) return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  if (!aligned16(q) || !aligned16(S) || !aligned16(o))
    return fail(LINATT_EINVAL, std::string(fn) + ": q, S and o must be 16-byte aligned");
  a.q = q; a.c = c; a.S = const_cast<float*>(S); a.z = const_cast<float*>(z); a.o = o; a.den = den;
  return gen_state_launch(fn, a, KATA_GEN_READOUT, dtype, stream);
}

int linatt_kata_gen_update(const void* k, const void* v, const float* c, float* S, float* z,
                           int init, int B, int T, int H, int dk, int dv, int num_groups,
                           int variant, float scale, int dtype, void* stream) {
  g_last_error.clear();
  const char* fn = "linatt_kata_gen_update";
  KataGenStateArgs a{};
  int st = gen_state_args(fn, a, B, T, H, dk, dv, num_groups, variant, scale, 1.f, dtype);
  if (st) return st;
  if (!k || !v || !S || !z) return fail(LINATT_EINVAL, std::string(fn) + ": null tensor pointer");
  if (!aligned16(S) || !aligned16(k) || !aligned16(v))
    return fail(LINATT_EINVAL, std::string(fn) + ": k, v and S must be 16-byte aligned");
  a.k = k; a.v = v; a.c = c; a.S = S; a.z = z; a.init = init ? 1 : 0;
  return gen_state_launch(fn, a, KATA_GEN_UPDATE, dtype, stream);
}


}  // extern "C"
