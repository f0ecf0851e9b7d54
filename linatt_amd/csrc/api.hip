// C-ABI entry points: argument validation, dispatch to the compiled kernel
// instantiations, and per-thread error reporting.  See include/linatt_hip.h.
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/linatt_hip.h"
#include "kata_kernels.h"

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

using namespace linatt;

// Returns 1 and sets *err when a kernel exists for the combination.
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

hipError_t dispatch_bwd(const KataArgs& a, int parts, int dtype, int variant, hipStream_t s,
                        bool* found) {
  *found = false;
#define LINATT_TRY_BWD(T, DK_, DV_, M_)                                             \
  if (dtype == dtype_of<T>() && a.DK == DK_ && a.DV == DV_ && a.M == M_) {          \
    *found = true;                                                                  \
    if (variant == LINATT_KATA_SUM) return launch_kata_bwd<T, DK_, DV_, M_, true>(a, parts, s); \
    return launch_kata_bwd<T, DK_, DV_, M_, false>(a, parts, s);                    \
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

size_t linatt_kata_bwd_workspace_bytes(int B, int T, int HQ) {
  if (B <= 0 || T <= 0 || HQ <= 0) return 0;
  return (size_t)B * T * HQ * sizeof(float);
}

// Shared body of the three backward entry points; `parts` selects the
// kernels (KATA_BWD_DQ and/or KATA_BWD_DKDV).  Pointers a part does not use
// may be null.
static int kata_bwd_entry(const char* fn, int parts, const void* q, const void* k, const void* v,
                          const void* o, const float* den, const void* dout, void* dq, void* dk,
                          void* dv, void* workspace, int B, int T, int HQ, int H, int dk_dim,
                          int dv_dim, int num_groups, float scale, int variant, int dtype,
                          void* stream) {
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
  bool found = false;
  hipError_t e = dispatch_bwd(a, parts, dtype, variant, (hipStream_t)stream, &found);
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

}  // extern "C"
