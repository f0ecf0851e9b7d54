// Elementwise prologue / epilogue of the KATA token mixer, for gfx950.
//
// Replaces the two non-GEMM pieces of kata/layer.py's KataAttention.forward
// around the attention op: the causal short convolutions with SiLU on the
// projected q, k, v (:299-318, fla.modules.ShortConvolution, constructed at
// :178-197) and the fp32 output RMSNorm over each head (:539, fla.modules.
// RMSNorm constructed at :199-205; also the q/k RMSNorm at :126-128, :347).
// The projections and o_proj stay plain library GEMMs.
//
// Short convolution (depthwise, causal, kernel W):
//   z[t, c] = bias[c] + sum_{w < W} weight[c, w] x[t - (W - 1) + w, c]
//   y = silu(z) = z / (1 + e^-z)  (or y = z), the reciprocal by v_rcp_f32
// with x[t < 0] taken from a cache of the W inputs before the chunk (the
// newest last), or zero.  One lane owns kConvCh = 4 adjacent channels (one
// 8-byte load per token in 16-bit types, so C = 768 fills its 64-lane waves
// exactly) and a run of kConvTB tokens, sliding the window in registers;
// each input row is read once plus a W - 1 row halo.  The
// backward recomputes z, forms dz = dy silu'(z), dx[s] = sum_w weight[c, w]
// dz[s + W - 1 - w], and per-lane partial sums of dweight and dbias that a
// second kernel adds up in a fixed order.
//
// Rotary position embedding: see rope_kernel.
//
// RMSNorm over rows of d (fp32 arithmetic): y = x r w, r = (mean x^2 + eps)^-1/2;
// backward dx = r (g - xh mean(g xh)), g = dy w, xh = x r; dw = sum_rows dy xh.
// d / 8 lanes own a row (16 bytes each).
#include "common.h"
#include "misc_kernels.h"

namespace linatt {

namespace {

// 1 / (1 + e^-z) with the hardware reciprocal (1 ulp; an IEEE division is a
// ten-instruction sequence, and the convolutions take one per element)
__device__ __forceinline__ float sigmoidf(float z) { return __builtin_amdgcn_rcpf(1.f + __expf(-z)); }

constexpr int kConvTB = 16;  // tokens per lane
constexpr int kConvCh = 4;   // channels per lane of the short convolution

template <typename T>
__device__ __forceinline__ void load4f(const T* p, float* out) {
  const v4_t<T> v = *reinterpret_cast<const v4_t<T>*>(p);
#pragma unroll
  for (int e = 0; e < 4; ++e) out[e] = (float)v[e];
}
template <typename T>
__device__ __forceinline__ void store4f(T* p, const float* v) {
  v4_t<T> o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = (T)v[e];
  *reinterpret_cast<v4_t<T>*>(p) = o;
}

template <typename T>
__device__ __forceinline__ void load8f(const T* p, float* out) {
  const v8_t<T> v = *reinterpret_cast<const v8_t<T>*>(p);
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = (float)v[e];
}
template <>
__device__ __forceinline__ void load8f<float>(const float* p, float* out) {
  const f32x4 a = reinterpret_cast<const f32x4*>(p)[0], b = reinterpret_cast<const f32x4*>(p)[1];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    out[e] = a[e];
    out[4 + e] = b[e];
  }
}
template <typename T>
__device__ __forceinline__ void store8f(T* p, const float* v) {
  v8_t<T> o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (T)v[e];
  *reinterpret_cast<v8_t<T>*>(p) = o;
}
template <>
__device__ __forceinline__ void store8f<float>(float* p, const float* v) {
  reinterpret_cast<f32x4*>(p)[0] = f32x4{v[0], v[1], v[2], v[3]};
  reinterpret_cast<f32x4*>(p)[1] = f32x4{v[4], v[5], v[6], v[7]};
}

// kConvCh channels of input position pos of batch row b (pos < 0: the
// cache, or 0)
template <typename T, int W, typename A>
__device__ __forceinline__ void conv_input(const A& a, int b, int c0, int pos, float* out) {
  if (pos >= 0) {
    load4f<T>((const T*)a.x + ((int64_t)b * a.T + pos) * a.C + c0, out);
  } else if (a.cache_in) {
    const T* cb = (const T*)a.cache_in + ((int64_t)b * a.C + c0) * W + (W + pos);
#pragma unroll
    for (int e = 0; e < kConvCh; ++e) out[e] = (float)cb[e * W];
  } else {
#pragma unroll
    for (int e = 0; e < kConvCh; ++e) out[e] = 0.f;
  }
}

}  // namespace

template <typename T, int W>
__global__ __launch_bounds__(64) void short_conv_fwd_kernel(ConvArgs a) {
  const int cg = blockIdx.x * 64 + threadIdx.x, tb = blockIdx.y, b = blockIdx.z;
  if (kConvCh * cg >= a.C) return;
  const int c0 = kConvCh * cg, t0 = tb * kConvTB;
  float wv[kConvCh][W], bv[kConvCh];
#pragma unroll
  for (int e = 0; e < kConvCh; ++e) {
#pragma unroll
    for (int w = 0; w < W; ++w) wv[e][w] = a.w[(c0 + e) * W + w];
    bv[e] = a.bias ? a.bias[c0 + e] : 0.f;
  }
  float win[W][kConvCh];  // win[j] = input t - (W - 1) + j for the current t
#pragma unroll
  for (int j = 0; j < W - 1; ++j) conv_input<T, W>(a, b, c0, t0 - (W - 1) + j, win[j + 1]);
  const T* __restrict__ xb = (const T*)a.x + (int64_t)b * a.T * a.C + c0;
  T* __restrict__ yb = (T*)a.y + (int64_t)b * a.T * a.C + c0;
  // the run's rows up front (independent loads in flight), rows past T as zero
  v4_t<T> xr[kConvTB];
#pragma unroll
  for (int i = 0; i < kConvTB; ++i)
    xr[i] = t0 + i < a.T ? *reinterpret_cast<const v4_t<T>*>(xb + (int64_t)(t0 + i) * a.C) : v4_t<T>{};
#pragma unroll
  for (int i = 0; i < kConvTB; ++i) {
    const int t = t0 + i;
#pragma unroll
    for (int j = 0; j < W - 1; ++j)
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) win[j][e] = win[j + 1][e];
#pragma unroll
    for (int e = 0; e < kConvCh; ++e) win[W - 1][e] = (float)xr[i][e];
    if (t >= a.T) break;
    float yv[kConvCh];
#pragma unroll
    for (int e = 0; e < kConvCh; ++e) {
      float z = bv[e];
#pragma unroll
      for (int w = 0; w < W; ++w) z += wv[e][w] * win[w][e];
      yv[e] = a.act ? z * sigmoidf(z) : z;
    }
    store4f<T>(yb + (int64_t)t * a.C, yv);
  }
  // the W inputs before position T, for a later call (decode)
  if (a.cache_out && t0 <= a.T - 1 && a.T - 1 < t0 + kConvTB) {
    T* co = (T*)a.cache_out + ((int64_t)b * a.C + c0) * W;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      float v[kConvCh];
      conv_input<T, W>(a, b, c0, a.T - W + w, v);
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) co[e * W + w] = (T)v[e];
    }
  }
}

template <typename T, int W>
__global__ __launch_bounds__(64) void short_conv_bwd_kernel(ConvArgs a) {
  const int cg = blockIdx.x * 64 + threadIdx.x, tb = blockIdx.y, b = blockIdx.z;
  if (kConvCh * cg >= a.C) return;
  const int c0 = kConvCh * cg, t0 = tb * kConvTB, t1 = min(t0 + kConvTB, a.T);
  float wv[kConvCh][W], bv[kConvCh];
#pragma unroll
  for (int e = 0; e < kConvCh; ++e) {
#pragma unroll
    for (int w = 0; w < W; ++w) wv[e][w] = a.w[(c0 + e) * W + w];
    bv[e] = a.bias ? a.bias[c0 + e] : 0.f;
  }
  float win[W][kConvCh], dz[W][kConvCh];  // inputs u - (W - 1) .. u; dz[u - (W - 1)] .. dz[u]
  float dwp[kConvCh][W], dbp[kConvCh];
#pragma unroll
  for (int e = 0; e < kConvCh; ++e) {
#pragma unroll
    for (int w = 0; w < W; ++w) {
      dwp[e][w] = 0.f;
      dz[w][e] = 0.f;
    }
    dbp[e] = 0.f;
  }
#pragma unroll
  for (int j = 0; j < W - 1; ++j) conv_input<T, W>(a, b, c0, t0 - (W - 1) + j, win[j + 1]);
  const int64_t rowb = (int64_t)b * a.T;
  const T* __restrict__ xb = (const T*)a.x + rowb * a.C + c0;
  const T* __restrict__ gb = (const T*)a.dy + rowb * a.C + c0;
  T* __restrict__ dxb = (T*)a.dx + rowb * a.C + c0;
  constexpr int NU = kConvTB + W - 1;  // positions u whose dz reaches dx[t0 .. t0 + kConvTB - 1]
  v4_t<T> xr[NU], gr[NU];
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    const bool in = t0 + i < a.T;
    xr[i] = in ? *reinterpret_cast<const v4_t<T>*>(xb + (int64_t)(t0 + i) * a.C) : v4_t<T>{};
    gr[i] = in ? *reinterpret_cast<const v4_t<T>*>(gb + (int64_t)(t0 + i) * a.C) : v4_t<T>{};
  }
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    const int u = t0 + i;
    if (u >= t1 + W - 1) break;
#pragma unroll
    for (int j = 0; j < W - 1; ++j)
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) {
        win[j][e] = win[j + 1][e];
        dz[j][e] = dz[j + 1][e];
      }
    if (u < a.T) {
      float g[kConvCh];
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) {
        win[W - 1][e] = (float)xr[i][e];
        g[e] = (float)gr[i][e];
      }
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) {
        float z = bv[e];
#pragma unroll
        for (int w = 0; w < W; ++w) z += wv[e][w] * win[w][e];
        float d = g[e];
        if (a.act) {
          const float s = sigmoidf(z);
          d *= s * (1.f + z * (1.f - s));
        }
        dz[W - 1][e] = d;
      }
      if (u < t1) {  // this lane's own positions: weight and bias gradients
#pragma unroll
        for (int e = 0; e < kConvCh; ++e) {
#pragma unroll
          for (int w = 0; w < W; ++w) dwp[e][w] += dz[W - 1][e] * win[w][e];
          dbp[e] += dz[W - 1][e];
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) dz[W - 1][e] = 0.f;
    }
    const int s = u - (W - 1);  // dx[s] = sum_w weight[w] dz[s + W - 1 - w]
    if (s >= t0) {
      float dxv[kConvCh];
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) {
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) acc += wv[e][w] * dz[W - 1 - w][e];
        dxv[e] = acc;
      }
      store4f<T>(dxb + (int64_t)s * a.C, dxv);
    }
  }
  // partials: part[(b * ntb + tb)][c][0 .. W - 1 weight, W bias]
  float* pp = a.part + ((int64_t)(b * gridDim.y + tb) * a.C + c0) * (W + 1);
#pragma unroll
  for (int e = 0; e < kConvCh; ++e) {
#pragma unroll
    for (int w = 0; w < W; ++w) pp[e * (W + 1) + w] = dwp[e][w];
    pp[e * (W + 1) + W] = dbp[e];
  }
}

// out[y][i] = sum_p part[p][i] for i < n over the rows p of block row y
// (rows y rows_per .. min(np, (y + 1) rows_per) - 1), in a fixed order: 1024
// threads per block, 32 columns by 32 row phases (phase k sums rows k, k + 32,
// ... of the range, eight loads in flight), then one thread per column adds
// the 32 phase sums.  With split_w > 0 the columns are [c][0 .. split_w - 1
// weight, split_w bias] of a convolution and go to dw[c][w] and db[c] instead.
__global__ __launch_bounds__(1024) void colsum_kernel(const float* __restrict__ part,
                                                      float* __restrict__ out, int np, int n,
                                                      int rows_per, int split_w = 0,
                                                      float* __restrict__ db = nullptr) {
  __shared__ float red[32][33];
  const int c = blockIdx.x * 32 + (threadIdx.x & 31), k = threadIdx.x >> 5;
  const int p0 = blockIdx.y * rows_per, p1 = min(np, p0 + rows_per);
  float s = 0.f;
  if (c < n) {
    int p = p0 + k;
    for (; p + 7 * 32 < p1; p += 8 * 32) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = part[(int64_t)(p + 32 * j) * n + c];
#pragma unroll
      for (int j = 0; j < 8; ++j) s += v[j];
    }
    for (; p < p1; p += 32) s += part[(int64_t)p * n + c];
  }
  red[k][threadIdx.x & 31] = s;
  __syncthreads();
  if (threadIdx.x < 32 && c < n) {
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < 32; ++j) t += red[j][threadIdx.x];
    if (split_w == 0) {
      out[(int64_t)blockIdx.y * n + c] = t;
    } else {
      const int cc = c / (split_w + 1), w = c % (split_w + 1);
      if (w < split_w) out[cc * split_w + w] = t;
      else if (db) db[cc] = t;
    }
  }
}

// column sums of a (np, n) array in one block row
static void colsum(const float* part, float* out, int np, int n, hipStream_t stream) {
  colsum_kernel<<<dim3((n + 31) / 32), dim3(1024), 0, stream>>>(part, out, np, n, np);
}

hipError_t launch_colsum(const float* part, float* out, int np, int n, hipStream_t stream) {
  colsum(part, out, np, n, stream);
  return hipGetLastError();
}

// dweight (C, W) and dbias (C) from the convolution partials [np][C][W + 1]
static void conv_grad_sums(const float* part, float* dw, float* db, int np, int C, int W,
                           hipStream_t stream) {
  const int n = C * (W + 1);
  colsum_kernel<<<dim3((n + 31) / 32), dim3(1024), 0, stream>>>(part, dw, np, n, np, W, db);
}

template <typename T>
hipError_t launch_short_conv(const ConvArgs& a, int W, bool bwd, hipStream_t stream) {
  const int ntb = (a.T + kConvTB - 1) / kConvTB;
  const dim3 grid((a.C / kConvCh + 63) / 64, ntb, a.B);
#define LINATT_CONV_W(WW)                                                              \
  case WW:                                                                             \
    if (bwd) short_conv_bwd_kernel<T, WW><<<grid, dim3(64), 0, stream>>>(a);           \
    else short_conv_fwd_kernel<T, WW><<<grid, dim3(64), 0, stream>>>(a);               \
    break;
  switch (W) {
    LINATT_CONV_W(2)
    LINATT_CONV_W(3)
    LINATT_CONV_W(4)
    default: return hipErrorInvalidValue;
  }
#undef LINATT_CONV_W
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !bwd) return e;
  conv_grad_sums(a.part, a.dw, a.db, a.B * ntb, a.C, W, stream);
  return hipGetLastError();
}

size_t short_conv_bwd_workspace(int B, int T, int C, int W) {
  const size_t ntb = (size_t)(T + kConvTB - 1) / kConvTB;
  return (size_t)B * ntb * C * (W + 1) * sizeof(float);  // the partials
}

// ---------------------------------------------------------------------------
// RMSNorm
// ---------------------------------------------------------------------------
constexpr int kRmsRows = 4;  // rows per lane group and step, forward and backward

template <typename T, int L>  // L = d / 8 lanes per row
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const T* __restrict__ x,
                                                          const float* __restrict__ wt,
                                                          T* __restrict__ y,
                                                          float* __restrict__ rstd, int n,
                                                          float eps) {
  constexpr int d = 8 * L, RPB = 256 / L;
  const int li = threadIdx.x % L;
  const int row0 = blockIdx.x * RPB * kRmsRows + threadIdx.x / L;
  float wv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) wv[e] = wt ? wt[8 * li + e] : 1.f;
  float v[kRmsRows][8];
#pragma unroll
  for (int r = 0; r < kRmsRows; ++r) {
    const int row = row0 + r * RPB;
    if (row < n) load8f<T>(x + (int64_t)row * d + 8 * li, v[r]);
  }
#pragma unroll
  for (int r = 0; r < kRmsRows; ++r) {
    const int row = row0 + r * RPB;
    if (row >= n) break;  // uniform over the row's L lanes
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[r][e] * v[r][e];
    ss = group_sum<L>(ss);
    const float rr = rsqrtf(ss / d + eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[r][e] *= rr * wv[e];
    store8f<T>(y + (int64_t)row * d + 8 * li, v[r]);
    if (li == 0) rstd[row] = rr;
  }
}

template <typename T, int L>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const T* __restrict__ x,
                                                          const float* __restrict__ wt,
                                                          const float* __restrict__ rstd,
                                                          const T* __restrict__ dy,
                                                          T* __restrict__ dx,
                                                          float* __restrict__ part, int n) {
  constexpr int d = 8 * L, RPB = 256 / L;
  __shared__ float red[RPB][d + 1];
  const int li = threadIdx.x % L, rg = threadIdx.x / L;
  float dwp[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) dwp[e] = 0.f;
  float wv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) wv[e] = wt ? wt[8 * li + e] : 1.f;
  // kRmsRows rows per lane group and step: every load of the step is issued
  // before the first row's arithmetic
  for (int row0 = blockIdx.x * RPB * kRmsRows + rg; row0 < n; row0 += gridDim.x * RPB * kRmsRows) {
    float xv[kRmsRows][8], g[kRmsRows][8], r[kRmsRows];
#pragma unroll
    for (int k = 0; k < kRmsRows; ++k) {
      const int row = row0 + k * RPB;
      if (row < n) {
        load8f<T>(x + (int64_t)row * d + 8 * li, xv[k]);
        load8f<T>(dy + (int64_t)row * d + 8 * li, g[k]);
        r[k] = rstd[row];
      }
    }
#pragma unroll
    for (int k = 0; k < kRmsRows; ++k) {
      const int row = row0 + k * RPB;
      if (row >= n) break;  // uniform over the row's L lanes
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xv[k][e] *= r[k];  // xh
        dwp[e] += g[k][e] * xv[k][e];
        g[k][e] *= wv[e];
        dot += g[k][e] * xv[k][e];
      }
      dot = group_sum<L>(dot) / d;
#pragma unroll
      for (int e = 0; e < 8; ++e) g[k][e] = r[k] * (g[k][e] - xv[k][e] * dot);
      store8f<T>(dx + (int64_t)row * d + 8 * li, g[k]);
    }
  }
  // per-block weight-gradient partial: sum over the block's row groups
#pragma unroll
  for (int e = 0; e < 8; ++e) red[rg][8 * li + e] = dwp[e];
  __syncthreads();
  for (int c = threadIdx.x; c < d; c += 256) {
    float s = 0.f;
    for (int k = 0; k < RPB; ++k) s += red[k][c];
    part[(int64_t)blockIdx.x * d + c] = s;
  }
}

int rmsnorm_bwd_blocks(int n, int d) {
  const int rpb = 256 / (d / 8) * kRmsRows;
  const int need = (n + rpb - 1) / rpb;
  return need < 1024 ? need : 1024;
}

template <typename T>
hipError_t launch_rmsnorm(const void* x, const float* w, const float* rstd_in, const void* dy,
                          void* out, float* rstd_out, float* dw, float* part, int n, int d,
                          float eps, bool bwd, hipStream_t stream) {
  const int L = d / 8;
  const int rpb = 256 / L;
  const int nbf = (n + rpb * kRmsRows - 1) / (rpb * kRmsRows), nbb = rmsnorm_bwd_blocks(n, d);
#define LINATT_RMS_L(LL)                                                                          \
  case LL:                                                                                        \
    if (bwd)                                                                                      \
      rmsnorm_bwd_kernel<T, LL><<<dim3(nbb), dim3(256), 0, stream>>>(                             \
          (const T*)x, w, rstd_in, (const T*)dy, (T*)out, part, n);                               \
    else                                                                                          \
      rmsnorm_fwd_kernel<T, LL><<<dim3(nbf), dim3(256), 0, stream>>>((const T*)x, w, (T*)out,     \
                                                                     rstd_out, n, eps);           \
    break;
  switch (L) {
    LINATT_RMS_L(1)
    LINATT_RMS_L(2)
    LINATT_RMS_L(4)
    LINATT_RMS_L(8)
    LINATT_RMS_L(16)
    LINATT_RMS_L(32)
    LINATT_RMS_L(64)
    default: return hipErrorInvalidValue;
  }
#undef LINATT_RMS_L
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !bwd || !dw) return e;
  colsum(part, dw, nbb, d, stream);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Rotary position embedding (fla.modules.RotaryEmbedding as the mixer uses
// it, kata/layer.py:130-148, 352-372): pair p of the first rot_dim dims of
// each (B, T, H, D) row -- (2p, 2p + 1) interleaved, (p, p + rot_dim / 2)
// otherwise -- is rotated by the angle (t + offset) base^(-2p / rot_dim),
// in fp32; inverse = 1 rotates by minus that angle (the backward).  Dims past
// rot_dim pass through.  rope_rows_kernel (after the fused q/k prologue, whose
// table and lane layout it shares) takes the shapes the mixer uses: 4 dims per
// lane, 16-token runs, one (cos, sin') table per block.  rope_kernel, one
// thread per pair, takes the rest.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                   int64_t rows, int T_, int H, int D,
                                                   int rot_dim, float log2_base, int offset,
                                                   int interleaved, float sign) {
  const int half = rot_dim / 2, npass = (D - rot_dim) / 2;
  const int per_row = half + npass;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * per_row) return;
  const int64_t row = i / per_row;
  const int p = (int)(i % per_row);
  const T* xr = x + row * D;
  T* yr = y + row * D;
  if (p >= half) {  // two pass-through dims past rot_dim
    const int d = rot_dim + 2 * (p - half);
    yr[d] = xr[d];
    yr[d + 1] = xr[d + 1];
    return;
  }
  const int t = (int)((row / H) % T_) + offset;
  const float inv_freq = exp2f(-(2.f * p / rot_dim) * log2_base);
  float sn, cs;
  sincosf((float)t * inv_freq, &sn, &cs);
  sn *= sign;
  const int d0 = interleaved ? 2 * p : p, d1 = interleaved ? 2 * p + 1 : p + half;
  const float a = (float)xr[d0], b = (float)xr[d1];
  yr[d0] = (T)(a * cs - b * sn);
  yr[d1] = (T)(a * sn + b * cs);
}


// ---------------------------------------------------------------------------
// Fused q/k prologue.  kata/layer.py:305-372 runs three modules in a row on q
// and on k: the short convolution with SiLU (fla ShortConvolution), the
// per-head norm (fla RMSNorm with an fp32 weight, or fla's l2norm) and the
// rotary embedding (fla RotaryEmbedding: interleaved over the whole head, or,
// with rope_group, non-interleaved over each E-dim group).  Here one pass
// reads the projection output once and writes the rotated rows once; the
// intermediates stay in fp32 registers (the three-module chain rounds them to
// the input dtype twice).  Per (token, head):
//   z = bias + sum_w weight[w] x[t - (W - 1) + w],   u = act(z),
//   n = u r nw,  r = (inv_n sum_d u^2 + eps)^-1/2    (RMSNorm: inv_n = 1 / D;
//                                                      L2: inv_n = 1, no nw),
//   y_j = n_j cos_j + n_partner(j) sin'_j,
// where, for rotation rows of rw dims whose first rot dims rotate, the pair
// of dim j is (j, j ^ 1) when interleaved and (j, j +- rot / 2) otherwise,
// cos_j / sin'_j hold cos and -sin (first of a pair) or +sin (second) of the
// angle (t + offset) base^(-2p / rot), and dims past rot have (1, 0).
// A lane owns kConvCh = 4 channels and a run of kQkTB tokens, as in the
// convolution; a head's D / 4 lanes are adjacent in one wave, so the norm's
// sums are DPP reductions over them.  The angles come from an LDS table
// per block (tokens x rotation dims) filled with the formula of rope_kernel,
// so each table entry costs one sincos per block rather than one per lane.
// The backward recomputes z, u, r, rotates dy back (sin' negated) to g, then
//   du = r (g nw - uh inv_n sum_d g nw uh),  uh = u r,  dnw += g uh,
//   dz = du act'(z), and dx, dweight, dbias as in short_conv_bwd_kernel.
// ---------------------------------------------------------------------------
constexpr int kQkTB = 16;      // tokens per lane and block
constexpr int kQkMaxRw = 128;  // widest rotation row (D <= 128)

namespace {
// (cos, sin') of rotation dims j < a.rw for the nrow positions from pos0:
// one sincos per rotated pair, written to both of its dims; (1, 0) past rot
__device__ __forceinline__ void fill_rot_table(const QKArgs& a, int pos0, int nrow,
                                               float (*tc)[kQkMaxRw], float (*ts)[kQkMaxRw]) {
  const int half = a.rot / 2, npair = half + (a.rw - a.rot);  // pairs, then pass-through dims
  for (int i = threadIdx.x; i < nrow * npair; i += blockDim.x) {
    const int r = i / npair, p = i % npair;
    if (p >= half) {
      const int j = a.rot + (p - half);
      tc[r][j] = 1.f;
      ts[r][j] = 0.f;
      continue;
    }
    float cs, sn;
    const float inv_freq = exp2f(-(2.f * p / a.rot) * a.log2_base);
    sincosf((float)(pos0 + r + a.offset) * inv_freq, &sn, &cs);
    const int j0 = a.interleaved ? 2 * p : p, j1 = a.interleaved ? 2 * p + 1 : p + half;
    tc[r][j0] = cs;
    ts[r][j0] = -sn;
    tc[r][j1] = cs;
    ts[r][j1] = sn;
  }
}

// the partner value of each of a lane's four rotation dims: in the lane when
// interleaved, else in lane + dl (dl = 0 past rot, where sin' = 0)
__device__ __forceinline__ void rot_partner(const float* v, float* p, bool inter, int src) {
  if (inter) {
#pragma unroll
    for (int e = 0; e < kConvCh; ++e) p[e] = v[e ^ 1];
  } else {
#pragma unroll
    for (int e = 0; e < kConvCh; ++e) p[e] = __shfl(v[e], src);
  }
}
}  // namespace

template <typename T, int W, int L>  // L = D / 4 lanes per head
__global__ __launch_bounds__(256) void qk_prologue_fwd_kernel(QKArgs a) {
  __shared__ __align__(16) float tc[kQkTB][kQkMaxRw], ts[kQkTB][kQkMaxRw];
  const int cg = blockIdx.x * blockDim.x + threadIdx.x, tb = blockIdx.y, b = blockIdx.z;
  const int t0 = tb * kQkTB;
  if (a.rot) fill_rot_table(a, t0, kQkTB, tc, ts);
  __syncthreads();
  // every lane is in range: the block is a whole number of heads dividing H
  const int c0 = kConvCh * cg, d0 = c0 % a.D, j0 = d0 % (a.rw > 0 ? a.rw : 1);
  const int lane = threadIdx.x & 63;
  const int src = lane + (j0 < a.rot / 2 ? a.rot / 8 : (j0 < a.rot ? -(a.rot / 8) : 0));
  float wv[kConvCh][W], bv[kConvCh], nwv[kConvCh];
#pragma unroll
  for (int e = 0; e < kConvCh; ++e) {
#pragma unroll
    for (int w = 0; w < W; ++w) wv[e][w] = a.w[(c0 + e) * W + w];
    bv[e] = a.bias ? a.bias[c0 + e] : 0.f;
    nwv[e] = a.nw ? a.nw[d0 + e] : 1.f;
  }
  float win[W][kConvCh];
#pragma unroll
  for (int j = 0; j < W - 1; ++j) conv_input<T, W>(a, b, c0, t0 - (W - 1) + j, win[j + 1]);
  const T* __restrict__ xb = (const T*)a.x + (int64_t)b * a.T * a.C + c0;
  T* __restrict__ yb = (T*)a.y + (int64_t)b * a.T * a.C + c0;
  v4_t<T> xr[kQkTB];
#pragma unroll
  for (int i = 0; i < kQkTB; ++i)
    xr[i] = t0 + i < a.T ? *reinterpret_cast<const v4_t<T>*>(xb + (int64_t)(t0 + i) * a.C) : v4_t<T>{};
#pragma unroll
  for (int i = 0; i < kQkTB; ++i) {
    const int t = t0 + i;
#pragma unroll
    for (int j = 0; j < W - 1; ++j)
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) win[j][e] = win[j + 1][e];
#pragma unroll
    for (int e = 0; e < kConvCh; ++e) win[W - 1][e] = (float)xr[i][e];
    if (t >= a.T) break;  // uniform over the block
    float u[kConvCh], ss = 0.f;
#pragma unroll
    for (int e = 0; e < kConvCh; ++e) {
      float z = bv[e];
#pragma unroll
      for (int w = 0; w < W; ++w) z += wv[e][w] * win[w][e];
      u[e] = a.act ? z * sigmoidf(z) : z;
      ss += u[e] * u[e];
    }
    if (a.norm) {
      const float r = rsqrtf(group_sum<L>(ss) * a.inv_n + a.eps);
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) u[e] *= r * nwv[e];
    }
    if (a.rot) {
      const f32x4 c = *reinterpret_cast<const f32x4*>(&tc[i][j0]);
      const f32x4 s = *reinterpret_cast<const f32x4*>(&ts[i][j0]);
      float pv[kConvCh];
      rot_partner(u, pv, a.interleaved, src);
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) u[e] = u[e] * c[e] + pv[e] * s[e];
    }
    store4f<T>(yb + (int64_t)t * a.C, u);
  }
  if (a.cache_out && t0 <= a.T - 1 && a.T - 1 < t0 + kQkTB) {
    T* co = (T*)a.cache_out + ((int64_t)b * a.C + c0) * W;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      float v[kConvCh];
      conv_input<T, W>(a, b, c0, a.T - W + w, v);
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) co[e * W + w] = (T)v[e];
    }
  }
}

template <typename T, int W, int L>
__global__ __launch_bounds__(256) void qk_prologue_bwd_kernel(QKArgs a) {
  constexpr int NU = kQkTB + W - 1;  // positions u whose dz reaches dx[t0 .. t0 + kQkTB - 1]
  __shared__ __align__(16) float tc[kQkTB + 3][kQkMaxRw], ts[kQkTB + 3][kQkMaxRw];
  const int cg = blockIdx.x * blockDim.x + threadIdx.x, tb = blockIdx.y, b = blockIdx.z;
  const int t0 = tb * kQkTB, t1 = min(t0 + kQkTB, a.T);
  if (a.rot) fill_rot_table(a, t0, NU, tc, ts);
  __syncthreads();
  // every lane is in range: the block is a whole number of heads dividing H
  const int c0 = kConvCh * cg, d0 = c0 % a.D, j0 = d0 % (a.rw > 0 ? a.rw : 1);
  const int lane = threadIdx.x & 63;
  const int src = lane + (j0 < a.rot / 2 ? a.rot / 8 : (j0 < a.rot ? -(a.rot / 8) : 0));
  float wv[kConvCh][W], bv[kConvCh], nwv[kConvCh];
#pragma unroll
  for (int e = 0; e < kConvCh; ++e) {
#pragma unroll
    for (int w = 0; w < W; ++w) wv[e][w] = a.w[(c0 + e) * W + w];
    bv[e] = a.bias ? a.bias[c0 + e] : 0.f;
    nwv[e] = a.nw ? a.nw[d0 + e] : 1.f;
  }
  float win[W][kConvCh], dz[W][kConvCh];
  float dwp[kConvCh][W], dbp[kConvCh], dnp[kConvCh];
#pragma unroll
  for (int e = 0; e < kConvCh; ++e) {
#pragma unroll
    for (int w = 0; w < W; ++w) {
      dwp[e][w] = 0.f;
      dz[w][e] = 0.f;
    }
    dbp[e] = 0.f;
    dnp[e] = 0.f;
  }
#pragma unroll
  for (int j = 0; j < W - 1; ++j) conv_input<T, W>(a, b, c0, t0 - (W - 1) + j, win[j + 1]);
  const int64_t rowb = (int64_t)b * a.T;
  const T* __restrict__ xb = (const T*)a.x + rowb * a.C + c0;
  const T* __restrict__ gb = (const T*)a.dy + rowb * a.C + c0;
  T* __restrict__ dxb = (T*)a.dx + rowb * a.C + c0;
  v4_t<T> xr[NU], gr[NU];
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    const bool in = t0 + i < a.T;
    xr[i] = in ? *reinterpret_cast<const v4_t<T>*>(xb + (int64_t)(t0 + i) * a.C) : v4_t<T>{};
    gr[i] = in ? *reinterpret_cast<const v4_t<T>*>(gb + (int64_t)(t0 + i) * a.C) : v4_t<T>{};
  }
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    const int u = t0 + i;
    if (u >= t1 + W - 1) break;  // uniform over the block
#pragma unroll
    for (int j = 0; j < W - 1; ++j)
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) {
        win[j][e] = win[j + 1][e];
        dz[j][e] = dz[j + 1][e];
      }
    if (u < a.T) {
      float z[kConvCh], uv[kConvCh], g[kConvCh], ss = 0.f;
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) {
        win[W - 1][e] = (float)xr[i][e];
        g[e] = (float)gr[i][e];
      }
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) {
        z[e] = bv[e];
#pragma unroll
        for (int w = 0; w < W; ++w) z[e] += wv[e][w] * win[w][e];
        uv[e] = a.act ? z[e] * sigmoidf(z[e]) : z[e];
        ss += uv[e] * uv[e];
      }
      if (a.rot) {  // g = R^T dy
        const f32x4 c = *reinterpret_cast<const f32x4*>(&tc[i][j0]);
        const f32x4 s = *reinterpret_cast<const f32x4*>(&ts[i][j0]);
        float pv[kConvCh];
        rot_partner(g, pv, a.interleaved, src);
#pragma unroll
        for (int e = 0; e < kConvCh; ++e) g[e] = g[e] * c[e] - pv[e] * s[e];
      }
      if (a.norm) {
        const float r = rsqrtf(group_sum<L>(ss) * a.inv_n + a.eps);
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < kConvCh; ++e) {
          const float uh = uv[e] * r;
          if (u < t1) dnp[e] += g[e] * uh;
          g[e] *= nwv[e];
          dot += g[e] * uh;
          uv[e] = uh;
        }
        dot = group_sum<L>(dot) * a.inv_n;
#pragma unroll
        for (int e = 0; e < kConvCh; ++e) g[e] = r * (g[e] - uv[e] * dot);
      }
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) {
        float d = g[e];
        if (a.act) {
          const float sg = sigmoidf(z[e]);
          d *= sg * (1.f + z[e] * (1.f - sg));
        }
        dz[W - 1][e] = d;
      }
      if (u < t1) {
#pragma unroll
        for (int e = 0; e < kConvCh; ++e) {
#pragma unroll
          for (int w = 0; w < W; ++w) dwp[e][w] += dz[W - 1][e] * win[w][e];
          dbp[e] += dz[W - 1][e];
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) dz[W - 1][e] = 0.f;
    }
    const int s = u - (W - 1);
    if (s >= t0) {
      float dxv[kConvCh];
#pragma unroll
      for (int e = 0; e < kConvCh; ++e) {
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) acc += wv[e][w] * dz[W - 1 - w][e];
        dxv[e] = acc;
      }
      store4f<T>(dxb + (int64_t)s * a.C, dxv);
    }
  }
  const int64_t prow = (int64_t)b * gridDim.y + tb;
  float* pp = a.part + (prow * a.C + c0) * (W + 1);
#pragma unroll
  for (int e = 0; e < kConvCh; ++e) {
#pragma unroll
    for (int w = 0; w < W; ++w) pp[e * (W + 1) + w] = dwp[e][w];
    pp[e * (W + 1) + W] = dbp[e];
  }
  if (a.nw) {  // the block's heads summed in LDS (the table's space): one row of D per block
    __syncthreads();
    float* red = &tc[0][0];
    *reinterpret_cast<f32x4*>(red + kConvCh * threadIdx.x) = f32x4{dnp[0], dnp[1], dnp[2], dnp[3]};
    __syncthreads();
    const int nh = blockDim.x / L;
    for (int d = threadIdx.x; d < a.D; d += blockDim.x) {
      float sum = 0.f;
      for (int hh = 0; hh < nh; ++hh) sum += red[hh * a.D + d];
      a.npart[(prow * gridDim.x + blockIdx.x) * a.D + d] = sum;
    }
  }
}

namespace {
// lanes per block: the D / 4 lanes of each of h heads, h the largest divisor
// of H with at most 256 lanes, so that blocks hold whole heads and no lane is
// out of range
int qk_threads(int C, int D) {
  const int L = D / kConvCh, H = C / D;
  int h = 1;
  for (int c = 1; c <= H && c * L <= 256; ++c)
    if (H % c == 0) h = c;
  return h * L;
}
}  // namespace

// backward workspace: the convolution partials [B ntb][C][W + 1], then the
// norm-weight partials [B ntb][H / h][D]
template <typename T>
hipError_t launch_qk_prologue(const QKArgs& args, int W, bool bwd, hipStream_t stream) {
  const int ntb = (args.T + kQkTB - 1) / kQkTB, nthr = qk_threads(args.C, args.D);
  const int n = args.C * (W + 1), np = args.B * ntb;
  QKArgs a = args;
  if (bwd) a.npart = a.part + (size_t)np * n;
  const dim3 grid(a.C / kConvCh / nthr, ntb, a.B), block(nthr);
#define LINATT_QK(WW, LL)                                                            \
  if (W == WW && a.D / 4 == LL) {                                                   \
    if (bwd) qk_prologue_bwd_kernel<T, WW, LL><<<grid, block, 0, stream>>>(a);      \
    else qk_prologue_fwd_kernel<T, WW, LL><<<grid, block, 0, stream>>>(a);          \
    launched = true;                                                                \
  }
  bool launched = false;
  LINATT_QK(2, 8) LINATT_QK(2, 16) LINATT_QK(2, 32)
  LINATT_QK(3, 8) LINATT_QK(3, 16) LINATT_QK(3, 32)
  LINATT_QK(4, 8) LINATT_QK(4, 16) LINATT_QK(4, 32)
#undef LINATT_QK
  if (!launched) return hipErrorInvalidValue;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !bwd) return e;
  conv_grad_sums(a.part, a.dw, a.db, np, a.C, W, stream);
  if ((e = hipGetLastError()) != hipSuccess || !a.nw || !a.dnw) return e;
  colsum(a.npart, a.dnw, np * (int)grid.x, a.D, stream);
  return hipGetLastError();
}

size_t qk_prologue_bwd_workspace(int B, int T, int C, int D, int W) {
  const size_t np = (size_t)B * ((T + kQkTB - 1) / kQkTB);
  const size_t nblk = (size_t)C / kConvCh / qk_threads(C, D);
  return (np * C * (W + 1) + np * nblk * D) * sizeof(float);
}

// Rotary embedding on the fused prologue's layout: x, y (B, T, H D) rows; a
// lane owns 4 dims and a run of kQkTB tokens; a block holds whole heads.
template <typename T>
__global__ __launch_bounds__(256) void rope_rows_kernel(QKArgs a, float sign) {
  __shared__ __align__(16) float tc[kQkTB][kQkMaxRw], ts[kQkTB][kQkMaxRw];
  const int cg = blockIdx.x * blockDim.x + threadIdx.x, t0 = blockIdx.y * kQkTB, b = blockIdx.z;
  fill_rot_table(a, t0, kQkTB, tc, ts);
  __syncthreads();
  const int c0 = kConvCh * cg, j0 = c0 % a.rw, lane = threadIdx.x & 63;
  const int src = lane + (j0 < a.rot / 2 ? a.rot / 8 : (j0 < a.rot ? -(a.rot / 8) : 0));
  const T* xb = (const T*)a.x + (int64_t)b * a.T * a.C + c0;  // y may equal x
  T* yb = (T*)a.y + (int64_t)b * a.T * a.C + c0;
  v4_t<T> xr[kQkTB];
#pragma unroll
  for (int i = 0; i < kQkTB; ++i)
    xr[i] = t0 + i < a.T ? *reinterpret_cast<const v4_t<T>*>(xb + (int64_t)(t0 + i) * a.C) : v4_t<T>{};
#pragma unroll
  for (int i = 0; i < kQkTB; ++i) {
    if (t0 + i >= a.T) break;  // uniform over the block
    float u[kConvCh], pv[kConvCh];
#pragma unroll
    for (int e = 0; e < kConvCh; ++e) u[e] = (float)xr[i][e];
    const f32x4 c = *reinterpret_cast<const f32x4*>(&tc[i][j0]);
    const f32x4 s = *reinterpret_cast<const f32x4*>(&ts[i][j0]);
    rot_partner(u, pv, a.interleaved, src);
#pragma unroll
    for (int e = 0; e < kConvCh; ++e) u[e] = u[e] * c[e] + pv[e] * (sign * s[e]);
    store4f<T>(yb + (int64_t)(t0 + i) * a.C, u);
  }
}

template <typename T>
hipError_t launch_rope(const void* x, void* y, int B, int T_, int H, int D, int rot_dim,
                       float base, int offset, int interleaved, int inverse, hipStream_t stream) {
  const float sign = inverse ? -1.f : 1.f;
  // half-split partners come from lane +- rot / 8 by a wave shuffle, so a
  // head's D / 4 lanes must not cross a wave boundary: D / 4 must divide 64
  const bool rows_form = D % 4 == 0 && D <= kQkMaxRw &&
                         (interleaved || (rot_dim % 8 == 0 && 64 % (D / 4) == 0)) &&
                         B <= 65535 && (T_ + kQkTB - 1) / kQkTB <= 65535 &&
                         (int64_t)H * D <= INT32_MAX / 8 &&
                         (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                         (reinterpret_cast<uintptr_t>(y) & 15) == 0;
  if (rows_form) {
    QKArgs a{};
    a.x = x; a.y = y; a.B = B; a.T = T_; a.C = H * D; a.D = D;
    a.rw = D; a.rot = rot_dim; a.interleaved = interleaved ? 1 : 0; a.offset = offset;
    a.log2_base = log2f(base);
    const int nthr = qk_threads(a.C, D);
    rope_rows_kernel<T><<<dim3(a.C / kConvCh / nthr, (T_ + kQkTB - 1) / kQkTB, B), dim3(nthr), 0,
                          stream>>>(a, sign);
    return hipGetLastError();
  }
  const int64_t rows = (int64_t)B * T_ * H;
  const int64_t n = rows * (rot_dim / 2 + (D - rot_dim) / 2);
  rope_kernel<T><<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream>>>(
      (const T*)x, (T*)y, rows, T_, H, D, rot_dim, log2f(base), offset, interleaved, sign);
  return hipGetLastError();
}

template hipError_t launch_qk_prologue<__bf16>(const QKArgs&, int, bool, hipStream_t);
template hipError_t launch_qk_prologue<_Float16>(const QKArgs&, int, bool, hipStream_t);
template hipError_t launch_qk_prologue<float>(const QKArgs&, int, bool, hipStream_t);

template hipError_t launch_rope<__bf16>(const void*, void*, int, int, int, int, int, float, int, int,
                                        int, hipStream_t);
template hipError_t launch_rope<_Float16>(const void*, void*, int, int, int, int, int, float, int,
                                          int, int, hipStream_t);
template hipError_t launch_rope<float>(const void*, void*, int, int, int, int, int, float, int, int,
                                       int, hipStream_t);

template hipError_t launch_short_conv<__bf16>(const ConvArgs&, int, bool, hipStream_t);
template hipError_t launch_short_conv<_Float16>(const ConvArgs&, int, bool, hipStream_t);
template hipError_t launch_short_conv<float>(const ConvArgs&, int, bool, hipStream_t);
template hipError_t launch_rmsnorm<__bf16>(const void*, const float*, const float*, const void*,
                                           void*, float*, float*, float*, int, int, float, bool,
                                           hipStream_t);
template hipError_t launch_rmsnorm<_Float16>(const void*, const float*, const float*, const void*,
                                             void*, float*, float*, float*, int, int, float, bool,
                                             hipStream_t);
template hipError_t launch_rmsnorm<float>(const void*, const float*, const float*, const void*,
                                          void*, float*, float*, float*, int, int, float, bool,
                                          hipStream_t);

}  // namespace linatt
