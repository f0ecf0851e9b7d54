// KATA-SPD recurrent state for every flash score the mixer trains, for
// decoding (gfx950).
//
// The reference's flash branch keeps no decode state (kata/layer.py:492,
// final_state = None), so each cached decode step there attends to itself
// only.  Every flash score has an exact state form.  With
//   psi_cat(x)_p = s x[gE + a] x[gE + b],        p = g E^2 + a E + b  (P = M E^2)
//   psi_sum(x)_p = s sum_g x[gE + a] x[gE + b],  p = a E + b          (P = E^2)
// (s = scale; psi(q) . psi(k) = sum_g (s q_g.k_g)^2 for the concat score of
// kata/parallel_kata_attn.py:49-75, sum_{g,h} (s q_g.k_h)^2 for the sum score
// of :539-576), and a decay factor f_ts = exp(c_t - c_s) for the decayed
// score of :291-310 (c non-increasing, as the mixer's
// c = cumsum(-exp(A_log) softplus(.)) is, so its min(., 0) clamp is inactive):
//   S_t = f_{t,t-1} S_{t-1} + psi(k_t) v_t^T,  z_t = f_{t,t-1} z_{t-1} + psi(k_t)
//   o_t = psi(q_t)^T S_t / max(psi(q_t) . z_t, eps).
// c is the cumulative log-decay within one call (the mixer's cumsum over the
// call's tokens), so a stored state sits at c = 0 of the next call.
//
// psi(x)_{(a,b)} = psi(x)_{(b,a)} for both scores, so the state may also be
// kept packed (tri = 1): one row per unordered pair a <= b of each group,
//   p = g TE + a E - a (a - 1) / 2 + (b - a),  TE = E (E + 1) / 2,
// (the concat score's P = M TE, the sum score's P = TE).  A packed row equals
// the full layout's row (a, b) bit for bit (the same products in the same
// order); the readouts weigh an off-diagonal row's q-side feature by 2.
//
// Three kernels, fp32 throughout (the state is fp32 (B, H, P, 64)):
//   kata_gen_decode_kernel   one token per (b, h): S, z updated in place, o
//   kata_gen_readout_kernel  a prefill continued from a state: the flash
//                            forward's (o, den) over the call's tokens plus
//                            f_t psi(q_t)^T S and f_t psi(q_t) . z
//   kata_gen_update_kernel   S <- f_T S + sum_s f_Ts psi(k_s) v_s^T (and z)
// The concat score without decay at (dk, M) = (64, 2), (64, 4) keeps its
// MFMA state-form kernels (kata_state.hip); these cover the rest.
#include "common.h"
#include "kata_kernels.h"

namespace linatt {

namespace {

constexpr int kGenDV = 64;

// State row p as (group, a, b) and the weight of its q-side feature in a
// readout (2 for an off-diagonal packed row, which stands for (a, b) and
// (b, a)).  The packed row index is inverted by the quadratic formula for
// the row start a E - a (a - 1) / 2 and an exact integer correction.
struct RowPair {
  int g, a, b;
  float w;
};

__device__ __forceinline__ RowPair row_pair(const KataGenStateArgs& k, int p) {
  RowPair r;
  if (!k.tri) {
    r.g = k.sum ? 0 : p >> (2 * k.lgE);
    r.a = (p >> k.lgE) & (k.E - 1);
    r.b = p & (k.E - 1);
    r.w = 1.f;
    return r;
  }
  r.g = k.sum ? 0 : p / k.TE;
  const int q = p - r.g * k.TE, n = 2 * k.E + 1;
  int i = (int)((n - sqrtf((float)(n * n - 8 * q))) * 0.5f);
  i = min(max(i, 0), k.E - 1);
  while (i > 0 && i * k.E - i * (i - 1) / 2 > q) --i;
  while (i + 1 < k.E && (i + 1) * k.E - (i + 1) * i / 2 <= q) ++i;
  r.a = i;
  r.b = i + q - (i * k.E - i * (i - 1) / 2);
  r.w = r.a == r.b ? 1.f : 2.f;
  return r;
}

// feature (a, b) of group g of the row x (fp32), scaled by s; the product
// x_a x_b is rounded before the scale, so (a, b) and (b, a) are equal bit
// for bit and the full layout's state is exactly symmetric
__device__ __forceinline__ float psi_feat(const float* x, const RowPair& r, int E, int M, bool sum,
                                          float s) {
  if (!sum) return s * (x[r.g * E + r.a] * x[r.g * E + r.b]);
  float acc = 0.f;
  for (int g = 0; g < M; ++g) acc += x[g * E + r.a] * x[g * E + r.b];
  return s * acc;
}

template <typename T>
__device__ __forceinline__ float ldf(const void* p, int64_t i) {
  return (float)reinterpret_cast<const T*>(p)[i];
}

}  // namespace

// One workgroup per (b, h); 16 threads per state row (4 value columns each),
// 16 rows per pass; q, k (B, H, dk), v, o (B, H, 64); c (B, H) the step's
// log-decay or null.
template <typename T>
__global__ __launch_bounds__(256) void kata_gen_decode_kernel(KataGenStateArgs a) {
  __shared__ float qs[128], ks[128], vs[kGenDV];
  __shared__ float4 red[16][16];
  __shared__ float dred[16];
  const int tid = threadIdx.x, bh = blockIdx.x;
  if (tid < a.dk) {
    qs[tid] = ldf<T>(a.q, (int64_t)bh * a.dk + tid);
    ks[tid] = ldf<T>(a.k, (int64_t)bh * a.dk + tid);
  }
  if (tid < kGenDV) vs[tid] = ldf<T>(a.v, (int64_t)bh * kGenDV + tid);
  __syncthreads();
  const float f = a.c ? __expf(a.c[bh]) : 1.f;
  const int c4 = tid & 15, r = tid >> 4;
  const float4 vv = *reinterpret_cast<const float4*>(vs + 4 * c4);
  float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
  float dacc = 0.f;
  float* S = a.S + (size_t)bh * a.P * kGenDV;
  float* z = a.z + (size_t)bh * a.P;
  // rows r, r + 16, ...: each thread loads kDecU rows before updating them,
  // so that kDecU loads per thread are in flight
  constexpr int kDecU = 4;
  for (int p0 = r; p0 < a.P; p0 += 16 * kDecU) {
    float4 xs[kDecU];
    float zs[kDecU];
#pragma unroll
    for (int u = 0; u < kDecU; ++u) {
      const int p = p0 + 16 * u;
      xs[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      zs[u] = 0.f;
      if (p < a.P) {
        xs[u] = *reinterpret_cast<const float4*>(S + (size_t)p * kGenDV + 4 * c4);
        if (c4 == 0) zs[u] = z[p];
      }
    }
#pragma unroll
    for (int u = 0; u < kDecU; ++u) {
      const int p = p0 + 16 * u;
      if (p >= a.P) break;
      const RowPair rp = row_pair(a, p);
      const float pk = psi_feat(ks, rp, a.E, a.M, a.sum, a.scale);
      const float pq = rp.w * psi_feat(qs, rp, a.E, a.M, a.sum, a.scale);
      float4 x = xs[u];
      x.x = f * x.x + pk * vv.x; x.y = f * x.y + pk * vv.y;
      x.z = f * x.z + pk * vv.z; x.w = f * x.w + pk * vv.w;
      *reinterpret_cast<float4*>(S + (size_t)p * kGenDV + 4 * c4) = x;
      num.x += pq * x.x; num.y += pq * x.y; num.z += pq * x.z; num.w += pq * x.w;
      if (c4 == 0) {
        const float zz = f * zs[u] + pk;
        z[p] = zz;
        dacc += pq * zz;
      }
    }
  }
  red[r][c4] = num;
  if (c4 == 0) dred[r] = dacc;
  __syncthreads();
  if (tid < 16) {
    float4 s = red[0][tid];
    for (int rr = 1; rr < 16; ++rr) {
      const float4 y = red[rr][tid];
      s.x += y.x; s.y += y.y; s.z += y.z; s.w += y.w;
    }
    float d = 0.f;
    for (int rr = 0; rr < 16; ++rr) d += dred[rr];
    const float inv = 1.f / fmaxf(d, a.eps);
    st4<T>((T*)a.o + (size_t)bh * kGenDV + 4 * tid, to4<T>(s.x * inv, s.y * inv, s.z * inv, s.w * inv));
  }
}

// Continued prefill: per (b, h, 64 queries).  Thread (qi, cj) = (tid / 16,
// tid % 16) owns queries 4 qi .. 4 qi + 3 of the tile and value columns
// 4 cj .. 4 cj + 3.  Per 32 state rows the workgroup forms psi of its 64
// queries into LDS and stages the rows of S and z (zeros past row P, which
// the packed layout need not fill to a multiple of 32), then each thread
// adds 16 products per row.  The result is combined with the flash forward's
// (o, den) of the call's tokens, which o and den hold on entry:
//   num = o den + f_t psi(q_t)^T S,  den' = den + f_t psi(q_t) . z,
//   o = num / max(den', eps),  den = max(den', eps).
template <typename T>
__global__ __launch_bounds__(256) void kata_gen_readout_kernel(KataGenStateArgs a) {
  __shared__ float Qs[64][129];
  __shared__ __attribute__((aligned(16))) float Ps[32][68];
  __shared__ __attribute__((aligned(16))) float4 Sr[32][16];
  __shared__ float Zs[32];
  const int tid = threadIdx.x;
  const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H, t0 = blockIdx.y * 64;
  const int qi = tid >> 4, cj = tid & 15;
  for (int i = tid; i < 64 * a.dk; i += 256) {
    const int t = i / a.dk, d = i % a.dk;
    Qs[t][d] = t0 + t < a.T ? ldf<T>(a.q, (((int64_t)b * a.T + t0 + t) * a.H + h) * a.dk + d) : 0.f;
  }
  float4 acc[4];
  float dacc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    dacc[i] = 0.f;
  }
  const float* S = a.S + (size_t)bh * a.P * kGenDV;
  const float* z = a.z + (size_t)bh * a.P;
  for (int p0 = 0; p0 < a.P; p0 += 32) {
    __syncthreads();  // the previous rows are consumed (and Qs is complete)
    for (int i = tid; i < 32 * 64; i += 256) {
      const int pp = i >> 6, t = i & 63;
      float f = 0.f;
      if (p0 + pp < a.P) {
        const RowPair rp = row_pair(a, p0 + pp);
        f = rp.w * psi_feat(Qs[t], rp, a.E, a.M, a.sum, a.scale);
      }
      Ps[pp][t] = f;
    }
    for (int i = tid; i < 32 * 16; i += 256)
      Sr[i >> 4][i & 15] = p0 + (i >> 4) < a.P
                               ? *reinterpret_cast<const float4*>(S + (size_t)(p0 + (i >> 4)) * kGenDV + 4 * (i & 15))
                               : make_float4(0.f, 0.f, 0.f, 0.f);
    if (tid < 32) Zs[tid] = p0 + tid < a.P ? z[p0 + tid] : 0.f;
    __syncthreads();
#pragma unroll 4
    for (int pp = 0; pp < 32; ++pp) {
      const float4 s = Sr[pp][cj];
      const float4 ps = *reinterpret_cast<const float4*>(&Ps[pp][4 * qi]);
      const float psv[4] = {ps.x, ps.y, ps.z, ps.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[i].x += psv[i] * s.x; acc[i].y += psv[i] * s.y;
        acc[i].z += psv[i] * s.z; acc[i].w += psv[i] * s.w;
        dacc[i] += psv[i] * Zs[pp];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = t0 + 4 * qi + i;
    if (t >= a.T) break;
    const int64_t row = ((int64_t)b * a.T + t) * a.H + h;
    const float fd = a.c ? __expf(a.c[row]) : 1.f;
    const float df = a.den[row];
    const float dd = df + fd * dacc[i];
    const float dsc = fmaxf(dd, a.eps), inv = 1.f / dsc;
    T* orow = (T*)a.o + row * kGenDV + 4 * cj;
    const v4_t<T> of = *reinterpret_cast<const v4_t<T>*>(orow);
    st4<T>(orow, to4<T>(((float)of[0] * df + fd * acc[i].x) * inv, ((float)of[1] * df + fd * acc[i].y) * inv,
                        ((float)of[2] * df + fd * acc[i].z) * inv, ((float)of[3] * df + fd * acc[i].w) * inv));
  }
  // den after every thread of the query has read it: a second pass by the
  // column-0 threads
  __syncthreads();
  if (cj == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = t0 + 4 * qi + i;
      if (t >= a.T) break;
      const int64_t row = ((int64_t)b * a.T + t) * a.H + h;
      const float fd = a.c ? __expf(a.c[row]) : 1.f;
      a.den[row] = fmaxf(a.den[row] + fd * dacc[i], a.eps);
    }
  }
}

// State update: per (b, h, 64 state rows).  Thread (ri, cj) owns rows
// 4 ri .. 4 ri + 3 of the tile and columns 4 cj .. 4 cj + 3; tokens stream
// through LDS 32 at a time with their weights f_Ts = exp(c_T - c_s).  Each
// thread forms the features of one row (p0 + tid % 64); rows past P (the
// packed layout's last tile) get zero features and are not stored.
//   S <- (init ? f_T S : 0) + sum_s f_Ts psi(k_s) v_s^T,  z likewise.
template <typename T>
__global__ __launch_bounds__(256) void kata_gen_update_kernel(KataGenStateArgs a) {
  __shared__ float Ks[32][129];
  __shared__ __attribute__((aligned(16))) float Ps[32][68];
  __shared__ __attribute__((aligned(16))) float4 Vs[32][16];
  __shared__ float Ws[32];
  const int tid = threadIdx.x;
  const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H, p0 = blockIdx.y * 64;
  const int ri = tid >> 4, cj = tid & 15;
  const float cT = a.c ? a.c[((int64_t)b * a.T + a.T - 1) * a.H + h] : 0.f;
  const int prow = p0 + (tid & 63);
  const bool live = prow < a.P;
  const RowPair rp = row_pair(a, live ? prow : 0);
  float4 acc[4];
  float zacc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    zacc[i] = 0.f;
  }
  for (int s0 = 0; s0 < a.T; s0 += 32) {
    __syncthreads();  // the previous tokens are consumed
    for (int i = tid; i < 32 * a.dk; i += 256) {
      const int s = i / a.dk, d = i % a.dk;
      Ks[s][d] = s0 + s < a.T ? ldf<T>(a.k, (((int64_t)b * a.T + s0 + s) * a.H + h) * a.dk + d) : 0.f;
    }
    for (int i = tid; i < 32 * 16; i += 256) {
      const int s = i >> 4, c4 = i & 15;
      float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
      if (s0 + s < a.T) {
        const int64_t base = (((int64_t)b * a.T + s0 + s) * a.H + h) * kGenDV + 4 * c4;
        x = make_float4(ldf<T>(a.v, base), ldf<T>(a.v, base + 1), ldf<T>(a.v, base + 2), ldf<T>(a.v, base + 3));
      }
      Vs[s][c4] = x;
    }
    if (tid < 32) {
      const int s = s0 + tid;
      Ws[tid] = s < a.T ? (a.c ? __expf(cT - a.c[((int64_t)b * a.T + s) * a.H + h]) : 1.f) : 0.f;
    }
    __syncthreads();
    for (int i = tid; i < 32 * 64; i += 256) {
      const int s = i >> 6, pp = i & 63;  // pp = tid % 64: the row of rp
      Ps[s][pp] = live ? Ws[s] * psi_feat(Ks[s], rp, a.E, a.M, a.sum, a.scale) : 0.f;
    }
    __syncthreads();
#pragma unroll 4
    for (int s = 0; s < 32; ++s) {
      const float4 vv = Vs[s][cj];
      const float4 ps = *reinterpret_cast<const float4*>(&Ps[s][4 * ri]);
      const float psv[4] = {ps.x, ps.y, ps.z, ps.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[i].x += psv[i] * vv.x; acc[i].y += psv[i] * vv.y;
        acc[i].z += psv[i] * vv.z; acc[i].w += psv[i] * vv.w;
        zacc[i] += psv[i];
      }
    }
  }
  const float fT = a.c ? __expf(cT) : 1.f;
  float* S = a.S + (size_t)bh * a.P * kGenDV;
  float* z = a.z + (size_t)bh * a.P;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = p0 + 4 * ri + i;
    if (p >= a.P) break;
    float4* sp = reinterpret_cast<float4*>(S + (size_t)p * kGenDV + 4 * cj);
    float4 x = acc[i];
    if (a.init) {
      const float4 o = *sp;
      x.x += fT * o.x; x.y += fT * o.y; x.z += fT * o.z; x.w += fT * o.w;
    }
    *sp = x;
    if (cj == 0) z[p] = (a.init ? fT * z[p] : 0.f) + zacc[i];
  }
}

template <typename T>
hipError_t launch_kata_gen_state(const KataGenStateArgs& a, int which, hipStream_t stream) {
  const int BH = a.B * a.H;
  if (which == KATA_GEN_DECODE)
    kata_gen_decode_kernel<T><<<dim3(BH), dim3(256), 0, stream>>>(a);
  else if (which == KATA_GEN_READOUT)
    kata_gen_readout_kernel<T><<<dim3(BH, (a.T + 63) / 64), dim3(256), 0, stream>>>(a);
  else
    kata_gen_update_kernel<T><<<dim3(BH, (a.P + 63) / 64), dim3(256), 0, stream>>>(a);
  return hipGetLastError();
}

template hipError_t launch_kata_gen_state<__bf16>(const KataGenStateArgs&, int, hipStream_t);
template hipError_t launch_kata_gen_state<_Float16>(const KataGenStateArgs&, int, hipStream_t);
template hipError_t launch_kata_gen_state<float>(const KataGenStateArgs&, int, hipStream_t);

}  // namespace linatt
