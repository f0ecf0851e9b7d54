// KATA-SPD causal attention backward for gfx950.
//
// Replaces parallel_kata_attn_bwd_preprocess, ..._bwd_kernel_dq_M{1,2,4},
// ..._bwd_kernel_dkdv_M{1,2,4} (kata/kernels/parallel_kata.py:348-1342) and
// the sum-score kernels (kata/kernels/parallel_kata_sum.py:7-825), launched
// from parallel_kata_attn_bwd_triton / ..._sum_bwd_triton_M{2,4}
// (kata/parallel_kata_attn.py:364-529, 755-901).  Math as in the reference's
// explicit backward (kata/parallel_kata_attn.py:97-146):
//
//   P = A / D, delta_t = <o_t, dO_t>, dV = P^T dO,
//   dA = (dO V^T - delta) / D (causal), da_g = 2 scale^2 r_g dA  (r_g = q_g.k_g)
//   dQ_g = sum_s da_g k_g,  dK_g = sum_t da_g^T q_g
//
// with D replaced by 1 where it is not positive (the kernels' safe divide).
// GQA (HQ = G*H) is handled natively: dK/dV of a kv head accumulate over its
// G query heads inside one workgroup.
//
// Kernel 1 (dq): a workgroup owns 128 queries (4 waves x 32); key tiles of
// 64 stream through LDS as K (natural), K^T and V (natural).  It also
// computes delta for its rows and writes it for kernel 2.
// Kernel 2 (dk/dv): a workgroup owns 128 keys (4 waves x 32); query tiles
// of 64 stream through LDS as Q, Q^T, dO, dO^T plus delta and 1/D.
#include "common.h"
#include "kata_kernels.h"

namespace linatt {

template <typename T, int DK, int DV, int M, bool SUM, bool DECAY>
__global__ __launch_bounds__(256, sizeof(T) == 2 ? 2 : 1) void kata_bwd_dq_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ o, const float* __restrict__ den, const T* __restrict__ dout,
    T* __restrict__ dq, float* __restrict__ delta_out, const float* __restrict__ c,
    float* __restrict__ dc, int Tn, int HQ, int H, float scale2, int nqt, int nbh) {
  constexpr int E = DK / M;
  constexpr int KE = E / 16;
  constexpr int PAD = (sizeof(T) == 2 ? 8 : 4);
  constexpr int KP = DK + PAD, VP = DV + PAD, TP = 64 + 4;
  __shared__ __attribute__((aligned(16))) T Ks[64 * KP];
  __shared__ __attribute__((aligned(16))) T Kt[DK * TP];
  __shared__ __attribute__((aligned(16))) T Vs[64 * VP];
  __shared__ __attribute__((aligned(16))) float Cs[64];
  __shared__ __attribute__((aligned(16))) T Zr[64];

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  if (tid < 64) Zr[tid] = T(0);
  // K^T row feeding dQ^T row 32 rb + cl of query group gi from key group gk;
  // for E = 16 a 32-row block holds two groups and the lanes of the other
  // group read the zero row instead
  auto kt_row = [&](int gi, int gk, int rb) -> const T* {
    if constexpr (E >= 32) return Kt + (gk * E + (32 * rb + cl - gi * E)) * TP;
    else return ((cl >> 4) == (gi & 1)) ? Kt + (gk * E + (cl & 15)) * TP : Zr;
  };
  int qt, bh;
  map_block(blockIdx.x, nqt, nbh, qt, bh, true);
  const int b = bh / HQ, hq = bh % HQ;
  const int G = HQ / H, h = hq / G;
  const int t0 = qt * 128;
  const int tw = t0 + 32 * w;
  const int tl = tw + cl;
  const bool tvalid = tl < Tn;

  const int64_t qs = (int64_t)HQ * DK, ks = (int64_t)H * DK, vs = (int64_t)H * DV,
                os = (int64_t)HQ * DV;
  const T* kb = k + ((int64_t)b * Tn) * ks + (int64_t)h * DK;
  const T* vb = v + ((int64_t)b * Tn) * vs + (int64_t)h * DV;
  const int64_t qrow = ((int64_t)b * Tn + tl) * HQ + hq;

  v8_t<T> qop[DK / 16], doop[DV / 16];
#pragma unroll
  for (int kk = 0; kk < DK / 16; ++kk)
    qop[kk] = tvalid ? ld8<T>(q + qrow * DK + 16 * kk + 8 * hh) : zero8<T>();
  float dpart = 0.f;
#pragma unroll
  for (int kk = 0; kk < DV / 16; ++kk) {
    doop[kk] = tvalid ? ld8<T>(dout + qrow * DV + 16 * kk + 8 * hh) : zero8<T>();
    const v8_t<T> ov = (tvalid && o) ? ld8<T>(o + qrow * DV + 16 * kk + 8 * hh) : zero8<T>();
#pragma unroll
    for (int j = 0; j < 8; ++j) dpart += (float)ov[j] * (float)doop[kk][j];
  }
  const float delta = dpart + __shfl_xor(dpart, 32);
  float pdl = 0.f;
  if (tvalid) {
    const float d = den[qrow];
    pdl = scale2 / (d > 0.f ? d : 1.f);
    if (hh == 0) {
      delta_out[qrow] = -delta;
      delta_out[(int64_t)nbh * Tn + qrow] = pdl;
    }
  }

  f32x16 acc[DK / 32];
#pragma unroll
  for (int rb = 0; rb < DK / 32; ++rb) acc[rb] = f32x16{};
  // decay: D[t,s] = exp(min(c_t - c_s, 0)) scales dA; dc_t gets
  // sum_s dA A [c_t - c_s <= 0] (the row part; the dk/dv kernel adds the column part)
  const float ct = (DECAY && tvalid) ? c[qrow] : 0.f;
  float dcr = 0.f;

  const int s_end = min(t0 + 128, Tn);
  const int nst = (s_end + 63) / 64;
  for (int st = 0; st < nst; ++st) {
    const int s0 = st * 64;
    __syncthreads();
    load_tile64<T, DK, KP, TP, true, true>(kb, s0, Tn, ks, Ks, Kt, tid);
    load_tile64<T, DV, VP, 1, true, false>(vb, s0, Tn, vs, Vs, nullptr, tid);
    if constexpr (DECAY) {
      if (tid < 64) Cs[tid] = (s0 + tid < Tn) ? c[((int64_t)b * Tn + s0 + tid) * HQ + hq] : 0.f;
    }
    __syncthreads();
    if (s0 > tw + 31 || tw >= Tn) continue;
    const bool need_mask = (s0 + 63 > tw) || (s0 + 64 > Tn);
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      // x^T[s][t] = dP^T - delta = V dO^T - delta  (rows s, column t)
      f32x16 x;
#pragma unroll
      for (int e = 0; e < 16; ++e) x[e] = -delta;
      const T* vrow = Vs + (32 * sb + cl) * VP + 8 * hh;
#pragma unroll
      for (int kk = 0; kk < DV / 16; ++kk) x = mma(ld8<T>(vrow + 16 * kk), doop[kk], x);
      if (need_mask) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int s = s0 + 32 * sb + 8 * i + 4 * hh + r;
            if (s > tl || s >= Tn) x[4 * i + r] = 0.f;
          }
      }
      f32x16 msk;  // [c_t - c_s <= 0] (decay only)
      if constexpr (DECAY) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4 cs4 = *reinterpret_cast<const f32x4*>(Cs + 32 * sb + 8 * i + 4 * hh);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float dd = ct - cs4[r];
            x[4 * i + r] *= __expf(fminf(dd, 0.f));
            msk[4 * i + r] = dd <= 0.f ? 1.f : 0.f;
          }
        }
      }
      f32x16 au{};
      const T* krow = Ks + (32 * sb + cl) * KP + 8 * hh;
#pragma unroll
      for (int gi = 0; gi < M; ++gi) {
#pragma unroll
        for (int gj = 0; gj < (SUM ? M : 1); ++gj) {
          const int gk = SUM ? gj : gi;  // key group paired with query group gi
          f32x16 r{};
#pragma unroll
          for (int kk = 0; kk < KE; ++kk) r = mma(ld8<T>(krow + gk * E + 16 * kk), qop[gi * KE + kk], r);
          if constexpr (DECAY) au += r * r;
          const f32x16 da = r * x;
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const v8_t<T> bop = c_to_b<T>(da, j);
            // dQ^T rows R = 32rb + cl belonging to query group gi take K^T rows of key group gk
#pragma unroll
            for (int rb = (gi * E) / 32; rb <= ((gi + 1) * E - 1) / 32; ++rb)
              acc[rb] = mma(ld_tr_op<T>(kt_row(gi, gk, rb) + 32 * sb, j, hh), bop, acc[rb]);
          }
        }
      }
      if constexpr (DECAY) {
#pragma unroll
        for (int e = 0; e < 16; ++e) dcr += x[e] * au[e] * msk[e];
      }
    }
  }

  if constexpr (DECAY) {
    dcr += __shfl_xor(dcr, 32);
    if (tvalid && hh == 0) dc[qrow] = dcr * pdl;
  }
  if (tvalid) {
    const float f = 2.f * pdl;
    T* drow = dq + qrow * DK;
#pragma unroll
    for (int rb = 0; rb < DK / 32; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st4<T>(drow + 32 * rb + 8 * i + 4 * hh,
               to4<T>(acc[rb][4 * i] * f, acc[rb][4 * i + 1] * f, acc[rb][4 * i + 2] * f,
                      acc[rb][4 * i + 3] * f));
  }
}

template <typename T, int DK, int DV, int M, bool SUM, bool DECAY>
__global__ __launch_bounds__(256, sizeof(T) == 2 ? 2 : 1) void kata_bwd_dkdv_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const float* __restrict__ den, const float* __restrict__ delta, const T* __restrict__ dout,
    T* __restrict__ dk, T* __restrict__ dv, const float* __restrict__ c, float* __restrict__ dc,
    int Tn, int HQ, int H, float scale2, int nst, int nbh) {
  constexpr int E = DK / M;
  constexpr int KE = E / 16;
  constexpr int PAD = (sizeof(T) == 2 ? 8 : 4);
  constexpr int QP = DK + PAD, OP = DV + PAD, TP = 64 + 4;
  constexpr float kPScale = __is_same(T, _Float16) ? 4096.f : 1.f;
  constexpr float kPInv = 1.f / kPScale;
  __shared__ __attribute__((aligned(16))) T Qs[64 * QP];
  __shared__ __attribute__((aligned(16))) T Qt[DK * TP];
  __shared__ __attribute__((aligned(16))) T Os[64 * OP];
  __shared__ __attribute__((aligned(16))) T Ot[DV * TP];
  __shared__ __attribute__((aligned(16))) float Dl[64];
  __shared__ __attribute__((aligned(16))) float Pd[64];
  __shared__ __attribute__((aligned(16))) float Ct[64];
  __shared__ __attribute__((aligned(16))) T Zr[64];

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  if (tid < 64) Zr[tid] = T(0);
  // Q^T row feeding dK^T row 32 rb + cl of key group gk from query group gi;
  // for E = 16 a 32-row block holds two groups and the lanes of the other
  // group read the zero row instead
  auto qt_row = [&](int gi, int gk, int rb) -> const T* {
    if constexpr (E >= 32) return Qt + (gi * E + (32 * rb + cl - gk * E)) * TP;
    else return ((cl >> 4) == (gk & 1)) ? Qt + (gi * E + (cl & 15)) * TP : Zr;
  };
  int stile, bh;
  map_block(blockIdx.x, nst, nbh, stile, bh, false);
  const int b = bh / H, h = bh % H;
  const int G = HQ / H;
  const int s0 = stile * 128;
  const int sw = s0 + 32 * w;
  const int sl = sw + cl;
  const bool svalid = sl < Tn;

  const int64_t qs = (int64_t)HQ * DK, os = (int64_t)HQ * DV;
  const int64_t krow = ((int64_t)b * Tn + sl) * H + h;

  v8_t<T> kop[DK / 16], vop[DV / 16];
#pragma unroll
  for (int kk = 0; kk < DK / 16; ++kk)
    kop[kk] = svalid ? ld8<T>(k + krow * DK + 16 * kk + 8 * hh) : zero8<T>();
#pragma unroll
  for (int kk = 0; kk < DV / 16; ++kk)
    vop[kk] = svalid ? ld8<T>(v + krow * DV + 16 * kk + 8 * hh) : zero8<T>();

  f32x16 dka[DK / 32], dva[DV / 32];
#pragma unroll
  for (int rb = 0; rb < DK / 32; ++rb) dka[rb] = f32x16{};
#pragma unroll
  for (int db = 0; db < DV / 32; ++db) dva[db] = f32x16{};

  const int ntt = (Tn + 63) / 64;
  for (int hq = h * G; hq < (h + 1) * G; ++hq) {
    const T* qb = q + ((int64_t)b * Tn) * qs + (int64_t)hq * DK;
    const T* ob = dout + ((int64_t)b * Tn) * os + (int64_t)hq * DV;
    const float csl = (DECAY && svalid) ? c[((int64_t)b * Tn + sl) * HQ + hq] : 0.f;
    float dcc = 0.f;
    for (int tt = s0 / 64; tt < ntt; ++tt) {
      const int t0 = tt * 64;
      __syncthreads();
      load_tile64<T, DK, QP, TP, true, true>(qb, t0, Tn, qs, Qs, Qt, tid);
      load_tile64<T, DV, OP, TP, true, true>(ob, t0, Tn, os, Os, Ot, tid);
      if (tid < 64) {
        const int t = t0 + tid;
        float dl = 0.f, pd = 0.f;
        if (t < Tn) {
          const int64_t r = ((int64_t)b * Tn + t) * HQ + hq;
          dl = -delta[r];
          const float d = den[r];
          pd = scale2 / (d > 0.f ? d : 1.f);
        }
        Dl[tid] = -dl;
        Pd[tid] = pd;
        if constexpr (DECAY) Ct[tid] = (t < Tn) ? c[((int64_t)b * Tn + t) * HQ + hq] : 0.f;
      }
      __syncthreads();
      if (t0 + 63 < sw || sw >= Tn) continue;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const int tb = t0 + 32 * mb;
        if (tb + 31 < sw) continue;
        const bool need_mask = (tb < sw + 31) || (tb + 32 > Tn);
        auto masked = [&](int e) {
          const int t = tb + 8 * (e >> 2) + 4 * hh + (e & 3);
          return t < sl || t >= Tn;
        };
        // x[t][s] = dO V^T - delta  (rows t, column s); Dl holds -delta
        f32x16 x, pdv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4 d4 = *reinterpret_cast<const f32x4*>(Dl + 32 * mb + 8 * i + 4 * hh);
          const f32x4 p4 = *reinterpret_cast<const f32x4*>(Pd + 32 * mb + 8 * i + 4 * hh);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            x[4 * i + r] = d4[r];
            pdv[4 * i + r] = p4[r];
          }
        }
        const T* orow = Os + (32 * mb + cl) * OP + 8 * hh;
#pragma unroll
        for (int kk = 0; kk < DV / 16; ++kk) x = mma(ld8<T>(orow + 16 * kk), vop[kk], x);
        const T* qrow = Qs + (32 * mb + cl) * QP + 8 * hh;
        // r = Q_gi K_gk^T for query group gi, key group gk (rows t, column s)
        auto score = [&](int gi, int gk) {
          f32x16 r{};
#pragma unroll
          for (int kk = 0; kk < KE; ++kk) r = mma(ld8<T>(qrow + gi * E + 16 * kk), kop[gk * KE + kk], r);
          return r;
        };
        // dK^T[(gk,e)][s] += sum_t Q^T[(gi,e)][t] r[t][s] xs[t][s]
        auto dk_product = [&](const f32x16& r, const f32x16& xs, int gi, int gk) {
          const f32x16 da = r * xs;
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const v8_t<T> bop = c_to_b<T>(da, j);
#pragma unroll
            for (int rb = (gk * E) / 32; rb <= ((gk + 1) * E - 1) / 32; ++rb)
              dka[rb] = mma(ld_tr_op<T>(qt_row(gi, gk, rb) + 32 * mb, j, hh), bop, dka[rb]);
          }
        };
        // decay factors exp(min(c_t - c_s, 0)) and the mask [c_t - c_s <= 0]
        auto decay_of = [&](int e, bool& nonpos) {
          const float dd = Ct[32 * mb + 8 * (e >> 2) + 4 * hh + (e & 3)] - csl;
          nonpos = dd <= 0.f;
          return __expf(fminf(dd, 0.f));
        };
        // one pass per group: the score feeds A and its dK product at once
        f32x16 A{};
        if (need_mask) {
#pragma unroll
          for (int e = 0; e < 16; ++e) x[e] = masked(e) ? 0.f : x[e];
        }
        if constexpr (DECAY) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            bool np;
            x[e] *= decay_of(e, np);
          }
        }
        const f32x16 xs = x * pdv;
#pragma unroll
        for (int gi = 0; gi < M; ++gi)
#pragma unroll
          for (int gj = 0; gj < (SUM ? M : 1); ++gj) {
            const f32x16 r = score(gi, SUM ? gj : gi);
            A += r * r;
            dk_product(r, xs, gi, SUM ? gj : gi);
          }
        if (need_mask) {
#pragma unroll
          for (int e = 0; e < 16; ++e) A[e] = masked(e) ? 0.f : A[e];
        }
        if constexpr (DECAY) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            bool np;
            const float dec = decay_of(e, np);
            // column part of dc_s: -sum_t dA A [c_t - c_s <= 0] (xs carries the decay)
            dcc -= np ? xs[e] * A[e] : 0.f;
            A[e] *= dec;
          }
        }
        // fp16 keeps P in [0, 2^12] so small weights stay out of its subnormal
        // range (bf16 and fp32 have the fp32 exponent range); undone at the store
        const f32x16 P = A * (pdv * kPScale);
        // dV^T[dv][s] += sum_t dO^T[dv][t] P[t][s]
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const v8_t<T> pb = c_to_b<T>(P, j);
#pragma unroll
          for (int db = 0; db < DV / 32; ++db)
            dva[db] = mma(ld_tr_op<T>(Ot + (32 * db + cl) * TP + 32 * mb, j, hh), pb, dva[db]);
        }
      }
    }
    if constexpr (DECAY) {
      dcc += __shfl_xor(dcc, 32);
      if (svalid && hh == 0) dc[((int64_t)b * Tn + sl) * HQ + hq] += dcc;
    }
  }

  if (svalid) {
    T* dkrow = dk + krow * DK;
    T* dvrow = dv + krow * DV;
#pragma unroll
    for (int rb = 0; rb < DK / 32; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st4<T>(dkrow + 32 * rb + 8 * i + 4 * hh,
               to4<T>(2.f * dka[rb][4 * i], 2.f * dka[rb][4 * i + 1], 2.f * dka[rb][4 * i + 2],
                      2.f * dka[rb][4 * i + 3]));
#pragma unroll
    for (int db = 0; db < DV / 32; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st4<T>(dvrow + 32 * db + 8 * i + 4 * hh,
               to4<T>(dva[db][4 * i] * kPInv, dva[db][4 * i + 1] * kPInv,
                      dva[db][4 * i + 2] * kPInv, dva[db][4 * i + 3] * kPInv));
  }
}

// ---------------------------------------------------------------------------
// 16-bit inputs: the two kernels above with their tiles brought in by direct
// global->LDS copies into double buffers (the next tile's copies in flight
// while the current one computes, one barrier per tile), stored swizzled in
// natural layout only.  Operands with k along the tile rows (K^T for dQ,
// Q^T for dK, dO^T for dV) come from transposing LDS reads.  Rows past T
// repeat the last valid row; every use of them is masked.
// ---------------------------------------------------------------------------
// ONORM: dy replaces dO, and the output RMSNorm's backward runs in the
// prologue (compile-time, so the plain kernel carries none of it)
template <typename T, int DK, int DV, int M, bool SUM, bool DECAY, bool ONORM>
__global__ __launch_bounds__(256, 2) void kata_bwd_dq_tile_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ o, const float* __restrict__ den, const T* __restrict__ dout,
    T* __restrict__ dq, float* __restrict__ delta_out, const float* __restrict__ c,
    float* __restrict__ dc, int Tn, int HQ, int H, float scale2, int nqt, int nbh, OutNorm on) {
  constexpr int E = DK / M;
  constexpr int KE = E / 16;
  static_assert(sizeof(T) == 2 && (DK == 64 || (DK == 128 && E >= 32)) && DV == 64,
                "64 x 64 16-bit tiles");
  constexpr int KT = DK / 64;  // key tiles as KT 64 x 64 sub-tiles (wtile_ld8)
  constexpr int NB = 3;  // ring depth: tiles st + 1 and st + 2 in flight during tile st
  __shared__ __attribute__((aligned(16))) T Kb[NB][KT * 64 * 64];
  __shared__ __attribute__((aligned(16))) T Vb[NB][64 * 64];
  __shared__ __attribute__((aligned(16))) float Cs[NB][64];
  __shared__ __attribute__((aligned(16))) float Wred[4][DV];  // output-norm weight gradient per wave

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  int qt, bh;
  map_block(blockIdx.x, nqt, nbh, qt, bh, true);
  const int b = bh / HQ, hq = bh % HQ;
  const int G = HQ / H, h = hq / G;
  const int t0 = qt * 128;
  const int tw = t0 + 32 * w;
  const int tl = tw + cl;
  const bool tvalid = tl < Tn;

  const int64_t ks = (int64_t)H * DK, vs = (int64_t)H * DV;
  const T* kb = k + ((int64_t)b * Tn) * ks + (int64_t)h * DK;
  const T* vb = v + ((int64_t)b * Tn) * vs + (int64_t)h * DV;
  const int64_t qrow = ((int64_t)b * Tn + tl) * HQ + hq;

  v8_t<T> qop[DK / 16], doop[DV / 16];
#pragma unroll
  for (int kk = 0; kk < DK / 16; ++kk)
    qop[kk] = tvalid ? ld8<T>(q + qrow * DK + 16 * kk + 8 * hh) : zero8<T>();
  // bf16: the dk/dv kernel takes dO scaled by scale^2/den (the row scale of P
  // and of dA), which saves it two products per score, and the matching
  // delta' = <o, dO'> from the same rounded dO', so x' = dO' v - delta' keeps
  // the cancellation of x = dO v - delta (zero for a lone key)
  constexpr bool kPre = __is_same(T, __bf16);
  float pdl = 0.f;
  if (tvalid) {
    const float d = den[qrow];
    pdl = scale2 / (d > 0.f ? d : 1.f);
  }
  float dpart = 0.f, dppart = 0.f;
  // this lane's dims 16 kk + 8 hh + 0..7 of dO (or of dy) and of o
  v8_t<T> ov[DV / 16];
  const T* dsrc = ONORM ? (const T*)on.y : dout;
#pragma unroll
  for (int kk = 0; kk < DV / 16; ++kk) {
    doop[kk] = tvalid ? ld8<T>(dsrc + qrow * DV + 16 * kk + 8 * hh) : zero8<T>();
    ov[kk] = (tvalid && o) ? ld8<T>(o + qrow * DV + 16 * kk + 8 * hh) : zero8<T>();
  }
  if constexpr (ONORM) {
    // output RMSNorm backward, y = o r w with r = rstd:
    // dO = r w dy - (r^3 / DV) <o, w dy> o, rounded to T as the unfused
    // norm's dx is; the weight gradient sum_rows dy o r goes to this
    // workgroup's partial (summed over the wave's 32 rows by DPP, eight dims
    // at a time to bound the live registers, then over the four waves at
    // the end of the kernel)
    const float rr = tvalid ? on.rstd[qrow] : 0.f;
    float wv[DV / 16][8];
    float sdot = 0.f;
#pragma unroll
    for (int kk = 0; kk < DV / 16; ++kk) {
      const int d0 = 16 * kk + 8 * hh;
      const f32x4 w0 = on.w ? *reinterpret_cast<const f32x4*>(on.w + d0) : f32x4{1.f, 1.f, 1.f, 1.f};
      const f32x4 w1 = on.w ? *reinterpret_cast<const f32x4*>(on.w + d0 + 4) : f32x4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        wv[kk][j] = w0[j];
        wv[kk][4 + j] = w1[j];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) sdot += wv[kk][j] * (float)doop[kk][j] * (float)ov[kk][j];
    }
    sdot += __shfl_xor(sdot, 32);
    const float cf = rr * rr * rr * sdot / DV;
#pragma unroll
    for (int kk = 0; kk < DV / 16; ++kk)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float g = (float)doop[kk][j], x = (float)ov[kk][j];
        const float wp = group_sum<32>(g * x * rr);
        if (cl == 0) Wred[w][16 * kk + 8 * hh + j] = wp;
        doop[kk][j] = (T)(rr * (wv[kk][j] * g) - cf * x);
        if (j == 7) __builtin_amdgcn_sched_barrier(0);
      }
  }
#pragma unroll
  for (int kk = 0; kk < DV / 16; ++kk) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      dpart += (float)ov[kk][j] * (float)doop[kk][j];
      if constexpr (kPre) dppart += (float)ov[kk][j] * (float)(T)((float)doop[kk][j] * pdl);
    }
  }
  const float delta = dpart + __shfl_xor(dpart, 32);
  const float deltap = dppart + __shfl_xor(dppart, 32);
  // the per-row terms for the dk/dv kernel, stored once q and dO have landed
  // (right after the drain below, so no wait covers these stores; the key
  // loop's copy waits stay exact because loads complete in order among
  // themselves)
  auto write_rows = [&]() __attribute__((always_inline)) {
    if constexpr (kPre) {
      // recomputed here, not kept from the delta' sum above: an opaque copy of
      // the scale stops the compiler from carrying dO' through the loop
      float ps = pdl;
      asm volatile("" : "+v"(ps));
      T* dop = reinterpret_cast<T*>(reinterpret_cast<char*>(delta_out) + kata_dop_offset((int64_t)nbh * Tn)) +
               qrow * DV;
#pragma unroll
      for (int kk = 0; kk < DV / 16; ++kk) {
        v8_t<T> y;
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = (T)((float)doop[kk][j] * ps);
        if (tvalid) *reinterpret_cast<v8_t<T>*>(dop + 16 * kk + 8 * hh) = y;
      }
    }
    if (tvalid && hh == 0) {
      delta_out[qrow] = kPre ? -deltap : -delta;
      delta_out[(int64_t)nbh * Tn + qrow] = pdl;
    }
  };

  // 16-wide groups (E = 16): dQ_g^T (16 x 32 queries) by two 16x16x32
  // products per group and key block, whose B operands come from da by one
  // lane swap per register pair (c_to_b16x2); wider groups fill whole 32-row
  // blocks of 32x32x16 products
  constexpr bool k16 = E == 16;
  f32x16 acc[k16 ? 1 : DK / 32];
  f32x4 acc16[k16 ? M : 1][2];
  if constexpr (k16) {
#pragma unroll
    for (int g = 0; g < M; ++g) acc16[g][0] = acc16[g][1] = f32x4{};
  } else {
#pragma unroll
    for (int rb = 0; rb < DK / 32; ++rb) acc[rb] = f32x16{};
  }
  const float ct = (DECAY && tvalid) ? c[qrow] : 0.f;
  float dcr = 0.f;

  // K^T operand feeding dQ^T rows 32 rb + cl of query group gi from key group
  // gk (E >= 32: whole 32-row blocks of the group)
  auto kt_op = [&](const T* Ks, int sb, int gi, int gk, int rb, int j) __attribute__((always_inline)) {
    return wtile_tr8<T>(Ks, 32 * sb, gk * E + 32 * rb - gi * E, j, lane);
  };

  const int s_end = min(t0 + 128, Tn);
  const int nst = (s_end + 63) / 64;
  // tile st: copies 2w and 2w + 1 of K and of V by wave w (full tiles from a
  // scalar base plus these per-lane offsets; the last tile clamps its rows)
  unsigned ko[2], vo[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    ko[i] = tile_lane_off(2 * w + i, lane, (int)(ks * sizeof(T)));
    vo[i] = tile_lane_off(2 * w + i, lane, (int)(vs * sizeof(T)));
  }
  auto issue = [&](int st) __attribute__((always_inline)) {
    char* kd = reinterpret_cast<char*>(Kb[st % NB]);
    char* vd = reinterpret_cast<char*>(Vb[st % NB]);
    if (64 * st + 64 <= Tn) {
      const T* kt = kb + (int64_t)64 * st * ks;
      const T* vt = vb + (int64_t)64 * st * vs;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int jt = 0; jt < KT; ++jt) dma16s(kt + 64 * jt, ko[i], kd + 8192 * jt + 1024 * (2 * w + i));
        dma16s(vt, vo[i], vd + 1024 * (2 * w + i));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int jt = 0; jt < KT; ++jt)
          dma_tile64<T>(kb + 64 * jt, ks, 64 * st, Tn, reinterpret_cast<T*>(kd) + 4096 * jt, 2 * w + i, lane);
        dma_tile64<T>(vb, vs, 64 * st, Tn, reinterpret_cast<T*>(vd), 2 * w + i, lane);
      }
    }
  };
  auto load_c = [&](int st) __attribute__((always_inline)) {
    if constexpr (DECAY) {
      if (w == 0) dma4(c + ((int64_t)b * Tn + min(64 * st + lane, Tn - 1)) * HQ + hq, Cs[st % NB]);
    }
  };
  const int ops = 2 * KT + 2 + (DECAY && w == 0 ? 1 : 0);  // copies per tile and wave
  vm_drain();  // q, dO (and c) of this wave's queries are in registers
  write_rows();
#pragma unroll
  for (int st = 0; st < NB - 1; ++st)
    if (st < nst) {
      issue(st);
      load_c(st);
    }
  // key tile st; MASKED applies the causal / past-T masks where the tile
  // reaches the workgroup's diagonal
  auto tile = [&](int st, auto masked_c, auto slot_c) __attribute__((always_inline)) {
    constexpr bool kMaskTile = decltype(masked_c)::value;
    const int buf = slot_c;
    const int s0 = st * 64;
    // tile st landed; tile st - 1's slot is free for tile st + 2
    vm_wait_barrier_n(st + 1 < nst ? ops : 0);
    if (st + NB - 1 < nst) {
      issue(st + NB - 1);
      load_c(st + NB - 1);
    }
    const T* Ks = Kb[buf];
    const T* Vs = Vb[buf];
    if (!(s0 > tw + 31 || tw >= Tn)) {
      const bool need_mask = kMaskTile && ((s0 + 63 > tw) || (s0 + 64 > Tn));
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        // a block of keys all after this wave's queries adds nothing
        if (kMaskTile && s0 + 32 * sb > tw + 31) continue;
        // x^T[s][t] = V dO^T - delta  (rows s, column t)
        f32x16 x;
#pragma unroll
        for (int e = 0; e < 16; ++e) x[e] = -delta;
#pragma unroll
        for (int kk = 0; kk < DV / 16; ++kk)
          x = mma(tile_ld8<T>(Vs, 32 * sb + cl, 16 * kk + 8 * hh), doop[kk], x);
        if (need_mask) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int s = s0 + 32 * sb + 8 * (e >> 2) + 4 * hh + (e & 3);
            if (s > tl || s >= Tn) x[e] = 0.f;
          }
        }
        if constexpr (DECAY) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const f32x4 cs4 = *reinterpret_cast<const f32x4*>(&Cs[buf][32 * sb + 8 * i + 4 * hh]);
#pragma unroll
            for (int r = 0; r < 4; ++r) x[4 * i + r] *= __expf(fminf(ct - cs4[r], 0.f));
          }
        }
        f32x16 au{};
#pragma unroll
        for (int gi = 0; gi < M; ++gi) {
#pragma unroll
          for (int gj = 0; gj < (SUM ? M : 1); ++gj) {
            const int gk = SUM ? gj : gi;
            f32x16 r{};
#pragma unroll
            for (int kk = 0; kk < KE; ++kk)
              r = mma(wtile_ld8<T>(Ks, 32 * sb + cl, gk * E + 16 * kk + 8 * hh), qop[gi * KE + kk], r);
            if constexpr (DECAY) au += r * r;
            const f32x16 da = r * x;
            if constexpr (k16) {
              v8_t<T> b0, b1;
              c_to_b16x2<T>(da, b0, b1);
              const v8_t<T> ka = tile_tr8_16<T>(Ks, 32 * sb, 16 * gk, lane);
              acc16[gi][0] = mma16(ka, b0, acc16[gi][0]);
              acc16[gi][1] = mma16(ka, b1, acc16[gi][1]);
            } else {
#pragma unroll
              for (int j = 0; j < 2; ++j) {
                const v8_t<T> bop = c_to_b<T>(da, j);
#pragma unroll
                for (int rb = (gi * E) / 32; rb <= ((gi + 1) * E - 1) / 32; ++rb)
                  acc[rb] = mma(kt_op(Ks, sb, gi, gk, rb, j), bop, acc[rb]);
              }
            }
          }
        }
        if constexpr (DECAY) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            // [c_t - c_s <= 0], from c in LDS again rather than kept
            // through the group loop (16 registers fewer)
            const f32x4 cs4 = *reinterpret_cast<const f32x4*>(&Cs[buf][32 * sb + 8 * i + 4 * hh]);
#pragma unroll
            for (int r = 0; r < 4; ++r)
              dcr += ct - cs4[r] <= 0.f ? x[4 * i + r] * au[4 * i + r] : 0.f;
          }
        }
      }
    }
  };
  // one body for every tile: a second, unmasked copy of it for the tiles
  // before the diagonal raises this kernel's register count past occupancy 3
  // unrolled by the ring depth where registers allow (M > 1): the slot is then
  // a constant in each body, its LDS base folds into the ds_read offsets, and
  // the unmasked block issues 116 VALU instructions instead of 128; with one
  // group the unrolled loop needs 170 VGPRs, past occupancy 3
  static_assert(NB == 3, "ring of three");
  if constexpr (M > 1) {
    for (int st = 0; st < nst; st += 3) {
      tile(st, BoolC<true>{}, IntC<0>{});
      if (st + 1 < nst) tile(st + 1, BoolC<true>{}, IntC<1>{});
      if (st + 2 < nst) tile(st + 2, BoolC<true>{}, IntC<2>{});
    }
  } else {
    for (int st = 0; st < nst; ++st) tile(st, BoolC<true>{}, st % NB);
  }

  if constexpr (DECAY) {
    dcr += __shfl_xor(dcr, 32);
    if (tvalid && hh == 0) dc[qrow] = dcr * pdl;
  }
  if constexpr (k16) {
    // lane (rho, i) holds dQ_g[t][4 rho + 0..3] for t = tw + 16 th + i; the
    // row scale of query t lives in lane t - tw
    const int rho = lane >> 4, i16 = lane & 15;
#pragma unroll
    for (int th = 0; th < 2; ++th) {
      const float f = 2.f * __shfl(pdl, 16 * th + i16);
      const int t = tw + 16 * th + i16;
      if (t < Tn) {
        T* drow = dq + (((int64_t)b * Tn + t) * HQ + hq) * DK;
#pragma unroll
        for (int g = 0; g < M; ++g)
          st4<T>(drow + 16 * g + 4 * rho, to4<T>(acc16[g][th][0] * f, acc16[g][th][1] * f,
                                                   acc16[g][th][2] * f, acc16[g][th][3] * f));
      }
    }
  } else if (tvalid) {
    const float f = 2.f * pdl;
    T* drow = dq + qrow * DK;
#pragma unroll
    for (int rb = 0; rb < DK / 32; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st4<T>(drow + 32 * rb + 8 * i + 4 * hh,
               to4<T>(acc[rb][4 * i] * f, acc[rb][4 * i + 1] * f, acc[rb][4 * i + 2] * f,
                      acc[rb][4 * i + 3] * f));
  }
  // output-norm weight gradient: this workgroup's partial, the four waves'
  // row sums added in a fixed order (every wave reaches this barrier)
  if (ONORM && on.part) {
    __syncthreads();
    if (tid < DV)
      on.part[((int64_t)bh * nqt + qt) * DV + tid] = (Wred[0][tid] + Wred[1][tid]) + (Wred[2][tid] + Wred[3][tid]);
  }
}

// waves (of 32 keys each) per workgroup of the tile dk/dv kernel: eight at
// dk = 128, where the k and v operands of four waves and a two-slot query
// ring would take 97 KiB of LDS (one workgroup, four waves, per CU); eight
// waves share one ring in 145 KiB, two waves per SIMD
template <int DK>
constexpr int kata_dkdv_waves() { return DK == 64 ? 4 : 8; }

template <typename T, int DK, int DV, int M, bool SUM, bool DECAY>
__global__ __launch_bounds__(64 * kata_dkdv_waves<DK>(), 2) void kata_bwd_dkdv_tile_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const float* __restrict__ den, const float* __restrict__ delta, const T* __restrict__ dout,
    T* __restrict__ dk, T* __restrict__ dv, const float* __restrict__ c, float* __restrict__ dc,
    int Tn, int HQ, int H, float scale2, int nst, int nbh) {
  constexpr int E = DK / M;
  constexpr int KE = E / 16;
  constexpr float kPScale = __is_same(T, _Float16) ? 4096.f : 1.f;
  constexpr float kPInv = 1.f / kPScale;
  static_assert(sizeof(T) == 2 && (DK == 64 || (DK == 128 && E >= 32)) && DV == 64,
                "64 x 64 16-bit tiles");
  constexpr int KT = DK / 64;  // query tiles as KT 64 x 64 sub-tiles (wtile_ld8)
  constexpr int NW = kata_dkdv_waves<DK>();
  constexpr int CPW = 8 / NW;  // 1 KiB copies per wave and 64 x 64 sub-tile
  // ring depth 2: tile n + 1 in flight during tile n (a third slot costs
  // registers in this kernel and spills)
  constexpr int NB = 2;
  __shared__ __attribute__((aligned(16))) T Qb[NB][KT * 64 * 64];
  __shared__ __attribute__((aligned(16))) T Ob[NB][64 * 64];
  __shared__ __attribute__((aligned(16))) float Dl[NB][64];  // -delta
  __shared__ __attribute__((aligned(16))) float Pd[NB][64];  // scale^2 / den
  __shared__ __attribute__((aligned(16))) float Ct[NB][64];
  // this wave's k and v rows as MFMA B operands (lane l: 16 bytes per k-step)
  __shared__ __attribute__((aligned(16))) u32x4 KVop[NW][(DK + DV) / 16][64];

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  int stile, bh;
  map_block(blockIdx.x, nst, nbh, stile, bh, false);
  const int b = bh / H, h = bh % H;
  const int G = HQ / H;
  const int s0 = stile * 32 * NW;
  const int sw = s0 + 32 * w;
  const int sl = sw + cl;
  const bool svalid = sl < Tn;

  const int64_t qs = (int64_t)HQ * DK, os = (int64_t)HQ * DV;
  const int64_t krow = ((int64_t)b * Tn + sl) * H + h;

#pragma unroll
  for (int kk = 0; kk < DK / 16; ++kk)
    KVop[w][kk][lane] = __builtin_bit_cast(u32x4, svalid ? ld8<T>(k + krow * DK + 16 * kk + 8 * hh) : zero8<T>());
#pragma unroll
  for (int kk = 0; kk < DV / 16; ++kk)
    KVop[w][DK / 16 + kk][lane] = __builtin_bit_cast(u32x4, svalid ? ld8<T>(v + krow * DV + 16 * kk + 8 * hh) : zero8<T>());
  auto kop = [&](int kk) __attribute__((always_inline)) { return __builtin_bit_cast(v8_t<T>, KVop[w][kk][lane]); };
  auto vop = [&](int kk) __attribute__((always_inline)) { return __builtin_bit_cast(v8_t<T>, KVop[w][DK / 16 + kk][lane]); };

  // 16-wide groups (E = 16): dK_g^T (16 x 32 keys) by two 16x16x32 products
  // per group and query block, B operands from da by one lane swap per
  // register pair (c_to_b16x2); wider groups fill whole 32-row blocks
  constexpr bool k16 = E == 16;
  f32x16 dka[k16 ? 1 : DK / 32], dva[DV / 32];
  f32x4 dk16[k16 ? M : 1][2];
  if constexpr (k16) {
#pragma unroll
    for (int g = 0; g < M; ++g) dk16[g][0] = dk16[g][1] = f32x4{};
  } else {
#pragma unroll
    for (int rb = 0; rb < DK / 32; ++rb) dka[rb] = f32x16{};
  }
#pragma unroll
  for (int db = 0; db < DV / 32; ++db) dva[db] = f32x16{};

  // Q^T operand feeding dK^T rows 32 rb + cl of key group gk from query group
  // gi (E >= 32: whole 32-row blocks of the group)
  auto qt_op = [&](const T* Qs, int mb, int gi, int gk, int rb, int j) __attribute__((always_inline)) {
    return wtile_tr8<T>(Qs, 32 * mb, gi * E + 32 * rb - gk * E, j, lane);
  };

  // query tiles (hq, tt) of this key tile, flattened over the G query heads
  const int ntt = (Tn + 63) / 64, tt0 = s0 / 64, nq = ntt - tt0;
  const int ntiles = G * nq;
  // tile n: copies CPW w .. CPW w + CPW - 1 of each sub-tile of q and of dO by
  // wave w (full tiles from a scalar base plus these per-lane offsets; a
  // head's last tile clamps rows)
  unsigned qo[CPW], oo[CPW];
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    qo[i] = tile_lane_off(CPW * w + i, lane, (int)(qs * sizeof(T)));
    oo[i] = tile_lane_off(CPW * w + i, lane, (int)(os * sizeof(T)));
  }
  // bf16: dO and delta come prescaled by scale^2/den from the dq kernel
  constexpr bool kPre = __is_same(T, __bf16);
  const int64_t nrows = (int64_t)(nbh / H) * Tn * HQ;
  const T* dsrc = kPre ? reinterpret_cast<const T*>(reinterpret_cast<const char*>(delta) + kata_dop_offset(nrows))
                       : dout;
  auto issue = [&](int n, int slot) __attribute__((always_inline)) {
    const int hq = h * G + n / nq, t0 = 64 * (tt0 + n % nq);
    const T* qb = q + ((int64_t)b * Tn) * qs + (int64_t)hq * DK;
    const T* ob = dsrc + ((int64_t)b * Tn) * os + (int64_t)hq * DV;
    char* qd = reinterpret_cast<char*>(Qb[slot]);
    char* od = reinterpret_cast<char*>(Ob[slot]);
    if (t0 + 64 <= Tn) {
      const T* qt = qb + (int64_t)t0 * qs;
      const T* ot = ob + (int64_t)t0 * os;
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
#pragma unroll
        for (int jt = 0; jt < KT; ++jt) dma16s(qt + 64 * jt, qo[i], qd + 8192 * jt + 1024 * (CPW * w + i));
        dma16s(ot, oo[i], od + 1024 * (CPW * w + i));
      }
    } else {
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
#pragma unroll
        for (int jt = 0; jt < KT; ++jt)
          dma_tile64<T>(qb + 64 * jt, qs, t0, Tn, reinterpret_cast<T*>(qd) + 4096 * jt, CPW * w + i, lane);
        dma_tile64<T>(ob, os, t0, Tn, reinterpret_cast<T*>(od), CPW * w + i, lane);
      }
    }
  };
  // per-row data of a query tile: -delta (bf16: prescaled) and scale^2/den
  // as the dq kernel wrote them (rows [0, B T HQ) and [B T HQ, 2 B T HQ) of
  // `delta`), and c; rows past T repeat the last one and are masked
  auto load_rows = [&](int n, int slot) __attribute__((always_inline)) {
    const int hq = h * G + n / nq, t = min(64 * (tt0 + n % nq) + lane, Tn - 1);
    const int64_t r = ((int64_t)b * Tn + t) * HQ + hq;
    if (w == 0) dma4(delta + r, Dl[slot]);
    if (w == 1) dma4(delta + nrows + r, Pd[slot]);
    if (DECAY && w == 2) dma4(c + r, Ct[slot]);
  };

  float csl = (DECAY && svalid) ? c[((int64_t)b * Tn + sl) * HQ + h * G] : 0.f;
  vm_drain();  // k, v (and c) of this wave's keys are in registers
  issue(0, 0);
  load_rows(0, 0);
  float dcc = 0.f;
  // query tile n (global index over the G heads) with or without the causal /
  // past-T masks: only the NW / 2 tiles on this workgroup's diagonal and a
  // ragged last tile take MASKED, so the other tiles' block bodies are each
  // one basic block
  auto tile = [&](int n, auto masked_c) __attribute__((always_inline)) {
    constexpr bool kMaskTile = decltype(masked_c)::value;
    const int buf = n % NB;
    const int hq = h * G + n / nq, t0 = 64 * (tt0 + n % nq);
    // tile n landed and every wave is done with the other slot
    vm_wait_barrier_n(0);
    if (n + 1 < ntiles) {
      issue(n + 1, 1 - buf);
      load_rows(n + 1, 1 - buf);
    }
    const T* Qs = Qb[buf];
    const T* Os = Ob[buf];
    // one 32-query block against this wave's 32 keys; NEED_MASK only for the
    // block on the diagonal (tb == sw) and one that crosses T
    auto block = [&](int mb, bool need_mask) __attribute__((always_inline)) {
        const int tb = t0 + 32 * mb;
        auto masked = [&](int e) {
          const int t = tb + 8 * (e >> 2) + 4 * hh + (e & 3);
          return t < sl || t >= Tn;
        };
        f32x16 x, pdv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4 d4 = *reinterpret_cast<const f32x4*>(&Dl[buf][32 * mb + 8 * i + 4 * hh]);
          const f32x4 p4 = kPre ? f32x4{} : *reinterpret_cast<const f32x4*>(&Pd[buf][32 * mb + 8 * i + 4 * hh]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            x[4 * i + r] = d4[r];
            pdv[4 * i + r] = p4[r];
          }
        }
        // fp16: the causal / past-T mask rides on the row scale scale^2/den,
        // which multiplies both x (into xs) and A (into P): zero where masked.
        // Its branch closes before the products, which stay one basic block.
        if (!kPre && need_mask) {
#pragma unroll
          for (int e = 0; e < 16; ++e) pdv[e] = masked(e) ? 0.f : pdv[e];
        }
        // x[t][s] = dO V^T - delta  (rows t, column s; bf16: both prescaled)
#pragma unroll
        for (int kk = 0; kk < DV / 16; ++kk)
          x = mma(tile_ld8<T>(Os + 2048 * mb, cl, 16 * kk + 8 * hh), vop(kk), x);
        // decayed score: the factors exp(min(c_t - c_s, 0)) once per block,
        // for x here and for A after the group loop
        f32x16 dec;
        if constexpr (DECAY) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            dec[e] = __expf(fminf(Ct[buf][32 * mb + 8 * (e >> 2) + 4 * hh + (e & 3)] - csl, 0.f));
            x[e] *= dec[e];
          }
        }
        f32x16 xs;
        if constexpr (kPre) {
          xs = x;
          if (need_mask) {
#pragma unroll
            for (int e = 0; e < 16; ++e) xs[e] = masked(e) ? 0.f : xs[e];
          }
        } else {
          xs = x * pdv;
        }
        // per (query group gi, key group gk): r = Q_gi K_gk^T, A += r^2 and
        // dK^T[(gk,e)][s] += sum_t Q^T[(gi,e)][t] r[t][s] xs[t][s]
        f32x16 A{};
#pragma unroll
        for (int gi = 0; gi < M; ++gi)
#pragma unroll
          for (int gj = 0; gj < (SUM ? M : 1); ++gj) {
            const int gk = SUM ? gj : gi;
            f32x16 r{};
#pragma unroll
            for (int kk = 0; kk < KE; ++kk)
              r = mma(wtile_ld8<T>(Qs + 2048 * mb, cl, gi * E + 16 * kk + 8 * hh), kop(gk * KE + kk), r);
            A += r * r;
            const f32x16 da = r * xs;
            if constexpr (k16) {
              v8_t<T> b0, b1;
              c_to_b16x2<T>(da, b0, b1);
              const v8_t<T> qa = tile_tr8_16<T>(Qs, 32 * mb, 16 * gi, lane);
              dk16[gk][0] = mma16(qa, b0, dk16[gk][0]);
              dk16[gk][1] = mma16(qa, b1, dk16[gk][1]);
            } else {
#pragma unroll
              for (int j = 0; j < 2; ++j) {
                const v8_t<T> bop = c_to_b<T>(da, j);
#pragma unroll
                for (int rb = (gk * E) / 32; rb <= ((gk + 1) * E - 1) / 32; ++rb)
                  dka[rb] = mma(qt_op(Qs, mb, gi, gk, rb, j), bop, dka[rb]);
              }
            }
            // sum and decay variants: keep the next group's score MFMAs from
            // being hoisted above this group's products (bounds the live
            // score registers; unbounded, they spill)
            if constexpr (SUM || DECAY) __builtin_amdgcn_sched_barrier(0);
          }
        if constexpr (DECAY) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const float dd = Ct[buf][32 * mb + 8 * (e >> 2) + 4 * hh + (e & 3)] - csl;
            // column part of dc_s: -sum_t dA A [c_t - c_s <= 0] (xs carries the decay)
            dcc -= dd <= 0.f ? xs[e] * A[e] : 0.f;
            A[e] *= dec[e];
          }
        }
        // bf16: P = A against the prescaled dO; fp16 keeps P in [0, 2^12]
        // (subnormal range), undone at the store
        f32x16 P;
        if constexpr (kPre) {
          P = A;
          if (need_mask) {
#pragma unroll
            for (int e = 0; e < 16; ++e) P[e] = masked(e) ? 0.f : P[e];
          }
        } else {
          P = A * (pdv * kPScale);
        }
        // dV^T[dv][s] += sum_t dO^T[dv][t] P[t][s], dO^T read transposed from dO
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const v8_t<T> pb = c_to_b<T>(P, j);
#pragma unroll
          for (int db = 0; db < DV / 32; ++db)
            dva[db] = mma(tile_tr8<T>(Os, 32 * mb, 32 * db, j, lane), pb, dva[db]);
        }
    };
    if (!(t0 + 63 < sw || sw >= Tn)) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        // blocks whose queries all precede this wave's keys are skipped (the
        // diagonal tiles only); the block on the diagonal, and one crossing
        // T, is masked; every other block runs unmasked
        const int tb = t0 + 32 * mb;
        if constexpr (kMaskTile) {
          if (tb + 31 < sw) continue;
          block(mb, tb < sw + 31 || tb + 32 > Tn);
        } else {
          block(mb, false);
        }
      }
    }
    if constexpr (DECAY) {
      if (n % nq == nq - 1) {  // last query tile of head hq
        dcc += __shfl_xor(dcc, 32);
        if (svalid && hh == 0) dc[((int64_t)b * Tn + sl) * HQ + hq] += dcc;
        dcc = 0.f;
        if (hq + 1 < (h + 1) * G) csl = svalid ? c[((int64_t)b * Tn + sl) * HQ + hq + 1] : 0.f;
      }
    }
  };
  // per query head: the diagonal tiles, the tiles wholly inside T, the ragged rest
  const int nfull = Tn / 64 - tt0;
  for (int hi = 0; hi < G; ++hi) {
    const int nb = hi * nq;
    int i = 0;
    for (; i < nq && i < NW / 2; ++i) tile(nb + i, BoolC<true>{});
    for (; i < nfull; ++i) tile(nb + i, BoolC<false>{});
    for (; i < nq; ++i) tile(nb + i, BoolC<true>{});
  }

  if constexpr (k16) {
    // lane (rho, i) holds dK_g[s][4 rho + 0..3] for s = sw + 16 sh + i
    const int rho = lane >> 4, i16 = lane & 15;
#pragma unroll
    for (int sh = 0; sh < 2; ++sh) {
      const int s = sw + 16 * sh + i16;
      if (s < Tn) {
        T* dkrow = dk + (((int64_t)b * Tn + s) * H + h) * DK;
#pragma unroll
        for (int g = 0; g < M; ++g)
          st4<T>(dkrow + 16 * g + 4 * rho, to4<T>(2.f * dk16[g][sh][0], 2.f * dk16[g][sh][1],
                                                    2.f * dk16[g][sh][2], 2.f * dk16[g][sh][3]));
      }
    }
  }
  if (svalid) {
    T* dkrow = dk + krow * DK;
    T* dvrow = dv + krow * DV;
    if constexpr (!k16) {
#pragma unroll
      for (int rb = 0; rb < DK / 32; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          st4<T>(dkrow + 32 * rb + 8 * i + 4 * hh,
                 to4<T>(2.f * dka[rb][4 * i], 2.f * dka[rb][4 * i + 1], 2.f * dka[rb][4 * i + 2],
                        2.f * dka[rb][4 * i + 3]));
    }
#pragma unroll
    for (int db = 0; db < DV / 32; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st4<T>(dvrow + 32 * db + 8 * i + 4 * hh,
               to4<T>(dva[db][4 * i] * kPInv, dva[db][4 * i + 1] * kPInv,
                      dva[db][4 * i + 2] * kPInv, dva[db][4 * i + 3] * kPInv));
  }
}

template <typename T, int DK, int DV, int M, bool SUM, bool DECAY>
hipError_t launch_kata_bwd(const KataArgs& a, int parts, hipStream_t stream) {
  if constexpr (SUM && M == 1) {
    // one group: the sum form is the concat form
    return launch_kata_bwd<T, DK, DV, M, false, DECAY>(a, parts, stream);
  } else {
    const float scale2 = a.scale * a.scale;
    const int nqt = (a.T + 127) / 128;
    // 16-bit tile kernels (both passes, which share the prescaled bf16 rows):
    // dv = 64, dk = 64 or dk = 128 with groups of at least 32
    constexpr bool kTiles = sizeof(T) == 2 && DV == 64 && (DK == 64 || (DK == 128 && DK / M >= 32));
    if (parts & KATA_BWD_DQ) {
      const int nbh = a.B * a.HQ;
      if constexpr (kTiles)
      {
        const OutNorm on{a.nw, const_cast<void*>(a.dy), a.rstd, a.nw_part, a.eps, nullptr};
        auto go = [&](auto onorm) {
          kata_bwd_dq_tile_kernel<T, DK, DV, M, SUM, DECAY, decltype(onorm)::value>
              <<<dim3(nqt * nbh), dim3(256), 0, stream>>>(
                  (const T*)a.q, (const T*)a.k, (const T*)a.v, (const T*)a.o, a.den,
                  (const T*)a.dout, (T*)a.dq, a.delta, a.c, a.dc, a.T, a.HQ, a.H, scale2, nqt,
                  nbh, on);
        };
        if (!a.dy) go(BoolC<false>{});
        else if constexpr (__is_same(T, __bf16)) go(BoolC<true>{});  // (the API admits bf16 only)
        else return hipErrorInvalidValue;
      }
      else if (a.dy)
        return hipErrorInvalidValue;  // the output norm is fused in the tile kernel only
      else
      kata_bwd_dq_kernel<T, DK, DV, M, SUM, DECAY><<<dim3(nqt * nbh), dim3(256), 0, stream>>>(
          (const T*)a.q, (const T*)a.k, (const T*)a.v, (const T*)a.o, a.den, (const T*)a.dout,
          (T*)a.dq, a.delta, a.c, a.dc, a.T, a.HQ, a.H, scale2, nqt, nbh);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    if (parts & KATA_BWD_DKDV) {
      const int nbk = a.B * a.H;
      if constexpr (kTiles) {
        constexpr int kw = kata_dkdv_waves<DK>();
        const int nkt = (a.T + 32 * kw - 1) / (32 * kw);
        kata_bwd_dkdv_tile_kernel<T, DK, DV, M, SUM, DECAY><<<dim3(nkt * nbk), dim3(64 * kw), 0, stream>>>(
            (const T*)a.q, (const T*)a.k, (const T*)a.v, a.den, a.delta, (const T*)a.dout,
            (T*)a.dk, (T*)a.dv, a.c, a.dc, a.T, a.HQ, a.H, scale2, nkt, nbk);
      } else
      kata_bwd_dkdv_kernel<T, DK, DV, M, SUM, DECAY><<<dim3(nqt * nbk), dim3(256), 0, stream>>>(
          (const T*)a.q, (const T*)a.k, (const T*)a.v, a.den, a.delta, (const T*)a.dout,
          (T*)a.dk, (T*)a.dv, a.c, a.dc, a.T, a.HQ, a.H, scale2, nqt, nbk);
      return hipGetLastError();
    }
    return hipSuccess;
  }
}

#define LINATT_BWD_INST(T, DK, DV, M)                                                                 \
  template hipError_t launch_kata_bwd<T, DK, DV, M, false, false>(const KataArgs&, int, hipStream_t); \
  template hipError_t launch_kata_bwd<T, DK, DV, M, true, false>(const KataArgs&, int, hipStream_t);  \
  template hipError_t launch_kata_bwd<T, DK, DV, M, false, true>(const KataArgs&, int, hipStream_t);

LINATT_KATA_SHAPES(LINATT_BWD_INST)

}  // namespace linatt
