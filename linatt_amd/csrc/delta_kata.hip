// SPD delta rule (DeltaKata), forward, for gfx950.
//
// Replaces the forward of the reference's flash_delta (kata/spd/flash_delta.py:
// _flash_U_kernel :25-183, _readout_kernel :898-972, _den_kernel :986-1046,
// _FlashDelta.forward :1060-1075), which the mixer's delta branch calls
// (kata/layer.py:377-420; configs/model/kata_delta_m1_340m.yaml:22).  With
// the sum-SPD kernel kappa(a, b) = sum_{g,h} (scale a_g . b_h)^2 (scale = s^2,
// s multiplies q and k in the reference):
//
//   A_kk = kappa(k, k),  U = (I + diag(beta) strict_lower(A_kk))^-1 diag(beta) V
//   num  = lower(kappa(q, k)) U,  den = rowsum(lower(kappa(q, k)))
//   o    = num / (den + eps)  (normalize)  or  num
//
// Chunks of 64 tokens.  Kernel 1 (dkata_prep), parallel over (batch, head,
// chunk): the chunk's own block of A_kk by MFMA and Tm = (I + N)^-1,
// N = diag(beta) strict_lower(A_kk), in fp32 in LDS; Tm leaves as a pair of
// 16-bit halves (Tm ~ hi + lo) so that MFMA products with it keep about
// 16 mantissa bits.  Kernel 2 (dkata_U), one workgroup per (batch, head),
// walks the chunks in order:
//
//   Ec^T = sum_{c' < c} U_c'^T A_kk[c', c]^T       (MFMA; A blocks recomputed)
//   U_c^T = (diag(beta) (V_c - Ec))^T Tm_c^T       (split 16-bit MFMA)
//
// and writes U (float32, the reference's dtype), a 16-bit copy for the
// readout, and U^T for the later chunks.  The readout is the KATA sum-score
// forward (kata_fwd_tile_kernel with SUM) applied to (q, k, U), whose o =
// num / den and den give num = o den; kernel 3 applies the normalisation.
#include "common.h"
#include "kata_kernels.h"

namespace linatt {

namespace {
inline size_t al256(size_t x) { return (x + 255) & ~size_t(255); }
}  // namespace

DKataLayout dkata_layout(int B, int T, int H, int D, int DV, int eb) {
  DKataLayout L{};
  const size_t NC = (size_t)(T + 63) / 64, Tp = NC * 64, BH = (size_t)B * H;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = al256(off + bytes); return o; };
  L.TmHi = take(BH * NC * 4096 * eb);
  L.TmLo = take(BH * NC * 4096 * eb);
  L.UT = take(BH * DV * Tp * eb);
  L.Ub = take((size_t)B * T * H * DV * eb);
  L.Ob = take((size_t)B * T * H * DV * eb);
  L.bytes = off;
  return L;
}

// ---------------------------------------------------------------------------
// Kernel 1: Tm = (I + N)^-1 per chunk, 4 waves.
// ---------------------------------------------------------------------------
template <typename T, int D, int M>
__global__ __launch_bounds__(256) void dkata_prep_kernel(DKataArgs a) {
  constexpr int E = D / M, KE = E / 16;
  static_assert(D == 64 && E % 16 == 0, "64-wide heads, groups of 16k");
  __shared__ __attribute__((aligned(16))) T Ks[64 * 64];
  __shared__ __attribute__((aligned(16))) float NT[64 * 64];  // N, then Tm (natural [i][j])
  __shared__ __attribute__((aligned(16))) float Bs[64];
  __shared__ __attribute__((aligned(16))) float Ys[16 * 48];

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int NC = (a.T + 63) / 64;
  const int ci = blockIdx.x % NC, bh = blockIdx.x / NC;
  const int b = bh / a.H, h = bh % a.H;
  const int t0 = 64 * ci;
  const T* kb = (const T*)a.k + ((int64_t)b * a.T * a.H + h) * D;
  const int64_t rs = (int64_t)a.H * D;

  // K tile (rows past T are zero) and beta
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int idx = tid + 256 * i, row = idx >> 3, ch = idx & 7;
    uint4 val = make_uint4(0, 0, 0, 0);
    if (t0 + row < a.T) val = *reinterpret_cast<const uint4*>(kb + (int64_t)(t0 + row) * rs + 8 * ch);
    *reinterpret_cast<uint4*>(reinterpret_cast<char*>(Ks) + tile_off(row, 8 * ch)) = val;
  }
  if (tid < 64) Bs[tid] = t0 + tid < a.T ? a.beta[((int64_t)b * a.T + t0 + tid) * a.H + h] : 0.f;
  __syncthreads();

  // N[i][j] = beta_i scale^2 sum_{g,h} (k_i,g . k_j,h)^2 for i > j, else 0;
  // wave w: rows 32 (w >> 1), columns 32 (w & 1) (the upper block is zero)
  {
    const int ib = w >> 1, jb = w & 1;
    if (ib == 0 && jb == 1) {
#pragma unroll
      for (int e = 0; e < 16; ++e) NT[(8 * (e >> 2) + 4 * hh + (e & 3)) * 64 + 32 + cl] = 0.f;
    } else {
      f32x16 A{};
#pragma unroll
      for (int g = 0; g < M; ++g)
#pragma unroll
        for (int g2 = 0; g2 < M; ++g2) {
          f32x16 r{};
#pragma unroll
          for (int kk = 0; kk < KE; ++kk)
            r = mma(tile_ld8<T>(Ks, 32 * ib + cl, g * E + 16 * kk + 8 * hh),
                    tile_ld8<T>(Ks, 32 * jb + cl, g2 * E + 16 * kk + 8 * hh), r);
          A += r * r;
        }
      const int j = 32 * jb + cl;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int i = 32 * ib + 8 * (e >> 2) + 4 * hh + (e & 3);
        NT[i * 64 + j] = i > j ? Bs[i] * a.scale2 * A[e] : 0.f;
      }
    }
  }
  __syncthreads();

  // diagonal blocks D_R = (I + N_RR)^-1, R = 0..3, by wave 0: lane 16 R + cc
  // solves for column cc by forward substitution (each finished x_k is
  // applied to every later row)
  if (w == 0) {
    const int R = lane >> 4, cc = lane & 15;
    float* blk = NT + 16 * R * 64 + 16 * R;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = i == cc ? 1.f : 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
#pragma unroll
      for (int i = k + 1; i < 16; ++i) x[i] -= blk[i * 64 + k] * x[k];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) blk[i * 64 + cc] = x[i];
  }
  __syncthreads();

  // block rows R = 1..3: Y = N_R,<R Tm_<R,<R, then Tm_R,<R = -D_R Y
  {
    const int ii = tid >> 4, cg = tid & 15;
    auto block_row = [&](auto RC) __attribute__((always_inline)) {
      constexpr int R = decltype(RC)::value;
      const int i = 16 * R + ii;
#pragma unroll
      for (int m = 0; m < R; ++m) {
        const int cc = cg + 16 * m;
        float y = 0.f;
#pragma unroll
        for (int j = 16 * m; j < 16 * R; ++j) y += NT[i * 64 + j] * NT[j * 64 + cc];
        Ys[ii * 48 + cc] = y;
      }
      __syncthreads();
#pragma unroll
      for (int m = 0; m < R; ++m) {
        const int cc = cg + 16 * m;
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k) t += NT[i * 64 + 16 * R + k] * Ys[k * 48 + cc];
        NT[i * 64 + cc] = -t;
      }
      __syncthreads();
    };
    block_row(IntC<1>{});
    block_row(IntC<2>{});
    block_row(IntC<3>{});
  }

  // Tm (unit lower triangular, zero above) as 16-bit hi + lo, natural [i][j]
  {
    const int r = tid >> 2, c0 = 16 * (tid & 3);
    const size_t base = ((size_t)bh * NC + ci) * 4096 + (size_t)r * 64 + c0;
    T* hi = (T*)(a.ws + a.L.TmHi) + base;
    T* lo = (T*)(a.ws + a.L.TmLo) + base;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      v8_t<T> vh, vl;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int j = c0 + 8 * hf + e;
        const float t = j < r ? NT[r * 64 + j] : (j == r ? 1.f : 0.f);
        const T th = (T)t;
        vh[e] = th;
        vl[e] = (T)(t - (float)th);
      }
      *reinterpret_cast<v8_t<T>*>(hi + 8 * hf) = vh;
      *reinterpret_cast<v8_t<T>*>(lo + 8 * hf) = vl;
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel 2: the pseudo-values U, chunk after chunk, one workgroup per (b, h).
// Wave w = (tb, ub): tb = w & 1 is its 32-row block of the current chunk's
// tokens t, ub = w >> 1 its 32-row block of each earlier chunk's tokens u
// (for Ec) and, afterwards, its 32-column block of U (jb = ub).
// ---------------------------------------------------------------------------
template <typename T, int D, int DV, int M>
__global__ __launch_bounds__(256) void dkata_U_kernel(DKataArgs a) {
  constexpr int E = D / M, KE = E / 16;
  static_assert(D == 64 && DV == 64 && E % 16 == 0, "64-wide heads");
  __shared__ __attribute__((aligned(16))) float Xc[4][16][64];   // Ec^T partials
  __shared__ __attribute__((aligned(16))) T Vh[64 * 64];          // (beta (V - Ec))^T hi, [j][u]
  __shared__ __attribute__((aligned(16))) T Vl[64 * 64];          // ... lo

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int tb = w & 1, ub = w >> 1;
  const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
  const int Tn = a.T, NC = (Tn + 63) / 64, Tp = 64 * NC;
  const int64_t rs = (int64_t)a.H * D, vrs = (int64_t)a.H * DV;
  const T* kb = (const T*)a.k + ((int64_t)b * Tn * a.H + h) * D;
  const T* vb = (const T*)a.v + ((int64_t)b * Tn * a.H + h) * DV;
  T* UT = (T*)(a.ws + a.L.UT) + (size_t)bh * DV * Tp;          // [j][t]
  const T* TmH = (const T*)(a.ws + a.L.TmHi) + (size_t)bh * NC * 4096;
  const T* TmL = (const T*)(a.ws + a.L.TmLo) + (size_t)bh * NC * 4096;

  auto krow = [&](int t, int kk) -> v8_t<T> {  // 8 dims of key row t (zero past T)
    return t < Tn ? ld8<T>(kb + (int64_t)t * rs + 16 * kk + 8 * hh) : zero8<T>();
  };

  for (int c = 0; c < NC; ++c) {
    const int t0 = 64 * c;
    const int tl = t0 + 32 * tb + cl;  // this lane's token of the current chunk
    v8_t<T> kc[D / 16];
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) kc[kk] = krow(tl, kk);

    // Ec^T[j][t] over the earlier chunks, u-block ub, both j-blocks
    f32x16 ec[2] = {f32x16{}, f32x16{}};
    v8_t<T> ka[D / 16], uo[2][2][2];  // operands of chunk cp (prefetched one ahead)
    auto fetch = [&](int cp, v8_t<T>* kx, v8_t<T> (*ux)[2][2]) __attribute__((always_inline)) {
      const int u0 = 64 * cp + 32 * ub;
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) kx[kk] = ld8<T>(kb + (int64_t)(u0 + cl) * rs + 16 * kk + 8 * hh);
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const T* row = UT + (size_t)(32 * jb + cl) * Tp + u0;
          ux[jb][ks][0] = ld_tr_op<T>(row, ks, hh);
        }
    };
    if (c > 0) fetch(0, ka, uo);
    for (int cp = 0; cp < c; ++cp) {
      v8_t<T> kn[D / 16], un[2][2][2];
      if (cp + 1 < c) fetch(cp + 1, kn, un);
      // A^T[u][t] = scale^2 sum_{g,g2} (k_u,g2 . k_t,g)^2  (u: chunk cp, block ub; t: block tb)
      f32x16 At{};
#pragma unroll
      for (int g = 0; g < M; ++g)
#pragma unroll
        for (int g2 = 0; g2 < M; ++g2) {
          f32x16 r{};
#pragma unroll
          for (int kk = 0; kk < KE; ++kk) r = mma(ka[g2 * KE + kk], kc[g * KE + kk], r);
          At += r * r;
        }
      At *= a.scale2;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const v8_t<T> bop = c_to_b<T>(At, ks);
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) ec[jb] = mma(uo[jb][ks][0], bop, ec[jb]);
      }
      if (cp + 1 < c) {
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) ka[kk] = kn[kk];
#pragma unroll
        for (int jb = 0; jb < 2; ++jb)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) uo[jb][ks][0] = un[jb][ks][0];
      }
    }
    // the partner wave (same tb, other ub) holds the other u-block's partial:
    // trade the j-block each does not keep (keep jb = ub)
#pragma unroll
    for (int e = 0; e < 16; ++e) Xc[w][e][lane] = ec[1 - ub][e];
    __syncthreads();
    const int partner = tb | ((1 - ub) << 1);
    f32x16 ecs = ec[ub];
#pragma unroll
    for (int e = 0; e < 16; ++e) ecs[e] += Xc[partner][e][lane];

    // beta_t (V[t][j] - Ec[t][j]) for j in block ub, as 16-bit hi + lo in [j][t]
    const float bt = tl < Tn ? a.beta[((int64_t)b * Tn + tl) * a.H + h] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const v4_t<T> vv = tl < Tn ? ld4<T>(vb + (int64_t)tl * vrs + 32 * ub + 8 * i + 4 * hh) : v4_t<T>{};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int e = 4 * i + r, j = 32 * ub + 8 * i + 4 * hh + r;
        const float x = bt * ((float)vv[r] - ecs[e]);
        const T xh = (T)x;
        T* ph = reinterpret_cast<T*>(reinterpret_cast<char*>(Vh) + tile_off(j, (32 * tb + cl) & ~3)) + (cl & 3);
        T* pl = reinterpret_cast<T*>(reinterpret_cast<char*>(Vl) + tile_off(j, (32 * tb + cl) & ~3)) + (cl & 3);
        *ph = xh;
        *pl = (T)(x - (float)xh);
      }
    }
    __syncthreads();

    // U^T[j][t] = sum_{u <= t} Vp^T[j][u] Tm[t][u]  (j block ub, t block tb)
    f32x16 uacc{};
    const T* tmh = TmH + (size_t)c * 4096 + (size_t)(32 * tb + cl) * 64;
    const T* tml = TmL + (size_t)c * 4096 + (size_t)(32 * tb + cl) * 64;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (ks >= 2 * (tb + 1)) break;  // Tm[t][u] = 0 for u > t
      const v8_t<T> bh8 = ld8<T>(tmh + 16 * ks + 8 * hh);
      const v8_t<T> bl8 = ld8<T>(tml + 16 * ks + 8 * hh);
      const v8_t<T> ah = tile_ld8<T>(Vh, 32 * ub + cl, 16 * ks + 8 * hh);
      const v8_t<T> alo = tile_ld8<T>(Vl, 32 * ub + cl, 16 * ks + 8 * hh);
      uacc = mma(ah, bh8, uacc);
      uacc = mma(ah, bl8, uacc);
      uacc = mma(alo, bh8, uacc);
    }

    // U (float32 and 16-bit, time-major) and U^T for the later chunks
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int j = 32 * ub + 8 * (e >> 2) + 4 * hh + (e & 3);
      UT[(size_t)j * Tp + tl] = (T)uacc[e];
    }
    if (tl < Tn) {
      const int64_t row = ((int64_t)b * Tn + tl) * a.H + h;
      T* ub16 = (T*)(a.ws + a.L.Ub) + row * DV;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j0 = 32 * ub + 8 * i + 4 * hh;
        st4<T>(ub16 + j0, to4<T>(uacc[4 * i], uacc[4 * i + 1], uacc[4 * i + 2], uacc[4 * i + 3]));
        if (a.U) *reinterpret_cast<float4*>(a.U + row * DV + j0) =
            make_float4(uacc[4 * i], uacc[4 * i + 1], uacc[4 * i + 2], uacc[4 * i + 3]);
      }
    }
    // U^T of this chunk is read by every wave from the next chunk on
    __threadfence_block();
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Kernel 3: o = num (/ (den + eps)) from the readout's o_k = num / den_k and
// den_k (the KATA forward leaves o_k = num where den_k = 0, num = 0 there).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void dkata_finish_kernel(DKataArgs a, int DV) {
  const int64_t rows = (int64_t)a.B * a.T * a.H;
  const int64_t n4 = rows * DV / 4;
  const T* ob = (const T*)(a.ws + a.L.Ob);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
    const int64_t row = 4 * i / DV;
    const float d = a.den[row];
    const float f = a.normalize ? d / (d + a.eps) : d;
    const v4_t<T> x = ld4<T>(ob + 4 * i);
    *reinterpret_cast<float4*>(a.o + 4 * i) =
        make_float4((float)x[0] * f, (float)x[1] * f, (float)x[2] * f, (float)x[3] * f);
  }
}

template <typename T, int D, int DV, int M>
hipError_t launch_dkata_fwd(const DKataArgs& a, hipStream_t stream) {
  const int NC = (a.T + 63) / 64, BH = a.B * a.H;
  dkata_prep_kernel<T, D, M><<<dim3(BH * NC), dim3(256), 0, stream>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  dkata_U_kernel<T, D, DV, M><<<dim3(BH), dim3(256), 0, stream>>>(a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  // readout: the KATA sum-score forward of (q, k, U) with the same scale
  KataArgs r{};
  r.q = a.q; r.k = a.k; r.v = a.ws + a.L.Ub; r.c = nullptr;
  r.o = a.ws + a.L.Ob; r.den = a.den;
  r.B = a.B; r.T = a.T; r.HQ = a.H; r.H = a.H; r.DK = D; r.DV = DV; r.M = M;
  r.scale = a.scale;
  e = launch_kata_fwd<T, D, DV, M, true, false>(r, stream);
  if (e != hipSuccess) return e;
  const int64_t n4 = (int64_t)a.B * a.T * a.H * DV / 4;
  const int blocks = (int)((n4 + 255) / 256 < 4096 ? (n4 + 255) / 256 : 4096);
  dkata_finish_kernel<T><<<dim3(blocks), dim3(256), 0, stream>>>(a, DV);
  return hipGetLastError();
}

#define LINATT_DKATA_INST(T, D, DV, M) \
  template hipError_t launch_dkata_fwd<T, D, DV, M>(const DKataArgs&, hipStream_t);
LINATT_DKATA_SHAPES(LINATT_DKATA_INST)

}  // namespace linatt
