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
#include "tri_inv.h"

namespace linatt {

namespace {
inline size_t al256(size_t x) { return (x + 255) & ~size_t(255); }
constexpr int kDkataSB = 8;  // chunks per super-chunk of the sequential passes
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
  L.Ein = take((size_t)B * T * H * DV * 4);
  L.bytes = off;
  return L;
}

DKataBwdLayout dkata_bwd_layout(int B, int T, int H, int D, int DV, int eb) {
  DKataBwdLayout L{};
  const size_t NC = (size_t)(T + 63) / 64, Tp = NC * 64, rows = (size_t)B * T * H;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = al256(off + bytes); return o; };
  L.dOp = take(rows * DV * eb);
  L.O16 = take(rows * DV * eb);
  L.ones = take(rows * 4);
  L.kws = take(kata_dop_offset((int64_t)rows) + (eb == 2 ? rows * DV * 2 : 0));
  L.dU = take(rows * DV * eb);
  L.dkr = take(rows * D * eb);
  L.Ksh = take(rows * D * eb);
  L.Xn = take(rows * DV * eb);
  L.XT = take((size_t)B * H * DV * Tp * eb);
  L.dbV = take(rows * DV * 4);
  L.dqe = take(rows * D * eb);
  L.dke = take(rows * D * eb);
  L.dve = take(rows * DV * eb);
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
  __shared__ __attribute__((aligned(16))) float Ys[512];

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

  // the off-diagonal blocks: 16 -> 32 merges in fp32, 32 -> 64 by MFMA
  tri_inv64_merge(NT, Ys, tid);

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
// Kernel 2: the pseudo-values U, chunk after chunk over one super-chunk of
// at most kDkataSB chunks [cb, ce), one workgroup per (b, h).  The chunks
// before cb enter through Ein (dkata_ext_kernel).  Wave w = (tb, ub): tb =
// w & 1 is its 32-row block of the current chunk's tokens t, ub = w >> 1 its
// 32-row block of each earlier chunk's tokens u (for Ec) and, afterwards,
// its 32-column block of U.
//
// The super-chunk's K and U^T tiles stay in LDS once their chunk is done
// (Ks, Us: 2 x 8 x 8 KB), so the Ec steps read only LDS and wait on no copy.
// The next chunk's key rows, values, beta and Tm operands are loaded into
// registers while the current chunk runs.
// ---------------------------------------------------------------------------
template <typename T, int D, int DV, int M>
__global__ __launch_bounds__(256) void dkata_U_kernel(DKataArgs a, int cb, int ce) {
  constexpr int E = D / M, KE = E / 16, TE = 64 * 64;
  static_assert(D == 64 && DV == 64 && E % 16 == 0, "64-wide heads");
  __shared__ __attribute__((aligned(16))) T Ks[kDkataSB][TE];  // K of chunk cb + i, [u][d]
  __shared__ __attribute__((aligned(16))) T Us[kDkataSB][TE];  // U^T of chunk cb + i, [j][u]
  // the Ec^T partials' exchange, then (beta (V - Ec))^T hi / lo, [j][u]
  __shared__ __attribute__((aligned(16))) float Xv[4 * 16 * 64];
  float(*Xc)[16][64] = reinterpret_cast<float(*)[16][64]>(Xv);
  T* Vh = reinterpret_cast<T*>(Xv);
  T* Vl = Vh + TE;

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int tb = w & 1, ub = w >> 1;
  const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
  const int Tn = a.T, NC = (Tn + 63) / 64, Tp = 64 * NC;
  const int64_t rs = (int64_t)a.H * D, vrs = (int64_t)a.H * DV;
  const T* kb = (const T*)a.k + ((int64_t)b * Tn * a.H + h) * D;
  const T* vb = (const T*)a.v + ((int64_t)b * Tn * a.H + h) * DV;
  T* UT = (T*)(a.ws + a.L.UT) + (size_t)bh * DV * Tp;          // [j][t]
  const T* TmH = (const T*)(a.ws + a.L.TmHi) + (size_t)bh * NC * TE;
  const T* TmL = (const T*)(a.ws + a.L.TmLo) + (size_t)bh * NC * TE;

  // this lane's token of chunk c: 8 dims of K per k-step, its 16 V columns,
  // beta, its row of Tm (hi, lo) as the B operands of the U product, and
  // (after the first super-chunk) its Ein columns
  auto load_chunk = [&](int c, v8_t<T>* kx, v4_t<T>* vx, float& bx, v8_t<T>* th, v8_t<T>* tlo,
                        float4* ex) __attribute__((always_inline)) {
    const int t = 64 * c + 32 * tb + cl;
    const bool in = t < Tn;
    if (cb > 0) {
      const float* er = (const float*)(a.ws + a.L.Ein) + (((int64_t)b * Tn + t) * a.H + h) * DV;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        ex[q] = in ? *reinterpret_cast<const float4*>(er + 32 * ub + 8 * q + 4 * hh) : float4{};
    }
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
      kx[kk] = in ? ld8<T>(kb + (int64_t)t * rs + 16 * kk + 8 * hh) : zero8<T>();
#pragma unroll
    for (int i = 0; i < 4; ++i)
      vx[i] = in ? ld4<T>(vb + (int64_t)t * vrs + 32 * ub + 8 * i + 4 * hh) : v4_t<T>{};
    bx = in ? a.beta[((int64_t)b * Tn + t) * a.H + h] : 0.f;
    const size_t tr = (size_t)c * TE + (size_t)(32 * tb + cl) * 64 + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      th[ks] = ld8<T>(TmH + tr + 16 * ks);
      tlo[ks] = ld8<T>(TmL + tr + 16 * ks);
    }
  };
  // A^T[u][t] / scale^2 = sum_{g,g2} (k_u,g2 . k_t,g)^2 for the 32 keys u of
  // block ub of one earlier chunk (K tile Kt) and this wave's 32 tokens t,
  // as the two B operands of the Ec product
  auto gram = [&](const T* Kt, const v8_t<T>* kc, v8_t<T>* bop) __attribute__((always_inline)) {
    v8_t<T> ka[D / 16];
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) ka[kk] = tile_ld8<T>(Kt, 32 * ub + cl, 16 * kk + 8 * hh);
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
    bop[0] = c_to_b<T>(At, 0);
    bop[1] = c_to_b<T>(At, 1);
  };
  // Ec^T[j][t] (/ scale^2) += U^T[j][u] A^T[u][t] over those 32 keys
  auto ec_update = [&](const T* Ut, const v8_t<T>* bop, f32x16 (&ec)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
        ec[jb] = mma(tile_ldp8<T>(Ut, 32 * jb + cl, 32 * ub, ks, hh), bop[ks], ec[jb]);
  };

  v8_t<T> kc[D / 16], tmh[4], tml[4];
  v4_t<T> vc[4];
  float bc;
  float4 einc[4] = {};
  load_chunk(cb, kc, vc, bc, tmh, tml, einc);
  vm_drain();  // the loop sees these operands as loaded, like the ones it prefetches

  for (int c = cb; c < ce; ++c) {
    const int i = c - cb;
    const int tl = 64 * c + 32 * tb + cl;  // this lane's token of the current chunk
    // the next chunk's operands, in flight while this one runs
    v8_t<T> kn[D / 16], tnh[4], tnl[4];
    v4_t<T> vn[4];
    float bn = 0.f;
    float4 einn[4] = {};
    if (c + 1 < ce) load_chunk(c + 1, kn, vn, bn, tnh, tnl, einn);

    // Ec over the super-chunk's earlier chunks cb .. c - 1, all in LDS; the
    // Gram block of step s + 1 is formed while the Ec product of step s runs
    f32x16 ec[2] = {f32x16{}, f32x16{}};
    if (i > 0) {
      v8_t<T> bop[2];
      gram(Ks[0], kc, bop);
      for (int s = 0; s < i; ++s) {
        v8_t<T> bnext[2];
        if (s + 1 < i) gram(Ks[s + 1], kc, bnext);
        ec_update(Us[s], bop, ec);
        bop[0] = bnext[0];
        bop[1] = bnext[1];
      }
    }

    // the partner wave (same tb, other ub) holds the other u-block's partial:
    // trade the j-block each does not keep (keep jb = ub)
#pragma unroll
    for (int e = 0; e < 16; ++e) Xc[w][e][lane] = ec[1 - ub][e];
    // K of this chunk for the later ones (rows 32 tb + cl)
    if (ub == 0) {
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk)
        *reinterpret_cast<v8_t<T>*>(reinterpret_cast<char*>(Ks[i]) + tile_off(32 * tb + cl, 16 * kk + 8 * hh)) = kc[kk];
    }
    block_barrier();
    const int partner = tb | ((1 - ub) << 1);
    f32x16 ecs = ec[ub];
#pragma unroll
    for (int e = 0; e < 16; ++e) ecs[e] = a.scale2 * (ecs[e] + Xc[partner][e][lane]);
    // Ein held the sum over the chunks before cb (dkata_ext_kernel)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ecs[4 * q] += einc[q].x;
      ecs[4 * q + 1] += einc[q].y;
      ecs[4 * q + 2] += einc[q].z;
      ecs[4 * q + 3] += einc[q].w;
    }
    // the next chunk's operands have landed during the steps: from here on
    // no load is waited for behind this chunk's stores
    vm_drain();
    if (a.keep_e && tl < Tn) {  // the whole inter-chunk part of E_t, for dbeta
      float* er = (float*)(a.ws + a.L.Ein) + (((int64_t)b * Tn + tl) * a.H + h) * DV;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<float4*>(er + 32 * ub + 8 * q + 4 * hh) =
            make_float4(ecs[4 * q], ecs[4 * q + 1], ecs[4 * q + 2], ecs[4 * q + 3]);
    }
    block_barrier();  // Vh / Vl overwrite the exchange

    // beta_t (V[t][j] - Ec[t][j]) for j in block ub, as 16-bit hi + lo in [j][t]
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int e = 4 * q + r, j = 32 * ub + 8 * q + 4 * hh + r;
        const float x = bc * ((float)vc[q][r] - ecs[e]);
        const T xh = (T)x;
        const int off = tile_off(j, (32 * tb + cl) & ~3);
        reinterpret_cast<T*>(reinterpret_cast<char*>(Vh) + off)[cl & 3] = xh;
        reinterpret_cast<T*>(reinterpret_cast<char*>(Vl) + off)[cl & 3] = (T)(x - (float)xh);
      }
    }
    block_barrier();

    // U^T[j][t] = sum_{u <= t} Vp^T[j][u] Tm[t][u]  (j block ub, t block tb)
    f32x16 uacc{};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (ks >= 2 * (tb + 1)) break;  // Tm[t][u] = 0 for u > t
      const v8_t<T> ah = tile_ld8<T>(Vh, 32 * ub + cl, 16 * ks + 8 * hh);
      const v8_t<T> alo = tile_ld8<T>(Vl, 32 * ub + cl, 16 * ks + 8 * hh);
      uacc = mma(ah, tmh[ks], uacc);
      uacc = mma(ah, tml[ks], uacc);
      uacc = mma(alo, tmh[ks], uacc);
    }

    // U^T for the later chunks (global and Us) and U (float32 and 16-bit,
    // time-major)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int j = 32 * ub + 8 * (e >> 2) + 4 * hh + (e & 3);
      const T u16 = (T)uacc[e];
      UT[(size_t)j * Tp + tl] = u16;
      reinterpret_cast<T*>(reinterpret_cast<char*>(Us[i]) + tile_off(j, (32 * tb + cl) & ~3))[cl & 3] = u16;
    }
    if (tl < Tn) {
      const int64_t row = ((int64_t)b * Tn + tl) * a.H + h;
      T* ub16 = (T*)(a.ws + a.L.Ub) + row * DV;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j0 = 32 * ub + 8 * q + 4 * hh;
        st4<T>(ub16 + j0, to4<T>(uacc[4 * q], uacc[4 * q + 1], uacc[4 * q + 2], uacc[4 * q + 3]));
        if (a.U) *reinterpret_cast<float4*>(a.U + row * DV + j0) =
            make_float4(uacc[4 * q], uacc[4 * q + 1], uacc[4 * q + 2], uacc[4 * q + 3]);
      }
    }
    // Us / Ks for the next chunk's steps, and the Vh / Vl reuse
    block_barrier();
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) kc[kk] = kn[kk];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      vc[q] = vn[q];
      tmh[q] = tnh[q];
      tml[q] = tnl[q];
      einc[q] = einn[q];
    }
    bc = bn;
  }
}

// ---------------------------------------------------------------------------
// Kernel 2a: the part of a chunk-sequential pass that comes from chunks
// outside the current super-chunk, in parallel over (b, h, pair of target
// chunks):
//   dst_t = scale^2 sum_{c' in [s0, s0 + n)} A[c, c'] Y_c'
// for the tokens t of the nsb chunks c0 .. c0 + nsb - 1, with A[t][u] /
// scale^2 = sum_{g,g2} (k_t,g . k_u,g2)^2 and Y^T = srcT ([j][t] per (b, h),
// rows padded to whole chunks).  The forward takes Y = U over the earlier
// chunks (into Ein), the backward Y = X = beta dbV over the later ones (into
// dbV's rows, which the dbV pass reads and then overwrites).  Waves and
// products as in dkata_U_kernel, for two target chunks at once, so each
// source tile copied into LDS serves twice the products; the source
// chunks' K and Y^T tiles stream through a 4-slot ring; a head's target
// chunks run on one XCD, where they share those tiles in L2.
// ---------------------------------------------------------------------------
template <typename T, int D, int DV, int M>
__global__ __launch_bounds__(256) void dkata_ext_kernel(const T* __restrict__ k, const T* __restrict__ srcT,
                                                        float* __restrict__ dst, int H, int Tn, float scale2,
                                                        int c0, int nsb, int s0, int n, int BH) {
  constexpr int E = D / M, KE = E / 16, kRing = 4, TE = 64 * 64;
  static_assert(D == 64 && DV == 64 && E % 16 == 0, "64-wide heads");
  __shared__ __attribute__((aligned(16))) T ring[kRing][2][TE];
  __shared__ __attribute__((aligned(16))) float Xc[4][16][64];

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int tb = w & 1, ub = w >> 1;
  const int npair = (nsb + 1) / 2;
  int bh, jp;
  map_block(blockIdx.x, npair, BH, jp, bh, false);
  const int b = bh / H, h = bh % H;
  const int NC = (Tn + 63) / 64, Tp = 64 * NC;
  const int64_t rs = (int64_t)H * D;
  const T* kb = k + ((int64_t)b * Tn * H + h) * D;
  const T* YT = srcT + (size_t)bh * DV * Tp;
  // this lane's token in each target chunk (the second past the range when
  // nsb is odd: its rows then hold zeros and are not stored)
  int tl[2];
  bool st[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    tl[x] = 64 * (c0 + 2 * jp + x) + 32 * tb + cl;
    st[x] = 2 * jp + x < nsb && tl[x] < Tn;
  }

  v8_t<T> kc[2][D / 16];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
      kc[x][kk] = st[x] ? ld8<T>(kb + (int64_t)tl[x] * rs + 16 * kk + 8 * hh) : zero8<T>();
  auto issue_step = [&](int s, int slot) __attribute__((always_inline)) {
    const int cp = s0 + s;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      dma_tile64<T>(kb, rs, 64 * cp, Tn, ring[slot][0], 2 * w + i, lane);
      dma_tile64<T>(YT + 64 * cp, Tp, 0, DV, ring[slot][1], 2 * w + i, lane);
    }
  };
  // the Gram blocks of source keys (block ub of tile Kt) against both target
  // chunks' tokens, as the B operands of the Y products
  auto gram = [&](const T* Kt, v8_t<T> (&bop)[2][2]) __attribute__((always_inline)) {
    v8_t<T> ka[D / 16];
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) ka[kk] = tile_ld8<T>(Kt, 32 * ub + cl, 16 * kk + 8 * hh);
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      f32x16 At{};
#pragma unroll(M > 2 ? 1 : M)  // M = 4 fully unrolled keeps 16 Gram blocks live and spills
      for (int g = 0; g < M; ++g)
#pragma unroll
        for (int g2 = 0; g2 < M; ++g2) {
          f32x16 r{};
#pragma unroll
          for (int kk = 0; kk < KE; ++kk) r = mma(ka[g2 * KE + kk], kc[x][g * KE + kk], r);
          At += r * r;
        }
      bop[x][0] = c_to_b<T>(At, 0);
      bop[x][1] = c_to_b<T>(At, 1);
    }
  };
  auto y_update = [&](const T* Yt, const v8_t<T> (&bop)[2][2], f32x16 (&ec)[2][2]) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        const v8_t<T> ya = tile_ldp8<T>(Yt, 32 * jb + cl, 32 * ub, ks, hh);
#pragma unroll
        for (int x = 0; x < 2; ++x) ec[x][jb] = mma(ya, bop[x][ks], ec[x][jb]);
      }
  };

  for (int s = 0; s < min(kRing - 1, n); ++s) issue_step(s, s);
  f32x16 ec[2][2] = {{f32x16{}, f32x16{}}, {f32x16{}, f32x16{}}};
  v8_t<T> bop[2][2];
  vm_wait_barrier_n(4 * (min(kRing - 1, n) - 1));
  gram(ring[0][0], bop);
  for (int s = 0; s < n; ++s) {
    v8_t<T> bnext[2][2];
    if (s + 1 < n) {
      // copies issued after slot s + 1's: step s + 2 when it exists
      vm_wait_barrier_n(4 * min(kRing - 3, n - 2 - s));
      if (s + kRing - 1 < n) issue_step(s + kRing - 1, (s + kRing - 1) % kRing);
      gram(ring[(s + 1) % kRing][0], bnext);
    }
    y_update(ring[s % kRing][1], bop, ec);
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      bop[x][0] = bnext[x][0];
      bop[x][1] = bnext[x][1];
    }
  }
  // the partner wave (same tb, other ub) holds the other u-block's partial:
  // trade the j-block each does not keep, one target chunk at a time
  const int partner = tb | ((1 - ub) << 1);
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const f32x16 keep = ub ? ec[x][1] : ec[x][0];
    const f32x16 give = ub ? ec[x][0] : ec[x][1];
    if (x) block_barrier();  // every wave has read the first chunk's partials
#pragma unroll
    for (int e = 0; e < 16; ++e) Xc[w][e][lane] = give[e];
    block_barrier();
    if (st[x]) {
      float* er = dst + (((int64_t)b * Tn + tl[x]) * H + h) * DV;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v4[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v4[r] = scale2 * (keep[4 * i + r] + Xc[partner][4 * i + r][lane]);
        *reinterpret_cast<float4*>(er + 32 * ub + 8 * i + 4 * hh) = make_float4(v4[0], v4[1], v4[2], v4[3]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel 3 (normalize only): o = num / (den + eps) in place, from the
// readout's float32 numerator and den.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dkata_finish_kernel(DKataArgs a, int DV) {
  const int64_t rows = (int64_t)a.B * a.T * a.H;
  const int64_t n4 = rows * DV / 4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
    const int64_t row = 4 * i / DV;
    const float f = 1.f / (a.den[row] + a.eps);
    float4 x = *reinterpret_cast<const float4*>(a.o + 4 * i);
    x.x *= f; x.y *= f; x.z *= f; x.w *= f;
    *reinterpret_cast<float4*>(a.o + 4 * i) = x;
  }
}

template <typename T, int D, int DV, int M>
hipError_t launch_dkata_fwd(const DKataArgs& a, hipStream_t stream) {
  const int NC = (a.T + 63) / 64, BH = a.B * a.H;
  dkata_prep_kernel<T, D, M><<<dim3(BH * NC), dim3(256), 0, stream>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // chunk-sequential only inside super-chunks of kDkataSB chunks; between
  // them, the earlier super-chunks' contribution in parallel
  for (int cb = 0; cb < NC; cb += kDkataSB) {
    const int ce = cb + kDkataSB < NC ? cb + kDkataSB : NC;
    if (cb > 0) {
      dkata_ext_kernel<T, D, DV, M><<<dim3(BH * ((ce - cb + 1) / 2)), dim3(256), 0, stream>>>(
          (const T*)a.k, (const T*)(a.ws + a.L.UT), (float*)(a.ws + a.L.Ein), a.H, a.T, a.scale2, cb,
          ce - cb, 0, cb, BH);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    dkata_U_kernel<T, D, DV, M><<<dim3(BH), dim3(256), 0, stream>>>(a, cb, ce);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  // readout: the KATA sum-score forward of (q, k, U) with the same scale,
  // its float32 numerator straight into o (no 16-bit rounding of o)
  KataArgs r{};
  r.q = a.q; r.k = a.k; r.v = a.ws + a.L.Ub; r.c = nullptr;
  r.o = nullptr; r.num32 = a.o; r.den = a.den;
  r.B = a.B; r.T = a.T; r.HQ = a.H; r.H = a.H; r.DK = D; r.DV = DV; r.M = M;
  r.scale = a.scale;
  e = launch_kata_fwd<T, D, DV, M, true, false>(r, stream);
  if (e != hipSuccess || !a.normalize) return e;
  const int64_t n4 = (int64_t)a.B * a.T * a.H * DV / 4;
  const int blocks = (int)((n4 + 255) / 256 < 4096 ? (n4 + 255) / 256 : 4096);
  dkata_finish_kernel<<<dim3(blocks), dim3(256), 0, stream>>>(a, DV);
  return hipGetLastError();
}

// ===========================================================================
// Backward (kata/spd/flash_delta.py:1084-1108, flash_delta_bwd :830-895).
// With do' = do / (den + eps), z_t = <do'_t, o_t> (normalize) or do' = do,
// z = 0, and X = diag(beta) dbV:
//
//   readout:  dA_qk[t,s] = <do'_t, U_s> - z_t (s <= t),  dU = lower(A_qk)^T do'
//   solve:    dbV = (I + diag(beta) strict_lower(A_kk))^-T dU
//   erase:    dA_kk[t,s] = -beta_t <dbV_t, U_s> (s < t)
//   dv = beta dbV,  dbeta_t = <v_t - E_t, dbV_t>,  E_t = sum_{s<t} A_kk[t,s] U_s
//
// and dq, dk through kappa.  The readout part is the KATA sum-score backward
// of (q, k, v := U) with den := 1 and o := the normalised output (or 0):
// it then forms exactly scale^2 dA_qk and returns dq, the readout part of dk
// and dU as its dv.  The erase part is the same backward run on queries
// shifted by one token, q'_t = k_{t+1}, keys k, values U, dO'_t = -X_{t+1},
// o := 0: its causal pairs s <= t are exactly the strict pairs s < t + 1 of
// A_kk, its dq' is the query side (dk_{t+1} += dq'_t) and its dk the key
// side.  The reverse solve walks the chunks backwards like dkata_U_kernel
// walks them forwards.
// ===========================================================================

template <typename T>
__global__ __launch_bounds__(256) void dkata_bwd_prep_kernel(DKataBwdArgs a, int D, int DV) {
  const int64_t rows = (int64_t)a.B * a.T * a.H, n4 = rows * DV / 4;
  const int64_t hrow = (int64_t)a.T * a.H;  // rows per batch entry
  // k one token later (rows t < T - 1 of each batch entry), zero at T - 1;
  // the last row of the shifted -X is zeroed here, the rest written by the
  // reverse solve
  T* ksh = (T*)(a.bws + a.BL.Ksh);
  T* xn = (T*)(a.bws + a.BL.Xn);
  const int64_t k4 = rows * D / 4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < k4; i += (int64_t)gridDim.x * 256) {
    const int64_t row = 4 * i / D, bt = row % hrow;  // (t, h) within the batch entry
    if (bt < hrow - a.H) {
      st4<T>(ksh + 4 * i, ld4<T>((const T*)a.k + 4 * i + (int64_t)a.H * D));
    } else {
      st4<T>(ksh + 4 * i, to4<T>(0.f, 0.f, 0.f, 0.f));
      const int64_t col = 4 * i - row * D;  // zero the same row of xn, D and DV apart
      for (int64_t c = col; c < DV; c += D) st4<T>(xn + row * DV + c, to4<T>(0.f, 0.f, 0.f, 0.f));
    }
  }
  T* dop = (T*)(a.bws + a.BL.dOp);
  T* o16 = (T*)(a.bws + a.BL.O16);
  float* ones = (float*)(a.bws + a.BL.ones);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
    const int64_t row = 4 * i / DV;
    const float f = a.normalize ? 1.f / (a.den[row] + a.eps) : 1.f;
    const float4 g = reinterpret_cast<const float4*>(a.dout)[i];
    st4<T>(dop + 4 * i, to4<T>(g.x * f, g.y * f, g.z * f, g.w * f));
    if (a.normalize) {
      const float4 o = reinterpret_cast<const float4*>(a.o)[i];
      st4<T>(o16 + 4 * i, to4<T>(o.x, o.y, o.z, o.w));
    }
    if ((4 * i) % DV == 0) ones[row] = 1.f;
  }
}

// dbV = (I + diag(beta) strict_lower(A_kk))^-T dU, chunk after chunk from the
// last of one super-chunk [cb, ce) to its first: R_c = sum_{c' > c} A_kk[c,
// c'] X_c' (A_kk is symmetric), dbV_c = Tm_c^T (dU_c - R_c), X_c = beta_c
// dbV_c.  The chunks at or after ce enter through dbV's rows
// (dkata_ext_kernel).  Layout and schedule as dkata_U_kernel with the chunk
// order reversed: wave w = (tb, ub), the super-chunk's K and X^T tiles
// resident in LDS; the next chunk's Tm is copied into LDS (read back
// transposed) and its other operands loaded into registers while the
// current chunk runs.  LDS: 160 KB.
template <typename T, int D, int DV, int M>
__global__ __launch_bounds__(256) void dkata_dbV_kernel(DKataBwdArgs a, int cb, int ce) {
  constexpr int E = D / M, KE = E / 16, TE = 64 * 64;
  static_assert(D == 64 && DV == 64 && E % 16 == 0, "64-wide heads");
  __shared__ __attribute__((aligned(16))) T Ks[kDkataSB][TE];  // K of chunk cb + i, [u][d]
  __shared__ __attribute__((aligned(16))) T Xs[kDkataSB][TE];  // X^T of chunk cb + i, [j][u]
  // the R^T partials' exchange, then (dU - R)^T hi / lo, [j][t]
  __shared__ __attribute__((aligned(16))) float Xv[4 * 16 * 64];
  __shared__ __attribute__((aligned(16))) T TmS[2][TE];  // Tm hi / lo of the chunk, [t][i]
  float(*Xc)[16][64] = reinterpret_cast<float(*)[16][64]>(Xv);
  T* Vh = reinterpret_cast<T*>(Xv);
  T* Vl = Vh + TE;

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int tb = w & 1, ub = w >> 1;
  const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
  const int Tn = a.T, NC = (Tn + 63) / 64, Tp = 64 * NC;
  const int64_t rs = (int64_t)a.H * D, vrs = (int64_t)a.H * DV;
  const T* kb = (const T*)a.k + ((int64_t)b * Tn * a.H + h) * D;
  const T* dub = (const T*)(a.bws + a.BL.dU) + ((int64_t)b * Tn * a.H + h) * DV;
  T* XT = (T*)(a.bws + a.BL.XT) + (size_t)bh * DV * Tp;  // [j][t]
  const T* TmH = (const T*)(a.ws + a.L.TmHi) + (size_t)bh * NC * TE;
  const T* TmL = (const T*)(a.ws + a.L.TmLo) + (size_t)bh * NC * TE;

  auto issue_tm = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      dma_tile64<T>(TmH + (size_t)c * TE, 64, 0, 64, TmS[0], 2 * w + i, lane);
      dma_tile64<T>(TmL + (size_t)c * TE, 64, 0, 64, TmS[1], 2 * w + i, lane);
    }
  };
  // this lane's token of chunk c: K row, dU columns, beta and (before the
  // last super-chunk) the part of R from the later super-chunks
  auto load_chunk = [&](int c, v8_t<T>* kx, v4_t<T>* dx, float& bx, float4* rx)
      __attribute__((always_inline)) {
    const int t = 64 * c + 32 * tb + cl;
    const bool in = t < Tn;
    if (ce < NC) {  // dbV's row holds the part of R_t from the chunks at or after ce
      const float* rr = (const float*)(a.bws + a.BL.dbV) + (((int64_t)b * Tn + t) * a.H + h) * DV;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        rx[q] = in ? *reinterpret_cast<const float4*>(rr + 32 * ub + 8 * q + 4 * hh) : float4{};
    }
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
      kx[kk] = in ? ld8<T>(kb + (int64_t)t * rs + 16 * kk + 8 * hh) : zero8<T>();
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dx[i] = in ? ld4<T>(dub + (int64_t)t * vrs + 32 * ub + 8 * i + 4 * hh) : v4_t<T>{};
    bx = in ? a.beta[((int64_t)b * Tn + t) * a.H + h] : 0.f;
  };
  auto gram = [&](const T* Kt, const v8_t<T>* kc, v8_t<T>* bop) __attribute__((always_inline)) {
    v8_t<T> ka[D / 16];
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) ka[kk] = tile_ld8<T>(Kt, 32 * ub + cl, 16 * kk + 8 * hh);
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
    bop[0] = c_to_b<T>(At, 0);
    bop[1] = c_to_b<T>(At, 1);
  };
  auto r_update = [&](const T* Xt, const v8_t<T>* bop, f32x16 (&ec)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
        ec[jb] = mma(tile_ldp8<T>(Xt, 32 * jb + cl, 32 * ub, ks, hh), bop[ks], ec[jb]);
  };

  v8_t<T> kc[D / 16];
  v4_t<T> duc[4];
  float bc;
  float4 rxc[4] = {};
  load_chunk(ce - 1, kc, duc, bc, rxc);
  issue_tm(ce - 1);
  vm_drain();  // the loop sees these operands as loaded, like the ones it prefetches

  for (int c = ce - 1; c >= cb; --c) {
    const int i = c - cb;
    const int tl = 64 * c + 32 * tb + cl;
    v8_t<T> kn[D / 16];
    v4_t<T> dun[4];
    float bn = 0.f;
    float4 rxn[4] = {};
    if (c > cb) load_chunk(c - 1, kn, dun, bn, rxn);

    // R over the super-chunk's later chunks c + 1 .. ce - 1, all in LDS
    f32x16 ec[2] = {f32x16{}, f32x16{}};
    const int n = ce - 1 - c;  // step s: chunk c + 1 + s
    if (n > 0) {
      v8_t<T> bop[2];
      gram(Ks[i + 1], kc, bop);
      for (int s = 0; s < n; ++s) {
        v8_t<T> bnext[2];
        if (s + 1 < n) gram(Ks[i + 2 + s], kc, bnext);
        r_update(Xs[i + 1 + s], bop, ec);
        bop[0] = bnext[0];
        bop[1] = bnext[1];
      }
    }

#pragma unroll
    for (int e = 0; e < 16; ++e) Xc[w][e][lane] = ec[1 - ub][e];
    if (ub == 0) {
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk)
        *reinterpret_cast<v8_t<T>*>(reinterpret_cast<char*>(Ks[i]) + tile_off(32 * tb + cl, 16 * kk + 8 * hh)) = kc[kk];
    }
    block_barrier();
    const int partner = tb | ((1 - ub) << 1);
    f32x16 ecs = ec[ub];
#pragma unroll
    for (int e = 0; e < 16; ++e) ecs[e] = a.scale2 * (ecs[e] + Xc[partner][e][lane]);
    // the part of R from the chunks at or after ce (dkata_ext_kernel, in
    // dbV's rows, which this lane overwrites with dbV below)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ecs[4 * q] += rxc[q].x;
      ecs[4 * q + 1] += rxc[q].y;
      ecs[4 * q + 2] += rxc[q].z;
      ecs[4 * q + 3] += rxc[q].w;
    }
    // this chunk's Tm and the next chunk's operands have landed during the
    // steps: from here on no load is waited for behind this chunk's stores
    vm_drain();
    block_barrier();  // Vh / Vl overwrite the exchange; every wave's Tm copies are in

    // (dU - R)^T[j][t] for j in block ub, as 16-bit hi + lo
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int e = 4 * q + r, j = 32 * ub + 8 * q + 4 * hh + r;
        const float x = (float)duc[q][r] - ecs[e];
        const T xh = (T)x;
        const int off = tile_off(j, (32 * tb + cl) & ~3);
        reinterpret_cast<T*>(reinterpret_cast<char*>(Vh) + off)[cl & 3] = xh;
        reinterpret_cast<T*>(reinterpret_cast<char*>(Vl) + off)[cl & 3] = (T)(x - (float)xh);
      }
    }
    block_barrier();

    // dbV^T[j][i] = sum_{t >= i} (dU - R)^T[j][t] Tm[t][i]  (j block ub, i block tb)
    f32x16 uacc{};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (ks < 2 * tb) continue;  // Tm[t][i] = 0 for t < i
      const v8_t<T> bh8 = tile_tr8<T>(TmS[0], 0, 32 * tb, ks, lane);
      const v8_t<T> bl8 = tile_tr8<T>(TmS[1], 0, 32 * tb, ks, lane);
      const v8_t<T> ah = tile_ldp8<T>(Vh, 32 * ub + cl, 0, ks, hh);
      const v8_t<T> alo = tile_ldp8<T>(Vl, 32 * ub + cl, 0, ks, hh);
      uacc = mma(ah, bh8, uacc);
      uacc = mma(ah, bl8, uacc);
      uacc = mma(alo, bh8, uacc);
    }

    // X = beta dbV: X^T for the earlier chunks (global, and Xs); dbV
    // (float32) and -X (the erase pass's dO), time-major
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int j = 32 * ub + 8 * (e >> 2) + 4 * hh + (e & 3);
      const T x16 = (T)(bc * uacc[e]);
      XT[(size_t)j * Tp + tl] = x16;
      reinterpret_cast<T*>(reinterpret_cast<char*>(Xs[i]) + tile_off(j, (32 * tb + cl) & ~3))[cl & 3] = x16;
    }
    if (tl < Tn) {
      const int64_t row = ((int64_t)b * Tn + tl) * a.H + h;
      float* dbv = (float*)(a.bws + a.BL.dbV) + row * DV;
      // -X_t goes to row t - 1 of the shifted erase dO
      T* xn = tl > 0 ? (T*)(a.bws + a.BL.Xn) + (row - a.H) * DV : nullptr;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j0 = 32 * ub + 8 * q + 4 * hh;
        *reinterpret_cast<float4*>(dbv + j0) =
            make_float4(uacc[4 * q], uacc[4 * q + 1], uacc[4 * q + 2], uacc[4 * q + 3]);
        if (xn)
          st4<T>(xn + j0, to4<T>(-(float)(T)(bc * uacc[4 * q]), -(float)(T)(bc * uacc[4 * q + 1]),
                                 -(float)(T)(bc * uacc[4 * q + 2]), -(float)(T)(bc * uacc[4 * q + 3])));
      }
    }
    block_barrier();
    if (c > cb) issue_tm(c - 1);  // every wave is done reading TmS
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) kc[kk] = kn[kk];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      duc[q] = dun[q];
      rxc[q] = rxn[q];
    }
    bc = bn;
  }
}

// Per (b, h, chunk), four waves (tb, ub) as in dkata_U_kernel:
//   E_t = Ein_t + sum_{s<t in the chunk} kappa(k_t, k_s) U_s  (MFMA, the
//         chunk's own Gram block masked strictly lower, U^T from the forward),
//   dbeta_t = <v_t - E_t, dbV_t>,  dv_t = beta_t dbV_t,
//   dk_t = readout part + key side of the erase pass + its query side one row
//          earlier.
template <typename T, int D, int DV, int M>
__global__ __launch_bounds__(256) void dkata_bwd_fix_kernel(DKataBwdArgs a) {
  constexpr int E = D / M, KE = E / 16, TE = 64 * 64;
  static_assert(D == 64 && DV == 64 && E % 16 == 0, "64-wide heads");
  __shared__ __attribute__((aligned(16))) T Ks[TE];   // K rows of the chunk
  __shared__ __attribute__((aligned(16))) T UTs[TE];  // U^T [j][s] of the chunk
  // sum over s of A^T[s][t] U^T[j][s], [t][j]; the odd pitch keeps both the
  // C-layout writes (32 tokens per instruction) and the row reads below free
  // of bank conflicts
  __shared__ float Ecs[64][65];

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int tb = w & 1, ub = w >> 1;
  const int Tn = a.T, NC = (Tn + 63) / 64, Tp = 64 * NC;
  const int ci = blockIdx.x % NC, bh = blockIdx.x / NC, b = bh / a.H, h = bh % a.H;
  const int t0 = 64 * ci;
  const int64_t rs = (int64_t)a.H * D;
  const T* kb = (const T*)a.k + ((int64_t)b * Tn * a.H + h) * D;
  const T* UT = (const T*)(a.ws + a.L.UT) + (size_t)bh * DV * Tp;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    dma_tile64<T>(kb, rs, t0, Tn, Ks, 2 * w + i, lane);
    dma_tile64<T>(UT + t0, Tp, 0, DV, UTs, 2 * w + i, lane);
  }
  const int tl = t0 + 32 * tb + cl;
  v8_t<T> kc[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk)
    kc[kk] = tl < Tn ? ld8<T>(kb + (int64_t)tl * rs + 16 * kk + 8 * hh) : zero8<T>();

  // the elementwise part's rows, loaded while the tiles land: thread
  // (tk, q) = (tid / 4, tid % 4) owns token t0 + tk, value columns and key
  // dims 16 q .. 16 q + 15, so four consecutive lanes cover a whole row
  const int tk = tid >> 2, q = tid & 3, tg = t0 + tk;
  const bool in = tg < Tn;
  const int64_t row = ((int64_t)b * Tn + (in ? tg : t0)) * a.H + h;
  float4 g4[4], e4[4];
  v4_t<T> v4[4], x4[4], y4[4], z4[4];
  const float bt = in ? a.beta[((int64_t)b * Tn + tg) * a.H + h] : 0.f;
  {
    const float* dbv = (const float*)(a.bws + a.BL.dbV) + row * DV + 16 * q;
    const float* ein = (const float*)(a.ws + a.L.Ein) + row * DV + 16 * q;
    const T* vr = (const T*)a.v + row * DV + 16 * q;
    const T* dkr = (const T*)(a.bws + a.BL.dkr) + row * D + 16 * q;
    const T* dke = (const T*)(a.bws + a.BL.dke) + row * D + 16 * q;
    const T* dqe = (const T*)(a.bws + a.BL.dqe) + (row - a.H) * D + 16 * q;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      g4[i] = in ? *reinterpret_cast<const float4*>(dbv + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
      e4[i] = in ? *reinterpret_cast<const float4*>(ein + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
      v4[i] = in ? ld4<T>(vr + 4 * i) : v4_t<T>{};
      x4[i] = in ? ld4<T>(dkr + 4 * i) : v4_t<T>{};
      y4[i] = in ? ld4<T>(dke + 4 * i) : v4_t<T>{};
      z4[i] = in && tg > 0 ? ld4<T>(dqe + 4 * i) : v4_t<T>{};
    }
  }
  vm_wait_barrier<0>();

  // A^T[s][t] / scale^2 for s in block ub, t in block tb, zero unless s < t
  f32x16 At{};
#pragma unroll
  for (int g = 0; g < M; ++g)
#pragma unroll
    for (int g2 = 0; g2 < M; ++g2) {
      f32x16 r{};
#pragma unroll
      for (int kk = 0; kk < KE; ++kk)
        r = mma(tile_ld8<T>(Ks, 32 * ub + cl, g2 * E + 16 * kk + 8 * hh), kc[g * KE + kk], r);
      At += r * r;
    }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int s_ = 32 * ub + 8 * (e >> 2) + 4 * hh + (e & 3), t_ = 32 * tb + cl;
    if (s_ >= t_) At[e] = 0.f;
  }
  f32x16 ec[2] = {f32x16{}, f32x16{}};
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const v8_t<T> bop = c_to_b<T>(At, ks);
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
      ec[jb] = mma(tile_ldp8<T>(UTs, 32 * jb + cl, 32 * ub, ks, hh), bop, ec[jb]);
  }
  // the s-block 0 waves write their part, then the s-block 1 waves add theirs
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    if (ub == pass) {
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float& d = Ecs[32 * tb + cl][32 * jb + 8 * (e >> 2) + 4 * hh + (e & 3)];
          d = pass == 0 ? ec[jb][e] : d + ec[jb][e];
        }
    }
    __syncthreads();
  }
  // dbeta over the row's value columns; dv; dk
  float part = 0.f;
  T* dvr = (T*)a.dv + row * DV + 16 * q;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float gv[4] = {g4[i].x, g4[i].y, g4[i].z, g4[i].w};
    const float ev[4] = {e4[i].x, e4[i].y, e4[i].z, e4[i].w};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float Et = ev[r] + a.scale2 * Ecs[tk][16 * q + 4 * i + r];
      part += ((float)v4[i][r] - Et) * gv[r];
    }
    if (in) st4<T>(dvr + 4 * i, to4<T>(bt * gv[0], bt * gv[1], bt * gv[2], bt * gv[3]));
  }
  part += __shfl_xor(part, 1);
  part += __shfl_xor(part, 2);
  if (in) {
    T* dko = (T*)a.dk + row * D + 16 * q;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      st4<T>(dko + 4 * i, to4<T>((float)x4[i][0] + (float)y4[i][0] + (float)z4[i][0],
                                 (float)x4[i][1] + (float)y4[i][1] + (float)z4[i][1],
                                 (float)x4[i][2] + (float)y4[i][2] + (float)z4[i][2],
                                 (float)x4[i][3] + (float)y4[i][3] + (float)z4[i][3]));
    if (q == 0) a.dbeta[((int64_t)b * Tn + tg) * a.H + h] = part;
  }
}

template <typename T, int D, int DV, int M>
hipError_t launch_dkata_bwd(const DKataBwdArgs& a, hipStream_t stream) {
  const int NC = (a.T + 63) / 64, BH = a.B * a.H;
  const int64_t n4 = (int64_t)a.B * a.T * a.H * DV / 4;
  const int blocks = (int)((n4 + 255) / 256 < 4096 ? (n4 + 255) / 256 : 4096);
  dkata_bwd_prep_kernel<T><<<dim3(blocks), dim3(256), 0, stream>>>(a, D, DV);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const float* ones = (const float*)(a.bws + a.BL.ones);
  // readout: KATA sum backward of (q, k, U), den := 1
  KataArgs r{};
  // (o: the normalised output when normalising, else none: delta = 0)
  r.q = a.q; r.k = a.k; r.v = a.ws + a.L.Ub; r.o = a.normalize ? a.bws + a.BL.O16 : nullptr;
  r.den = const_cast<float*>(ones);
  r.dout = a.bws + a.BL.dOp; r.dq = a.dq; r.dk = a.bws + a.BL.dkr; r.dv = a.bws + a.BL.dU;
  r.delta = (float*)(a.bws + a.BL.kws);
  r.B = a.B; r.T = a.T; r.HQ = a.H; r.H = a.H; r.DK = D; r.DV = DV; r.M = M; r.scale = a.scale;
  e = launch_kata_bwd<T, D, DV, M, true, false>(r, KATA_BWD_DQ | KATA_BWD_DKDV, stream);
  if (e != hipSuccess) return e;
  // chunk-sequential only inside super-chunks, last one first; the later
  // super-chunks' part of R in parallel before each
  for (int cb = (NC - 1) / kDkataSB * kDkataSB; cb >= 0; cb -= kDkataSB) {
    const int ce = cb + kDkataSB < NC ? cb + kDkataSB : NC;
    if (ce < NC) {
      dkata_ext_kernel<T, D, DV, M><<<dim3(BH * ((ce - cb + 1) / 2)), dim3(256), 0, stream>>>(
          (const T*)a.k, (const T*)(a.bws + a.BL.XT), (float*)(a.bws + a.BL.dbV), a.H, a.T, a.scale2,
          cb, ce - cb, ce, NC - ce, BH);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    dkata_dbV_kernel<T, D, DV, M><<<dim3(BH), dim3(256), 0, stream>>>(a, cb, ce);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  // erase: KATA sum backward of (k shifted one token, k, U) with the shifted
  // dO := -X, o := 0 (none), den := 1
  KataArgs x{};
  x.q = a.bws + a.BL.Ksh; x.k = a.k; x.v = a.ws + a.L.Ub; x.o = nullptr; x.den = const_cast<float*>(ones);
  x.dout = a.bws + a.BL.Xn; x.dq = a.bws + a.BL.dqe; x.dk = a.bws + a.BL.dke; x.dv = a.bws + a.BL.dve;
  x.delta = (float*)(a.bws + a.BL.kws);
  x.B = a.B; x.T = a.T; x.HQ = a.H; x.H = a.H; x.DK = D; x.DV = DV; x.M = M; x.scale = a.scale;
  e = launch_kata_bwd<T, D, DV, M, true, false>(x, KATA_BWD_DQ | KATA_BWD_DKDV, stream);
  if (e != hipSuccess) return e;
  dkata_bwd_fix_kernel<T, D, DV, M><<<dim3(BH * NC), dim3(256), 0, stream>>>(a);
  return hipGetLastError();
}

#define LINATT_DKATA_INST(T, D, DV, M)                                              \
  template hipError_t launch_dkata_fwd<T, D, DV, M>(const DKataArgs&, hipStream_t); \
  template hipError_t launch_dkata_bwd<T, D, DV, M>(const DKataBwdArgs&, hipStream_t);
LINATT_DKATA_SHAPES(LINATT_DKATA_INST)

}  // namespace linatt
