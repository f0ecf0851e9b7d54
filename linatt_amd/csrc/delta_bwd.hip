// Chunked (gated) delta rule, backward, for gfx950.
//
// Replaces the backward of fla.ops.delta_rule.chunk_delta_rule and
// fla.ops.gated_delta_rule.chunk_gated_delta_rule (third-party
// flash-linear-attention==0.5.0, scripts/setup.sh:27 of the reference).
// Reverse-mode of the chunk form computed by delta_fwd.hip, per chunk with
// S the state entering it, dS' the gradient of the state leaving it:
//
//   dVn = Aqk^T dO + diag(e^(gamma-G)) K dS'                     (kernel 1)
//   dS  = e^gamma dS' + (scale e^G Q)^T dO - W^T dVn              (kernel 1)
//   dQ  = scale e^G dO S^T + Mq K,  Mq = scale (dO Vn^T) o e^(G_i-G_j) [j<=i]
//   dK  = diag(e^(gamma-G)) Vn dS'^T + Mq^T Q + ...               (kernel 2)
//   dW  = -dVn S^T                                                (kernel 2)
//   dTm = dVn (diag(beta) V)^T + dW (diag(beta e^G) K)^T,  dA = -Tm^T dTm Tm^T
//   dV  = diag(beta) Tm^T dVn,  dK += diag(beta e^G) Tm^T dW + At K + At^T K
//   dbeta, dG from the same terms; dg = reverse cumsum of dG in the chunk  (kernel 3)
//
// Kernel 1 (delta_state_bwd) walks the chunks backwards, one workgroup per
// (b, h) with dS in MFMA accumulators.  Kernels 2 and 3 are parallel over
// (b, h, chunk).
#include "common.h"
#include "delta_kernels.h"

namespace linatt {

// ---------------------------------------------------------------------------
// Kernel 1: reverse state pass.  One workgroup per (b, h), one wave per 32
// value columns, dS in DK/32 accumulator tiles (lane column v).  Per chunk,
// with dS' the gradient of the state leaving it:
//   dVn = Aqk^T dO + diag(e^(gamma-G)) K dS'
//   dS  = e^gamma dS' + (scale e^G Q)^T dO - W^T dVn
// K, W^T, Qg = scale e^G Q, Aqk, dO and G of a chunk are shared by the
// waves of the head: they reach LDS by direct global->LDS copies (swizzled
// 64 x 64 tiles, see tile_slot) into two slots, the earlier chunk's copies
// in flight while the current one computes; Qg^T and Aqk^T operands come
// from transposing reads.  dh^T and dv_new^T leave
// through LDS staging in the wave's own columns of the dO tiles.
// ---------------------------------------------------------------------------
template <typename T, int DK, int DV, bool GATED>
__global__ __launch_bounds__(64 * (DV / 32)) void delta_state_bwd_kernel(DeltaArgs a, DeltaLayout L) {
  constexpr int NDT = DK / 32, NW = DV / 32;
  constexpr int KT = DK / 64, VT = DV / 64;      // 64 x 64 tiles per row block
  constexpr int TE = 64 * 64;                     // elements per tile
  constexpr int OPW = 8 / NW;                     // 1 KiB copies per wave per tile
  constexpr int NTILE = 3 * KT + 1 + VT;          // K, W^T, Qg, Aqk, dO
  constexpr int SLOT = NTILE * TE + 64 * 4 / (int)sizeof(T);  // + G of the chunk (f32)
  static_assert(OPW * NW == 8, "tile split");
  __shared__ __attribute__((aligned(16))) T Sh[2 * SLOT];

  const int lane = threadIdx.x & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int Tn = a.T, H = a.H, NT = a.NT;
  const int bh = blockIdx.x;
  const int b = bh / H, h = bh % H;
  const int v = 32 * w + cl;
  const size_t Tp = (size_t)NT * kChunk;

  const T* kb = (const T*)a.k + ((size_t)b * Tn * H + h) * DK;
  const T* dob = (const T*)a.dout + ((size_t)b * Tn * H + h) * DV;
  const float* Gc = reinterpret_cast<const float*>(a.ctx + L.Gc) + (size_t)bh * Tp;

  auto kt = [&](T* sl, int i) { return sl + i * TE; };                 // K tile i (key dims 64 i..)
  auto wt = [&](T* sl, int i) { return sl + (KT + i) * TE; };          // W^T rows 64 i..
  auto qt = [&](T* sl, int i) { return sl + (2 * KT + i) * TE; };      // Qg key dims 64 i..
  auto at = [&](T* sl) { return sl + 3 * KT * TE; };                   // Aqk
  auto ot = [&](T* sl, int i) { return sl + (3 * KT + 1 + i) * TE; };  // dO columns 64 i..
  auto gs = [&](T* sl) { return reinterpret_cast<float*>(sl + NTILE * TE); };

  auto issue = [&](int c) __attribute__((always_inline)) {
    T* sl = Sh + (c & 1) * SLOT;
    const int t0 = c * kChunk;
    const size_t ci = (size_t)bh * NT + c;
    const T* wtg = (const T*)(a.ctx + L.WT) + ci * DK * 64;
    const T* qgg = (const T*)(a.ctx + L.Qg) + ci * 64 * DK;
    const T* atg = (const T*)(a.ctx + L.Aqk) + ci * 4096;
#pragma unroll
    for (int o = 0; o < OPW; ++o) {
      const int op = OPW * w + o;
#pragma unroll
      for (int i = 0; i < KT; ++i) {
        dma_tile64<T>(kb + 64 * i, (int64_t)H * DK, t0, Tn, kt(sl, i), op, lane);
        dma_tile64<T>(wtg + (size_t)64 * i * 64, 64, 0, 64, wt(sl, i), op, lane);
        dma_tile64<T>(qgg + 64 * i, DK, 0, 64, qt(sl, i), op, lane);
      }
      dma_tile64<T>(atg, 64, 0, 64, at(sl), op, lane);
#pragma unroll
      for (int i = 0; i < VT; ++i) dma_tile64<T>(dob + 64 * i, (int64_t)H * DV, t0, Tn, ot(sl, i), op, lane);
    }
    if (GATED && w == 0 && lane < 16) dma16(Gc + t0 + 4 * lane, gs(sl));
  };

  f32x16 dS[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int d = 32 * dt + 8 * (e >> 2) + 4 * hh + (e & 3);
      dS[dt][e] = a.dht ? a.dht[((size_t)bh * DK + d) * DV + v] : 0.f;
    }

  vm_drain();  // dh_T is in registers
  issue(NT - 1);
#pragma unroll 1
  for (int c = NT - 1; c >= 0; --c) {
    const int t0 = c * kChunk;
    const size_t ci = (size_t)bh * NT + c;
    // chunk c landed for every wave; every wave is done with chunk c + 1
    vm_wait_barrier<0>();
    if (c > 0) issue(c - 1);
    T* sl = Sh + (c & 1) * SLOT;
    const T* Os = ot(sl, w / 2);  // this wave's 64-column dO tile
    const int oc0 = 32 * (w & 1);

    // the LDS operands of dVn, Z and K dS' into registers first: the one
    // wave per SIMD then never waits on a read inside the MFMA chains
    v8_t<T> oop[2][2], aop[2][2][2], qop[NDT][2][2], kop[NDT][2][2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        oop[s2][j] = tile_tr8<T>(Os, 32 * s2, oc0, j, lane);
#pragma unroll
        for (int jt = 0; jt < 2; ++jt) aop[jt][s2][j] = tile_tr8<T>(at(sl), 32 * s2, 32 * jt, j, lane);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) qop[dt][s2][j] = tile_tr8<T>(qt(sl, dt / 2), 32 * s2, 32 * (dt & 1), j, lane);
      }
#pragma unroll
    for (int db = 0; db < NDT; ++db)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int jt = 0; jt < 2; ++jt)
          kop[db][j][jt] = tile_ldp8<T>(kt(sl, db / 2), 32 * jt + cl, 32 * (db & 1), j, hh);
    __builtin_amdgcn_sched_barrier(0);

    // dVn = Aqk^T dO (rows j = 32 jt + ..., lane column v); Z = Qg^T dO
    f32x16 dVn[2], Z[NDT];
#pragma unroll
    for (int jt = 0; jt < 2; ++jt) {
      dVn[jt] = f32x16{};
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int j = 0; j < 2; ++j) dVn[jt] = mma(aop[jt][s2][j], oop[s2][j], dVn[jt]);
    }
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      Z[dt] = f32x16{};
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int j = 0; j < 2; ++j) Z[dt] = mma(qop[dt][s2][j], oop[s2][j], Z[dt]);
    }

    // + diag(e^(gamma - G)) K dS'  (K rows 32 jt + cl of the chunk)
    const float gam = GATED ? gs(sl)[63] : 0.f;
    if constexpr (!GATED) {
#pragma unroll
      for (int db = 0; db < NDT; ++db)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const v8_t<T> ys = c_to_b<T>(dS[db], j);
#pragma unroll
          for (int jt = 0; jt < 2; ++jt) dVn[jt] = mma(kop[db][j][jt], ys, dVn[jt]);
        }
    } else {
      f32x16 Pk[2];
      Pk[0] = Pk[1] = f32x16{};
#pragma unroll
      for (int db = 0; db < NDT; ++db)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const v8_t<T> ys = c_to_b<T>(dS[db], j);
#pragma unroll
          for (int jt = 0; jt < 2; ++jt) Pk[jt] = mma(kop[db][j][jt], ys, Pk[jt]);
        }
#pragma unroll
      for (int jt = 0; jt < 2; ++jt)
#pragma unroll
        for (int I = 0; I < 4; ++I) {
          const f32x4 g4 = *reinterpret_cast<const f32x4*>(gs(sl) + 32 * jt + 8 * I + 4 * hh);
#pragma unroll
          for (int r = 0; r < 4; ++r) dVn[jt][4 * I + r] += __expf(gam - g4[r]) * Pk[jt][4 * I + r];
        }
    }
    // W^T operands of the dS update, read while the MFMAs above run
    v8_t<T> wop[NDT][2][2];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int it = 0; it < 2; ++it)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          wop[dt][it][j] = tile_ld8<T>(wt(sl, dt / 2), 32 * (dt & 1) + cl, 32 * it + 16 * j + 8 * hh);
    if (t0 + 63 >= Tn) {  // rows past T: K repeats its last row there
#pragma unroll
      for (int jt = 0; jt < 2; ++jt)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (t0 + 32 * jt + 8 * (e >> 2) + 4 * hh + (e & 3) >= Tn) dVn[jt][e] = 0.f;
    }

    // dh^T (gradient of the state leaving the chunk, [v][d]) and dv_new^T out
    // through this wave's dO columns, which it alone reads and has consumed
    {
      char* ob = reinterpret_cast<char*>(const_cast<T*>(Os));
      auto slot = [&](int s) {
        const int tr = s >> 2, q = s & 3;
        return reinterpret_cast<u32x4*>(ob + tr * 128 + (tile_slot(tr, 4 * (w & 1) + q) << 4));
      };
      T* drows = (T*)(a.ws + L.dhT) + (ci * DV + 32 * w) * DK;
#pragma unroll
      for (int blk = 0; blk < NDT / 2; ++blk)
        store_rows_via<T>(dS[2 * blk], dS[2 * blk + 1], slot, drows + 64 * blk, DK, lane);
      store_rows_via<T>(dVn[0], dVn[1], slot, (T*)(a.ws + L.dVnT) + (ci * DV + 32 * w) * 64, 64, lane);
    }

    // dS <- e^gamma dS' + Z - W^T dVn
    const float eg = GATED ? __expf(gam) : 1.f;
    v8_t<T> nb[2][2];
#pragma unroll
    for (int it = 0; it < 2; ++it)
#pragma unroll
      for (int j = 0; j < 2; ++j) nb[it][j] = c_to_b<T>(-dVn[it], j);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      f32x16 acc = GATED ? dS[dt] * eg + Z[dt] : dS[dt] + Z[dt];
#pragma unroll
      for (int it = 0; it < 2; ++it)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc = mma(wop[dt][it][j], nb[it][j], acc);
      dS[dt] = acc;
    }
  }

  if (a.dh0) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int d = 32 * dt + 8 * (e >> 2) + 4 * hh + (e & 3);
        a.dh0[((size_t)bh * DK + d) * DV + v] = dS[dt][e];
      }
  }
}

// ---------------------------------------------------------------------------
// Kernel 2: dq, dW, the output/state part of dk and of dG.
// Wave w: row block ib = w & 1 (lane column = chunk row 32 ib + cl), key
// dims half dhalf = w >> 1.  The transposed per-chunk tiles (h^T, dh^T,
// v_new^T, dv_new^T) are turned back into value-contiguous rows through LDS
// in three phases: (A) S and dVn, (B) dS' and Vn, (C) K^T and Q^T.
// ---------------------------------------------------------------------------
template <typename T, int DK, int DV, bool GATED>
__global__ __launch_bounds__(256, 2) void delta_bwd_chunk_kernel(DeltaArgs a, DeltaLayout L) {
  constexpr int PX = 64 + 8;   // [d][row] tiles
  constexpr int PV = DV + 8;   // [row][v] tiles
  constexpr int NDW = DK / 64;  // key-dim tiles per wave
  constexpr int NS = DV / 16;
  constexpr int RA = DK * PV, RB = 64 * PV, RC = 2 * DK * PX;
  constexpr int RTOT = (RA + RB > RC) ? RA + RB : RC;
  __shared__ __attribute__((aligned(16))) T sm[RTOT];
  __shared__ float Gs[64];
  __shared__ float red_gi[2][64], red_kd[2][64], red_rc[64];
  __shared__ float red_s[4];
  T* Sx = sm;             // phase A: S [d][v];  phase B: dS' [d][v]
  T* Rx = sm + RA;        // phase A: dVn [i][v]; phase B: Vn [j][v]
  T* KT = sm;             // phase C: K^T [d][j]
  T* QT = sm + DK * PX;   // phase C: Q^T [d][i]

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int ib = w & 1, dhalf = w >> 1;
  const int Tn = a.T, H = a.H, NT = a.NT;
  const int c = blockIdx.x % NT, bh = blockIdx.x / NT;
  const int b = bh / H, h = bh % H;
  const int t0 = c * kChunk;
  const size_t Tp = (size_t)NT * kChunk;
  const size_t ci = (size_t)bh * NT + c;

  const T* qb = (const T*)a.q + ((size_t)b * Tn * H + h) * DK;
  const T* kb = (const T*)a.k + ((size_t)b * Tn * H + h) * DK;
  const int64_t qks = (int64_t)H * DK;
  const T* dob = (const T*)a.dout + ((size_t)b * Tn * H + h) * DV;
  const int64_t os = (int64_t)H * DV;
  const float* Gc = reinterpret_cast<const float*>(a.ctx + L.Gc) + (size_t)bh * Tp;
  const T* hg = (const T*)(a.ctx + L.hT) + ci * DV * DK;
  const T* dhg = (const T*)(a.ws + L.dhT) + ci * DV * DK;
  const T* vng = (const T*)(a.ctx + L.VnT) + ci * DV * 64;
  const T* dvng = (const T*)(a.ws + L.dVnT) + ci * DV * 64;
  const T* aq = (const T*)(a.ctx + L.Aqk) + ci * 4096;

  // phase A tiles
#pragma unroll
  for (int r0 = 0; r0 < DV; r0 += 64) {
    load_tile64x<T, T, DK, 1, PV, false, true>(hg + (size_t)r0 * DK, 0, 64, DK, nullptr, Sx + r0, tid, nullptr);
    load_tile64x<T, T, 64, 1, PV, false, true>(dvng + (size_t)r0 * 64, 0, 64, 64, nullptr, Rx + r0, tid, nullptr);
  }
  if (tid < 64) Gs[tid] = GATED ? Gc[t0 + tid] : 0.f;

  // <S, dS'> over the chunk's state pair (for d gamma); both stored [v][d].
  float sdot = 0.f;
  for (int idx = 8 * tid; idx < DK * DV; idx += 8 * 256) {
    const v8_t<T> x = ld8<T>(hg + idx), y = ld8<T>(dhg + idx);
#pragma unroll
    for (int j = 0; j < 8; ++j) sdot += (float)x[j] * (float)y[j];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sdot += __shfl_xor(sdot, off);
  if (lane == 0) red_s[w] = sdot;
  __syncthreads();

  const int i = 32 * ib + cl;  // this lane's chunk row (as query i and as key j)
  const int ti = t0 + i;
  const bool valid = ti < Tn;
  const float Gi = Gs[i];
  v8_t<T> ydo[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) ydo[s] = valid ? ld8<T>(dob + (int64_t)ti * os + 16 * s + 8 * hh) : zero8<T>();

  // (A) dQ_inter = scale e^G dO S^T, dW = -dVn S^T   (lane column i)
  float gi_part = 0.f, kd_part = 0.f;
  const float eG = GATED ? __expf(Gi) : 1.f;
  const float eGam = GATED ? __expf(Gs[63] - Gi) : 1.f;
  T* dWg = (T*)(a.ws + L.dW) + ((size_t)bh * Tp + t0 + i) * DK;
  float* dKg = reinterpret_cast<float*>(a.ws + L.dKp) + ((size_t)bh * Tp + t0 + i) * DK;
  T* dqg = (T*)a.dq + (((size_t)b * Tn + ti) * H + h) * DK;
  f32x16 dq[NDW], dks[NDW];
#pragma unroll
  for (int m = 0; m < NDW; ++m) {
    const int dt = dhalf * NDW + m;
    f32x16 acc{}, dw{};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const v8_t<T> xs = ld8<T>(Sx + (32 * dt + cl) * PV + 16 * s + 8 * hh);
      acc = mma(xs, ydo[s], acc);
      dw = mma(xs, ld8<T>(Rx + i * PV + 16 * s + 8 * hh), dw);
    }
    acc *= a.scale * eG;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const int d = 32 * dt + 8 * I + 4 * hh;
      const v4_t<T> q4 = valid ? ld4<T>(qb + (int64_t)ti * qks + d) : v4_t<T>{};
#pragma unroll
      for (int r = 0; r < 4; ++r) gi_part += (float)q4[r] * acc[4 * I + r];
      st4<T>(dWg + d, to4<T>(-dw[4 * I], -dw[4 * I + 1], -dw[4 * I + 2], -dw[4 * I + 3]));
    }
    dq[m] = acc;
  }
  __syncthreads();

  // phase B tiles
#pragma unroll
  for (int r0 = 0; r0 < DV; r0 += 64) {
    load_tile64x<T, T, DK, 1, PV, false, true>(dhg + (size_t)r0 * DK, 0, 64, DK, nullptr, Sx + r0, tid, nullptr);
    load_tile64x<T, T, 64, 1, PV, false, true>(vng + (size_t)r0 * 64, 0, 64, 64, nullptr, Rx + r0, tid, nullptr);
  }
  __syncthreads();

  // (B) dK_state = e^(gamma-G_j) Vn dS'^T   (lane column j = i)
#pragma unroll
  for (int m = 0; m < NDW; ++m) {
    const int dt = dhalf * NDW + m;
    f32x16 acc{};
#pragma unroll
    for (int s = 0; s < NS; ++s)
      acc = mma(ld8<T>(Sx + (32 * dt + cl) * PV + 16 * s + 8 * hh), ld8<T>(Rx + i * PV + 16 * s + 8 * hh), acc);
    acc *= eGam;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const int d = 32 * dt + 8 * I + 4 * hh;
      const v4_t<T> k4 = valid ? ld4<T>(kb + (int64_t)ti * qks + d) : v4_t<T>{};
#pragma unroll
      for (int r = 0; r < 4; ++r) kd_part += (float)k4[r] * acc[4 * I + r];
    }
    dks[m] = acc;
  }

  // Mq (lane column i, rows j) and its transpose MqT (lane column j, rows i).
  f32x16 Mq[2], MqT[2];
  float rowsum = 0.f, colsum = 0.f;
#pragma unroll
  for (int jt = 0; jt < 2; ++jt) {
    f32x16 dm{}, dmt{};
    const int rr0 = 32 * jt + cl;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      dm = mma(ld8<T>(Rx + rr0 * PV + 16 * s + 8 * hh), ydo[s], dm);
      dmt = mma(t0 + rr0 < Tn ? ld8<T>(dob + (int64_t)(t0 + rr0) * os + 16 * s + 8 * hh) : zero8<T>(),
                ld8<T>(Rx + i * PV + 16 * s + 8 * hh), dmt);
    }
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const int r0 = 32 * jt + 8 * I + 4 * hh;
      const v4_t<T> aq4 = ld4<T>(aq + i * 64 + r0);  // Aqk[i][r0 + r]
      v4_t<T> aqt4;                                  // Aqk[r0 + r][i]
#pragma unroll
      for (int r = 0; r < 4; ++r) aqt4[r] = aq[(r0 + r) * 64 + i];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rr = r0 + r;
        const float x = dm[4 * I + r], y = dmt[4 * I + r];
        rowsum += x * (float)aq4[r];
        colsum += y * (float)aqt4[r];
        float fm = a.scale, ft = a.scale;
        if constexpr (GATED) {
          fm *= __expf(Gi - Gs[rr]);
          ft *= __expf(Gs[rr] - Gi);
        }
        Mq[jt][4 * I + r] = rr <= i ? x * fm : 0.f;
        MqT[jt][4 * I + r] = rr >= i ? y * ft : 0.f;
      }
    }
  }
  rowsum += __shfl_xor(rowsum, 32);
  colsum += __shfl_xor(colsum, 32);
  __syncthreads();

  // phase C tiles: K^T, Q^T
  load_tile64x<T, T, DK, 1, PX, false, true>(kb, t0, Tn, qks, nullptr, KT, tid, nullptr);
  load_tile64x<T, T, DK, 1, PX, false, true>(qb, t0, Tn, qks, nullptr, QT, tid, nullptr);
  __syncthreads();

  // (C) intra terms: dQ += Mq K, dK += Mq^T Q
#pragma unroll
  for (int m = 0; m < NDW; ++m) {
    const int dt = dhalf * NDW + m;
#pragma unroll
    for (int jt = 0; jt < 2; ++jt)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        dq[m] = mma(ld_tr_op<T>(KT + (32 * dt + cl) * PX + 32 * jt, j, hh), c_to_b<T>(Mq[jt], j), dq[m]);
        dks[m] = mma(ld_tr_op<T>(QT + (32 * dt + cl) * PX + 32 * jt, j, hh), c_to_b<T>(MqT[jt], j), dks[m]);
      }
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const int d = 32 * dt + 8 * I + 4 * hh;
      if (valid)
        st4<T>(dqg + d, to4<T>(dq[m][4 * I], dq[m][4 * I + 1], dq[m][4 * I + 2], dq[m][4 * I + 3]));
      *reinterpret_cast<float4*>(dKg + d) =
          make_float4(dks[m][4 * I], dks[m][4 * I + 1], dks[m][4 * I + 2], dks[m][4 * I + 3]);
    }
  }
  gi_part += __shfl_xor(gi_part, 32);
  kd_part += __shfl_xor(kd_part, 32);
  if (hh == 0) {
    red_gi[dhalf][i] = gi_part;
    red_kd[dhalf][i] = kd_part;
    if (dhalf == 0) red_rc[i] = rowsum - colsum;
  }
  __syncthreads();
  if (tid < 64) {
    const float kd = red_kd[0][tid] + red_kd[1][tid];
    float dG = red_gi[0][tid] + red_gi[1][tid] - kd + red_rc[tid];
    // d gamma = sum_j k_j . dKs_j + e^gamma <S, dS'>, added at row 63
    float kds = kd;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) kds += __shfl_xor(kds, off);
    if (tid == 63) {
      const float st = red_s[0] + red_s[1] + red_s[2] + red_s[3];
      dG += kds + (GATED ? __expf(Gs[63]) : 1.f) * st;
    }
    reinterpret_cast<float*>(a.ws + L.dGp)[(size_t)bh * Tp + t0 + tid] = dG;
  }
}

// ---------------------------------------------------------------------------
// Kernel 3: backward through W = Tm diag(beta e^G) K, U = Tm diag(beta) V,
// Tm = (I + A)^-1; final dk, dv, dbeta, dg.  One workgroup of four waves
// per chunk; Tm, dU^T, V, K and dW reach LDS by one up-front copy.
//   dv  = diag(beta) Tm^T dU                       (wave: rows j, 64 v)
//   dkW = diag(beta e^G) Tm^T dW                   (wave: rows j, 64 d)
//   dTm = dU (diag(beta) V)^T + dW (diag(beta e^G) K)^T   (one 32 x 32 block per wave)
//   M^T = dTm^T Tm,  dA^T = -Tm M^T                (bf16 tiles through LDS)
//   P[a][l] = dA[a][l] beta_a e^(G_a - G_l) (l < a),  dk = dKp + dkW + (P + P^T) K
// dbeta and dG gather the row / column sums of the same terms; dg is the
// reverse cumulative sum of dG within the chunk.
// ---------------------------------------------------------------------------
template <typename T, int DK, int DV, bool GATED>
__global__ __launch_bounds__(256, 2) void delta_wy_bwd_kernel(DeltaArgs a, DeltaLayout L) {
  constexpr int KT = DK / 64, VT = DV / 64;
  constexpr int TE = 64 * 64;
  constexpr int SE = 8192 / (int)sizeof(T) * 2;            // 16 KiB of T
  constexpr int WE = KT * TE > SE ? KT * TE : SE;          // dW tiles, then store staging
  constexpr int XE = 2 * VT * TE > SE * 2 ? 2 * VT * TE : SE * 2;
  static_assert(DK % 64 == 0 && DV % 64 == 0 && DK <= 128 && DV <= 128, "64 or 128 wide");
  __shared__ __attribute__((aligned(16))) T Tmt[TE];      // Tm [i][j]
  __shared__ __attribute__((aligned(16))) T Kt[KT * TE];  // K [j][d], tile kt: d in 64 kt..
  __shared__ __attribute__((aligned(16))) T dWt[WE];      // dW [i][d]; phase 5: store staging
  // dU^T [v][i] (tile vt: v in 64 vt..) and V [j][v]; after phase 1:
  // dTm^T then P [a][l] (0 .. TE), M^T as [a][j] (TE .. 2 TE), Q^T fp32 [l][a] (2 TE ..)
  __shared__ __attribute__((aligned(16))) T Xr[XE];
  __shared__ float Bs[64], Gs[64];
  __shared__ float red_b[4][64], red_g[4][64];
  T* dUt = Xr;
  T* Vt = Xr + VT * TE;
  T* dTT = Xr;
  T* Pn = Xr;
  T* MTt = Xr + TE;
  float* Qb = reinterpret_cast<float*>(Xr + 2 * TE);

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int Tn = a.T, H = a.H, NT = a.NT;
  const int c = blockIdx.x % NT, bh = blockIdx.x / NT;
  const int b = bh / H, h = bh % H;
  const int t0 = c * kChunk;
  const size_t Tp = (size_t)NT * kChunk;
  const size_t ci = (size_t)bh * NT + c;
  const int lb = w & 1, hf = w >> 1;  // lane block (output rows j / a), column half
  const int ja = 32 * lb + cl;        // this lane's output row within the chunk
  const int nvalid = Tn - (t0 + 32 * lb);

  const T* kb = (const T*)a.k + ((size_t)b * Tn * H + h) * DK;
  const T* vb = (const T*)a.v + ((size_t)b * Tn * H + h) * DV;
  const int64_t ks = (int64_t)H * DK, vs = (int64_t)H * DV;

  // 0. copies; beta and G (wave 3); dKp of this wave's dk blocks
#pragma unroll
  for (int o = 0; o < 2; ++o) {
    const int op = 2 * w + o;
    dma_tile64<T>((const T*)(a.ctx + L.Tm) + ci * 4096, 64, 0, 64, Tmt, op, lane);
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) {
      dma_tile64<T>((const T*)(a.ws + L.dVnT) + (ci * DV + 64 * vt) * 64, 64, 0, 64, dUt + vt * TE, op, lane);
      dma_tile64<T>(vb + 64 * vt, vs, t0, Tn, Vt + vt * TE, op, lane);
    }
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      dma_tile64<T>(kb + 64 * kt, ks, t0, Tn, Kt + kt * TE, op, lane);
      dma_tile64<T>((const T*)(a.ws + L.dW) + ((size_t)bh * Tp + t0) * DK + 64 * kt, DK, 0, 64, dWt + kt * TE, op,
                    lane);
    }
  }
  if (w == 3) {
    const int t = t0 + lane;
    Bs[lane] = t < Tn ? a.beta[((size_t)b * Tn + t) * H + h] : 0.f;
    Gs[lane] = GATED ? reinterpret_cast<const float*>(a.ctx + L.Gc)[(size_t)bh * Tp + t0 + lane] : 0.f;
  }
  const bool has_dk = 2 * hf < DK / 32, has_dv = 2 * hf < DV / 32;
  f32x16 dk[2];
  if (has_dk) {
    const float* p = reinterpret_cast<const float*>(a.ws + L.dKp) + ((size_t)bh * Tp + t0 + ja) * DK + 64 * hf;
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        const f32x4 v4 = *reinterpret_cast<const f32x4*>(p + 32 * m + 8 * I + 4 * hh);
#pragma unroll
        for (int r = 0; r < 4; ++r) dk[m][4 * I + r] = v4[r];
      }
  }
  vm_wait_barrier<0>();

  const float Bj = Bs[ja], Gj = Gs[ja];
  const float eGj = GATED ? __expf(Gj) : 1.f;
  float db_part = 0.f, dg_part = 0.f, rq_part = 0.f;

  // 1a. dv[j][v] = beta_j (Tm^T dU)[j][v] as D[v][j] = sum_i dU^T[v][i] Tm[i][j]
  f32x16 dv[2];
  if (has_dv) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int vb2 = 2 * hf + m;
      const T* du = dUt + (vb2 / 2) * TE;
      dv[m] = f32x16{};
#pragma unroll
      for (int ib = 0; ib < 2; ++ib)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          dv[m] = mma(tile_ldp8<T>(du, 32 * (vb2 & 1) + cl, 32 * ib, jj, hh),
                      tile_tr8<T>(Tmt, 32 * ib, 32 * lb, jj, lane), dv[m]);
      // dbeta_j += v_j . (Tm^T dU)_j
      const char* vt = reinterpret_cast<const char*>(Vt + (vb2 / 2) * TE);
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        const v4_t<T> v4 = *reinterpret_cast<const v4_t<T>*>(vt + tile_off(ja, 32 * (vb2 & 1) + 8 * I + 4 * hh));
#pragma unroll
        for (int r = 0; r < 4; ++r) db_part += (float)v4[r] * dv[m][4 * I + r];
      }
      dv[m] *= Bj;
    }
  }
  // 1b. dkW[j][d] = beta_j e^G_j (Tm^T dW)[j][d] as D[d][j] = sum_i dW^T[d][i] Tm[i][j]
  if (has_dk) {
    float kdot = 0.f;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int db2 = 2 * hf + m;
      const T* dwt = dWt + (db2 / 2) * TE;
      f32x16 x{};
#pragma unroll
      for (int ib = 0; ib < 2; ++ib)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          x = mma(tile_tr8<T>(dwt, 32 * ib, 32 * (db2 & 1), jj, lane), tile_tr8<T>(Tmt, 32 * ib, 32 * lb, jj, lane), x);
      const char* kt = reinterpret_cast<const char*>(Kt + (db2 / 2) * TE);
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        const v4_t<T> k4 = *reinterpret_cast<const v4_t<T>*>(kt + tile_off(ja, 32 * (db2 & 1) + 8 * I + 4 * hh));
#pragma unroll
        for (int r = 0; r < 4; ++r) kdot += (float)k4[r] * x[4 * I + r];
      }
      dk[m] += x * (Bj * eGj);
    }
    db_part += eGj * kdot;
    dg_part += Bj * eGj * kdot;
  }
  // 1c. dTm block (rows i = 32 hf + .., lane column j = 32 lb + cl):
  //     beta_j (dU_i . v_j) + beta_j e^G_j (dW_i . k_j)
  f32x16 dtm{};
  {
    f32x16 d2{};
#pragma unroll
    for (int vt = 0; vt < VT; ++vt)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          dtm = mma(tile_tr8<T>(dUt + vt * TE, 32 * s2, 32 * hf, jj, lane),
                    tile_ldp8<T>(Vt + vt * TE, ja, 32 * s2, jj, hh), dtm);
#pragma unroll
    for (int kk = 0; kk < DK / 16; ++kk)
      d2 = mma(tile_ld8<T>(dWt + (kk / 4) * TE, 32 * hf + cl, 16 * (kk % 4) + 8 * hh),
               tile_ld8<T>(Kt + (kk / 4) * TE, ja, 16 * (kk % 4) + 8 * hh), d2);
    dtm = (dtm + d2 * eGj) * Bj;
  }
  // KK block (rows l = 32 hf + .., lane column a = ja) of the Gram matrix;
  // the block above the diagonal (hf > lb) is not needed
  const bool lower = hf <= lb;
  f32x16 kk{};
  if (lower) {
#pragma unroll
    for (int q = 0; q < DK / 16; ++q)
      kk = mma(tile_ld8<T>(Kt + (q / 4) * TE, 32 * hf + cl, 16 * (q % 4) + 8 * hh),
               tile_ld8<T>(Kt + (q / 4) * TE, ja, 16 * (q % 4) + 8 * hh), kk);
  }
  __syncthreads();  // dU^T and V no longer read

  // 2. dTm^T as a [j][i] tile (row j = this lane, columns i of block hf)
  {
    char* t = reinterpret_cast<char*>(dTT);
#pragma unroll
    for (int I = 0; I < 4; ++I)
      *reinterpret_cast<v4_t<T>*>(t + tile_off(ja, 32 * hf + 8 * I + 4 * hh)) =
          to4<T>(dtm[4 * I], dtm[4 * I + 1], dtm[4 * I + 2], dtm[4 * I + 3]);
  }
  __syncthreads();

  // 3. M^T[j][a] = sum_i dTm^T[j][i] Tm[i][a]: block (rows j = 32 hf + .., lane
  //    column a = ja), stored as a [a][j] tile
  {
    f32x16 x{};
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        x = mma(tile_ldp8<T>(dTT, 32 * hf + cl, 32 * ib, jj, hh), tile_tr8<T>(Tmt, 32 * ib, 32 * lb, jj, lane), x);
    char* t = reinterpret_cast<char*>(MTt);
#pragma unroll
    for (int I = 0; I < 4; ++I)
      *reinterpret_cast<v4_t<T>*>(t + tile_off(ja, 32 * hf + 8 * I + 4 * hh)) =
          to4<T>(x[4 * I], x[4 * I + 1], x[4 * I + 2], x[4 * I + 3]);
  }
  __syncthreads();

  // 4. dA^T[l][a] = -sum_j Tm[l][j] M^T[j][a] (rows l = 32 hf + .., lane a = ja);
  //    P[a][l] = dA[a][l] beta_a e^(G_a - G_l) and Q = P o KK for l < a.
  //    P goes to a [a][l] tile over dTm^T, Q^T to fp32 [l][a].
  {
    f32x16 x{};
    if (lower) {
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          x = mma(tile_ldp8<T>(Tmt, 32 * hf + cl, 32 * jb, jj, hh), tile_ldp8<T>(MTt, ja, 32 * jb, jj, hh), x);
    }
    f32x16 pq, qq;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int l = 32 * hf + 8 * (e >> 2) + 4 * hh + (e & 3);
      float p = 0.f, q = 0.f;
      if (lower && l < ja) {
        const float dA = -x[e];
        const float g = GATED ? __expf(Gj - Gs[l]) : 1.f;
        p = dA * Bj * g;
        q = p * kk[e];
        db_part += dA * kk[e] * g;
        rq_part += q;
      }
      pq[e] = p;
      qq[e] = q;
    }
    char* t = reinterpret_cast<char*>(Pn);
#pragma unroll
    for (int I = 0; I < 4; ++I)
      *reinterpret_cast<v4_t<T>*>(t + tile_off(ja, 32 * hf + 8 * I + 4 * hh)) =
          to4<T>(pq[4 * I], pq[4 * I + 1], pq[4 * I + 2], pq[4 * I + 3]);
#pragma unroll
    for (int e = 0; e < 16; ++e) Qb[(32 * hf + 8 * (e >> 2) + 4 * hh + (e & 3)) * 64 + ja] = qq[e];
  }
  __syncthreads();

  // 5. dk[a][d] += sum_l K[l][d] (P[a][l] + P[l][a]); dk and dv out through
  //    this wave's 4 KiB of the dW area
  u32x4* stage = reinterpret_cast<u32x4*>(dWt) + 256 * w;
  if (has_dk) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int db2 = 2 * hf + m;
      const T* ktile = Kt + (db2 / 2) * TE;
#pragma unroll
      for (int lbk = 0; lbk < 2; ++lbk)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const v8_t<T> kop = tile_tr8<T>(ktile, 32 * lbk, 32 * (db2 & 1), jj, lane);
          dk[m] = mma(kop, tile_ldp8<T>(Pn, ja, 32 * lbk, jj, hh), dk[m]);
          dk[m] = mma(kop, tile_tr8<T>(Pn, 32 * lbk, 32 * lb, jj, lane), dk[m]);
        }
    }
    store_rows_staged<T>(dk[0], dk[1], stage, (T*)a.dk + (((size_t)b * Tn + t0 + 32 * lb) * H + h) * DK + 64 * hf,
                         (int64_t)H * DK, lane, nvalid);
  }
  if (has_dv)
    store_rows_staged<T>(dv[0], dv[1], stage, (T*)a.dv + (((size_t)b * Tn + t0 + 32 * lb) * H + h) * DV + 64 * hf,
                         (int64_t)H * DV, lane, nvalid);

  db_part += __shfl_xor(db_part, 32);
  dg_part += __shfl_xor(dg_part, 32);
  rq_part += __shfl_xor(rq_part, 32);
  if (hh == 0) {
    red_b[w][ja] = db_part;
    red_g[w][ja] = dg_part + rq_part;
  }
  __syncthreads();
  if (tid < 64) {
    // column part of dG: sum_a Q[a][l] = row l of Q^T
    float cq = 0.f;
#pragma unroll
    for (int q4 = 0; q4 < 16; ++q4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(Qb + tid * 64 + 4 * q4);
      cq += (v[0] + v[1]) + (v[2] + v[3]);
    }
    const int t = t0 + tid;
    const int l2 = tid >> 5;  // lane block of this row
    const float dbeta = red_b[l2][tid] + red_b[l2 + 2][tid];
    float x = reinterpret_cast<const float*>(a.ws + L.dGp)[(size_t)bh * Tp + t0 + tid] + red_g[l2][tid] +
              red_g[l2 + 2][tid] - cq;
    // reverse inclusive cumsum over the chunk: dg_l = sum_{i >= l} dG_i
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_down(x, off);
      if (tid + off < 64) x += y;
    }
    if (t < Tn) {
      a.dbeta[((size_t)b * Tn + t) * H + h] = dbeta;
      if constexpr (GATED) a.dg[((size_t)b * Tn + t) * H + h] = x;
    }
  }
}

template <typename T, int DK, int DV, bool GATED>
hipError_t launch_delta_bwd(const DeltaArgs& a, hipStream_t stream) {
  const DeltaLayout L = delta_layout(a.B, a.T, a.H, DK, DV, sizeof(T));
  const int BH = a.B * a.H;
  delta_state_bwd_kernel<T, DK, DV, GATED><<<dim3(BH), dim3(64 * (DV / 32)), 0, stream>>>(a, L);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  delta_bwd_chunk_kernel<T, DK, DV, GATED><<<dim3(BH * a.NT), dim3(256), 0, stream>>>(a, L);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  delta_wy_bwd_kernel<T, DK, DV, GATED><<<dim3(BH * a.NT), dim3(256), 0, stream>>>(a, L);
  return hipGetLastError();
}

#define LINATT_DELTA_BWD_INST(T, DK, DV)                                              \
  template hipError_t launch_delta_bwd<T, DK, DV, false>(const DeltaArgs&, hipStream_t); \
  template hipError_t launch_delta_bwd<T, DK, DV, true>(const DeltaArgs&, hipStream_t);

LINATT_DELTA_SHAPES(LINATT_DELTA_BWD_INST)

}  // namespace linatt
