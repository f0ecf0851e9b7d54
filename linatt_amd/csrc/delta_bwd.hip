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
  float* dWg = reinterpret_cast<float*>(a.ws + L.dW) + ((size_t)bh * Tp + t0 + i) * DK;
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
      *reinterpret_cast<float4*>(dWg + d) =
          make_float4(-dw[4 * I], -dw[4 * I + 1], -dw[4 * I + 2], -dw[4 * I + 3]);
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
// Tm = (I + A)^-1; final dk, dv, dbeta, dg.
// Wave w: row block ib = w & 1, column half chf = w >> 1.
// ---------------------------------------------------------------------------
template <typename T, int DK, int DV, bool GATED>
__global__ __launch_bounds__(256, 2) void delta_wy_bwd_kernel(DeltaArgs a, DeltaLayout L) {
  constexpr int PX = 64 + 8;
  constexpr int NKW = DK / 64, NVW = DV / 64;
  __shared__ __attribute__((aligned(16))) T TmT[64 * PX];
  __shared__ __attribute__((aligned(16))) T X1T[64 * PX];
  constexpr int PV = DV + 8;
  __shared__ __attribute__((aligned(16))) T buf[64 * PV + DK * PX];
  __shared__ float Gs[64], Bs[64];
  __shared__ float red_b[2][64], red_g[2][64], red_rb[64];

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int ib = w & 1, chf = w >> 1;
  const int Tn = a.T, H = a.H, NT = a.NT;
  const int c = blockIdx.x % NT, bh = blockIdx.x / NT;
  const int b = bh / H, h = bh % H;
  const int t0 = c * kChunk;
  const size_t Tp = (size_t)NT * kChunk;
  const size_t ci = (size_t)bh * NT + c;

  const T* kb = (const T*)a.k + ((size_t)b * Tn * H + h) * DK;
  const T* vb = (const T*)a.v + ((size_t)b * Tn * H + h) * DV;
  const int64_t ks = (int64_t)H * DK, vs = (int64_t)H * DV;
  const T* tmg = (const T*)(a.ctx + L.Tm) + ci * 4096;
  const T* dUt = (const T*)(a.ws + L.dVnT) + ci * DV * 64;  // dU^T [v][i]
  const float* dWg = reinterpret_cast<const float*>(a.ws + L.dW) + ((size_t)bh * Tp + t0) * DK;
  const float* Gc = reinterpret_cast<const float*>(a.ctx + L.Gc) + (size_t)bh * Tp;

  T* dUn = buf;             // dU natural [i][v]
  T* dWT = buf + 64 * PV;   // dW^T [d][i]
  T* KT = buf;

  load_tile64x<T, T, 64, 1, PX, false, true>(tmg, 0, 64, 64, nullptr, TmT, tid, nullptr);
#pragma unroll
  for (int r0 = 0; r0 < DV; r0 += 64)
    load_tile64x<T, T, 64, 1, PV, false, true>(dUt + (size_t)r0 * 64, 0, 64, 64, nullptr, dUn + r0, tid, nullptr);
  load_tile64x<float, T, DK, 1, PX, false, true>(dWg, 0, 64, DK, nullptr, dWT, tid, nullptr);
  if (tid < 64) {
    const int t = t0 + tid;
    Gs[tid] = GATED ? Gc[t0 + tid] : 0.f;
    Bs[tid] = t < Tn ? a.beta[((size_t)b * Tn + t) * H + h] : 0.f;
  }
  __syncthreads();

  const int i = 32 * ib + cl;  // lane's chunk row
  const int ti = t0 + i;
  const bool valid = ti < Tn;
  const float Gi = Gs[i], Bi = Bs[i];
  const float eGi = GATED ? __expf(Gi) : 1.f;

  // (a) Tm^T dU -> dv; (b) Tm^T dW -> dk (W part).  Lane column i.
  float db_part = 0.f, dg_part = 0.f;
  T* dvg = (T*)a.dv + (((size_t)b * Tn + ti) * H + h) * DV;
#pragma unroll
  for (int m = 0; m < NVW; ++m) {
    const int vt = chf * NVW + m;
    f32x16 acc{};
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = mma(ld8<T>(dUt + (32 * vt + cl) * 64 + 16 * s + 8 * hh),
                ld8<T>(TmT + i * PX + 16 * s + 8 * hh), acc);
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const int d = 32 * vt + 8 * I + 4 * hh;
      const v4_t<T> v4 = valid ? ld4<T>(vb + (int64_t)ti * vs + d) : v4_t<T>{};
#pragma unroll
      for (int r = 0; r < 4; ++r) db_part += (float)v4[r] * acc[4 * I + r];
      if (valid)
        st4<T>(dvg + d, to4<T>(Bi * acc[4 * I], Bi * acc[4 * I + 1], Bi * acc[4 * I + 2],
                               Bi * acc[4 * I + 3]));
    }
  }
  f32x16 dkacc[NKW];
#pragma unroll
  for (int m = 0; m < NKW; ++m) {
    const int dt = chf * NKW + m;
    f32x16 acc{};
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = mma(ld8<T>(dWT + (32 * dt + cl) * PX + 16 * s + 8 * hh),
                ld8<T>(TmT + i * PX + 16 * s + 8 * hh), acc);
    float kdot = 0.f;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const int d = 32 * dt + 8 * I + 4 * hh;
      const v4_t<T> k4 = valid ? ld4<T>(kb + (int64_t)ti * ks + d) : v4_t<T>{};
#pragma unroll
      for (int r = 0; r < 4; ++r) kdot += (float)k4[r] * acc[4 * I + r];
    }
    db_part += eGi * kdot;
    dg_part += Bi * eGi * kdot;
    dkacc[m] = acc * (Bi * eGi);
  }

  // (c) dTm^T (lane column i, rows j): beta_j (V_j . dU_i) + beta_j e^G_j (K_j . dW_i)
  f32x16 dTmT[2];
#pragma unroll
  for (int jt = 0; jt < 2; ++jt) {
    const int jr = 32 * jt + cl;
    const bool jv = t0 + jr < Tn;
    f32x16 av{}, ak{};
#pragma unroll
    for (int s = 0; s < DV / 16; ++s)
      av = mma(jv ? ld8<T>(vb + (int64_t)(t0 + jr) * vs + 16 * s + 8 * hh) : zero8<T>(),
               ld8<T>(dUn + i * PV + 16 * s + 8 * hh), av);
#pragma unroll
    for (int s = 0; s < DK / 16; ++s)
      ak = mma(jv ? ld8<T>(kb + (int64_t)(t0 + jr) * ks + 16 * s + 8 * hh) : zero8<T>(),
               ld8_f32<T>(dWg + (size_t)i * DK + 16 * s + 8 * hh), ak);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int j = 32 * jt + 8 * (e >> 2) + 4 * hh + (e & 3);
      const float bj = Bs[j];
      dTmT[jt][e] = bj * (av[e] + (GATED ? __expf(Gs[j]) : 1.f) * ak[e]);
    }
  }
  // (c2) X1[i][l] = sum_j dTm[i][j] Tm[l][j]: tile l in half chf, lane column i -> X1T[l][i]
  {
    const int lt = chf;
    f32x16 x1{};
#pragma unroll
    for (int jt = 0; jt < 2; ++jt)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        x1 = mma(ld_tr_op<T>(tmg + (32 * lt + cl) * 64 + 32 * jt, j, hh), c_to_b<T>(dTmT[jt], j), x1);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int l = 32 * lt + 8 * (e >> 2) + 4 * hh + (e & 3);
      X1T[l * PX + i] = (T)x1[e];
    }
  }
  __syncthreads();  // X1T complete; dUn / dWT no longer needed
  load_tile64x<T, T, DK, 1, PX, false, true>(kb, t0, Tn, ks, nullptr, KT, tid, nullptr);
  __syncthreads();

  // KK tiles: regs index in tile x, lane index i:  KK[x-row][i]
  f32x16 KK[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int xr = 32 * x + cl;
    const bool xv = t0 + xr < Tn;
    f32x16 acc{};
#pragma unroll
    for (int s = 0; s < DK / 16; ++s)
      acc = mma(xv ? ld8<T>(kb + (int64_t)(t0 + xr) * ks + 16 * s + 8 * hh) : zero8<T>(),
                valid ? ld8<T>(kb + (int64_t)ti * ks + 16 * s + 8 * hh) : zero8<T>(), acc);
    KK[x] = acc;
  }

  // (d) orientation 1: lane column a = i, regs l.  dA[a][l] = -sum_i' X1[i'][l] Tm[i'][a]
  float rb_sum = 0.f, rg_sum = 0.f, cg_sum = 0.f;
  f32x16 At1[2], At2[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    f32x16 acc{};
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = mma(ld8<T>(X1T + (32 * x + cl) * PX + 16 * s + 8 * hh),
                ld8<T>(TmT + i * PX + 16 * s + 8 * hh), acc);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int l = 32 * x + 8 * (e >> 2) + 4 * hh + (e & 3);
      float at = 0.f;
      if (l < i) {
        const float dA = -acc[e];
        const float gam = GATED ? __expf(Gi - Gs[l]) : 1.f;
        const float e1 = dA * KK[x][e] * gam;
        rb_sum += e1;
        rg_sum += Bi * e1;
        at = dA * Bi * gam;
      }
      At1[x][e] = at;
    }
  }
  // (e) orientation 2: lane column l = i, regs a.  dA[a][l] = -sum_i' Tm[i'][a] X1[i'][l]
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    f32x16 acc{};
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = mma(ld8<T>(TmT + (32 * x + cl) * PX + 16 * s + 8 * hh),
                ld8<T>(X1T + i * PX + 16 * s + 8 * hh), acc);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int aa = 32 * x + 8 * (e >> 2) + 4 * hh + (e & 3);
      float at = 0.f;
      if (aa > i) {
        const float dA = -acc[e];
        const float gam = GATED ? __expf(Gs[aa] - Gi) : 1.f;
        const float ba = Bs[aa];
        cg_sum += dA * ba * KK[x][e] * gam;
        at = dA * ba * gam;
      }
      At2[x][e] = at;
    }
  }
  rb_sum += __shfl_xor(rb_sum, 32);
  rg_sum += __shfl_xor(rg_sum, 32);
  cg_sum += __shfl_xor(cg_sum, 32);

  // dk = dKp + dKW + At K + At^T K   (lane column i, this wave's key-dim half)
  const float* dKp = reinterpret_cast<const float*>(a.ws + L.dKp) + ((size_t)bh * Tp + t0 + i) * DK;
  T* dkg = (T*)a.dk + (((size_t)b * Tn + ti) * H + h) * DK;
#pragma unroll
  for (int m = 0; m < NKW; ++m) {
    const int dt = chf * NKW + m;
    f32x16 acc = dkacc[m];
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const v8_t<T> xo = ld_tr_op<T>(KT + (32 * dt + cl) * PX + 32 * x, j, hh);
        acc = mma(xo, c_to_b<T>(At1[x], j), acc);
        acc = mma(xo, c_to_b<T>(At2[x], j), acc);
      }
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const int d = 32 * dt + 8 * I + 4 * hh;
      const float4 p = *reinterpret_cast<const float4*>(dKp + d);
      if (valid)
        st4<T>(dkg + d, to4<T>(acc[4 * I] + p.x, acc[4 * I + 1] + p.y, acc[4 * I + 2] + p.z,
                               acc[4 * I + 3] + p.w));
    }
  }

  db_part += __shfl_xor(db_part, 32);
  dg_part += __shfl_xor(dg_part, 32);
  if (hh == 0) {
    red_b[chf][i] = db_part;
    red_g[chf][i] = dg_part;
    if (chf == 0) {
      red_rb[i] = rb_sum;
      red_g[0][i] += rg_sum - cg_sum;
    }
  }
  __syncthreads();
  if (tid < 64) {
    const int t = t0 + tid;
    const float dbeta = red_b[0][tid] + red_b[1][tid] + red_rb[tid];
    float x = reinterpret_cast<const float*>(a.ws + L.dGp)[(size_t)bh * Tp + t0 + tid] +
              red_g[0][tid] + red_g[1][tid];
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
