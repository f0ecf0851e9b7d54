// KATA-SPD in psi-state form for long-context prefill and recurrent decode
// (gfx950).
//
// The reference's O(T) concat-state path is spd_chunk_scan_cat
// (kata/spd/chunk_scan_cat.py:219-345, kernels :32-216, scan
// kata/spd/chunk_scan.py:182-292): per group g of width E, psi(x) =
// vec(x_g x_g^T) (full E^2, not packed), o = (sum_g psi(q_g)^T H_g + intra) /
// max(sum_g psi(q_g).Z_g + intra, EPS).  The reference materialises every
// chunk state; its flash path keeps no decode state at all (kata/layer.py:492),
// so the decode step has no reference implementation and is pinned by the
// identity "decode after n tokens == row n of the parallel form".
//
// Prefill here splits T into segments of L tokens (L a multiple of 128):
//   kata_seg_state_kernel   per (b, h, segment, 768 packed state rows):
//                           S_seg = Psi(K_seg)^T V_seg, z_seg = Psi(K_seg)^T 1
//                           (MFMA; the psi features are formed in registers
//                           from a transposed K tile in LDS)
//   kata_seg_scan_kernel    exclusive prefix over segments -> H (T, [v][p])
//                           and z entering each segment; the final state
//   kata_prefill_out_kernel per (b, h, 128 queries): psi(q)^T H + the flash
//                           (quadratic) score over the keys of the query's
//                           own segment, normalised with the EPS floor.
// State rows are p = g E^2 + a E + b.  Inside the prefill psi is unscaled
// (o is scale-invariant); the returned state is psi(sqrt(scale) x) as in the
// reference, i.e. the unscaled sums times scale.
//
// Packed rows: psi(x)_g = vec(x_g x_g^T) is symmetric in (a, b), so the
// segment states and the prefix keep 3/4 of each group's rows (pk_ab): the
// rows a < E/2 with every b, then the rows a >= E/2 with b >= E/2.  Each
// unordered pair {a, b} is one of them with a <= b, and the scan folds the
// pair weight c_ab (2 for a < b, 1 for a = b, 0 for the rows below the
// diagonal, which repeat a pair) into the prefix state, so
// psi(q)^T H = sum over packed rows of q_a q_b (c_ab H_ab).  z stays in the
// full layout (the den product reads it as E x E blocks), and the returned
// state is unpacked to the full layout.
#include "common.h"
#include "kata_kernels.h"

namespace linatt {

// packed rows per group, and (a, b) of packed row r of a group
template <int E>
constexpr int kPkRows = 3 * E * E / 4;
template <int E>
__host__ __device__ __forceinline__ void pk_ab(int r, int& a, int& b) {
  if (r < E * E / 2) {
    a = r / E;
    b = r % E;
  } else {
    const int s = r - E * E / 2;
    a = E / 2 + s / (E / 2);
    b = E / 2 + s % (E / 2);
  }
}
// weight of packed pair (a, b) in psi(q)^T H
__host__ __device__ __forceinline__ float pk_weight(int a, int b) { return b < a ? 0.f : (a == b ? 1.f : 2.f); }

// ---------------------------------------------------------------------------
// Segment states.  One workgroup of 8 waves covers 768 packed state rows of
// one (b, h, segment), so each key/value tile is read once per 768 rows; wave
// w owns packed rows p = 768 pb + 96 w + 32 i4 + [0, 32), i4 = 0..2 (its
// X-operand rows).  K^T sits in LDS as fp32 so the psi products need no
// unpacking.
// ---------------------------------------------------------------------------
template <typename T, int DK, int DV, int M>
__global__ __launch_bounds__(512) void kata_seg_state_kernel(KataStateArgs a) {
  constexpr int E = DK / M, P = M * E * E, PR = kPkRows<E>, PP = M * PR;
  constexpr int PK = 64 + 4;  // fp32 K^T pitch
  constexpr int PV = 64 + 8;  // V^T pitch
  constexpr int WR = 768, NI = WR / 256;  // rows per workgroup, 32-row blocks per wave
  constexpr int NPB = PP / WR;
  static_assert(PP % WR == 0 && (M == 2 || M == 4), "768 packed rows per workgroup");
  // one LDS area: K^T (fp32) | V^T | per-wave partial 32 x 32 tiles of the
  // Gram matrix K^T K (z, below) during the key loop, then the stage of
  // S_seg^T: VC value rows of 1024 state rows (pitch SP) per pass
  constexpr int VC = 16, SP = WR + 4;
  constexpr int LOOPF = DK * PK + DV * PV * (int)sizeof(T) / 4 + 8 * 1024;
  constexpr int LDSF = LOOPF > VC * SP ? LOOPF : VC * SP;
  __shared__ __attribute__((aligned(16))) float Lds[LDSF];
  float* const Kt = Lds;
  T* const Vt = reinterpret_cast<T*>(Lds + DK * PK);
  float (*const Gp)[32 * 32] = reinterpret_cast<float (*)[32 * 32]>(Lds + DK * PK + DV * PV * (int)sizeof(T) / 4);
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  int blk = blockIdx.x;
  const int pb = blk % NPB;
  blk /= NPB;
  const int seg = blk % a.nseg;
  const int bh = blk / a.nseg;
  const int b = bh / a.H, h = bh % a.H;
  const T* kb = (const T*)a.k + (int64_t)b * a.sb + (int64_t)h * a.sh;
  const T* vb = (const T*)a.v + (int64_t)b * a.vsb + (int64_t)h * a.vsh;

  const int p0 = WR * pb + 96 * w;
  int ra[NI], rb[NI];
#pragma unroll
  for (int i4 = 0; i4 < NI; ++i4) {
    const int p = p0 + 32 * i4 + cl, g = p / PR;
    int ga, gb;
    pk_ab<E>(p % PR, ga, gb);
    ra[i4] = g * E + ga;
    rb[i4] = g * E + gb;
  }
  // K^T row d holds keys in groups of four, group q at 4 (q ^ ((d >> 4) & 3)):
  // the conversion's 16-lane f32x4 writes (rows 4 cb + cc, groups rq) then
  // fall in 16 distinct bank quads, and the reads of 16 distinct rows stay so
  auto kt_off = [](int d, int q) { return d * PK + 4 * (q ^ ((d >> 4) & 3)); };
  // V^T row d the same way in groups of eight keys (16 bytes), group q at
  // 8 (q ^ ((d >> 4) & 3)); the read of group 2 s + hh splits into a lane
  // base for even and for odd s plus 16 s
  int vo[DV / 32][2];
#pragma unroll
  for (int vt = 0; vt < DV / 32; ++vt) {
    const int d = 32 * vt + cl, f = (d >> 4) & 3;
    const int b0 = d * PV + 8 * (hh ^ (f & 1)), fs = 16 * (f >> 1);
    vo[vt][0] = b0 + fs;  // even s: s ^ (f >> 1) = s + (f >> 1)
    vo[vt][1] = b0 - fs;  // odd s: s ^ (f >> 1) = s - (f >> 1)
  }
  int ko[4][NI];  // per i4: rows ra (key groups 2 hh, 2 hh + 1) and rb, before + 16 s
#pragma unroll
  for (int i4 = 0; i4 < NI; ++i4) {
    ko[0][i4] = kt_off(ra[i4], 2 * hh);
    ko[1][i4] = kt_off(ra[i4], 2 * hh + 1);
    ko[2][i4] = kt_off(rb[i4], 2 * hh);
    ko[3][i4] = kt_off(rb[i4], 2 * hh + 1);
  }

  f32x16 acc[NI][DV / 32];
#pragma unroll
  for (int i4 = 0; i4 < NI; ++i4)
#pragma unroll
    for (int vt = 0; vt < DV / 32; ++vt) acc[i4][vt] = f32x16{};
  // z_p = sum_s k_s[ra] k_s[rb] = (K^T K)[ra][rb]: the workgroup's rows need
  // two 32 x 32 tiles of the Gram matrix (M = 1: the two column halves of
  // row half pb / 2; M = 2: the diagonal tile of group pb, twice; M = 4: both
  // diagonal tiles).  Waves 4 u .. 4 u + 3 accumulate tile u, each over its
  // own 16-key step w % 4 of every key tile, so z costs one MFMA per wave
  // and key tile instead of a sum per psi feature.
  auto gt_i = [&](int u) { return M == 1 ? pb >> 1 : (M == 2 ? pb : u); };
  auto gt_j = [&](int u) { return M == 1 ? u : gt_i(u); };
  const int gti = gt_i(w >> 2), gtj = gt_j(w >> 2);
  f32x16 gz{};
  const int s_begin = seg * a.L, s_end = min(s_begin + a.L, a.T);
  // next tile prefetched into registers during the current one's compute:
  // waves 0-3 carry K, waves 4-7 V, one 4 x 4 block per thread
  const bool isK = w < 4;
  const int lt = tid & 255, cb = lt % 16, rq = lt / 16;
  const T* src = isK ? kb : vb;
  const int64_t rs = isK ? a.st : a.vst;
  v4_t<T> pre[4];
  auto gload = [&](int s0) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = s0 + 4 * rq + r;
      pre[r] = row < a.T ? ld4<T>(src + (int64_t)row * rs + 4 * cb) : v4_t<T>{};
    }
  };
  auto lstore = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      if (isK)
        *reinterpret_cast<f32x4*>(Kt + (4 * cb + cc) * PK + 4 * (rq ^ (cb >> 2))) =
            f32x4{(float)pre[0][cc], (float)pre[1][cc], (float)pre[2][cc], (float)pre[3][cc]};
      else
        st4<T>(Vt + (4 * cb + cc) * PV + 8 * ((rq >> 1) ^ (cb >> 2)) + 4 * (rq & 1),
               v4_t<T>{pre[0][cc], pre[1][cc], pre[2][cc], pre[3][cc]});
    }
  };
  static_assert(DK == 64 && DV == 64, "64 x 64 tiles");
  gload(s_begin);
  for (int s0 = s_begin; s0 < s_end; s0 += 64) {
    __syncthreads();
    lstore();
    __syncthreads();
    if (s0 + 64 < s_end) gload(s0 + 64);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      v8_t<T> vop[DV / 32];
#pragma unroll
      for (int vt = 0; vt < DV / 32; ++vt) vop[vt] = ld8<T>(Vt + vo[vt][s & 1] + 16 * s);
#pragma unroll
      for (int i4 = 0; i4 < NI; ++i4) {
        const f32x4 a0 = *reinterpret_cast<const f32x4*>(Kt + ko[0][i4] + 16 * s);
        const f32x4 a1 = *reinterpret_cast<const f32x4*>(Kt + ko[1][i4] + 16 * s);
        const f32x4 c0 = *reinterpret_cast<const f32x4*>(Kt + ko[2][i4] + 16 * s);
        const f32x4 c1 = *reinterpret_cast<const f32x4*>(Kt + ko[3][i4] + 16 * s);
        const f32x8 pf{a0[0] * c0[0], a0[1] * c0[1], a0[2] * c0[2], a0[3] * c0[3],
                       a1[0] * c1[0], a1[1] * c1[1], a1[2] * c1[2], a1[3] * c1[3]};
        const v8_t<T> x = __builtin_convertvector(pf, v8_t<T>);
#pragma unroll
        for (int vt = 0; vt < DV / 32; ++vt) acc[i4][vt] = mma(x, vop[vt], acc[i4][vt]);
      }
    }
    {
      // Gram step: rows 32 gti + cl and columns 32 gtj + cl of K^T, keys
      // 16 (w % 4) + 8 hh + [0, 8) (the same k-order on both operands)
      const f32x4 a0 = *reinterpret_cast<const f32x4*>(Kt + kt_off(32 * gti + cl, 4 * (w & 3) + 2 * hh));
      const f32x4 a1 = *reinterpret_cast<const f32x4*>(Kt + kt_off(32 * gti + cl, 4 * (w & 3) + 2 * hh + 1));
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(Kt + kt_off(32 * gtj + cl, 4 * (w & 3) + 2 * hh));
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(Kt + kt_off(32 * gtj + cl, 4 * (w & 3) + 2 * hh + 1));
      const v8_t<T> xa = __builtin_convertvector(f32x8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]}, v8_t<T>);
      const v8_t<T> xb = __builtin_convertvector(f32x8{b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]}, v8_t<T>);
      gz = mma(xa, xb, gz);
    }
  }
  // partial Gram tiles -> LDS (C layout: row 8 I + 4 hh + r, lane column),
  // summed over the four waves of each tile in a fixed order
#pragma unroll
  for (int e = 0; e < 16; ++e) Gp[w][(8 * (e >> 2) + 4 * hh + (e & 3)) * 32 + cl] = gz[e];
  __syncthreads();
  // z in the full layout: each unordered pair is the packed row with
  // ra <= rb, which writes both of its entries
#pragma unroll
  for (int i4 = 0; i4 < NI; ++i4) {
    const int u = (ra[i4] >> 5) == gt_i(0) && (rb[i4] >> 5) == gt_j(0) ? 0 : 1;
    const int o = (ra[i4] & 31) * 32 + (rb[i4] & 31);
    const float z = (Gp[4 * u][o] + Gp[4 * u + 1][o]) + (Gp[4 * u + 2][o] + Gp[4 * u + 3][o]);
    if (hh == 0 && ra[i4] <= rb[i4]) {
      const int g = ra[i4] / E, za = ra[i4] % E, zb = rb[i4] % E;
      float* zs = a.seg_z + ((size_t)bh * a.nseg + seg) * P + g * E * E;
      zs[za * E + zb] = z;
      if (za != zb) zs[zb * E + za] = z;
    }
  }
  // acc[i4][vt] = D[p'][v]: rows p' = 96 w + 32 i4 + 8 I + 4 hh + r of the
  // workgroup's 768, lane column v = 32 vt + cl  ->  stage [v - vc0][p'],
  // then S_seg^T [v][768 pb + p'] rows by whole 16-byte runs
  float* st = a.seg_S + ((size_t)bh * a.nseg + seg) * DV * PP + WR * pb;
#pragma unroll
  for (int pass = 0; pass < DV / VC; ++pass) {
    const int vc0 = VC * pass, vt = vc0 / 32, vl = 32 * vt + cl - vc0;
    __syncthreads();  // the Gram partials (or the previous pass) are read
    if (vl >= 0 && vl < VC) {
#pragma unroll
      for (int i4 = 0; i4 < NI; ++i4)
#pragma unroll
        for (int I = 0; I < 4; ++I)
          *reinterpret_cast<f32x4*>(Lds + vl * SP + 96 * w + 32 * i4 + 8 * I + 4 * hh) =
              f32x4{acc[i4][vt][4 * I], acc[i4][vt][4 * I + 1], acc[i4][vt][4 * I + 2], acc[i4][vt][4 * I + 3]};
    }
    __syncthreads();
    static_assert(VC * WR / 4 % 512 == 0, "whole store rounds");
#pragma unroll
    for (int it = 0; it < VC * WR / 4 / 512; ++it) {
      const int idx = 512 * it + tid, row = idx / (WR / 4), c4 = idx % (WR / 4);
      *reinterpret_cast<f32x4*>(st + (size_t)(vc0 + row) * PP + 4 * c4) =
          *reinterpret_cast<const f32x4*>(Lds + row * SP + 4 * c4);
    }
  }
}

// ---------------------------------------------------------------------------
// Exclusive prefix over segments.  One thread per (bh, value row v, 4
// consecutive packed state rows, which share their a), then one per (bh, 4
// consecutive full rows of z).  The prefix state is written as c_ab H_ab.
// S_in / S_out and z_in / z_out are in the full or the packed layout
// (a.tri).  A thread reads, then writes, only its own state elements, so
// the full layout's S_in / z_in may alias S_out / z_out; in the packed
// layout a full row of z below the diagonal reads its pair's element, which
// another thread writes, so the host hands an aliased z_in over as a copy.
// The packed state rows below the diagonal, whose prefix is weighted by 0,
// start from zero.
// ---------------------------------------------------------------------------
template <typename T, int DK, int DV, int M>
__global__ __launch_bounds__(256) void kata_seg_scan_kernel(KataStateArgs a) {
  constexpr int E = DK / M, P = M * E * E, PR = kPkRows<E>, PP = M * PR;
  constexpr int PT = M * E * (E + 1) / 2;  // unordered pairs (packed layout rows)
  static_assert(PR % 4 == 0 && (E / 2) % 4 == 0, "4 packed rows share their a");
  constexpr int64_t nS = (int64_t)DV * (PP / 4), per_bh = nS + P / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)a.B * a.H * per_bh) return;
  const int bh = (int)(idx / per_bh);
  const int64_t rem = idx % per_bh;
  const float is = 1.f / a.scale, sc = a.scale;
  if (rem >= nS) {
    // z: full rows p .. p + 3 = pairs (za, zb0 + j) of group zg
    const int p = 4 * (int)(rem - nS);
    const int zg = p / (E * E), za = (p / E) % E, zb0 = p % E;
    auto tri = [&](int j) {
      const int zb = zb0 + j;
      return (size_t)bh * PT + kata_state_tri_row(E, zg, za < zb ? za : zb, za < zb ? zb : za);
    };
    float4 run = make_float4(0.f, 0.f, 0.f, 0.f);
    if (a.z_in) {
      if (a.tri) {
        run = make_float4(a.z_in[tri(0)] * is, a.z_in[tri(1)] * is, a.z_in[tri(2)] * is,
                          a.z_in[tri(3)] * is);
      } else {
        const float4 zi = *reinterpret_cast<const float4*>(a.z_in + (size_t)bh * P + p);
        run = make_float4(zi.x * is, zi.y * is, zi.z * is, zi.w * is);
      }
    }
    for (int seg = 0; seg < a.nseg; ++seg) {
      const size_t base = ((size_t)bh * a.nseg + seg) * P + p;
      const float4 x = *reinterpret_cast<const float4*>(a.seg_z + base);
      *reinterpret_cast<float4*>(a.Hz + base) = run;
      run.x += x.x; run.y += x.y; run.z += x.z; run.w += x.w;
    }
    if (a.z_out) {
      if (a.tri) {
        // the pair's element, from its full row with za <= zb
        const float r4[4] = {run.x * sc, run.y * sc, run.z * sc, run.w * sc};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (zb0 + j >= za) a.z_out[tri(j)] = r4[j];
      } else {
        *reinterpret_cast<float4*>(a.z_out + (size_t)bh * P + p) =
            make_float4(run.x * sc, run.y * sc, run.z * sc, run.w * sc);
      }
    }
    return;
  }
  // S: value row v, packed rows p .. p + 3 = pairs (a, b0 + j) of group g
  const int v = (int)(rem / (PP / 4));
  const int p = 4 * (int)(rem % (PP / 4));
  const int g = p / PR;
  int pa, pb0;
  pk_ab<E>(p % PR, pa, pb0);
  const int pf0 = g * E * E + pa * E + pb0;  // full row of (a, b0)
  float cw[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) cw[j] = pk_weight(pa, pb0 + j);
  float r4[4] = {0.f, 0.f, 0.f, 0.f};
  if (a.S_in) {
    // the rows b >= a read their pair's element; the initial state is
    // stored scaled by `scale`, the scan runs unscaled
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int b = pb0 + j;
      if (b < pa) continue;
      r4[j] = (a.tri ? a.S_in[((size_t)bh * PT + kata_state_tri_row(E, g, pa, b)) * DV + v]
                     : a.S_in[((size_t)bh * P + pf0 + j) * DV + v]) * is;
    }
  }
  float4 run = make_float4(r4[0], r4[1], r4[2], r4[3]);
  for (int seg = 0; seg < a.nseg; ++seg) {
    const size_t base = (size_t)bh * a.nseg + seg;
    const float4 x = *reinterpret_cast<const float4*>(a.seg_S + (base * DV + v) * PP + p);
    st4<T>((T*)a.HT + (base * DV + v) * PP + p,
           to4<T>(run.x * cw[0], run.y * cw[1], run.z * cw[2], run.w * cw[3]));
    run.x += x.x; run.y += x.y; run.z += x.z; run.w += x.w;
  }
  if (a.S_out) {
    // rows (a, b) with a <= b write their pair: once (packed layout) or
    // both entries (full layout)
    const float o4[4] = {run.x * sc, run.y * sc, run.z * sc, run.w * sc};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int b = pb0 + j;
      if (b < pa) continue;
      if (a.tri) {
        a.S_out[((size_t)bh * PT + kata_state_tri_row(E, g, pa, b)) * DV + v] = o4[j];
      } else {
        float* so = a.S_out + (size_t)bh * P * DV + v;
        so[(size_t)(pf0 + j) * DV] = o4[j];
        if (b != pa) so[(size_t)(g * E * E + b * E + pa) * DV] = o4[j];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Prefill output: per (b, h, 128 queries) with 32 queries per wave as in
// kata_fwd_kernel (Q^T in registers as the B operand, lane column = query).
//   num = psi(q)^T H_seg + sum_{seg_start <= s <= t} A[t,s] v_s
//   den = psi(q).z_seg  + sum_{seg_start <= s <= t} A[t,s]        (unscaled)
//   o = num / max(den, eps / scale^2),   den_out = max(scale^2 den, eps)
// ---------------------------------------------------------------------------
template <typename T, int DK, int DV, int M>
__global__ __launch_bounds__(256, 2) void kata_prefill_out_kernel(KataStateArgs a, int nqt, int nbh) {
  constexpr int E = DK / M, P = M * E * E, KE = E / 16;
  static_assert(E % 16 == 0, "group width must be a multiple of 16");
  constexpr int QP = DK + 8;
  __shared__ __attribute__((aligned(16))) T Qa[128 * QP];
  // One 32 KiB LDS area, used first for the prefix state H^T [v][p] in
  // chunks of 128 state rows p, double-buffered (64 rows of 256 bytes,
  // 16-byte chunks swizzled by row), then for the intra-segment key and value
  // tiles, double-buffered (swizzled 64 x 64 tiles, see tile_slot).
  constexpr int HCH = 128, HCPR = HCH * (int)sizeof(T) / 16;
  static_assert(DK == 64 && DV == 64 && HCPR == 16 && P % HCH == 0, "64 x 128 16-bit state chunks");
  __shared__ __attribute__((aligned(16))) u32x4 Hs[2][DV * HCPR];
  T* const Kb0 = reinterpret_cast<T*>(Hs[0]);
  T* const Vb0 = Kb0 + 64 * 64;
  T* const Kb1 = reinterpret_cast<T*>(Hs[1]);
  T* const Vb1 = Kb1 + 64 * 64;

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  int qt, bh;
  map_block(blockIdx.x, nqt, nbh, qt, bh, true);
  const int b = bh / a.H, h = bh % a.H;
  const int Tn = a.T;
  const int t0 = qt * 128, tw = t0 + 32 * w, tl = tw + cl;
  const bool tvalid = tl < Tn;
  const T* qb = (const T*)a.q + (int64_t)b * a.sb + (int64_t)h * a.sh;
  const T* kb = (const T*)a.k + (int64_t)b * a.sb + (int64_t)h * a.sh;
  const T* vb = (const T*)a.v + (int64_t)b * a.vsb + (int64_t)h * a.vsh;

  v8_t<T> qop[DK / 16];
#pragma unroll
  for (int kk = 0; kk < DK / 16; ++kk)
    qop[kk] = tvalid ? ld8<T>(qb + (int64_t)tl * a.st + 16 * kk + 8 * hh) : zero8<T>();

  f32x16 oacc[DV / 32];
#pragma unroll
  for (int db = 0; db < DV / 32; ++db) oacc[db] = f32x16{};
  float dpart = 0.f;

  const int seg = t0 / a.L;
  const int seg_start = seg * a.L;

  // inter-segment term from the prefix state (wave-uniform branch): the
  // features psi(q)_p = q_a q_b, p = g E^2 + a E + b, taken 8 columns b at a
  // time: q_b from this lane's B operand registers, q_a from an LDS copy.
  T* qa_row = Qa + (32 * w + cl) * QP;
#pragma unroll
  for (int kk = 0; kk < DK / 16; ++kk) {
    const v8_t<T> x = qop[kk];
    st4<T>(qa_row + 16 * kk + 8 * hh, v4_t<T>{x[0], x[1], x[2], x[3]});
    st4<T>(qa_row + 16 * kk + 8 * hh + 4, v4_t<T>{x[4], x[5], x[6], x[7]});
  }
  __syncthreads();
  // uniform: a 128-query tile never straddles a segment; the first segment's
  // prefix is the initial state, or zero
  if (seg > 0 || a.S_in) {
    const size_t base = (size_t)bh * a.nseg + seg;
    constexpr int PR = kPkRows<E>, PP = M * PR, NC = PP / HCH, KSG = PR / 16;
    static_assert(PP % HCH == 0 && (E == 16 || E == 32), "whole chunks of packed rows");
    const u32x4* hT = reinterpret_cast<const u32x4*>((const T*)a.HT + base * DV * PP);
    const float* hz = a.Hz + base * P;
    // chunk c: rows v of H^T, packed columns [128 c, 128 c + 128); 16 KiB = 4 x 1 KiB per
    // wave, from a scalar base per chunk plus these chunk-invariant lane offsets
    unsigned hoff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = (64 * (4 * w + i) + lane) / HCPR, slot = lane % HCPR;
      hoff[i] = (unsigned)((row * (PP / 8) + (slot ^ (row & 15))) * 16);
    }
    auto issue = [&](int c) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < 4; ++i) dma16s(hT + c * HCPR, hoff[i], Hs[c & 1] + 64 * (4 * w + i));
    };
    vm_drain();  // q of this wave's queries is in registers
    issue(0);
    // den's prefix part psi(q).z = sum_g q_g^T Z_g q_g with Z_g[a][b] =
    // z[g E^2 + a E + b]: Y = blockdiag(Z_g) Q^T by MFMA (A rows (g, a) of
    // row tile rt, k = features (g', b) of k-steps 2 rt, 2 rt + 1, zero where
    // g != g'), then q^T Y per query from the LDS copy of its q row
    static_assert(E <= 32, "a group lies within one 32-row tile");
#pragma unroll
    for (int rt = 0; rt < DK / 32; ++rt) {
      f32x16 y{};
      const int ar = 32 * rt + cl, ga = ar / E;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int ks = 2 * rt + u, f = 16 * ks + 8 * hh, gf = f / E;
        const float* zr = hz + ga * E * E + (ar % E) * E + f % E;
        const f32x4 z0 = ga == gf ? *reinterpret_cast<const f32x4*>(zr) : f32x4{};
        const f32x4 z1 = ga == gf ? *reinterpret_cast<const f32x4*>(zr + 4) : f32x4{};
        // z as 16-bit hi + lo parts: the sums grow with the prefix length,
        // and one rounding of them would cost den its fp32 accuracy
        const f32x8 zf{z0[0], z0[1], z0[2], z0[3], z1[0], z1[1], z1[2], z1[3]};
        const v8_t<T> za = __builtin_convertvector(zf, v8_t<T>);
        const v8_t<T> zl = __builtin_convertvector(zf - __builtin_convertvector(za, f32x8), v8_t<T>);
        y = mma(za, qop[ks], y);
        y = mma(zl, qop[ks], y);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const v4_t<T> q4 = *reinterpret_cast<const v4_t<T>*>(qa_row + 32 * rt + 8 * i + 4 * hh);
#pragma unroll
        for (int r = 0; r < 4; ++r) dpart += (float)q4[r] * y[4 * i + r];
      }
    }
    // k-step ks of the packed rows (16 of them): group ks / KSG; rows a < E/2
    // take one a and 16 b's, as do E = 32's rows a >= 16 (b = 16..31);
    // E = 16's rows a >= 8 pair up, a = 8 + 2 i + hh per lane half, both on
    // b = 8..15.  q_a and the lane's eight q_b come from the LDS copy of its
    // query row, so the k-step may be a runtime index
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      vm_wait_barrier<0>();
      if (c + 1 < NC) issue(c + 1);
      if (tw < Tn) {
        const u32x4* Hb = Hs[c & 1];
#pragma unroll
        for (int j = 0; j < HCH / 16; ++j) {
          const int ks = c * (HCH / 16) + j, g = ks / KSG, l = ks % KSG;
          int aU, bU;
          bool pair = false;
          if (l < E * E / 32) {
            aU = 16 * l / E;
            bU = 16 * l % E;
          } else if (E == 16) {
            aU = 8 + 2 * (l - 8);
            bU = 8;
            pair = true;
          } else {
            aU = E / 2 + (l - E * E / 32);
            bU = E / 2;
          }
          const float qa = (float)qa_row[g * E + aU + (pair ? hh : 0)];
          const v8_t<T> qb = *reinterpret_cast<const v8_t<T>*>(qa_row + g * E + bU + (pair ? 0 : 8 * hh));
          f32x8 pf;
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) pf[jj] = qa * (float)qb[jj];
          const v8_t<T> y = __builtin_convertvector(pf, v8_t<T>);
#pragma unroll
          for (int db = 0; db < DV / 32; ++db) {
            const int row = 32 * db + cl;
            const u32x4 hv = Hb[row * HCPR + ((2 * j + hh) ^ (row & 15))];
            oacc[db] = mma(__builtin_bit_cast(v8_t<T>, hv), y, oacc[db]);
          }
        }
      }
    }
  }

  // intra-segment flash term, keys in [seg_start, min(t0 + 128, T)): key and
  // value tiles by direct global->LDS copies, double-buffered, V^T through
  // transposing reads (as kata_fwd_tile_kernel)
  const int s_end = min(t0 + 128, Tn);
  const int nst = (s_end - seg_start + 63) / 64;
  auto issue = [&](int st) __attribute__((always_inline)) {
    T* kt = (st & 1) ? Kb1 : Kb0;
    T* vt = (st & 1) ? Vb1 : Vb0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      dma_tile64<T>(kb, a.st, seg_start + 64 * st, Tn, kt, 2 * w + i, lane);
      dma_tile64<T>(vb, a.vst, seg_start + 64 * st, Tn, vt, 2 * w + i, lane);
    }
  };
  __syncthreads();  // every wave is done with the prefix-state chunks
  vm_drain();
  issue(0);
  for (int st = 0; st < nst; ++st) {
    const int s0 = seg_start + 64 * st;
    vm_wait_barrier<0>();
    if (st + 1 < nst) issue(st + 1);
    const T* Kt = (st & 1) ? Kb1 : Kb0;
    const T* Vs = (st & 1) ? Vb1 : Vb0;
    if (s0 > tw + 31 || tw >= Tn) continue;
    const bool need_mask = (s0 + 63 > tw) || (s0 + 64 > Tn);
    f32x16 sc[2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      sc[sb] = f32x16{};
#pragma unroll
      for (int g = 0; g < M; ++g) {
        f32x16 r{};
#pragma unroll
        for (int kk = 0; kk < KE; ++kk)
          r = mma(tile_ld8<T>(Kt, 32 * sb + cl, g * E + 16 * kk + 8 * hh), qop[g * KE + kk], r);
        sc[sb] += r * r;
      }
      if (need_mask) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int s = s0 + 32 * sb + 8 * i + 4 * hh + r;
            if (s > tl || s >= Tn) sc[sb][4 * i + r] = 0.f;
          }
      }
    }
#pragma unroll
    for (int ks4 = 0; ks4 < 4; ++ks4) {
      const v8_t<T> pb = c_to_b<T>(sc[ks4 >> 1], ks4 & 1);
      dpart = sum8<T>(pb, dpart);
#pragma unroll
      for (int db = 0; db < DV / 32; ++db)
        oacc[db] = mma(tile_tr8<T>(Vs, 32 * (ks4 >> 1), 32 * db, ks4 & 1, lane), pb, oacc[db]);
    }
  }

  const float dsum = dpart + __shfl_xor(dpart, 32);
  if (tvalid) {
    const float dsc = fmaxf(dsum * a.scale2, a.eps);
    const float inv = a.scale2 / dsc;
    T* orow = (T*)a.o + (int64_t)b * a.osb + (int64_t)tl * a.ost + (int64_t)h * a.osh;
#pragma unroll
    for (int db = 0; db < DV / 32; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st4<T>(orow + 32 * db + 8 * i + 4 * hh,
               to4<T>(oacc[db][4 * i] * inv, oacc[db][4 * i + 1] * inv, oacc[db][4 * i + 2] * inv,
                      oacc[db][4 * i + 3] * inv));
    if (hh == 0) a.den[(int64_t)b * a.dsb + (int64_t)tl * a.dst + (int64_t)h * a.dsh] = dsc;
  }
}

// n floats from src to dst (the packed layout's aliased z_in, handed to the
// scan as a copy)
__global__ __launch_bounds__(256) void kata_copy_f32_kernel(const float* __restrict__ src,
                                                            float* __restrict__ dst, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    dst[i] = src[i];
}

hipError_t launch_f32_copy(const float* src, float* dst, int64_t n, hipStream_t stream) {
  const int64_t blocks = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
  if (blocks > 0) kata_copy_f32_kernel<<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(src, dst, n);
  return hipGetLastError();
}

template <typename T, int DK, int DV, int M>
hipError_t launch_kata_prefill(const KataStateArgs& a, hipStream_t stream) {
  constexpr int E = DK / M, P = M * E * E;
  const int BH = a.B * a.H;
  kata_seg_state_kernel<T, DK, DV, M><<<dim3(BH * a.nseg * (M * kPkRows<E> / 768)), dim3(512), 0, stream>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t items = (int64_t)BH * (DV * (M * kPkRows<E> / 4) + P / 4);
  kata_seg_scan_kernel<T, DK, DV, M><<<dim3((unsigned)((items + 255) / 256)), dim3(256), 0, stream>>>(a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int nqt = (a.T + 127) / 128;
  kata_prefill_out_kernel<T, DK, DV, M><<<dim3(nqt * BH), dim3(256), 0, stream>>>(a, nqt, BH);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Decode step: one workgroup per (b, h) streams its (P x DV) f32 state once:
//   S += psi(k) v^T, z += psi(k);  o = psi(q)^T S / max(psi(q).z, eps)
// with psi(x)_p = scale x_a x_b.  16 threads cover one state row (4 value
// columns each), 16 rows per pass.  TRI: the packed state, one row per
// unordered pair (a <= b, kata_state_tri_row), whose readout weight is 2 off
// the diagonal; it moves M E (E + 1) / 2 rows instead of M E^2.
// ---------------------------------------------------------------------------
template <typename T, int DK, int DV, int M, bool TRI>
__global__ __launch_bounds__(256) void kata_decode_kernel(KataDecodeArgs a) {
  constexpr int E = DK / M, P = M * E * E, PT = M * E * (E + 1) / 2;
  constexpr int NR = TRI ? PT : P;  // state rows
  static_assert(DV == 64, "decode maps 16 threads x 4 columns onto a row");
  static_assert(DK <= 256, "8-bit dims in the pair table");
  __shared__ float qs[DK], ks[DK], vs[DV];
  __shared__ float4 red[16][16];
  __shared__ float dred[16];
  __shared__ unsigned short pairs[TRI ? PT : 1];  // packed row -> (dim a << 8) | dim b
  const int tid = threadIdx.x;
  const int bh = blockIdx.x, sp = blockIdx.y;
  // this workgroup's rows [p_lo, p_hi) of the a.nsplit runs (multiples of 16)
  const int run = ((NR + a.nsplit - 1) / a.nsplit + 15) & ~15;
  const int p_lo = sp * run, p_hi = min(NR, p_lo + run);
  if (tid < DK) {
    qs[tid] = (float)((const T*)a.q)[(size_t)bh * DK + tid];
    ks[tid] = (float)((const T*)a.k)[(size_t)bh * DK + tid];
  }
  if (tid < DV) vs[tid] = (float)((const T*)a.v)[(size_t)bh * DV + tid];
  if constexpr (TRI) {
    for (int t = p_lo + tid; t < p_hi; t += 256) {
      const int g = t / (E * (E + 1) / 2);
      int za = 0, r = t % (E * (E + 1) / 2);
      while (r >= E - za) {
        r -= E - za;
        ++za;
      }
      pairs[t] = (unsigned short)(((g * E + za) << 8) | (g * E + za + r));
    }
  }
  __syncthreads();
  const int c4 = tid & 15, r = tid >> 4;
  const float4 vv = *reinterpret_cast<const float4*>(vs + 4 * c4);
  float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
  float dacc = 0.f;
  float* S = a.S + (size_t)bh * NR * DV;
  float* z = a.z + (size_t)bh * NR;
  for (int p = p_lo + r; p < p_hi; p += 16) {
    int ia, ib;
    float wq = a.scale;
    if constexpr (TRI) {
      const unsigned pr = pairs[p];
      ia = (int)(pr >> 8);
      ib = (int)(pr & 255u);
      if (ia != ib) wq *= 2.f;
    } else {
      const int g = p / (E * E);
      ia = g * E + (p / E) % E;
      ib = g * E + p % E;
    }
    const float pk = a.scale * ks[ia] * ks[ib];
    const float pq = wq * qs[ia] * qs[ib];
    float4* sp = reinterpret_cast<float4*>(S + (size_t)p * DV + 4 * c4);
    float4 x = *sp;
    x.x += pk * vv.x; x.y += pk * vv.y; x.z += pk * vv.z; x.w += pk * vv.w;
    *sp = x;
    num.x += pq * x.x; num.y += pq * x.y; num.z += pq * x.z; num.w += pq * x.w;
    if (c4 == 0) {
      const float zz = z[p] + pk;
      z[p] = zz;
      dacc += pq * zz;
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
    if (a.nsplit == 1) {
      const float inv = 1.f / fmaxf(d, a.eps);
      st4<T>((T*)a.o + (size_t)bh * DV + 4 * tid, to4<T>(s.x * inv, s.y * inv, s.z * inv, s.w * inv));
    } else {
      float* pt = a.part + ((size_t)bh * a.nsplit + sp) * kGenDecPart;
      *reinterpret_cast<float4*>(pt + 4 * tid) = s;
      if (tid == 0) pt[DV] = d;
    }
  }
}

// A split decode step's output: per (b, h), the partials of its a.nsplit
// workgroups added in split order, o = num / max(den, eps).
template <typename T>
__global__ __launch_bounds__(64) void kata_decode_finish_kernel(KataDecodeArgs a) {
  const int bh = blockIdx.x, n = threadIdx.x;
  const float* pt = a.part + (size_t)bh * a.nsplit * kGenDecPart;
  float num = 0.f, den = 0.f;
  for (int s = 0; s < a.nsplit; ++s) {
    num += pt[s * kGenDecPart + n];
    den += pt[s * kGenDecPart + 64];
  }
  reinterpret_cast<T*>(a.o)[(size_t)bh * 64 + n] = (T)(num / fmaxf(den, a.eps));
}

template <typename T, int DK, int DV, int M>
hipError_t launch_kata_decode(const KataDecodeArgs& a, hipStream_t stream) {
  if (a.tri)
    kata_decode_kernel<T, DK, DV, M, true><<<dim3(a.B * a.H, a.nsplit), dim3(256), 0, stream>>>(a);
  else
    kata_decode_kernel<T, DK, DV, M, false><<<dim3(a.B * a.H, a.nsplit), dim3(256), 0, stream>>>(a);
  if (a.nsplit > 1) kata_decode_finish_kernel<T><<<dim3(a.B * a.H), dim3(64), 0, stream>>>(a);
  return hipGetLastError();
}

#define LINATT_STATE_INST(T, DK, DV, M)                                              \
  template hipError_t launch_kata_prefill<T, DK, DV, M>(const KataStateArgs&, hipStream_t); \
  template hipError_t launch_kata_decode<T, DK, DV, M>(const KataDecodeArgs&, hipStream_t);

LINATT_KATA_STATE_SHAPES(LINATT_STATE_INST)

}  // namespace linatt
