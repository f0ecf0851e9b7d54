// KATA-SPD causal attention forward for gfx950.
//
// Replaces the reference's parallel_kata_attn_fwd_kernel and
// parallel_kata_attn_sum_fwd_kernel (kata/kernels/parallel_kata.py:8-197,
// 200-345), launched from parallel_kata_attn_fwd_impl /
// parallel_kata_attn_sum_fwd_impl (kata/parallel_kata_attn.py:211-288,
// 539-576).
//
//   A[t,s] = sum_g (q_g[t].k_g[s])^2          (concat)
//          = sum_{i,j} (q_i[t].k_j[s])^2      (sum)
//            [* exp(min(c_t - c_s, 0))]        (decay)
//   o[t]   = sum_{s<=t} A[t,s] v[s] / den[t],  den[t] = scale^2 * sum_{s<=t} A[t,s]
//
// scale^2 is folded into den only: o is scale-invariant.  Where den is not
// positive the output row is left unnormalised (the reference's safe divide).
// den is accumulated from the weights as rounded for the P.V product
// (v.dtype, as the reference's b_scores.to(b_v.dtype)); it differs from the
// fp32 sum by at most one rounding unit of that type.
//
// Work split: a workgroup owns 128 queries of one (batch, query head); each
// of its four waves owns 32 queries.  Key tiles of 64 rows stream through
// LDS: K in natural layout (A operand of S^T = K Q^T), V transposed (A
// operand of O^T = V^T P^T).  Q^T stays in registers as the B operand, so
// the score block comes out in C layout with one query per lane column and
// goes back into the P.V product without leaving registers.
#include "common.h"
#include "kata_kernels.h"

namespace linatt {

template <typename T, int DK, int DV, int M, bool SUM, bool DECAY>
__global__ __launch_bounds__(256, sizeof(T) == 2 ? 2 : 1) void kata_fwd_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const float* __restrict__ c, T* __restrict__ o, float* __restrict__ den,
    int Tn, int HQ, int H, float scale2, int nqt, int nbh) {
  constexpr int E = DK / M;
  constexpr int KE = E / 16;           // 16-wide k-steps per group
  constexpr int KP = DK + (sizeof(T) == 2 ? 8 : 4);   // K tile pitch
  constexpr int VP = 64 + (sizeof(T) == 2 ? 4 : 4);   // V^T tile pitch
  static_assert(E % 16 == 0 && DV % 32 == 0, "unsupported head shape");
  __shared__ __attribute__((aligned(16))) T Ks[64 * KP];
  __shared__ __attribute__((aligned(16))) T Vt[DV * VP];
  __shared__ __attribute__((aligned(16))) float Cs[64];

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  int qt, bh;
  map_block(blockIdx.x, nqt, nbh, qt, bh, true);
  const int b = bh / HQ, hq = bh % HQ;
  const int G = HQ / H, h = hq / G;
  const int t0 = qt * 128;
  const int tw = t0 + 32 * w;
  const int tl = tw + cl;

  const int64_t qs = (int64_t)HQ * DK, ks = (int64_t)H * DK, vs = (int64_t)H * DV;
  const T* qb = q + ((int64_t)b * Tn) * qs + (int64_t)hq * DK;
  const T* kb = k + ((int64_t)b * Tn) * ks + (int64_t)h * DK;
  const T* vb = v + ((int64_t)b * Tn) * vs + (int64_t)h * DV;

  // Q^T as B operands: lane (column tl) holds q[tl][16kk + 8hh .. +7].
  v8_t<T> qop[DK / 16];
#pragma unroll
  for (int kk = 0; kk < DK / 16; ++kk)
    qop[kk] = (tl < Tn) ? ld8<T>(qb + (int64_t)tl * qs + 16 * kk + 8 * hh) : zero8<T>();
  float ct = 0.f;
  if constexpr (DECAY) ct = (tl < Tn) ? c[((int64_t)b * Tn + tl) * HQ + hq] : 0.f;

  f32x16 oacc[DV / 32];
#pragma unroll
  for (int db = 0; db < DV / 32; ++db) oacc[db] = f32x16{};
  float dpart = 0.f;
  // fp16 only: the weights of query tl are multiplied by the power of two pe
  // that puts the running row maximum in [2^11, 2^12) before rounding, so
  // small weights stay out of fp16's subnormal range; oacc and dpart are
  // rescaled (exactly) whenever pe changes, and pe cancels in o.
  constexpr bool kRescale = __is_same(T, _Float16);
  float pe = 1.f, mrun = 0.f;

  const int s_end = min(t0 + 128, Tn);
  const int nst = (s_end + 63) / 64;
  for (int st = 0; st < nst; ++st) {
    const int s0 = st * 64;
    __syncthreads();
    load_tile64<T, DK, KP, 1, true, false>(kb, s0, Tn, ks, Ks, nullptr, tid);
    load_tile64<T, DV, 1, VP, false, true>(vb, s0, Tn, vs, nullptr, Vt, tid);
    if constexpr (DECAY) {
      if (tid < 64) Cs[tid] = (s0 + tid < Tn) ? c[((int64_t)b * Tn + s0 + tid) * HQ + hq] : 0.f;
    }
    __syncthreads();
    if (s0 > tw + 31 || tw >= Tn) continue;  // whole tile after this wave's queries
    const bool need_mask = (s0 + 63 > tw) || (s0 + 64 > Tn);

    f32x16 a[2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      a[sb] = f32x16{};
      const T* krow = Ks + (32 * sb + cl) * KP + 8 * hh;
      if constexpr (!SUM) {
#pragma unroll
        for (int g = 0; g < M; ++g) {
          f32x16 r{};
#pragma unroll
          for (int kk = 0; kk < KE; ++kk)
            r = mma(ld8<T>(krow + g * E + 16 * kk), qop[g * KE + kk], r);
          a[sb] += r * r;
        }
      } else {
#pragma unroll
        for (int gi = 0; gi < M; ++gi) {
#pragma unroll
          for (int gj = 0; gj < M; ++gj) {
            f32x16 r{};
#pragma unroll
            for (int kk = 0; kk < KE; ++kk)
              r = mma(ld8<T>(krow + gj * E + 16 * kk), qop[gi * KE + kk], r);
            a[sb] += r * r;
          }
        }
      }
      // element 4i+r of block sb is key s0 + 32sb + 8i + 4hh + r, query tl
      if constexpr (DECAY) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4 cs = *reinterpret_cast<const f32x4*>(Cs + 32 * sb + 8 * i + 4 * hh);
#pragma unroll
          for (int r = 0; r < 4; ++r) a[sb][4 * i + r] *= __expf(fminf(ct - cs[r], 0.f));
        }
      }
      if (need_mask) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int s = s0 + 32 * sb + 8 * i + 4 * hh + r;
            if (s > tl || s >= Tn) a[sb][4 * i + r] = 0.f;
          }
      }
    }

    if constexpr (kRescale) {
      float mx = 0.f;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, a[sb][e]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      if (mx > mrun) {
        int ex;
        frexpf(mx, &ex);
        const float pnew = ldexpf(1.f, 12 - max(ex, -100));
        const float ratio = pnew / pe;
#pragma unroll
        for (int db = 0; db < DV / 32; ++db) oacc[db] *= ratio;
        dpart *= ratio;
        pe = pnew;
        mrun = mx;
      }
      a[0] *= pe;
      a[1] *= pe;
    }

    // O^T[dv][t] += sum_s V^T[dv][s] P^T[s][t].  den sums the same rounded
    // weights the product uses, so every output row is an exact convex
    // combination of v rows (a lone key gives o = v exactly).
#pragma unroll
    for (int ks4 = 0; ks4 < 4; ++ks4) {
      const v8_t<T> pb = c_to_b<T>(a[ks4 >> 1], ks4 & 1);
      dpart = sum8<T>(pb, dpart);
#pragma unroll
      for (int db = 0; db < DV / 32; ++db) {
        const T* vrow = Vt + (32 * db + cl) * VP + 32 * (ks4 >> 1);
        oacc[db] = mma(ld_tr_op<T>(vrow, ks4 & 1, hh), pb, oacc[db]);
      }
    }
  }

  const float dsum = dpart + __shfl_xor(dpart, 32);
  if (tl < Tn) {
    const float inv = dsum > 0.f ? 1.f / dsum : 1.f;
    T* orow = o + (((int64_t)b * Tn + tl) * HQ + hq) * DV;
#pragma unroll
    for (int db = 0; db < DV / 32; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st4<T>(orow + 32 * db + 8 * i + 4 * hh,
               to4<T>(oacc[db][4 * i] * inv, oacc[db][4 * i + 1] * inv,
                      oacc[db][4 * i + 2] * inv, oacc[db][4 * i + 3] * inv));
    if (hh == 0) den[((int64_t)b * Tn + tl) * HQ + hq] = dsum * (scale2 / pe);
  }
}

// 16-bit inputs: the same computation with the key tiles brought in by
// direct global->LDS copies through a three-slot ring (tiles st + 1 and
// st + 2 in flight while tile st computes, one barrier per tile) and stored
// swizzled in natural layout: K feeds the score MFMAs with 16-byte reads and
// V^T comes from V through transposing LDS reads, so no transposed copy is
// built.  Rows past T repeat the last valid row and are masked.  The loop is
// unrolled over the ring so every LDS operand address is a per-lane offset
// fixed for the kernel plus an immediate, and full tiles are copied from a
// scalar base: the VALU, which bounds this kernel, only does the math.
// EPI: 0 writes o; 1 also the output RMSNorm's y and rstd; 2 the float32
// numerator o den instead of o (compile-time, so each variant carries only
// its own epilogue).  Three waves per SIMD at dk = 64 (at most 168 VGPRs;
// the compiler otherwise lets some variants grow just past it)
template <typename T, int DK, int DV, int M, bool SUM, bool DECAY, int EPI>
__global__ __launch_bounds__(256, DK == 64 ? 3 : 2) void kata_fwd_tile_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const float* __restrict__ c, T* __restrict__ o, float* __restrict__ den,
    int Tn, int HQ, int H, float scale2, int nqt, int nbh, OutNorm on) {
  constexpr int E = DK / M;
  constexpr int KE = E / 16;
  static_assert(sizeof(T) == 2 && (DK == 64 || DK == 128) && DV == 64, "64 x 64 16-bit tiles");
  constexpr int NB = 3;
  constexpr int KT = DK / 64;  // key tiles as KT 64 x 64 sub-tiles (wtile_ld8)
  __shared__ __attribute__((aligned(16))) T Kb[NB][KT * 64 * 64];
  __shared__ __attribute__((aligned(16))) T Vb[NB][64 * 64];
  __shared__ __attribute__((aligned(16))) float Cs[NB][64];

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  int qt, bh;
  map_block(blockIdx.x, nqt, nbh, qt, bh, true);
  const int b = bh / HQ, hq = bh % HQ;
  const int G = HQ / H, h = hq / G;
  const int t0 = qt * 128;
  const int tw = t0 + 32 * w;
  const int tl = tw + cl;

  const int64_t qs = (int64_t)HQ * DK, ks = (int64_t)H * DK, vs = (int64_t)H * DV;
  const T* qb = q + ((int64_t)b * Tn) * qs + (int64_t)hq * DK;
  const T* kb = k + ((int64_t)b * Tn) * ks + (int64_t)h * DK;
  const T* vb = v + ((int64_t)b * Tn) * vs + (int64_t)h * DV;

  v8_t<T> qop[DK / 16];
#pragma unroll
  for (int kk = 0; kk < DK / 16; ++kk)
    qop[kk] = (tl < Tn) ? ld8<T>(qb + (int64_t)tl * qs + 16 * kk + 8 * hh) : zero8<T>();
  float ct = 0.f;
  if constexpr (DECAY) ct = (tl < Tn) ? c[((int64_t)b * Tn + tl) * HQ + hq] : 0.f;

  f32x16 oacc[DV / 32];
#pragma unroll
  for (int db = 0; db < DV / 32; ++db) oacc[db] = f32x16{};
  float dpart = 0.f;
  constexpr bool kRescale = __is_same(T, _Float16);
  float pe = 1.f, mrun = 0.f;

  const int s_end = min(t0 + 128, Tn);
  const int nst = (s_end + 63) / 64;
  // tile st: 8 KiB of K and 8 KiB of V, copies 2w and 2w + 1 of each by wave w
  // (full tiles: scalar base + these per-lane offsets)
  unsigned ko[2], vo[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    ko[i] = tile_lane_off(2 * w + i, lane, (int)(ks * sizeof(T)));
    vo[i] = tile_lane_off(2 * w + i, lane, (int)(vs * sizeof(T)));
  }
  auto issue = [&](int st, auto slot) __attribute__((always_inline)) {
    constexpr int sl = decltype(slot)::value;
    if (64 * st + 64 <= Tn) {
      const T* kt = kb + (int64_t)64 * st * ks;
      const T* vt = vb + (int64_t)64 * st * vs;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < KT; ++j)
          dma16s(kt + 64 * j, ko[i], reinterpret_cast<char*>(Kb[sl] + 4096 * j) + 1024 * (2 * w + i));
        dma16s(vt, vo[i], reinterpret_cast<char*>(Vb[sl]) + 1024 * (2 * w + i));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < KT; ++j)
          dma_tile64<T>(kb + 64 * j, ks, 64 * st, Tn, Kb[sl] + 4096 * j, 2 * w + i, lane);
        dma_tile64<T>(vb, vs, 64 * st, Tn, Vb[sl], 2 * w + i, lane);
      }
    }
    // decay: c of the tile's keys (rows past T repeat the last one; masked)
    if constexpr (DECAY) {
      if (w == 0) dma4(c + ((int64_t)b * Tn + min(64 * st + lane, Tn - 1)) * HQ + hq, Cs[sl]);
    }
  };
  // copies per tile and wave: two of each K sub-tile, two of V, c by wave 0
  const int ops = 2 * KT + 2 + (DECAY && w == 0 ? 1 : 0);

  auto step = [&](int st, auto slot) __attribute__((always_inline)) {
    constexpr int buf = decltype(slot)::value;
    const int s0 = st * 64;
    // tile st landed (only tile st + 1's copies may be in flight) and every
    // wave passed tile st - 1, whose slot tile st + 2 takes
    vm_wait_barrier_n(st + 1 < nst ? ops : 0);
    if (st + 2 < nst) issue(st + 2, IntC<(buf + 2) % NB>{});
    const T* Ks = Kb[buf];
    const T* Vs = Vb[buf];
    if (s0 > tw + 31 || tw >= Tn) return;
    const bool need_mask = (s0 + 63 > tw) || (s0 + 64 > Tn);
    f32x16 a[2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      a[sb] = f32x16{};
      // a block of keys all after this wave's queries adds nothing
      if (s0 + 32 * sb > tw + 31) continue;
      const int krow = 32 * sb + cl;
      if constexpr (!SUM) {
#pragma unroll
        for (int g = 0; g < M; ++g) {
          f32x16 r{};
#pragma unroll
          for (int kk = 0; kk < KE; ++kk)
            r = mma(wtile_ld8<T>(Ks, krow, g * E + 16 * kk + 8 * hh), qop[g * KE + kk], r);
          a[sb] += r * r;
        }
      } else {
#pragma unroll
        for (int gi = 0; gi < M; ++gi) {
#pragma unroll
          for (int gj = 0; gj < M; ++gj) {
            f32x16 r{};
#pragma unroll
            for (int kk = 0; kk < KE; ++kk)
              r = mma(wtile_ld8<T>(Ks, krow, gj * E + 16 * kk + 8 * hh), qop[gi * KE + kk], r);
            a[sb] += r * r;
          }
        }
      }
      if constexpr (DECAY) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4 cs = *reinterpret_cast<const f32x4*>(&Cs[buf][32 * sb + 8 * i + 4 * hh]);
#pragma unroll
          for (int r = 0; r < 4; ++r) a[sb][4 * i + r] *= __expf(fminf(ct - cs[r], 0.f));
        }
      }
      if (need_mask) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int s = s0 + 32 * sb + 8 * i + 4 * hh + r;
            if (s > tl || s >= Tn) a[sb][4 * i + r] = 0.f;
          }
      }
    }
    if constexpr (kRescale) {
      float mx = 0.f;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, a[sb][e]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      if (mx > mrun) {
        int ex;
        frexpf(mx, &ex);
        const float pnew = ldexpf(1.f, 12 - max(ex, -100));
        const float ratio = pnew / pe;
#pragma unroll
        for (int db = 0; db < DV / 32; ++db) oacc[db] *= ratio;
        dpart *= ratio;
        pe = pnew;
        mrun = mx;
      }
      a[0] *= pe;
      a[1] *= pe;
    }
    // O^T[dv][t] += sum_s V^T[dv][s] P^T[s][t], V^T read transposed from V
#pragma unroll
    for (int ks4 = 0; ks4 < 4; ++ks4) {
      const v8_t<T> pb = c_to_b<T>(a[ks4 >> 1], ks4 & 1);
      dpart = sum8<T>(pb, dpart);
#pragma unroll
      for (int db = 0; db < DV / 32; ++db)
        oacc[db] = mma(tile_tr8<T>(Vs, 32 * (ks4 >> 1), 32 * db, ks4 & 1, lane), pb, oacc[db]);
    }
  };

  // concat, no decay, 16-bit without rescaling: key tiles wholly before the
  // workgroup's queries need no mask, and there the group score MFMAs run one
  // (block, group) unit ahead of the squares that consume them, with block
  // 0's P.V products issued under block 1's squares; the body is one basic
  // block
  auto step_plain = [&](int st, auto slot) __attribute__((always_inline)) {
    constexpr int buf = decltype(slot)::value;
    vm_wait_barrier_n(st + 1 < nst ? ops : 0);
    if (st + 2 < nst) issue(st + 2, IntC<(buf + 2) % NB>{});
    const T* Ks = Kb[buf];
    const T* Vs = Vb[buf];
    if (tw >= Tn) return;
    auto score = [&](int sb, int g) __attribute__((always_inline)) {
      f32x16 r{};
#pragma unroll
      for (int kk = 0; kk < KE; ++kk)
        r = mma(wtile_ld8<T>(Ks, 32 * sb + cl, g * E + 16 * kk + 8 * hh), qop[g * KE + kk], r);
      return r;
    };
    auto finish = [&](int sb, const f32x16& ab) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const v8_t<T> pb = c_to_b<T>(ab, j);
        dpart = sum8<T>(pb, dpart);
#pragma unroll
        for (int db = 0; db < DV / 32; ++db)
          oacc[db] = mma(tile_tr8<T>(Vs, 32 * sb, 32 * db, j, lane), pb, oacc[db]);
      }
    };
    if constexpr (M == 1) {
      // one group: its score is a chain of four MFMAs; running a second
      // block's chain ahead costs the registers of occupancy 3
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        const f32x16 r = score(sb, 0);
        finish(sb, r * r);
      }
    } else {
      f32x16 a0, a1;
      f32x16 rc = score(0, 0);
#pragma unroll
      for (int u = 1; u < 2 * M; ++u) {
        const f32x16 rn = score(u / M, u % M);
        const int pg = (u - 1) % M;
        if ((u - 1) / M == 0) {
          if (pg == 0) a0 = rc * rc; else a0 += rc * rc;
          if (pg == M - 1) finish(0, a0);
        } else {
          if (pg == 0) a1 = rc * rc; else a1 += rc * rc;
        }
        rc = rn;
      }
      a1 += rc * rc;
      finish(1, a1);
    }
  };

  vm_drain();  // q (and c) of this wave's queries are in registers
  issue(0, IntC<0>{});
  if (nst > 1) issue(1, IntC<1>{});
  constexpr bool kPlain = !SUM && !DECAY && !kRescale;
  int st = 0;
  if constexpr (kPlain) {
    // tiles wholly before this workgroup's first query, then the rest
    const int nplain = min(t0 / 64, nst);
    for (; st + NB <= nplain; st += NB) {
      step_plain(st, IntC<0>{});
      step_plain(st + 1, IntC<1>{});
      step_plain(st + 2, IntC<2>{});
    }
    if (st < nplain) step_plain(st++, IntC<0>{});
    if (st < nplain) step_plain(st++, IntC<1>{});
  }
  for (; st < nst; ++st) {
    switch (st % NB) {
      case 0: step(st, IntC<0>{}); break;
      case 1: step(st, IntC<1>{}); break;
      default: step(st, IntC<2>{}); break;
    }
  }

  const float dsum = dpart + __shfl_xor(dpart, 32);
  const float inv = dsum > 0.f ? 1.f / dsum : 1.f;
  // this lane's 32 elements of its query's output row (dims 32 db + 8 i +
  // 4 hh + r), rounded to T as stored
  v4_t<T> ov[DV / 32][4];
#pragma unroll
  for (int db = 0; db < DV / 32; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ov[db][i] = to4<T>(oacc[db][4 * i] * inv, oacc[db][4 * i + 1] * inv,
                         oacc[db][4 * i + 2] * inv, oacc[db][4 * i + 3] * inv);
  const int64_t row = ((int64_t)b * Tn + tl) * HQ + hq;
  if (tl < Tn) {
    if constexpr (EPI == 2) {
      // float32 numerator o den = oacc scale^2 / pe, unrounded
      const float f = scale2 / pe;
      float* nrow = on.num + row * DV;
#pragma unroll
      for (int db = 0; db < DV / 32; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<f32x4*>(nrow + 32 * db + 8 * i + 4 * hh) =
              f32x4{oacc[db][4 * i] * f, oacc[db][4 * i + 1] * f, oacc[db][4 * i + 2] * f,
                    oacc[db][4 * i + 3] * f};
    } else {
      T* orow = o + row * DV;
#pragma unroll
      for (int db = 0; db < DV / 32; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) st4<T>(orow + 32 * db + 8 * i + 4 * hh, ov[db][i]);
    }
    if (hh == 0) den[row] = dsum * (scale2 / pe);
  }
  // output RMSNorm (uniform branch): y = o rsqrt(mean(o^2) + eps) w over the
  // row of the stored (rounded) o, whose two halves are lanes l and l ^ 32
  if constexpr (EPI == 1) {
    float ss = 0.f;
#pragma unroll
    for (int db = 0; db < DV / 32; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) ss += (float)ov[db][i][r] * (float)ov[db][i][r];
    ss += __shfl_xor(ss, 32);
    const float rr = rsqrtf(ss / DV + on.eps);
    if (tl < Tn) {
      T* yrow = (T*)on.y + row * DV;
#pragma unroll
      for (int db = 0; db < DV / 32; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d0 = 32 * db + 8 * i + 4 * hh;
          const f32x4 w4 = on.w ? *reinterpret_cast<const f32x4*>(on.w + d0) : f32x4{1.f, 1.f, 1.f, 1.f};
          st4<T>(yrow + d0, to4<T>((float)ov[db][i][0] * (rr * w4[0]), (float)ov[db][i][1] * (rr * w4[1]),
                                   (float)ov[db][i][2] * (rr * w4[2]), (float)ov[db][i][3] * (rr * w4[3])));
        }
      if (hh == 0) on.rstd[row] = rr;
    }
  }
}

template <typename T, int DK, int DV, int M, bool SUM, bool DECAY>
hipError_t launch_kata_fwd(const KataArgs& a, hipStream_t stream) {
  if constexpr (SUM && M == 1) {
    // one group: the sum form sum_{g,g'} (q_g . k_g')^2 is the concat form
    // (q . k)^2, whose tile kernel has the pipelined body for unmasked tiles
    return launch_kata_fwd<T, DK, DV, M, false, DECAY>(a, stream);
  } else {
    const int nqt = (a.T + 127) / 128;
    const int nbh = a.B * a.HQ;
    dim3 grid(nqt * nbh), block(256);
    if constexpr (sizeof(T) == 2 && (DK == 64 || DK == 128) && DV == 64) {
      const OutNorm on{a.nw, a.y, a.rstd, nullptr, a.eps, a.num32};
      auto go = [&](auto epi) {
        kata_fwd_tile_kernel<T, DK, DV, M, SUM, DECAY, decltype(epi)::value><<<grid, block, 0, stream>>>(
            (const T*)a.q, (const T*)a.k, (const T*)a.v, a.c, (T*)a.o, a.den, a.T, a.HQ, a.H,
            a.scale * a.scale, nqt, nbh, on);
      };
      if (a.y && a.num32) return hipErrorInvalidValue;
      if (a.y) go(IntC<1>{});
      else if (a.num32) go(IntC<2>{});
      else go(IntC<0>{});
    } else {
      // the output norm and the float32 numerator are tile-kernel options
      if (a.y || a.num32) return hipErrorInvalidValue;
      kata_fwd_kernel<T, DK, DV, M, SUM, DECAY><<<grid, block, 0, stream>>>(
          (const T*)a.q, (const T*)a.k, (const T*)a.v, a.c, (T*)a.o, a.den, a.T, a.HQ, a.H,
          a.scale * a.scale, nqt, nbh);
    }
    return hipGetLastError();
  }
}

#define LINATT_FWD_INST(T, DK, DV, M)                                                  \
  template hipError_t launch_kata_fwd<T, DK, DV, M, false, false>(const KataArgs&, hipStream_t); \
  template hipError_t launch_kata_fwd<T, DK, DV, M, true, false>(const KataArgs&, hipStream_t);  \
  template hipError_t launch_kata_fwd<T, DK, DV, M, false, true>(const KataArgs&, hipStream_t);

LINATT_KATA_SHAPES(LINATT_FWD_INST)

}  // namespace linatt
