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
// The kernels (the state is fp32 (B, H, P, 64)):
//   kata_gen_decode_kernel   one token per (b, h): S, z updated in place, o
//   kata_gen_readout_kernel  a prefill continued from a state: the flash
//                            forward's (o, den) over the call's tokens plus
//                            f_t psi(q_t)^T S and f_t psi(q_t) . z
//   kata_gen_update_kernel   S <- f_T S + sum_s f_Ts psi(k_s) v_s^T (and z)
// The readout and the update are fp32 VALU kernels for fp32 inputs; 16-bit
// inputs take kata_gen_readout_mfma_kernel / kata_gen_update_mfma_kernel,
// whose products psi . S and psi v^T run on the matrix cores with bf16
// operands (psi formed in fp32, then rounded; S rounded for the readout) and
// fp32 sums, z and den in fp32.  The decode step is fp32 throughout.
// The concat score without decay at (dk, M) = (64, 2), (64, 4) keeps its
// MFMA state-form kernels (kata_state.hip); these cover the rest.
#include <type_traits>

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

// One workgroup per (b, h) and split (blockIdx.y of a.nsplit, each a run of
// rows); 16 threads per state row (4 value columns each), 16 rows per pass;
// q, k (B, H, dk), v, o (B, H, 64); c (B, H) the step's log-decay or null.
// With one split the workgroup writes o; with more, each writes its partial
// numerator and denominator to a.part and kata_gen_decode_finish_kernel adds
// them in split order (a small batch then fills the chip: its rows are few
// workgroups' dependent loads otherwise).  The packed layout's rows are mapped to their dimensions
// once per workgroup into an LDS table (dims < 256: 8 bits each), not by
// each of a row's 16 threads.
constexpr int kMaxPackedRows = 128 * 129 / 2;  // dk <= 128, one group of 128

template <typename T>
__global__ __launch_bounds__(256) void kata_gen_decode_kernel(KataGenStateArgs a) {
  __shared__ float qs[128], ks[128], vs[kGenDV];
  __shared__ float4 red[16][16];
  __shared__ float dred[16];
  __shared__ unsigned short pairs[kMaxPackedRows];
  const int tid = threadIdx.x, bh = blockIdx.x, sp = blockIdx.y;
  // this workgroup's rows [p_lo, p_hi): runs of a multiple of 16 rows
  const int run = ((a.P + a.nsplit - 1) / a.nsplit + 15) & ~15;
  const int p_lo = sp * run, p_hi = min(a.P, p_lo + run);
  if (tid < a.dk) {
    qs[tid] = ldf<T>(a.q, (int64_t)bh * a.dk + tid);
    ks[tid] = ldf<T>(a.k, (int64_t)bh * a.dk + tid);
  }
  if (tid < kGenDV) vs[tid] = ldf<T>(a.v, (int64_t)bh * kGenDV + tid);
  if (a.tri) {
    for (int p = p_lo + tid; p < p_hi; p += 256) {
      const RowPair rp = row_pair(a, p);
      pairs[p] = (unsigned short)(((rp.g * a.E + rp.a) << 8) | (rp.g * a.E + rp.b));
    }
  }
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
  for (int p0 = p_lo + r; p0 < p_hi; p0 += 16 * kDecU) {
    float4 xs[kDecU];
    float zs[kDecU];
#pragma unroll
    for (int u = 0; u < kDecU; ++u) {
      const int p = p0 + 16 * u;
      xs[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      zs[u] = 0.f;
      if (p < p_hi) {
        xs[u] = *reinterpret_cast<const float4*>(S + (size_t)p * kGenDV + 4 * c4);
        if (c4 == 0) zs[u] = z[p];
      }
    }
#pragma unroll
    for (int u = 0; u < kDecU; ++u) {
      const int p = p0 + 16 * u;
      if (p >= p_hi) break;
      RowPair rp;
      if (a.tri) {
        const unsigned pr = pairs[p];
        rp.g = 0;  // the group is folded into the dimensions
        rp.a = (int)(pr >> 8);
        rp.b = (int)(pr & 255u);
        rp.w = rp.a == rp.b ? 1.f : 2.f;
      } else {
        rp = row_pair(a, p);
      }
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
    if (a.nsplit == 1) {
      const float inv = 1.f / fmaxf(d, a.eps);
      st4<T>((T*)a.o + (size_t)bh * kGenDV + 4 * tid, to4<T>(s.x * inv, s.y * inv, s.z * inv, s.w * inv));
    } else {
      float* pt = a.part + ((size_t)bh * a.nsplit + sp) * kGenDecPart;
      *reinterpret_cast<float4*>(pt + 4 * tid) = s;
      if (tid == 0) pt[kGenDV] = d;
    }
  }
}

// The split decode step's output: per (b, h), the partials of its a.nsplit
// workgroups added in split order, o = num / max(den, eps).
template <typename T>
__global__ __launch_bounds__(64) void kata_gen_decode_finish_kernel(KataGenStateArgs a) {
  const int bh = blockIdx.x, n = threadIdx.x;
  const float* pt = a.part + (size_t)bh * a.nsplit * kGenDecPart;
  float num = 0.f, den = 0.f;
  for (int s = 0; s < a.nsplit; ++s) {
    num += pt[s * kGenDecPart + n];
    den += pt[s * kGenDecPart + kGenDV];
  }
  reinterpret_cast<T*>(a.o)[(size_t)bh * kGenDV + n] = (T)(num / fmaxf(den, a.eps));
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

// State update for 16-bit inputs, by MFMA: per (b, h, 128 RB state rows),
// four waves of RB 32-row blocks, and NCB of the two 32-column halves of the
// state (NCB = 1: blockIdx.z picks the half; a small state takes RB = 1,
// NCB = 1, so that more workgroups share it).  Tokens stream through LDS 64 at
// a time, the next 64's global loads in flight while the current ones are used:
//   Kt[d][s] = sqrt(scale f_Ts) k_s[d]  (fp32, dimension-major),
//   Vt[n][s] = v_s[n]                   (bf16, column-major).
// Lane l of a wave forms, for each of its rows p (l % 32 of a block) and the
// tokens 8 (l / 32) + 0..7 of each 16-token step, the features
// scale f_Ts k_s[a] k_s[b] = Kt[a][s] Kt[b][s] (the sum score: summed over
// the groups) in fp32, rounded to bf16 as the A operand of
// v_mfma_f32_32x32x16_bf16; the 32-column halves of Vt are the B operands,
// shared by the row blocks.  z sums the fp32 features per lane (the two lane
// halves are added at the end; with NCB = 1 the first half's workgroup
// stores it).  Staging moves token pairs: one 8-byte LDS write per
// (dimension, pair) of K, one 4-byte write per (column, pair) of V, the 32
// pairs of a chunk on consecutive lanes so that each write instruction covers
// consecutive banks (a mapping with the dimensions on consecutive lanes put
// eight lanes on two bank offsets; SQ counters showed 5 to 8 conflict cycles
// per LDS instruction).  Vt's 16-byte chunks are XOR-swizzled by bit 4 of the
// column, so the B-operand reads of columns 16 apart (same banks at the
// 144-byte pitch) fall on different banks.
//   S <- (init ? f_T S : 0) + sum_s f_Ts psi(k_s) v_s^T,  z likewise.
constexpr int kUpTok = 64, kUpKp = kUpTok + 4, kUpVp = kUpTok + 8;

template <typename T, int MS, int RB, int NCB>
__global__ __launch_bounds__(256) void kata_gen_update_mfma_kernel(KataGenStateArgs a) {
  // MS: the sum score's groups (0: the concat score, -1: the sum score over
  // a.M groups, counted at run time)
  constexpr bool SUM = MS != 0;
  static_assert(sizeof(T) == 2, "16-bit inputs");
  __shared__ __attribute__((aligned(16))) float Kt[128][kUpKp];
  __shared__ __attribute__((aligned(16))) __bf16 Vt[32 * NCB][kUpVp];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hh = lane >> 5, cl = lane & 31;
  const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
  const int n0c = NCB == 2 ? 0 : 32 * blockIdx.z;  // first state column of this workgroup
  const int pw = blockIdx.y * 128 * RB + 32 * RB * w;  // this wave's first row
  const bool wlive = pw < a.P;
  int ia[RB], ib[RB];
  bool live[RB];
#pragma unroll
  for (int k = 0; k < RB; ++k) {
    const int p = pw + 32 * k + cl;
    live[k] = p < a.P;
    const RowPair rp = row_pair(a, live[k] ? p : 0);
    ia[k] = rp.g * a.E + rp.a;
    ib[k] = rp.g * a.E + rp.b;
  }
  const float cT = a.c ? a.c[((int64_t)b * a.T + a.T - 1) * a.H + h] : 0.f;
  const int dk8 = a.dk >> 3;
  const T* kg = reinterpret_cast<const T*>(a.k);
  const T* vg = reinterpret_cast<const T*>(a.v);

  // prefetch registers: K items (token pair, 8 dimensions), up to two per
  // thread (32 pairs x dk / 8 / 256 threads at dk = 128); one V item (token
  // pair, 8 columns; the first 128 threads when NCB = 1), one chunk ahead
  // (two chunks ahead measured no faster at 44 more registers)
  struct Pf {
    v8_t<T> kr[2][2], vr[2];
    float kc[2][2];
  };
  Pf pf;
  auto load = [&](Pf& f, int s0) __attribute__((always_inline)) {
    auto& kr = f.kr;
    auto& vr = f.vr;
    auto& kc = f.kc;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int i = tid + 256 * it, sp = i & 31, d0 = 8 * (i >> 5);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int t = s0 + 2 * sp + u;
        kr[it][u] = zero8<T>();
        kc[it][u] = 0.f;
        if (i < (kUpTok / 2) * dk8 && t < a.T) {
          const int64_t row = ((int64_t)b * a.T + t) * a.H + h;
          kr[it][u] = ld8<T>(kg + row * a.dk + d0);
          kc[it][u] = a.c ? a.c[row] : 0.f;
        }
      }
    }
    const int sp = tid & 31, n0 = 8 * (tid >> 5);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = s0 + 2 * sp + u;
      vr[u] = n0 < 32 * NCB && t < a.T ? ld8<T>(vg + (((int64_t)b * a.T + t) * a.H + h) * kGenDV + n0c + n0)
                                          : zero8<T>();
    }
  };
  auto stage = [&](const Pf& f, int s0) __attribute__((always_inline)) {
    const auto& kr = f.kr;
    const auto& vr = f.vr;
    const auto& kc = f.kc;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int i = tid + 256 * it;
      if (i < (kUpTok / 2) * dk8) {
        const int sp = i & 31, d0 = 8 * (i >> 5);
        float fs[2];
#pragma unroll
        for (int u = 0; u < 2; ++u)
          fs[u] = s0 + 2 * sp + u < a.T ? sqrtf(a.scale * (a.c ? __expf(cT - kc[it][u]) : 1.f)) : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          *reinterpret_cast<float2*>(&Kt[d0 + j][2 * sp]) =
              make_float2((float)kr[it][0][j] * fs[0], (float)kr[it][1][j] * fs[1]);
      }
    }
    const int sp = tid & 31, n0 = 8 * (tid >> 5);
    if (n0 < 32 * NCB) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        const int n = n0 + j;
        *reinterpret_cast<bf16x2*>(&Vt[n][(2 * sp) ^ (8 * ((n >> 4) & 1))]) =
            bf16x2{(__bf16)(float)vr[0][j], (__bf16)(float)vr[1][j]};
      }
    }
  };
  auto features = [&](int k, int sb) __attribute__((always_inline)) {
    f32x8 fe{};
#pragma unroll
    for (int g = 0; g < (MS > 0 ? MS : MS < 0 ? a.M : 1); ++g) {
      const float* ra = &Kt[ia[k] + g * a.E][sb];
      const float* rb = &Kt[ib[k] + g * a.E][sb];
      const f32x4 a0 = *reinterpret_cast<const f32x4*>(ra), a1 = *reinterpret_cast<const f32x4*>(ra + 4);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(rb), b1 = *reinterpret_cast<const f32x4*>(rb + 4);
      fe += f32x8{a0[0] * b0[0], a0[1] * b0[1], a0[2] * b0[2], a0[3] * b0[3],
                  a1[0] * b1[0], a1[1] * b1[1], a1[2] * b1[2], a1[3] * b1[3]};
    }
    // a row past P (its (a, b) those of row 0) is neither stored nor added
    // to z, so its features need no mask
    return fe;
  };

  f32x16 acc[RB][NCB] = {};
  float zacc[RB] = {};
  auto compute = [&]() __attribute__((always_inline)) {
    if (wlive) {
#pragma unroll
      for (int kk = 0; kk < kUpTok / 16; ++kk) {
        const int sb = 16 * kk + 8 * hh;
        bf16x8 Bv[NCB];
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
          Bv[cb] = *reinterpret_cast<const bf16x8*>(&Vt[32 * cb + cl][sb ^ (8 * ((cl >> 4) & 1))]);
#pragma unroll
        for (int k = 0; k < RB; ++k) {
          const f32x8 fe = features(k, sb);
          zacc[k] += ((fe[0] + fe[1]) + (fe[2] + fe[3])) + ((fe[4] + fe[5]) + (fe[6] + fe[7]));
          const bf16x8 A = __builtin_convertvector(fe, bf16x8);
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) acc[k][cb] = mma(A, Bv[cb], acc[k][cb]);
        }
      }
    }
  };
  load(pf, 0);
  for (int s0 = 0; s0 < a.T; s0 += kUpTok) {
    __syncthreads();  // the previous tokens are consumed
    stage(pf, s0);
    __syncthreads();
    if (s0 + kUpTok < a.T) load(pf, s0 + kUpTok);
    compute();
  }
  if (!wlive) return;
  const float fT = a.c ? __expf(cT) : 1.f;
  float* S = a.S + (size_t)bh * a.P * kGenDV;
  float* z = a.z + (size_t)bh * a.P;
#pragma unroll
  for (int k = 0; k < RB; ++k) {
    zacc[k] += __shfl_xor(zacc[k], 32);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int p = pw + 32 * k + 8 * i + 4 * hh + r;
        if (p < a.P) {
          float* sp = S + (size_t)p * kGenDV + n0c;
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) {
            float x = acc[k][cb][4 * i + r];
            if (a.init) x += fT * sp[32 * cb + cl];
            sp[32 * cb + cl] = x;
          }
        }
      }
    const int p = pw + 32 * k + cl;
    if (hh == 0 && live[k] && n0c == 0) z[p] = (a.init ? fT * z[p] : 0.f) + zacc[k];
  }
}

// Continued prefill's state part for 16-bit inputs, by MFMA: per (b, h, 128
// queries), four waves of 32 queries.  The queries sit in LDS as fp32
// q~ = sqrt(scale) q.  The state rows are taken in chunks of 16 with one
// first index a and consecutive second indices b = 16 j .. 16 j + 15 of a
// group g: the full layout's rows in order; for the packed layout every
// (a, j) with 16 j + 15 >= a, the rows b < a of such a chunk being zero.  So
// lane l of a wave forms, for its query t (l % 32) and the rows
// 8 (l / 32) + 0..7 of a chunk, the features q~_t[gE + a] q~_t[gE + b] from
// one scalar and two 16-byte LDS reads (summed over the groups for the sum
// score), in fp32, rounded to bf16 as the A operand of
// v_mfma_f32_32x32x16_bf16.  Per four chunks the workgroup stages
//   Bt[n][r] = w_r S[row r][n] (bf16, column-major: the B operands) and
//   Zs[r] = w_r z[row r],
// w_r = 2 for an off-diagonal packed row (exact in bf16), 1 on the diagonal
// and in the full layout, 0 for a padding row; the next four chunks' S and z
// are in registers meanwhile.  den adds the fp32 features times Zs.  The
// result is combined with the flash forward's (o, den) as the VALU kernel
// does.  Each group has the same chunks, a multiple of four of them; their
// (a, 16 j) sit in an LDS table built once per workgroup.  DKMAX (64 or 128)
// sizes the query tile and the table (at most E^2 / 16 chunks, E <= dk); at
// DKMAX = 128 the tile keeps the inputs' 16-bit values (exact), converted as
// they are read, and the scale multiplies the sums instead, so that three
// workgroups fit a CU's LDS.
constexpr int kRoRows = 64, kRoBp = kRoRows + 8;

// chunk cc of a group in the readout's chunk order: (a, 16 j)
__device__ __forceinline__ int2 readout_chunk(const KataGenStateArgs& k, int cc) {
  const int nb = k.E >> 4;
  int a, j;
  if (!k.tri) {
    a = cc / nb;
    j = cc - a * nb;
  } else {
    // a in block beta = a / 16 has nb - beta chunks (j = beta .. nb - 1)
    int beta = 0, base = 0;
    while (beta + 1 < nb && base + 16 * (nb - beta) <= cc) {
      base += 16 * (nb - beta);
      ++beta;
    }
    const int per = nb - beta, rem = cc - base;
    a = 16 * beta + rem / per;
    j = beta + rem % per;
  }
  return make_int2(a, 16 * j);
}

template <typename T, int MS, int DKMAX>
__global__ __launch_bounds__(256) void kata_gen_readout_mfma_kernel(KataGenStateArgs a) {
  // MS: the sum score's groups (0: the concat score, -1: the sum score over
  // a.M groups, counted at run time)
  constexpr bool SUM = MS != 0;
  static_assert(sizeof(T) == 2, "16-bit inputs");
  constexpr bool kQ16 = DKMAX > 64;
  using QT = typename std::conditional<kQ16, T, float>::type;
  constexpr int kRoQp = DKMAX + (kQ16 ? 8 : 4), kRoMaxCpg = DKMAX * DKMAX / 16;
  __shared__ __attribute__((aligned(16))) QT Qs[128 * kRoQp];
  __shared__ __attribute__((aligned(16))) __bf16 Bt[kGenDV][kRoBp];
  __shared__ __attribute__((aligned(16))) float Zs[kRoRows];
  __shared__ int2 Ci[kRoRows / 16];
  __shared__ int2 Ctab[kRoMaxCpg];
  __shared__ float Dq[4][32];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hh = lane >> 5, cl = lane & 31;
  const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H, t0 = blockIdx.y * 128;
  const T* qg = reinterpret_cast<const T*>(a.q);
  const float sq = sqrtf(a.scale);
  {
    const int dk8 = a.dk >> 3;
    for (int i = tid; i < 128 * dk8; i += 256) {
      const int t = i / dk8, d0 = 8 * (i % dk8);
      v8_t<T> x = zero8<T>();
      if (t0 + t < a.T) x = ld8<T>(qg + (((int64_t)b * a.T + t0 + t) * a.H + h) * a.dk + d0);
      if constexpr (kQ16) {
        *reinterpret_cast<v8_t<T>*>(&Qs[t * kRoQp + d0]) = x;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) Qs[t * kRoQp + d0 + j] = (float)x[j] * sq;
      }
    }
  }
  const float* S = a.S + (size_t)bh * a.P * kGenDV;
  const float* z = a.z + (size_t)bh * a.P;
  const int nb = a.E >> 4;
  const int cpg = a.tri ? a.E * (a.E + 16) / 32 : a.E * nb;  // chunks per group
  const int nch = (a.sum ? 1 : a.M) * cpg;
  for (int c = tid; c < cpg; c += 256) Ctab[c] = readout_chunk(a, c);
  __syncthreads();
  // thread (rp, cg) = (tid % 32, tid / 32): rows 2 rp, 2 rp + 1 of the four
  // chunks' 64 (chunk r / 16, b offset r % 16), column groups cg and cg + 8
  // (4 columns each), so that the staging writes one 4-byte row pair per
  // column with the row pairs of 32 lanes on consecutive banks; Bt's
  // 16-byte chunks are XOR-swizzled by bit 4 of the column, so the B-operand
  // reads of columns 16 apart fall on different banks.  z of row tid by the
  // first 64 threads.
  const int rp = tid & 31, cg = tid >> 5;
  float4 sr[2][2];
  float wr[2];
  float zr = 0.f;
  auto row_of = [&](int g, int2 t, int bo, float& wgt) __attribute__((always_inline)) {
    // t = (a, 16 j) of group g: the storage row of (a, b = 16 j + bo), or -1
    const int ra = t.x, rb = t.y + bo;
    if (!a.tri) {
      wgt = 1.f;
      return (g * a.E + ra) * a.E + rb;
    }
    if (rb < ra) {
      wgt = 0.f;
      return -1;
    }
    wgt = rb == ra ? 1.f : 2.f;
    return g * a.TE + ra * a.E - ra * (ra - 1) / 2 + (rb - ra);
  };
  // c0: a multiple of four, so the four chunks share the group g
  int g = 0, cc0 = 0;
  auto load = [&](int c0) __attribute__((always_inline)) {
    g = c0 / cpg;
    cc0 = c0 - g * cpg;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int r = 2 * rp + u;
      float wg = 0.f;
      const int p = row_of(g, Ctab[cc0 + (r >> 4)], r & 15, wg);
      wr[u] = p >= 0 ? wg : 0.f;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        sr[u][hf] = p >= 0 ? *reinterpret_cast<const float4*>(S + (size_t)p * kGenDV + 4 * (cg + 8 * hf))
                           : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (tid < kRoRows) {
      float wg = 0.f;
      const int p = row_of(g, Ctab[cc0 + (tid >> 4)], tid & 15, wg);
      zr = p >= 0 ? wg * z[p] : 0.f;
    }
  };
  auto stage = [&]() __attribute__((always_inline)) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const float x0[4] = {sr[0][hf].x, sr[0][hf].y, sr[0][hf].z, sr[0][hf].w};
      const float x1[4] = {sr[1][hf].x, sr[1][hf].y, sr[1][hf].z, sr[1][hf].w};
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        const int n = 4 * (cg + 8 * hf) + cc;
        *reinterpret_cast<bf16x2*>(&Bt[n][(2 * rp) ^ (8 * ((n >> 4) & 1))]) =
            bf16x2{(__bf16)(wr[0] * x0[cc]), (__bf16)(wr[1] * x1[cc])};
      }
    }
    if (tid < kRoRows) Zs[tid] = zr;
    if (tid < 4) {
      const int2 t = Ctab[cc0 + tid];
      Ci[tid] = make_int2(g * a.E + t.x, g * a.E + t.y);
    }
  };

  const QT* qrow = Qs + (32 * w + cl) * kRoQp;
  f32x16 acc0{}, acc1{};
  float dacc = 0.f;
  load(0);
  for (int c0 = 0; c0 < nch; c0 += kRoRows / 16) {
    __syncthreads();  // the previous rows are consumed (and Qs is complete)
    stage();
    __syncthreads();
    if (c0 + kRoRows / 16 < nch) load(c0 + kRoRows / 16);
#pragma unroll
    for (int kk = 0; kk < kRoRows / 16; ++kk) {
      const int2 ci = Ci[kk];
      const int rb = 16 * kk + 8 * hh;
      f32x8 fe{};
#pragma unroll
      for (int g = 0; g < (MS > 0 ? MS : MS < 0 ? a.M : 1); ++g) {
        const float qa = (float)qrow[ci.x + g * a.E];
        const QT* qb = qrow + ci.y + g * a.E + 8 * hh;
        f32x8 bq;
        if constexpr (kQ16) {
          const v8_t<T> x = *reinterpret_cast<const v8_t<T>*>(qb);
#pragma unroll
          for (int j = 0; j < 8; ++j) bq[j] = (float)x[j];
        } else {
          const f32x4 b0 = *reinterpret_cast<const f32x4*>(qb), b1 = *reinterpret_cast<const f32x4*>(qb + 4);
          bq = f32x8{b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
        }
        fe += qa * bq;
      }
      const f32x4 z0 = *reinterpret_cast<const f32x4*>(&Zs[rb]);
      const f32x4 z1 = *reinterpret_cast<const f32x4*>(&Zs[rb + 4]);
      dacc += ((fe[0] * z0[0] + fe[1] * z0[1]) + (fe[2] * z0[2] + fe[3] * z0[3])) +
              ((fe[4] * z1[0] + fe[5] * z1[1]) + (fe[6] * z1[2] + fe[7] * z1[3]));
      const bf16x8 A = __builtin_convertvector(fe, bf16x8);
      const int rbs = rb ^ (8 * ((cl >> 4) & 1));
      acc0 = mma(A, *reinterpret_cast<const bf16x8*>(&Bt[cl][rbs]), acc0);
      acc1 = mma(A, *reinterpret_cast<const bf16x8*>(&Bt[32 + cl][rbs]), acc1);
    }
  }
  // den part of query 32 w + l % 32: the two lane halves; then every lane
  // reads the queries of its C-layout rows
  dacc += __shfl_xor(dacc, 32);
  // the 16-bit tile holds q, not q~: the scale multiplies the sums
  const float fs = kQ16 ? a.scale : 1.f;
  if (hh == 0) Dq[w][cl] = dacc;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tq = 32 * w + 8 * i + 4 * hh + r, t = t0 + tq;
      if (t >= a.T) continue;
      const int64_t row = ((int64_t)b * a.T + t) * a.H + h;
      const float fd = (a.c ? __expf(a.c[row]) : 1.f) * fs;
      const float df = a.den[row];
      const float dsc = fmaxf(df + fd * Dq[w][8 * i + 4 * hh + r], a.eps), inv = 1.f / dsc;
      T* orow = (T*)a.o + row * kGenDV;
      orow[cl] = (T)(((float)orow[cl] * df + fd * acc0[4 * i + r]) * inv);
      orow[32 + cl] = (T)(((float)orow[32 + cl] * df + fd * acc1[4 * i + r]) * inv);
    }
  // den after every lane of the wave has read it (its queries are this
  // wave's alone)
  __syncthreads();
  if (hh == 0) {
    const int t = t0 + 32 * w + cl;
    if (t < a.T) {
      const int64_t row = ((int64_t)b * a.T + t) * a.H + h;
      const float fd = (a.c ? __expf(a.c[row]) : 1.f) * fs;
      a.den[row] = fmaxf(a.den[row] + fd * Dq[w][cl], a.eps);
    }
  }
}

// the sum score's group count as a template argument where it is 2, 4 or 8
// (so the group loop unrolls), -1 for the other counts dk <= 128 allows
// (3, 5, 6, 7: a loop bounded at run time); the sum score over one group is
// the concat score
template <typename F>
hipError_t by_sum_groups(const KataGenStateArgs& a, F&& f) {
  if (!a.sum || a.M == 1) return f(std::integral_constant<int, 0>{});
  if (a.M == 2) return f(std::integral_constant<int, 2>{});
  if (a.M == 4) return f(std::integral_constant<int, 4>{});
  if (a.M == 8) return f(std::integral_constant<int, 8>{});
  return f(std::integral_constant<int, -1>{});
}

template <typename T>
hipError_t launch_kata_gen_state(const KataGenStateArgs& a, int which, hipStream_t stream) {
  const int BH = a.B * a.H;
  if (which == KATA_GEN_DECODE) {
    kata_gen_decode_kernel<T><<<dim3(BH, a.nsplit), dim3(256), 0, stream>>>(a);
    if (a.nsplit > 1) kata_gen_decode_finish_kernel<T><<<dim3(BH), dim3(kGenDV), 0, stream>>>(a);
  } else if (which == KATA_GEN_READOUT) {
    if constexpr (sizeof(T) == 2) {
      const dim3 grid(BH, (a.T + 127) / 128);
      by_sum_groups(a, [&](auto ms) {
        if (a.dk <= 64)
          kata_gen_readout_mfma_kernel<T, decltype(ms)::value, 64><<<grid, dim3(256), 0, stream>>>(a);
        else
          kata_gen_readout_mfma_kernel<T, decltype(ms)::value, 128><<<grid, dim3(256), 0, stream>>>(a);
        return hipSuccess;
      });
    } else {
      kata_gen_readout_kernel<T><<<dim3(BH, (a.T + 63) / 64), dim3(256), 0, stream>>>(a);
    }
  } else if constexpr (sizeof(T) == 2) {
    // 256 rows and both column halves per workgroup; a state of at most
    // 256 rows that would leave CUs idle takes 128 rows and one half (more
    // workgroups, each streaming every token: the staging, not the products,
    // is this kernel's cost, so larger states keep the 256-row tiles)
    by_sum_groups(a, [&](auto ms) {
      constexpr int MS = decltype(ms)::value;
      if (a.P > 256 || (int64_t)BH * ((a.P + 255) / 256) >= 512)
        kata_gen_update_mfma_kernel<T, MS, 2, 2><<<dim3(BH, (a.P + 255) / 256), dim3(256), 0, stream>>>(a);
      else
        kata_gen_update_mfma_kernel<T, MS, 1, 1><<<dim3(BH, (a.P + 127) / 128, 2), dim3(256), 0, stream>>>(a);
      return hipSuccess;
    });
  } else {
    kata_gen_update_kernel<T><<<dim3(BH, (a.P + 63) / 64), dim3(256), 0, stream>>>(a);
  }
  return hipGetLastError();
}

template hipError_t launch_kata_gen_state<__bf16>(const KataGenStateArgs&, int, hipStream_t);
template hipError_t launch_kata_gen_state<_Float16>(const KataGenStateArgs&, int, hipStream_t);
template hipError_t launch_kata_gen_state<float>(const KataGenStateArgs&, int, hipStream_t);

}  // namespace linatt
