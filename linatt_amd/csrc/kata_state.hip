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
//   kata_seg_state_kernel   per (b, h, segment, 128 state rows):
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
#include "common.h"
#include "kata_kernels.h"

namespace linatt {

// ---------------------------------------------------------------------------
// Segment states.  Wave w of block (bh, seg, pb) owns state rows
// p = 128 pb + 32 w + [0, 32) (its X-operand rows) for every value column.
// ---------------------------------------------------------------------------
template <typename T, int DK, int DV, int M>
__global__ __launch_bounds__(256) void kata_seg_state_kernel(KataStateArgs a) {
  constexpr int E = DK / M, P = M * E * E;
  constexpr int PX = 64 + 8;
  __shared__ __attribute__((aligned(16))) T Kt[DK * PX];
  __shared__ __attribute__((aligned(16))) T Vt[DV * PX];
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  constexpr int NPB = P / 128;
  int blk = blockIdx.x;
  const int pb = blk % NPB;
  blk /= NPB;
  const int seg = blk % a.nseg;
  const int bh = blk / a.nseg;
  const int b = bh / a.H, h = bh % a.H;
  const T* kb = (const T*)a.k + (int64_t)b * a.sb + (int64_t)h * a.sh;
  const T* vb = (const T*)a.v + (int64_t)b * a.vsb + (int64_t)h * a.vsh;

  const int p = 128 * pb + 32 * w + cl;  // this lane's X row
  const int g = p / (E * E), ra = g * E + (p / E) % E, rb = g * E + p % E;

  f32x16 acc[DV / 32];
#pragma unroll
  for (int vt = 0; vt < DV / 32; ++vt) acc[vt] = f32x16{};
  float zp = 0.f;
  const int s_begin = seg * a.L, s_end = min(s_begin + a.L, a.T);
  for (int s0 = s_begin; s0 < s_end; s0 += 64) {
    __syncthreads();
    load_tile64x<T, T, DK, 1, PX, false, true>(kb, s0, a.T, a.st, nullptr, Kt, tid, nullptr);
    load_tile64x<T, T, DV, 1, PX, false, true>(vb, s0, a.T, a.vst, nullptr, Vt, tid, nullptr);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const v8_t<T> ka = ld8<T>(Kt + ra * PX + 16 * s + 8 * hh);
      const v8_t<T> kc = ld8<T>(Kt + rb * PX + 16 * s + 8 * hh);
      f32x8 pf;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        pf[j] = (float)ka[j] * (float)kc[j];
        zp += pf[j];
      }
      const v8_t<T> x = __builtin_convertvector(pf, v8_t<T>);
#pragma unroll
      for (int vt = 0; vt < DV / 32; ++vt)
        acc[vt] = mma(x, ld8<T>(Vt + (32 * vt + cl) * PX + 16 * s + 8 * hh), acc[vt]);
    }
  }
  // acc[vt] = D[p'][v]: rows p' = 128 pb + 32 w + 8 I + 4 hh + r, lane column
  // v = 32 vt + cl  ->  S_seg^T [v][p'] with 16-byte stores.
  float* st = a.seg_S + ((size_t)bh * a.nseg + seg) * DV * P;
#pragma unroll
  for (int vt = 0; vt < DV / 32; ++vt)
#pragma unroll
    for (int I = 0; I < 4; ++I)
      *reinterpret_cast<float4*>(st + (size_t)(32 * vt + cl) * P + 128 * pb + 32 * w + 8 * I + 4 * hh) =
          make_float4(acc[vt][4 * I], acc[vt][4 * I + 1], acc[vt][4 * I + 2], acc[vt][4 * I + 3]);
  zp += __shfl_xor(zp, 32);
  if (hh == 0) a.seg_z[((size_t)bh * a.nseg + seg) * P + p] = zp;
}

// ---------------------------------------------------------------------------
// Exclusive prefix over segments.  One thread per (bh, row v in [0, DV]
// (row DV is z), 4 consecutive state rows p).
// ---------------------------------------------------------------------------
template <typename T, int DK, int DV, int M>
__global__ __launch_bounds__(256) void kata_seg_scan_kernel(KataStateArgs a) {
  constexpr int E = DK / M, P = M * E * E;
  const int64_t per_bh = (int64_t)(DV + 1) * (P / 4);
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)a.B * a.H * per_bh) return;
  const int bh = (int)(idx / per_bh);
  const int64_t rem = idx % per_bh;
  const int v = (int)(rem / (P / 4));
  const int p = 4 * (int)(rem % (P / 4));
  float4 run = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int seg = 0; seg < a.nseg; ++seg) {
    const size_t base = (size_t)bh * a.nseg + seg;
    float4 x;
    if (v < DV) {
      x = *reinterpret_cast<const float4*>(a.seg_S + (base * DV + v) * P + p);
      st4<T>((T*)a.HT + (base * DV + v) * P + p, to4<T>(run.x, run.y, run.z, run.w));
    } else {
      x = *reinterpret_cast<const float4*>(a.seg_z + base * P + p);
      *reinterpret_cast<float4*>(a.Hz + base * P + p) = run;
    }
    run.x += x.x; run.y += x.y; run.z += x.z; run.w += x.w;
  }
  const float s = a.scale;
  if (v < DV) {
    if (a.S_out) {
      float* so = a.S_out + ((size_t)bh * P + p) * DV + v;
      so[0] = run.x * s;
      so[DV] = run.y * s;
      so[2 * DV] = run.z * s;
      so[3 * DV] = run.w * s;
    }
  } else if (a.z_out) {
    *reinterpret_cast<float4*>(a.z_out + (size_t)bh * P + p) =
        make_float4(run.x * s, run.y * s, run.z * s, run.w * s);
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
  constexpr int KP = DK + 8, VP = 64 + 4;
  static_assert(E % 16 == 0, "group width must be a multiple of 16");
  constexpr int QP = DK + 8;
  __shared__ __attribute__((aligned(16))) T Ks[64 * KP];
  __shared__ __attribute__((aligned(16))) T Vt[DV * VP];
  __shared__ __attribute__((aligned(16))) T Qa[128 * QP];

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
  if (seg > 0 && tw < Tn) {
    const size_t base = (size_t)bh * a.nseg + seg;
    const T* hT = (const T*)a.HT + base * DV * P;
    const float* hz = a.Hz + base * P;
#pragma unroll
    for (int g = 0; g < M; ++g) {
#pragma unroll 2
      for (int ai = 0; ai < E; ++ai) {
        const float qa = (float)qa_row[g * E + ai];
#pragma unroll
        for (int b0 = 0; b0 < E; b0 += 16) {
          const int p0 = g * E * E + ai * E + b0;
          const int kk = (g * E + b0) / 16;
          const f32x4 z0 = *reinterpret_cast<const f32x4*>(hz + p0 + 8 * hh);
          const f32x4 z1 = *reinterpret_cast<const f32x4*>(hz + p0 + 8 * hh + 4);
          f32x8 pf;
#pragma unroll
          for (int j = 0; j < 8; ++j) pf[j] = qa * (float)qop[kk][j];
#pragma unroll
          for (int j = 0; j < 4; ++j) dpart += pf[j] * z0[j] + pf[4 + j] * z1[j];
          const v8_t<T> y = __builtin_convertvector(pf, v8_t<T>);
#pragma unroll
          for (int db = 0; db < DV / 32; ++db)
            oacc[db] = mma(ld8<T>(hT + (size_t)(32 * db + cl) * P + p0 + 8 * hh), y, oacc[db]);
        }
      }
    }
  }

  // intra-segment flash term, keys in [seg_start, min(t0 + 128, T))
  const int s_end = min(t0 + 128, Tn);
  for (int s0 = seg_start; s0 < s_end; s0 += 64) {
    __syncthreads();
    load_tile64x<T, T, DK, KP, 1, true, false>(kb, s0, Tn, a.st, Ks, nullptr, tid, nullptr);
    load_tile64x<T, T, DV, 1, VP, false, true>(vb, s0, Tn, a.vst, nullptr, Vt, tid, nullptr);
    __syncthreads();
    if (s0 > tw + 31 || tw >= Tn) continue;
    const bool need_mask = (s0 + 63 > tw) || (s0 + 64 > Tn);
    f32x16 sc[2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      sc[sb] = f32x16{};
      const T* krow = Ks + (32 * sb + cl) * KP + 8 * hh;
#pragma unroll
      for (int g = 0; g < M; ++g) {
        f32x16 r{};
#pragma unroll
        for (int kk = 0; kk < KE; ++kk) r = mma(ld8<T>(krow + g * E + 16 * kk), qop[g * KE + kk], r);
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
        oacc[db] = mma(ld_tr_op<T>(Vt + (32 * db + cl) * VP + 32 * (ks4 >> 1), ks4 & 1, hh), pb, oacc[db]);
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

template <typename T, int DK, int DV, int M>
hipError_t launch_kata_prefill(const KataStateArgs& a, hipStream_t stream) {
  constexpr int E = DK / M, P = M * E * E;
  const int BH = a.B * a.H;
  kata_seg_state_kernel<T, DK, DV, M><<<dim3(BH * a.nseg * (P / 128)), dim3(256), 0, stream>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t items = (int64_t)BH * (DV + 1) * (P / 4);
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
// columns each), 16 rows per pass.
// ---------------------------------------------------------------------------
template <typename T, int DK, int DV, int M>
__global__ __launch_bounds__(256) void kata_decode_kernel(KataDecodeArgs a) {
  constexpr int E = DK / M, P = M * E * E;
  static_assert(DV == 64, "decode maps 16 threads x 4 columns onto a row");
  __shared__ float qs[DK], ks[DK], vs[DV];
  __shared__ float4 red[16][16];
  __shared__ float dred[16];
  const int tid = threadIdx.x;
  const int bh = blockIdx.x;
  if (tid < DK) {
    qs[tid] = (float)((const T*)a.q)[(size_t)bh * DK + tid];
    ks[tid] = (float)((const T*)a.k)[(size_t)bh * DK + tid];
  }
  if (tid < DV) vs[tid] = (float)((const T*)a.v)[(size_t)bh * DV + tid];
  __syncthreads();
  const int c4 = tid & 15, r = tid >> 4;
  const float4 vv = *reinterpret_cast<const float4*>(vs + 4 * c4);
  float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
  float dacc = 0.f;
  float* S = a.S + (size_t)bh * P * DV;
  float* z = a.z + (size_t)bh * P;
  for (int p = r; p < P; p += 16) {
    const int g = p / (E * E), ia = g * E + (p / E) % E, ib = g * E + p % E;
    const float pk = a.scale * ks[ia] * ks[ib];
    const float pq = a.scale * qs[ia] * qs[ib];
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
    const float inv = 1.f / fmaxf(d, a.eps);
    st4<T>((T*)a.o + (size_t)bh * DV + 4 * tid, to4<T>(s.x * inv, s.y * inv, s.z * inv, s.w * inv));
  }
}

template <typename T, int DK, int DV, int M>
hipError_t launch_kata_decode(const KataDecodeArgs& a, hipStream_t stream) {
  kata_decode_kernel<T, DK, DV, M><<<dim3(a.B * a.H), dim3(256), 0, stream>>>(a);
  return hipGetLastError();
}

#define LINATT_STATE_INST(T, DK, DV, M)                                              \
  template hipError_t launch_kata_prefill<T, DK, DV, M>(const KataStateArgs&, hipStream_t); \
  template hipError_t launch_kata_decode<T, DK, DV, M>(const KataDecodeArgs&, hipStream_t);

LINATT_KATA_STATE_SHAPES(LINATT_STATE_INST)

}  // namespace linatt
