// Causal linear attention in chunked state form, for gfx950.
//
// Replaces the feature="linear" path of the reference's concat tree-scan,
// spd_chunk_scan_cat (kata/spd/chunk_scan_cat.py:219-345, kernels :24-178):
// psi(x) = sqrt(scale) x per group, concatenated over the groups, so
//
//   kappa(q, k) = scale (q . k)           (the group split drops out)
//   den_t = max(sum_{s<=t} kappa(q_t, k_s), eps)
//   o_t   = sum_{s<=t} kappa(q_t, k_s) v_s / den_t
//
// with the reference's numerics: the state S = sum k^T v enters the
// inter-chunk product as 16-bit operands, z = sum k and both row sums stay
// float32, and the intra-chunk weights are rounded to the input type for
// their product with v.
//
// One workgroup per (batch, head), four waves, 64-token chunks in order.
// Wave w = (tb, vb): tb = w & 1 is its 32-row block of the chunk's tokens
// and of S's key dims, vb = w >> 1 its 32-column block of v.  Per chunk:
//   O^T[v][t]  = S^T Q^T (inter: S^T as the A operand from c_to_b images the
//                waves trade through LDS) + V^T A^T (intra: A^T = K Q^T,
//                causal-masked), both into one accumulator;
//   S[d][v]   += K^T V (wave (tb, vb) owns the block d in 32 tb.., v in 32 vb..);
//   z[d]      += sum_t k_t[d] (threads 0-63, float32).
// Q, K, V tiles arrive by direct global->LDS copies; rows past T are zeroed
// in LDS, so they add nothing to S, z or the row sums.
#include "common.h"
#include "misc_kernels.h"

namespace linatt {

template <typename T>
__global__ __launch_bounds__(256) void linear_scan_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                          const T* __restrict__ v, T* __restrict__ o,
                                                          float* __restrict__ den, int Tn, float scale,
                                                          float eps) {
  constexpr int D = 64, DV = 64, TE = 64 * 64;
  __shared__ __attribute__((aligned(16))) T Qs[TE];
  __shared__ __attribute__((aligned(16))) T Ks[TE];
  __shared__ __attribute__((aligned(16))) T Vs[TE];
  __shared__ __attribute__((aligned(16))) u32x4 Sx[4][2][64];  // c_to_b images of S blocks, by owner wave
  __shared__ __attribute__((aligned(16))) float zs[D];

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int tb = w & 1, vb = w >> 1;
  const int64_t bh = blockIdx.x;
  const T* qb = q + bh * Tn * D;
  const T* kb = k + bh * Tn * D;
  const T* vbp = v + bh * Tn * DV;
  T* ob = o + bh * Tn * DV;
  float* dnb = den + bh * Tn;
  const int NC = (Tn + 63) / 64;

  f32x16 S{};       // S[32 tb + rows][32 vb + lane column], before the current chunk
  float zreg = 0.f;  // z[tid] for tid < 64
  // the state before chunk 0 is zero
  Sx[w][0][lane] = u32x4{0u, 0u, 0u, 0u};
  Sx[w][1][lane] = u32x4{0u, 0u, 0u, 0u};
  if (tid < D) zs[tid] = 0.f;

  for (int c = 0; c < NC; ++c) {
    const int t0 = 64 * c;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      dma_tile64<T>(qb, D, t0, Tn, Qs, 2 * w + i, lane);
      dma_tile64<T>(kb, D, t0, Tn, Ks, 2 * w + i, lane);
      dma_tile64<T>(vbp, DV, t0, Tn, Vs, 2 * w + i, lane);
    }
    vm_wait_barrier<0>();  // the tiles, and the previous chunk's Sx / zs
    const int nvalid = Tn - t0 < 64 ? Tn - t0 : 64;
    if (nvalid < 64) {
      // rows past T repeat the last valid row: zero them in all three tiles
      for (int idx = tid; idx < (64 - nvalid) * 8; idx += 256) {
        const int r = nvalid + idx / 8, s8 = idx % 8;
        reinterpret_cast<u32x4*>(Qs + r * 64)[s8] = u32x4{0u, 0u, 0u, 0u};
        reinterpret_cast<u32x4*>(Ks + r * 64)[s8] = u32x4{0u, 0u, 0u, 0u};
        reinterpret_cast<u32x4*>(Vs + r * 64)[s8] = u32x4{0u, 0u, 0u, 0u};
      }
      block_barrier();
    }

    const int t = 32 * tb + cl;  // this lane's token within the chunk (output column)
    f32x16 acc{};
    // inter: O^T[v][t] += sum_d S^T[v][d] Q^T[d][t]
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc = mma(__builtin_bit_cast(v8_t<T>, Sx[db | (vb << 1)][j][lane]),
                  tile_ldp8<T>(Qs, t, 32 * db, j, hh), acc);
    // den, inter part: q_t . z (this lane's half of the key dims)
    float dl = 0.f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const v8_t<T> q8 = tile_ld8<T>(Qs, t, 32 * hh + 8 * m);
#pragma unroll
      for (int e = 0; e < 8; ++e) dl += (float)q8[e] * zs[32 * hh + 8 * m + e];
    }
    // intra: A^T[s][t] = k_s . q_t for key blocks sb <= tb, causal-masked
    v8_t<T> qop[D / 16];
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) qop[kk] = tile_ld8<T>(Qs, t, 16 * kk + 8 * hh);
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      if (sb > tb) break;
      f32x16 a{};
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) a = mma(tile_ld8<T>(Ks, 32 * sb + cl, 16 * kk + 8 * hh), qop[kk], a);
      if (sb == tb) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int s = 32 * sb + 8 * (e >> 2) + 4 * hh + (e & 3);
          if (s > t) a[e] = 0.f;
        }
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) dl += a[e];
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc = mma(tile_tr8<T>(Vs, 32 * sb, 32 * vb, j, lane), c_to_b<T>(a, j), acc);
    }
    dl += __shfl_xor(dl, 32);
    const float dn = fmaxf(scale * dl, eps);
    if (t < nvalid) {
      const float f = scale / dn;
      T* orow = ob + (int64_t)(t0 + t) * DV + 32 * vb;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st4<T>(orow + 8 * i + 4 * hh, to4<T>(acc[4 * i] * f, acc[4 * i + 1] * f, acc[4 * i + 2] * f,
                                             acc[4 * i + 3] * f));
      if (vb == 0 && hh == 0) dnb[t0 + t] = dn;
    }

    // S[d][v] += sum_t K^T[d][t] V[t][v]  (d block tb, v block vb); z += column sums of K
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        S = mma(tile_tr8<T>(Ks, 32 * tt, 32 * tb, j, lane), tile_tr8<T>(Vs, 32 * tt, 32 * vb, j, lane), S);
    if (tid < D) {
      const char* kt = reinterpret_cast<const char*>(Ks);
      for (int r = 0; r < 64; ++r)
        zreg += (float)reinterpret_cast<const T*>(kt + tile_off(r, tid & ~3))[tid & 3];
    }
    block_barrier();  // every wave is done with the tiles, Sx and zs of this chunk
    Sx[w][0][lane] = __builtin_bit_cast(u32x4, c_to_b<T>(S, 0));
    Sx[w][1][lane] = __builtin_bit_cast(u32x4, c_to_b<T>(S, 1));
    if (tid < D) zs[tid] = zreg;
  }
}

template <typename T>
hipError_t launch_linear_scan(const void* q, const void* k, const void* v, void* o, float* den, int B,
                              int H, int T_, float scale, float eps, hipStream_t stream) {
  linear_scan_kernel<T><<<dim3(B * H), dim3(256), 0, stream>>>((const T*)q, (const T*)k, (const T*)v,
                                                               (T*)o, den, T_, scale, eps);
  return hipGetLastError();
}

template hipError_t launch_linear_scan<__bf16>(const void*, const void*, const void*, void*, float*, int,
                                              int, int, float, float, hipStream_t);
template hipError_t launch_linear_scan<_Float16>(const void*, const void*, const void*, void*, float*, int,
                                                 int, int, float, float, hipStream_t);

}  // namespace linatt
