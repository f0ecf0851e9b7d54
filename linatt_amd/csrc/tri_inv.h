// In-LDS completion of the 64 x 64 unit lower-triangular inverse used by the
// chunked delta rules: Tm = (I + N)^-1, N strictly lower triangular.
#pragma once
#include "common.h"

namespace linatt {

// AT (LDS, fp32, row stride 64) holds N below the diagonal blocks, zeros
// above the diagonal, and in its four diagonal 16 x 16 blocks their own
// inverses D_R = (I + N_RR)^-1.  On return AT holds Tm.  Two merges:
//
//   16 -> 32 (all 256 threads, fp32):  X_p = -D_{2p+1} (N_{2p+1,2p} D_{2p}),
//            p = 0, 1, giving the 32 x 32 diagonal blocks T_0, T_1 of Tm;
//   32 -> 64 (wave 0, MFMA):           Tm_10 = -T_1 (N_10 T_0).
//
// The 32 x 32 products run on v_mfma_f32_32x32x16_bf16 with every operand
// split into bf16 hi + lo parts (hi.hi + hi.lo + lo.hi, about 16 mantissa
// bits): bf16 rather than the caller's 16-bit type because Tm's entries can
// exceed the fp16 range.  Ys: 512 floats of LDS scratch.  Called by all 256
// threads of the workgroup; ends with a barrier.
__device__ __forceinline__ void tri_inv64_merge(float* AT, float* Ys, int tid) {
  {
    const int p = tid >> 7, c = tid & 15, i0 = 2 * ((tid >> 4) & 7);
    const int r0 = 32 * p;
    float y0 = 0.f, y1 = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const float d = AT[(r0 + k) * 64 + r0 + c];
      y0 += AT[(r0 + 16 + i0) * 64 + r0 + k] * d;
      y1 += AT[(r0 + 17 + i0) * 64 + r0 + k] * d;
    }
    Ys[p * 256 + i0 * 16 + c] = y0;
    Ys[p * 256 + (i0 + 1) * 16 + c] = y1;
    block_barrier();
    float x0 = 0.f, x1 = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const float yk = Ys[p * 256 + k * 16 + c];
      x0 += AT[(r0 + 16 + i0) * 64 + r0 + 16 + k] * yk;
      x1 += AT[(r0 + 17 + i0) * 64 + r0 + 16 + k] * yk;
    }
    AT[(r0 + 16 + i0) * 64 + r0 + c] = -x0;
    AT[(r0 + 17 + i0) * 64 + r0 + c] = -x1;
    block_barrier();
  }
  if (tid < 64) {
    const int lane = tid, cl = lane & 31, hh = lane >> 5;
    auto split8 = [](f32x4 a0, f32x4 a1, bf16x8& hi, bf16x8& lo) __attribute__((always_inline)) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        hi[e] = (__bf16)a0[e];
        lo[e] = (__bf16)(a0[e] - (float)hi[e]);
        hi[4 + e] = (__bf16)a1[e];
        lo[4 + e] = (__bf16)(a1[e] - (float)hi[4 + e]);
      }
    };
    // Z = N_10 T_0: lane row i = cl of N_10 (k = 16 ks + 8 hh + 0..7), lane
    // column j = cl of T_0 (the same k)
    f32x16 z{};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 ah, al, bh, bl;
      const float* ar = AT + (32 + cl) * 64 + 16 * ks + 8 * hh;
      split8(*reinterpret_cast<const f32x4*>(ar), *reinterpret_cast<const f32x4*>(ar + 4), ah, al);
      f32x4 b0, b1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        b0[e] = AT[(16 * ks + 8 * hh + e) * 64 + cl];
        b1[e] = AT[(16 * ks + 8 * hh + 4 + e) * 64 + cl];
      }
      split8(b0, b1, bh, bl);
      z = mma(ah, bh, z);
      z = mma(ah, bl, z);
      z = mma(al, bh, z);
    }
    // Tm_10 = -T_1 Z: Z (C layout) is the B operand in ld_tr_op k order;
    // T_1's row cl supplies the matching columns 16 ks + 4 hh + {0..3, 8..11}
    f32x16 zl;
#pragma unroll
    for (int e = 0; e < 16; ++e) zl[e] = z[e] - (float)(__bf16)z[e];
    f32x16 y{};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const bf16x8 bh = c_to_b<__bf16>(z, ks), bl = c_to_b<__bf16>(zl, ks);
      bf16x8 ah, al;
      const float* ar = AT + (32 + cl) * 64 + 32 + 16 * ks + 4 * hh;
      split8(*reinterpret_cast<const f32x4*>(ar), *reinterpret_cast<const f32x4*>(ar + 8), ah, al);
      y = mma(ah, bh, y);
      y = mma(ah, bl, y);
      y = mma(al, bh, y);
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) AT[(32 + 8 * (e >> 2) + 4 * hh + (e & 3)) * 64 + cl] = -y[e];
  }
  block_barrier();
}

}  // namespace linatt
