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

// Row sums of a 32 x 32 fp32 block held in C layout (lane column l & 31,
// rows 8 (e >> 2) + 4 (l >> 5) + (e & 3), e = 0..15): dst[row] = the sum
// over the 32 columns.  Each value is summed over its 16-lane row by DPP
// moves (quad xor 1, quad xor 2, half-row mirror, row mirror: after each
// step every lane holds the sum over twice as many lanes), then over the
// two rows of its 32-lane half by one xor-16 shuffle.
__device__ __forceinline__ float dpp_add(float v, int ctrl_sel) {
  int m;
  switch (ctrl_sel) {
    case 0: m = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false); break;
    case 1: m = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false); break;
    case 2: m = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false); break;
    default: m = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false); break;
  }
  return v + __builtin_bit_cast(float, m);
}
__device__ __forceinline__ void row_sums32(f32x16 x, float* dst, int lane) {
#pragma unroll
  for (int st = 0; st < 4; ++st)
#pragma unroll
    for (int e = 0; e < 16; ++e) x[e] = dpp_add(x[e], st);
#pragma unroll
  for (int e = 0; e < 16; ++e) x[e] += __shfl_xor(x[e], 16);
  if ((lane & 31) == 0) {
#pragma unroll
    for (int e = 0; e < 16; ++e) dst[8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)] = x[e];
  }
}

// ---------------------------------------------------------------------------
// Kernel 1: reverse state pass.  One workgroup per (b, h, 32 value columns):
// two compute waves and the copy waves.  Per chunk, with dS' the gradient
// of the state leaving it:
//   dVn = Aqk^T dO + diag(e^(gamma-G)) K dS'
//   dS  = e^gamma dS' + (scale e^G Q)^T dO - W^T dVn
// Compute wave p holds dS key-dim blocks ND2 p .. ND2 p + ND2 - 1 in MFMA
// accumulators and forms dVn for the chunk rows 32 p .. 32 p + 31.  The
// two trade 16-bit operand images through LDS: each wave's dS blocks (for
// the other's K dS' product, written at the end of the previous chunk) and
// its dVn rows (for the other's W^T dVn product, before the mid-chunk
// barrier).  K, W, Qg (ungated: q), Aqk, dO and G of a chunk reach LDS by
// direct global->LDS copies (swizzled 64 x 64 tiles, see tile_slot) into
// two slots, issued by the copy waves one chunk ahead; dh^T and dv_new^T
// leave through LDS staging, stored by the copy waves one chunk later.
//
// Barriers per chunk c (every wave): TOP (chunk c landed; the dS images of
// chunk c are written; chunk c + 1's slot and staged outputs are free) and
// MID (every ring read and dS-image read of chunk c is done, the dVn images
// are written, and the copy waves have read chunk c + 1's staged outputs).
// The dS images of chunk c live in the staging buffer of chunk c, which is
// free from TOP until the outputs of chunk c are staged after MID.
// ---------------------------------------------------------------------------
constexpr int kStateBwdComputeWaves = 2;
// four copy waves: the copies of a chunk (64 KiB at K = V = 128) then take
// less of the chain's time than with two (measured: 48.5 -> 46.2 us per pass)
constexpr int kStateBwdCopyWaves = 4;
constexpr int state_bwd_threads() { return 64 * (kStateBwdComputeWaves + kStateBwdCopyWaves); }

template <typename T, int DK, int DV, bool GATED>
__global__ __launch_bounds__(state_bwd_threads()) void delta_state_bwd_kernel(DeltaArgs a, DeltaLayout L) {
  constexpr int SPLIT = DV / 32;                  // workgroups per head, 32 value columns each
  constexpr int NDT = DK / 32, ND2 = NDT / 2;     // dS key-dim blocks: all, per compute wave
  constexpr int NCW = kStateBwdComputeWaves;
  constexpr int KT = DK / 64;                     // 64 x 64 tiles per row block
  constexpr int TE = 64 * 64;                     // elements per tile
  constexpr int OPW = 8;                          // 1 KiB copies per tile, split over the copy waves
  constexpr int OPC = OPW / kStateBwdCopyWaves;      // per copy wave
  constexpr int NTILE = 3 * KT + 2;               // K, W, Qg, Aqk, dO (the 64 columns holding ours)
  constexpr int SLOT = NTILE * TE + 2 * 64 * 4 / (int)sizeof(T);  // + G and e^(gamma - G) of the chunk (f32)
  static_assert(NDT % 2 == 0 && NCW == 2 && OPW % kStateBwdCopyWaves == 0, "key dims over two compute waves");
  // per chunk (two buffers): the dh^T blocks (64 key dims each) and the
  // dv_new^T block of the 32 columns, staged for the copy waves' stores;
  // also the home of the chunk's dS images (2 ND2 * 128 slots, before MID)
  constexpr int NSTG = NDT / 2 + 1;
  // ring slots: three (copies two chunks ahead) where LDS allows (K = V = 64),
  // else two
  constexpr int FIXED = (2 * NSTG * 256 + NCW * 2 * 64) * 16;
  constexpr int NSLOT = 3 * SLOT * (int)sizeof(T) + FIXED <= 160 * 1024 ? 3 : 2;
  __shared__ __attribute__((aligned(16))) T Sh[NSLOT * SLOT];
  __shared__ __attribute__((aligned(16))) u32x4 Stg[2][NSTG][256];
  static_assert(2 * ND2 * 128 <= (NSTG - 1) * 256, "dS images fit below the dv_new^T block");
  // dVn images: -dVn rows of compute wave p as B operands (k-steps j = 0, 1)
  __shared__ __attribute__((aligned(16))) u32x4 Xv[NCW][2][64];
  static_assert(NSLOT * SLOT * (int)sizeof(T) + FIXED <= 160 * 1024, "LDS");

  const int lane = threadIdx.x & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int Tn = a.T, H = a.H, NT = a.NT;
  const int BH = a.B * H;
  const int bh = blockIdx.x % BH, part = blockIdx.x / BH;
  const int b = bh / H, h = bh % H;
  const int v = 32 * part + cl;
  const size_t Tp = (size_t)NT * kChunk;

  const T* kb = (const T*)a.k + ((size_t)b * Tn * H + h) * DK;
  const T* dob = (const T*)a.dout + ((size_t)b * Tn * H + h) * DV + 64 * (part / 2);  // the 64 columns holding ours
  const float* Gc = reinterpret_cast<const float*>(a.ctx + L.Gc) + (size_t)bh * Tp;
  const float* Fk = reinterpret_cast<const float*>(a.ctx + L.Fk) + (size_t)bh * Tp;

  auto kt = [&](T* sl, int i) { return sl + i * TE; };                 // K tile i (key dims 64 i..)
  auto wt = [&](T* sl, int i) { return sl + (KT + i) * TE; };          // W [i][d], key dims 64 i..
  auto qt = [&](T* sl, int i) { return sl + (2 * KT + i) * TE; };      // Qg key dims 64 i..
  auto at = [&](T* sl) { return sl + 3 * KT * TE; };                   // Aqk
  auto ot = [&](T* sl) { return sl + (3 * KT + 1) * TE; };             // dO
  auto gs = [&](T* sl) { return reinterpret_cast<float*>(sl + NTILE * TE); };

  // copy wave cw takes ops [OPC cw, OPC cw + OPC) of every tile, i.e. tile
  // rows [8 OPC cw, 8 OPC cw + 8 OPC); per-lane byte offsets for full
  // chunks, the general path for the last one (rows past T clamped)
  const int cw = w - NCW;
  auto issue = [&](int c) __attribute__((always_inline)) {
    T* sl = Sh + (c % NSLOT) * SLOT;
    const int t0 = c * kChunk;
    const size_t ci = (size_t)bh * NT + c;
    const T* wtg = (const T*)(a.ctx + L.W) + ci * 64 * DK;  // W [i][d], natural
    const T* qgg = (const T*)(a.ctx + L.Qg) + ci * 64 * DK;
    const T* qb = (const T*)a.q + ((size_t)b * Tn * H + h) * DK;  // ungated: q tiles
    const T* atg = (const T*)(a.ctx + L.Aqk) + ci * 4096;
    if (t0 + 64 > Tn) {
#pragma unroll
      for (int op = OPC * cw; op < OPC * cw + OPC; ++op) {
#pragma unroll
        for (int i = 0; i < KT; ++i) {
          dma_tile64<T>(kb + 64 * i, (int64_t)H * DK, t0, Tn, kt(sl, i), op, lane);
          dma_tile64<T>(wtg + 64 * i, DK, 0, 64, wt(sl, i), op, lane);
          if constexpr (GATED) dma_tile64<T>(qgg + 64 * i, DK, 0, 64, qt(sl, i), op, lane);
          else dma_tile64<T>(qb + 64 * i, (int64_t)H * DK, t0, Tn, qt(sl, i), op, lane);
        }
        dma_tile64<T>(atg, 64, 0, 64, at(sl), op, lane);
        dma_tile64<T>(dob, (int64_t)H * DV, t0, Tn, ot(sl), op, lane);
      }
    } else {
      const T* kr = kb + (size_t)t0 * H * DK;
      const T* qr = qb + (size_t)t0 * H * DK;
      const T* dr = dob + (size_t)t0 * H * DV;
#pragma unroll
      for (int op = OPC * cw; op < OPC * cw + OPC; ++op) {
        const unsigned ok = tile_lane_off(op, lane, H * DK * (int)sizeof(T));
        const unsigned ow = tile_lane_off(op, lane, 64 * (int)sizeof(T));
        const unsigned oq = tile_lane_off(op, lane, DK * (int)sizeof(T));
        const unsigned oo = tile_lane_off(op, lane, H * DV * (int)sizeof(T));
#pragma unroll
        for (int i = 0; i < KT; ++i) {
          dma16s(kr + 64 * i, ok, reinterpret_cast<char*>(kt(sl, i)) + 1024 * op);
          dma16s(wtg + 64 * i, oq, reinterpret_cast<char*>(wt(sl, i)) + 1024 * op);
          if constexpr (GATED) dma16s(qgg + 64 * i, oq, reinterpret_cast<char*>(qt(sl, i)) + 1024 * op);
          else dma16s(qr + 64 * i, ok, reinterpret_cast<char*>(qt(sl, i)) + 1024 * op);
        }
        dma16s(atg, ow, reinterpret_cast<char*>(at(sl)) + 1024 * op);
        dma16s(dr, oo, reinterpret_cast<char*>(ot(sl)) + 1024 * op);
      }
    }
    if (GATED && cw == 0 && lane < 32)  // G (lanes 0-15), then e^(gamma - G) (lanes 16-31)
      dma16((lane < 16 ? Gc : Fk) + t0 + 4 * (lane & 15), gs(sl));
  };

  // staged outputs of chunk c: dh^T rows (ci DV + 32 part) and dv_new^T rows;
  // copy wave cw stores the blocks with index cw modulo the copy waves
  auto flush = [&](int c) __attribute__((always_inline)) {
    const size_t ci = (size_t)bh * NT + c;
    T* drows = (T*)(a.ws + L.dhT) + (ci * DV + 32 * part) * DK;
#pragma unroll
    for (int blk = 0; blk < NDT / 2; ++blk)
      if (blk % kStateBwdCopyWaves == cw) flush_rows<T, kStoreStream>(Stg[c & 1][blk], drows + 64 * blk, DK, lane);
    if ((NDT / 2) % kStateBwdCopyWaves == cw)
      flush_rows<T, kStoreStream>(Stg[c & 1][NDT / 2], (T*)(a.ws + L.dVnT) + (ci * DV + 32 * part) * 64, 64, lane);
  };
  if (w >= NCW) {
    // this wave's vector-memory ops per chunk of copies (G and e^(gamma - G):
    // one more for copy wave 0)
    const int nops = OPC * NTILE + (GATED && cw == 0 ? 1 : 0);
    issue(NT - 1);
    if (NSLOT == 3 && NT > 1) issue(NT - 2);
#pragma unroll 1
    for (int c = NT - 1; c >= 0; --c) {
      // chunk c's copies are done.  With three slots the previous iteration
      // ended with chunk c - 2's copies (issued after its stores), which may
      // stay in flight; the first chunk and chunk 0 wait for everything.
      if (NSLOT == 3 && c > 0 && c < NT - 1) vm_wait_n(nops);
      else vm_drain();
      const int t0 = c * kChunk;
      if (!GATED && t0 + kChunk > Tn) {
        // ungated Z = scale q^T dO with raw q tiles: dO rows past T (copies
        // of the last row) are zeroed, each copy wave in its own rows
        const int r0 = max(Tn - t0, 8 * OPC * cw), r1 = 8 * OPC * (cw + 1);
        for (int idx = lane; idx < (r1 - r0) * 8; idx += 64)
          reinterpret_cast<u32x4*>(ot(Sh + (c % NSLOT) * SLOT) + (r0 + idx / 8) * 64)[idx % 8] = u32x4{0u, 0u, 0u, 0u};
      }
      block_barrier();  // TOP
      if (NSLOT == 3) {
        if (c < NT - 1) flush(c + 1);
        if (c > 1) issue(c - 2);  // into chunk c + 1's slot
      } else {
        if (c > 0) issue(c - 1);
        if (c < NT - 1) flush(c + 1);
      }
      block_barrier();  // MID: chunk c + 1's staged outputs are read
    }
    block_barrier();  // chunk 0 staged
    flush(0);
    return;
  }

  const int p = w;  // compute wave: dS blocks ND2 p .., chunk rows 32 p ..
  f32x16 dS[ND2];
#pragma unroll
  for (int i = 0; i < ND2; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int d = 32 * (ND2 * p + i) + 8 * (e >> 2) + 4 * hh + (e & 3);
      dS[i][e] = a.dht ? a.dht[((size_t)bh * DK + d) * DV + v] : 0.f;
    }
  // this wave's dS images for chunk c (B operands of K dS', k-steps j)
  auto write_img = [&](int c) __attribute__((always_inline)) {
    u32x4* img = &Stg[c & 1][0][0] + p * (ND2 * 2 * 64);
#pragma unroll
    for (int i = 0; i < ND2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) img[(2 * i + j) * 64 + lane] = __builtin_bit_cast(u32x4, c_to_b<T>(dS[i], j));
  };
  vm_drain();  // dh_T is in registers
  write_img(NT - 1);

#pragma unroll 1
  for (int c = NT - 1; c >= 0; --c) {
    const int t0 = c * kChunk;
    block_barrier();  // TOP
    T* sl = Sh + (c % NSLOT) * SLOT;
    const T* Os = ot(sl);
    const int oc0 = 32 * (part & 1);
    const u32x4* oimg = &Stg[c & 1][0][0] + (1 - p) * (ND2 * 2 * 64);

    // the LDS operands of dVn and Z into registers first: the one wave per
    // SIMD then never waits on a read inside the MFMA chains
    v8_t<T> oop[2][2], aop[2][2], qop[ND2][2][2], kop[NDT][2], ysx[ND2][2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        oop[s2][j] = tile_tr8<T>(Os, 32 * s2, oc0, j, lane);
        aop[s2][j] = tile_tr8<T>(at(sl), 32 * s2, 32 * p, j, lane);
#pragma unroll
        for (int i = 0; i < ND2; ++i) {
          const int dt = ND2 * p + i;
          qop[i][s2][j] = tile_tr8<T>(qt(sl, dt / 2), 32 * s2, 32 * (dt & 1), j, lane);
        }
      }
#pragma unroll
    for (int db = 0; db < NDT; ++db)
#pragma unroll
      for (int j = 0; j < 2; ++j) kop[db][j] = tile_ldp8<T>(kt(sl, db / 2), 32 * p + cl, 32 * (db & 1), j, hh);
#pragma unroll
    for (int i = 0; i < ND2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) ysx[i][j] = __builtin_bit_cast(v8_t<T>, oimg[(2 * i + j) * 64 + lane]);
    __builtin_amdgcn_sched_barrier(0);

    // dVn = Aqk^T dO (rows 32 p + ..., lane column v)
    f32x16 dVn{};
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int j = 0; j < 2; ++j) dVn = mma(aop[s2][j], oop[s2][j], dVn);
    // + diag(e^(gamma - G)) K dS', dS' blocks in key-dim order (ours from
    // registers, the other wave's from its images)
    auto ys_op = [&](int db, int j) __attribute__((always_inline)) {
      return db / ND2 == p ? c_to_b<T>(dS[db % ND2], j) : ysx[db % ND2][j];
    };
    if constexpr (!GATED) {
#pragma unroll
      for (int db = 0; db < NDT; ++db)
#pragma unroll
        for (int j = 0; j < 2; ++j) dVn = mma(kop[db][j], ys_op(db, j), dVn);
    } else {
      f32x16 Pk{};
#pragma unroll
      for (int db = 0; db < NDT; ++db)
#pragma unroll
        for (int j = 0; j < 2; ++j) Pk = mma(kop[db][j], ys_op(db, j), Pk);
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        const f32x4 f4 = *reinterpret_cast<const f32x4*>(gs(sl) + 64 + 32 * p + 8 * I + 4 * hh);
#pragma unroll
        for (int r = 0; r < 4; ++r) dVn[4 * I + r] += f4[r] * Pk[4 * I + r];
      }
    }
    if (t0 + 63 >= Tn) {  // rows past T: K repeats its last row there
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (t0 + 32 * p + 8 * (e >> 2) + 4 * hh + (e & 3) >= Tn) dVn[e] = 0.f;
    }
    // Z = Qg^T dO for our key dims (independent of the chain)
    f32x16 Z[ND2];
#pragma unroll
    for (int i = 0; i < ND2; ++i) {
      Z[i] = f32x16{};
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int j = 0; j < 2; ++j) Z[i] = mma(qop[i][s2][j], oop[s2][j], Z[i]);
    }
    // our -dVn rows as B operands: for us, and as the image for the other wave
    v8_t<T> nb_own[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      nb_own[j] = c_to_b<T>(-dVn, j);
      Xv[p][j][lane] = __builtin_bit_cast(u32x4, nb_own[j]);
    }
    // dv_new^T: our 32 of the block's 64 columns, stored by a copy wave
    // during the next chunk
    stage_half<T>(dVn, p, Stg[c & 1][NDT / 2], lane);
    // W^T operands of our key dims (transposing reads of W)
    v8_t<T> wop[ND2][2][2];
#pragma unroll
    for (int i = 0; i < ND2; ++i)
#pragma unroll
      for (int it = 0; it < 2; ++it)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int dt = ND2 * p + i;
          wop[i][it][j] = tile_tr8<T>(wt(sl, dt / 2), 32 * it, 32 * (dt & 1), j, lane);
        }
    const float eg = GATED ? __expf(gs(sl)[63]) : 1.f;
    block_barrier();  // MID

    // dh^T (gradient of the state leaving the chunk, [v][d]) of our key
    // dims, staged over our dS images of this chunk (read before MID)
    if constexpr (ND2 == 2) {
      stage_rows<T>(dS[0], dS[1], Stg[c & 1][p], lane);
    } else {
      stage_half<T>(dS[0], p, Stg[c & 1][0], lane);
    }
    // dS <- e^gamma dS' + Z - W^T dVn, the -dVn rows in chunk-row order
    // (rows 0-31 first) whichever wave holds them
    v8_t<T> nb[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const v8_t<T> oth = __builtin_bit_cast(v8_t<T>, Xv[1 - p][j][lane]);
      nb[0][j] = p == 0 ? nb_own[j] : oth;
      nb[1][j] = p == 0 ? oth : nb_own[j];
    }
#pragma unroll
    for (int i = 0; i < ND2; ++i) {
      f32x16 acc = GATED ? dS[i] * eg + Z[i] : dS[i] + Z[i] * a.scale;
#pragma unroll
      for (int it = 0; it < 2; ++it)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc = mma(wop[i][it][j], nb[it][j], acc);
      dS[i] = acc;
    }
    if (c > 0) write_img(c - 1);
  }

  block_barrier();  // chunk 0's staged outputs are complete for the copy waves
  if (a.dh0) {
#pragma unroll
    for (int i = 0; i < ND2; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int d = 32 * (ND2 * p + i) + 8 * (e >> 2) + 4 * hh + (e & 3);
        a.dh0[((size_t)bh * DK + d) * DV + v] = dS[i][e];
      }
  }
}

// ---------------------------------------------------------------------------
// Kernel 2: everything of the backward that is local to a chunk: dq, then
// dk, dv, dbeta and dg through W = Tm diag(beta e^G) K and
// U = Tm diag(beta) V, Tm = (I + A)^-1.  One workgroup of eight waves per
// chunk.  Input tiles arrive by direct copies issued at the start in the
// order of use, so the dq / dW products run while the tiles of the later
// phases are still landing (rows past T repeat the last valid row and are
// masked where they could reach a result); Tm and V follow once the state
// tiles are consumed.  Wave w owns the 32 x 32 output blocks with rows
// 32 (w & 1) .. and key / value columns 32 (w >> 1) ..:
//   1a. dq = scale e^G dO S^T and dW = -dVn S^T            (S, dVn, dO, q)
//   1b. dKs = e^(gamma - G) Vn dS'^T                        (dS', Vn, k);
//       waves 0-2: the nonzero blocks of X = dO Vn^T
//   2.  Mq = scale X o e^(G_i-G_j) [j <= i] to an LDS tile, Z = X o Aqk
//   3.  dq += Mq K, dKs += Mq^T Q; dq out, dW to LDS, dG of these terms
//   4.  dv = diag(beta) Tm^T dU,  dk = dKs + diag(beta e^G) Tm^T dW
//       dTm = dU (diag(beta) V)^T + dW (diag(beta e^G) K)^T   (waves 0-3)
//       KK = K K^T, lower blocks                               (waves 4-7)
//   5.  M^T = dTm^T Tm (waves 0-3), dA^T = -Tm M^T and
//       P[a][l] = dA[a][l] beta_a e^(G_a - G_l) (l < a) (waves 4-7)
//   6.  dk += (P + P^T) K; dk, dv out; dbeta and dg (reverse cumulative
//       sum of dG within the chunk)
// dW, dKs and the dG of phase 3 stay in LDS / registers.
// ---------------------------------------------------------------------------
template <typename T, int DK, int DV, bool GATED>
__global__ __launch_bounds__(512) void delta_bwd_chunk_kernel(DeltaArgs a, DeltaLayout L) {
  constexpr int KT = DK / 64, VT = DV / 64, TE = 64 * 64;
  // St after phase 1: Mq then dTm^T / P (0 .. TE), Tm (TE .. 2 TE; phase 6:
  // the dbeta / dG reductions), V (2 TE ..).  At K = V = 64 the kernel then
  // needs under 80 KB of LDS, so two workgroups share a CU.
  constexpr int SE0 = 2 * VT * KT * TE, SE1 = 2 * TE + VT * TE;
  constexpr int SE = SE0 > SE1 ? SE0 : SE1;
  static_assert(DK % 64 == 0 && DV % 64 == 0 && DK <= 128 && DV <= 128, "64 or 128 wide");
  // S^T then dS'^T as [v][d] tiles (tile vt * KT + kt) in phase 1
  __shared__ __attribute__((aligned(16))) T St[SE];
  __shared__ __attribute__((aligned(16))) T dVt[VT * TE];  // dVn^T [v][i]
  // dO [i][v] (tiles 0 .. VT), Vn^T [v][j] (tiles VT .. 2 VT); both are read
  // only in phase 1, then their first 16 KiB are the waves' store staging
  __shared__ __attribute__((aligned(16))) T OVt[2 * VT * TE];
  T* const Ot = OVt;
  T* const Vnt = OVt + VT * TE;
  __shared__ __attribute__((aligned(16))) T Qt[KT * TE];   // q [i][d]; from phase 3: dW [i][d]
  __shared__ __attribute__((aligned(16))) T Kt[KT * TE];   // k [j][d]
  __shared__ __attribute__((aligned(16))) T At[TE];        // Aqk [i][j]; phase 5: M^T as [a][j]
  __shared__ __attribute__((aligned(16))) float Gs[64];
  __shared__ __attribute__((aligned(16))) float Bs[64];  // beta of the chunk's rows
  __shared__ float red_gi[4][64], red_kd[4][64], red_rs[2][64], red_s[8];
  // row sums over a 32-column block: Z = X o Aqk (phase 2, by i block) and
  // Q = P o KK (phase 5b, by a block)
  __shared__ float zrow[2][64], qrow[2][64];
  static_assert(2 * VT * TE * (int)sizeof(T) >= 8 * 2048, "store staging fits in the dO / Vn^T tiles");
  T* Mqt = St;

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int Tn = a.T, H = a.H, NT = a.NT;
  const int c = blockIdx.x % NT, bh = blockIdx.x / NT;
  const int b = bh / H, h = bh % H;
  const int t0 = c * kChunk;
  const size_t Tp = (size_t)NT * kChunk;
  const size_t ci = (size_t)bh * NT + c;

  const T* qb = (const T*)a.q + ((size_t)b * Tn * H + h) * DK;
  const T* kb = (const T*)a.k + ((size_t)b * Tn * H + h) * DK;
  const T* dob = (const T*)a.dout + ((size_t)b * Tn * H + h) * DV;
  const int64_t qks = (int64_t)H * DK, os = (int64_t)H * DV;

  // 0. copies, op w of every tile: phase 1a's (S, dVn, dO, q, G), then 1b's
  //    (dS', Vn, k: 2 KT VT... ops), then Aqk
  constexpr int N1B = VT * KT + VT + KT;  // copies per wave after phase 1a's
  {
    const T* hg = (const T*)(a.ctx + L.hT) + ci * DV * DK;
    const T* dhg = (const T*)(a.ws + L.dhT) + ci * DV * DK;
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) {
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
        dma_tile64<T>(hg + (size_t)64 * vt * DK + 64 * kt, DK, 0, 64, St + (vt * KT + kt) * TE, w, lane);
      dma_tile64<T>((const T*)(a.ws + L.dVnT) + (ci * DV + 64 * vt) * 64, 64, 0, 64, dVt + vt * TE, w, lane);
      dma_tile64<T>(dob + 64 * vt, os, t0, Tn, Ot + vt * TE, w, lane);
    }
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) dma_tile64<T>(qb + 64 * kt, qks, t0, Tn, Qt + kt * TE, w, lane);
    if (GATED && w == 0 && lane < 16)
      dma16(reinterpret_cast<const float*>(a.ctx + L.Gc) + (size_t)bh * Tp + t0 + 4 * lane, Gs);
    // phase 1b
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) {
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
        dma_tile64<T>(dhg + (size_t)64 * vt * DK + 64 * kt, DK, 0, 64, St + (VT * KT + vt * KT + kt) * TE, w, lane);
      dma_tile64<T>((const T*)(a.ctx + L.VnT) + (ci * DV + 64 * vt) * 64, 64, 0, 64, Vnt + vt * TE, w, lane);
    }
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) dma_tile64<T>(kb + 64 * kt, qks, t0, Tn, Kt + kt * TE, w, lane);
    dma_tile64<T>((const T*)(a.ctx + L.Aqk) + ci * 4096, 64, 0, 64, At, w, lane);
  }
  if (!GATED && tid < 64) Gs[tid] = 0.f;
  if (tid < 256) {
    red_gi[tid >> 6][tid & 63] = 0.f;
    red_kd[tid >> 6][tid & 63] = 0.f;
  }
  if (tid < 128) red_rs[tid >> 6][tid & 63] = 0.f;
  vm_wait_barrier<N1B + 1>();  // phase 1a's tiles

  const int lb = w & 1, db = w >> 1;  // row block, 32 key dims (tile db / 2, columns 32 (db & 1))
  const int r = 32 * lb + cl;         // this lane's row (i or j) in the chunk
  const bool rvalid = t0 + r < Tn;
  const bool active = db < DK / 32;
  const T* stile = St + (db / 2) * TE;  // + vt * KT * TE
  f32x16 dqa{}, dwa{}, dka{};
  float gi = 0.f, kd = 0.f;

  // 1a. dq (scaled) and dW, rows i = r, key dims 32 db ..
  if (active) {
#pragma unroll
    for (int vt = 0; vt < VT; ++vt)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const v8_t<T> hop = tile_tr8<T>(stile + vt * KT * TE, 32 * s2, 32 * (db & 1), jj, lane);
          dqa = mma(hop, tile_ldp8<T>(Ot + vt * TE, r, 32 * s2, jj, hh), dqa);
          dwa = mma(hop, tile_tr8<T>(dVt + vt * TE, 32 * s2, 32 * lb, jj, lane), dwa);
        }
    dqa *= a.scale * (GATED ? __expf(Gs[r]) : 1.f);
    dwa = -dwa;
    const char* qrow = reinterpret_cast<const char*>(Qt + (db / 2) * TE);
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const v4_t<T> q4 = *reinterpret_cast<const v4_t<T>*>(qrow + tile_off(r, 32 * (db & 1) + 8 * I + 4 * hh));
#pragma unroll
      for (int e = 0; e < 4; ++e) gi += (float)q4[e] * dqa[4 * I + e];
    }
    if (!rvalid) gi = 0.f;
  }
  vm_wait_barrier<1>();  // phase 1b's tiles

  // 1b. dKs rows j = r, key dims 32 db ..; the state-pair dot; X blocks
  const float gam = Gs[63];
  if (active) {
#pragma unroll
    for (int vt = 0; vt < VT; ++vt)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          dka = mma(tile_tr8<T>(stile + (VT * KT + vt * KT) * TE, 32 * s2, 32 * (db & 1), jj, lane),
                    tile_tr8<T>(Vnt + vt * TE, 32 * s2, 32 * lb, jj, lane), dka);
    dka *= GATED ? __expf(gam - Gs[r]) : 1.f;
    const char* krow = reinterpret_cast<const char*>(Kt + (db / 2) * TE);
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const v4_t<T> k4 = *reinterpret_cast<const v4_t<T>*>(krow + tile_off(r, 32 * (db & 1) + 8 * I + 4 * hh));
#pragma unroll
      for (int e = 0; e < 4; ++e) kd += (float)k4[e] * dka[4 * I + e];
    }
    if (!rvalid) kd = 0.f;
  }
  float sdot = 0.f;
  {
    constexpr int N16 = VT * KT * TE / 8;  // 16-byte chunks per state
    const u32x4* s0 = reinterpret_cast<const u32x4*>(St);
    const u32x4* s1 = s0 + N16;
#pragma unroll
    for (int k = 0; k < N16 / 512; ++k) {
      const v8_t<T> x = __builtin_bit_cast(v8_t<T>, s0[tid + 512 * k]);
      const v8_t<T> y = __builtin_bit_cast(v8_t<T>, s1[tid + 512 * k]);
#pragma unroll
      for (int e = 0; e < 8; ++e) sdot += (float)x[e] * (float)y[e];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sdot += __shfl_xor(sdot, off);
  }
  // waves 0..2: X block (ib, jb) = (0,0), (1,0), (1,1) as D[j][i] (lane column i);
  // wave 3: the zero block (0, 1)
  const int xib = w == 1 || w == 2, xjb = w >= 2;
  f32x16 xs{};
  if (w < 3) {
#pragma unroll
    for (int vt = 0; vt < VT; ++vt)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          xs = mma(tile_tr8<T>(Vnt + vt * TE, 32 * s2, 32 * xjb, jj, lane),
                   tile_ldp8<T>(Ot + vt * TE, 32 * xib + cl, 32 * s2, jj, hh), xs);
  }
  vm_wait_barrier<0>();  // Aqk landed; the state tiles are no longer read
  // copies for phases 4-6, landing during phases 2-3: Tm, V (rows past T
  // repeat the last valid row; beta is zeroed there), beta
  dma_tile64<T>((const T*)(a.ctx + L.Tm) + ci * 4096, 64, 0, 64, St + TE, w, lane);
#pragma unroll
  for (int vt = 0; vt < VT; ++vt)
    dma_tile64<T>((const T*)a.v + ((size_t)b * Tn * H + h) * DV + 64 * vt, os, t0, Tn, St + 2 * TE + vt * TE, w,
                  lane);
  if (w == 0) dma4(a.beta + ((size_t)b * Tn + min(t0 + lane, Tn - 1)) * H + h, Bs);

  // 2. Mq [i][j] tile and the row sums of Z = X o Aqk (waves 0-3)
  if (w < 4) {
    const int xi = 32 * xib + cl;  // this lane's i
    const float Gi = Gs[xi];
    const bool iv = t0 + xi < Tn;
    f32x16 mq, zs;
    float rs = 0.f;
    const char* arow = reinterpret_cast<const char*>(At);
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const int j0 = 32 * xjb + 8 * I + 4 * hh;
      const v4_t<T> a4 = w < 3 ? *reinterpret_cast<const v4_t<T>*>(arow + tile_off(xi, j0)) : v4_t<T>{};
      const f32x4 g4 = *reinterpret_cast<const f32x4*>(Gs + j0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = j0 + e;
        const float x = w < 3 ? xs[4 * I + e] : 0.f;
        const float z = x * (float)a4[e];
        rs += z;
        zs[4 * I + e] = z;
        // branch-free: the exponent is zeroed where the entry is masked
        const bool m = w < 3 && iv && j <= xi;
        const float g = GATED ? __expf(m ? Gi - g4[e] : 0.f) : 1.f;
        mq[4 * I + e] = m ? a.scale * x * g : 0.f;
      }
      *reinterpret_cast<v4_t<T>*>(reinterpret_cast<char*>(Mqt) + tile_off(xi, j0)) =
          to4<T>(mq[4 * I], mq[4 * I + 1], mq[4 * I + 2], mq[4 * I + 3]);
    }
    rs += __shfl_xor(rs, 32);
    if (hh == 0 && w < 3) red_rs[xjb][xi] = rs;
    // row j's sum over this block's 32 columns i (wave 3: the zero block)
    row_sums32(zs, &zrow[xib][32 * xjb], lane);
  }
  u32x4* stage = reinterpret_cast<u32x4*>(OVt) + 128 * w;
  __syncthreads();

  // 3. dq += Mq K (rows i), dKs += Mq^T Q (rows j)
  if (active) {
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        dqa = mma(tile_tr8<T>(Kt + (db / 2) * TE, 32 * jb, 32 * (db & 1), jj, lane),
                  tile_ldp8<T>(Mqt, r, 32 * jb, jj, hh), dqa);
        dka = mma(tile_tr8<T>(Qt + (db / 2) * TE, 32 * jb, 32 * (db & 1), jj, lane),
                  tile_tr8<T>(Mqt, 32 * jb, 32 * lb, jj, lane), dka);
      }
    store_rows32<T, kStoreStream>(dqa, stage, (T*)a.dq + (((size_t)b * Tn + t0 + 32 * lb) * H + h) * DK + 32 * db, qks, lane,
                    Tn - (t0 + 32 * lb));
  }
  gi += __shfl_xor(gi, 32);
  kd += __shfl_xor(kd, 32);
  if (active && hh == 0) {
    red_gi[db][r] = gi;
    red_kd[db][r] = kd;
  }
  if (lane == 0) red_s[w] = sdot;
  __syncthreads();  // phase 3 done: q, Mq and the staging of dq are free

  // dW [i][d] into the q tiles
  T* dWt = Qt;
  if (active) {
    char* t = reinterpret_cast<char*>(dWt + (db / 2) * TE);
#pragma unroll
    for (int I = 0; I < 4; ++I)
      *reinterpret_cast<v4_t<T>*>(t + tile_off(r, 32 * (db & 1) + 8 * I + 4 * hh)) =
          to4<T>(dwa[4 * I], dwa[4 * I + 1], dwa[4 * I + 2], dwa[4 * I + 3]);
  }
  // dG of the output / state terms, row tid (threads 0..63), kept for phase 6
  float dGo = 0.f;
  if (tid < 64) {
    const float cs = zrow[0][tid] + zrow[1][tid];  // sum_i Z[tid][i]
    float kdt = 0.f, git = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      kdt += red_kd[q][tid];
      git += red_gi[q][tid];
    }
    dGo = git - kdt + (red_rs[0][tid] + red_rs[1][tid]) - cs;
    // d gamma = sum_j k_j . dKs_j + e^gamma <S, dS'>, added at row 63
    float kds = kdt;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) kds += __shfl_xor(kds, off);
    if (tid == 63) {
      float st = 0.f;
#pragma unroll
      for (int q = 0; q < 8; ++q) st += red_s[q];
      dGo += kds + (GATED ? __expf(gam) : 1.f) * st;
    }
  }
  vm_wait_barrier<0>();  // Tm, V and beta landed; dW written

  // 4.-6. backward through W and U.  dU = dVn (dU^T tiles in dVt); rows j,
  // a and l index the chunk; this lane's row is r; column block cb = w >> 1, hf = cb & 1.
  const T* Tmt = St + TE;            // Tm [i][j]
  const T* Vt = St + 2 * TE;         // V [j][v]
  T* const PT = St;                  // dTm^T [j][i], then P [a][l]
  T* const MTt = At;                 // M^T as [a][j]
  // phase 6, after Tm's last read: [8][64] each
  float* const red_b = reinterpret_cast<float*>(St + TE);
  float* const red_g = red_b + 8 * 64;
  const int cb = w >> 1, hf = cb & 1;
  const bool has_dv = cb < DV / 32;
  const bool lower = hf <= lb;
  const float Bj = t0 + r < Tn ? Bs[r] : 0.f, Gj = Gs[r];
  const float eGj = GATED ? __expf(Gj) : 1.f;
  float db_part = 0.f, dg_part = 0.f, rq_part = 0.f;

  // 4a. dv[j][v] = beta_j (Tm^T dU)[j][v], values 32 cb .., as D[v][j]
  f32x16 dvx{};
  if (has_dv) {
    const T* du = dVt + (cb / 2) * TE;
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        dvx = mma(tile_ldp8<T>(du, 32 * (cb & 1) + cl, 32 * ib, jj, hh), tile_tr8<T>(Tmt, 32 * ib, 32 * lb, jj, lane),
                  dvx);
    // dbeta_j += v_j . (Tm^T dU)_j
    const char* vt = reinterpret_cast<const char*>(Vt + (cb / 2) * TE);
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const v4_t<T> v4 = *reinterpret_cast<const v4_t<T>*>(vt + tile_off(r, 32 * (cb & 1) + 8 * I + 4 * hh));
#pragma unroll
      for (int e = 0; e < 4; ++e) db_part += (float)v4[e] * dvx[4 * I + e];
    }
    dvx *= Bj;
  }
  // 4b. dk += beta_j e^G_j (Tm^T dW)[j][d], key dims 32 db .., as D[d][j]
  if (active) {
    f32x16 x{};
    const T* dwt = dWt + (db / 2) * TE;
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        x = mma(tile_tr8<T>(dwt, 32 * ib, 32 * (db & 1), jj, lane), tile_tr8<T>(Tmt, 32 * ib, 32 * lb, jj, lane), x);
    const char* krow = reinterpret_cast<const char*>(Kt + (db / 2) * TE);
    float kdot = 0.f;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const v4_t<T> k4 = *reinterpret_cast<const v4_t<T>*>(krow + tile_off(r, 32 * (db & 1) + 8 * I + 4 * hh));
#pragma unroll
      for (int e = 0; e < 4; ++e) kdot += (float)k4[e] * x[4 * I + e];
    }
    dka += x * (Bj * eGj);
    db_part += eGj * kdot;
    dg_part += Bj * eGj * kdot;
  }
  // 4c. waves 0-3: dTm block (rows i = 32 hf .., lane column j = r):
  //     beta_j (dU_i . v_j) + beta_j e^G_j (dW_i . k_j);
  //     waves 4-7: KK block (rows l = 32 hf .., lane column a = r), lower only
  f32x16 dtm{}, kk{};
  if (w < 4) {
    f32x16 d2{};
#pragma unroll
    for (int vt = 0; vt < VT; ++vt)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          dtm = mma(tile_tr8<T>(dVt + vt * TE, 32 * s2, 32 * hf, jj, lane),
                    tile_ldp8<T>(Vt + vt * TE, r, 32 * s2, jj, hh), dtm);
#pragma unroll
    for (int kq = 0; kq < DK / 16; ++kq)
      d2 = mma(tile_ld8<T>(dWt + (kq / 4) * TE, 32 * hf + cl, 16 * (kq % 4) + 8 * hh),
               tile_ld8<T>(Kt + (kq / 4) * TE, r, 16 * (kq % 4) + 8 * hh), d2);
    dtm = (dtm + d2 * eGj) * Bj;
    char* t = reinterpret_cast<char*>(PT);
#pragma unroll
    for (int I = 0; I < 4; ++I)
      *reinterpret_cast<v4_t<T>*>(t + tile_off(r, 32 * hf + 8 * I + 4 * hh)) =
          to4<T>(dtm[4 * I], dtm[4 * I + 1], dtm[4 * I + 2], dtm[4 * I + 3]);
  } else if (lower) {
#pragma unroll
    for (int kq = 0; kq < DK / 16; ++kq)
      kk = mma(tile_ld8<T>(Kt + (kq / 4) * TE, 32 * hf + cl, 16 * (kq % 4) + 8 * hh),
               tile_ld8<T>(Kt + (kq / 4) * TE, r, 16 * (kq % 4) + 8 * hh), kk);
  }
  __syncthreads();

  // 5a. waves 0-3: M^T[j][a] = sum_i dTm^T[j][i] Tm[i][a], block (rows j =
  //     32 hf .., lane column a = r), stored as a [a][j] tile
  if (w < 4) {
    f32x16 x{};
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        x = mma(tile_ldp8<T>(PT, 32 * hf + cl, 32 * ib, jj, hh), tile_tr8<T>(Tmt, 32 * ib, 32 * lb, jj, lane), x);
    char* t = reinterpret_cast<char*>(MTt);
#pragma unroll
    for (int I = 0; I < 4; ++I)
      *reinterpret_cast<v4_t<T>*>(t + tile_off(r, 32 * hf + 8 * I + 4 * hh)) =
          to4<T>(x[4 * I], x[4 * I + 1], x[4 * I + 2], x[4 * I + 3]);
  }
  __syncthreads();

  // 5b. waves 4-7: dA^T[l][a] = -sum_j Tm[l][j] M^T[j][a] (rows l = 32 hf ..,
  //     lane a = r); P[a][l] = dA[a][l] beta_a e^(G_a - G_l) and Q = P o KK
  //     for l < a.  P goes to a [a][l] tile over dTm^T, Q^T to fp32 [l][a].
  if (w >= 4) {
    f32x16 x{};
    if (lower) {
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          x = mma(tile_ldp8<T>(Tmt, 32 * hf + cl, 32 * jb, jj, hh), tile_ldp8<T>(MTt, r, 32 * jb, jj, hh), x);
    }
    f32x16 pq, qq;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int l = 32 * hf + 8 * (e >> 2) + 4 * hh + (e & 3);
      // branch-free: the exponent is zeroed where the entry is masked
      const bool m = lower && l < r;
      const float dA = -x[e];
      const float Gl = reinterpret_cast<const f32x4*>(Gs + 32 * hf + 8 * (e >> 2) + 4 * hh)[0][e & 3];
      const float g = GATED ? __expf(m ? Gj - Gl : 0.f) : 1.f;
      const float p = m ? dA * Bj * g : 0.f;
      const float q = p * kk[e];
      db_part += m ? dA * kk[e] * g : 0.f;
      rq_part += q;
      pq[e] = p;
      qq[e] = q;
    }
    char* t = reinterpret_cast<char*>(PT);
#pragma unroll
    for (int I = 0; I < 4; ++I)
      *reinterpret_cast<v4_t<T>*>(t + tile_off(r, 32 * hf + 8 * I + 4 * hh)) =
          to4<T>(pq[4 * I], pq[4 * I + 1], pq[4 * I + 2], pq[4 * I + 3]);
    // row l's sum over this wave's 32 columns a
    row_sums32(qq, &qrow[lb][32 * hf], lane);
  }
  __syncthreads();

  // 6. dk[a][d] += sum_l K[l][d] (P[a][l] + P[l][a]); dk and dv out
  if (active) {
    const T* ktile = Kt + (db / 2) * TE;
#pragma unroll
    for (int lbk = 0; lbk < 2; ++lbk)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const v8_t<T> kop = tile_tr8<T>(ktile, 32 * lbk, 32 * (db & 1), jj, lane);
        dka = mma(kop, tile_ldp8<T>(PT, r, 32 * lbk, jj, hh), dka);
        dka = mma(kop, tile_tr8<T>(PT, 32 * lbk, 32 * lb, jj, lane), dka);
      }
    store_rows32<T, kStoreStream>(dka, stage, (T*)a.dk + (((size_t)b * Tn + t0 + 32 * lb) * H + h) * DK + 32 * db, qks, lane,
                    Tn - (t0 + 32 * lb));
  }
  if (has_dv)
    store_rows32<T, kStoreStream>(dvx, stage, (T*)a.dv + (((size_t)b * Tn + t0 + 32 * lb) * H + h) * DV + 32 * cb, os, lane,
                    Tn - (t0 + 32 * lb));

  db_part += __shfl_xor(db_part, 32);
  dg_part += __shfl_xor(dg_part, 32);
  rq_part += __shfl_xor(rq_part, 32);
  if (hh == 0) {
    red_b[w * 64 + r] = db_part;
    red_g[w * 64 + r] = dg_part + rq_part;
  }
  __syncthreads();
  if (tid < 64) {
    // column part of dG: sum_a Q[a][l], l = tid
    const float cq = qrow[0][tid] + qrow[1][tid];
    const int t = t0 + tid;
    const int l2 = tid >> 5;  // row block of this row; waves l2 + 2 q hold it
    float dbeta = 0.f, gsum = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      dbeta += red_b[(l2 + 2 * q) * 64 + tid];
      gsum += red_g[(l2 + 2 * q) * 64 + tid];
    }
    float x = dGo + gsum - cq;
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
  hipError_t e = hipSuccess;
  if (a.stages & 1) {
    delta_state_bwd_kernel<T, DK, DV, GATED><<<dim3(BH * (DV / 32)), dim3(state_bwd_threads()), 0, stream>>>(a, L);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (a.stages & 2) {
    delta_bwd_chunk_kernel<T, DK, DV, GATED><<<dim3(BH * a.NT), dim3(512), 0, stream>>>(a, L);
    e = hipGetLastError();
  }
  return e;
}

#define LINATT_DELTA_BWD_INST(T, DK, DV)                                              \
  template hipError_t launch_delta_bwd<T, DK, DV, false>(const DeltaArgs&, hipStream_t); \
  template hipError_t launch_delta_bwd<T, DK, DV, true>(const DeltaArgs&, hipStream_t);

LINATT_DELTA_SHAPES(LINATT_DELTA_BWD_INST)

}  // namespace linatt
