// Chunked (gated) delta rule, forward, for gfx950.
//
// Replaces the forward of fla.ops.delta_rule.chunk_delta_rule and
// fla.ops.gated_delta_rule.chunk_gated_delta_rule (third-party
// flash-linear-attention==0.5.0, pinned at scripts/setup.sh:27 of the
// reference; reached through model_type delta_net / gated_deltanet,
// configs/model/200m/delta_net_200m.yaml:3, gated_deltanet_200m.yaml:4).
// Algorithm: the WY/UT chunk form of Yang et al. (NeurIPS 2024) with the
// gate of Yang, Kautz, Hatamizadeh (ICLR 2025).  Per chunk of 64 tokens
// with G the chunk-local inclusive cumsum of g and gamma = G at the last
// row:
//
//   A   = strict_lower(diag(beta) K K^T o e^(G_i - G_j))
//   Tm  = (I + A)^-1                       (fp32, in LDS)
//   W   = Tm diag(beta e^G) K,   U = Tm diag(beta) V
//   Vn  = U - W S                          (S: state entering the chunk)
//   o   = scale e^G o (Q S) + Aqk Vn,      Aqk = scale (Q K^T) o e^(G_i-G_j), j <= i
//   S  <- e^gamma S + (diag(e^(gamma - G)) K)^T Vn
//
// Kernel 1 (delta_prep) is parallel over (batch, head, chunk): G, the Gram
// matrix, the triangular solve, W, U and the transposed / pre-scaled
// operand copies the state pass reads.  Kernel 2 (delta_state_fwd) walks
// the chunks in order: one wave per (batch, head, 32 value columns) keeps
// its slice of S in MFMA accumulators and writes v_new and the per-chunk
// states, with every operand read straight into registers.  Kernel 3
// (delta_out) forms o in parallel over chunks from those.
#include "common.h"
#include "delta_kernels.h"

namespace linatt {

namespace {
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
}  // namespace

DeltaLayout delta_layout(int B, int T, int H, int DK, int DV, int eb) {
  DeltaLayout L{};
  const size_t NT = (size_t)(T + kChunk - 1) / kChunk, Tp = NT * kChunk, BH = (size_t)B * H;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = align256(off + bytes); return o; };
  L.Gc = take(BH * Tp * 4);
  L.Tm = take(BH * NT * 4096 * eb);
  L.W = take(BH * Tp * DK * eb);
  L.UT = take(BH * Tp * DV * eb);
  L.WT = take(BH * Tp * DK * eb);
  L.KdT = take(BH * Tp * DK * eb);
  L.QgT = take(BH * Tp * DK * eb);
  L.Aqk = take(BH * NT * 4096 * eb);
  L.AqkT = take(BH * NT * 4096 * eb);
  L.hT = take(BH * NT * DK * DV * eb);
  L.VnT = take(BH * Tp * DV * eb);
  L.ctx_bytes = off;
  off = 0;
  L.dVnT = take(BH * Tp * DV * eb);
  L.dhT = take(BH * NT * DK * DV * eb);
  L.dW = take(BH * Tp * DK * 4);
  L.dKp = take(BH * Tp * DK * 4);
  L.dGp = take(BH * Tp * 4);
  L.bwd_bytes = off;
  return L;
}

// ---------------------------------------------------------------------------
// Kernel 1: per-chunk preparation.
// ---------------------------------------------------------------------------
template <typename T, int DK, int DV, bool GATED>
__global__ __launch_bounds__(256) void delta_prep_kernel(DeltaArgs a, DeltaLayout L) {
  constexpr int PK = DK + 8;   // natural K tile pitch
  constexpr int PX = 64 + 8;   // transposed tile pitch
  constexpr int PA = 68;       // fp32 A / Tm pitch
  constexpr int XR = DK > DV ? DK : DV;
  constexpr int U0 = (64 * PK > XR * PX ? 64 * PK : XR * PX);
  __shared__ __attribute__((aligned(16))) T Un[U0];          // K natural, then X^T tiles
  __shared__ __attribute__((aligned(16))) float As[64 * PA];  // A, then Tm as T (pitch PX)
  __shared__ __attribute__((aligned(16))) float Ts[64 * PA];  // Tm fp32
  __shared__ __attribute__((aligned(16))) float Gs[64], Bs[64], Sc[64];

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int Tn = a.T, H = a.H, NT = a.NT;
  const int c = blockIdx.x % NT, bh = blockIdx.x / NT;
  const int b = bh / H, h = bh % H;
  const int t0 = c * kChunk;
  const size_t Tp = (size_t)NT * kChunk;
  const size_t ci = (size_t)bh * NT + c;

  T* Kn = Un;
  T* Xt = Un;
  T* Tt = reinterpret_cast<T*>(As);
  float* Gc = reinterpret_cast<float*>(a.ctx + L.Gc);

  const T* qb = (const T*)a.q + ((size_t)b * Tn * H + h) * DK;
  const T* kb = (const T*)a.k + ((size_t)b * Tn * H + h) * DK;
  const T* vb = (const T*)a.v + ((size_t)b * Tn * H + h) * DV;
  const int64_t qks = (int64_t)H * DK, vs = (int64_t)H * DV;

  // beta and G (inclusive cumsum of g; rows past T add 0, so G[63] = gamma).
  if (tid < 64) {
    const int t = t0 + tid;
    float bt = 0.f, gt = 0.f;
    if (t < Tn) {
      bt = a.beta[((size_t)b * Tn + t) * H + h];
      if constexpr (GATED) gt = a.g[((size_t)b * Tn + t) * H + h];
    }
    Bs[tid] = bt;
    float x = gt;
    if constexpr (GATED) {
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(x, off);
        if (tid >= off) x += y;
      }
      Gc[(size_t)bh * Tp + t0 + tid] = x;
    }
    Gs[tid] = x;
  }
  for (int idx = tid; idx < 64 * PA; idx += 256) Ts[idx] = 0.f;
  load_tile64x<T, T, DK, PK, 1, true, false>(kb, t0, Tn, qks, Kn, nullptr, tid, nullptr);
  __syncthreads();

  // Gram (wave w: tile (w >> 1, w & 1)) -> A in LDS; Q K^T -> Aqk, Aqk^T.
  {
    const int ai = w >> 1, bj = w & 1;
    f32x16 kk{};
#pragma unroll
    for (int s = 0; s < DK / 16; ++s)
      kk = mma(ld8<T>(Kn + (32 * ai + cl) * PK + 16 * s + 8 * hh),
               ld8<T>(Kn + (32 * bj + cl) * PK + 16 * s + 8 * hh), kk);
    const int j = 32 * bj + cl;
#pragma unroll
    for (int I = 0; I < 4; ++I)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 32 * ai + 8 * I + 4 * hh + r;
        float val = 0.f;
        if (i > j) {
          val = Bs[i] * kk[4 * I + r];
          if constexpr (GATED) val *= __expf(Gs[i] - Gs[j]);
        }
        As[i * PA + j] = val;
      }
    // D[j][i] = k_j . q_i   (j-tile ai, i-tile bj; lane column i)
    const int i = 32 * bj + cl;
    const bool qv = t0 + i < Tn;
    f32x16 qk{};
#pragma unroll
    for (int s = 0; s < DK / 16; ++s)
      qk = mma(ld8<T>(Kn + (32 * ai + cl) * PK + 16 * s + 8 * hh),
               qv ? ld8<T>(qb + (int64_t)(t0 + i) * qks + 16 * s + 8 * hh) : zero8<T>(), qk);
    T* aq = (T*)(a.ctx + L.Aqk) + ci * 4096;
    T* aqt = (T*)(a.ctx + L.AqkT) + ci * 4096;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      float vals[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int jj = 32 * ai + 8 * I + 4 * hh + r;
        float val = 0.f;
        if (jj <= i) {
          val = a.scale * qk[4 * I + r];
          if constexpr (GATED) val *= __expf(Gs[i] - Gs[jj]);
        }
        vals[r] = val;
        aqt[jj * 64 + i] = (T)val;
      }
      st4<T>(aq + i * 64 + 32 * ai + 8 * I + 4 * hh, to4<T>(vals[0], vals[1], vals[2], vals[3]));
    }
  }
  __syncthreads();

  // Tm = (I + A)^-1 by 16-row blocks: off-block rows from the finished
  // rows (all threads), then forward substitution inside the diagonal block
  // with one column per lane (wave 0).
#pragma unroll 1
  for (int R = 0; R < 4; ++R) {
    if (R > 0) {
      const int i = 16 * R + (tid >> 4);
      const int cg = tid & 15;
      for (int m = 0; m < R; ++m) {
        const int cc = cg + 16 * m;
        float y = 0.f;
        for (int j = cc; j < 16 * R; ++j) y -= As[i * PA + j] * Ts[j * PA + cc];
        Ts[i * PA + cc] = y;
      }
    }
    __syncthreads();
    if (tid < 64) {
      const int cc = tid;
      float x[16];
#pragma unroll
      for (int ii = 0; ii < 16; ++ii) {
        const int i = 16 * R + ii;
        float acc = (cc == i ? 1.f : 0.f) + (cc < 16 * R ? Ts[i * PA + cc] : 0.f);
#pragma unroll
        for (int jj = 0; jj < ii; ++jj) acc -= As[i * PA + 16 * R + jj] * x[jj];
        x[ii] = (cc <= i) ? acc : 0.f;
        Ts[i * PA + cc] = x[ii];
      }
    }
    __syncthreads();
  }

  // Tm -> T (natural [i][j], pitch PX) over A, and to the context.
  {
    T* tmg = (T*)(a.ctx + L.Tm) + ci * 4096;
    for (int idx = tid; idx < 4096; idx += 256) {
      const int i = idx >> 6, j = idx & 63;
      const T val = (T)Ts[i * PA + j];
      Tt[i * PX + j] = val;
      tmg[idx] = val;
    }
  }
  if (tid < 64) Sc[tid] = a.scale * (GATED ? __expf(Gs[tid]) : 1.f);
  __syncthreads();

  // (scale e^G q)^T and (e^(gamma - G) k)^T per chunk, through LDS.
  {
    load_tile64x<T, T, DK, 1, PX, false, true>(qb, t0, Tn, qks, nullptr, Xt, tid, Sc);
    __syncthreads();
    T* dst = (T*)(a.ctx + L.QgT) + ci * DK * 64;
    for (int idx = tid; idx < DK * 64; idx += 256) dst[idx] = Xt[(idx >> 6) * PX + (idx & 63)];
    __syncthreads();
    if (tid < 64) Sc[tid] = GATED ? __expf(Gs[63] - Gs[tid]) : 1.f;
    __syncthreads();
    load_tile64x<T, T, DK, 1, PX, false, true>(kb, t0, Tn, qks, nullptr, Xt, tid, Sc);
    __syncthreads();
    dst = (T*)(a.ctx + L.KdT) + ci * DK * 64;
    for (int idx = tid; idx < DK * 64; idx += 256) {
      const int i = idx & 63;
      dst[(idx & ~63) + (i & 32) + opord32(i & 31)] = Xt[(idx >> 6) * PX + i];
    }
    __syncthreads();
    if (tid < 64) Sc[tid] = Bs[tid] * (GATED ? __expf(Gs[tid]) : 1.f);
    __syncthreads();
  }

  // W = Tm (diag(beta e^G) K): D[d][i] = sum_j Xt[d][j] Tt[i][j]; lane column i.
  {
    load_tile64x<T, T, DK, 1, PX, false, true>(kb, t0, Tn, qks, nullptr, Xt, tid, Sc);
    __syncthreads();
    const int it = w & 1;
    const int i = 32 * it + cl;
    T* wrow = (T*)(a.ctx + L.W) + ((size_t)bh * Tp + t0 + i) * DK;
    T* wt = (T*)(a.ctx + L.WT) + ci * DK * 64;
#pragma unroll
    for (int m = 0; m < DK / 64; ++m) {
      const int dt = (w >> 1) + 2 * m;
      f32x16 acc{};
#pragma unroll
      for (int s = 0; s < 4; ++s)
        acc = mma(ld8<T>(Xt + (32 * dt + cl) * PX + 16 * s + 8 * hh),
                  ld8<T>(Tt + i * PX + 16 * s + 8 * hh), acc);
      const int ip = (i & 32) + opord32(i & 31);
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        const int d = 32 * dt + 8 * I + 4 * hh;
        st4<T>(wrow + 32 * dt + opord32(8 * I + 4 * hh),
               to4<T>(acc[4 * I], acc[4 * I + 1], acc[4 * I + 2], acc[4 * I + 3]));
#pragma unroll
        for (int r = 0; r < 4; ++r) wt[(d + r) * 64 + ip] = (T)acc[4 * I + r];
      }
    }
    __syncthreads();
    if (tid < 64) Sc[tid] = Bs[tid];
    __syncthreads();
  }

  // U = Tm (diag(beta) V).
  {
    load_tile64x<T, T, DV, 1, PX, false, true>(vb, t0, Tn, vs, nullptr, Xt, tid, Sc);
    __syncthreads();
    const int it = w & 1;
    const int i = 32 * it + cl;
    T* ut = (T*)(a.ctx + L.UT) + ci * DV * 64;
#pragma unroll
    for (int m = 0; m < DV / 64; ++m) {
      const int vt = (w >> 1) + 2 * m;
      f32x16 acc{};
#pragma unroll
      for (int s = 0; s < 4; ++s)
        acc = mma(ld8<T>(Xt + (32 * vt + cl) * PX + 16 * s + 8 * hh),
                  ld8<T>(Tt + i * PX + 16 * s + 8 * hh), acc);
      const int ip = (i & 32) + opord32(i & 31);
#pragma unroll
      for (int e = 0; e < 16; ++e)
        ut[(32 * vt + 8 * (e >> 2) + 4 * hh + (e & 3)) * 64 + ip] = (T)acc[e];
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel 2: sequential state pass.  One workgroup per (b, h) with one wave
// per 32 value columns; S[d][v] lives in DK/32 accumulator tiles with lane
// column v.  Per chunk the chain is
//   v_new = U - W S  ->  S <- e^gamma S + Kd^T v_new.
// W and Kd^T are the same for every wave of the head and U^T is split by
// wave: all three reach LDS by direct global->LDS copies into a ring of three
// slots, issued two chunks ahead (each wave copies 1/NW of W and of Kd^T and
// its own U^T rows).  Tiles are stored XOR-swizzled by 16-byte chunk so the
// operand reads of 16 consecutive rows hit distinct banks.
// ---------------------------------------------------------------------------

// Wave-level copy of 1 KiB (64 x 16 bytes) of a row-major tile with CPR
// 16-byte chunks per row into its swizzled LDS image: op covers tile chunks
// [64 op, 64 op + 64).
template <int CPR>
__device__ __forceinline__ void dma_tile_1k(const u32x4* g, u32x4* lds, int op, int lane) {
  const int row = (64 * op + lane) / CPR, slot = lane % CPR;
  const int ch = swz_slot<CPR>(row, slot) - row * CPR;  // global chunk held by this slot
  dma16(g + row * CPR + ch, lds + 64 * op);
}

template <typename T, int DK, int DV, bool GATED>
__global__ __launch_bounds__(64 * (DV / 32)) void delta_state_fwd_kernel(DeltaArgs a, DeltaLayout L,
                                                                       const float* __restrict__ gcum) {
  constexpr int NDT = DK / 32, NW = DV / 32;
  constexpr int WT16 = 64 * DK * (int)sizeof(T) / 16;   // 16-byte chunks per W (= Kd^T) tile
  constexpr int UT16 = 32 * 64 * (int)sizeof(T) / 16;   // per wave's U^T rows
  constexpr int WCPR = DK * (int)sizeof(T) / 16;         // chunks per W row
  constexpr int KCPR = 64 * (int)sizeof(T) / 16;         // chunks per Kd^T / U^T row
  constexpr int SLOT = 2 * WT16 + NW * UT16;             // W | Kd^T | U^T per chunk
  constexpr int WOPS = WT16 / 64 / NW, UOPS = UT16 / 64;  // 1 KiB copies per wave
  constexpr int DMA_PER_CHUNK = 2 * WOPS + UOPS;
  static_assert(WOPS * 64 * NW == WT16 && UOPS * 64 == UT16, "tile split");
  __shared__ __attribute__((aligned(16))) u32x4 Sh[3 * SLOT];

  const int lane = threadIdx.x & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int NT = a.NT;
  const int bh = blockIdx.x;
  const int v = 32 * w + cl;
  const size_t Tp = (size_t)NT * kChunk;

  // gcum = the Gc context buffer, passed on its own as __restrict__ so the
  // per-chunk gate is a scalar load (no vector-memory wait in the chain)
  const float* Gc = gcum + (size_t)bh * Tp;
  const u32x4* Wg = reinterpret_cast<const u32x4*>(a.ctx + L.W) + (size_t)bh * NT * WT16;
  const u32x4* Kg = reinterpret_cast<const u32x4*>(a.ctx + L.KdT) + (size_t)bh * NT * WT16;
  const u32x4* Ug = reinterpret_cast<const u32x4*>(a.ctx + L.UT) + (size_t)bh * NT * NW * UT16;

  // this wave's share of chunk c into ring slot c % 3
  auto issue = [&](int c) __attribute__((always_inline)) {
    u32x4* sl = Sh + (c % 3) * SLOT;
#pragma unroll
    for (int i = 0; i < WOPS; ++i) {
      dma_tile_1k<WCPR>(Wg + (size_t)c * WT16, sl, WOPS * w + i, lane);
      dma_tile_1k<KCPR>(Kg + (size_t)c * WT16, sl + WT16, WOPS * w + i, lane);
    }
#pragma unroll
    for (int i = 0; i < UOPS; ++i)
      dma_tile_1k<KCPR>(Ug + ((size_t)c * NW + w) * UT16, sl + 2 * WT16 + w * UT16, i, lane);
  };

  f32x16 S[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int d = 32 * dt + 8 * (e >> 2) + 4 * hh + (e & 3);
      S[dt][e] = a.h0 ? a.h0[((size_t)bh * DK + d) * DV + v] : 0.f;
    }

  vm_drain();  // h0 is in registers
  issue(0);
  if (NT > 1) issue(1);
#pragma unroll 1
  for (int c = 0; c < NT; ++c) {
    // chunk c landed for every wave (only chunk c + 1's copies may remain in
    // flight), and every wave is done with chunk c - 1, whose slot is refilled
    if (c + 1 < NT) vm_wait_barrier<DMA_PER_CHUNK>();
    else vm_wait_barrier<0>();
    if (c + 2 < NT) issue(c + 2);
    const size_t ci = (size_t)bh * NT + c;
    const u32x4* Ws = Sh + (c % 3) * SLOT;
    const u32x4* Ks = Ws + WT16;
    const u32x4* Us = Ws + 2 * WT16 + w * UT16;

    // P = W S  (W rows 32 it + cl, key dims in operand order)
    f32x16 P[2];
    P[0] = P[1] = f32x16{};
#pragma unroll
    for (int db = 0; db < NDT; ++db)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const v8_t<T> ys = c_to_b<T>(S[db], j);
#pragma unroll
        for (int it = 0; it < 2; ++it)
          P[it] = mma(__builtin_bit_cast(v8_t<T>, Ws[swz_slot<WCPR>(32 * it + cl, 4 * db + 2 * j + hh)]), ys, P[it]);
      }

    // v_new = U - P (rows past T are zero in U and W); U^T rows of this
    // wave, chunk rows in operand order
    f32x16 Vn[2];
#pragma unroll
    for (int it = 0; it < 2; ++it)
#pragma unroll
      for (int jq = 0; jq < 2; ++jq) {
        const v8_t<T> u8 = __builtin_bit_cast(v8_t<T>, Us[swz_slot<KCPR>(cl, 4 * it + 2 * jq + hh)]);
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const int I = 2 * jq + s2;
#pragma unroll
          for (int r = 0; r < 4; ++r) Vn[it][4 * I + r] = (float)u8[4 * s2 + r] - P[it][4 * I + r];
        }
      }
    // v_new^T and the state entering the chunk (h^T, [v][d]) go out through
    // this wave's U^T area of the slot, which the wave alone reads and has
    // finished with
    u32x4* stage = const_cast<u32x4*>(Us);
    T* rows = (T*)(a.ctx + L.VnT) + (ci * DV + 32 * w) * 64;
    store_rows_staged<T>(Vn[0], Vn[1], stage, rows, 64, lane);
    T* hrows = (T*)(a.ctx + L.hT) + (ci * DV + 32 * w) * DK;
#pragma unroll
    for (int blk = 0; blk < NDT / 2; ++blk)
      store_rows_staged<T>(S[2 * blk], S[2 * blk + 1], stage, hrows + 64 * blk, DK, lane);

    // S <- e^gamma S + Kd^T v_new  (Kd^T rows 32 dt + cl, chunk rows in operand order)
    const float eg = GATED ? __expf(Gc[c * kChunk + 63]) : 1.f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      if constexpr (GATED) S[dt] *= eg;
#pragma unroll
      for (int it = 0; it < 2; ++it)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          S[dt] = mma(__builtin_bit_cast(v8_t<T>, Ks[swz_slot<KCPR>(32 * dt + cl, 4 * it + 2 * jj + hh)]),
                      c_to_b<T>(Vn[it], jj), S[dt]);
    }
  }

  if (a.ht) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int d = 32 * dt + 8 * (e >> 2) + 4 * hh + (e & 3);
        a.ht[((size_t)bh * DK + d) * DV + v] = S[dt][e];
      }
  }
}

// ---------------------------------------------------------------------------
// Kernel 3: output, parallel over (b, h, chunk):
//   o = scale e^G (Q h_c) + Aqk v_new.
// Wave w: rows 32 (w & 1) + lane (lane column i), value half w >> 1.
// ---------------------------------------------------------------------------
template <typename T, int DK, int DV, bool GATED>
__global__ __launch_bounds__(256) void delta_out_kernel(DeltaArgs a, DeltaLayout L) {
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int Tn = a.T, H = a.H, NT = a.NT;
  const int c = blockIdx.x % NT, bh = blockIdx.x / NT;
  const int b = bh / H, h = bh % H;
  const int t0 = c * kChunk;
  const size_t Tp = (size_t)NT * kChunk;
  const size_t ci = (size_t)bh * NT + c;
  const int i = 32 * (w & 1) + cl, ti = t0 + i;
  const bool valid = ti < Tn;

  const T* qrow = (const T*)a.q + (((size_t)b * Tn + ti) * H + h) * DK;
  const T* arow = (const T*)(a.ctx + L.Aqk) + ci * 4096 + i * 64;
  const T* hg = (const T*)(a.ctx + L.hT) + ci * DV * DK;
  const T* vg = (const T*)(a.ctx + L.VnT) + ci * DV * 64;
  v8_t<T> yq[DK / 16], ya[4];
#pragma unroll
  for (int s = 0; s < DK / 16; ++s) yq[s] = valid ? ld8<T>(qrow + 16 * s + 8 * hh) : zero8<T>();
#pragma unroll
  for (int s = 0; s < 4; ++s) ya[s] = ld8<T>(arow + 16 * s + 8 * hh);
  float f = a.scale;
  if constexpr (GATED) f *= __expf(reinterpret_cast<const float*>(a.ctx + L.Gc)[(size_t)bh * Tp + t0 + i]);
  T* orow = (T*)a.o + (((size_t)b * Tn + ti) * H + h) * DV;
#pragma unroll
  for (int m = 0; m < DV / 64; ++m) {
    const int vt = (w >> 1) * (DV / 64) + m;
    f32x16 acc{};
#pragma unroll
    for (int s = 0; s < DK / 16; ++s)
      acc = mma(ld8<T>(hg + (32 * vt + cl) * DK + 16 * s + 8 * hh), yq[s], acc);
    acc *= f;
#pragma unroll
    for (int s = 0; s < 4; ++s) acc = mma(ld8<T>(vg + (32 * vt + cl) * 64 + 16 * s + 8 * hh), ya[s], acc);
    if (valid) {
#pragma unroll
      for (int I = 0; I < 4; ++I)
        st4<T>(orow + 32 * vt + 8 * I + 4 * hh,
               to4<T>(acc[4 * I], acc[4 * I + 1], acc[4 * I + 2], acc[4 * I + 3]));
    }
  }
}

template <typename T, int DK, int DV, bool GATED>
hipError_t launch_delta_fwd(const DeltaArgs& a, hipStream_t stream) {
  const DeltaLayout L = delta_layout(a.B, a.T, a.H, DK, DV, sizeof(T));
  const int BH = a.B * a.H;
  delta_prep_kernel<T, DK, DV, GATED><<<dim3(BH * a.NT), dim3(256), 0, stream>>>(a, L);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  delta_state_fwd_kernel<T, DK, DV, GATED><<<dim3(BH), dim3(64 * (DV / 32)), 0, stream>>>(
      a, L, reinterpret_cast<const float*>(a.ctx + L.Gc));
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  delta_out_kernel<T, DK, DV, GATED><<<dim3(BH * a.NT), dim3(256), 0, stream>>>(a, L);
  return hipGetLastError();
}

#define LINATT_DELTA_FWD_INST(T, DK, DV)                                              \
  template hipError_t launch_delta_fwd<T, DK, DV, false>(const DeltaArgs&, hipStream_t); \
  template hipError_t launch_delta_fwd<T, DK, DV, true>(const DeltaArgs&, hipStream_t);

LINATT_DELTA_SHAPES(LINATT_DELTA_FWD_INST)

}  // namespace linatt
