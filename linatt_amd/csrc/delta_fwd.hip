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
// states, with every operand read straight into registers, and forms o from
// the states it stages.
#include "common.h"
#include "delta_kernels.h"
#include "tri_inv.h"

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
  L.Fk = take(BH * Tp * 4);
  L.Tm = take(BH * NT * 4096 * eb);
  L.W = take(BH * Tp * DK * eb);
  L.UT = take(BH * Tp * DV * eb);
  L.KdT = take(BH * Tp * DK * eb);
  L.Qg = take(BH * Tp * DK * eb);
  L.Aqk = take(BH * NT * 4096 * eb);
  L.hT = take(BH * NT * DK * DV * eb);
  L.VnT = take(BH * Tp * DV * eb);
  L.ctx_bytes = off;
  off = 0;
  L.dVnT = take(BH * Tp * DV * eb);
  L.dhT = take(BH * NT * DK * DV * eb);
  L.bwd_bytes = off;
  return L;
}

// ---------------------------------------------------------------------------
// Kernel 1: per-chunk preparation, one workgroup of four waves per chunk.
// The chunk's K and V rows reach LDS by direct copies at the start (rows
// past T repeat the last valid row; beta = 0 there zeroes every use); q rows
// go straight to registers.  Phases (barrier between each):
//   1. Gram A (fp32, LDS) by waves 1-3; Aqk rows 0-31 by wave 0
//   2. diagonal 16 x 16 inverses of I + A in place (wave 0); Aqk rows
//      32-63 (wave 1); Qg = scale e^G q (waves 2, 3)
//   3. the off-diagonal blocks of Tm = (I + A)^-1 by two merges (16 -> 32
//      in fp32 by all threads, 32 -> 64 by MFMA in wave 0)
//   4. Tm -> context, Tw = Tm diag(beta e^G) and Tu = Tm diag(beta) as
//      bf16 tiles; the fp32 area becomes the waves' store staging
//   5. W, W^T, U^T, Kd^T by MFMA / transposing reads, and the Aqk rows,
//      out as whole 16-byte rows
// ---------------------------------------------------------------------------
template <typename T, int DK, int DV, bool GATED>
__global__ __launch_bounds__(256, 2) void delta_prep_kernel(DeltaArgs a, DeltaLayout L) {
  constexpr int KT = DK / 64, VT = DV / 64;
  static_assert(DK % 64 == 0 && DV % 64 == 0 && DK <= 128 && DV <= 128, "64 or 128 wide");
  __shared__ __attribute__((aligned(16))) T Kt[KT][64 * 64];  // K rows (swizzled tiles)
  __shared__ __attribute__((aligned(16))) T Vt[VT][64 * 64];  // V rows
  __shared__ __attribute__((aligned(16))) float AT[64 * 64];  // A, then Tm in place; then staging
  __shared__ __attribute__((aligned(16))) T Tw[64 * 64];      // Tm diag(beta e^G)
  __shared__ __attribute__((aligned(16))) T Tu[64 * 64];      // Tm diag(beta)
  __shared__ __attribute__((aligned(16))) float Ys[16 * 48];  // scratch of the inverse merges
  __shared__ __attribute__((aligned(16))) float Bs[64];
  __shared__ __attribute__((aligned(16))) float Gs[64];

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
  const T* vb = (const T*)a.v + ((size_t)b * Tn * H + h) * DV;
  const int64_t qks = (int64_t)H * DK, vs = (int64_t)H * DV;

  // 0. copies, q rows, beta and G (wave 3)
#pragma unroll
  for (int o = 0; o < 2; ++o) {
#pragma unroll
    for (int i = 0; i < KT; ++i) dma_tile64<T>(kb + 64 * i, qks, t0, Tn, Kt[i], 2 * w + o, lane);
#pragma unroll
    for (int i = 0; i < VT; ++i) dma_tile64<T>(vb + 64 * i, vs, t0, Tn, Vt[i], 2 * w + o, lane);
  }
  v8_t<T> qop[DK / 16];  // q row 32 (w & 1) + cl: Aqk operand (waves 0, 1), Qg source (waves 2, 3)
  {
    const int ti = t0 + 32 * (w & 1) + cl;
#pragma unroll
    for (int kk = 0; kk < DK / 16; ++kk)
      qop[kk] = ti < Tn ? ld8<T>(qb + (int64_t)ti * qks + 16 * kk + 8 * hh) : zero8<T>();
  }
  if (w == 3) {
    const int t = t0 + lane;
    float bt = 0.f, gt = 0.f;
    if (t < Tn) {
      bt = a.beta[((size_t)b * Tn + t) * H + h];
      if constexpr (GATED) gt = a.g[((size_t)b * Tn + t) * H + h];
    }
    float x = gt;
    if constexpr (GATED) {
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(x, off);
        if (lane >= off) x += y;
      }
      reinterpret_cast<float*>(a.ctx + L.Gc)[(size_t)bh * Tp + t0 + lane] = x;
      reinterpret_cast<float*>(a.ctx + L.Fk)[(size_t)bh * Tp + t0 + lane] = __expf(__shfl(x, 63) - x);
    }
    Bs[lane] = bt;
    Gs[lane] = x;
  }
  vm_wait_barrier<0>();

  // Aqk block (rows i of block ib, columns j of block jb) as D[j][i]: lane
  // column i, scale (q_i . k_j) e^(G_i - G_j) for j <= i
  auto aqk_block = [&](int ib, int jb) __attribute__((always_inline)) {
    f32x16 acc{};
#pragma unroll
    for (int kk = 0; kk < DK / 16; ++kk)
      acc = mma(tile_ld8<T>(Kt[kk / 4], 32 * jb + cl, 16 * (kk % 4) + 8 * hh), qop[kk], acc);
    const int i = 32 * ib + cl;
    const float Giv = Gs[i];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int j = 32 * jb + 8 * (e >> 2) + 4 * hh + (e & 3);
      // branch-free: the exponent is zeroed where the entry is masked
      const bool m = j <= i;
      const float Gjv = reinterpret_cast<const f32x4*>(Gs + 32 * jb + 8 * (e >> 2) + 4 * hh)[0][e & 3];
      float val = a.scale * acc[e];
      if constexpr (GATED) val *= __expf(m ? Giv - Gjv : 0.f);
      acc[e] = m ? val : 0.f;
    }
    return acc;
  };
  f32x16 aq0{}, aq1{};

  // 1. Gram A[i][j] = beta_i (k_i . k_j) e^(G_i - G_j), i > j (zero above)
  if (w == 0) {
    aq0 = aqk_block(0, 0);
    // the all-zero upper block of A / Tm
#pragma unroll
    for (int e = 0; e < 16; ++e) AT[(8 * (e >> 2) + 4 * hh + (e & 3)) * 64 + 32 + cl] = 0.f;
  } else {
    const int ib = w >= 2, jb = w == 3;
    f32x16 acc{};
#pragma unroll
    for (int kk = 0; kk < DK / 16; ++kk)
      acc = mma(tile_ld8<T>(Kt[kk / 4], 32 * ib + cl, 16 * (kk % 4) + 8 * hh),
                tile_ld8<T>(Kt[kk / 4], 32 * jb + cl, 16 * (kk % 4) + 8 * hh), acc);
    const int j = 32 * jb + cl;
    const float Gjv = Gs[j];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int i = 32 * ib + 8 * (e >> 2) + 4 * hh + (e & 3);
      const bool m = i > j;
      const int i4 = 32 * ib + 8 * (e >> 2) + 4 * hh;
      const float Biv = reinterpret_cast<const f32x4*>(Bs + i4)[0][e & 3];
      const float Giv = reinterpret_cast<const f32x4*>(Gs + i4)[0][e & 3];
      float val = Biv * acc[e];
      if constexpr (GATED) val *= __expf(m ? Giv - Gjv : 0.f);
      AT[i * 64 + j] = m ? val : 0.f;
    }
  }
  __syncthreads();

  // 2. wave 0: D_R = (I + A_RR)^-1 for the four diagonal 16 x 16 blocks, one
  //    column per lane (lane = 16 R + column), by right-looking substitution
  //    (each finished x_k updates every later row: one FMA deep per step),
  //    written over A_RR
  if (w == 0) {
    const int R = lane >> 4, cc = lane & 15;
    float* blk = AT + 16 * R * 64 + 16 * R;
    float acc[16];
#pragma unroll
    for (int ii = 0; ii < 16; ++ii) acc[ii] = ii == cc ? 1.f : 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      // A_RR columns 4 g .. 4 g + 3 of the rows below, then four steps
      float ag[16][4];
#pragma unroll
      for (int ii = 0; ii < 16; ++ii) {
        if (ii > 4 * g) {
          const f32x4 a4 = *reinterpret_cast<const f32x4*>(blk + ii * 64 + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) ag[ii][r] = a4[r];
        }
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const float xk = acc[4 * g + kk];
#pragma unroll
        for (int ii = 0; ii < 16; ++ii)
          if (ii > 4 * g + kk) acc[ii] -= ag[ii][kk] * xk;
      }
    }
#pragma unroll
    for (int ii = 0; ii < 16; ++ii) blk[ii * 64 + cc] = acc[ii];
  } else if (w == 1) {
    aq0 = aqk_block(1, 0);
    aq1 = aqk_block(1, 1);
  } else {
    // Qg[i][d] = scale e^G_i q_i[d] (zero past T), rows 32 (w - 2) + cl
    const int i = 32 * (w - 2) + cl, ti = t0 + i;
    const float eg = GATED ? __expf(Gs[i]) : 1.f;
    const float sc = ti < Tn ? a.scale * eg : 0.f;
    T* qg = (T*)(a.ctx + L.Qg) + ((size_t)bh * Tp + t0 + i) * DK;
#pragma unroll
    for (int kk = 0; kk < DK / 16; ++kk) {
      v8_t<T> y;
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = (T)((float)qop[kk][e] * sc);
      if constexpr (GATED) *reinterpret_cast<v8_t<T>*>(qg + 16 * kk + 8 * hh) = y;
    }
  }
  __syncthreads();

  // 3. the off-diagonal blocks of Tm = (I + A)^-1: 16 -> 32 merges in fp32,
  //    32 -> 64 by MFMA on split bf16 operands (tri_inv.h)
  tri_inv64_merge(AT, Ys, tid);

  // 4. Tm (natural [i][j]) to the context; Tw, Tu tiles.  Thread: row
  //    tid >> 2, columns 16 (tid & 3) .. +15
  {
    const int r = tid >> 2, c0 = 16 * (tid & 3);
    T* tmg = (T*)(a.ctx + L.Tm) + ci * 4096 + r * 64 + c0;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      v8_t<T> tm, tw, tu;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int j = c0 + 8 * hf + e;
        const float t = AT[r * 64 + j];
        const float bj = Bs[j];
        tm[e] = (T)t;
        tu[e] = (T)(t * bj);
        tw[e] = (T)(t * bj * (GATED ? __expf(Gs[j]) : 1.f));
      }
      *reinterpret_cast<v8_t<T>*>(tmg + 8 * hf) = tm;
      *reinterpret_cast<v8_t<T>*>(reinterpret_cast<char*>(Tw) + tile_off(r, c0 + 8 * hf)) = tw;
      *reinterpret_cast<v8_t<T>*>(reinterpret_cast<char*>(Tu) + tile_off(r, c0 + 8 * hf)) = tu;
    }
  }
  __syncthreads();

  // 5. outputs through this wave's 4 KiB of the fp32 area
  u32x4* stage = reinterpret_cast<u32x4*>(AT) + 256 * w;
  // W[i][d] (natural): D[d][i] = sum_j K[j][d] Tw[i][j]; both state passes
  // read it, the reverse pass through transposing reads
  if (w >> 1 < KT) {
    const int ib = w & 1, kt = w >> 1;
    f32x16 x[2];
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      x[db] = f32x16{};
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          x[db] = mma(tile_tr8<T>(Kt[kt], 32 * s2, 32 * db, j, lane),
                      tile_ldp8<T>(Tw, 32 * ib + cl, 32 * s2, j, hh), x[db]);
    }
    store_rows_staged<T>(x[0], x[1], stage, (T*)(a.ctx + L.W) + ((size_t)bh * Tp + t0 + 32 * ib) * DK + 64 * kt,
                         DK, lane);
  }
  // U^T[v][i] (rows i in operand order): D[i][v] = sum_j Tu[i][j] V[j][v]
  auto trans_out = [&](const T* tile, const T* Tx, T* dst) __attribute__((always_inline)) {
    f32x16 x[2];
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      x[ib] = f32x16{};
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          x[ib] = mma(tile_ldp8<T>(Tx, 32 * ib + cl, 32 * s2, j, hh),
                      tile_tr8<T>(tile, 32 * s2, 32 * (w & 1), j, lane), x[ib]);
    }
    store_rows_staged<T, true>(x[0], x[1], stage, dst, 64, lane);
  };
  if (w < DV / 32) trans_out(Vt[w >> 1], Tu, (T*)(a.ctx + L.UT) + (ci * DV + 32 * w) * 64);
  // Kd^T[d][i] = e^(gamma - G_i) k_i[d] (zero past T), rows i in operand
  // order; gated only (ungated, the forward state pass reads k itself)
  if (GATED && w < DK / 32) {
    f32x16 x[2];
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const v8_t<T> k8 = tile_tr8<T>(Kt[w >> 1], 32 * ib, 32 * (w & 1), j, lane);
#pragma unroll
        for (int p = 0; p < 8; ++p) {
          const int e = 8 * j + p;  // C-layout slot: row 8 (e >> 2) + 4 hh + (e & 3)
          const int i = 32 * ib + 8 * (e >> 2) + 4 * hh + (e & 3);
          const float eg = GATED ? __expf(Gs[63] - Gs[i]) : 1.f;
          const float sc = t0 + i < Tn ? eg : 0.f;
          x[ib][e] = (float)k8[p] * sc;
        }
      }
    store_rows_staged<T, true>(x[0], x[1], stage, (T*)(a.ctx + L.KdT) + (ci * DK + 32 * w) * 64, 64, lane);
  }
  // Aqk rows (natural [i][j]): wave 0 rows 0-31 (upper block zero), wave 1 rows 32-63
  if (w < 2)
    store_rows_staged<T>(aq0, aq1, stage, (T*)(a.ctx + L.Aqk) + ci * 4096 + 32 * w * 64, 64, lane);
}

// ---------------------------------------------------------------------------
// Kernel 2: sequential state pass and output.  The value columns of a head
// are split over DV/32 workgroups; each holds its 32 columns of S[d][v] in
// DK/32 accumulator tiles (lane column v) on one compute wave.  Per chunk
// the chain is
//   v_new = U - W S  ->  S <- e^gamma S + Kd^T v_new.
// Two copy waves issue W, Kd^T (ungated: the chunk's k rows, read
// transposed) and this workgroup's U^T rows two chunks ahead into a ring of
// three slots, and store the v_new^T / h^T blocks the compute wave staged
// one chunk earlier (and the output wave's o blocks).  W, Kd^T and U^T rows are stored XOR-swizzled by
// 16-byte chunk so the operand reads of 16 consecutive rows hit distinct
// banks.  The output wave forms the workgroup's 32 columns of
//   o = scale e^G (Q h) + Aqk v_new
// for each chunk from the same staged h^T and v_new^T blocks while the
// compute wave runs the next chunk, with q and Aqk rows loaded one chunk
// ahead into registers, so no output pass reads h and v_new back.  It
// stages o for the copy waves, which store it two barriers later.  Every
// store of the pass is non-temporal: the written lines then leave L2 first
// and do not evict the W / k tiles the head's workgroups share there.
// ---------------------------------------------------------------------------

template <typename T, int DK, int DV, bool GATED>
__global__ __launch_bounds__(state_threads<DV>()) void delta_state_fwd_kernel(
    DeltaArgs a, DeltaLayout L, const float* __restrict__ gcum) {
  constexpr int SPLIT = state_split<DV>();
  constexpr int NDT = DK / 32, NW = DV / 32 / SPLIT;      // compute waves of this workgroup (+ one copy wave)
  constexpr int WT16 = 64 * DK * (int)sizeof(T) / 16;   // 16-byte chunks per W (= Kd^T) tile
  constexpr int UT16 = 32 * 64 * (int)sizeof(T) / 16;   // per wave's U^T rows
  constexpr int WCPR = DK * (int)sizeof(T) / 16;         // chunks per W row
  constexpr int KCPR = 64 * (int)sizeof(T) / 16;         // chunks per Kd^T / U^T row
  constexpr int SLOT = 2 * WT16 + NW * UT16;             // W | Kd^T | U^T per chunk
  constexpr int WOPS = WT16 / 64, UOPS = NW * UT16 / 64;  // 1 KiB copies per chunk
  constexpr int NCW = kStateCopyWaves;                     // copy waves, each a 1 / NCW share
  constexpr int WOPC = WOPS / NCW, UOPC = UOPS / NCW;
  constexpr int DMA_PER_CHUNK = (2 * WOPS + UOPS) / NCW;   // per copy wave
  static_assert(WOPS * 64 == WT16 && UOPS * 64 == NW * UT16 && WOPC * NCW == WOPS && UOPC * NCW == UOPS &&
                    8 % NCW == 0 && DMA_PER_CHUNK <= 63,
                "tile split");
  __shared__ __attribute__((aligned(16))) u32x4 Sh[3 * SLOT];
  // per chunk (two buffers): the compute waves' v_new^T block and h^T blocks
  // (NDT / 2 each), staged for the copy wave's stores
  constexpr int NSTG = NW * (NDT / 2 + 1);
  __shared__ __attribute__((aligned(16))) u32x4 Stg[2][NSTG][256];
  // the output wave's chunk c rows of o (two 32 x 32 blocks), staged in
  // Ostg[c & 1] for the copy waves, which store them two barriers later
  __shared__ __attribute__((aligned(16))) u32x4 Ostg[2][2][128];
  static_assert(NW == 1, "one compute wave per workgroup (the output wave reads its staged blocks)");

  const int lane = threadIdx.x & 63, w = wave_id();
  const int cl = lane & 31, hh = lane >> 5;
  const int NT = a.NT;
  const int BH = a.B * a.H;
  const int bh = blockIdx.x % BH;
  const int gw = (blockIdx.x / BH) * NW + w;  // this wave's 32-column block of the head
  const int v = 32 * gw + cl;
  const size_t Tp = (size_t)NT * kChunk;

  // gcum = the Gc context buffer, passed on its own as __restrict__ so the
  // per-chunk gate is a scalar load (no vector-memory wait in the chain)
  const float* Gc = gcum + (size_t)bh * Tp;
  if (w == NW + kStateCopyWaves) {
    // The output wave: chunk c's rows of o in this workgroup's 32 value
    // columns, once the barrier that opens chunk c + 1 has closed chunk c
    // (its h^T and v_new^T blocks are staged in Stg[c & 1] until the compute
    // wave stages chunk c + 2 there, after the next barrier).  As MFMA
    // products with the value columns as rows: D[v][i] = sum_d h^T[v][d]
    // q[i][d] (A operand from the staged h^T rows, B from q row i in
    // registers), scaled per query row i, plus sum_j v_new^T[v][j] Aqk[i][j].
    const int b = bh / a.H, h = bh % a.H, Tn = a.T, H = a.H;
    const T* qh = (const T*)a.q + ((size_t)b * Tn * H + h) * DK;
    const T* ah = (const T*)(a.ctx + L.Aqk) + (size_t)bh * NT * 4096;
    v8_t<T> yq[2][DK / 16], ya[2][4];
    float f[2];
    // chunk c's q rows, Aqk rows and row factors scale e^G of this lane's
    // query rows 32 ib + cl (rows past T: zero q; their o is not stored),
    // issued once chunk c - 1's products have read the registers, a chunk
    // ahead of their use
    auto load = [&](int c) __attribute__((always_inline)) {
      const int t0 = c * kChunk;
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) {
        const int i = 32 * ib + cl;
        const bool valid = t0 + i < Tn;
        const T* qr = qh + (size_t)(t0 + i) * H * DK;
#pragma unroll
        for (int s = 0; s < DK / 16; ++s) yq[ib][s] = valid ? ld8<T>(qr + 16 * s + 8 * hh) : zero8<T>();
#pragma unroll
        for (int s = 0; s < 4; ++s) ya[ib][s] = ld8<T>(ah + (size_t)c * 4096 + i * 64 + 16 * s + 8 * hh);
        f[ib] = a.scale;
        if constexpr (GATED) f[ib] *= __expf(Gc[t0 + i]);
      }
    };
    load(0);
    block_barrier();  // opens chunk 0
#pragma unroll 1
    for (int c = 0; c < NT; ++c) {
      block_barrier();  // chunk c staged (the compute wave's barrier opening chunk c + 1, or its last)
      const u32x4* vs = &Stg[c & 1][0][0];  // v_new^T [v][j]
      const u32x4* hs = vs + 256;          // h^T [v][d], NDT / 2 blocks of 64 columns
      // every staged operand read first, so the products run back to back
      u32x4 hop[DK / 16], vop[4];
#pragma unroll
      for (int s = 0; s < DK / 16; ++s) hop[s] = hs[(s / 4) * 256 + swz_slot<8>(cl, 2 * (s % 4) + hh)];
#pragma unroll
      for (int s = 0; s < 4; ++s) vop[s] = vs[swz_slot<8>(cl, 2 * s + hh)];
      __builtin_amdgcn_sched_barrier(0);
      f32x16 x[2];
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) x[ib] = f32x16{};
#pragma unroll
      for (int s = 0; s < DK / 16; ++s)
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) x[ib] = mma(__builtin_bit_cast(v8_t<T>, hop[s]), yq[ib][s], x[ib]);
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) x[ib] *= f[ib];
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) x[ib] = mma(__builtin_bit_cast(v8_t<T>, vop[s]), ya[ib][s], x[ib]);
      if (c + 1 < NT) load(c + 1);
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) stage_rows32<T>(x[ib], Ostg[c & 1][ib], lane);
    }
    block_barrier();  // the last chunk's o staged for the copy waves
    return;
  }
  // The copy waves (w >= NW) issue every copy, two chunks ahead, into a ring
  // of three slots; the compute waves never stall on copy issue.  Copy wave
  // cw issues share cw of each tile's copies.
  if (w >= NW) {  // (the output wave has returned above)
    const int cw = w - NW;
    // wave-uniform byte bases of this head's W, Kd^T and this workgroup's
    // U^T rows; chunk c sits at + c * (bytes per chunk).  A 1 KiB copy op
    // covers tile chunks [64 op, 64 op + 64); slot lane of row r holds
    // global chunk swz(r, lane).
    const char* Wg = a.ctx + L.W + (size_t)bh * NT * WT16 * 16;
    const char* Kg = a.ctx + L.KdT + (size_t)bh * NT * WT16 * 16;
    const int b = bh / a.H, h = bh % a.H, Tn = a.T;
    const T* kb = (const T*)a.k + ((size_t)b * Tn * a.H + h) * DK;
    const int kbytes = a.H * DK * (int)sizeof(T);  // k row stride
    const char* Ug = a.ctx + L.UT + ((size_t)bh * NT * NW * SPLIT + (gw - w)) * UT16 * 16;
    auto issue = [&](int c) __attribute__((always_inline)) {
      u32x4* sl = Sh + (c % 3) * SLOT;
#pragma unroll
      for (int op = WOPC * cw; op < WOPC * cw + WOPC; ++op)
        dma16s(Wg + (size_t)c * WT16 * 16, 16u * swz_slot<WCPR>((64 * op + lane) / WCPR, lane % WCPR), sl + 64 * op);
      if constexpr (GATED) {
#pragma unroll
        for (int op = WOPC * cw; op < WOPC * cw + WOPC; ++op)
          dma16s(Kg + (size_t)c * WT16 * 16, 16u * swz_slot<KCPR>((64 * op + lane) / KCPR, lane % KCPR),
                 sl + WT16 + 64 * op);
      } else {
        // the chunk's k rows as DK/64 natural 64 x 64 tiles (rows past T
        // repeat the last one; v_new is zero there)
        T* kt = reinterpret_cast<T*>(sl + WT16);
        const int t0 = c * kChunk;
        if (t0 + kChunk <= Tn) {
#pragma unroll
          for (int op = 8 / NCW * cw; op < 8 / NCW * (cw + 1); ++op)
#pragma unroll
            for (int i = 0; i < DK / 64; ++i)
              dma16s(kb + (size_t)t0 * a.H * DK + 64 * i, tile_lane_off(op, lane, kbytes),
                     reinterpret_cast<char*>(kt + i * 4096) + 1024 * op);
        } else {
#pragma unroll
          for (int op = 8 / NCW * cw; op < 8 / NCW * (cw + 1); ++op)
#pragma unroll
            for (int i = 0; i < DK / 64; ++i)
              dma_tile64<T>(kb + 64 * i, (int64_t)a.H * DK, t0, Tn, kt + i * 4096, op, lane);
        }
      }
#pragma unroll
      for (int op = UOPC * cw; op < UOPC * cw + UOPC; ++op)
        dma16s(Ug + (size_t)c * NW * SPLIT * UT16 * 16, 16u * swz_slot<KCPR>((64 * op + lane) / KCPR, lane % KCPR),
               sl + 2 * WT16 + 64 * op);
    };
    // o rows of chunk c in the compute wave's columns: copy wave cw stores
    // block cw (rows 32 cw ..) of Ostg[c & 1]
    T* oh = (T*)a.o + ((size_t)b * Tn * a.H + h) * DV + 32 * (gw - w);
    auto flush_o = [&](int c) __attribute__((always_inline)) {
      const int r0 = c * kChunk + 32 * cw;
      flush_rows32<T, kStoreStream>(Ostg[c & 1][cw], oh + (size_t)r0 * a.H * DV, (int64_t)a.H * DV, lane, Tn - r0);
    };
    static_assert(NCW == 2, "one o block per copy wave");
    // staged outputs of chunk c: v_new^T and h^T rows (ci DV + 32 g2); copy
    // wave cw stores the blocks with index cw modulo the copy waves
    auto flush = [&](int c) __attribute__((always_inline)) {
      const size_t ci = (size_t)bh * NT + c;
#pragma unroll
      for (int q = 0; q < NW; ++q) {
        const int g2 = gw - w + q;
        if ((q * (NDT / 2 + 1)) % NCW == cw)
          flush_rows<T, kStoreStream>(Stg[c & 1][q * (NDT / 2 + 1)], (T*)(a.ctx + L.VnT) + (ci * DV + 32 * g2) * 64, 64, lane);
#pragma unroll
        for (int blk = 0; blk < NDT / 2; ++blk)
          if ((q * (NDT / 2 + 1) + 1 + blk) % NCW == cw)
            flush_rows<T, kStoreStream>(Stg[c & 1][q * (NDT / 2 + 1) + 1 + blk],
                          (T*)(a.ctx + L.hT) + (ci * DV + 32 * g2) * DK + 64 * blk, DK, lane);
      }
    };
    issue(0);
    if (NT > 1) issue(1);
#pragma unroll 1
    for (int c = 0; c < NT; ++c) {
      // chunk c landed (only chunk c + 1's copies may remain in flight;
      // stores only add to the count) before the barrier that opens it;
      // the barrier also closes chunk c - 1, whose staged outputs this wave
      // stores and whose slot then takes chunk c + 2
      if (c + 1 < NT) vm_wait_barrier<DMA_PER_CHUNK>();
      else vm_wait_barrier<0>();
      if (c > 0) flush(c - 1);
      if (c > 1) flush_o(c - 2);
      if (c + 2 < NT) issue(c + 2);
    }
    block_barrier();  // the last chunk staged
    flush(NT - 1);
    if (NT > 1) flush_o(NT - 2);
    block_barrier();  // the last chunk's o staged
    flush_o(NT - 1);
    return;
  }


  f32x16 S[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int d = 32 * dt + 8 * (e >> 2) + 4 * hh + (e & 3);
      S[dt][e] = a.h0 ? a.h0[((size_t)bh * DK + d) * DV + v] : 0.f;
    }

  // one chunk in ring slot SL; the loop below is unrolled by the ring depth
  // so every LDS address is a chunk-invariant register plus a constant
  // gated: G at the last row of chunks 64 m + lane, reloaded every 64 chunks
  float gl = 0.f;
  auto load_gl = [&](int c0) __attribute__((always_inline)) {
    if constexpr (GATED) gl = c0 + lane < NT ? Gc[(size_t)(c0 + lane) * kChunk + 63] : 0.f;
  };
  auto step = [&](auto SL, int c) __attribute__((always_inline)) {
    constexpr int sl = decltype(SL)::value;
    if (GATED && c > 0 && (c & 63) == 0) load_gl(c);
    // chunk c landed (the copy wave waited for it); every wave is done
    // with chunk c - 1, whose slot the copy wave refills
    block_barrier();
    const u32x4* Ws = Sh + sl * SLOT;
    const u32x4* Ks = Ws + WT16;
    const u32x4* Us = Ws + 2 * WT16 + w * UT16;

    // the chunk's LDS operands into registers ahead of their MFMA chains (W
    // first, U^T and Kd^T behind the W S products): the one wave per SIMD
    // then never waits on a read inside a chain
    u32x4 wv[2][NDT][2], kv[GATED ? NDT : 1][2][2], uv[2][2];
    v8_t<T> kt8[GATED ? 1 : NDT][2][2];
#pragma unroll
    for (int db = 0; db < NDT; ++db)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int it = 0; it < 2; ++it) {
          // k-step (db, j) of row 32 it + cl in ld_tr_op order: the 8-byte
          // halves hh of its two 16-byte chunks 4 db + 2 j and 4 db + 2 j + 1
          const char* row = reinterpret_cast<const char*>(Ws);
          const v4_t<T> lo = *reinterpret_cast<const v4_t<T>*>(
              row + 16 * swz_slot<WCPR>(32 * it + cl, 4 * db + 2 * j) + 8 * hh);
          const v4_t<T> hi = *reinterpret_cast<const v4_t<T>*>(
              row + 16 * swz_slot<WCPR>(32 * it + cl, 4 * db + 2 * j + 1) + 8 * hh);
          wv[it][db][j] = __builtin_bit_cast(u32x4, cat44<T>(lo, hi));
        }
    __builtin_amdgcn_sched_barrier(0);

    // P = W S  (W rows 32 it + cl)
    f32x16 P[2];
    P[0] = P[1] = f32x16{};
#pragma unroll
    for (int db = 0; db < NDT; ++db)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const v8_t<T> ys = c_to_b<T>(S[db], j);
#pragma unroll
        for (int it = 0; it < 2; ++it) P[it] = mma(__builtin_bit_cast(v8_t<T>, wv[it][db][j]), ys, P[it]);
      }
    // the state entering the chunk (h^T, [v][d]) is staged here, before the
    // decay, and stored by the copy wave during the next chunk
#pragma unroll
    for (int blk = 0; blk < NDT / 2; ++blk)
      stage_rows<T>(S[2 * blk], S[2 * blk + 1], Stg[c & 1][w * (NDT / 2 + 1) + 1 + blk], lane);
    // gated: S's decay for the update, applied while the products above run
    // (they read S through the bf16 operands already formed); e^gamma of
    // chunk c from lane c % 64 of gl
    if constexpr (GATED) {
      const float eg = __expf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gl), c & 63)));
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) S[dt] *= eg;
    }
    // U^T and the Kd^T operands of the state update, read while the MFMAs
    // above run
#pragma unroll
    for (int it = 0; it < 2; ++it)
#pragma unroll
      for (int jq = 0; jq < 2; ++jq) uv[it][jq] = Us[swz_slot<KCPR>(cl, 4 * it + 2 * jq + hh)];
    if constexpr (!GATED) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int it = 0; it < 2; ++it)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj)  // k^T by transposing reads of the natural k tiles
            kt8[dt][it][jj] = tile_tr8<T>(reinterpret_cast<const T*>(Ks) + (dt / 2) * 4096, 32 * it, 32 * (dt & 1), jj, lane);
    }
    __builtin_amdgcn_sched_barrier(0);

    // v_new = U - P (rows past T are zero in U and W); U^T rows of this
    // wave, chunk rows in operand order
    f32x16 Vn[2];
#pragma unroll
    for (int it = 0; it < 2; ++it)
#pragma unroll
      for (int jq = 0; jq < 2; ++jq) {
        const v8_t<T> u8 = __builtin_bit_cast(v8_t<T>, uv[it][jq]);
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const int I = 2 * jq + s2;
#pragma unroll
          for (int r = 0; r < 4; ++r) Vn[it][4 * I + r] = (float)u8[4 * s2 + r] - P[it][4 * I + r];
        }
      }
    // gated: the Kd^T operands only now, once the W operands are dead (read
    // with the W operands, they pushed the wave past 256 VGPRs and 28 values
    // per chunk went through AGPRs)
    if constexpr (GATED) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int it = 0; it < 2; ++it)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) kv[dt][it][jj] = Ks[swz_slot<KCPR>(32 * dt + cl, 4 * it + 2 * jj + hh)];
    }
    // v_new^T: staged here, stored by the copy wave during the next chunk
    stage_rows<T>(Vn[0], Vn[1], Stg[c & 1][w * (NDT / 2 + 1)], lane);

    // S <- e^gamma S + Kd^T v_new  (Kd^T rows 32 dt + cl)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int it = 0; it < 2; ++it)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          S[dt] = mma(GATED ? __builtin_bit_cast(v8_t<T>, kv[GATED ? dt : 0][it][jj]) : kt8[GATED ? 0 : dt][it][jj],
                      c_to_b<T>(Vn[it], jj), S[dt]);
    }
  };

  load_gl(0);
  vm_drain();  // h0 (and gl) are in registers
#pragma unroll 1
  for (int c = 0; c < NT; c += 3) {
    step(IntC<0>{}, c);
    if (c + 1 < NT) step(IntC<1>{}, c + 1);
    if (c + 2 < NT) step(IntC<2>{}, c + 2);
  }
  block_barrier();  // the last chunk's staged outputs are complete for the copy wave
  block_barrier();  // the output wave's last o is staged (a barrier every wave takes)

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

template <typename T, int DK, int DV, bool GATED>
hipError_t launch_delta_fwd(const DeltaArgs& a, hipStream_t stream) {
  const DeltaLayout L = delta_layout(a.B, a.T, a.H, DK, DV, sizeof(T));
  const int BH = a.B * a.H;
  hipError_t e = hipSuccess;
  if (a.stages & 1) {
    delta_prep_kernel<T, DK, DV, GATED><<<dim3(BH * a.NT), dim3(256), 0, stream>>>(a, L);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (a.stages & 2) {
    delta_state_fwd_kernel<T, DK, DV, GATED><<<dim3(BH * state_split<DV>()), dim3(state_threads<DV>()), 0,
                                               stream>>>(
        a, L, reinterpret_cast<const float*>(a.ctx + L.Gc));
    e = hipGetLastError();
  }
  return e;
}

#define LINATT_DELTA_FWD_INST(T, DK, DV)                                              \
  template hipError_t launch_delta_fwd<T, DK, DV, false>(const DeltaArgs&, hipStream_t); \
  template hipError_t launch_delta_fwd<T, DK, DV, true>(const DeltaArgs&, hipStream_t);

LINATT_DELTA_SHAPES(LINATT_DELTA_FWD_INST)

}  // namespace linatt
