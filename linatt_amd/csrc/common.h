// Shared device helpers for the linatt HIP kernels (gfx950 / CDNA4, wave64).
//
// Matrix-core conventions used by every kernel in this library
// (v_mfma_f32_32x32x16_{bf16,f16}; fp32 operands use eight
// v_mfma_f32_32x32x2f32 steps that consume the same per-lane k-slots):
//
//   lane l, half h = l >> 5, column c = l & 31
//   A operand (32 x 16, row-major m x k): lane holds A[c][8h + j], j = 0..7
//   B operand (16 x 32, k x n):           lane holds B[8h + j][c]
//   C/D (32 x 32 fp32, 16 per lane):      acc[4i + r] = D[8i + 4h + r][c]
//
// A reduction (k) index may be permuted freely as long as A and B use the
// same permutation.  The kernels use this to feed a C-layout result
// straight back as a B operand: for a 32-row C block, k-step j (0 or 1)
// takes acc elements i in {2j, 2j+1}, so slot p of lane half h maps to row
//   8 * (2j + (p >> 2)) + 4h + (p & 3)      (see c_to_b below),
// and the matching A operand reads two runs of four consecutive rows
// (16j + 4h .. +3 and 16j + 8 + 4h .. +3) from a transposed LDS tile.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace linatt {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T> struct vt;
template <> struct vt<__bf16> { using v8 = bf16x8; using v4 = bf16x4; };
template <> struct vt<_Float16> { using v8 = f16x8; using v4 = f16x4; };
template <> struct vt<float> { using v8 = f32x8; using v4 = f32x4; };
template <typename T> using v8_t = typename vt<T>::v8;
template <typename T> using v4_t = typename vt<T>::v4;

__device__ __forceinline__ f32x16 mma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mma(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mma(f32x8 a, f32x8 b, f32x16 c) {
#pragma unroll
  for (int j = 0; j < 8; ++j) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j], b[j], c, 0, 0, 0);
  return c;
}

// 8 contiguous elements (16 B for 16-bit types, 32 B for fp32); p must be
// 16-byte aligned.
template <typename T>
__device__ __forceinline__ v8_t<T> ld8(const T* p) {
  if constexpr (sizeof(T) == 2) {
    return __builtin_bit_cast(v8_t<T>, *reinterpret_cast<const uint4*>(p));
  } else {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    return f32x8{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  }
}

// 4 contiguous elements (8 B for 16-bit types, 16 B for fp32).
template <typename T>
__device__ __forceinline__ v4_t<T> ld4(const T* p) {
  if constexpr (sizeof(T) == 2) {
    return __builtin_bit_cast(v4_t<T>, *reinterpret_cast<const uint2*>(p));
  } else {
    return __builtin_bit_cast(f32x4, *reinterpret_cast<const float4*>(p));
  }
}

template <typename T>
__device__ __forceinline__ void st4(T* p, v4_t<T> v) {
  if constexpr (sizeof(T) == 2) {
    *reinterpret_cast<uint2*>(p) = __builtin_bit_cast(uint2, v);
  } else {
    *reinterpret_cast<float4*>(p) = __builtin_bit_cast(float4, v);
  }
}

template <typename T>
__device__ __forceinline__ v8_t<T> cat44(v4_t<T> a, v4_t<T> b) {
  return v8_t<T>{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Two runs of four consecutive elements: rows 16j + 4h .. +3 and +8.
template <typename T>
__device__ __forceinline__ v8_t<T> ld_tr_op(const T* row, int j, int h) {
  return cat44<T>(ld4<T>(row + 16 * j + 4 * h), ld4<T>(row + 16 * j + 8 + 4 * h));
}

// Index of the calling wave in its workgroup, read from the first lane so the
// compiler treats it (and what derives from it) as wave-uniform: branches on
// it become scalar branches instead of exec-masked regions.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// Direct global -> LDS copy (global_load_lds_dwordx4): lane l's 16 bytes at
// p land at lds_base + 16 l; lds_base must be the same for the whole wave.
// The copy counts as an outstanding vector-memory load of the issuing wave
// until it lands, and readers wait for it with vm_wait_barrier.  It is
// issued from inline assembly so that the compiler, which would otherwise
// stall every later LDS read until all copies in flight have landed (it
// cannot tell the slots apart), leaves the scheduling of the waits to that
// explicit barrier; the compiler's own vmcnt waits stay correct because
// vector-memory loads of a wave complete in issue order.
__device__ __forceinline__ void dma16(const void* p, void* lds_base) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(
      (unsigned)(uintptr_t)(__attribute__((address_space(3))) void*)lds_base);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(p), "s"(m0)
               : "memory", "m0");
}

// The same copy addressed as a wave-uniform 64-bit base (SGPRs) plus a
// per-lane 32-bit byte offset: a loop that walks a tensor then only moves
// the scalar base, with no per-lane 64-bit address arithmetic.
__device__ __forceinline__ void dma16s(const void* sbase, unsigned voff, void* lds_base) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(
      (unsigned)(uintptr_t)(__attribute__((address_space(3))) void*)lds_base);
  // the base is wave-uniform by contract; readfirstlane lets the compiler
  // keep it in SGPRs where it cannot prove that itself
  const uint64_t a = (uint64_t)(uintptr_t)sbase;
  const uint64_t u = ((uint64_t)__builtin_amdgcn_readfirstlane((unsigned)(a >> 32)) << 32) |
                     (unsigned)__builtin_amdgcn_readfirstlane((unsigned)a);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(u), "s"(m0)
               : "memory", "m0");
}

// Raw buffer resource over [p, p + bytes): stores past the end are dropped.
// Bulk output goes through buffer stores: on gfx950 a wave's 16-byte-per-lane
// buffer_store moves about five times the bytes per CU cycle of the same
// global_store (measured: ~39 vs ~7.5 B/cycle/CU).  p must be wave-uniform.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, unsigned bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  const uint64_t u = ((uint64_t)__builtin_amdgcn_readfirstlane((unsigned)(a >> 32)) << 32) |
                     (unsigned)__builtin_amdgcn_readfirstlane((unsigned)a);
  return __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)u, (short)0, (int)bytes, 0x00020000);
}

// 4-byte variant: lane l's float at p lands at lds_base + 4 l.
__device__ __forceinline__ void dma4(const void* p, void* lds_base) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(
      (unsigned)(uintptr_t)(__attribute__((address_space(3))) void*)lds_base);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :
               : "v"(p), "s"(m0)
               : "memory", "m0");
}

// s_waitcnt vmcnt(0) that the compiler's wait tracking sees: every earlier
// global load of the wave has landed.  Used once before a loop that keeps
// copies in flight, so no load issued before it is waited for inside the loop
// (a compiler-inserted vmcnt(0) there would also wait for the copies).
__device__ __forceinline__ void vm_drain() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Copy of n4 x 16 bytes (n4 <= 64) from src to lds_base by the calling wave.
__device__ __forceinline__ void dma_small(const void* src, void* lds_base, int n4, int lane) {
  if (lane < n4) dma16(reinterpret_cast<const char*>(src) + 16 * lane, lds_base);
}

// s_barrier as a compiler-opaque step (memory clobber).  The wave's LDS
// operations drain first (lgkmcnt(0)): s_barrier itself does not wait for
// them, and LDS accesses of different waves are not ordered, so an LDS write
// still queued at the barrier could be read stale by another wave after it.
__device__ __forceinline__ void block_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// s_waitcnt vmcnt(N) lgkmcnt(0) then s_barrier, as one compiler-opaque step
// (memory clobber: no memory access moves across it).  Vector-memory loads
// of a wave complete in issue order, so with N = the number of loads issued
// after some load X, X has landed once vmcnt <= N, whatever stores are also
// in flight (they only add to the count); LDS operations drain as in
// block_barrier.
template <int N>
__device__ __forceinline__ void vm_wait_barrier() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"i"(N) : "memory");
}

// vm_wait_barrier for a wave-uniform count n in [0, 12] (the counter field is
// an immediate); larger n waits for everything.
__device__ __forceinline__ void vm_wait_barrier_n(int n) {
  switch (n) {
    case 12: vm_wait_barrier<12>(); break;
    case 11: vm_wait_barrier<11>(); break;
    case 10: vm_wait_barrier<10>(); break;
    case 9: vm_wait_barrier<9>(); break;
    case 8: vm_wait_barrier<8>(); break;
    case 7: vm_wait_barrier<7>(); break;
    case 6: vm_wait_barrier<6>(); break;
    case 5: vm_wait_barrier<5>(); break;
    case 4: vm_wait_barrier<4>(); break;
    case 3: vm_wait_barrier<3>(); break;
    case 2: vm_wait_barrier<2>(); break;
    case 1: vm_wait_barrier<1>(); break;
    default: vm_wait_barrier<0>(); break;
  }
}

// s_waitcnt vmcnt(n) alone, for a wave-uniform n in [0, 15] (larger n waits
// for everything); the same in-order argument as vm_wait_barrier.
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N) : "memory");
}
__device__ __forceinline__ void vm_wait_n(int n) {
  switch (n) {
    case 15: vm_wait<15>(); break;
    case 14: vm_wait<14>(); break;
    case 13: vm_wait<13>(); break;
    case 12: vm_wait<12>(); break;
    case 11: vm_wait<11>(); break;
    case 10: vm_wait<10>(); break;
    case 9: vm_wait<9>(); break;
    case 8: vm_wait<8>(); break;
    case 7: vm_wait<7>(); break;
    case 6: vm_wait<6>(); break;
    case 5: vm_wait<5>(); break;
    case 4: vm_wait<4>(); break;
    case 3: vm_wait<3>(); break;
    case 2: vm_wait<2>(); break;
    case 1: vm_wait<1>(); break;
    default: vm_wait<0>(); break;
  }
}

// ---------------------------------------------------------------------------
// 64 x 64 tiles of 16-bit elements in LDS: 128-byte rows, unpadded, with the
// 16-byte chunk c of row r stored in slot c ^ f(r),
//   f(r) = ((r >> 1) & 1) << 2 | ((r >> 2) & 3),
// which keeps both access patterns free of bank conflicts: 16-byte operand
// reads of 16 consecutive rows at one chunk, and the transposing 8-byte
// reads (4 rows x 4 chunks per 32 lanes) of ld_tr8.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int tile_slot(int row, int ch) {
  return ch ^ ((((row >> 1) & 1) << 2) | ((row >> 2) & 3));
}
__device__ __forceinline__ int tile_off(int row, int col) {  // byte offset, col % 4 == 0
  return row * 128 + (tile_slot(row, col >> 3) << 4) + ((col & 7) << 1);
}

// Wave-level copy of tile rows [8 op, 8 op + 8) from global rows row0 + r
// (clamped to nrows - 1: rows past the end repeat the last valid row, which
// every consumer masks) into the swizzled LDS tile.
template <typename T>
__device__ __forceinline__ void dma_tile64(const T* g, int64_t rs, int row0, int nrows, T* tile,
                                           int op, int lane) {
  const int row = 8 * op + (lane >> 3), slot = lane & 7;
  const int grow = min(row0 + row, nrows - 1);
  dma16(g + (int64_t)grow * rs + 8 * tile_slot(row, slot), reinterpret_cast<char*>(tile) + 1024 * op);
}

// Byte offset (from the tile's first global row) of the 16 bytes that lane
// copies in op `op` of dma_tile64 for global rows rs_bytes apart: with a
// wave-uniform base per tile, dma16s(base, tile_lane_off(..), tile + 1 KiB op)
// makes the same copy without per-lane 64-bit address arithmetic (rows are
// not clamped: full tiles only).
__device__ __forceinline__ unsigned tile_lane_off(int op, int lane, int rs_bytes) {
  const int row = 8 * op + (lane >> 3);
  return (unsigned)(row * rs_bytes + 16 * tile_slot(row, lane & 7));
}

// 8 consecutive elements of row `row` from column col (col % 8 == 0).
template <typename T>
__device__ __forceinline__ v8_t<T> tile_ld8(const T* tile, int row, int col) {
  return *reinterpret_cast<const v8_t<T>*>(reinterpret_cast<const char*>(tile) + tile_off(row, col));
}

// A tile of 64 rows and KT * 64 columns kept as KT natural 64 x 64
// sub-tiles (columns 64 j .. 64 j + 63 in sub-tile j, 4096 elements apart,
// each swizzled as tile_slot says).  An operand's 8 or 32 columns never
// straddle two sub-tiles.
template <typename T>
__device__ __forceinline__ v8_t<T> wtile_ld8(const T* tile, int row, int col) {
  return *reinterpret_cast<const v8_t<T>*>(reinterpret_cast<const char*>(tile + (col >> 6) * 4096) +
                                          tile_off(row, col & 63));
}

// Eight elements of row `row` in the k order of ld_tr_op: columns
// c0 + 16 j + 4 hh + 0..3 and c0 + 16 j + 8 + 4 hh + 0..3 (two 8-byte reads).
template <typename T>
__device__ __forceinline__ v8_t<T> tile_ldp8(const T* tile, int row, int c0, int j, int hh) {
  const char* base = reinterpret_cast<const char*>(tile);
  return cat44<T>(*reinterpret_cast<const v4_t<T>*>(base + tile_off(row, c0 + 16 * j + 4 * hh)),
                  *reinterpret_cast<const v4_t<T>*>(base + tile_off(row, c0 + 16 * j + 8 + 4 * hh)));
}

// Transposing 8-byte LDS read (ds_read_tr16_b64): within each 16-lane group,
// lane i receives element i % 4 of the 4 values read by lanes 4c + i / 4,
// c = 0..3.
template <typename T>
__device__ __forceinline__ v4_t<T> ds_tr4(const T* p) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(v4_t<T>, x);
}

// MFMA operand with k running down the rows of a natural tile: lane
// (column c0 + (lane & 31)) receives rows r0 + 16 j + 4 hh + 0..3 and
// r0 + 16 j + 8 + 4 hh + 0..3, the same k order as ld_tr_op on the
// transposed tile.  r0 is a multiple of 16.
template <typename T>
__device__ __forceinline__ v8_t<T> tile_tr8(const T* tile, int r0, int c0, int j, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const int row = 4 * (g >> 1) + (i >> 2);
  const int col = c0 + 16 * (g & 1) + 4 * (i & 3);
  // the slot depends on row bits 1-3 only, so rows r0 + 16 j + .. are the
  // lane's rows moved by a plain byte offset (an immediate of the read where
  // r0 and j are constants; the lane part is then loop-invariant)
  const char* base = reinterpret_cast<const char*>(tile) + (r0 + 16 * j) * 128;
  return cat44<T>(ds_tr4<T>(reinterpret_cast<const T*>(base + tile_off(row, col))),
                  ds_tr4<T>(reinterpret_cast<const T*>(base + tile_off(row + 8, col))));
}
// tile_tr8 on a wide tile (see wtile_ld8); c0 a multiple of 32
template <typename T>
__device__ __forceinline__ v8_t<T> wtile_tr8(const T* tile, int r0, int c0, int j, int lane) {
  return tile_tr8<T>(tile + (c0 >> 6) * 4096, r0, c0 & 63, j, lane);
}

// Compile-time bool for generic lambdas: body(BoolC<true>{}) instantiates
// the masked variant of a loop body, so the unmasked one carries no selects.
template <bool B>
struct BoolC {
  static constexpr bool value = B;
};
template <int V>
struct IntC {
  static constexpr int value = V;
  constexpr operator int() const { return V; }
};

// Position of logical element e (0..31) of a 32-block in the "operand
// order" layout: the eight elements ld_tr_op gathers for (j, h), rows
// 16j + 4h + 0..3 and 16j + 8 + 4h + 0..3, become the 8 contiguous elements
// at 16j + 8h, so a single 16-byte load (ld8 at 16j + 8h) replaces two.
__host__ __device__ constexpr int opord32(int e) {
  return (e & 16) | ((e & 4) << 1) | ((e & 8) >> 1) | (e & 3);
}

// C-layout fp32 block -> B operand (k-step j of its 32 rows), converted to T.
template <typename T>
__device__ __forceinline__ v8_t<T> c_to_b(const f32x16& a, int j) {
  f32x8 f{a[8 * j + 0], a[8 * j + 1], a[8 * j + 2], a[8 * j + 3],
          a[8 * j + 4], a[8 * j + 5], a[8 * j + 6], a[8 * j + 7]};
  if constexpr (sizeof(T) == 2) {
    return __builtin_convertvector(f, v8_t<T>);
  } else {
    return f;
  }
}

// ---------------------------------------------------------------------------
// 16 x 16 x 32 products for 16-wide outputs (a 16-dim SPD group).  Layout of
// v_mfma_f32_16x16x32_{bf16,f16}, lane l, row rho = l >> 4, i = l & 15:
//   A (16 x 32): lane holds A[i][8 rho + j],  B (32 x 16): B[8 rho + j][i],
//   C/D (16 x 16, 4 per lane): acc[r] = D[4 rho + r][i].
// A 32 x 32 fp32 block X in the 32x32 C layout (rows k, lane column n) feeds
// the two 16-column halves of such a product after one v_permlane16_swap per
// packed register pair: lane rows 1 and 3 trade their k-rows {0-11}+4h with
// rows 0 and 2's {16-27}+4h, after which 16-lane row rho holds, for column
// n = (half) 16 + i, the eight k-rows
//   t0(rho) + {0, 1, 2, 3, 8, 9, 10, 11},  t0(rho) = 16 (rho & 1) + 4 (rho >> 1),
// in that order.  The matching A operand reads the same k-rows (tile_tr8_16).
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// X (32x32 C layout, converted to T) -> B operands for columns 0-15 (b0) and 16-31 (b1).
template <typename T>
__device__ __forceinline__ void c_to_b16x2(const f32x16& x, v8_t<T>& b0, v8_t<T>& b1) {
  static_assert(sizeof(T) == 2, "16-bit operands");
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  u32x4 lo = __builtin_bit_cast(u32x4, c_to_b<T>(x, 0));
  u32x4 hi = __builtin_bit_cast(u32x4, c_to_b<T>(x, 1));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x2 sw = __builtin_amdgcn_permlane16_swap(lo[i], hi[i], false, false);
    lo[i] = sw[0];
    hi[i] = sw[1];
  }
  b0 = __builtin_bit_cast(v8_t<T>, lo);
  b1 = __builtin_bit_cast(v8_t<T>, hi);
}

// The A operand matching c_to_b16x2 from a natural 64 x 64 tile (tile_off
// layout): lane (rho, i) receives column c0 + i of rows r0 + t0(rho) + 0..3
// and r0 + t0(rho) + 8..11 (two transposing 8-byte reads).  r0 is a
// multiple of 16 (a plain byte offset, as in tile_tr8).
template <typename T>
__device__ __forceinline__ v8_t<T> tile_tr8_16(const T* tile, int r0, int c0, int lane) {
  const int rho = lane >> 4, i = lane & 15;
  const int row = 16 * (rho & 1) + 4 * (rho >> 1) + (i >> 2);
  const int col = c0 + 4 * (i & 3);
  const char* base = reinterpret_cast<const char*>(tile) + r0 * 128;
  return cat44<T>(ds_tr4<T>(reinterpret_cast<const T*>(base + tile_off(row, col))),
                  ds_tr4<T>(reinterpret_cast<const T*>(base + tile_off(row + 8, col))));
}

template <int CTRL>
__device__ __forceinline__ float dpp_plus(float v) {
  return v + __builtin_bit_cast(
                 float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// sum over each aligned group of L lanes (a power of two up to 64), the same
// bits on every lane: DPP steps inside a 16-lane row (quad xor 1, quad xor 2,
// half-row mirror, row mirror; each adds the same two partial sums on both
// sides), then xor-16 and xor-32 shuffles for wider groups
template <int L>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(L >= 1 && L <= 64 && (L & (L - 1)) == 0, "a power of two up to 64 lanes");
  if constexpr (L >= 2) v = dpp_plus<0xB1>(v);
  if constexpr (L >= 4) v = dpp_plus<0x4E>(v);
  if constexpr (L >= 8) v = dpp_plus<0x141>(v);
  if constexpr (L >= 16) v = dpp_plus<0x140>(v);
  if constexpr (L >= 32) v += __shfl_xor(v, 16);
  if constexpr (L >= 64) v += __shfl_xor(v, 32);
  return v;
}

// acc + sum of the 8 elements of an operand, in fp32.  For 16-bit types one
// v_dot2 against (1, 1) adds two elements, so a row sum over the rounded
// operand costs half an instruction per element.
template <typename T>
__device__ __forceinline__ float sum8(const v8_t<T>& p, float acc) {
  if constexpr (__is_same(T, __bf16)) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{p[2 * j], p[2 * j + 1]}, one, acc, false);
  } else if constexpr (__is_same(T, _Float16)) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_fdot2(f16x2{p[2 * j], p[2 * j + 1]}, one, acc, false);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += p[j];
  }
  return acc;
}

template <typename T>
__device__ __forceinline__ v4_t<T> to4(float a, float b, float c, float d) {
  f32x4 f{a, b, c, d};
  if constexpr (sizeof(T) == 2) return __builtin_convertvector(f, v4_t<T>);
  else return f;
}

template <typename T>
__device__ __forceinline__ v8_t<T> zero8() {
  return v8_t<T>{};
}

// Cooperative copy of a (64 x C) row-major tile of global rows
// [row0, row0 + 64) into LDS, natural (pitch NP) and/or transposed (pitch
// TP, element [c][r]).  Rows at or beyond nrows are written as zero.
// 4x4 element blocks per thread; 16 consecutive threads read one 64-element
// row segment, so global reads are coalesced.
template <typename T, int C, int NP, int TP, bool NAT, bool TRANS, int NT = 256>
__device__ __forceinline__ void load_tile64(const T* __restrict__ g, int row0, int nrows,
                                            int64_t row_stride, T* nat, T* trans, int tid) {
  constexpr int CB = C / 4;
  constexpr int NB = 16 * CB;
#pragma unroll
  for (int blk = tid; blk < NB; blk += NT) {
    const int cb = blk % CB, rb = blk / CB;
    v4_t<T> vals[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row0 + 4 * rb + r;
      if (row < nrows) vals[r] = ld4<T>(g + (int64_t)row * row_stride + 4 * cb);
      else vals[r] = v4_t<T>{};
    }
    if constexpr (NAT) {
#pragma unroll
      for (int r = 0; r < 4; ++r) st4<T>(nat + (4 * rb + r) * NP + 4 * cb, vals[r]);
    }
    if constexpr (TRANS) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        st4<T>(trans + (4 * cb + c) * TP + 4 * rb,
               v4_t<T>{vals[0][c], vals[1][c], vals[2][c], vals[3][c]});
    }
  }
}

// Block id -> (tile, head) with every head's tiles on one XCD (the hardware
// deals consecutive workgroups round-robin over the 8 XCDs, each with its
// own L2) and heavy (late, causal-long) tiles dispatched first.
__device__ __forceinline__ void map_block(int L, int ntiles, int nheads, int& tile, int& head,
                                          bool heavy_last_index) {
  int j;
  if ((nheads & 7) == 0) {
    const int x = L & 7;
    const int jj = L >> 3;
    const int hpx = nheads >> 3;
    j = jj / hpx;
    head = x + 8 * (jj % hpx);
  } else {
    j = L / nheads;
    head = L % nheads;
  }
  tile = heavy_last_index ? (ntiles - 1 - j) : j;
}

}  // namespace linatt

namespace linatt {

// Cooperative copy of a (64 x C) tile with type conversion and an optional
// per-row scale: rows [row0, row0 + 64) of g (element type S, row stride
// rs elements) go to LDS as T, natural (pitch NP, element [r][c]) and/or
// transposed (pitch TP, element [c][r]).  Rows at or beyond nrows are zero;
// rowscale (LDS, 64 floats, indexed by tile row) multiplies in fp32 before
// the conversion.  4x4 element blocks per thread, coalesced global reads.
template <typename S, typename T, int C, int NP, int TP, bool NAT, bool TRANS, int NT = 256>
__device__ __forceinline__ void load_tile64x(const S* __restrict__ g, int row0, int nrows,
                                             int64_t rs, T* nat, T* trans, int tid,
                                             const float* rowscale) {
  constexpr int CB = C / 4;
  constexpr int NB = 16 * CB;
#pragma unroll
  for (int blk = tid; blk < NB; blk += NT) {
    const int cb = blk % CB, rb = blk / CB;
    float vals[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row0 + 4 * rb + r;
      const float sc = rowscale ? rowscale[4 * rb + r] : 1.f;
      if (row < nrows) {
        const S* p = g + (int64_t)row * rs + 4 * cb;
        if constexpr (sizeof(S) == 4) {
          const float4 x = *reinterpret_cast<const float4*>(p);
          vals[r][0] = x.x * sc; vals[r][1] = x.y * sc; vals[r][2] = x.z * sc; vals[r][3] = x.w * sc;
        } else {
          const v4_t<S> x = ld4<S>(p);
#pragma unroll
          for (int cc = 0; cc < 4; ++cc) vals[r][cc] = (float)x[cc] * sc;
        }
      } else {
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) vals[r][cc] = 0.f;
      }
    }
    if constexpr (NAT) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        st4<T>(nat + (4 * rb + r) * NP + 4 * cb, to4<T>(vals[r][0], vals[r][1], vals[r][2], vals[r][3]));
    }
    if constexpr (TRANS) {
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
        st4<T>(trans + (4 * cb + cc) * TP + 4 * rb,
               to4<T>(vals[0][cc], vals[1][cc], vals[2][cc], vals[3][cc]));
    }
  }
}

// 8 consecutive fp32 values converted to an MFMA operand of type T.
template <typename T>
__device__ __forceinline__ v8_t<T> ld8_f32(const float* p) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  const f32x8 f{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  if constexpr (sizeof(T) == 2) return __builtin_convertvector(f, v8_t<T>);
  else return f;
}

// Swizzled 16-byte slot of (row, chunk) in a row-major LDS tile with CPR
// 16-byte chunks per row (XOR keeps it an involution within a row).
template <int CPR>
__device__ __forceinline__ int swz_slot(int row, int ch) {
  if constexpr (CPR >= 16) return row * CPR + (ch ^ (row & 15));
  else return row * CPR + (ch ^ ((row >> 1) & 7));
}

// A wave's 32 x 64 block of 16-bit values held in C layout (lane column =
// block row cl; columns 32 b + 8 I + 4 hh + r of the fp32 blocks X[b],
// b = 0, 1) written to global rows g + row * ld through 4 KiB of LDS: 8-byte
// LDS writes, then 16-byte reads that give each global store instruction
// 1 KiB of whole rows.  slot(s), s = 0..255, maps the 16-byte staging slots
// (row-major 32 x 8, XOR-swizzled by row) to LDS addresses owned by the
// calling wave.  OPORD stores each 32-column block in operand order
// (column e at 32 b + opord32(e)).
// The LDS half of store_rows_via alone: the block into 256 staging slots.
template <typename T, bool OPORD = false>
__device__ __forceinline__ void stage_rows(const f32x16& x0, const f32x16& x1, u32x4* stage, int lane) {
  const int cl = lane & 31, hh = lane >> 5;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const f32x16& x = b ? x1 : x0;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const int ch = OPORD ? 4 * b + 2 * (I >> 1) + hh : 4 * b + I;
      const int bo = OPORD ? 8 * (I & 1) : 8 * hh;
      *reinterpret_cast<v4_t<T>*>(reinterpret_cast<char*>(stage + swz_slot<8>(cl, ch)) + bo) =
          to4<T>(x[4 * I], x[4 * I + 1], x[4 * I + 2], x[4 * I + 3]);
    }
  }
}

// One half of stage_rows: the 32 x 32 block x as columns 32 b .. 32 b + 31
// of the 32 x 64 staged block (the other half is another wave's).
template <typename T>
__device__ __forceinline__ void stage_half(const f32x16& x, int b, u32x4* stage, int lane) {
  const int cl = lane & 31, hh = lane >> 5;
#pragma unroll
  for (int I = 0; I < 4; ++I)
    *reinterpret_cast<v4_t<T>*>(reinterpret_cast<char*>(stage + swz_slot<8>(cl, 4 * b + I)) + 8 * hh) =
        to4<T>(x[4 * I], x[4 * I + 1], x[4 * I + 2], x[4 * I + 3]);
}

// A wave's 32 x 32 block of 16-bit values in C layout (lane column = block
// row cl; columns 8 I + 4 hh + r) through 2 KiB of LDS (128 16-byte slots,
// row-major 32 x 4, XOR-swizzled by row) to rows g + row * ld: 8-byte LDS
// writes, then two buffer-store instructions of 16 whole 64-byte rows each
// (g wave-uniform, rows >= nvalid dropped).
__device__ __forceinline__ int swz4(int row, int ch) { return row * 4 + (ch ^ ((row >> 1) & 3)); }
// Cache policy of a buffer store: non-temporal (nt), for outputs the storing
// kernel does not read back.  Their lines then leave L2 first and do not
// displace the input tiles that a kernel's workgroups share through L2.
constexpr int kStoreStream = 2;
// Its LDS half: the block into the 128 staging slots.
template <typename T>
__device__ __forceinline__ void stage_rows32(const f32x16& x, u32x4* stage, int lane) {
  const int cl = lane & 31, hh = lane >> 5;
#pragma unroll
  for (int I = 0; I < 4; ++I)
    *reinterpret_cast<v4_t<T>*>(reinterpret_cast<char*>(stage + swz4(cl, I)) + 8 * hh) =
        to4<T>(x[4 * I], x[4 * I + 1], x[4 * I + 2], x[4 * I + 3]);
}
// Its global half, by any wave of the workgroup once the block is staged.
// CP is the stores' cache policy (kStoreStream: non-temporal).
template <typename T, int CP = 0>
__device__ __forceinline__ void flush_rows32(const u32x4* stage, T* g, int64_t ld, int lane, int nvalid = 32) {
  const int nv = nvalid < 0 ? 0 : (nvalid > 32 ? 32 : nvalid);
  const unsigned ldb = (unsigned)(ld * (int64_t)sizeof(T));
  const __amdgpu_buffer_rsrc_t rs = buf_rsrc(g, nv == 0 ? 0u : (unsigned)(nv - 1) * ldb + 64u);
#pragma unroll
  for (int op = 0; op < 2; ++op) {
    const int gi = 64 * op + lane, row = gi >> 2, ch = gi & 3;
    __builtin_amdgcn_raw_buffer_store_b128(stage[swz4(row, ch)], rs, (int)(row * ldb + 16 * ch), 0, CP);
  }
}
template <typename T, int CP = 0>
__device__ __forceinline__ void store_rows32(const f32x16& x, u32x4* stage, T* g, int64_t ld, int lane,
                                             int nvalid = 32) {
  stage_rows32<T>(x, stage, lane);
  flush_rows32<T, CP>(stage, g, ld, lane, nvalid);
}

// The global half: a staged block's 32 rows to g + row * ld (g wave-uniform,
// rows >= nvalid dropped), by any wave of the workgroup.
template <typename T, int CP = 0>
__device__ __forceinline__ void flush_rows(const u32x4* stage, T* g, int64_t ld, int lane, int nvalid = 32) {
  const int nv = nvalid < 0 ? 0 : (nvalid > 32 ? 32 : nvalid);
  const unsigned ldb = (unsigned)(ld * (int64_t)sizeof(T));
  const __amdgpu_buffer_rsrc_t rs = buf_rsrc(g, nv == 0 ? 0u : (unsigned)(nv - 1) * ldb + 128u);
#pragma unroll
  for (int op = 0; op < 4; ++op) {
    const int gi = 64 * op + lane, row = gi >> 3, ch = gi & 7;
    __builtin_amdgcn_raw_buffer_store_b128(stage[swz_slot<8>(row, ch)], rs, (int)(row * ldb + 16 * ch), 0, CP);
  }
}

template <typename T, bool OPORD = false, typename SlotFn>
__device__ __forceinline__ void store_rows_via(const f32x16& x0, const f32x16& x1, SlotFn slot,
                                               T* g, int64_t ld, int lane, int nvalid = 32) {
  // g (wave-uniform) .. row nvalid - 1: buffer stores, rows >= nvalid dropped
  const int nv = nvalid < 0 ? 0 : (nvalid > 32 ? 32 : nvalid);
  const unsigned ldb = (unsigned)(ld * (int64_t)sizeof(T));
  const __amdgpu_buffer_rsrc_t rs = buf_rsrc(g, nv == 0 ? 0u : (unsigned)(nv - 1) * ldb + 128u);
  const int cl = lane & 31, hh = lane >> 5;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const f32x16& x = b ? x1 : x0;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      // natural: columns 8 I + 4 hh + 0..3; operand order: 16 (I >> 1) + 8 hh + 4 (I & 1) + 0..3
      const int ch = OPORD ? 4 * b + 2 * (I >> 1) + hh : 4 * b + I;
      const int bo = OPORD ? 8 * (I & 1) : 8 * hh;
      *reinterpret_cast<v4_t<T>*>(reinterpret_cast<char*>(slot(swz_slot<8>(cl, ch))) + bo) =
          to4<T>(x[4 * I], x[4 * I + 1], x[4 * I + 2], x[4 * I + 3]);
    }
  }
#pragma unroll
  for (int op = 0; op < 4; ++op) {
    const int gi = 64 * op + lane, row = gi >> 3, ch = gi & 7;
    const u32x4 val = *slot(swz_slot<8>(row, ch));
    __builtin_amdgcn_raw_buffer_store_b128(val, rs, (int)(row * ldb + 16 * ch), 0, 0);
  }
}

// The same through a contiguous 4 KiB staging area (rows >= nvalid are
// not stored).
template <typename T, bool OPORD = false>
__device__ __forceinline__ void store_rows_staged(const f32x16& x0, const f32x16& x1, u32x4* stage,
                                                  T* g, int64_t ld, int lane, int nvalid = 32) {
  store_rows_via<T, OPORD>(x0, x1, [&](int s) { return stage + s; }, g, ld, lane, nvalid);
}

// store_rows_staged with buffer stores: rows at byte offset soff (wave-
// uniform) + row * ld_bytes of the buffer rs; the per-lane part of every
// address is chunk-invariant.
template <typename T>
__device__ __forceinline__ void store_rows_buf(const f32x16& x0, const f32x16& x1, u32x4* stage,
                                               __amdgpu_buffer_rsrc_t rs, int soff, int ld_bytes,
                                               int lane) {
  const int cl = lane & 31, hh = lane >> 5;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const f32x16& x = b ? x1 : x0;
#pragma unroll
    for (int I = 0; I < 4; ++I)
      *reinterpret_cast<v4_t<T>*>(reinterpret_cast<char*>(stage + swz_slot<8>(cl, 4 * b + I)) + 8 * hh) =
          to4<T>(x[4 * I], x[4 * I + 1], x[4 * I + 2], x[4 * I + 3]);
  }
  const int voff = (lane >> 3) * ld_bytes + 16 * (lane & 7);
#pragma unroll
  for (int op = 0; op < 4; ++op) {
    const u32x4 val = stage[swz_slot<8>(8 * op + (lane >> 3), lane & 7)];
    __builtin_amdgcn_raw_buffer_store_b128(val, rs, voff + 8 * op * ld_bytes, soff, 0);
  }
}

}  // namespace linatt
