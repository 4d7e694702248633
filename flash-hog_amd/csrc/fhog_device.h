// Device-side building blocks shared by every Flash-HOG kernel on gfx950.
//
// All kernels work on one 64-lane wavefront per 32-row slab and use the CDNA
// 32x32x16 matrix instruction (v_mfma_f32_32x32x16_{bf16,f16}); fp32 inputs use
// eight v_mfma_f32_32x32x2f32 per 16-deep step so that one code path serves all
// three dtypes.
//
// Operand layouts of the 32x32x16 instruction (lane l, n = l & 31, g = l >> 5):
//   A (32 x 16):  lane holds A[m = n][k = 8g + e],          e = 0..7
//   B (16 x 32):  lane holds B[k = 8g + e][n],              e = 0..7
//   C (32 x 32):  lane holds C[m = 8(r/4) + 4g + r%4][n],    r = 0..15
// Because a C tile is indexed by the lane along n, a C tile converted to the
// input dtype can be fed straight back as an A or B operand for a product that
// contracts over its m index. Register r = 8s + e of step s then stands for
// m = cperm(s, g, e) = 16s + 8(e/4) + 4g + e%4; the other operand is read from
// LDS with the same permutation (two 4-element runs per lane).
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>
#include <stdint.h>

namespace fhog {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

template <typename T> struct Vec;
template <> struct Vec<__bf16> { typedef bf16x8 x8; typedef bf16x4 x4; };
template <> struct Vec<_Float16> { typedef f16x8 x8; typedef f16x4 x4; };
template <> struct Vec<float> { typedef f32x8 x8; typedef f32x4 x4; };

template <typename T> using V8 = typename Vec<T>::x8;
template <typename T> using V4 = typename Vec<T>::x4;

// C += A * B on a 32x32 tile with a 16-deep contraction.
template <typename T> __device__ __forceinline__ f32x16 mma(V8<T> a, V8<T> b, f32x16 c);

template <> __device__ __forceinline__ f32x16 mma<__bf16>(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
template <> __device__ __forceinline__ f32x16 mma<_Float16>(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
// fp32: instruction e contracts over lane groups g = 0, 1, i.e. logical k = 8g + e.
template <> __device__ __forceinline__ f32x16 mma<float>(f32x8 a, f32x8 b, f32x16 c) {
#pragma unroll
  for (int e = 0; e < 8; ++e) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], b[e], c, 0, 0, 0);
  return c;
}

template <typename T> __device__ __forceinline__ V8<T> cvt8(f32x8 x) {
  return __builtin_convertvector(x, V8<T>);
}
template <typename T> __device__ __forceinline__ V4<T> cvt4(f32x4 x) {
  return __builtin_convertvector(x, V4<T>);
}

__device__ __forceinline__ f32x8 lo8(f32x16 x) {
  return __builtin_shufflevector(x, x, 0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ f32x8 hi8(f32x16 x) {
  return __builtin_shufflevector(x, x, 8, 9, 10, 11, 12, 13, 14, 15);
}

template <typename T> __device__ __forceinline__ V8<T> zero8() {
  V8<T> z;
#pragma unroll
  for (int e = 0; e < 8; ++e) z[e] = (T)0.0f;
  return z;
}

template <typename T> __device__ __forceinline__ V8<T> ones8() {
  V8<T> z;
#pragma unroll
  for (int e = 0; e < 8; ++e) z[e] = (T)1.0f;
  return z;
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int r = 0; r < 16; ++r) z[r] = 0.0f;
  return z;
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Sum of a lane value with the lane 32 positions away (the other row group of
// a 32x32 tile).
__device__ __forceinline__ float xgroup_sum(float x) { return x + __shfl_xor(x, 32, 64); }
__device__ __forceinline__ float xgroup_max(float x) { return fmaxf(x, __shfl_xor(x, 32, 64)); }

// Row index (within a 32-row C tile) held by register r of a lane in group g.
__device__ __forceinline__ int crow(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

// acc + <a, b> over eight 2-byte elements, two products per v_dot2, pairs in
// order. The first backward's two dQ kernels form D = rowsum(O dO) with it,
// so that D does not depend on which of them runs (left to itself the
// compiler turns such a sum into v_dot2 in one kernel and into mixed-precision
// fmas in another, which round differently).
template <typename T> __device__ __forceinline__ float dot8(V8<T> a, V8<T> b, float acc) {
  typedef T T2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const T2 x = {a[2 * i], a[2 * i + 1]};
    const T2 y = {b[2 * i], b[2 * i + 1]};
    if constexpr (std::is_same_v<T, __bf16>)
      acc = __builtin_amdgcn_fdot2_f32_bf16(x, y, acc, false);
    else
      acc = __builtin_amdgcn_fdot2(x, y, acc, false);
  }
  return acc;
}

// ---------------------------------------------------------------------------
// Swizzled tiles written straight from global memory into LDS.
//
// A tile is 32 rows x D columns, stored row-major without padding; each row is
// split into 16-byte chunks and chunk c of row r is stored at chunk position
// c ^ key(r) (within aligned groups of 8 chunks). Two keys are used, chosen by
// measurement (a probe timing each read pattern of the kernels alone, 8 waves
// per CU, ns per wave-wide read per CU; a contiguous 1 KB ds_read_b128 takes
// 2.17):
//   kSwzPairs, key = bit reversal of (r / 2) mod 8, for the 32x32x16 operand
//     reads: row fragments 2.17, transposed fragments 1.36;
//   kSwzRows, key = r mod 8, for the 16x16x32 operand reads: row fragments
//     2.07, transposed fragments 1.31.
// Each key is slow for the other instruction's row reads (3.6-3.7 ns, and the
// PMC counter SQ_LDS_BANK_CONFLICT reports the extra cycles), so a tile's key
// follows the instruction that reads it. Both keys repeat every 16 rows, and
// key(r + 8) = key(r) ^ 1 for kSwzPairs.
//
// global_load_lds with 16 bytes per lane writes lane l's data to
// lds_base + 16 l, so lane l of load t fills chunk position l % CH of row
// t * (64 / CH) + l / CH and fetches the logical chunk stored there.
// ---------------------------------------------------------------------------
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) const char lds_cchar;

constexpr int kSwzPairs = 0;
constexpr int kSwzRows = 1;

template <int SWZ = kSwzPairs> __device__ __forceinline__ int swz(int r) {
  if constexpr (SWZ == kSwzRows) {
    return r & 7;
  } else {
    const int m = (r >> 1) & 7;
    return ((m & 1) << 2) | (m & 2) | (m >> 2);
  }
}
template <int SWZ = kSwzPairs> __device__ __forceinline__ int phys_chunk(int r, int c) {
  return (c & ~7) | ((c & 7) ^ swz<SWZ>(r));
}

template <typename T, int D> struct SwzTile {
  static constexpr int kRows = 32;
  static constexpr int kRowBytes = D * (int)sizeof(T);
  static constexpr int kChunks = kRowBytes / 16;        // 16-byte chunks per row
  static constexpr int kRowsPerLoad = 64 / kChunks;     // rows one wave-wide 16-byte load fills
  static constexpr int kLoads = kRows / kRowsPerLoad;   // wave-wide loads per tile
  static constexpr int kElems = kRows * D;
  static_assert(kChunks % 8 == 0 && kChunks <= 64, "row must be a multiple of 128 bytes");
};

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// Wave-uniform LDS byte address of p (the M0 operand of the LDS DMAs).
__device__ __forceinline__ uint32_t lds_base_u32(const void* p) {
  return __builtin_amdgcn_readfirstlane(lds_addr(p));
}

// fp32 operands read from a swizzled tile (4-byte elements, 16-byte chunks of
// 4): frag_row_swz contracts over columns (lane (n, g) gets row n, columns
// 16 ks + 8 g .. +7), frag_tr_swz over the 32 tile rows in the permuted order
// of a C tile fed back as an operand (lane l gets column dbase + (l & 31), rows
// 16 s + 8 (e / 4) + 4 g + e % 4).
template <typename T, int D>
__device__ __forceinline__ V8<T> frag_row_swz(const T* tile, int n, int g, int ks) {
  static_assert(sizeof(T) == 4, "2-byte types use SwzFrags' LDS reads");
  const T* row = tile + n * D;
  const V4<T> a = *reinterpret_cast<const V4<T>*>(row + 4 * phys_chunk(n, 4 * ks + 2 * g));
  const V4<T> b = *reinterpret_cast<const V4<T>*>(row + 4 * phys_chunk(n, 4 * ks + 2 * g + 1));
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

template <typename T, int D>
__device__ __forceinline__ V8<T> frag_tr_swz(const T* tile, int dbase, int lane, int s) {
  static_assert(sizeof(T) == 4, "2-byte types use SwzFrags' LDS reads");
  const int g = lane >> 5;
  const int col = dbase + (lane & 31);
  V8<T> v;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int row = 16 * s + 8 * (e >> 2) + 4 * g + (e & 3);
    v[e] = tile[row * D + 4 * phys_chunk(row, col >> 2) + (col & 3)];
  }
  return v;
}

// Wait until this wave's outstanding vector-memory operations (including
// global_load_lds) have completed; lgkm and exp counters are left alone.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Wait until at most N vector-memory operations of this wave are outstanding
// (s_waitcnt encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
// Loads complete in issue order for this counter, so after the wait every load
// issued before the last N has landed.
template <int N> __device__ __forceinline__ void wait_vmem_le() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// Waits until the tile of iteration `it` (of `total`) of an NST-stage ring has
// landed in LDS, for a wave that issues LOADS loads per tile and keeps NST - 1
// tiles in flight: the loads of at most NST - 2 later tiles may be outstanding.
template <int NST, int LOADS>
__device__ __forceinline__ void wait_tile(int it, int total) {
  if constexpr (NST >= 3) {
    if (it + NST - 2 < total) {
      wait_vmem_le<(NST - 2) * LOADS>();
      return;
    }
  }
  wait_vmem_le<0>();
}

// Position of an iteration of a key-tiled sweep over a group of query heads:
// query tile qt (relative to the first) of head gi of the group, heads
// innermost. Advanced one iteration at a time, so no division by the group size.
struct GroupCursor {
  int qt = 0, gi = 0;
  __device__ __forceinline__ void next(int grp) {
    if (++gi == grp) {
      gi = 0;
      ++qt;
    }
  }
};

// Global -> LDS loads (LDS DMA). Each is a wave-wide global_load_lds whose
// lane l writes its bytes to lds_byte_addr + (4 or 16) l, issued as inline
// assembly so that the compiler does not track it: its waitcnt pass would
// otherwise wait for every in-flight LDS DMA before each LDS read (it cannot
// prove they touch different buffers), serialising the prefetch with the
// compute that should hide it. Completion is ordered explicitly instead: an
// explicit vmcnt wait and a workgroup barrier before a staged tile is read, a
// barrier before a stage is overwritten. Untracked vector-memory operations
// only make the compiler's own vmcnt waits more conservative, never less.
//
// The LDS destination goes in M0. It is an operand bound to that register
// ("{m0}"), so the compiler itself writes M0 before the statement and knows
// its value afterwards; the statement only reads M0.
//
// Wait states. The compiler's hazard check does not look inside inline
// assembly, so each statement starts with the ones its operands need: one
// between an SALU write of M0 and an LDS DMA, and five between a VALU write of
// an SGPR and a vector-memory instruction that reads that SGPR. The second
// arises whenever the compiler reloads a spilled SGPR of the scalar base with
// v_readlane just before the statement; the load could then read the base's
// previous contents (say, a saved exec mask) and fault. s_nop 4 gives five;
// the DMAs that follow one from the same base in a tile's sequence need only
// the first.

// 16 bytes per lane, addressed as a uniform 64-bit base (SGPR pair) plus a
// per-lane 32-bit byte offset.
__device__ __forceinline__ void dma16s(const void* sbase, uint32_t voff, uint32_t lds_byte_addr) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "{m0}"(lds_byte_addr)
               : "memory");
}

// dma16s directly after another dma16s from the same base: the base is already
// settled, so only M0's wait state is needed (tests/test_dma_wait_states.py
// checks the built code for a VALU write of any DMA base within five states).
__device__ __forceinline__ void dma16s_next(const void* sbase, uint32_t voff, uint32_t lds_byte_addr) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "{m0}"(lds_byte_addr)
               : "memory");
}

// 4 bytes per lane, addressed as a uniform base plus a per-lane byte offset.
__device__ __forceinline__ void dma4s(const void* sbase, uint32_t voff, uint32_t lds_byte_addr) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, %1"
               :
               : "v"(voff), "s"(sbase), "{m0}"(lds_byte_addr)
               : "memory");
}

// Per-lane source offsets of the wave-wide loads that fill one swizzled 32 x D
// tile: loads first .. first + COUNT - 1 of the tile's kLoads (a wave may fill
// only part of a tile). They depend only on the lane, the row stride and the
// number of valid rows, so a streaming loop computes them once and then only
// advances the uniform base address per tile.
template <typename T, int D, int COUNT = SwzTile<T, D>::kLoads, int SWZ = kSwzPairs> struct TileDma {
  typedef SwzTile<T, D> G;
  static_assert(COUNT >= 1 && COUNT <= G::kLoads, "bad load count");
  uint32_t voff[COUNT];
  int first;

  // Rows at or beyond nvalid are redirected to row nvalid - 1 (finite data for
  // rows that every consumer masks). first_load must be wave-uniform.
  __device__ __forceinline__ void init(uint32_t row_stride_bytes, int nvalid, int lane, int first_load = 0) {
    first = first_load;
    const int p = lane % G::kChunks;
#pragma unroll
    for (int i = 0; i < COUNT; ++i) {
      const int row = (first + i) * G::kRowsPerLoad + lane / G::kChunks;
      const int src_row = min(row, nvalid - 1);
      voff[i] = (uint32_t)src_row * row_stride_bytes + 16u * (uint32_t)phys_chunk<SWZ>(row, p);
    }
  }

  // lds_tile_addr (the tile's first byte) must be wave-uniform; gbase is the
  // tile's first row.
  __device__ __forceinline__ void issue(uint32_t lds_tile_addr, const void* gbase) const {
    dma16s(gbase, voff[0], lds_tile_addr + 1024u * first);
#pragma unroll
    for (int i = 1; i < COUNT; ++i) dma16s_next(gbase, voff[i], lds_tile_addr + 1024u * (first + i));
  }
};

// MFMA operand fragments read from a swizzled 32 x D tile in LDS. `stage` is
// the wave-uniform LDS byte address of a ring stage and `off` the tile's byte
// offset within it (a constant after inlining). For 2-byte types the per-lane
// byte offsets are computed once per kernel, so that a read is one add of the
// stage to a fixed per-lane offset (shared by every tile of the stage) with
// the constant in the instruction's offset field; computing addresses from
// pointers instead leaves the compiler to rebuild the swizzled offsets inside
// the loop when registers are scarce.
template <typename T, int D> struct SwzFrags {
  uint32_t row[D / 16];  // row operand of step ks
  uint32_t tr[D / 32];   // first transposed read of column block dt, step 0 (rows 4 g + i / 4)
  int lane;

  __device__ __forceinline__ void init(int lane_id) {
    lane = lane_id;
    if constexpr (sizeof(T) == 2) {
      const int n = lane & 31, g = lane >> 5;
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks)
        row[ks] = 2u * (uint32_t)(n * D + 8 * phys_chunk(n, 2 * ks + g));
      const int i = lane & 15;
      const int r = 4 * g + (i >> 2);
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        const int d = 32 * dt + 16 * ((lane >> 4) & 1) + 4 * (i & 3);
        tr[dt] = 2u * (uint32_t)(r * D + 8 * phys_chunk(r, d >> 3) + (d & 7));
      }
    }
  }

  // Operand contracting over columns: lane (n, g) gets row n, columns 16 ks + 8 g .. +7.
  __device__ __forceinline__ V8<T> rowf(uint32_t stage, int off, int ks) const {
    if constexpr (sizeof(T) == 2) {
      const lds_cchar* p = reinterpret_cast<const lds_cchar*>((uintptr_t)(stage + row[ks]));
      return *reinterpret_cast<const __attribute__((address_space(3))) V8<T>*>(p + off);
    } else {
      return frag_row_swz<T, D>(tile_ptr(stage, off), lane & 31, lane >> 5, ks);
    }
  }

  // Operand contracting over the tile rows in the permuted C order: lane l gets
  // column 32 dt + (l & 31), rows 16 s + 8 (e / 4) + 4 g + e % 4. For 2-byte
  // types that is two ds_read_b64_tr_b16 (rows 16 s + 4 g + {0..3} and the same
  // + 8): within each 16-lane group, lane i receives element i % 4 of the 8
  // bytes that lane 4 e + i / 4 addresses, so lane i addresses columns
  // 4 (i % 4) .. +3 of row i / 4 of the 4-row block. The swizzle repeats every
  // 16 rows, so step s is a constant offset from step 0; and swz(r + 8) =
  // swz(r) ^ 1, so the second read's address is the first one with bit 4 (the
  // chunk's lowest bit) flipped, 8 rows further on. That needs stage + off to
  // be a multiple of 32, which every ring stage and tile offset here is.
  __device__ __forceinline__ V8<T> trf(uint32_t stage, int off, int dt, int s) const {
    if constexpr (sizeof(T) == 2) {
      const uint32_t a0 = stage + tr[dt];
      const lds_cchar* a = reinterpret_cast<const lds_cchar*>((uintptr_t)a0) + off + s * 32 * D;
      const lds_cchar* b = reinterpret_cast<const lds_cchar*>((uintptr_t)(a0 ^ 16u)) + off + s * 32 * D + 16 * D;
      const i16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(a));
      const i16x4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(b));
      return __builtin_shufflevector(__builtin_bit_cast(V4<T>, x), __builtin_bit_cast(V4<T>, y), 0, 1, 2, 3, 4, 5,
                                     6, 7);
    } else {
      return frag_tr_swz<T, D>(tile_ptr(stage, off), 32 * dt, lane, s);
    }
  }

 private:
  __device__ __forceinline__ static const T* tile_ptr(uint32_t stage, int off) {
    // an address-space conversion, which only a C-style cast expresses
    return (const T*)((const lds_cchar*)(uintptr_t)stage + off);
  }
};

// ---------------------------------------------------------------------------
// The 16x16x32 matrix instruction (v_mfma_f32_16x16x32_{bf16,f16}), used by
// the kernels that give each wave 16 rows (lane l, n = l % 16, g = l / 16):
//   A (16 x 32): lane holds A[m = n][k = 8 g + e],   e = 0..7
//   B (32 x 16): lane holds B[k = 8 g + e][n]
//   C (16 x 16): lane holds C[m = 4 g + i][n],      i = 0..3
// A pair of C tiles (rows 0..15 and 16..31 of a 32-row tile) fed back as the
// B operand of a product contracting over those 32 rows stands for rows
// 4 g + e (e < 4) and 16 + 4 g + e - 4 (e >= 4) in register e; the other
// operand is read from LDS in the same order (SwzFrags16::trf).
// ---------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ f32x4 mma16(V8<T> a, V8<T> b, f32x4 c);
template <> __device__ __forceinline__ f32x4 mma16<__bf16>(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
template <> __device__ __forceinline__ f32x4 mma16<_Float16>(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Sum over the four 16-lane groups (the lanes that hold the same column n).
// acc + the sum of the eight values of v as rounded to T (the values an MFMA
// that takes v as an operand multiplies), by dot products with ones.
template <typename T> __device__ __forceinline__ float add_sum8(V8<T> v, float acc) {
  typedef T T2 __attribute__((ext_vector_type(2)));
  const T2 ones = {(T)1.0f, (T)1.0f};
  const T2 pairs[4] = {__builtin_shufflevector(v, v, 0, 1), __builtin_shufflevector(v, v, 2, 3),
                       __builtin_shufflevector(v, v, 4, 5), __builtin_shufflevector(v, v, 6, 7)};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (std::is_same_v<T, __bf16>)
      acc = __builtin_amdgcn_fdot2_f32_bf16(pairs[i], ones, acc, false);
    else
      acc = __builtin_amdgcn_fdot2(pairs[i], ones, acc, false);
  }
  return acc;
}

__device__ __forceinline__ float group4_sum(float x) {
  x += __shfl_xor(x, 16, 64);
  return x + __shfl_xor(x, 32, 64);
}

// Per-lane LDS byte offsets of the 16x16x32 operand fragments read from a
// swizzled 32 x D tile (2-byte types).
template <typename T, int D> struct SwzFrags16 {
  static_assert(sizeof(T) == 2, "2-byte types only");
  uint32_t row[D / 32];  // score A operand: row l % 16, columns 32 ks + 8 (l / 16) .. +7
  uint32_t tr[D / 16];   // output A operand of column block db: rows 4 (l / 16) + i / 4
  __device__ __forceinline__ void init(int lane) {
    const int n = lane & 15, g = lane >> 4;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) row[ks] = 2u * (uint32_t)(n * D + 8 * phys_chunk<kSwzRows>(n, 4 * ks + g));
    const int r = 4 * g + (n >> 2);
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      const int d = 16 * db + 4 * (n & 3);
      tr[db] = 2u * (uint32_t)(r * D + 8 * phys_chunk<kSwzRows>(r, d >> 3) + (d & 7));
    }
  }
  // Keys 16 kb + l % 16 of the tile at stage + off, step ks. The swizzle
  // repeats every 16 rows, so kb is a constant offset.
  __device__ __forceinline__ V8<T> rowf(uint32_t stage, int off, int kb, int ks) const {
    const lds_cchar* p = reinterpret_cast<const lds_cchar*>((uintptr_t)(stage + row[ks])) + off + kb * 16 * D * 2;
    return *reinterpret_cast<const __attribute__((address_space(3))) V8<T>*>(p);
  }
  // Column 16 db + l % 16, keys 4 g + {0..3} and 16 + 4 g + {0..3}: within a
  // 16-lane group, lane i addresses row 4 g + i / 4, columns 16 db + 4 (i % 4)
  // .. +3, and receives column 16 db + i of the four rows.
  __device__ __forceinline__ V8<T> trf(uint32_t stage, int off, int db) const {
    const lds_cchar* a = reinterpret_cast<const lds_cchar*>((uintptr_t)(stage + tr[db])) + off;
    const i16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(a));
    const i16x4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(a + 16 * D * 2));
    return __builtin_shufflevector(__builtin_bit_cast(V4<T>, x), __builtin_bit_cast(V4<T>, y), 0, 1, 2, 3, 4, 5, 6,
                                   7);
  }
};


// Grid order of the sequence-tiled kernels. A workgroup takes one (batch,
// head) pair and one block along the sequence, its `rank` (for causal grids
// rank 0 is the block with the most unmasked tiles). Pairs are taken in
// chunks of `chunk`: all ranks of one chunk precede the next chunk, so the
// blocks of one pair run close together in time and share the pair's streamed
// tiles in L2; with `chunk` a multiple of 8 they also run on one XCD, since
// workgroup i goes to XCD i mod 8. chunk = npairs is the plain rank-major
// order over all pairs.
struct GridSlot {
  int rank, pair;
};
__device__ __forceinline__ GridSlot grid_slot(int wg, int npairs, int nranks, int chunk) {
  const int per = chunk * nranks;
  const int c = wg / per;
  const int rem = wg - c * per;
  const int n = min(chunk, npairs - c * chunk);  // pairs in this chunk (the last may be short)
  const int rank = rem / n;
  return GridSlot{rank, c * chunk + rem - rank * n};
}

// Mirror pairing of causal blocks. Block r of a causal grid holds work
// proportional to nb - r (key-tiled) or r + 1 (query-tiled, in rank order:
// rank r is block nb - 1 - r), so a workgroup that takes rank r and then rank
// nb - 1 - r does about the same work for every r, and the grid has no tail of
// short blocks. pairs = 2 is for a paired grid of exactly two workgroups per
// CU (nb a multiple of 4): workgroup i and i + (grid size) / 2 then share a CU
// and i, placed first, is favoured by the wave arbiter (oldest first), so with
// equal work it ends long before its neighbour, which then runs alone. The
// favoured ranks r < q = nb / 4 therefore take the longer second rank
// nb - 1 - q - r and the others nb - 1 + q - r: the two workgroups of a CU then
// carry nb + 1 + q and nb + 1 - q units of work. pairs = 0: one rank per
// workgroup.
struct BlockPair {
  int first, second, count;
};
__device__ __forceinline__ BlockPair block_pair(int rank, int nb, int pairs) {
  int second = nb - 1 - rank;
  if (pairs == 2) second += rank < nb / 4 ? -(nb / 4) : nb / 4;
  return BlockPair{rank, second, (pairs && second != rank) ? 2 : 1};
}

// Workgroups of 4 waves resident on the current device at once, at `waves`
// waves per SIMD (0 if the device cannot be queried).
inline int resident_workgroups(int waves) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  return cus * waves;
}

// The chunk for grid_slot. A grid of at most 8 rounds of resident
// workgroups keeps the rank-major order, whose last round holds the blocks
// with the least work; a longer grid takes about one round per chunk (at
// least 8 pairs, a multiple of 8), so that the streamed tiles of the pairs
// in flight stay in L2 instead of being fetched again by every block.
inline int grid_chunk(int npairs, int nranks, int resident) {
  if (resident <= 0 || (long)npairs * nranks <= 8L * resident) return npairs;
  const int c = resident / nranks / 8 * 8;
  return c < 8 ? 8 : (c < npairs ? c : npairs);
}

// The `pairs` argument of block_pair for a grid of nb causal blocks per
// (batch, head) pair: mirror pairs when the unpaired grid outnumbers the
// resident workgroups, skewed ones when the paired grid is exactly one round
// at two workgroups per CU.
inline int block_pairing(bool causal, int nb, int npairs, int resident, int waves) {
  int pairs = causal && resident > 0 && (long)nb * npairs > resident;
  if (pairs && nb % 4 == 0 && (long)((nb + 1) / 2) * npairs == resident && waves == 2) pairs = 2;
  return pairs;
}

}  // namespace fhog
