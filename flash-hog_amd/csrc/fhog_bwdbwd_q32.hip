// Stage 1 of the Flash-HOG double backward (passes 1-3 in one sweep over the
// keys) for 2-byte types at D = 64: 32 queries per wave on the 32x32x16
// matrix instruction, one wave per SIMD, software-pipelined three tiles deep.
// The math and outputs are those of fhog_bwdbwd_fused.hip (which serves
// D = 128 and 256): with u = dP - D, x = P ddS, X = P (dPa + ddS u),
//   dQ2 = scale (sum_j P u ddK + sum_j X K - dD sum_j P u K - c sum_j P K),
//   ddO = sum_j P ddV + sum_j x V - dD' O,     c = D dD + B,
//   c = sum_j X - dD sum_j P u,  B = c - D dD,
// summed per pair in fp32 (flash_hog/_jax_refs/jax_impl.py:273-336, the pass
// split of flash_hog/jax/_pallas_gpu_kernel.py:149-278).
//
// Why this shape. A 16-query wave (the fused kernel) reads every key-side
// tile twice from LDS per 16 queries and issues a 16x16x32 instruction per
// 8192 multiply-adds; two such waves share a SIMD so that one wave's vector
// work overlaps the other's matrix work, and the matrix pipe stays about 43 %
// busy. With 32 queries per wave each LDS fragment serves twice the pairs and
// each matrix instruction does twice the work, but the four 32 x 64
// accumulators, two score sets and the resident operands need about 420
// registers, i.e. one wave per SIMD. A lone wave keeps the pipe fed only if
// its own instruction stream interleaves matrix, vector and LDS work, so each
// step of the loop mixes three tiles: the output products of tile t - 1, the
// element-wise step of tile t and the score products of tile t + 1, all
// independent of one another. (A loop of 44 such matrix instructions, 200
// vector and 48 LDS instructions and a barrier runs at 37.5 cycles per
// matrix instruction at one wave per SIMD: 85 % of the pipe.)
//
// The default stage 1 for 2-byte types at D = 64: 177-180 us at B4 N2048 H16
// causal bf16 against 184-189 us for the fused kernel, 3-6 % faster on every
// D = 64 configuration measured.
//
// Layouts (32x32x16, see fhog_device.h): score tiles are transposed,
// S^T = K Q^T, so lane n of a wave holds query q0 + n and register r key
// 8 (r / 4) + 4 g + r % 4 of the tile; a tile's registers 8 s .. 8 s + 7,
// converted to T, are the B operand of an output product over keys
// 16 s + 8 (e / 4) + 4 g + e % 4, whose A operand is the key-side tile read
// transposed in that order (SwzFrags::trf).
#include <cmath>
#include <cstdint>
#include <type_traits>

#include "fhog_device.h"
#include "fhog_params.h"
#include "fhog_q32_loop.inc"

namespace fhog {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

__device__ __forceinline__ uint32_t uni(uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); }
__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ const void* uni(const void* x) {
  const uint64_t u = (uint64_t)(uintptr_t)x;
  return (const void*)(uintptr_t)((uint64_t)uni((uint32_t)u) | ((uint64_t)uni((uint32_t)(u >> 32)) << 32));
}

// A workgroup's share of the grid. The grid is persistent (at most one
// workgroup per CU, the most that fit at one wave per SIMD) and walks a list
// of items: with a causal mask item r of a (batch, head) pair is the query
// block of rank r (nqb - 1 - r, the longest rows first) followed by the block
// of rank nqb - 1 - r, so every item but a middle one holds the same number
// of key tiles; without a mask an item is one block. Workgroup w takes items
// w', w' + G, w' + 2 G, ... where w' numbers the workgroups XCD by XCD (the
// hardware hands workgroup w to XCD w mod 8), so that the blocks a (batch,
// head) pair has in flight share one L2.
struct Q32Walk {
  int item, half;
};

template <typename T, bool CAUSAL, bool PRE>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
bwdbwd_q32_kernel(BwdBwdParams<T> p, int nitems) {
  constexpr int D = 64;
  typedef SwzTile<T, D> G;
  constexpr int KS = D / 16;       // 16-deep steps over the head dim
  constexpr int DT = D / 32;       // 32-wide output column blocks
  constexpr int BQ = 32 * kWaves;  // queries per block (one workgroup's block)
  constexpr int BK = 32;           // keys per streamed tile
  // Ring: in a pipelined step tiles t - 1 (output products), t (whose
  // output products come next step) and t + 1 (score products) are in use
  // and tiles t + 2 .. t + 6 are in flight.
  constexpr int NST = 8;
  constexpr int kTile = G::kElems * (int)sizeof(T);
  constexpr int kStage = 4 * kTile;  // K, V, ddK, ddV
  // the ring, then per wave a dQ2 and a ddO tile staged for row-wise stores
  __shared__ __attribute__((aligned(1024))) char s_kv[NST * kStage + kWaves * 2 * kTile];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int n = lane & 31, g = lane >> 5;
  const int nqb = (p.nq + BQ - 1) / BQ;
  const int npr = CAUSAL ? (nqb + 1) / 2 : nqb;  // items per (batch, head) pair
  const int ngrid = (int)gridDim.x;
  const int w = (int)blockIdx.x;
  Q32Walk walk{ngrid % 8 == 0 ? (w % 8) * (ngrid / 8) + w / 8 : w, 0};
  if (walk.item >= nitems) return;
  const long rs = (long)p.heads * D;      // query-side row stride
  const long rsk = (long)p.kv_heads * D;  // key-side row stride
  const float scale = p.scale;

  // Wave w streams key-side tensor w (K, V, ddK, ddV) into the ring.
  const T* gsrc = wave == 0 ? p.k : wave == 1 ? p.v : wave == 2 ? p.ddk : p.ddv;
  const uint32_t row_bytes = (uint32_t)(rsk * (long)sizeof(T));
  const uint32_t row_bytes_q = (uint32_t)(rs * (long)sizeof(T));
  TileDma<T, D> dma, part;
  dma.init(row_bytes, BK, lane);
  // A ragged key tail can only be a block's last streamed tile; its loads
  // repeat row nk - 1 for the missing rows.
  part.init(row_bytes, p.nk % BK != 0 ? p.nk % BK : BK, lane);
  const uint32_t lds_kv = uni(lds_base_u32(s_kv));
  const uint32_t lds_wave = uni(lds_kv + wave * kTile);
  const uint32_t lds_out = uni(lds_kv + NST * kStage + wave * 2 * kTile);
  const unsigned long gstep = (unsigned long)BK * (unsigned long)row_bytes;

  // One block: its coordinates, streamed tiles and masks.
  struct Blk {
    long qbase, sbase, roff;
    const T* g0;   // this wave's first key-side tile
    int q0, qi, nkt, nfull, rag, klb;
    bool qvalid, one_key;
  };
  auto block_of = [&](Q32Walk it) {
    Blk k;
    const int bh = it.item / npr, r = it.item % npr;
    const int rank = CAUSAL && it.half ? nqb - 1 - r : r;
    const int qb = CAUSAL ? nqb - 1 - rank : rank;  // causal: rank 0 is the last block
    const int b = bh / p.heads, h = bh % p.heads;
    const int hk = h / (p.heads / p.kv_heads);
    k.qbase = ((long)b * p.nq * p.heads + h) * D;
    k.sbase = (long)bh * p.nq;
    k.g0 = gsrc + ((long)b * p.nk * p.kv_heads + hk) * D;
    k.q0 = qb * BQ + wave * 32;
    k.qi = k.q0 + n;
    k.qvalid = k.qi < p.nq;
    k.roff = k.qbase + (long)min(k.qi, p.nq - 1) * rs;
    // Keys [0, kend) are visible to some query of the block. Every wave
    // sweeps all of them (the sweep's barriers and LDS DMAs are shared); a
    // wave whose queries see none of a tile's keys masks all of its pairs.
    int kend = p.nk;
    if (CAUSAL) kend = min(kend, qb * BQ + BQ + p.coff);
    k.nkt = uni(kend > 0 ? (kend + BK - 1) / BK : 0);
    k.rag = uni(p.nk % BK != 0 && k.nkt == (p.nk + BK - 1) / BK ? k.nkt - 1 : -1);
    // Full tiles [0, nfull) are visible to every query of the block and
    // inside nk; the element-wise step of a later tile masks keys past the
    // lane's last visible key (klb, less 4 g: the key of accumulator register
    // r is 8 (r / 4) + 4 g + r % 4 of its tile).
    int full = p.nk / BK;
    if (CAUSAL) full = min(full, max(0, qb * BQ + p.coff + 1) / BK);
    k.nfull = uni(min(full, k.nkt));
    k.klb = min(p.nk - 1, CAUSAL ? k.qi + p.coff : p.nk - 1) - 4 * g;
    k.one_key = (CAUSAL ? min(p.nk, k.qi + p.coff + 1) : p.nk) == 1;
    return k;
  };
  // The item after `it` in this workgroup's list.
  auto next_of = [&](Q32Walk it) {
    if (CAUSAL && it.half == 0 && 2 * (it.item % npr) + 1 != nqb) return Q32Walk{it.item, 1};
    return Q32Walk{it.item + ngrid, 0};
  };
  // Tile j of block k into ring stage (t0 + j) mod 8.
  auto issue_tile = [&](const Blk& k, uint32_t t0, int j) {
    const uint32_t dst = lds_wave + (((t0 + (uint32_t)j) & (NST - 1)) * (uint32_t)kStage);
    const T* src = k.g0 + (long)j * BK * rsk;
    if (j == k.rag)
      part.issue(dst, src);
    else
      dma.issue(dst, src);
  };
  // The query side of a block (Q, ddQ, dO, O: B operands of the score
  // products, and O for D_i = <O_i, dO_i> and the epilogue) is staged in
  // LDS: this wave's 32 rows of tensor j go to its own slice of ring stage
  // t0 + 1 + j, which tiles 1 .. 4 of the block take over once the rows have
  // been read back. Loaded row by row (eight 128-byte rows per instruction),
  // the rows cost a quarter of the cache-line accesses of loads in the
  // operand layout (32 rows per instruction), and the loads go out while the
  // previous block's results are formed. Rows past the last query repeat
  // row nq - 1: their results are never stored, and a matrix product column
  // or row sum of one query never mixes in another's, so finite values are
  // all they need.
  auto qstage = [&](uint32_t t0, int j) {
    return lds_wave + ((t0 + 1u + (uint32_t)j) & (NST - 1)) * (uint32_t)kStage;
  };
  auto issue_query_side = [&](const Blk& k, uint32_t t0, int ln) {
    const int q0c = min(k.q0, p.nq - 1);
    TileDma<T, D> qd;
    qd.init(row_bytes_q, p.nq - q0c, ln);
    const long off = k.qbase + (long)q0c * rs;
    qd.issue(qstage(t0, 0), uni((const void*)(p.q + off)));
    qd.issue(qstage(t0, 1), uni((const void*)(p.ddq + off)));
    qd.issue(qstage(t0, 2), uni((const void*)(p.dout + off)));
    qd.issue(qstage(t0, 3), uni((const void*)(p.o + off)));
  };
  V8<T> qf[KS], ddqf[KS], dof[KS], of[KS];
  float lse;

  // The first block's first tile and query side.
  Blk cur = block_of(walk);
  uint32_t t0 = 0;  // ring tile of the block's first key tile, mod 8
  if (cur.nkt > 0) issue_tile(cur, t0, 0);
  issue_query_side(cur, t0, lane);
  lse = p.lse[cur.sbase + min(cur.qi, p.nq - 1)];
  asm volatile("s_waitcnt vmcnt(0)" : "+v"(lse)::"memory");

  while (true) {
    // The lane's coordinates, opaque once per block: addresses built from
    // them are rebuilt per block instead of being hoisted out of the loop,
    // where they would stay alive across the sweep (whose clobbers leave the
    // compiler 67 vector registers for everything alive across it).
    int lane_b = lane;
    asm volatile("" : "+v"(n), "+v"(g), "+v"(lane_b));
    // The sweep's LDS read offsets and its DMAs' per-lane source offsets,
    // likewise rebuilt per block. The transposed reads' second address is
    // the first with bit 4 flipped (SwzFrags::trf); ring stages are 32-byte
    // aligned, so the flip can be applied to the per-lane offset.
    SwzFrags<T, D> fr;
    fr.init(lane_b);
    dma.init(row_bytes, BK, lane_b);
    part.init(row_bytes, p.nk % BK != 0 ? p.nk % BK : BK, lane_b);
    const uint32_t ta0 = fr.tr[0], ta1 = fr.tr[1], tb0 = fr.tr[0] ^ 16u, tb1 = fr.tr[1] ^ 16u;

    // The staged query side, in the operand layout (lane (n, g): row n,
    // columns 16 ks + 8 g .. +7). O is also copied, in the same layout, to
    // this wave's ddO staging tile, where it stays through the sweep for the
    // epilogue (kept in registers instead, its 16 would not fit beside the
    // sweep's operands).
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qf[ks] = fr.rowf(qstage(t0, 0), 0, ks);
      ddqf[ks] = fr.rowf(qstage(t0, 1), 0, ks);
      dof[ks] = fr.rowf(qstage(t0, 2), 0, ks);
      of[ks] = fr.rowf(qstage(t0, 3), 0, ks);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      *reinterpret_cast<__attribute__((address_space(3))) V8<T>*>((uintptr_t)(lds_out + kTile + fr.row[ks])) = of[ks];

    float dpart = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) dpart = dot8<T>(of[ks], dof[ks], dpart);
    if constexpr (PRE) {
      // scale is a power of two: Q and ddQ carry it exactly, so S and
      // ddS = ddQ K^T + Q ddK^T come out of the matrix products already scaled
      // (bit-identical to scaling them afterwards) and the element-wise step
      // skips one multiply.
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          qf[ks][e] = (T)((float)qf[ks][e] * scale);
          ddqf[ks][e] = (T)((float)ddqf[ks][e] * scale);
        }
    }
    const float c2 = PRE ? kLog2e : scale * kLog2e;
    const float Di = xgroup_sum(dpart);
    const float nD = -Di;
    const float nL2 = -lse * kLog2e;
    // Every read of the staged rows has returned before tiles 1 .. 4 are
    // issued into their stages (the empty statement makes the compiler wait
    // for them here).
    asm volatile("" ::"v"(qf[0]), "v"(qf[1]), "v"(qf[2]), "v"(qf[3]), "v"(ddqf[0]), "v"(ddqf[1]), "v"(ddqf[2]),
                 "v"(ddqf[3]), "v"(dof[0]), "v"(dof[1]), "v"(dof[2]), "v"(dof[3]), "v"(of[0]), "v"(of[1]), "v"(of[2]),
                 "v"(of[3]), "v"(nD), "v"(nL2)
                 : "memory");
#pragma unroll
    for (int j = 1; j < NST - 3; ++j)
      if (j < cur.nkt) issue_tile(cur, t0, j);

    f32x16 acc_a[DT], acc_s[DT], acc_p[DT], acc_o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc_a[dt] = acc_s[dt] = acc_p[dt] = acc_o[dt] = zero16();
    float dd_acc = 0.f;   // dD = sum P ddS over this lane's keys
    // every row of ddm: the same sum over P ddS rounded to T, as the ddO
    // products take it (a matrix product with a ones operand)
    f32x16 ddm = zero16();
    const V8<T> ones = ones8<T>();
    float xs_acc = 0.f;   // sum X over this lane's keys
    float pu_acc = 0.f;   // sum P u over this lane's keys

    if (cur.nkt > 0) {
      // the sweep's operands in ring-tile numbers (gen_q32_loop.py)
      const int issued = min(cur.nkt, NST - 3);
      const uint32_t u_t0 = uni(t0);
      const uint32_t u_nkt = uni(t0 + (uint32_t)cur.nkt), u_nfull = uni(t0 + (uint32_t)cur.nfull);
      const uint32_t u_rag = cur.rag >= 0 ? uni(t0 + (uint32_t)cur.rag) : 0xffffffffu;
      const uint32_t u_hi = uni(t0 + (uint32_t)issued - 1u);
      const int klb = cur.klb + 32 * (int)t0;
      const void* gnext = uni((const void*)(cur.g0 + (long)issued * BK * rsk));
#define FHOG_Q32_ARGS(LOOP)                                                                                 \
  asm volatile(LOOP                                                                                         \
               : [aa0] "+a"(acc_a[0]), [aa1] "+a"(acc_a[1]), [as0] "+a"(acc_s[0]), [as1] "+a"(acc_s[1]),   \
                 [ap0] "+a"(acc_p[0]), [ap1] "+a"(acc_p[1]), [ao0] "+a"(acc_o[0]), [ao1] "+a"(acc_o[1]),   \
                 [dd] "+v"(dd_acc), [ddm] "+a"(ddm), [xs] "+v"(xs_acc), [pu] "+v"(pu_acc)                  \
               : [q0] "a"(qf[0]), [q1] "a"(qf[1]), [q2] "a"(qf[2]), [q3] "a"(qf[3]), [dq0] "a"(ddqf[0]),   \
                 [dq1] "a"(ddqf[1]), [dq2] "a"(ddqf[2]), [dq3] "a"(ddqf[3]), [do0] "a"(dof[0]),            \
                 [do1] "a"(dof[1]), [do2] "a"(dof[2]), [do3] "a"(dof[3]), [nl2] "v"(nL2), [nd] "v"(nD),     \
                 [ones] "v"(ones),                                                                         \
                 [ro0] "v"(fr.row[0]), [ro1] "v"(fr.row[1]), [ro2] "v"(fr.row[2]), [ro3] "v"(fr.row[3]),   \
                 [ta0] "v"(ta0), [ta1] "v"(ta1), [tb0] "v"(tb0), [tb1] "v"(tb1), [vo0] "v"(dma.voff[0]),   \
                 [vo1] "v"(dma.voff[1]), [vo2] "v"(dma.voff[2]), [vo3] "v"(dma.voff[3]),                   \
                 [vp0] "v"(part.voff[0]), [vp1] "v"(part.voff[1]), [vp2] "v"(part.voff[2]),                \
                 [vp3] "v"(part.voff[3]), [klb] "v"(klb), [gptr] "s"(gnext), [gstep] "s"(gstep),           \
                 [hi0] "s"(u_hi), [t0] "s"(u_t0), [ldskv] "s"(lds_kv), [ldsw] "s"(lds_wave),               \
                 [nkt] "s"(u_nkt), [nfull] "s"(u_nfull), [rag] "s"(u_rag), [c2] "s"(c2), [scl] "s"(scale)  \
               : FHOG_Q32_CLOBBERS)
      if constexpr (std::is_same_v<T, __bf16> && PRE)
        FHOG_Q32_ARGS(FHOG_Q32_LOOP_BF16_PRE);
      else if constexpr (std::is_same_v<T, __bf16>)
        FHOG_Q32_ARGS(FHOG_Q32_LOOP_BF16);
      else
        FHOG_Q32_ARGS(FHOG_Q32_LOOP_F16);
#undef FHOG_Q32_ARGS
    }

    // The next block's first tile and query side go out first, into the
    // stages after the ones this block used last (a wave can still be
    // reading this block's last three tiles, never an older one: every wave
    // has passed the barrier before them); then this block's results are
    // formed while they land. The block is selected unconditionally (the
    // last one again after the last block) so that the old block's values do
    // not stay alive across the next sweep.
    const Blk done = cur;
    const Q32Walk nw = next_of(walk);
    const bool more = nw.item < nitems;
    if (more) walk = nw;
    cur = block_of(walk);
    t0 = (t0 + (uint32_t)done.nkt) & (NST - 1);
    if (more) {
      if (cur.nkt > 0) issue_tile(cur, t0, 0);
      issue_query_side(cur, t0, lane_b);
    }
    lse = p.lse[cur.sbase + min(cur.qi, p.nq - 1)];

    const float dD = xgroup_sum(dd_acc);
    const float dDo = ddm[0];
    const float c = xgroup_sum(xs_acc) - dD * xgroup_sum(pu_acc);
    const float Bi = c - Di * dD;
    // O in the accumulator layout (register 4 a + i of column block dt holds
    // column 32 dt + 8 a + 4 g + i), read before ddO overwrites it.
    V4<T> oe[DT][4];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const uint32_t off = 2u * (uint32_t)(n * D + 8 * phys_chunk(n, 4 * dt + a) + 4 * g);
        oe[dt][a] = *reinterpret_cast<const __attribute__((address_space(3))) V4<T>*>((uintptr_t)(lds_out + kTile + off));
      }
    asm volatile("" ::"v"(oe[0][0]), "v"(oe[0][1]), "v"(oe[0][2]), "v"(oe[0][3]), "v"(oe[1][0]), "v"(oe[1][1]),
                 "v"(oe[1][2]), "v"(oe[1][3]) : "memory");
    // dQ2 and ddO into this wave's staging tiles (rows swizzled by row mod 8,
    // so that neither these writes nor the row reads below conflict), one
    // column block at a time: accumulator register 4 a + i of column block dt
    // holds column 32 dt + 8 a + 4 g + i of this lane's query.
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const V4<T> ov = oe[dt][a];
        f32x4 x, y;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * a + i;
          x[i] = done.one_key ? 0.f : scale * (acc_a[dt][r] - dD * acc_s[dt][r] - c * acc_p[dt][r]);
          y[i] = acc_o[dt][r] - dDo * (float)ov[i];
        }
        const uint32_t off = (uint32_t)(n * 128 + 16 * phys_chunk<kSwzRows>(n, 4 * dt + a) + 8 * g);
        *reinterpret_cast<__attribute__((address_space(3))) V4<T>*>((uintptr_t)(lds_out + off)) = cvt4<T>(x);
        *reinterpret_cast<__attribute__((address_space(3))) V4<T>*>((uintptr_t)(lds_out + kTile + off)) = cvt4<T>(y);
      }
      // the next column block's accumulators are read after these writes,
      // so that only one block's 64 are held in vector registers at a time
      if (dt + 1 < DT)
        asm volatile("" : "+a"(acc_a[dt + 1]), "+a"(acc_s[dt + 1]), "+a"(acc_p[dt + 1]), "+a"(acc_o[dt + 1])::"memory");
    }
    // The next block's query side has landed (nothing but it, its first
    // tile and the logsumexp is in flight), before any store is issued.
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(lse)::"memory");
    if (done.qvalid && g == 0) {
      p.delta[done.sbase + done.qi] = Di;
      p.ddelta[done.sbase + done.qi] = dD;
      p.bstat[done.sbase + done.qi] = Bi;
    }
    // The staged rows, eight per instruction: lane l takes 16 bytes of row
    // 8 i + l / 8 (chunk position l % 8, holding logical chunk
    // (l % 8) ^ (row mod 8)).
    V8<T> rows[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        rows[t][i] = *reinterpret_cast<const __attribute__((address_space(3))) V8<T>*>(
            (uintptr_t)(lds_out + t * kTile + 1024 * i + 16 * lane_b));
    const int lc = (lane_b & 7) ^ ((lane_b >> 3) & 7);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      T* dst = (t == 0 ? p.dq2 : p.ddo) + done.qbase + 8 * lc;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 8 * i + (lane_b >> 3);
        if (done.q0 + r < p.nq) *reinterpret_cast<V8<T>*>(dst + (long)(done.q0 + r) * rs) = rows[t][i];
      }
    }
    if (!more) break;
  }
}

}  // namespace

template <typename T, bool CAUSAL>
hipError_t launch_bwdbwd_stage1_q32(const BwdBwdParams<T>& p, hipStream_t stream) {
  const int nqb = (p.nq + 32 * kWaves - 1) / (32 * kWaves);
  const int nitems = p.batch * p.heads * (CAUSAL ? (nqb + 1) / 2 : nqb);
  const int resident = resident_workgroups(1);
  const dim3 grid(resident > 0 && resident < nitems ? resident : nitems);
  int e2;
  if (std::is_same_v<T, __bf16> && std::frexp(p.scale, &e2) == 0.5f)  // scale = 2^(e2 - 1)
    hipLaunchKernelGGL((bwdbwd_q32_kernel<T, CAUSAL, std::is_same_v<T, __bf16>>), grid, dim3(kThreads), 0, stream, p,
                       nitems);
  else
    hipLaunchKernelGGL((bwdbwd_q32_kernel<T, CAUSAL, false>), grid, dim3(kThreads), 0, stream, p, nitems);
  return hipGetLastError();
}

#define FHOG_INST(T, C) template hipError_t launch_bwdbwd_stage1_q32<T, C>(const BwdBwdParams<T>&, hipStream_t);
FHOG_INST(__bf16, true)
FHOG_INST(__bf16, false)
FHOG_INST(_Float16, true)
FHOG_INST(_Float16, false)
#undef FHOG_INST

}  // namespace fhog
