// Key-tiled kernel of the first-order attention backward (dK and dV) for
// 2-byte types at D = 64: 64 keys per wave at one wave per SIMD, the query
// sweep generated as inline assembly (gen_bwd_k64_loop.py ->
// fhog_bwd_k64_loop.inc). It computes what bwd_k_kernel (fhog_bwd.hip)
// computes, replacing part of the cuDNN backward the reference calls through
// flash_hog/jax/_attention_impl.py:242-261 (equations of
// flash_hog/_jax_refs/jax_impl.py:142-191):
//   P = exp2(S' c2) with S' = S - L / scale, u = dP - D,
//   dK = scale sum_q (P u) Q,  dV = sum_q P dO,
// a pair (query, key) entering iff query >= key - coff (causal) and
// query < nq.
//
// Why this shape. bwd_k_kernel holds 32 keys per wave at two waves per SIMD
// (184 registers) and keeps the matrix pipe about 30 % busy: each wave forms
// a tile's scores, then its element-wise step, then its output products, and
// the two waves of a SIMD hide little of each other's dependency chains. Here
// one wave holds 64 keys (two halves of 32 with their own resident K and V,
// score tiles and dK/dV accumulators: 192 AGPRs and 185 pinned VGPRs), so
// every query-side LDS fragment it reads serves twice the pairs, and the
// generated sweep interleaves the output products of tile t - 1, the
// element-wise step of tile t and the score products of tile t + 1.
//
// A workgroup owns 256 keys of one (batch, key/value head) pair and streams
// 32-query tiles of Q (wave 0), dO (wave 1) and the tiles' row statistics L
// and D (wave 2) through an 8-stage LDS ring of 16 KiB stages: tile i sits in
// stage i mod 8, tile i + 6 is loaded at step i into the stage tile i - 2
// left. Grouped-query heads are visited query tile by query tile, the heads
// of the group in turn, as in bwd_k_kernel. Causal key blocks are taken in
// mirror pairs (block r, then block nkb - 1 - r) when the grid outnumbers
// the CUs.
#include <cmath>
#include <cstdint>

#include "fhog_bwd_k64_loop.inc"
#include "fhog_device.h"
#include "fhog_params.h"

namespace fhog {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

__device__ __forceinline__ uint32_t uni(uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); }
__device__ __forceinline__ float uni(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}
__device__ __forceinline__ uint64_t uni(uint64_t x) {
  return (uint64_t)uni((uint32_t)x) | ((uint64_t)uni((uint32_t)(x >> 32)) << 32);
}

template <typename T, bool CAUSAL>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
bwd_k64_kernel(BwdParams<T> p, int pairs, int chunk) {
  constexpr int D = 64;
  typedef SwzTile<T, D> G;
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  constexpr int KW = 64;            // keys per wave
  constexpr int BKB = KW * kWaves;  // keys per workgroup
  constexpr int BQ = 32;            // queries per streamed tile
  constexpr int NST = 8;
  constexpr int kTile = G::kElems * (int)sizeof(T);
  constexpr int kStage = 16384;                  // Q, dO, statistics
  constexpr int kStOff = FHOG_BK64_STAT_OFF;     // L at kStOff + 4 lane, D at + 256
  static_assert(kTile == 4096 && kStOff == 2 * kTile, "the generated sweep assumes 4 KiB tiles");
  __shared__ __attribute__((aligned(1024))) char s_q[NST * kStage];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 31, g = lane >> 5;
  const int nbh = p.batch * p.kv_heads;
  const int nkb = (p.nk + BKB - 1) / BKB;
  const GridSlot slot = grid_slot(blockIdx.x, nbh, pairs ? (nkb + 1) / 2 : nkb, chunk);
  const int bh = slot.pair;
  const BlockPair bp = block_pair(slot.rank, nkb, pairs);
  const float scale = p.scale;

  for (int blk = 0; blk < bp.count; ++blk) {
    const int kb = blk == 0 ? bp.first : bp.second;
    if (blk > 0) __syncthreads();  // every wave is done with the previous block's ring
    const int b = bh / p.kv_heads, hk = bh % p.kv_heads;
    const int grp = p.heads / p.kv_heads;
    const long rs = (long)p.heads * D;
    const long rsk = (long)p.kv_heads * D;
    const long qbase = ((long)b * p.nq * p.heads + (long)hk * grp) * D;
    const long kbase = ((long)b * p.nk * p.kv_heads + hk) * D;
    const long sbase = ((long)b * p.heads + (long)hk * grp) * p.nq;
    const int k0 = kb * BKB + wave * KW;  // half h holds keys k0 + 32 h + n
    const int nqt = (p.nq + BQ - 1) / BQ;
    const int qt_begin = CAUSAL ? max(0, kb * BKB - p.coff) / BQ : 0;
    const int ntot = __builtin_amdgcn_readfirstlane(max(0, nqt - qt_begin) * grp);

    f32x16 acc_k[2][DT], acc_v[2][DT];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc_k[h][dt] = acc_v[h][dt] = zero16();

    if (ntot > 0) {
      SwzFrags<T, D> fr;
      fr.init(lane);
      const uint32_t ta0 = fr.tr[0], ta1 = fr.tr[1], tb0 = fr.tr[0] ^ 16u, tb1 = fr.tr[1] ^ 16u;
      const uint32_t lds_q = lds_base_u32(s_q);
      const bool tens = wave < 2, stw = wave == 2;

      // Streams and their per-lane offsets. The ragged last query tile (if
      // nq % 32 != 0) repeats row (or statistic) nq - 1 for its missing rows.
      const int rag_rows = p.nq - (nqt - 1) * BQ;
      const uint32_t ragq0 = rag_rows < BQ ? (uint32_t)((nqt - 1) * BQ) : 0xffffffffu;
      const uint32_t row_bytes = (uint32_t)(rs * (long)sizeof(T));
      TileDma<T, D> dma, part;
      dma.init(row_bytes, BQ, lane);
      part.init(row_bytes, rag_rows, lane);
      uint32_t vo[4], vp[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        vo[j] = tens ? dma.voff[j] : 4u * (uint32_t)n;
        vp[j] = tens ? part.voff[j] : 4u * (uint32_t)min(n, rag_rows - 1);
      }
      const T* tsrc = wave == 0 ? p.q : p.dout;
      // wave 2 loads L and D twice per tile (four loads, as the other streams)
      const float* stat[4] = {p.lse, p.delta, p.lse, p.delta};
      const char* ptr[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        ptr[j] = tens ? reinterpret_cast<const char*>(tsrc + qbase + (long)qt_begin * BQ * rs)
                      : reinterpret_cast<const char*>(stat[j] + sbase + (long)qt_begin * BQ);
      // the next head of the group, and from the last head to the first head
      // of the next query tile
      const long stepa = tens ? (long)D * (long)sizeof(T) : 4L * p.nq;
      const long stepb = tens ? ((long)BQ * rs - (long)(grp - 1) * D) * (long)sizeof(T)
                              : 4L * (BQ - (long)(grp - 1) * p.nq);
      const uint32_t ldsw = wave == 0 ? 0u : wave == 1 ? (uint32_t)kTile : stw ? (uint32_t)kStOff
                                                                                : (uint32_t)FHOG_BK64_WAVE_NONE;

      // DMA cursor: the next tile to issue is (query tile dq0 / 32, head dgi)
      int dgi = 0;
      uint32_t dq0 = (uint32_t)(qt_begin * BQ);
      int hi = -1;
      auto issue_tile = [&]() {
        ++hi;
        const uint32_t dst = lds_q + (uint32_t)((hi % NST) * kStage) + ldsw;
        const uint32_t* off = dq0 == ragq0 ? vp : vo;
        if (tens) {
          dma16s(ptr[0], off[0], dst);
#pragma unroll
          for (int j = 1; j < 4; ++j) dma16s_next(ptr[0], off[j], dst + 1024u * j);
        } else if (stw) {
#pragma unroll
          for (int j = 0; j < 4; ++j) dma4s(ptr[j], off[j], dst + 256u * j);
        }
        const bool wrap = ++dgi == grp;
        if (wrap) {
          dgi = 0;
          dq0 += BQ;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) ptr[j] += wrap ? stepb : stepa;
      };
      // Tiles 0 and 1 first, then the key-side loads, then tiles 2 .. 4 once
      // those have been used (the compiler's waits for its loads also wait
      // for every DMA issued before them; the sweep's waits count DMAs and
      // are only made stricter by older loads).
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if (i < ntot) issue_tile();

      // Key-side operands (B of the score products). A lane past the last key
      // loads the last key: its results are never stored, and a column of a
      // matrix product never mixes in another key's.
      V8<T> kf[2][KS], vf[2][KS];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const long koff = kbase + (long)min(k0 + 32 * h + n, p.nk - 1) * rsk;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const long off = koff + 16 * ks + 8 * g;
          kf[h][ks] = *reinterpret_cast<const V8<T>*>(p.k + off);
          vf[h][ks] = *reinterpret_cast<const V8<T>*>(p.v + off);
        }
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        asm volatile("" ::"v"(kf[0][ks]), "v"(kf[1][ks]), "v"(vf[0][ks]), "v"(vf[1][ks]));
      asm volatile("" ::: "memory");
#pragma unroll
      for (int i = 2; i < NST - 3; ++i)
        if (i < ntot) issue_tile();

      // Constants operand pieces (gen_bwd_k64_loop.py): lanes of half 0 turn
      // L into a = -L / scale and D into b = -D; the other lanes hold zeros.
      const float ca = g ? 0.0f : -1.0f / scale;
      const float cb = g ? 0.0f : -1.0f;
      const uint32_t sta = (uint32_t)(kStOff + 4 * n);
      // selectors (bf16 for both input types): ones at k = {0, 2, 4} (a) or
      // {1, 3, 5} (b), lanes of half 0
      bf16x8 sels, selp;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sels[e] = (__bf16)((g == 0 && e < 6 && e % 2 == 0) ? 1.0f : 0.0f);
        selp[e] = (__bf16)((g == 0 && e < 6 && e % 2 == 1) ? 1.0f : 0.0f);
      }
      const float c2 = scale * kLog2e;

      // Masked steps: those whose tile has rows some key of the workgroup
      // must not see (the causal diagonal, from the first tile to the first
      // one past query kb * 256 + 256 - coff) and the ragged last query
      // tile. A masked step keeps row q0 + 4 g + c of its tile for key half h
      // iff (c - (qfirst_h - 4 g - q0)) < nq - qfirst_h, qfirst_h the first
      // query that sees the lane's key.
      int qlo[2];
      uint32_t qw[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int qfirst = CAUSAL ? k0 + 32 * h + n - p.coff : 0;
        qlo[h] = qfirst - 4 * g;
        qw[h] = (uint32_t)max(0, p.nq - qfirst);
      }
      int lead = 0;
      if (CAUSAL) lead = min(nqt - qt_begin, max(0, (kb * BKB + BKB - p.coff + BQ - 1) / BQ - qt_begin));
      int mlo = __builtin_amdgcn_readfirstlane(lead * grp);
      int mhi = __builtin_amdgcn_readfirstlane(ntot - (rag_rows < BQ ? grp : 0));
      // steady steps (no branches in their DMA) need tile t + 6 to be a full tile
      const int nsd = __builtin_amdgcn_readfirstlane(ntot - (rag_rows < BQ ? grp : 0));
      // Scalar operands: the values are uniform; saying so keeps the
      // compiler from handing an "s" operand a VGPR. The sweep's DMA cursor
      // (last tile issued, its head and query offset, the element-wise
      // step's query offset, the four stream pointers) is bound to the
      // registers the sweep keeps it in.
      const uint32_t u_ldsq = uni(lds_q), u_ldsw = uni(ldsw), u_grp = uni((uint32_t)grp);
      const uint32_t u_ragq0 = uni(ragq0);
      uint32_t r_hi = uni((uint32_t)hi), r_dgi = uni((uint32_t)dgi), r_dq0 = uni(dq0);
      uint32_t r_eq0 = uni((uint32_t)(qt_begin * BQ));
      const float u_c2 = uni(c2);
      const uint64_t u_stepa = uni((uint64_t)stepa), u_stepb = uni((uint64_t)stepb);
      uint64_t r_p0 = uni((uint64_t)(uintptr_t)ptr[0]), r_p1 = uni((uint64_t)(uintptr_t)ptr[1]);
      uint64_t r_p2 = uni((uint64_t)(uintptr_t)ptr[2]), r_p3 = uni((uint64_t)(uintptr_t)ptr[3]);

#define FHOG_BK64_ARGS(LOOP)                                                                                  \
  asm volatile(LOOP                                                                                           \
               : [ak00] "+a"(acc_k[0][0]), [ak01] "+a"(acc_k[0][1]), [ak10] "+a"(acc_k[1][0]),             \
                 [ak11] "+a"(acc_k[1][1]), [av00] "+a"(acc_v[0][0]), [av01] "+a"(acc_v[0][1]),             \
                 [av10] "+a"(acc_v[1][0]), [av11] "+a"(acc_v[1][1]),                                       \
                 FHOG_BK64_BOUND(r_hi, r_dgi, r_dq0, r_eq0, r_p0, r_p1, r_p2, r_p3)                          \
               : [k00] "a"(kf[0][0]), [k01] "a"(kf[0][1]), [k02] "a"(kf[0][2]), [k03] "a"(kf[0][3]),       \
                 [k10] "a"(kf[1][0]), [k11] "a"(kf[1][1]), [k12] "a"(kf[1][2]), [k13] "a"(kf[1][3]),       \
                 [v00] "a"(vf[0][0]), [v01] "a"(vf[0][1]), [v02] "a"(vf[0][2]), [v03] "a"(vf[0][3]),       \
                 [v10] "a"(vf[1][0]), [v11] "a"(vf[1][1]), [v12] "a"(vf[1][2]), [v13] "a"(vf[1][3]),       \
                 [sels] "v"(sels), [selp] "v"(selp), [ro0] "v"(fr.row[0]), [ro1] "v"(fr.row[1]),           \
                 [ro2] "v"(fr.row[2]), [ro3] "v"(fr.row[3]), [ta0] "v"(ta0), [ta1] "v"(ta1), [tb0] "v"(tb0), \
                 [tb1] "v"(tb1), [vo0] "v"(vo[0]), [vo1] "v"(vo[1]), [vo2] "v"(vo[2]), [vo3] "v"(vo[3]),    \
                 [vp0] "v"(vp[0]), [vp1] "v"(vp[1]), [vp2] "v"(vp[2]), [vp3] "v"(vp[3]), [sta] "v"(sta),    \
                 [qlo0] "v"(qlo[0]), [qlo1] "v"(qlo[1]), [qw0] "v"(qw[0]), [qw1] "v"(qw[1]), [ca] "v"(ca),  \
                 [cb] "v"(cb), [ldsq] "s"(u_ldsq), [ldsw] "s"(u_ldsw), [ntot] "s"(ntot), [grp] "s"(u_grp),  \
                 [mlo] "s"(mlo), [mhi] "s"(mhi), [nsd] "s"(nsd), [ragq0] "s"(u_ragq0), [c2] "s"(u_c2),      \
                 [stepa] "s"(u_stepa), [stepb] "s"(u_stepb)                                                \
               : FHOG_BK64_CLOBBERS)
      if constexpr (std::is_same_v<T, __bf16>)
        FHOG_BK64_ARGS(FHOG_BK64_LOOP_BF16);
      else
        FHOG_BK64_ARGS(FHOG_BK64_LOOP_F16);
#undef FHOG_BK64_ARGS
    }

    // dK and dV go to HBM as whole 128-byte rows, eight rows per store
    // instruction, through a 16 KiB staging area per wave (in the operand
    // layout each store would touch 32 rows). Wave w stages in the ring stage
    // of tile ntot - 8 + w: every wave has passed the barrier that waited for
    // tile ntot - 1, so no wave reads a tile older than ntot - 2 any more, and
    // no DMA is in flight. Rows are swizzled by key mod 8 so that neither the
    // writes nor the row reads conflict.
    // (The lane index is made opaque here, so that the addresses below are
    // formed after the sweep instead of being hoisted out of the block loop
    // and kept alive across the sweep, whose clobbers leave the compiler 71
    // vector registers.)
    int le = lane;
    asm volatile("" : "+v"(le));
    const int ne = le & 31, ge = le >> 5;
    const uint32_t stg = lds_base_u32(s_q) + (uint32_t)(((uint32_t)(ntot + wave) & (NST - 1)) * kStage);
    // accumulator register 4 a + i of column block dt holds column
    // 32 dt + 8 a + 4 g + i of this lane's key (row 32 h + n of the stage)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = 32 * h + ne;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          f32x4 x, y;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            x[i] = acc_k[h][dt][4 * a + i] * scale;
            y[i] = acc_v[h][dt][4 * a + i];
          }
          const uint32_t off = (uint32_t)(r * 128 + 16 * phys_chunk<kSwzRows>(r, 4 * dt + a) + 8 * ge);
          *reinterpret_cast<__attribute__((address_space(3))) V4<T>*>((uintptr_t)(stg + off)) = cvt4<T>(x);
          *reinterpret_cast<__attribute__((address_space(3))) V4<T>*>((uintptr_t)(stg + 8192u + off)) = cvt4<T>(y);
        }
    }
    // lane l takes 16 bytes of row 8 i + l / 8 (chunk position l % 8, holding
    // logical chunk (l % 8) ^ (row mod 8))
    const int lc = (le & 7) ^ ((le >> 3) & 7);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      V8<T> rows[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        rows[i] = *reinterpret_cast<const __attribute__((address_space(3))) V8<T>*>(
            (uintptr_t)(stg + 8192u * t + 1024u * i + 16u * (uint32_t)le));
      T* dst = (t == 0 ? p.dk : p.dv) + kbase + 8 * lc;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int kr = k0 + 8 * i + (le >> 3);
        if (kr < p.nk) *reinterpret_cast<V8<T>*>(dst + (long)kr * rsk) = rows[i];
      }
    }
  }
}

}  // namespace

template <typename T, bool CAUSAL>
hipError_t launch_bwd_k64(const BwdParams<T>& p, hipStream_t stream) {
  const int nkb = (p.nk + 64 * kWaves - 1) / (64 * kWaves);
  const int npairs = p.batch * p.kv_heads;
  const int resident = resident_workgroups(1);
  const int pairs = block_pairing(CAUSAL, nkb, npairs, resident, 1);
  const int nranks = pairs ? (nkb + 1) / 2 : nkb;
  const int chunk = grid_chunk(npairs, nranks, resident);
  hipLaunchKernelGGL((bwd_k64_kernel<T, CAUSAL>), dim3(nranks * npairs), dim3(kThreads), 0, stream, p, pairs,
                     chunk);
  return hipGetLastError();
}

template hipError_t launch_bwd_k64<__bf16, true>(const BwdParams<__bf16>&, hipStream_t);
template hipError_t launch_bwd_k64<__bf16, false>(const BwdParams<__bf16>&, hipStream_t);
template hipError_t launch_bwd_k64<_Float16, true>(const BwdParams<_Float16>&, hipStream_t);
template hipError_t launch_bwd_k64<_Float16, false>(const BwdParams<_Float16>&, hipStream_t);

}  // namespace fhog
