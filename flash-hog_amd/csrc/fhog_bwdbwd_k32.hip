// Stage 2 of the double backward (pass 4: dK2 = dS^T ddQ + dS2^T Q,
// dV2 = ddP^T dO) for bf16 at D = 64: 32 keys per wave at one wave per SIMD,
// the query sweep generated as inline assembly (gen_k32_loop.py ->
// fhog_k32_loop.inc).
//
// A workgroup owns 128 keys of one (batch, key/value head) pair and streams
// 32-query tiles of Q, dO, ddQ (waves 0-2, one tensor each) and the tiles'
// row statistics L, D, dD, B (wave 3) through an 8-stage LDS ring of 16 KiB
// stages: tile i sits in stage i mod 8, tile i + 6 is loaded at step i into
// the stage tile i - 2 left. Grouped-query heads are visited query tile by
// query tile, the heads of the group in turn (the group reduction of
// flash_hog/jax/_pallas_gpu_kernel.py:333-370), as the compiled stage 2 does.
//
// The key-side operands (K, ddK, V, ddV of the lane's key; B of the score
// products) and the dK2/dV2 accumulators stay in AGPRs for the whole sweep.
// The per-query constants that start the score accumulators
// (-L, -dD, -D, -(D dD + B)) enter through one matrix product per chain with
// an operand holding their exact bf16 parts (see gen_k32_loop.py). Element
// math and the pair mask follow the compiled stage 2 (fhog_bwdbwd.hip):
//   P = exp2(S' c2), t = ddS', x = u t + dPa', dS = P u, dS2 = P x, ddP = P t,
// and a pair (query, key) enters iff first_contributing_query <= query < nq.
#include <cmath>
#include <cstdint>

#include "fhog_device.h"
#include "fhog_k32_loop.inc"
#include "fhog_params.h"

namespace fhog {

namespace {

constexpr int kWaves = 4;

__device__ __forceinline__ uint32_t uni(uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); }
__device__ __forceinline__ float uni(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}
__device__ __forceinline__ uint64_t uni(uint64_t x) {
  return (uint64_t)uni((uint32_t)x) | ((uint64_t)uni((uint32_t)(x >> 32)) << 32);
}
constexpr int kThreads = 64 * kWaves;

template <bool CAUSAL, bool PRE>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
bwdbwd_k32_kernel(BwdBwdParams<__bf16> p, int pairs, int chunk) {
  typedef __bf16 T;
  constexpr int D = 64;
  typedef SwzTile<T, D> G;
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  constexpr int BKB = 32 * kWaves;  // keys per workgroup
  constexpr int BQ = 32;            // queries per streamed tile
  constexpr int NST = 8;
  constexpr int kTile = G::kElems * (int)sizeof(T);
  constexpr int kStage = 4 * kTile;  // Q, dO, ddQ, statistics
  constexpr int kStOff = 3 * kTile;  // statistic j at kStOff + 256 j + 4 lane
  static_assert(kTile == 4096, "the generated sweep assumes 4 KiB tiles");
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
  const float inv_scale = 1.0f / scale;

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
    const int k0 = kb * BKB + wave * 32;
    const int kj = k0 + n;
    const bool kvalid = kj < p.nk;
    const int nqt = (p.nq + BQ - 1) / BQ;
    const int qt_begin = CAUSAL ? max(0, kb * BKB - p.coff) / BQ : 0;
    const int ntot = __builtin_amdgcn_readfirstlane(max(0, nqt - qt_begin) * grp);

    f32x16 acc_k[DT], acc_v[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc_k[dt] = acc_v[dt] = zero16();

    if (ntot > 0) {
      SwzFrags<T, D> fr;
      fr.init(lane);
      const uint32_t ta0 = fr.tr[0], ta1 = fr.tr[1], tb0 = fr.tr[0] ^ 16u, tb1 = fr.tr[1] ^ 16u;
      const uint32_t lds_q = lds_base_u32(s_q);
      const bool w3 = wave == 3;

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
        vo[j] = w3 ? 4u * (uint32_t)n : dma.voff[j];
        vp[j] = w3 ? 4u * (uint32_t)min(n, rag_rows - 1) : part.voff[j];
      }
      const T* tsrc = wave == 0 ? p.q : wave == 1 ? p.dout : p.ddq;
      const float* stat[4] = {p.lse, p.delta, p.ddelta, p.bstat};
      // byte pointers of tile (query tile qt_begin, head 0 of the group)
      const char* ptr[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        ptr[j] = w3 ? reinterpret_cast<const char*>(stat[j] + sbase + (long)qt_begin * BQ)
                    : reinterpret_cast<const char*>(tsrc + qbase + (long)qt_begin * BQ * rs);
      // the next head of the group, and from the last head to the first head
      // of the next query tile
      const long stepa = w3 ? 4L * p.nq : (long)D * (long)sizeof(T);
      const long stepb = w3 ? 4L * (BQ - (long)(grp - 1) * p.nq)
                            : ((long)BQ * rs - (long)(grp - 1) * D) * (long)sizeof(T);
      const uint32_t ldsw = w3 ? (uint32_t)kStOff : (uint32_t)(wave * kTile);

      // DMA cursor: the next tile to issue is (query tile dq0 / 32, head dgi)
      int dgi = 0;
      uint32_t dq0 = (uint32_t)(qt_begin * BQ);
      int hi = -1;
      auto issue_tile = [&]() {
        ++hi;
        const uint32_t dst = lds_q + (uint32_t)((hi % NST) * kStage) + ldsw;
        const uint32_t* off = dq0 == ragq0 ? vp : vo;
        if (!w3) {
          dma16s(ptr[0], off[0], dst);
#pragma unroll
          for (int j = 1; j < 4; ++j) dma16s_next(ptr[0], off[j], dst + 1024u * j);
        } else {
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
      const long koff = kbase + (long)min(kj, p.nk - 1) * rsk;
      V8<T> kf[KS], dkf[KS], vf[KS], dvf[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const long off = koff + 16 * ks + 8 * g;
        kf[ks] = *reinterpret_cast<const V8<T>*>(p.k + off);
        dkf[ks] = *reinterpret_cast<const V8<T>*>(p.ddk + off);
        vf[ks] = *reinterpret_cast<const V8<T>*>(p.v + off);
        dvf[ks] = *reinterpret_cast<const V8<T>*>(p.ddv + off);
      }
      if constexpr (PRE) {
        // scale is a power of two: K and ddK carry it exactly, so S and ddS
        // come out of the matrix products already scaled.
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            kf[ks][e] = (T)((float)kf[ks][e] * scale);
            dkf[ks][e] = (T)((float)dkf[ks][e] * scale);
          }
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) asm volatile("" ::"v"(kf[ks]), "v"(dkf[ks]), "v"(vf[ks]), "v"(dvf[ks]));
      asm volatile("" ::: "memory");
#pragma unroll
      for (int i = 2; i < NST - 3; ++i)
        if (i < ntot) issue_tile();

      // Constants operand pieces (gen_k32_loop.py): lane (query m, half h)
      // turns r1 = L (h = 0) or D (h = 1), r2 = dD, r3 = B into
      // a = r1 ca and b = r2 (h ? -r1 : nk2) + r3 cb.
      const float k12 = PRE ? 1.0f : inv_scale;  // -L / scale and -dD / scale when K, ddK lack the scale
      const float ca = g ? -1.0f : -k12;
      const float cb = g ? -1.0f : 0.0f;
      const float cnb = g ? -1.0f : 0.0f;  // x = r1 cnb + knb: -k2 (h = 0) or -D (h = 1)
      const float knb = g ? 0.0f : -k12;
      const uint32_t sta = (uint32_t)(kStOff + 256 * g + 4 * n);
      const uint32_t stb = (uint32_t)(kStOff + 4 * n);
      // selectors: ones at k = 8 h + {0, 2, 4} (a) or 8 h + {1, 3, 5} (b)
      V8<T> sels, seld, selp, sela;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float on_a = (e < 6 && e % 2 == 0) ? 1.0f : 0.0f;
        const float on_b = (e < 6 && e % 2 == 1) ? 1.0f : 0.0f;
        sels[e] = (T)(g == 0 ? on_a : 0.0f);
        seld[e] = (T)(g == 0 ? on_b : 0.0f);
        selp[e] = (T)(g == 1 ? on_a : 0.0f);
        sela[e] = (T)(g == 1 ? on_b : 0.0f);
      }
      const float c2 = PRE ? kLog2e : scale * kLog2e;

      // Masked steps: those whose tile has rows some key of the workgroup
      // must not see (the causal diagonal, from the first tile to the first
      // one past query kb * 128 + 128 - coff), the ragged last query tile,
      // and every step when nk = 1. A masked step keeps row
      // q0 + 4 g + c of its tile iff (c - (qfirst - 4 g - q0)) < nq - qfirst.
      const int qfirst = first_contributing_query(p, kj, CAUSAL);
      const int qlo = qfirst - 4 * g;
      const uint32_t qw = (uint32_t)max(0, p.nq - qfirst);
      int lead = 0;
      if (CAUSAL) lead = min(nqt - qt_begin, max(0, (kb * BKB + BKB - p.coff + BQ - 1) / BQ - qt_begin));
      int mlo = lead * grp;
      int mhi = ntot - (rag_rows < BQ ? grp : 0);
      if (p.nk == 1) mlo = ntot;
      mlo = __builtin_amdgcn_readfirstlane(mlo);
      mhi = __builtin_amdgcn_readfirstlane(mhi);
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
      const float u_c2 = uni(c2), u_scl = uni(scale);
      const uint64_t u_stepa = uni((uint64_t)stepa), u_stepb = uni((uint64_t)stepb);
      uint64_t r_p0 = uni((uint64_t)(uintptr_t)ptr[0]), r_p1 = uni((uint64_t)(uintptr_t)ptr[1]);
      uint64_t r_p2 = uni((uint64_t)(uintptr_t)ptr[2]), r_p3 = uni((uint64_t)(uintptr_t)ptr[3]);

#define FHOG_K32_ARGS(LOOP)                                                                                     \
  asm volatile(LOOP                                                                                             \
               : [ak0] "+a"(acc_k[0]), [ak1] "+a"(acc_k[1]), [av0] "+a"(acc_v[0]), [av1] "+a"(acc_v[1]),     \
                 FHOG_K32_BOUND(r_hi, r_dgi, r_dq0, r_eq0, r_p0, r_p1, r_p2, r_p3)                             \
               : [k0] "a"(kf[0]), [k1] "a"(kf[1]), [k2] "a"(kf[2]), [k3] "a"(kf[3]), [dk0] "a"(dkf[0]),        \
                 [dk1] "a"(dkf[1]), [dk2] "a"(dkf[2]), [dk3] "a"(dkf[3]), [v0] "a"(vf[0]), [v1] "a"(vf[1]),   \
                 [v2] "a"(vf[2]), [v3] "a"(vf[3]), [dv0] "a"(dvf[0]), [dv1] "a"(dvf[1]), [dv2] "a"(dvf[2]),   \
                 [dv3] "a"(dvf[3]), [sels] "v"(sels), [seld] "v"(seld), [selp] "v"(selp), [sela] "v"(sela),  \
                 [ro0] "v"(fr.row[0]), [ro1] "v"(fr.row[1]), [ro2] "v"(fr.row[2]), [ro3] "v"(fr.row[3]),      \
                 [ta0] "v"(ta0), [ta1] "v"(ta1), [tb0] "v"(tb0), [tb1] "v"(tb1), [vo0] "v"(vo[0]),             \
                 [vo1] "v"(vo[1]), [vo2] "v"(vo[2]), [vo3] "v"(vo[3]), [vp0] "v"(vp[0]), [vp1] "v"(vp[1]),     \
                 [vp2] "v"(vp[2]), [vp3] "v"(vp[3]), [sta] "v"(sta), [stb] "v"(stb), [qlo] "v"(qlo),          \
                 [qw] "v"(qw), [ca] "v"(ca), [cb] "v"(cb), [cnb] "v"(cnb), [knb] "v"(knb),                     \
                 [ldsq] "s"(u_ldsq), [ldsw] "s"(u_ldsw), [ntot] "s"(ntot), [grp] "s"(u_grp), [mlo] "s"(mlo),   \
                 [mhi] "s"(mhi), [nsd] "s"(nsd), [ragq0] "s"(u_ragq0), [c2] "s"(u_c2), [scl] "s"(u_scl),       \
                 [stepa] "s"(u_stepa), [stepb] "s"(u_stepb)                                                    \
               : FHOG_K32_CLOBBERS)
      if constexpr (PRE)
        FHOG_K32_ARGS(FHOG_K32_LOOP_BF16_PRE);
      else
        FHOG_K32_ARGS(FHOG_K32_LOOP_BF16);
#undef FHOG_K32_ARGS
    }

    if (kvalid) {
      T* dk2 = p.dk2 + kbase + (long)kj * rsk;
      T* dv2 = p.dv2 + kbase + (long)kj * rsk;
      // accumulator register 4 a + i of column block dt holds column
      // 32 dt + 8 a + 4 g + i of this lane's key
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int d = 32 * dt + 8 * a + 4 * g;
          f32x4 x, y;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            x[i] = acc_k[dt][4 * a + i] * scale;
            y[i] = acc_v[dt][4 * a + i];
          }
          *reinterpret_cast<V4<T>*>(dk2 + d) = cvt4<T>(x);
          *reinterpret_cast<V4<T>*>(dv2 + d) = cvt4<T>(y);
        }
    }
  }
}

}  // namespace

template <bool CAUSAL>
hipError_t launch_bwdbwd_stage2_k32(const BwdBwdParams<__bf16>& p, hipStream_t stream) {
  const int nkb = (p.nk + 32 * kWaves - 1) / (32 * kWaves);
  const int npairs = p.batch * p.kv_heads;
  const int resident = resident_workgroups(1);
  const int pairs = block_pairing(CAUSAL, nkb, npairs, resident, 1);
  const int nranks = pairs ? (nkb + 1) / 2 : nkb;
  const int chunk = grid_chunk(npairs, nranks, resident);
  const dim3 grid(nranks * npairs);
  int e2;
  if (std::frexp(p.scale, &e2) == 0.5f)  // scale = 2^(e2 - 1)
    hipLaunchKernelGGL((bwdbwd_k32_kernel<CAUSAL, true>), grid, dim3(kThreads), 0, stream, p, pairs, chunk);
  else
    hipLaunchKernelGGL((bwdbwd_k32_kernel<CAUSAL, false>), grid, dim3(kThreads), 0, stream, p, pairs, chunk);
  return hipGetLastError();
}

template hipError_t launch_bwdbwd_stage2_k32<true>(const BwdBwdParams<__bf16>&, hipStream_t);
template hipError_t launch_bwdbwd_stage2_k32<false>(const BwdBwdParams<__bf16>&, hipStream_t);

}  // namespace fhog
